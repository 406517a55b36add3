"""Group-wise affine 2/4-bit values on MI355X (drop-in for inquant.value_codec).

Per token and contiguous channel group: f16 offset = group minimum, f16
scale = (max - min) / (2^bits - 1) (at least 2^-14), codes packed LSB-first.
Interface and semantics follow src/inquant/value_codec.py of the reference:
PackedValues (:12-48), quantize_values (:51-72), quantize_value_blocks (:75-88).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as nat
from .codec import _per_block, _view_nbytes


@dataclass(frozen=True)
class PackedValues:
    payload: torch.Tensor
    scales: torch.Tensor
    offsets: torch.Tensor
    shape: tuple
    original_dtype: torch.dtype
    bits: int
    group_size: int

    @property
    def tensors(self) -> dict:
        return {"payload": self.payload, "scales": self.scales, "offsets": self.offsets}

    @property
    def payload_nbytes(self) -> int:
        return _view_nbytes(self.payload)

    @property
    def nbytes(self) -> int:
        return sum(_view_nbytes(t) for t in self.tensors.values())

    @property
    def metadata_nbytes(self) -> int:
        return self.nbytes - self.payload_nbytes

    @torch.no_grad()
    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = self.original_dtype if dtype is None else dtype
        if not dtype.is_floating_point:
            raise ValueError("dequantize dtype must be floating point")
        device = nat.require_gpu(self.payload, what="PackedValues.dequantize")
        out_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        out = torch.empty(self.shape, dtype=out_dtype, device=device)
        D = self.shape[-1]
        rows = out.numel() // D
        nat.check(nat.lib().iq_v_dequantize(
            self.payload.contiguous().data_ptr(), self.scales.contiguous().data_ptr(),
            self.offsets.contiguous().data_ptr(), rows, D, self.bits, self.group_size, out.data_ptr(),
            nat.dtype_code(out_dtype), nat.stream_handle(device)))
        return out if out_dtype == dtype else out.to(dtype)


_BAD_V = "Values and stored FP16 quantization parameters must be finite"


@torch.no_grad()
def quantize_values(x: torch.Tensor, bits: int = 2, group_size: int = 64, *,
                    _flag: torch.Tensor | None = None) -> PackedValues:
    """Group-wise V2/V4 codes (value_codec.py:51-72); ValueError for non-finite
    data or parameters, checked with one device sync (value_codec.py:64)
    unless the private `_flag` hands the check to the caller."""
    bad = _flag
    if type(bits) is not int or bits not in (2, 4):
        raise ValueError("Value bits must be 2 or 4")
    if type(group_size) is not int or group_size not in (32, 64, 128):
        raise ValueError("Value group size must be 32, 64 or 128")
    if x.ndim != 4 or min(x.shape) < 1 or not x.is_floating_point() or x.shape[-1] % group_size:
        raise ValueError("Expected nonempty floating [batch, heads, tokens, channels] divisible by group_size")
    device = nat.require_gpu(x, what="quantize_values")
    original_dtype = x.dtype
    x = x.detach()
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
        x = x.to(torch.float32)
    B, H, T, D = x.shape
    payload = torch.empty((B, H, T, D * bits // 8), dtype=torch.uint8, device=device)
    scales = torch.empty((B, H, T, D // group_size), dtype=torch.float16, device=device)
    offsets = torch.empty_like(scales)
    own_flag = bad is None
    if own_flag:
        bad = torch.zeros(1, dtype=torch.int32, device=device)
    nat.check(nat.lib().iq_v_quantize(
        x.data_ptr(), nat.dtype_code(x.dtype), nat.strides4(x), B, H, T, D, bits, group_size,
        payload.data_ptr(), scales.data_ptr(), offsets.data_ptr(), bad.data_ptr(), nat.stream_handle(device)))
    if own_flag and int(bad.item()):
        raise ValueError(_BAD_V)
    return PackedValues(payload, scales, offsets, tuple(x.shape), original_dtype, bits, group_size)


def quantize_value_blocks(tensor: torch.Tensor, block_count: int, block_size: int, bits: int, group_size: int):
    """Encode the first `block_count` temporal blocks of [1, H, T, D] with
    statistics per (block, head) (value_codec.py:75-88): one launch over the
    strided [blocks, H, B, D] view, one PackedValues view per block."""
    return _value_blocks(tensor, block_count, block_size, bits, group_size, None)


def _value_blocks(tensor, block_count, block_size, bits, group_size, bad):
    """quantize_value_blocks with the private non-finite flag of quantize_values."""
    if not block_count:
        return []
    _, heads, _, dim = tensor.shape
    blocked = tensor[0, :, :block_count * block_size].unflatten(1, (block_count, block_size)).transpose(0, 1)
    packed = quantize_values(blocked, bits, group_size, _flag=bad)
    return _per_block(packed, block_count, (1, heads, block_size, dim), PackedValues, bits=bits,
                      group_size=group_size)
