"""K4 neighbor-slot key codec on MI355X (drop-in for the reference's inquant.codec).

Every channel owns one 4-bit slot of the packed payload; the `count` most
salient channels (sampled mean |x|) store an 8-bit code whose high nibble
sits in their own slot and whose low nibble borrows a donor channel's slot.
Donor channels decode to their sampled temporal mean ("padding").

Interface and semantics follow src/inquant/codec.py of the reference:
CodecConfig (:38-55), PackedTensor (:58-134), _reuse_map (:137-178) and
quantize (:181-243).  All arithmetic runs in libinquant_hip.so and is
bit-identical to the reference's CPU torch implementation; CPU tensors are
rejected rather than silently served by another implementation.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as nat

_POLICIES = ("neighbors", "min_error")
_BACKENDS = ("torch", "triton", "auto")


@dataclass(frozen=True)
class CodecConfig:
    """Codec options, validated like codec.py:38-55.

    `donor_backend` is accepted for compatibility; every backend name runs
    the same fused HIP selector.
    """

    sample_stride: int = 8
    salient_fraction: float = 0.125
    donor_policy: str = "neighbors"
    donor_backend: str = "torch"

    def __post_init__(self) -> None:
        if self.donor_backend not in _BACKENDS:
            raise ValueError("donor_backend must be torch, triton or auto")
        stride = self.sample_stride
        if isinstance(stride, bool) or not isinstance(stride, int) or stride < 1:
            raise ValueError("sample_stride must be a positive integer")
        fraction = self.salient_fraction
        if not math.isfinite(fraction) or fraction < 0 or fraction > 0.5:
            raise ValueError("salient_fraction must be finite and in [0, 0.5]")
        if self.donor_policy not in _POLICIES:
            raise ValueError("donor_policy must be neighbors or min_error")


def _view_nbytes(t: torch.Tensor) -> int:
    """Bytes a field occupies.  A field is either an owned compact tensor
    (its whole storage) or a per-block view of a batched encode; the views
    of one encode tile its storage exactly, so summing them counts every
    stored byte once (the reference clones each block and counts storage,
    codec.py:98-110, with the same totals)."""
    return t.numel() * t.element_size()


def _per_block(packed, count: int, shape, cls, **extra) -> list:
    """Per-block objects whose fields are views of a batched [count, H, ...] encode."""
    if count == 1:
        return [cls(**packed.tensors, shape=shape, original_dtype=packed.original_dtype, **extra)]
    names = list(packed.tensors)
    pieces = [t.split(1) for t in packed.tensors.values()]
    return [cls(**dict(zip(names, parts)), shape=shape, original_dtype=packed.original_dtype, **extra)
            for parts in zip(*pieces)]


@dataclass(frozen=True)
class PackedTensor:
    """One packed K4 tensor; layout of codec.py:58-110.

    payload u8 [B, H, T, D/2] (even channel in the low nibble), scales f32
    [B, H, D], salient/donor channel indices [B, H, S] (u8, int32 if D > 256)
    and padding f32 [B, H, S].
    """

    payload: torch.Tensor
    scales: torch.Tensor
    salient_channels: torch.Tensor
    donor_channels: torch.Tensor
    padding: torch.Tensor
    shape: tuple
    original_dtype: torch.dtype

    @property
    def tensors(self) -> dict:
        return {"payload": self.payload, "scales": self.scales, "salient_channels": self.salient_channels,
                "donor_channels": self.donor_channels, "padding": self.padding}

    @property
    def payload_nbytes(self) -> int:
        return _view_nbytes(self.payload)

    @property
    def nbytes(self) -> int:
        return sum(_view_nbytes(t) for t in self.tensors.values())

    @property
    def metadata_nbytes(self) -> int:
        return self.nbytes - self.payload_nbytes

    def storage_stats(self) -> dict:
        dense = math.prod(self.shape) * self.original_dtype.itemsize
        descriptors = _view_nbytes(self.salient_channels) + _view_nbytes(self.donor_channels)
        return {
            "payload_nbytes": self.payload_nbytes,
            "scale_nbytes": _view_nbytes(self.scales),
            "descriptor_nbytes": descriptors,
            "padding_nbytes": _view_nbytes(self.padding),
            "metadata_nbytes": self.metadata_nbytes,
            "nbytes": self.nbytes,
            "source_nbytes": dense,
            "compression_ratio": dense / self.nbytes,
        }

    @torch.no_grad()
    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """Dense reconstruction (codec.py:112-134), computed by the HIP decoder."""
        dtype = self.original_dtype if dtype is None else dtype
        if not dtype.is_floating_point:
            raise ValueError("dequantize dtype must be floating point")
        device = nat.require_gpu(self.payload, what="PackedTensor.dequantize")
        B, H, T, D = self.shape
        count = self.salient_channels.shape[-1]
        out_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        out = torch.empty((B, H, T, D), dtype=out_dtype, device=device)
        payload = self.payload.contiguous()
        src = self.salient_channels.contiguous()
        don = self.donor_channels.contiguous()
        padding = self.padding.contiguous()
        scales = self.scales.contiguous()
        nat.check(nat.lib().iq_k4_dequantize(
            payload.data_ptr(), scales.data_ptr(), src.data_ptr() if count else None,
            don.data_ptr() if count else None, src.element_size(), padding.data_ptr() if count else None,
            B * H, T, D, count, out.data_ptr(), nat.dtype_code(out_dtype), nat.stream_handle(device)))
        return out if out_dtype == dtype else out.to(dtype)


def _reuse_map(saliency: torch.Tensor, count: int, donor_error: torch.Tensor | None = None):
    """Disjoint sources/donors per row of `saliency` (codec.py:137-178), on the GPU."""
    device = nat.require_gpu(saliency, donor_error, what="_reuse_map")
    *prefix, channels = saliency.shape
    sources = torch.empty((*prefix, count), dtype=torch.int64, device=device)
    donors = torch.empty_like(sources)
    rows = math.prod(prefix)
    if count and rows:
        if 2 * count > channels:
            raise ValueError("count must leave at least as many donor candidates as sources")
        sal = saliency.to(torch.float32).contiguous()
        err = None if donor_error is None else donor_error.to(torch.float32).contiguous()
        nat.check(nat.lib().iq_reuse_map(sal.data_ptr(), nat.ptr(err), rows, channels, count,
                                         sources.data_ptr(), donors.data_ptr(), nat.stream_handle(device)))
    return sources, donors


def _check_bad_flag(flag: torch.Tensor, message: str) -> None:
    if int(flag.item()):
        raise ValueError(message)


_BAD_K = "x must contain finite values representable in float32"


@torch.no_grad()
def quantize(x: torch.Tensor, config: CodecConfig = CodecConfig(), *,
             _flag: torch.Tensor | None = None) -> PackedTensor:
    """Pack one [batch, heads, tokens, even_head_dim] tensor (codec.py:181-243).

    floor(head_dim * salient_fraction) channels get 8-bit codes; as many
    low-saliency channels donate their slot and decode to their sampled mean.
    Raises ValueError for empty, non-floating, odd-width or non-finite input;
    the non-finite check costs one device sync (as the reference's finite
    check at codec.py:197).  With the private `_flag` (a one-element int32
    device tensor) the kernel raises the flag there instead and the caller
    checks it, so that a caller encoding several tensors syncs once.
    """
    bad = _flag
    if x.ndim != 4 or any(size < 1 for size in x.shape):
        raise ValueError("x must have nonempty [batch, heads, tokens, channels] dimensions")
    if not x.is_floating_point():
        raise ValueError("x must have a floating-point dtype")
    if x.shape[-1] % 2:
        raise ValueError("head dimension must be even for two nibbles per byte")
    device = nat.require_gpu(x, what="quantize")
    original_dtype = x.dtype
    x = x.detach()
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
        x = x.to(torch.float32)
    B, H, T, D = x.shape
    if D > 1024:
        raise ValueError("head dimension above 1024 is not supported by the HIP codec")
    count = math.floor(D * config.salient_fraction)
    desc_dtype = torch.uint8 if D <= 256 else torch.int32
    payload = torch.empty((B, H, T, D // 2), dtype=torch.uint8, device=device)
    scales = torch.empty((B, H, D), dtype=torch.float32, device=device)
    src = torch.empty((B, H, count), dtype=desc_dtype, device=device)
    don = torch.empty((B, H, count), dtype=desc_dtype, device=device)
    padding = torch.empty((B, H, count), dtype=torch.float32, device=device)
    own_flag = bad is None
    if own_flag:
        bad = torch.zeros(1, dtype=torch.int32, device=device)
    nat.check(nat.lib().iq_k4_quantize(
        x.data_ptr(), nat.dtype_code(x.dtype), nat.strides4(x), B, H, T, D, count, config.sample_stride,
        int(config.donor_policy == "min_error"), payload.data_ptr(), scales.data_ptr(),
        src.data_ptr() if count else None, don.data_ptr() if count else None, src.element_size(),
        padding.data_ptr() if count else None, bad.data_ptr(), nat.stream_handle(device)))
    if own_flag:
        _check_bad_flag(bad, _BAD_K)
    return PackedTensor(payload, scales, src, don, padding, tuple(x.shape), original_dtype)
