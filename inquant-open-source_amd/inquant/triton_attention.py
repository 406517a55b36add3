"""Single-query GQA decode directly over packed InQuant blocks (MI355X).

Module and class names are kept from the reference (src/inquant/triton_attention.py)
so callers switch without edits; no Triton is used.  PackedDecodeState keeps
the reference's reusable metadata -- an i64 pointer table [cap, 8] (the
reference's six block addresses plus the K descriptor addresses) and int8
role maps [cap, H, 128] appended incrementally (:294-369) -- and decode()
runs the fused HIP kernel over [sink | packed blocks | tail] followed by the
log-sum-exp merge (:377-448).  Keys and values are decoded and rounded to the
query dtype exactly as the dequantize-then-attend path does; softmax weights
and accumulation stay in fp32.

Limits follow the reference: batch 1, head_dim 128, one query token, uniform
packed block length, query heads divisible by KV heads (at most 16 per KV
head here), no mask.  Not safe for concurrent calls from different streams.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat
from .codec import PackedTensor
from .value_codec import PackedValues

_DENSE_SPLIT = 256
# pointer-table columns: the reference's six block addresses plus the K
# source/donor descriptor addresses read directly by the decode kernel
_TABLE_COLS = 8


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


class SharedDecodeWorkspace:
    """One fp32 scratch allocation per request, usable on one stream (triton_attention.py:184-208)."""

    def __init__(self):
        self.tensor = None
        self._stream_identity = None

    @property
    def nbytes(self) -> int:
        return 0 if self.tensor is None else self.tensor.untyped_storage().nbytes()

    def acquire(self, shape, device):
        stream = torch.cuda.current_stream(device)
        identity = (stream.device, stream.cuda_stream)
        if self._stream_identity is not None and identity != self._stream_identity:
            raise RuntimeError("Shared decode workspace requires one CUDA stream per cache")
        self._stream_identity = identity
        needed = math.prod(shape)
        if self.tensor is None or self.tensor.numel() < needed:
            self.tensor = torch.empty(needed, dtype=torch.float32, device=device)
        return self.tensor[:needed].view(shape)


class PackedDecodeState:
    """Reusable descriptors for immutable packed blocks; sink/tail are per-call inputs."""

    def __init__(self, key_blocks, value_blocks, *, workspace_pool=None):
        if len(key_blocks) != len(value_blocks):
            raise ValueError("Key and value block counts must match")
        self.key_blocks = ()
        self.value_blocks = ()
        self._workspace = None
        self._workspace_pool = workspace_pool
        self._tables = None
        self._key_map = None
        self._value_map = None
        self._device = None
        self._kv_heads = None
        self._packed_tokens = 256
        self._salient = 0
        self._value_bits = 0
        self._value_group = 64
        self._capacity = 0
        self._stream_identity = None
        self.extend(key_blocks, value_blocks)

    def extend(self, key_blocks, value_blocks):
        """Append immutable blocks; descriptors are written only for the new suffix.

        Capacity grows as in the reference: exact first, then
        max(n, min(2 * cap, n + 7)) blocks.
        """
        if len(key_blocks) != len(value_blocks):
            raise ValueError("Key and value block counts must match")
        old = len(self.key_blocks)
        if (len(key_blocks) < old or any(a is not b for a, b in zip(self.key_blocks, key_blocks))
                or any(a is not b for a, b in zip(self.value_blocks, value_blocks))):
            raise ValueError("PackedDecodeState.extend requires an immutable append-only prefix")
        if len(key_blocks) == old:
            return
        first = key_blocks[0]
        if first.shape[0] != 1 or first.shape[-1] != 128 or first.payload.device.type != "cuda":
            raise ValueError("Packed decode requires CUDA blocks with batch=1 and head_dim=128")
        stream = torch.cuda.current_stream(first.payload.device)
        identity = (stream.device, stream.cuda_stream)
        if self._stream_identity is not None and self._stream_identity != identity:
            raise RuntimeError("Descriptor updates require one CUDA stream per state")
        self._stream_identity = identity
        self._device = first.payload.device
        self._kv_heads = first.shape[1]
        self._packed_tokens = first.shape[2]
        self._salient = first.salient_channels.shape[-1]
        # The prefix was validated against the same first block by an earlier
        # call and is identical (checked above), so only the new suffix is
        # checked; the reference re-checks every block on every append
        # (triton_attention.py:257-269), which costs O(blocks) host time per seal.
        for block in key_blocks[old:]:
            if (not isinstance(block, PackedTensor) or block.shape != first.shape
                    or block.salient_channels.shape[-1] != self._salient):
                raise ValueError("All packed K/V blocks must share shape and salient-channel count")
        v0 = value_blocks[0]
        self._value_bits = v0.bits if isinstance(v0, PackedValues) else 0
        self._value_group = v0.group_size if self._value_bits else 64
        for block in value_blocks[old:]:
            if block.shape != first.shape:
                raise ValueError("All packed blocks must share shape")
            if self._value_bits:
                if not isinstance(block, PackedValues) or (block.bits, block.group_size) != (
                        self._value_bits, self._value_group):
                    raise ValueError("All V blocks must share the same quantizer")
            elif not isinstance(block, PackedTensor) or block.salient_channels.shape[-1] != self._salient:
                raise ValueError("All InQuant V blocks must share the salient-channel count")
        for block in (*key_blocks[old:], *value_blocks[old:]):
            if any(t.device != self._device for t in block.tensors.values()):
                raise ValueError("All packed tensors must share the same CUDA device")
        if self._salient > 64:
            raise ValueError("Packed decode supports at most 64 salient channels (int8 roles)")

        count = len(key_blocks)
        if count > self._capacity:
            capacity = count if not self._capacity else max(count, min(self._capacity * 2, count + 7))
            tables = torch.empty((capacity, _TABLE_COLS), dtype=torch.int64, device=self._device)
            key_map = torch.empty((capacity, self._kv_heads, 128), dtype=torch.int8, device=self._device)
            value_map = (torch.empty((0,), dtype=torch.int8, device=self._device) if self._value_bits
                         else torch.empty_like(key_map))
            if old:
                tables[:old].copy_(self._tables[:old])
                key_map[:old].copy_(self._key_map[:old])
                if not self._value_bits:
                    value_map[:old].copy_(self._value_map[:old])
            self._tables, self._key_map, self._value_map = tables, key_map, value_map
            self._capacity = capacity

        new_k, new_v = key_blocks[old:], value_blocks[old:]
        ptrs = (nat.BlockPtrs * len(new_k))()
        for i, (k, v) in enumerate(zip(new_k, new_v)):
            entry = ptrs[i]
            entry.k_payload, entry.k_scales, entry.k_padding = (
                k.payload.data_ptr(), k.scales.data_ptr(), k.padding.data_ptr())
            entry.v_payload, entry.v_scales = v.payload.data_ptr(), v.scales.data_ptr()
            entry.v_offsets = (v.offsets if self._value_bits else v.padding).data_ptr()
            entry.k_src, entry.k_don = k.salient_channels.data_ptr(), k.donor_channels.data_ptr()
            if not self._value_bits:
                entry.v_src, entry.v_don = v.salient_channels.data_ptr(), v.donor_channels.data_ptr()
        nat.check(nat.lib().iq_decode_append(
            self._tables.data_ptr(), self._key_map.data_ptr(),
            None if self._value_bits else self._value_map.data_ptr(), old, len(new_k), ptrs,
            self._kv_heads, self._salient, first.salient_channels.element_size(), identity[1]))
        self.key_blocks, self.value_blocks = tuple(key_blocks), tuple(value_blocks)

    @property
    def nbytes(self) -> int:
        """Auxiliary GPU allocations of this state (tables, maps, private workspace)."""
        return sum(t.untyped_storage().nbytes() for t in
                   (self._tables, self._key_map, self._value_map, self._workspace) if t is not None)

    @torch.no_grad()
    def decode(self, query, *, sink_key=None, sink_value=None, residual_key=None, residual_value=None,
               scale=None, output=None):
        """Attention of `query` over sink, packed blocks and tail.

        `output` (an extension of the reference signature) may be a
        contiguous [1, Hq, 1, 128] tensor of the query dtype or float32 to
        receive the result, e.g. to read the unrounded fp32 value.
        """
        if query.ndim != 4 or query.shape[0] != 1 or query.shape[1] < 1 or tuple(query.shape[-2:]) != (1, 128):
            raise ValueError("query must have shape [1, query_heads, 1, 128]")
        if query.device.type != "cuda" or query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("query must be a CUDA FP16, BF16 or FP32 tensor")
        if query.stride(-1) != 1:
            raise ValueError("query head dimension must be contiguous")
        if self._device is not None and query.device != self._device:
            raise ValueError("query and packed blocks must share a device")
        kv_heads = self._kv_heads
        dense = []
        for name, key, value in (("sink", sink_key, sink_value), ("residual", residual_key, residual_value)):
            if (key is None) != (value is None):
                raise ValueError(f"{name} key/value must both be provided")
            if key is None:
                dense.append((None, None, 0))
                continue
            if key.ndim != 4 or key.shape != value.shape or key.shape[0] != 1 or key.shape[-1] != 128:
                raise ValueError(f"{name} K/V must have matching [1, KV_heads, tokens, 128] shapes")
            if (key.dtype != query.dtype or value.dtype != query.dtype or key.device != query.device
                    or value.device != query.device):
                raise ValueError(f"{name} K/V must match query dtype and device")
            if key.stride(-1) != 1 or value.stride(-1) != 1:
                raise ValueError(f"{name} head dimension must be contiguous")
            kv_heads = key.shape[1] if kv_heads is None else kv_heads
            if key.shape[1] != kv_heads:
                raise ValueError("All inputs must share their KV head count")
            dense.append((key, value, key.shape[2]))
        if kv_heads is None or query.shape[1] % kv_heads:
            raise ValueError("query_heads must be divisible by the nonempty KV head count")
        (sk, sv, sink_t), (tk, tv, tail_t) = dense
        partitions = len(self.key_blocks) + _cdiv(sink_t, _DENSE_SPLIT) + _cdiv(tail_t, _DENSE_SPLIT)
        if not partitions:
            raise ValueError("Attention requires at least one key/value token")
        if scale is None:
            scale = 128 ** -0.5
        if not math.isfinite(scale) or scale <= 0:
            raise ValueError("attention scale must be positive and finite")
        if query.shape[1] // kv_heads > 16:
            raise ValueError("Packed decode supports at most 16 query heads per KV head")
        shape = (query.shape[1], partitions, 130)
        if self._workspace_pool is not None:
            workspace = self._workspace_pool.acquire(shape, query.device)
        else:
            if self._workspace is None or tuple(self._workspace.shape) != shape or self._workspace.device != query.device:
                self._workspace = torch.empty(shape, dtype=torch.float32, device=query.device)
            workspace = self._workspace
        if output is None:
            output = torch.empty_like(query, memory_format=torch.contiguous_format)
        elif (tuple(output.shape) != tuple(query.shape) or not output.is_contiguous()
              or output.dtype not in (query.dtype, torch.float32) or output.device != query.device):
            raise ValueError("output must be a contiguous query-shaped tensor of the query dtype or float32")
        if self._tables is None:
            # zero-element placeholders keep nbytes accounting identical to the reference
            self._tables = torch.empty((0, _TABLE_COLS), dtype=torch.int64, device=query.device)
            self._key_map = torch.empty((0, kv_heads, 128), dtype=torch.int8, device=query.device)
            self._value_map = torch.empty_like(self._key_map)
            self._device = query.device
        n_blocks = len(self.key_blocks)
        stream = nat.stream_handle(query.device)
        lib = nat.lib()

        def st(t, dim):
            return 0 if t is None else t.stride(dim)

        nat.check(lib.iq_decode_attention(
            query.data_ptr(), nat.dtype_code(query.dtype), query.stride(1), query.shape[1],
            self._tables.data_ptr() if n_blocks else None, self._key_map.data_ptr() if n_blocks else None,
            self._value_map.data_ptr() if (n_blocks and not self._value_bits) else None,
            n_blocks, self._packed_tokens, kv_heads, self._salient, self._value_bits, self._value_group,
            nat.ptr(sk), nat.ptr(sv), st(sk, 1), st(sk, 2), st(sv, 1), st(sv, 2), sink_t,
            nat.ptr(tk), nat.ptr(tv), st(tk, 1), st(tk, 2), st(tv, 1), st(tv, 2), tail_t,
            float(scale), workspace.data_ptr(), workspace.numel(), output.data_ptr(),
            nat.dtype_code(output.dtype), stream))
        return output


def packed_decode(query, key_blocks, value_blocks, sink_key=None, sink_value=None, residual_key=None,
                  residual_value=None, *, scale=None):
    """One-shot wrapper; reuse PackedDecodeState for repeated decoding (triton_attention.py:391-399)."""
    return PackedDecodeState(key_blocks, value_blocks).decode(
        query, sink_key=sink_key, sink_value=sink_value, residual_key=residual_key,
        residual_value=residual_value, scale=scale)
