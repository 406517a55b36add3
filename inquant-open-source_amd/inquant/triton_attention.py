"""Single-query GQA decode over packed InQuant blocks on MI355X.

The module keeps the reference's name (src/inquant/triton_attention.py) so
callers switch without edits, but nothing here is Triton: ``decode`` runs the
fused HIP decode of libinquant_hip.so over [sink | packed blocks | tail],
followed by the log-sum-exp merge of its partitions.

Public surface (triton_attention.py:184-399): ``SharedDecodeWorkspace``
(``acquire``, ``nbytes``, ``tensor``), ``PackedDecodeState`` (``extend``,
``decode``, ``nbytes``, ``key_blocks``, ``value_blocks`` and the inspected
``_tables`` / ``_key_map`` / ``_value_map`` / ``_workspace``) and
``packed_decode``.  Argument errors carry the reference's exception types and
messages.  Host structure of this build:

* ``_StreamPin`` holds the one stream a workspace or state may be used on.
* ``_BlockFormat`` is the uniform block layout every appended block must
  match, read from the first block.
* ``_Descriptors`` owns the device pointer table (int64 [capacity, 8]: the
  reference's six block addresses, then the K source and donor descriptor
  addresses the decode kernel reads) and the int8 role maps [capacity, H,
  128]; ``iq_decode_append`` writes the rows of new blocks from addresses
  passed as kernel arguments (no host-to-device copy).

Limits follow the reference: batch 1, head_dim 128, one query token, uniform
block length, query heads a multiple of KV heads (at most 16 per KV head
here), no mask.
"""
from __future__ import annotations

import math
import operator

import torch

from . import _native as nat
from .codec import PackedTensor
from .value_codec import PackedValues

_SPLIT = 32           # tokens per dense partition (the native kernels' split)
_COLUMNS = 8          # pointer-table columns


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


class _StreamPin:
    """Binds an object to the first CUDA stream it runs on."""

    __slots__ = ("key", "message")

    def __init__(self, message: str):
        self.key = None
        self.message = message

    def check(self, device) -> int:
        index = device.index if device.index is not None else torch.cuda.current_device()
        handle = torch._C._cuda_getCurrentRawStream(index)
        key = (index, handle)
        if self.key is None:
            self.key = key
        elif key != self.key:
            raise RuntimeError(self.message)
        return handle


class SharedDecodeWorkspace:
    """fp32 scratch of one request, reused by all its layers on one stream.

    The cache counts it once; decode states do not.  The allocation only
    grows (to the largest request seen)."""

    def __init__(self):
        self.tensor = None
        self._pin = _StreamPin("Shared decode workspace requires one CUDA stream per cache")

    @property
    def nbytes(self) -> int:
        return self.tensor.untyped_storage().nbytes() if self.tensor is not None else 0

    def acquire(self, shape, device):
        self._pin.check(device)
        needed = math.prod(shape)
        have = self.tensor
        if have is None or have.numel() < needed:
            have = self.tensor = torch.empty(needed, dtype=torch.float32, device=device)
        return have[:needed].view(shape)


class _BlockFormat:
    """Layout shared by all blocks of a decode state."""

    __slots__ = ("device", "heads", "tokens", "salient", "desc_bytes", "value_bits", "value_group")

    def __init__(self, key0, value0):
        if key0.shape[0] != 1 or key0.shape[-1] != 128 or key0.payload.device.type != "cuda":
            raise ValueError("Packed decode requires CUDA blocks with batch=1 and head_dim=128")
        self.device = key0.payload.device
        self.heads = key0.shape[1]
        self.tokens = key0.shape[2]
        self.salient = key0.salient_channels.shape[-1]
        self.desc_bytes = key0.salient_channels.element_size()
        coded = isinstance(value0, PackedValues)
        self.value_bits = value0.bits if coded else 0
        self.value_group = value0.group_size if coded else 64

    def same(self, other: "_BlockFormat") -> bool:
        return all(getattr(self, f) == getattr(other, f) for f in self.__slots__)

    def admit(self, keys, values) -> None:
        """Raise the reference's errors for blocks that break the layout."""
        for k in keys:
            if (not isinstance(k, PackedTensor) or k.shape != (1, self.heads, self.tokens, 128)
                    or k.salient_channels.shape[-1] != self.salient):
                raise ValueError("All packed K/V blocks must share shape and salient-channel count")
        for v in values:
            if v.shape != (1, self.heads, self.tokens, 128):
                raise ValueError("All packed blocks must share shape")
            if self.value_bits:
                if not isinstance(v, PackedValues) or v.bits != self.value_bits or v.group_size != self.value_group:
                    raise ValueError("All V blocks must share the same quantizer")
            elif not isinstance(v, PackedTensor) or v.salient_channels.shape[-1] != self.salient:
                raise ValueError("All InQuant V blocks must share the salient-channel count")
        index = self.device.index
        for block in (*keys, *values):
            for t in block.tensors.values():
                if t.get_device() != index:
                    raise ValueError("All packed tensors must share the same CUDA device")
        if self.salient > 64:
            raise ValueError("Packed decode supports at most 64 salient channels (int8 roles)")


def _field_addresses(k, v, k4_values):
    """A block's addresses in pointer-table column order."""
    return (k.payload.data_ptr(), k.scales.data_ptr(), k.padding.data_ptr(), v.payload.data_ptr(),
            v.scales.data_ptr(), (v.padding if k4_values else v.offsets).data_ptr(),
            k.salient_channels.data_ptr(), k.donor_channels.data_ptr())


def _field_bytes(fmt: "_BlockFormat") -> tuple:
    """Bytes per block of each field, when blocks come from one batched encode."""
    h, t, s = fmt.heads, fmt.tokens, fmt.salient
    vbytes = 128 * fmt.value_bits // 8
    groups = 128 // fmt.value_group
    return (h * t * 64, h * 512, h * s * 4, h * t * vbytes, h * t * groups * 2, h * t * groups * 2,
            h * s * fmt.desc_bytes, h * s * fmt.desc_bytes)


class _Descriptors:
    """Pointer table and role maps, grown on demand: exact at first, then
    max(n, min(2 * capacity, n + 7)) blocks (triton_attention.py:282-283)."""

    def __init__(self, device, heads: int, k4_values: bool):
        self.run = nat.BlockRun()          # leading blocks at a fixed stride (one batched encode)
        self.run_open = True               # the run may still grow
        self.tables = torch.empty((0, _COLUMNS), dtype=torch.int64, device=device)
        self.key_map = torch.empty((0, heads, 128), dtype=torch.int8, device=device)
        self.value_map = torch.empty((0, heads, 128) if k4_values else (0,), dtype=torch.int8, device=device)
        self.k4_values = k4_values

    def reserve(self, used: int, needed: int) -> None:
        capacity = self.tables.shape[0]
        if needed <= capacity:
            return
        grown = needed if capacity == 0 else max(needed, min(2 * capacity, needed + 7))

        def regrow(old, shape):
            new = torch.empty(shape, dtype=old.dtype, device=old.device)
            if used:
                new[:used].copy_(old[:used])
            return new

        self.tables = regrow(self.tables, (grown, _COLUMNS))
        self.key_map = regrow(self.key_map, (grown, *self.key_map.shape[1:]))
        if self.k4_values:
            self.value_map = regrow(self.value_map, (grown, *self.value_map.shape[1:]))

    def grow_run(self, first: int, keys, values, fmt: _BlockFormat) -> None:
        """Extend the fixed-stride run over the new blocks while they continue it."""
        if not self.run_open or fmt.value_bits == 0:
            self.run_open = False
            return
        step = _field_bytes(fmt)
        run = self.run
        for i, (k, v) in enumerate(zip(keys, values)):
            addr = _field_addresses(k, v, False)
            if run.blocks == 0 and first + i == 0:
                for f in range(_COLUMNS):
                    run.base[f] = addr[f]
            elif run.blocks != first + i or any(addr[f] != run.base[f] + run.blocks * step[f]
                                                for f in range(_COLUMNS)):
                self.run_open = False
                return
            run.blocks += 1

    def write(self, first: int, keys, values, fmt: _BlockFormat, stream: int) -> None:
        self.grow_run(first, keys, values, fmt)
        rows = (nat.BlockPtrs * len(keys))()
        for row, k, v in zip(rows, keys, values):
            row.k_payload, row.k_scales, row.k_padding = k.payload.data_ptr(), k.scales.data_ptr(), k.padding.data_ptr()
            row.k_src, row.k_don = k.salient_channels.data_ptr(), k.donor_channels.data_ptr()
            row.v_payload, row.v_scales = v.payload.data_ptr(), v.scales.data_ptr()
            if self.k4_values:
                row.v_offsets = v.padding.data_ptr()
                row.v_src, row.v_don = v.salient_channels.data_ptr(), v.donor_channels.data_ptr()
            else:
                row.v_offsets = v.offsets.data_ptr()
        nat.check(nat.lib().iq_decode_append(
            self.tables.data_ptr(), self.key_map.data_ptr(),
            self.value_map.data_ptr() if self.k4_values else None, first, len(keys), rows, fmt.heads,
            fmt.salient, fmt.desc_bytes, stream))

    def tensors(self):
        return self.tables, self.key_map, self.value_map


def _dense_segment(name, key, value, query, heads):
    """Validate one exact segment; returns (key, value, tokens, heads)."""
    if key is None and value is None:
        return None, None, 0, heads
    if key is None or value is None:
        raise ValueError(f"{name} key/value must both be provided")
    if key.ndim != 4 or key.shape != value.shape or key.shape[0] != 1 or key.shape[-1] != 128:
        raise ValueError(f"{name} K/V must have matching [1, KV_heads, tokens, 128] shapes")
    if {key.dtype, value.dtype} != {query.dtype} or key.device != query.device or value.device != query.device:
        raise ValueError(f"{name} K/V must match query dtype and device")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError(f"{name} head dimension must be contiguous")
    if heads is not None and key.shape[1] != heads:
        raise ValueError("All inputs must share their KV head count")
    return key, value, key.shape[2], key.shape[1]


class PackedDecodeState:
    """Decode descriptors of immutable packed blocks, appended incrementally;
    sink and tail are per-call inputs (triton_attention.py:211-388)."""

    def __init__(self, key_blocks, value_blocks, *, workspace_pool=None):
        if len(key_blocks) != len(value_blocks):
            raise ValueError("Key and value block counts must match")
        self._keys: list = []       # the blocks held, grown by each extend's new suffix
        self._values: list = []
        self._held = None           # (key tuple, value tuple) of them, built on request
        self._format: _BlockFormat | None = None
        self._desc: _Descriptors | None = None
        self._pin = _StreamPin("Descriptor updates require one CUDA stream per state")
        self._workspace_pool = workspace_pool
        self._workspace = None
        self.extend(key_blocks, value_blocks)

    @property
    def key_blocks(self) -> tuple:
        return self._held_blocks()[0]

    @property
    def value_blocks(self) -> tuple:
        return self._held_blocks()[1]

    @property
    def block_count(self) -> int:
        """Blocks held (len(key_blocks), without building the tuple)."""
        return len(self._keys)

    def _held_blocks(self) -> tuple:
        if self._held is None:
            self._held = (tuple(self._keys), tuple(self._values))
        return self._held

    # inspected by the reference's tests
    @property
    def _tables(self):
        return None if self._desc is None else self._desc.tables

    @property
    def _key_map(self):
        return None if self._desc is None else self._desc.key_map

    @property
    def _value_map(self):
        return None if self._desc is None else self._desc.value_map

    def extend(self, key_blocks, value_blocks) -> None:
        """Append blocks; the known blocks must be an unchanged prefix (identity)."""
        if len(key_blocks) != len(value_blocks):
            raise ValueError("Key and value block counts must match")
        have = len(self._keys)
        prefix_ok = len(key_blocks) >= have and all(map(operator.is_, self._keys, key_blocks)) \
            and all(map(operator.is_, self._values, value_blocks))
        if not prefix_ok:
            raise ValueError("PackedDecodeState.extend requires an immutable append-only prefix")
        if len(key_blocks) == have:
            return
        if have:
            # the first blocks are the ones held (identity), so is their format
            fmt = self._format
        else:
            fmt = _BlockFormat(key_blocks[0], value_blocks[0])
            if self._format is not None and not self._format.same(fmt):
                raise ValueError("All packed K/V blocks must share shape and salient-channel count")
        stream = self._pin.check(fmt.device)
        new_keys, new_values = tuple(key_blocks[have:]), tuple(value_blocks[have:])
        fmt.admit(new_keys, new_values)
        if self._desc is None or self._desc.tables.device != fmt.device:
            self._desc = _Descriptors(fmt.device, fmt.heads, fmt.value_bits == 0)
        self._format = fmt
        self._desc.reserve(have, len(key_blocks))
        self._desc.write(have, new_keys, new_values, fmt, stream)
        # only the new blocks are added (the held prefix is identical): no
        # pass over the whole history beyond the identity check
        self._keys.extend(new_keys)
        self._values.extend(new_values)
        self._held = None

    @property
    def nbytes(self) -> int:
        """Device bytes this state owns: tables, role maps and a private workspace."""
        owned = [] if self._desc is None else list(self._desc.tensors())
        if self._workspace is not None:
            owned.append(self._workspace)
        return sum(t.untyped_storage().nbytes() for t in owned)

    def _scratch(self, shape, device):
        if self._workspace_pool is not None:
            return self._workspace_pool.acquire(shape, device)
        ws = self._workspace
        if ws is None or tuple(ws.shape) != tuple(shape) or ws.device != device:
            ws = self._workspace = torch.empty(shape, dtype=torch.float32, device=device)
        return ws

    @torch.no_grad()
    def decode(self, query, *, sink_key=None, sink_value=None, residual_key=None, residual_value=None,
               scale=None, output=None):
        """softmax(scale * q K^T) V over sink ++ blocks ++ tail for every query head.

        ``output`` (not in the reference signature) may be a contiguous
        query-shaped tensor of the query dtype or float32 that receives the
        result, so that calls can be captured in a HIP graph."""
        if query.ndim != 4 or query.shape[0] != 1 or query.shape[1] < 1 or tuple(query.shape[2:]) != (1, 128):
            raise ValueError("query must have shape [1, query_heads, 1, 128]")
        if query.device.type != "cuda" or query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("query must be a CUDA FP16, BF16 or FP32 tensor")
        if query.stride(-1) != 1:
            raise ValueError("query head dimension must be contiguous")
        fmt = self._format
        if fmt is not None and query.device != fmt.device:
            raise ValueError("query and packed blocks must share a device")
        heads = None if fmt is None else fmt.heads
        sk, sv, sink_t, heads = _dense_segment("sink", sink_key, sink_value, query, heads)
        tk, tv, tail_t, heads = _dense_segment("residual", residual_key, residual_value, query, heads)
        hq = query.shape[1]
        if heads is None or hq % heads:
            raise ValueError("query_heads must be divisible by the nonempty KV head count")
        n_blocks = len(self._keys)
        partitions = n_blocks + _ceil_div(sink_t, _SPLIT) + _ceil_div(tail_t, _SPLIT)
        if partitions == 0:
            raise ValueError("Attention requires at least one key/value token")
        scale = 128 ** -0.5 if scale is None else scale
        if not (math.isfinite(scale) and scale > 0):
            raise ValueError("attention scale must be positive and finite")
        if hq // heads > 16:
            raise ValueError("Packed decode supports at most 16 query heads per KV head")
        workspace = self._scratch((hq, partitions, 130), query.device)
        if output is None:
            output = torch.empty_like(query, memory_format=torch.contiguous_format)
        elif (tuple(output.shape) != tuple(query.shape) or not output.is_contiguous()
              or output.dtype not in (query.dtype, torch.float32) or output.device != query.device):
            raise ValueError("output must be a contiguous query-shaped tensor of the query dtype or float32")
        if self._desc is None:
            # dense-only state: zero-row tables (no storage) keep nbytes as the reference reports it
            self._desc = _Descriptors(query.device, heads, True)
        desc = self._desc
        bits = 0 if fmt is None else fmt.value_bits
        k4_values = n_blocks and bits == 0

        def strides(t):
            return (0, 0) if t is None else (t.stride(1), t.stride(2))

        nat.check(nat.lib().iq_decode_attention(
            query.data_ptr(), nat.dtype_code(query.dtype), query.stride(1), hq,
            desc.tables.data_ptr() if n_blocks else None, desc.key_map.data_ptr() if n_blocks else None,
            desc.value_map.data_ptr() if k4_values else None, desc.run if desc.run.blocks else None, n_blocks,
            256 if fmt is None else fmt.tokens, heads, 0 if fmt is None else fmt.salient, bits,
            64 if fmt is None else fmt.value_group,
            nat.ptr(sk), nat.ptr(sv), *strides(sk), *strides(sv), sink_t,
            nat.ptr(tk), nat.ptr(tv), *strides(tk), *strides(tv), tail_t,
            float(scale), workspace.data_ptr(), workspace.numel(), output.data_ptr(),
            nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
        return output


def packed_decode(query, key_blocks, value_blocks, sink_key=None, sink_value=None, residual_key=None,
                  residual_value=None, *, scale=None):
    """Decode once without keeping a state (triton_attention.py:391-399)."""
    state = PackedDecodeState(key_blocks, value_blocks)
    return state.decode(query, sink_key=sink_key, sink_value=sink_value, residual_key=residual_key,
                        residual_value=residual_value, scale=scale)
