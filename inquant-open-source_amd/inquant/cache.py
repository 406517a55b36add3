"""Append-only InQuant KV cache of one request on MI355X.

Drop-in for the reference's ``inquant.cache`` (src/inquant/cache.py): the
same ``CacheConfig`` fields and validation messages, the same
``InQuantCache`` methods and Hugging Face cache protocol, the same sealing
rule (sink = first ``sink_tokens`` tokens; blocks of ``block_size`` tokens
are sealed from the front of tail ++ new while at least
``residual_length + block_size`` tokens are pending, cache.py:271-306) and
the same byte accounting (cache.py:308-394).

How a layer is stored here (not how the reference stores it):

* Sink and tail are rows of two preallocated buffers of shape
  [2 (keys, values), KV heads, rows, head_dim].  The tail buffer holds
  ``residual_length + block_size`` rows; the live tail is rows
  [start, start + count).  A one-token append writes one row in place with a
  single kernel (``iq_tail_append``) instead of concatenating the whole tail
  (the reference's two ``torch.cat`` per layer per token,
  cache.py:256-259).  When the tail reaches ``residual_length + block_size``
  rows its first ``block_size`` rows are sealed and ``start`` moves past them;
  the first append after that moves the survivors back to row 0 in the same
  launch.  A view handed out by ``append_for_attention`` therefore stays
  valid until the append after the next seal.
* Sealed blocks are per-block views of one batched encode (one K4 and one
  value launch per seal, no per-block copies).  Their byte counts are the
  bytes of their views, which tile the batched allocation exactly, so the
  totals equal the reference's per-block clones.
* ``cache_position`` is compared on the device by the append kernel.  With
  ``validate_positions`` a position tensor not yet verified for this start
  (the first layer of each decode step, or any layer after the tensor was
  written in place: its version counter moved) synchronizes and raises
  before anything changes, as the reference does on every layer.  The other
  layers of the step get the same tensor, unchanged, for the same start, so
  they hold the positions already verified and need no second sync.  An
  inference-mode tensor keeps no version counter: an in-place change of it
  between layers of one step is caught by the device comparison and raised
  at the next synchronization (the next step's check or the next seal).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, NamedTuple

import torch

try:
    from transformers.cache_utils import Cache as _HFCache
except ImportError:  # the codec and cache do not need transformers
    class _HFCache:
        pass

from . import _native as nat
from .codec import _BAD_K, CodecConfig, PackedTensor, _per_block, quantize
from .value_codec import _BAD_V, PackedValues, _value_blocks

_POSITION_ERROR = "Only contiguous append positions are supported; reset before a new request"


def _version(t):
    """The tensor's in-place write counter (None for inference tensors)."""
    return None if t.is_inference() else t._version
# flag words of a cache: key non-finite, value non-finite, position mismatch
_KEY_BAD, _VALUE_BAD, _POSITION_BAD = 0, 1, 2


@dataclass(frozen=True)
class CacheConfig:
    """Cache options (cache.py:24-54).  ``validate_positions=False`` skips the
    position comparison (the caller guarantees contiguous positions)."""

    codec: CodecConfig = field(default_factory=CodecConfig)
    block_size: int = 256
    residual_length: int = 128
    sink_tokens: int = 4
    validate_positions: bool = True
    shared_workspace: bool = False
    value_bits: int | None = None
    value_group_size: int = 64
    track_peak_bytes: bool = False

    def __post_init__(self) -> None:
        for name in ("block_size", "residual_length", "sink_tokens"):
            if type(getattr(self, name)) is not int:
                raise ValueError(f"{name} must be an integer")
        if min(self.block_size - 1, self.residual_length, self.sink_tokens) < 0:
            raise ValueError("block_size must be positive; residual_length and sink_tokens nonnegative")
        for name in ("validate_positions", "shared_workspace", "track_peak_bytes"):
            if type(getattr(self, name)) is not bool:
                raise ValueError(f"{name} must be a boolean")
        if self.value_bits not in (None, 2, 4) or type(self.value_bits) not in (type(None), int):
            raise ValueError("value_bits must be None, 2 or 4")
        if self.value_group_size not in (32, 64, 128) or type(self.value_group_size) is not int:
            raise ValueError("value_group_size must be 32, 64 or 128")


class PackedAttentionView(NamedTuple):
    """What one decode step attends to: the blocks sealed before this step,
    the exact sink, and the exact tail including the new token (cache.py:72-82).
    Immutable, with the reference's field names."""

    key_blocks: tuple
    value_blocks: tuple
    sink_key: torch.Tensor | None
    sink_value: torch.Tensor | None
    residual_key: torch.Tensor
    residual_value: torch.Tensor
    seq_length: int


class _Rows:
    """A [2, H, capacity, D] buffer of dense rows; keys at [0], values at [1]."""

    __slots__ = ("buf", "kbuf", "vbuf", "start", "count", "desc", "row_strides", "_views")

    def __init__(self, heads: int, capacity: int, dim: int, dtype: torch.dtype, device: torch.device):
        self.buf = torch.empty((2, heads, capacity, dim), dtype=dtype, device=device)
        self.kbuf, self.vbuf = self.buf[0:1], self.buf[1:2]      # [1, H, capacity, D] each
        self.start = 0
        self.count = 0
        self.desc = None            # ctypes descriptor of the append kernel
        self.row_strides = None     # (key strides, value strides) the descriptor holds
        self._views = {}            # (start, count) -> (keys, values): the buffer never moves

    @property
    def capacity(self) -> int:
        return self.buf.shape[2]

    def views(self) -> tuple:
        key = (self.start, self.count)
        pair = self._views.get(key)
        if pair is None:
            pair = self._views[key] = (self.kbuf.narrow(2, self.start, self.count),
                                       self.vbuf.narrow(2, self.start, self.count))
        return pair

    def keys(self) -> torch.Tensor:
        return self.views()[0]

    def values(self) -> torch.Tensor:
        return self.views()[1]

    def live_nbytes(self) -> int:
        return 2 * self.buf.shape[1] * self.count * self.buf.shape[3] * self.buf.element_size()

    def write(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Copy new rows after the live ones (host-ordered torch copies)."""
        n = keys.shape[2]
        if self.start + self.count + n > self.capacity:
            self.compact()
        end = self.start + self.count
        self.buf[0:1, :, end:end + n].copy_(keys)
        self.buf[1:2, :, end:end + n].copy_(values)

    def compact(self) -> None:
        if self.start:
            live = self.buf[:, :, self.start:self.start + self.count].clone()
            self.buf[:, :, :self.count].copy_(live)
            self.start = 0


class _LayerCache:
    """One layer's sink rows, dense tail rows and sealed blocks."""

    def __init__(self, shape, dtype, device):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.device = device
        self.seq_length = 0
        self.sink: _Rows | None = None
        self.tail: _Rows | None = None
        self.key_blocks: list = []
        self.value_blocks: list = []
        self.runs: list = []            # [first, stop) of the blocks of each seal (one batched encode)
        self.packed_nbytes = 0
        self.full_sink = None          # (keys, values) views once the sink holds all its rows
        self.block_tuples = None       # (key blocks, value blocks) as tuples, rebuilt after a seal
        self.seal_out = None           # outputs of the next one-block seal, carved ahead of it

    # the reference's field names, as views of the rows
    @property
    def sink_key(self):
        return None if self.sink is None else self.sink.keys()

    @property
    def sink_value(self):
        return None if self.sink is None else self.sink.values()

    @property
    def residual_key(self):
        return None if self.tail is None else self.tail.keys()

    @property
    def residual_value(self):
        return None if self.tail is None else self.tail.values()

    def dense_nbytes(self) -> tuple[int, int]:
        """(live sink bytes, live tail bytes)."""
        return (0 if self.sink is None else self.sink.live_nbytes(),
                0 if self.tail is None else self.tail.live_nbytes())

    def reserved_nbytes(self) -> int:
        """Bytes of the dense row buffers beyond their live rows."""
        held = sum(r.buf.numel() * r.buf.element_size() for r in (self.sink, self.tail) if r is not None)
        return held - sum(self.dense_nbytes())

    def seal_reserve_nbytes(self) -> int:
        """Bytes carved for the next seal's outputs (not yet a block)."""
        return 0 if self.seal_out is None else self.seal_out[0].untyped_storage().nbytes()


def _quantize_temporal_blocks(tensor: torch.Tensor, block_count: int, block_size: int,
                              config: CodecConfig, bad: torch.Tensor | None = None) -> list[PackedTensor]:
    """K4-encode the first ``block_count`` blocks of [1, H, T, D] as
    independent (block, head) rows (cache.py:89-119): one launch over the
    strided [blocks, H, B, D] view, one PackedTensor view per block.  With
    ``bad`` the non-finite flag is left there for the caller."""
    if block_count == 0:
        return []
    _, heads, _, dim = tensor.shape
    blocked = tensor[0, :, :block_count * block_size].unflatten(1, (block_count, block_size)).transpose(0, 1)
    packed = quantize(blocked, config, _flag=bad)
    return _per_block(packed, block_count, (1, heads, block_size, dim), PackedTensor)


_CARVE_PLANS: dict = {}


def _carve_plan(fields):
    """(total bytes, dtypes in first-use order, per field (dtype index, shape,
    strides, element offset)) of a field list; computed once per list."""
    plan = _CARVE_PLANS.get(fields)
    if plan is None:
        total, dtypes, views = 0, [], []
        for shape, dtype in fields:
            if dtype not in dtypes:
                dtypes.append(dtype)
            strides, acc = [], 1
            for n in reversed(shape):
                strides.append(acc)
                acc *= n
            views.append((dtypes.index(dtype), shape, tuple(strides[::-1]), total // dtype.itemsize))
            total += -(-math.prod(shape) * dtype.itemsize // 16) * 16
        plan = _CARVE_PLANS[fields] = (total, tuple(dtypes), tuple(views))
    return plan


def _carve(device, fields):
    """The seal's output tensors as views of one allocation, each starting on
    a 16-byte boundary for the encoders' vector stores ((shape, dtype) pairs
    in order).  The byte accounting counts each view's own bytes, as for
    separate allocations; the allocation holds at most 15 alignment bytes
    per field beyond them (none for 128-channel, 16-descriptor blocks)."""
    total, dtypes, views = _carve_plan(fields)
    raw = torch.empty(total, dtype=torch.uint8, device=device)
    typed = [raw.view(dtype) for dtype in dtypes]   # one reinterpretation per dtype
    return [torch.as_strided(typed[i], shape, strides, offset) for i, shape, strides, offset in views]


def _run_block(blocks, i: int, j: int):
    """blocks[i:j], the per-block views of one batched encode (consecutive
    equal-size slices of each field's allocation), as one batched
    [j - i, H, T, D] block over the same memory."""
    first = blocks[i]
    if j - i == 1:
        return first
    n = j - i
    fields = {name: torch.as_strided(t, (n, *t.shape[1:]), (t.numel(), *t.stride()[1:]), t.storage_offset())
              for name, t in first.tensors.items()}
    shape = (n, *first.shape[1:])
    if isinstance(first, PackedValues):
        return PackedValues(**fields, shape=shape, original_dtype=first.original_dtype, bits=first.bits,
                            group_size=first.group_size)
    return PackedTensor(**fields, shape=shape, original_dtype=first.original_dtype)


_SEAL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)   # what the batched seal encoders read
_STRIDES: dict = {}


def _block_strides(strides, T: int):
    """The encoders' (block, head, token, channel) element strides of the
    [blocks, H, T, D] view of a [1, H, tokens, D] tensor with these strides,
    as a ctypes array (one per stride pattern: the tail buffers' never change;
    the library only reads it)."""
    key = (strides, T)
    arr = _STRIDES.get(key)
    if arr is None:
        if len(_STRIDES) > 256:
            _STRIDES.clear()
        arr = _STRIDES[key] = (nat._i64 * 4)(T * strides[2], strides[1], strides[2], strides[3])
    return arr


def _seal_native(dim: int, bits: int | None, group_size: int) -> bool:
    """Whether a seal of this head size runs as one batched library call."""
    return dim % 2 == 0 and dim <= 1024 and (bits is None or dim % group_size == 0)


def _seal_fields(B: int, H: int, T: int, D: int, count: int, bits: int | None, group_size: int) -> tuple:
    """(shape, dtype) of a batched seal's outputs, in the encoder's argument
    order: the K4 keys' payload, scales, sources, donors and padding, then
    the group-wise values' payload, scales and offsets, or (bits None) the
    K4-coded values' five fields."""
    desc_dtype = torch.uint8 if D <= 256 else torch.int32
    k4 = (((B, H, T, D // 2), torch.uint8), ((B, H, D), torch.float32), ((B, H, count), desc_dtype),
          ((B, H, count), desc_dtype), ((B, H, count), torch.float32))
    if bits is None:
        return k4 + k4
    return k4 + (((B, H, T, D * bits // 8), torch.uint8), ((B, H, T, D // group_size), torch.float16),
                 ((B, H, T, D // group_size), torch.float16))


def _kv_blocks(keys: torch.Tensor, values: torch.Tensor, block_count: int, block_size: int, config: CodecConfig,
               bits: int, group_size: int, key_flag: torch.Tensor, value_flag: torch.Tensor, out=None):
    """K4 keys and group-wise values of the first ``block_count`` blocks of
    [1, H, T, D] in one library call (iq_kv_quantize: one launch for sealed
    256-token blocks of 128 16-bit channels, the two encoders back to back
    otherwise), with the per-block objects and flags of
    _quantize_temporal_blocks + _value_blocks (cache.py:288-295).  ``out``:
    the outputs as carved for _seal_fields, allocated beforehand."""
    if block_count == 0:
        return [], []
    _, heads, _, dim = keys.shape
    native = (keys.dtype == values.dtype and keys.dtype in _SEAL_DTYPES and keys.shape == values.shape
              and _seal_native(dim, bits, group_size))
    if not native:      # the separate encoders, with their own argument errors
        return (_quantize_temporal_blocks(keys, block_count, block_size, config, key_flag),
                _value_blocks(values, block_count, block_size, bits, group_size, value_flag))
    device = nat.require_gpu(keys, what="quantize")
    # the [blocks, H, B, D] view of the first blocks, as pointer and strides
    # (no view objects: the encoder reads them directly)
    B, H, T, D = block_count, heads, block_size, dim
    k_strides = _block_strides(keys.stride(), T)
    v_strides = _block_strides(values.stride(), T)
    count = math.floor(D * config.salient_fraction)
    payload, scales, src, don, padding, v_payload, v_scales, v_offsets = (
        out if out is not None else _carve(device, _seal_fields(B, H, T, D, count, bits, group_size)))
    nat.check(nat.lib().iq_kv_quantize(
        keys.data_ptr(), values.data_ptr(), nat.dtype_code(keys.dtype), k_strides, v_strides, B, H, T, D,
        count, config.sample_stride, int(config.donor_policy == "min_error"), payload.data_ptr(),
        scales.data_ptr(), src.data_ptr() if count else None, don.data_ptr() if count else None,
        src.element_size(), padding.data_ptr() if count else None, bits, group_size, v_payload.data_ptr(),
        v_scales.data_ptr(), v_offsets.data_ptr(), key_flag.data_ptr(), value_flag.data_ptr(),
        nat.stream_handle(device)))
    shape = (1, heads, block_size, dim)
    if B == 1:          # a seal's one block: the objects directly
        return ([PackedTensor(payload, scales, src, don, padding, shape, keys.dtype)],
                [PackedValues(v_payload, v_scales, v_offsets, shape, values.dtype, bits, group_size)])
    packed_k = PackedTensor(payload, scales, src, don, padding, (B, H, T, D), keys.dtype)
    packed_v = PackedValues(v_payload, v_scales, v_offsets, (B, H, T, D), values.dtype, bits, group_size)
    return (_per_block(packed_k, block_count, shape, PackedTensor),
            _per_block(packed_v, block_count, shape, PackedValues, bits=bits, group_size=group_size))


def _k4_pair_blocks(keys: torch.Tensor, values: torch.Tensor, block_count: int, block_size: int,
                    config: CodecConfig, key_flag: torch.Tensor, value_flag: torch.Tensor, out=None):
    """K4 keys and K4-coded values (value_bits None) of the first
    ``block_count`` blocks in one library call (iq_k4_quantize_kv: one launch
    for 16-bit blocks of 128 channels), with the per-block objects and flags
    of two _quantize_temporal_blocks calls (cache.py:288-291).  ``out`` as
    for _kv_blocks."""
    if block_count == 0:
        return [], []
    _, heads, _, dim = keys.shape
    native = (keys.dtype == values.dtype and keys.dtype in _SEAL_DTYPES and keys.shape == values.shape
              and _seal_native(dim, None, 0))
    if not native:      # the separate encodes, with their own argument errors
        return (_quantize_temporal_blocks(keys, block_count, block_size, config, key_flag),
                _quantize_temporal_blocks(values, block_count, block_size, config, value_flag))
    device = nat.require_gpu(keys, what="quantize")
    B, H, T, D = block_count, heads, block_size, dim
    k_strides = _block_strides(keys.stride(), T)
    v_strides = _block_strides(values.stride(), T)
    count = math.floor(D * config.salient_fraction)
    carved = out if out is not None else _carve(device, _seal_fields(B, H, T, D, count, None, 0))
    ko, vo = carved[:5], carved[5:]
    ptrs = lambda o: [o[0].data_ptr(), o[1].data_ptr()] + [t.data_ptr() if count else None for t in o[2:]]
    nat.check(nat.lib().iq_k4_quantize_kv(
        keys.data_ptr(), values.data_ptr(), nat.dtype_code(keys.dtype), k_strides, v_strides, B, H, T, D,
        count, config.sample_stride, int(config.donor_policy == "min_error"), *ptrs(ko), *ptrs(vo),
        ko[2].element_size(), key_flag.data_ptr(), value_flag.data_ptr(), nat.stream_handle(device)))
    shape = (1, heads, block_size, dim)
    if B == 1:          # a seal's one block: the objects directly
        return [PackedTensor(*ko, shape, keys.dtype)], [PackedTensor(*vo, shape, values.dtype)]
    return (_per_block(PackedTensor(*ko, (B, H, T, D), keys.dtype), block_count, shape, PackedTensor),
            _per_block(PackedTensor(*vo, (B, H, T, D), values.dtype), block_count, shape, PackedTensor))


class InQuantCache(_HFCache):
    """Immutable packed history, exact sink and a bounded exact tail
    (batch 1, append-only), as src/inquant/cache.py:122-419."""

    is_compileable = False

    def __init__(self, config: CacheConfig | None = None) -> None:
        try:
            super().__init__()
        except (TypeError, ValueError):
            super().__init__(layers=[])     # transformers >= 5 wants an explicit layer list
        self.config = config or CacheConfig()
        self._layers: dict[int, _LayerCache] = {}
        self._attention_states: dict[int, Any] = {}
        self._shared_decode_workspace = None
        self._seen_tokens = 0
        self.peak_nbytes = 0
        # running totals for track_peak_bytes: layer -> (owned, auxiliary)
        self._owned: dict[int, tuple[int, int]] = {}
        self._owned_total = 0
        self._flags: torch.Tensor | None = None          # int32 [3] on the cache's device
        self._position_checked: tuple | None = None      # (tensor, version, expected start) verified by a sync

    # ------------------------------------------------------------ HF protocol
    def __len__(self) -> int:
        return 1 + max(self._layers, default=-1)

    def __getitem__(self, layer_idx: int):
        return self.materialize(layer_idx)

    def __iter__(self):
        return (self.materialize(i) for i in range(len(self)))

    def get_seq_length(self, layer_idx: int | None = 0) -> int:
        layer = self._layers.get(layer_idx or 0)
        return layer.seq_length if layer is not None else 0

    def get_usable_length(self, new_seq_length: int, layer_idx: int | None = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_max_cache_shape(self, *args, **kwargs):
        return None

    def get_max_length(self):
        return None

    def get_mask_sizes(self, cache_position, layer_idx: int = 0):
        new = cache_position.numel() if isinstance(cache_position, torch.Tensor) else int(cache_position)
        return self.get_seq_length(layer_idx) + int(new), 0

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    # ------------------------------------------------------------ validation
    def _check(self, keys, values, layer_idx, cache_kwargs):
        """Argument checks of cache.py:202-240; returns (layer or None, position tensor or None)."""
        if type(layer_idx) is not int or layer_idx < 0:
            raise ValueError("layer_idx must be a nonnegative integer")
        shape = keys.shape
        if len(shape) != 4 or values.shape != shape:
            raise ValueError("K/V must have matching [batch, KV_heads, tokens, head_dim] shapes")
        if shape[0] != 1:
            raise NotImplementedError("InQuantCache currently supports batch size 1 only")
        if not (keys.is_floating_point() and values.is_floating_point()):
            raise ValueError("K/V must be floating-point tensors")
        dtype, device = keys.dtype, keys.device
        if values.dtype != dtype or values.device != device:
            raise ValueError("K/V must share dtype and device")
        if 0 in shape:
            raise ValueError("K/V dimensions must be nonempty")
        if shape[3] & 1:
            raise ValueError("Packed cache requires an even head dimension")
        layer = self._layers.get(layer_idx)
        if layer is not None and (shape[1] != layer.shape[1] or shape[3] != layer.shape[3]
                                  or dtype != layer.dtype or device != layer.device):
            raise ValueError("Layer shape, dtype and device must remain unchanged")
        position = cache_kwargs.get("cache_position") if cache_kwargs else None
        if position is not None and not (
                isinstance(position, torch.Tensor) and position.ndim == 1 and position.numel() == shape[2]
                and position.dtype in (torch.int32, torch.int64)):
            raise ValueError("cache_position must be a 1D integer tensor with one position per new token")
        return layer, position if self.config.validate_positions else None

    def _flag_words(self, device) -> torch.Tensor:
        if self._flags is None or self._flags.device != device:
            self._flags = torch.zeros(3, dtype=torch.int32, device=device)
        return self._flags

    def _host_position_check(self, position: torch.Tensor, start: int) -> None:
        """Synchronous comparison with start, start + 1, ... (raises before any change)."""
        host = position.cpu()
        wanted = torch.arange(start, start + host.numel(), dtype=host.dtype)
        flags = self._flags
        deferred = flags is not None and bool(flags[_POSITION_BAD].item())
        if deferred:
            flags[_POSITION_BAD].zero_()
        if deferred or not bool((host == wanted).all()):
            self._position_checked = None
            raise ValueError(_POSITION_ERROR)

    # ------------------------------------------------------------ updates
    @torch.no_grad()
    def update(self, key_states, value_states, layer_idx, cache_kwargs=None, *args, **kwargs):
        """Store new tokens; return the layer's full K/V (the inputs themselves
        on the first call, else dequantized history ++ the new tokens)."""
        layer, position = self._check(key_states, value_states, layer_idx, cache_kwargs)
        start = 0 if layer is None else layer.seq_length
        if position is not None:
            self._host_position_check(position, start)
        if layer is None:
            layer = _LayerCache(key_states.shape, key_states.dtype, key_states.device)
            result = (key_states, value_states)
        else:
            result = self._dense(layer, key_states, value_states)     # history ++ the new tokens
        self._ingest(layer, key_states, value_states)
        self._layers[layer_idx] = layer
        self._after_write(layer_idx, layer)
        return result

    def append_for_attention(self, key_states, value_states, layer_idx, cache_kwargs=None) -> PackedAttentionView:
        """Append one decode token and return the view that step attends to.

        Blocks sealed by this append are attended from the next step on
        (cache.py:242-269)."""
        layer, position = self._check(key_states, value_states, layer_idx, cache_kwargs)
        if layer is None or key_states.shape[2] != 1:
            raise ValueError("append_for_attention requires one new token after an existing prefill")
        blocks = layer.block_tuples
        if blocks is None:
            blocks = layer.block_tuples = (tuple(layer.key_blocks), tuple(layer.value_blocks))
        if layer.full_sink is not None and layer.tail is not None and key_states.is_cuda:
            view = self._append_token(layer, key_states, value_states, position, blocks, layer.full_sink)
        else:
            with torch.no_grad():      # the sink is still filling or nothing is dense yet
                view = self._append_general(layer, key_states, value_states, position, blocks)
        if layer_idx == 0:
            self._seen_tokens = layer.seq_length
        if self.config.track_peak_bytes:
            self.record_peak(layer_idx)
        return view

    def _append_general(self, layer, key_states, value_states, position, blocks) -> PackedAttentionView:
        if position is not None:
            self._host_position_check(position, layer.seq_length)
        sink = (layer.sink_key, layer.sink_value)
        before = (layer.residual_key, layer.residual_value)
        pending_k = key_states if before[0] is None else torch.cat((before[0], key_states), 2)
        pending_v = value_states if before[1] is None else torch.cat((before[1], value_states), 2)
        self._ingest(layer, key_states, value_states)
        return PackedAttentionView(*blocks, *sink, pending_k, pending_v, layer.seq_length)

    def _append_token(self, layer, key, value, position, blocks, sink) -> PackedAttentionView:
        """One row written in place by iq_tail_append; seal when the tail is full."""
        cfg = self.config
        tail = layer.tail
        flags = self._flag_words(key.device)
        start, count, capacity = tail.start, tail.count, tail.capacity
        shift = start + count + 1 > capacity
        if shift and start < count + 1:
            tail.compact()              # survivors and the new row would overlap: move them first
            start, shift = 0, False
        check_now = False
        pos_ptr, pos_bytes = None, 0
        if position is not None:
            if position.device.type != "cuda":
                self._host_position_check(position, layer.seq_length)
            else:
                pos_ptr, pos_bytes = position.data_ptr(), position.element_size()
                # a position tensor already verified against this start, and not
                # written since (same version counter), needs no second sync;
                # inference tensors keep no version counter (None)
                checked = self._position_checked
                check_now = not (checked is not None and checked[0] is position
                                 and checked[1] == _version(position) and checked[2] == layer.seq_length)
        desc = tail.desc
        if desc is None:
            buf = tail.buf
            desc = tail.desc = nat.TailDesc(buf.data_ptr(), buf.stride(0), buf.stride(1), buf.stride(2),
                                            buf.shape[1], buf.shape[3], capacity, buf.element_size(), 8,
                                            flags[_POSITION_BAD:].data_ptr())
        strides = (key.stride(), value.stride())
        if strides != tail.row_strides:
            desc.k_sh, desc.k_st, desc.v_sh, desc.v_st = strides[0][1], strides[0][2], strides[1][1], strides[1][2]
            tail.row_strides = strides
        if pos_bytes and pos_bytes != desc.pos_bytes:
            desc.pos_bytes = pos_bytes
        status = nat.tail_append_row(
            desc, key.data_ptr(), value.data_ptr(), count if shift else start + count, start if shift else 0,
            count if shift else 0, pos_ptr, layer.seq_length, torch._C._cuda_getCurrentRawStream(key.device.index))
        if status:
            nat.check(status)
        if shift:
            tail.start = start = 0
        seals = tail.count + 1 >= cfg.residual_length + cfg.block_size
        verified = (position, _version(position), layer.seq_length) if check_now else None
        if check_now and not seals:
            # the first layer of a step: raise now, before the row counts (an
            # append that seals reads this flag with the encoders' flags in
            # its one synchronization, position first, and raises the same way)
            if bool(flags[_POSITION_BAD].item()):
                flags[_POSITION_BAD].zero_()
                self._position_checked = None
                raise ValueError(_POSITION_ERROR)
            self._position_checked = verified
        tail.count += 1
        layer.seq_length += 1
        tail_k, tail_v = tail.views()
        view = PackedAttentionView(*blocks, *sink, tail_k, tail_v, layer.seq_length)
        if seals:
            out, layer.seal_out = layer.seal_out, None
            try:
                with torch.no_grad():
                    self._seal(layer, tail_k, tail_v, 1, out)
            except ValueError:
                tail.count -= 1                  # the reference leaves the layer unchanged on errors
                layer.seq_length -= 1
                layer.seal_out = out             # rewritten in full by the next seal
                raise
            if verified is not None:
                self._position_checked = verified
            tail.start += cfg.block_size
            tail.count -= cfg.block_size
        elif layer.seal_out is None and not torch.cuda.is_current_stream_capturing():
            # an append that does not seal (and is not being captured in a
            # graph) carves the next seal's outputs, so the seal launches its
            # encoder without allocating first
            heads, dim = layer.shape[1], layer.shape[3]
            if layer.dtype in _SEAL_DTYPES and _seal_native(dim, cfg.value_bits, cfg.value_group_size):
                count = math.floor(dim * cfg.codec.salient_fraction)
                layer.seal_out = _carve(layer.device, _seal_fields(1, heads, cfg.block_size, dim, count,
                                                                   cfg.value_bits, cfg.value_group_size))
        return view

    def _seal(self, layer, keys, values, count, out=None) -> None:
        """Encode the first ``count`` blocks of keys/values [1, H, >= count * B, D]
        and append them; non-finite data raise ValueError with the layer unchanged.
        The key and value encoders raise flags into one buffer read by a single
        synchronization (the reference syncs once per encoder, codec.py:197 and
        value_codec.py:64); a pending position mismatch is reported first."""
        cfg = self.config
        # the encoders only ever raise these words; they are zero here (every
        # error path below clears what it raised)
        flags = self._flag_words(keys.device)
        if cfg.value_bits is None:
            new_keys, new_values = _k4_pair_blocks(keys, values, count, cfg.block_size, cfg.codec,
                                                   flags[_KEY_BAD:_KEY_BAD + 1], flags[_VALUE_BAD:_VALUE_BAD + 1],
                                                   out)
            value_error = _BAD_K
        else:
            new_keys, new_values = _kv_blocks(keys, values, count, cfg.block_size, cfg.codec, cfg.value_bits,
                                              cfg.value_group_size, flags[_KEY_BAD:_KEY_BAD + 1],
                                              flags[_VALUE_BAD:_VALUE_BAD + 1], out)
            value_error = _BAD_V
        bad_key, bad_value, bad_position = flags.tolist()
        if bad_key or bad_value or bad_position:
            flags.zero_()
        if bad_position:
            self._position_checked = None
            raise ValueError(_POSITION_ERROR)
        if bad_key:
            raise ValueError(_BAD_K)
        if bad_value:
            raise ValueError(value_error)
        layer.runs.append((len(layer.key_blocks), len(layer.key_blocks) + len(new_keys)))
        layer.key_blocks.extend(new_keys)
        layer.value_blocks.extend(new_values)
        layer.block_tuples = None
        if cfg.track_peak_bytes:
            layer.packed_nbytes += sum(b.nbytes for b in new_keys) + sum(b.nbytes for b in new_values)

    def _ingest(self, layer: _LayerCache, keys, values) -> None:
        """General append of any number of tokens (cache.py:271-306 semantics)."""
        cfg = self.config
        _, heads, n, dim = keys.shape
        have = 0 if layer.sink is None else layer.sink.count
        take = min(cfg.sink_tokens - have, n)
        if take > 0:
            if layer.sink is None:
                layer.sink = _Rows(heads, cfg.sink_tokens, dim, keys.dtype, keys.device)
            layer.sink.write(keys[:, :, :take], values[:, :, :take])
        else:
            take = 0
        rest_k, rest_v = keys[:, :, take:], values[:, :, take:]
        m = n - take
        tail = layer.tail
        live = 0 if tail is None else tail.count
        blocks = max(0, (live + m - cfg.residual_length) // cfg.block_size)
        if blocks:
            pending_k = rest_k if not live else torch.cat((tail.keys(), rest_k), 2)
            pending_v = rest_v if not live else torch.cat((tail.values(), rest_v), 2)
            self._seal(layer, pending_k, pending_v, blocks)
            done = blocks * cfg.block_size
            rest_k, rest_v = pending_k[:, :, done:], pending_v[:, :, done:]
            m = live + m - done
            if tail is not None:
                tail.start = tail.count = 0
        if m > 0:
            if tail is None:
                tail = layer.tail = _Rows(heads, cfg.residual_length + cfg.block_size, dim, keys.dtype,
                                          keys.device)
            tail.write(rest_k, rest_v)
        if take:
            layer.sink.count += take
            if layer.sink.count == cfg.sink_tokens:
                layer.full_sink = (layer.sink.keys(), layer.sink.values())
        elif cfg.sink_tokens == 0 and layer.full_sink is None:
            layer.full_sink = (None, None)
        if m > 0:
            tail.count += rest_k.shape[2]
        layer.seq_length += n

    def _after_write(self, layer_idx: int, layer: _LayerCache) -> None:
        if layer_idx == 0:
            self._seen_tokens = layer.seq_length
        self.record_peak(layer_idx)

    def record_peak(self, layer_idx) -> None:
        """Update peak_nbytes with this layer's current persistent and auxiliary bytes."""
        if not self.config.track_peak_bytes:
            return
        layer = self._layers[layer_idx]
        state = self._attention_states.get(layer_idx)
        now = (layer.packed_nbytes + sum(layer.dense_nbytes()), 0 if state is None else state.nbytes)
        before = self._owned.get(layer_idx, (0, 0))
        self._owned[layer_idx] = now
        self._owned_total += sum(now) - sum(before)
        shared = self._shared_decode_workspace
        total = self._owned_total + (0 if shared is None else shared.nbytes)
        if total > self.peak_nbytes:
            self.peak_nbytes = total

    # ------------------------------------------------------------ reads
    @torch.no_grad()
    def materialize(self, layer_idx: int = 0):
        """Dense (keys, values) of one layer: sink ++ dequantized blocks ++ tail
        (not retained).  Blocks that are consecutive views of one batched
        encode (a prefill's blocks) dequantize in one launch per run, straight
        into their rows of the output (the cache records each seal's run)."""
        layer = self._layers.get(layer_idx)
        if layer is None:
            raise KeyError(f"No cached layer {layer_idx}")
        return self._dense(layer)

    def _dense(self, layer, new_keys=None, new_values=None):
        """sink ++ dequantized blocks ++ tail (++ new_keys / new_values, tokens
        not yet stored) of one layer, written once into fresh tensors."""
        _, heads, _, dim = layer.shape
        sink_n = 0 if layer.sink is None else layer.sink.count
        tail_n = 0 if layer.tail is None else layer.tail.count
        new_n = 0 if new_keys is None else new_keys.shape[2]
        out = []
        for side, blocks in ((0, layer.key_blocks), (1, layer.value_blocks)):
            total = sink_n + sum(b.shape[2] for b in blocks) + tail_n + new_n
            dense = torch.empty((1, heads, total, dim), dtype=layer.dtype, device=layer.device)
            at = 0
            if sink_n:
                rows = layer.sink
                dense[:, :, :sink_n].copy_(rows.buf[side:side + 1, :, rows.start:rows.start + sink_n])
                at = sink_n
            for i, j in layer.runs:
                n, T = j - i, blocks[i].shape[2]
                deq = _run_block(blocks, i, j).dequantize(dtype=layer.dtype)     # [n, H, T, D]
                dense[:, :, at:at + n * T].view(1, heads, n, T, dim).copy_(deq.permute(1, 0, 2, 3).unsqueeze(0))
                at += n * T
            if tail_n:
                dense[:, :, at:at + tail_n].copy_(layer.tail.keys() if side == 0 else layer.tail.values())
            if new_n:
                dense[:, :, at + tail_n:].copy_(new_keys if side == 0 else new_values)
            out.append(dense)
        return out[0], out[1]

    # ------------------------------------------------------------ accounting (cache.py:346-394)
    def _blocks(self):
        for layer in self._layers.values():
            yield from layer.key_blocks
            yield from layer.value_blocks

    @property
    def payload_nbytes(self) -> int:
        return sum(b.payload_nbytes for b in self._blocks())

    @property
    def metadata_nbytes(self) -> int:
        return sum(b.metadata_nbytes for b in self._blocks())

    @property
    def residual_nbytes(self) -> int:
        return sum(layer.dense_nbytes()[1] for layer in self._layers.values())

    @property
    def sink_nbytes(self) -> int:
        return sum(layer.dense_nbytes()[0] for layer in self._layers.values())

    @property
    def auxiliary_nbytes(self) -> int:
        shared = self._shared_decode_workspace
        return (0 if shared is None else shared.nbytes) + sum(s.nbytes for s in self._attention_states.values())

    @property
    def nbytes(self) -> int:
        """Live persistent bytes: packed blocks, exact sink and tail rows, decode state."""
        return self.payload_nbytes + self.metadata_nbytes + self.residual_nbytes + self.sink_nbytes \
            + self.auxiliary_nbytes

    @property
    def bf16_nbytes(self) -> int:
        return sum(2 * 2 * l.shape[1] * l.seq_length * l.shape[3] for l in self._layers.values())

    def memory_stats(self) -> dict:
        total, dense = self.nbytes, self.bf16_nbytes
        return {
            "nbytes": total,
            "peak_nbytes": self.peak_nbytes if self.config.track_peak_bytes else None,
            "payload_nbytes": self.payload_nbytes,
            "metadata_nbytes": self.metadata_nbytes,
            "residual_nbytes": self.residual_nbytes,
            "sink_nbytes": self.sink_nbytes,
            "auxiliary_nbytes": self.auxiliary_nbytes,
            "bf16_nbytes": dense,
            "quantized_layer_tokens": sum(b.shape[2] for l in self._layers.values() for b in l.key_blocks),
            "kv_reduction_vs_bf16": (1 - total / dense) if dense else 0.0,
            # preallocated dense rows not yet holding tokens (not part of nbytes)
            "dense_reserve_nbytes": sum(l.reserved_nbytes() for l in self._layers.values()),
            # outputs carved for each layer's next one-block seal (not part of nbytes)
            "seal_reserve_nbytes": sum(l.seal_reserve_nbytes() for l in self._layers.values()),
        }

    def reset(self) -> None:
        self._layers.clear()
        self._attention_states.clear()
        self._shared_decode_workspace = None
        self._owned.clear()
        self._owned_total = 0
        self.peak_nbytes = 0
        self._seen_tokens = 0
        self._flags = None
        self._position_checked = None

    def release(self) -> None:
        self.reset()

    def reorder_cache(self, beam_idx) -> None:
        raise NotImplementedError("Beam search/reordering is unsupported; use num_beams=1")

    def crop(self, max_length: int) -> None:
        raise NotImplementedError("Cache rollback/speculative decoding is unsupported; use append-only generation")

    def batch_repeat_interleave(self, repeats: int) -> None:
        raise NotImplementedError("Batch expansion is unsupported; use batch size 1")

    def batch_select_indices(self, indices) -> None:
        raise NotImplementedError("Batch selection is unsupported; use batch size 1")
