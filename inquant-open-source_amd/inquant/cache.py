"""Append-only InQuant KV cache (drop-in for the reference's inquant.cache).

Per layer: an exact dense sink (first `sink_tokens` tokens), immutable K4
(and K4 or V2/V4) packed temporal blocks, and a dense recent tail of
`residual_length` .. `residual_length + block_size - 1` tokens.  Blocks are
sealed from the front of (tail ++ new) whenever at least
`residual_length + block_size` tokens are pending.  Semantics, validation and
byte accounting follow src/inquant/cache.py of the reference (CacheConfig
:24-54, _quantize_temporal_blocks :89-119, InQuantCache :122-419); the codec
work runs in libinquant_hip.so.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch

try:
    from transformers.cache_utils import Cache as _HFCache
except ImportError:  # codec/cache use does not need transformers
    class _HFCache:
        pass

from .codec import _BAD_K, CodecConfig, PackedTensor, quantize
from .value_codec import _BAD_V, _value_blocks


@dataclass(frozen=True)
class CacheConfig:
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
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int):
                raise ValueError(f"{name} must be an integer")
        if self.block_size < 1 or self.residual_length < 0 or self.sink_tokens < 0:
            raise ValueError("block_size must be positive; residual_length and sink_tokens nonnegative")
        for name in ("validate_positions", "shared_workspace", "track_peak_bytes"):
            if not isinstance(getattr(self, name), bool):
                raise ValueError(f"{name} must be a boolean")
        if self.value_bits is not None and (type(self.value_bits) is not int or self.value_bits not in (2, 4)):
            raise ValueError("value_bits must be None, 2 or 4")
        if type(self.value_group_size) is not int or self.value_group_size not in (32, 64, 128):
            raise ValueError("value_group_size must be 32, 64 or 128")


@dataclass
class _Layer:
    shape: tuple
    dtype: torch.dtype
    device: torch.device
    seq_length: int = 0
    sink_key: torch.Tensor | None = None
    sink_value: torch.Tensor | None = None
    residual_key: torch.Tensor | None = None
    residual_value: torch.Tensor | None = None
    key_blocks: list = field(default_factory=list)
    value_blocks: list = field(default_factory=list)
    packed_nbytes: int = 0


@dataclass(frozen=True)
class PackedAttentionView:
    """Snapshot for one decode: old packed blocks plus the exact sink and tail (with the new token)."""

    key_blocks: tuple
    value_blocks: tuple
    sink_key: torch.Tensor | None
    sink_value: torch.Tensor | None
    residual_key: torch.Tensor
    residual_value: torch.Tensor
    seq_length: int


def _tensor_bytes(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _quantize_temporal_blocks(tensor: torch.Tensor, block_count: int, block_size: int,
                              config: CodecConfig, bad: torch.Tensor | None = None) -> list[PackedTensor]:
    """Encode `block_count` leading blocks of [1, H, T, D] in one launch, one owned PackedTensor each.

    The blocked [nb, H, B, D] view is read in place by the kernel (no copy);
    statistics stay per (block, head).  With `bad` given, the non-finite flag
    goes to bad[0] and is left for the caller to check.
    """
    if block_count == 0:
        return []
    if block_count == 1:
        return [quantize(tensor[:, :, :block_size], config, _flag=bad)]
    _, heads, _, channels = tensor.shape
    blocked = tensor[0, :, :block_count * block_size].reshape(heads, block_count, block_size, channels).permute(1, 0, 2, 3)
    packed = quantize(blocked, config, _flag=bad)
    shape = (1, heads, block_size, channels)
    return [PackedTensor(**{name: t[i:i + 1].clone(memory_format=torch.contiguous_format)
                            for name, t in packed.tensors.items()},
                         shape=shape, original_dtype=tensor.dtype)
            for i in range(block_count)]


class InQuantCache(_HFCache):
    """Immutable quantized history plus exact sink and a bounded recent tail (batch 1, append-only)."""

    is_compileable = False

    def __init__(self, config: CacheConfig | None = None) -> None:
        try:
            super().__init__()
        except (TypeError, ValueError):
            super().__init__(layers=[])  # transformers >= 5 requires an explicit layer list
        self.config = config or CacheConfig()
        self._layers: dict[int, _Layer] = {}
        self._attention_states: dict[int, Any] = {}
        self._shared_decode_workspace = None
        self._tracked_storage: dict[int, int] = {}
        self._tracked_auxiliary: dict[int, int] = {}
        self._tracked_live_bytes = 0
        self._tracked_aux_bytes = 0
        self.peak_nbytes = 0
        self._seen_tokens = 0
        # (tensor, its in-place version, expected first position) of the last
        # cache_position that passed the check
        self._checked_position = None

    # ---- Hugging Face cache protocol
    def __len__(self) -> int:
        return max(self._layers, default=-1) + 1

    def __getitem__(self, layer_idx: int):
        return self.materialize(layer_idx)

    def __iter__(self):
        for idx in range(len(self)):
            yield self.materialize(idx)

    def get_seq_length(self, layer_idx: int | None = 0) -> int:
        layer = self._layers.get(0 if layer_idx is None else layer_idx)
        return 0 if layer is None else layer.seq_length

    def get_usable_length(self, new_seq_length: int, layer_idx: int | None = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_max_cache_shape(self, *args, **kwargs):
        return None

    def get_max_length(self):
        return None

    def get_mask_sizes(self, cache_position, layer_idx: int = 0):
        n = int(cache_position.numel()) if isinstance(cache_position, torch.Tensor) else int(cache_position)
        return self.get_seq_length(layer_idx) + n, 0

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    # ---- updates
    @torch.no_grad()
    def update(self, key_states, value_states, layer_idx, cache_kwargs=None, *args, **kwargs):
        layer = self._validate_update(key_states, value_states, layer_idx, cache_kwargs)
        if layer is None:
            layer = _Layer(tuple(key_states.shape), key_states.dtype, key_states.device)
            full_key, full_value = key_states, value_states
        else:
            old_key, old_value = self.materialize(layer_idx)
            full_key = torch.cat((old_key, key_states), dim=2)
            full_value = torch.cat((old_value, value_states), dim=2)
        self._append(layer, key_states, value_states)
        self._layers[layer_idx] = layer
        self.record_peak(layer_idx)
        if layer_idx == 0:
            self._seen_tokens = layer.seq_length
        return full_key, full_value

    def _validate_update(self, key_states, value_states, layer_idx, cache_kwargs):
        if not isinstance(layer_idx, int) or layer_idx < 0:
            raise ValueError("layer_idx must be a nonnegative integer")
        if key_states.ndim != 4 or value_states.shape != key_states.shape:
            raise ValueError("K/V must have matching [batch, KV_heads, tokens, head_dim] shapes")
        if key_states.shape[0] != 1:
            raise NotImplementedError("InQuantCache currently supports batch size 1 only")
        if not key_states.is_floating_point() or not value_states.is_floating_point():
            raise ValueError("K/V must be floating-point tensors")
        if key_states.dtype != value_states.dtype or key_states.device != value_states.device:
            raise ValueError("K/V must share dtype and device")
        if any(size < 1 for size in key_states.shape):
            raise ValueError("K/V dimensions must be nonempty")
        if key_states.shape[3] % 2:
            raise ValueError("Packed cache requires an even head dimension")
        layer = self._layers.get(layer_idx)
        old_length = 0 if layer is None else layer.seq_length
        if layer is not None:
            same = (key_states.shape[0], key_states.shape[1], key_states.shape[3]) == (
                layer.shape[0], layer.shape[1], layer.shape[3])
            if not same or key_states.dtype != layer.dtype or key_states.device != layer.device:
                raise ValueError("Layer shape, dtype and device must remain unchanged")
        position = (cache_kwargs or {}).get("cache_position")
        if position is not None:
            if (not isinstance(position, torch.Tensor) or position.ndim != 1
                    or position.numel() != key_states.shape[2] or position.dtype not in (torch.int32, torch.int64)):
                raise ValueError("cache_position must be a 1D integer tensor with one position per new token")
            # Inference-mode tensors keep no in-place version counter, so they
            # are checked every time.
            version = None if position.is_inference() else position._version
            checked = self._checked_position
            if self.config.validate_positions and not (
                    version is not None and checked is not None and checked[0] is position
                    and checked[1] == version and checked[2] == old_length):
                # Compared on the host: one copy instead of two kernels and a
                # reduction.  The layers of one decode step share the step's
                # cache_position tensor and expect the same first position,
                # so a tensor that already passed, unmodified since (its
                # in-place version counter is unchanged), for the same
                # expected start is not copied again; the device-to-host copy
                # waits for all queued GPU work.
                host = position.cpu()
                if host.numel() == 1:
                    ok = int(host[0]) == old_length
                else:
                    ok = torch.equal(host, torch.arange(old_length, old_length + key_states.shape[2],
                                                        dtype=position.dtype))
                if not ok:
                    raise ValueError("Only contiguous append positions are supported; reset before a new request")
                self._checked_position = None if version is None else (position, version, old_length)
        return layer

    @torch.no_grad()
    def append_for_attention(self, key_states, value_states, layer_idx, cache_kwargs=None) -> PackedAttentionView:
        """Append one token and return the pre-seal view (blocks sealed now are seen next step)."""
        layer = self._validate_update(key_states, value_states, layer_idx, cache_kwargs)
        if key_states.shape[2] != 1 or layer is None:
            raise ValueError("append_for_attention requires one new token after an existing prefill")
        blocks = (tuple(layer.key_blocks), tuple(layer.value_blocks))
        sink = (layer.sink_key, layer.sink_value)
        length = layer.seq_length + 1
        sink_full = (0 if sink[0] is None else sink[0].shape[2]) >= self.config.sink_tokens
        if sink_full and layer.residual_key is not None:
            # the pre-seal tail is exactly the concatenation the append builds
            tail_key, tail_value = self._append(layer, key_states, value_states)
        else:
            tail_key, tail_value = key_states, value_states
            if layer.residual_key is not None:
                tail_key = torch.cat((layer.residual_key, tail_key), dim=2)
                tail_value = torch.cat((layer.residual_value, tail_value), dim=2)
            self._append(layer, key_states, value_states)
        view = PackedAttentionView(blocks[0], blocks[1], sink[0], sink[1], tail_key, tail_value, length)
        self.record_peak(layer_idx)
        if layer_idx == 0:
            self._seen_tokens = layer.seq_length
        return view

    def _append(self, layer: _Layer, keys, values) -> None:
        cfg = self.config
        have = 0 if layer.sink_key is None else layer.sink_key.shape[2]
        take = min(cfg.sink_tokens - have, keys.shape[2])
        sink_key, sink_value = layer.sink_key, layer.sink_value
        if take:
            nk, nv = keys[:, :, :take], values[:, :, :take]
            if sink_key is not None:
                nk = torch.cat((sink_key, nk), dim=2)
                nv = torch.cat((sink_value, nv), dim=2)
            sink_key, sink_value = nk.clone(), nv.clone()
        pending_key, pending_value = keys[:, :, take:], values[:, :, take:]
        fresh = layer.residual_key is not None      # pending is a new tensor, not a view of the input
        if fresh:
            pending_key = torch.cat((layer.residual_key, pending_key), dim=2)
            pending_value = torch.cat((layer.residual_value, pending_value), dim=2)
        blocks = max(0, (pending_key.shape[2] - cfg.residual_length) // cfg.block_size)
        # Both encoders raise their non-finite flag into one buffer that is
        # read with a single device sync; the reference syncs once per
        # encoder (codec.py:197, value_codec.py:64).  The key error wins, as
        # the reference raises it before encoding the values.
        flags = torch.zeros(2, dtype=torch.int32, device=keys.device) if blocks else None
        new_keys = _quantize_temporal_blocks(pending_key, blocks, cfg.block_size, cfg.codec,
                                             flags[0:1] if blocks else None)
        if cfg.value_bits is None:
            new_values = _quantize_temporal_blocks(pending_value, blocks, cfg.block_size, cfg.codec,
                                                   flags[1:2] if blocks else None)
            bad_v = _BAD_K
        else:
            new_values = _value_blocks(pending_value, blocks, cfg.block_size, cfg.value_bits,
                                       cfg.value_group_size, flags[1:2] if blocks else None)
            bad_v = _BAD_V
        if blocks:
            bad_k_set, bad_v_set = flags.tolist()
            if bad_k_set:
                raise ValueError(_BAD_K)
            if bad_v_set:
                raise ValueError(bad_v)
        offset = blocks * cfg.block_size
        if fresh and offset == 0:
            # nothing sealed: the concatenation is already an owned tensor
            residual_key, residual_value = pending_key, pending_value
        else:
            residual_key = pending_key[:, :, offset:].clone()
            residual_value = pending_value[:, :, offset:].clone()
        layer.sink_key, layer.sink_value = sink_key, sink_value
        layer.residual_key, layer.residual_value = residual_key, residual_value
        layer.key_blocks.extend(new_keys)
        layer.value_blocks.extend(new_values)
        if cfg.track_peak_bytes:
            layer.packed_nbytes += sum(block.nbytes for block in new_keys + new_values)
        layer.seq_length += keys.shape[2]
        return pending_key, pending_value

    def record_peak(self, layer_idx) -> None:
        if not self.config.track_peak_bytes:
            return
        layer = self._layers[layer_idx]
        owned = layer.packed_nbytes + sum(_tensor_bytes(t) for t in (
            layer.sink_key, layer.sink_value, layer.residual_key, layer.residual_value))
        self._tracked_live_bytes += owned - self._tracked_storage.get(layer_idx, 0)
        self._tracked_storage[layer_idx] = owned
        state = self._attention_states.get(layer_idx)
        aux = 0 if state is None else state.nbytes
        self._tracked_aux_bytes += aux - self._tracked_auxiliary.get(layer_idx, 0)
        self._tracked_auxiliary[layer_idx] = aux
        shared = 0 if self._shared_decode_workspace is None else self._shared_decode_workspace.nbytes
        self.peak_nbytes = max(self.peak_nbytes, self._tracked_live_bytes + self._tracked_aux_bytes + shared)

    @torch.no_grad()
    def materialize(self, layer_idx: int = 0):
        """Dense reconstruction of one layer (not retained by the cache)."""
        if layer_idx not in self._layers:
            raise KeyError(f"No cached layer {layer_idx}")
        layer = self._layers[layer_idx]

        def restore(sink, blocks, tail):
            pieces = [] if sink is None else [sink]
            pieces.extend(block.dequantize(dtype=layer.dtype) for block in blocks)
            if tail is not None:
                pieces.append(tail)
            return torch.cat(pieces, dim=2)

        return (restore(layer.sink_key, layer.key_blocks, layer.residual_key),
                restore(layer.sink_value, layer.value_blocks, layer.residual_value))

    # ---- accounting
    @property
    def payload_nbytes(self) -> int:
        return sum(b.payload_nbytes for layer in self._layers.values() for b in layer.key_blocks + layer.value_blocks)

    @property
    def metadata_nbytes(self) -> int:
        return sum(b.metadata_nbytes for layer in self._layers.values()
                   for b in layer.key_blocks + layer.value_blocks)

    @property
    def residual_nbytes(self) -> int:
        return sum(_tensor_bytes(l.residual_key) + _tensor_bytes(l.residual_value) for l in self._layers.values())

    @property
    def sink_nbytes(self) -> int:
        return sum(_tensor_bytes(l.sink_key) + _tensor_bytes(l.sink_value) for l in self._layers.values())

    @property
    def auxiliary_nbytes(self) -> int:
        shared = 0 if self._shared_decode_workspace is None else self._shared_decode_workspace.nbytes
        return shared + sum(state.nbytes for state in self._attention_states.values())

    @property
    def nbytes(self) -> int:
        return (self.payload_nbytes + self.metadata_nbytes + self.residual_nbytes + self.sink_nbytes
                + self.auxiliary_nbytes)

    @property
    def bf16_nbytes(self) -> int:
        return sum(4 * l.shape[0] * l.shape[1] * l.seq_length * l.shape[3] for l in self._layers.values())

    def memory_stats(self) -> dict:
        total, baseline = self.nbytes, self.bf16_nbytes
        return {
            "nbytes": total,
            "peak_nbytes": self.peak_nbytes if self.config.track_peak_bytes else None,
            "payload_nbytes": self.payload_nbytes,
            "metadata_nbytes": self.metadata_nbytes,
            "residual_nbytes": self.residual_nbytes,
            "sink_nbytes": self.sink_nbytes,
            "auxiliary_nbytes": self.auxiliary_nbytes,
            "bf16_nbytes": baseline,
            "quantized_layer_tokens": sum(b.shape[2] for l in self._layers.values() for b in l.key_blocks),
            "kv_reduction_vs_bf16": 1 - total / baseline if baseline else 0.0,
        }

    def reset(self) -> None:
        self._layers.clear()
        self._attention_states.clear()
        self._shared_decode_workspace = None
        self._tracked_storage.clear()
        self._tracked_auxiliary.clear()
        self._tracked_live_bytes = self._tracked_aux_bytes = self.peak_nbytes = 0
        self._seen_tokens = 0
        self._checked_position = None

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
