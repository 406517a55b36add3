"""Instance-local Qwen2.5 / Mistral single-token decode over packed KV (MI355X).

Drop-in for the reference's inquant.qwen_fused (qwen_fused.py:1-188): the
same entry points (enable_fused_attention / enable_fused_qwen2 /
enable_fused_mistral), handle (fused_decode_calls, cpu_reference_calls,
restore(), context manager) and eligibility rules.  Prefill, masked or
multi-token calls and other cache types keep the model's own forward; a
single-token step with an InQuantCache appends the token and runs the fused
HIP decode through PackedDecodeState.

The attention keyword is `past_key_value` in Transformers 4.53 and
`past_key_values` in 5.x; both are accepted.  There is no CPU decode path in
this build (the codec runs on the GPU only), so `allow_cpu_reference` keeps
its meaning for the head-size check but a CPU tensor still raises.
"""
from __future__ import annotations

import inspect
from dataclasses import dataclass
from types import MethodType
from typing import Any

import torch
import torch.nn.functional as F

from .cache import InQuantCache, PackedAttentionView


def _reference_decode(query: torch.Tensor, view: PackedAttentionView, scale: float) -> torch.Tensor:
    """Test oracle (qwen_fused.py:21-30): materializes every old block and runs SDPA in fp32."""
    def restore(sink, blocks, tail):
        pieces = [] if sink is None else [sink]
        pieces.extend(block.dequantize(dtype=query.dtype) for block in blocks)
        pieces.append(tail)
        return torch.cat(pieces, dim=2)
    key = restore(view.sink_key, view.key_blocks, view.residual_key)
    value = restore(view.sink_value, view.value_blocks, view.residual_value)
    groups = query.shape[1] // key.shape[1]
    key = key.float().repeat_interleave(groups, dim=1)
    value = value.float().repeat_interleave(groups, dim=1)
    return F.scaled_dot_product_attention(query.float(), key, value, scale=scale).to(query.dtype)


@dataclass
class _KernelState:
    kernel: Any

    @property
    def nbytes(self) -> int:
        return self.kernel.nbytes


@dataclass
class FusedQwen2Handle:
    """Owns only this model's forward overrides; restore removes them."""
    originals: list[tuple[Any, Any]]
    restored: bool = False

    @property
    def fused_decode_calls(self) -> int:
        return sum(getattr(module, "_inquant_fused_decode_calls", 0) for module, _ in self.originals)

    @property
    def cpu_reference_calls(self) -> int:
        return sum(getattr(module, "_inquant_cpu_reference_calls", 0) for module, _ in self.originals)

    def restore(self) -> None:
        if self.restored:
            return
        for module, original in self.originals:
            module.forward = original
            delattr(module, "_inquant_original_forward")
        self.restored = True

    def __enter__(self) -> "FusedQwen2Handle":
        return self

    def __exit__(self, *_args) -> None:
        self.restore()


def _cache_keyword(module) -> str:
    params = inspect.signature(module.forward).parameters
    if "past_key_values" in params:
        return "past_key_values"
    if "past_key_value" in params:
        return "past_key_value"
    raise RuntimeError("Unsupported Transformers attention interface; validated versions are 4.53.x and 5.x")


def enable_fused_attention(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Patch this instantiated model only; its weights and prefill forward stay.

    The accelerated path requires a ROCm device, head_dim=128, batch=1,
    q_len=1, full attention, no padding mask and an InQuantCache.  Other
    query lengths and cache types keep the original forward.
    """
    model_type = getattr(model.config, "model_type", None)
    if model_type == "qwen2":
        from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention as Attention, apply_rotary_pos_emb
    elif model_type == "mistral":
        from transformers.models.mistral.modeling_mistral import MistralAttention as Attention, apply_rotary_pos_emb
        if getattr(model.config, "sliding_window", None) is not None:
            raise ValueError("Mistral sliding-window attention requires a window-aware cache and is not supported")
    else:
        raise ValueError("Expected a dense Qwen2 or Mistral model")
    if model.training:
        raise ValueError("Call model.eval() before enabling inference-only packed decode")
    modules = [layer.self_attn for layer in model.model.layers]
    keyword = None
    for module in modules:
        if not isinstance(module, Attention):
            raise TypeError("Expected an unmodified attention instance for this model family")
        if hasattr(module, "_inquant_original_forward"):
            raise ValueError("This model already has fused InQuant decode enabled")
        if "position_embeddings" not in inspect.signature(module.forward).parameters:
            raise RuntimeError("Unsupported Transformers attention interface; validated versions are 4.53.x and 5.x")
        keyword = _cache_keyword(module)
        if getattr(module, "sliding_window", None) is not None:
            raise ValueError("Sliding-window attention is unsupported by packed decode")
        if not allow_cpu_reference and module.head_dim != 128:
            raise ValueError("The packed decode kernel currently requires head_dim=128")

    def forward(attention, hidden_states: torch.Tensor, position_embeddings, attention_mask=None, *args, **kwargs):
        cache = kwargs.get(keyword)
        cache_position = kwargs.get("cache_position")
        use_packed = (
            isinstance(cache, InQuantCache)
            and hidden_states.shape[1] == 1
            and cache.get_seq_length(attention.layer_idx) > 0
            and attention_mask is None
            and not kwargs.get("output_attentions", False)
        )
        if not use_packed:
            return attention._inquant_original_forward(hidden_states, position_embeddings, attention_mask,
                                                       *args, **kwargs)
        if attention.training or torch.is_grad_enabled():
            raise RuntimeError("Packed decode is inference-only; use model.eval() and torch.no_grad()")
        if hidden_states.shape[0] != 1:
            raise ValueError("Packed decode supports batch size 1 only")
        if hidden_states.device.type != "cuda":
            raise RuntimeError("Packed decode requires CUDA (ROCm) tensors; this build has no CPU decode path")
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, attention.head_dim)
        query = attention.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        key = attention.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        value = attention.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        query, key = apply_rotary_pos_emb(query, key, cos, sin)
        cache_kwargs = {"sin": sin, "cos": cos}
        if cache_position is not None:
            cache_kwargs["cache_position"] = cache_position
        view = cache.append_for_attention(key, value, attention.layer_idx, cache_kwargs)
        from .triton_attention import PackedDecodeState, SharedDecodeWorkspace
        if cache.config.shared_workspace and cache._shared_decode_workspace is None:
            cache._shared_decode_workspace = SharedDecodeWorkspace()
        state = cache._attention_states.get(attention.layer_idx)
        if state is None:
            state = _KernelState(PackedDecodeState(view.key_blocks, view.value_blocks,
                                                   workspace_pool=cache._shared_decode_workspace))
            cache._attention_states[attention.layer_idx] = state
        elif len(state.kernel.key_blocks) != len(view.key_blocks):
            state.kernel.extend(view.key_blocks, view.value_blocks)
        result = state.kernel.decode(query, sink_key=view.sink_key, sink_value=view.sink_value,
                                     residual_key=view.residual_key, residual_value=view.residual_value,
                                     scale=attention.scaling)
        cache.record_peak(attention.layer_idx)
        attention._inquant_fused_decode_calls += 1
        output = result.transpose(1, 2).reshape(*input_shape, -1).contiguous()
        return attention.o_proj(output), None

    originals = []
    for module in modules:
        originals.append((module, module.forward))
        module._inquant_original_forward = module.forward
        module._inquant_fused_decode_calls = 0
        module._inquant_cpu_reference_calls = 0
        module.forward = MethodType(forward, module)
    return FusedQwen2Handle(originals)


def enable_fused_qwen2(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Backward-compatible Qwen-only entry point."""
    if getattr(model.config, "model_type", None) != "qwen2":
        raise ValueError("Expected a dense Qwen2/Qwen2.5 model")
    return enable_fused_attention(model, allow_cpu_reference=allow_cpu_reference)


def enable_fused_mistral(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Mistral full-attention entry point; keeps the native projections and RoPE."""
    if getattr(model.config, "model_type", None) != "mistral":
        raise ValueError("Expected a dense Mistral model")
    return enable_fused_attention(model, allow_cpu_reference=allow_cpu_reference)
