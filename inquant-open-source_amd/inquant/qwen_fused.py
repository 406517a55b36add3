"""Packed single-token decode for Hugging Face Qwen2 / Mistral models (MI355X).

Drop-in for the reference's ``inquant.qwen_fused`` (src/inquant/qwen_fused.py):
``enable_fused_attention``, ``enable_fused_qwen2`` and ``enable_fused_mistral``
patch the attention modules of one model instance and return a handle with
``fused_decode_calls``, ``cpu_reference_calls``, ``restore()`` and context
manager support.  The eligibility rules and error messages are the
reference's; the structure is this build's own:

* every attention module gets a ``_PackedAttention`` object as its forward;
  it hands prefill, masked, multi-token and non-InQuant calls to the saved
  original forward untouched;
* an eligible decode step projects q/k/v, applies the model's RoPE, appends
  the token with ``InQuantCache.append_for_attention`` (one in-place tail
  write), brings the layer's ``PackedDecodeState`` up to date with the blocks
  sealed so far and runs the fused HIP decode, then ``o_proj``.

Transformers 4.53 passes the cache as ``past_key_value`` and 5.x as
``past_key_values``; the keyword is read from the module's signature.  There
is no CPU decode: a CPU step raises (``allow_cpu_reference`` only lifts the
head-size check, as in the reference).
"""
from __future__ import annotations

import importlib
import inspect
from typing import Any

import torch

from .cache import InQuantCache

_FAMILIES = {
    "qwen2": ("transformers.models.qwen2.modeling_qwen2", "Qwen2Attention"),
    "mistral": ("transformers.models.mistral.modeling_mistral", "MistralAttention"),
}
_INTERFACE_ERROR = "Unsupported Transformers attention interface; validated versions are 4.53.x and 5.x"


def _attention_family(model):
    """(attention class, apply_rotary_pos_emb) of a dense Qwen2 or Mistral model."""
    kind = getattr(model.config, "model_type", None)
    if kind not in _FAMILIES:
        raise ValueError("Expected a dense Qwen2 or Mistral model")
    if kind == "mistral" and getattr(model.config, "sliding_window", None) is not None:
        raise ValueError("Mistral sliding-window attention requires a window-aware cache and is not supported")
    module_name, class_name = _FAMILIES[kind]
    module = importlib.import_module(module_name)
    return getattr(module, class_name), module.apply_rotary_pos_emb


def _cache_keyword(forward) -> str:
    params = inspect.signature(forward).parameters
    if "position_embeddings" not in params:
        raise RuntimeError(_INTERFACE_ERROR)
    for name in ("past_key_values", "past_key_value"):
        if name in params:
            return name
    raise RuntimeError(_INTERFACE_ERROR)


def _layer_state(cache: InQuantCache, layer: int, view):
    """The layer's decode state, extended with blocks sealed since the last step."""
    from .triton_attention import PackedDecodeState, SharedDecodeWorkspace
    state = cache._attention_states.get(layer)
    if state is None:
        if cache.config.shared_workspace and cache._shared_decode_workspace is None:
            cache._shared_decode_workspace = SharedDecodeWorkspace()
        state = PackedDecodeState(view.key_blocks, view.value_blocks,
                                  workspace_pool=cache._shared_decode_workspace)
        cache._attention_states[layer] = state
    elif state.block_count != len(view.key_blocks):
        state.extend(view.key_blocks, view.value_blocks)
    return state


class _PackedAttention:
    """Forward of one patched attention module."""

    def __init__(self, module, rotary, cache_keyword: str):
        self.module = module
        self.rotary = rotary
        self.cache_keyword = cache_keyword
        self.own_forward = "forward" in vars(module)    # an instance attribute to put back on restore
        self.original = module.forward
        self.fused_calls = 0
        self.cpu_reference_calls = 0

    def __call__(self, hidden_states, position_embeddings, attention_mask=None, *args, **kwargs):
        cache = kwargs.get(self.cache_keyword)
        eligible = (isinstance(cache, InQuantCache) and hidden_states.shape[1] == 1
                    and attention_mask is None and not kwargs.get("output_attentions", False)
                    and cache.get_seq_length(self.module.layer_idx) > 0)
        if not eligible:
            return self.original(hidden_states, position_embeddings, attention_mask, *args, **kwargs)
        return self._step(cache, hidden_states, position_embeddings, kwargs.get("cache_position"))

    def _step(self, cache, hidden, position_embeddings, cache_position):
        attn = self.module
        if attn.training or torch.is_grad_enabled():
            raise RuntimeError("Packed decode is inference-only; use model.eval() and torch.no_grad()")
        if hidden.shape[0] != 1:
            raise ValueError("Packed decode supports batch size 1 only")
        if hidden.device.type != "cuda":
            raise RuntimeError("Packed decode requires CUDA (ROCm) tensors; this build has no CPU decode path")
        split = (1, 1, -1, attn.head_dim)
        q = attn.q_proj(hidden).view(split).transpose(1, 2)
        k = attn.k_proj(hidden).view(split).transpose(1, 2)
        v = attn.v_proj(hidden).view(split).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = self.rotary(q, k, cos, sin)
        extra = {"sin": sin, "cos": cos}
        if cache_position is not None:
            extra["cache_position"] = cache_position
        layer = attn.layer_idx
        view = cache.append_for_attention(k, v, layer, extra)
        out = _layer_state(cache, layer, view).decode(
            q, sink_key=view.sink_key, sink_value=view.sink_value, residual_key=view.residual_key,
            residual_value=view.residual_value, scale=attn.scaling)
        cache.record_peak(layer)
        self.fused_calls += 1
        # [1, Hq, 1, D] contiguous is already the [1, 1, Hq * D] row o_proj takes
        return attn.o_proj(out.view(1, 1, -1)), None

    def remove(self) -> None:
        if self.own_forward:
            self.module.forward = self.original
        else:
            del self.module.forward
        del self.module._inquant_patch


class FusedQwen2Handle:
    """The patches of one model; ``restore()`` (or leaving the ``with`` block) removes them."""

    def __init__(self, patches: list[_PackedAttention]):
        self._patches = patches
        self.restored = False

    @property
    def fused_decode_calls(self) -> int:
        return sum(p.fused_calls for p in self._patches)

    @property
    def cpu_reference_calls(self) -> int:
        return sum(p.cpu_reference_calls for p in self._patches)

    def restore(self) -> None:
        if not self.restored:
            for patch in self._patches:
                patch.remove()
            self.restored = True

    def __enter__(self) -> "FusedQwen2Handle":
        return self

    def __exit__(self, *exc) -> None:
        self.restore()


def enable_fused_attention(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Patch the attention modules of this model instance (weights and prefill untouched).

    Decode steps take the packed path when the cache is an InQuantCache, the
    batch and query length are 1, there is no attention mask and the module
    is not windowed; the HIP kernel needs head_dim 128."""
    attention_class, rotary = _attention_family(model)
    if model.training:
        raise ValueError("Call model.eval() before enabling inference-only packed decode")
    modules = [layer.self_attn for layer in model.model.layers]
    keywords = []
    for module in modules:
        if not isinstance(module, attention_class):
            raise TypeError("Expected an unmodified attention instance for this model family")
        if hasattr(module, "_inquant_patch"):
            raise ValueError("This model already has fused InQuant decode enabled")
        keywords.append(_cache_keyword(module.forward))
        if getattr(module, "sliding_window", None) is not None:
            raise ValueError("Sliding-window attention is unsupported by packed decode")
        if module.head_dim != 128 and not allow_cpu_reference:
            raise ValueError("The packed decode kernel currently requires head_dim=128")
    patches = []
    for module, keyword in zip(modules, keywords):
        patch = _PackedAttention(module, rotary, keyword)
        module._inquant_patch = patch
        module.forward = patch
        patches.append(patch)
    return FusedQwen2Handle(patches)


def enable_fused_qwen2(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Qwen2 / Qwen2.5 only."""
    if getattr(model.config, "model_type", None) != "qwen2":
        raise ValueError("Expected a dense Qwen2/Qwen2.5 model")
    return enable_fused_attention(model, allow_cpu_reference=allow_cpu_reference)


def enable_fused_mistral(model: Any, *, allow_cpu_reference: bool = False) -> FusedQwen2Handle:
    """Mistral with full attention only."""
    if getattr(model.config, "model_type", None) != "mistral":
        raise ValueError("Expected a dense Mistral model")
    return enable_fused_attention(model, allow_cpu_reference=allow_cpu_reference)
