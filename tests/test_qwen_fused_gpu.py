"""Qwen2 / Mistral adapters on the GPU: the patched single-token forward runs the
fused HIP decode and matches the model's own forward over the materialized
(dequantize-then-attend) cache (restates test_qwen_fused.py:112-146)."""
import copy
from unittest.mock import patch

import pytest
import torch

pytestmark = pytest.mark.gpu


def _qwen(head_dim=128, layers=1):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    return Qwen2ForCausalLM(Qwen2Config(
        vocab_size=97, hidden_size=4 * head_dim, intermediate_size=8 * head_dim, num_hidden_layers=layers,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=65536, bos_token_id=1,
        eos_token_id=96, pad_token_id=0, attn_implementation="sdpa")).eval()


def _mistral(layers=1):
    from transformers import MistralConfig, MistralForCausalLM
    return MistralForCausalLM(MistralConfig(
        vocab_size=97, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers, num_attention_heads=8,
        num_key_value_heads=2, head_dim=128, max_position_embeddings=65536, sliding_window=None,
        bos_token_id=1, eos_token_id=96, pad_token_id=0, attn_implementation="sdpa")).eval()


@pytest.mark.parametrize("family", ["qwen2", "mistral"])
@pytest.mark.parametrize("prefill_tokens", [3, 98])
def test_packed_kernel_logits_and_auxiliary_accounting(family, prefill_tokens):
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.qwen_fused import enable_fused_attention
    torch.manual_seed(37)
    model = (_qwen() if family == "qwen2" else _mistral()).to(device="cuda", dtype=torch.bfloat16)
    reference_model = copy.deepcopy(model)
    config = CacheConfig(CodecConfig(salient_fraction=.125), block_size=32, residual_length=4, sink_tokens=2)
    with enable_fused_attention(model) as handle, torch.no_grad():
        reference, packed = InQuantCache(config), InQuantCache(config)
        tokens = torch.randint(2, 90, (1, prefill_tokens), device="cuda")
        expected = reference_model(tokens, past_key_values=reference).logits
        actual = model(tokens, past_key_values=packed).logits
        assert torch.equal(actual, expected)
        for step in range(7):
            token = torch.tensor([[3 + step]], device="cuda")
            expected = reference_model(token, past_key_values=reference).logits
            with patch.object(packed, "materialize", side_effect=AssertionError("Unexpected full materialization")):
                actual = model(token, past_key_values=packed).logits
            torch.testing.assert_close(actual.float(), expected.float(), rtol=.035, atol=.012)
            assert packed.get_seq_length() == reference.get_seq_length()
        assert handle.fused_decode_calls == 7 and handle.cpu_reference_calls == 0
        assert packed.auxiliary_nbytes > 0
        stats = packed.memory_stats()
        assert stats["nbytes"] == sum(stats[name] for name in (
            "payload_nbytes", "metadata_nbytes", "residual_nbytes", "sink_nbytes", "auxiliary_nbytes"))
        if prefill_tokens == 3:
            assert stats["quantized_layer_tokens"] == 0
        packed.release()
        assert packed.auxiliary_nbytes == 0


def test_generate_patch_restore_and_rejections():
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.qwen_fused import enable_fused_mistral, enable_fused_qwen2
    torch.manual_seed(41)
    model = _qwen(layers=2).to(device="cuda", dtype=torch.bfloat16)
    original = model.model.layers[0].self_attn.forward
    config = CacheConfig(CodecConfig(salient_fraction=.125), block_size=16, residual_length=4, sink_tokens=2)
    handle = enable_fused_qwen2(model)
    tokens = torch.randint(2, 90, (1, 40), device="cuda")
    with torch.no_grad():
        generated = model.generate(tokens, attention_mask=torch.ones_like(tokens), past_key_values=InQuantCache(config),
                                   do_sample=False, num_beams=1, max_new_tokens=4, min_new_tokens=4)
    assert tuple(generated.shape) == (1, 44)
    with pytest.raises(ValueError, match="already"):
        enable_fused_qwen2(model)
    with pytest.raises(ValueError, match="Mistral"):
        enable_fused_mistral(model)
    handle.restore()
    handle.restore()
    assert model.model.layers[0].self_attn.forward == original
    model.train()
    with pytest.raises(ValueError, match="eval"):
        enable_fused_qwen2(model)
    with pytest.raises(ValueError, match="head_dim=128"):
        enable_fused_qwen2(_qwen(head_dim=64).to("cuda"))


def test_grad_mode_is_refused():
    from inquant.cache import InQuantCache
    from inquant.qwen_fused import enable_fused_qwen2
    model = _qwen().to(device="cuda", dtype=torch.bfloat16)
    cache = InQuantCache()
    with enable_fused_qwen2(model):
        with torch.no_grad():
            model(torch.tensor([[2, 3, 4]], device="cuda"), past_key_values=cache)
        with pytest.raises(RuntimeError, match="inference-only"):
            model(torch.tensor([[5]], device="cuda"), past_key_values=cache)


@pytest.mark.parametrize("value_bits", [None, 2])
def test_qwen_three_layers_shared_workspace_and_cache_reset(value_bits):
    # test_value_codec.py:124-159: three layers share one decode workspace
    # with bit-identical logits to per-layer workspaces, the byte accounting
    # differs by exactly the two saved workspaces, and reset drops the pool
    from dataclasses import replace
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.qwen_fused import enable_fused_qwen2
    torch.manual_seed(87)
    model = _qwen(layers=3).to(device="cuda", dtype=torch.bfloat16)
    original_model = copy.deepcopy(model)
    cfg = CacheConfig(CodecConfig(donor_policy="min_error"), block_size=32, residual_length=4, sink_tokens=2,
                      value_bits=value_bits, shared_workspace=True, track_peak_bytes=True)
    packed = InQuantCache(cfg)
    independent = InQuantCache(replace(cfg, shared_workspace=False))
    dense_ref = InQuantCache(cfg)
    tokens = torch.randint(0, 97, (1, 99), device="cuda")
    with enable_fused_qwen2(model), torch.inference_mode():
        for cache in (packed, independent):
            model(tokens, past_key_values=cache)
        original_model(tokens, past_key_values=dense_ref)
        for step in range(10):
            token = torch.tensor([[step + 3]], device="cuda")
            expected = model(token, past_key_values=independent).logits
            dense = original_model(token, past_key_values=dense_ref).logits
            with patch.object(packed, "materialize", side_effect=AssertionError("dense history not allowed")):
                actual = model(token, past_key_values=packed).logits
            torch.testing.assert_close(actual, expected, rtol=0, atol=0)
            torch.testing.assert_close(actual.float(), dense.float(), rtol=.035, atol=.015)
    per_layer = next(iter(independent._attention_states.values()))._workspace.untyped_storage().nbytes()
    assert independent.nbytes - packed.nbytes == 2 * per_layer
    for cache in (packed, independent):
        shared = cache._shared_decode_workspace.nbytes if cache._shared_decode_workspace else 0
        assert cache._owned_total + shared == cache.nbytes
        assert cache.peak_nbytes >= cache.nbytes
    old_pool = packed._shared_decode_workspace
    packed.reset()
    assert packed.nbytes == 0 and packed._shared_decode_workspace is None
    assert old_pool is not InQuantCache(cfg)._shared_decode_workspace


def test_mistral_v2_cache_logits_across_sealing_boundaries():
    # test_mistral_fused.py:12-40 (GPU case): two layers, K4 keys with V2
    # values, a 66-token prompt in 32-token blocks, eight decode steps that
    # cross a seal, restored attention forward afterwards
    from transformers import MistralConfig, MistralForCausalLM
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.qwen_fused import enable_fused_mistral
    torch.manual_seed(673)
    cfg = MistralConfig(vocab_size=97, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=32768,
                        sliding_window=None, rope_theta=1e6, bos_token_id=1, eos_token_id=96, pad_token_id=0,
                        attn_implementation="sdpa")
    model = MistralForCausalLM(cfg).to(device="cuda", dtype=torch.bfloat16).eval()
    ref = copy.deepcopy(model)
    cache_cfg = CacheConfig(CodecConfig(donor_policy="min_error"), block_size=32, residual_length=4, sink_tokens=4,
                            value_bits=2, value_group_size=64)
    original = model.model.layers[0].self_attn.forward
    with enable_fused_mistral(model) as handle, torch.no_grad():
        a, b = InQuantCache(cache_cfg), InQuantCache(cache_cfg)
        prompt = torch.randint(2, 90, (1, 66), device="cuda")
        torch.testing.assert_close(model(prompt, past_key_values=a).logits, ref(prompt, past_key_values=b).logits,
                                   atol=0, rtol=0)
        for i in range(8):
            token = torch.tensor([[i + 5]], device="cuda")
            expected = ref(token, past_key_values=b).logits
            with patch.object(a, "materialize", side_effect=AssertionError("dense fallback")):
                actual = model(token, past_key_values=a).logits
            torch.testing.assert_close(actual.float(), expected.float(), atol=.012, rtol=.035)
        assert handle.fused_decode_calls == 16 and handle.cpu_reference_calls == 0
    assert model.model.layers[0].self_attn.forward == original
