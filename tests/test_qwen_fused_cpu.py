"""Adapter behaviour that needs no GPU (test_qwen_fused.py:90-98): CPU inputs never
reach a silent CPU decode, and a CPU prefill that would seal a block is refused."""
import pytest
import torch

transformers = pytest.importorskip("transformers")


def _qwen(head_dim=128, layers=1):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    return Qwen2ForCausalLM(Qwen2Config(
        vocab_size=97, hidden_size=4 * head_dim, intermediate_size=8 * head_dim, num_hidden_layers=layers,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096, bos_token_id=1,
        eos_token_id=96, pad_token_id=0, attn_implementation="sdpa")).eval()


def test_default_does_not_silently_use_cpu_reference():
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.qwen_fused import enable_fused_qwen2
    model = _qwen()
    cache = InQuantCache()
    with enable_fused_qwen2(model) as handle, torch.no_grad():
        model(torch.tensor([[2, 3, 4]]), past_key_values=cache)        # prefill: dense sink/tail only
        with pytest.raises(RuntimeError, match="requires CUDA"):
            model(torch.tensor([[5]]), past_key_values=cache)
        assert cache.get_seq_length() == 3 and handle.fused_decode_calls == 0
        with pytest.raises(RuntimeError, match="ROCm GPU tensors"):  # a prefill that seals a block
            model(torch.randint(2, 90, (1, 12)), past_key_values=InQuantCache(CacheConfig(block_size=4,
                                                                                         residual_length=2)))


def test_model_family_and_mode_checks():
    from transformers import MistralConfig, MistralForCausalLM
    from inquant.qwen_fused import enable_fused_attention, enable_fused_mistral, enable_fused_qwen2
    with pytest.raises(ValueError, match="sliding-window"):
        enable_fused_mistral(MistralForCausalLM(MistralConfig(
            vocab_size=97, hidden_size=512, intermediate_size=512, num_hidden_layers=1, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, sliding_window=4096)).eval())
    model = _qwen()
    with pytest.raises(ValueError, match="Mistral"):
        enable_fused_mistral(model)
    with pytest.raises(ValueError, match="head_dim=128"):
        enable_fused_qwen2(_qwen(head_dim=64))
    handle = enable_fused_attention(_qwen(head_dim=64), allow_cpu_reference=True)
    handle.restore()
    model.train()
    with pytest.raises(ValueError, match="eval"):
        enable_fused_qwen2(model)
