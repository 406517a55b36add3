"""Persistent bytes of the Hugging Face cache at the reference's published
point: Qwen2.5-7B (28 layers, 4 KV heads, head_dim 128), a 32,768-token
prompt and 128 decode tokens, the reference's 32K K4/V2 configuration
(configs/qwen2.5_7b_32k_latest_k4v2.json: blocks of 256, residual 128, sink
4, min_error donors, V2 with 64-channel groups, one shared decode workspace,
peak tracking).  The reference records 413,194,880 bytes of KV and decode
state for this workload (benchmarks/runtime_20260925.json:12, README.md:127,
cache.py:308-394 accounting)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

LAYERS, H, HQ, D = 28, 4, 28, 128
PROMPT, NEW = 32768, 128
REFERENCE_RECORDED = 413_194_880


def _closed_form(table_columns, dense_split):
    """Bytes of the cache after PROMPT + NEW tokens: sealed blocks (K4 payload,
    f32 scales, u8 source/donor descriptors, f32 padding; V2 payload, f16
    scales and offsets), the bf16 sink and tail, one decode state per layer
    (an int64 pointer table of `table_columns` columns and an int8 role map per
    block) and the shared fp32 workspace [Hq, partitions, 130], partitions =
    blocks + ceil(sink / split) + ceil(tail / split) at the longest tail."""
    sink = 4
    blocks = (PROMPT - sink - 128) // 256
    tail = PROMPT + NEW - sink - 256 * blocks
    key_block = H * (256 * 64 + 128 * 4 + 2 * 16 + 16 * 4)
    value_block = H * (256 * 32 + 2 * 256 * 2 * 2)
    per_layer = blocks * (key_block + value_block) + (sink + tail) * H * D * 2 * 2
    state = blocks * (table_columns * 8 + H * D)
    parts = blocks + -(-sink // dense_split) + -(-tail // dense_split)
    return LAYERS * (per_layer + state) + HQ * parts * 130 * 4, blocks, tail


def test_hf_cache_bytes_at_32k_plus_128_tokens_match_the_recorded_total():
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.qwen_fused import _layer_state
    cfg = CacheConfig(codec=CodecConfig(donor_policy="min_error"), value_bits=2, value_group_size=64,
                      shared_workspace=True, track_peak_bytes=True, validate_positions=False)
    cache = InQuantCache(cfg)
    g = torch.Generator(device="cuda").manual_seed(394)
    for layer in range(LAYERS):
        k = torch.randn((1, H, PROMPT, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((1, H, PROMPT, D), generator=g, device="cuda").to(torch.bfloat16)
        cache.update(k, v, layer)
    q = torch.randn((1, HQ, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    for step in range(NEW):
        if step % 32 == 0:
            print(f"cache bytes: decode step {step}", flush=True)
        t = torch.randn((1, H, 1, D), generator=g, device="cuda").to(torch.bfloat16)
        for layer in range(LAYERS):
            view = cache.append_for_attention(t, t, layer)
            state = _layer_state(cache, layer, view)
            state.decode(q, sink_key=view.sink_key, sink_value=view.sink_value, residual_key=view.residual_key,
                         residual_value=view.residual_value, output=out)
    torch.cuda.synchronize()
    stats = cache.memory_stats()
    ours, blocks, tail = _closed_form(8, 32)
    reference, _, _ = _closed_form(6, 256)
    assert (blocks, tail) == (127, 380)
    assert stats["quantized_layer_tokens"] == LAYERS * blocks * 256
    # this build's accounting equals its closed form exactly, and the
    # reference's closed form matches the recorded total to 0.02 %
    assert stats["nbytes"] == ours, (stats, ours)
    assert abs(reference - REFERENCE_RECORDED) / REFERENCE_RECORDED < 2e-4
    # the two deliberate differences: two more pointer-table columns (the K
    # source/donor descriptor addresses) and 32-token dense partitions in
    # the shared workspace
    delta = ours - reference
    assert delta == LAYERS * blocks * 2 * 8 + HQ * ((1 + 12) - (1 + 2)) * 130 * 4
    assert abs(ours - REFERENCE_RECORDED) / REFERENCE_RECORDED < 1e-3
    assert stats["peak_nbytes"] >= stats["nbytes"]
    print(f"cache bytes {stats['nbytes']} (reference closed form {reference}, recorded {REFERENCE_RECORDED}, "
          f"+{100 * (stats['nbytes'] / REFERENCE_RECORDED - 1):.3f} %)", flush=True)
