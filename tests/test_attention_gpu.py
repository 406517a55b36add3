"""GPU parity of fused packed decode attention against the fp64
dequantize-then-attend oracle (qwen_fused.py:21-30 semantics).

Bar: max |out_fp32 - oracle| <= 2e-3, with keys and
values decoded and rounded to the query dtype exactly as the reference does.
"""
import numpy as np
import pytest
import torch

from kvcase import make_case, oracle_decode, to_np

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _decode_f32(state, case, scale=None):
    out = torch.empty(case.query.shape, dtype=torch.float32, device="cuda")
    state.decode(case.query, scale=scale, output=out, **case.kwargs())
    return to_np(out)[0, :, 0]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("fraction", [0.0, 0.125, 0.5])
@pytest.mark.parametrize("policy", ["neighbors", "min_error"])
def test_k4_values_with_sink_and_unsealed_tail(dtype, fraction, policy):
    # restates test_triton_attention.py:23-46 (K4-coded values, 281-token tail)
    from inquant.triton_attention import PackedDecodeState
    case = make_case(921, n_blocks=3, tail=281, dtype=dtype, fraction=fraction, policy=policy, value_bits=0)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    descriptor_bytes = state.nbytes
    got = _decode_f32(state, case)
    np.testing.assert_allclose(got, case.expected(), atol=ATOL, rtol=0)
    typed = state.decode(case.query, **case.kwargs())
    assert typed.shape == case.query.shape and typed.dtype == dtype and torch.isfinite(typed).all()
    # the typed result is the fp32 result rounded once
    expect_typed = torch.from_numpy(got).to("cuda").to(dtype).view_as(typed)
    assert torch.equal(typed, expect_typed)
    assert state.nbytes == descriptor_bytes + state._workspace.numel() * 4
    pointer = state._workspace.data_ptr()
    state.decode(case.query, **case.kwargs())
    assert state._workspace.data_ptr() == pointer


@pytest.mark.parametrize("bits,group", [(2, 32), (2, 64), (2, 128), (4, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k4v2_gqa_matches_oracle(bits, group, dtype):
    from inquant.triton_attention import PackedDecodeState
    case = make_case(125, n_blocks=2, sink=0, tail=267, dtype=dtype, value_bits=bits, group=group)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)
    assert state._value_map.numel() == 0


def test_qwen_shape_8k_context_cfg1():
    # config 1: 28 query heads over 4 KV heads, 32 packed blocks, 4 sink, 128 tail
    from inquant.triton_attention import PackedDecodeState
    case = make_case(1, n_blocks=32, sink=4, tail=128)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    got = _decode_f32(state, case)
    err = np.abs(got - case.expected()).max()
    assert err <= ATOL, err


def test_mistral_shape_dense_outliers_cfg3():
    # config 3 shape: G = 4 over 8 KV heads, 8% outliers in 3-wide runs
    from inquant.triton_attention import PackedDecodeState
    case = make_case(3, H=8, G=4, n_blocks=8, groups=(3, 3, 3, 1))
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


@pytest.mark.parametrize("tokens", [1, 4, 257])
def test_dense_only_before_any_block_is_sealed(tokens):
    from inquant.triton_attention import packed_decode, PackedDecodeState
    case = make_case(7, H=2, G=7, n_blocks=0, sink=0, tail=tokens)
    out = packed_decode(case.query, [], [], residual_key=case.tail_k, residual_value=case.tail_v)
    state = PackedDecodeState([], [])
    got = _decode_f32(state, case)
    np.testing.assert_allclose(got, case.expected(), atol=ATOL, rtol=0)
    assert torch.equal(out, torch.from_numpy(got).to("cuda").to(out.dtype).view_as(out))


def test_nondefault_block_length_and_no_dense_tensors():
    from inquant.triton_attention import PackedDecodeState
    case = make_case(41, H=1, G=3, n_blocks=1, block=41, sink=0, tail=0, dtype=torch.float16, value_bits=0)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


def test_extreme_softmax_and_zero_blocks_remain_finite():
    from inquant.codec import quantize
    from inquant.triton_attention import packed_decode
    key = torch.zeros((1, 1, 256, 128), device="cuda", dtype=torch.bfloat16)
    key[..., 0, :] = 30
    value = torch.randn(key.shape, device="cuda", dtype=torch.bfloat16)
    query = torch.full((1, 7, 1, 128), 20, device="cuda", dtype=torch.bfloat16)
    keys, values = [quantize(key)], [quantize(value)]
    out = packed_decode(query, keys, values)
    assert torch.isfinite(out).all()
    expected = oracle_decode(query, keys, values)
    np.testing.assert_allclose(to_np(out)[0, :, 0], expected, atol=ATOL + 2 ** -8 * np.abs(expected).max(), rtol=0)


def test_growing_tail_with_runtime_strides():
    # test_triton_attention.py:79-97: compact tails change head stride every step
    from inquant.triton_attention import PackedDecodeState
    case = make_case(79, n_blocks=1, sink=0, tail=192)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    for length in (129, 150, 192):
        tk = case.tail_k[:, :, :length].contiguous()
        tv = case.tail_v[:, :, :length].contiguous()
        out = torch.empty(case.query.shape, dtype=torch.float32, device="cuda")
        state.decode(case.query, residual_key=tk, residual_value=tv, output=out)
        exp = oracle_decode(case.query, case.key_blocks, case.value_blocks, tail_k=tk, tail_v=tv)
        np.testing.assert_allclose(to_np(out)[0, :, 0], exp, atol=ATOL, rtol=0)


def test_growing_state_matches_fresh_state_and_rejects_replacement():
    # test_incremental_state.py:8-34
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant.triton_attention import PackedDecodeState
    torch.manual_seed(831)
    keys, values = [], []
    state = PackedDecodeState([], [])
    q = torch.randn(1, 8, 1, 128, device="cuda", dtype=torch.bfloat16)
    for i in range(11):
        k = torch.randn(1, 2, 32, 128, device="cuda", dtype=torch.bfloat16)
        k[..., 127] *= 20
        keys.append(quantize(k, CodecConfig(donor_policy="min_error")))
        values.append(quantize_values(torch.randn_like(k)))
        state.extend(keys, values)
        fresh = PackedDecodeState(keys, values)
        assert torch.equal(state.decode(q), fresh.decode(q))
        assert state._key_map.dtype == torch.int8
        assert torch.equal(state._key_map[:i + 1], fresh._key_map[:i + 1])
        assert state.nbytes == sum(x.untyped_storage().nbytes() for x in
                                   (state._tables, state._key_map, state._value_map, state._workspace)
                                   if x is not None)
    with pytest.raises(ValueError, match="append-only"):
        state.extend(keys[:-1], values[:-1])
    with pytest.raises(ValueError, match="append-only"):
        state.extend(list(reversed(keys)), values)
    state.extend(keys, values)
    assert torch.equal(state.decode(q), fresh.decode(q))


def test_role_maps_and_tables_match_oracle():
    from oracle import oracle
    from inquant.triton_attention import PackedDecodeState
    case = make_case(5, n_blocks=3, value_bits=0)
    state = PackedDecodeState(case.key_blocks[:1], case.value_blocks[:1])
    state.extend(case.key_blocks, case.value_blocks)
    for i, (k, v) in enumerate(zip(case.key_blocks, case.value_blocks)):
        for blk, table in ((k, state._key_map), (v, state._value_map)):
            roles = oracle.role_map(blk.salient_channels[0].long().cpu().numpy(),
                                    blk.donor_channels[0].long().cpu().numpy())
            np.testing.assert_array_equal(table[i].cpu().numpy().astype(np.int16), roles)
        row = state._tables[i].cpu().tolist()
        assert row == [k.payload.data_ptr(), k.scales.data_ptr(), k.padding.data_ptr(), v.payload.data_ptr(),
                       v.scales.data_ptr(), v.padding.data_ptr(), k.salient_channels.data_ptr(),
                       k.donor_channels.data_ptr()]


def test_workspace_pool_is_shared_once_and_rejects_other_stream():
    from inquant.triton_attention import PackedDecodeState, SharedDecodeWorkspace
    pool = SharedDecodeWorkspace()
    q = torch.randn(1, 28, 1, 128, device="cuda", dtype=torch.bfloat16)
    k, v = [torch.randn(1, 4, 19, 128, device="cuda", dtype=torch.bfloat16) for _ in range(2)]
    states = [PackedDecodeState([], [], workspace_pool=pool) for _ in range(3)]
    for i, state in enumerate(states):
        out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
        state.decode(q, residual_key=k, residual_value=v + i, output=out)
        exp = oracle_decode(q, [], [], tail_k=k, tail_v=v + i)
        np.testing.assert_allclose(to_np(out)[0, :, 0], exp, atol=ATOL, rtol=0)
        assert state._workspace is None and state.nbytes == 0   # one partition: no merge counters
    assert pool.nbytes == 28 * 130 * 4
    first = pool.tensor.data_ptr()
    states[0].decode(q, residual_key=k, residual_value=v)
    assert pool.tensor.data_ptr() == first
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.Stream()):
        with pytest.raises(RuntimeError, match="one CUDA stream"):
            states[0].decode(q, residual_key=k, residual_value=v)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fraction", [0.0, 0.125, 0.5])
@pytest.mark.parametrize("block,sink,tail", [(256, 4, 128), (41, 0, 281), (32, 4, 0), (300, 3, 1),
                                              (64, 100, 300), (64, 300, 20)])
def test_matrix_core_path_matches_oracle(dtype, fraction, block, sink, tail):
    # bf16/f16 queries with V2 values take the MFMA kernel: partial tiles,
    # 0..64 salient channels, blocks longer than one 256-token pass
    from inquant.triton_attention import PackedDecodeState
    case = make_case(17 + block, n_blocks=3, block=block, sink=sink, tail=tail, dtype=dtype, fraction=fraction)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    got = _decode_f32(state, case)
    np.testing.assert_allclose(got, case.expected(), atol=ATOL, rtol=0)
    typed = state.decode(case.query, **case.kwargs())
    assert torch.equal(typed, torch.from_numpy(got).to("cuda").to(dtype).view_as(typed))


def _kernels_run(fn):
    """Names of the GPU kernels launched by fn()."""
    from torch.profiler import ProfilerActivity, profile
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return [e.name for e in prof.events() if e.device_type.name == "CUDA"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fraction,policy", [(0.0, "min_error"), (0.0625, "neighbors"), (0.125, "min_error"),
                                             (0.125, "neighbors")])
@pytest.mark.parametrize("block,sink,tail", [(256, 4, 128), (41, 0, 281), (32, 4, 0), (64, 300, 20)])
def test_k4_values_take_the_matrix_core_path(dtype, fraction, policy, block, sink, tail):
    # K4-coded values (CacheConfig's default, value_bits=None) with at most 16
    # salient channels decode on the matrix-core kernel: the value role map,
    # the 8-bit codes split across source and donor slots and the donor
    # padding, against the fp64 dequantize-then-attend oracle
    from inquant.triton_attention import PackedDecodeState
    case = make_case(31 + block, n_blocks=3, block=block, sink=sink, tail=tail, dtype=dtype, fraction=fraction,
                     policy=policy, value_bits=0)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    names = _kernels_run(lambda: _decode_f32(state, case))
    assert any("decode_fast" in n for n in names) and not any("decode_partials_generic" in n for n in names)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


def test_k4_values_peaked_attention_with_salient_value_outliers():
    # one dominant token whose value outlier channels (x40) are salient: their
    # 8-bit codes and the donor padding carry the output
    from inquant.codec import CodecConfig, quantize
    from inquant.triton_attention import PackedDecodeState
    from kvcase import oracle_decode
    import synth
    cfg = CodecConfig(salient_fraction=0.125, donor_policy="neighbors")
    k = torch.from_numpy(synth.kv_like(15, 4, 256)).cuda().to(torch.bfloat16)
    v = torch.from_numpy(synth.kv_like(16, 4, 256, scale=40.0)).cuda().to(torch.bfloat16)
    q = (k[:, :, 200:201, :].repeat_interleave(7, dim=1) * 0.5).contiguous()
    kp, vp = quantize(k, cfg), quantize(v, cfg)
    state = PackedDecodeState([kp], [vp])
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    state.decode(q, output=out)
    np.testing.assert_allclose(to_np(out)[0, :, 0], oracle_decode(q, [kp], [vp]), atol=ATOL, rtol=0)


def test_cfg2_full_context_with_k4_values_matches_oracle():
    # config 2 layer with the reference's default value codec (K4-coded values)
    from inquant.triton_attention import PackedDecodeState
    case = make_case(4, n_blocks=128, sink=4, tail=128, value_bits=0)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


def test_matrix_core_path_peaked_attention_keeps_precision():
    # one dominant token with large outlier values: P must keep more than
    # bf16 precision for the 2e-3 bound to hold
    from inquant.codec import quantize
    from inquant.value_codec import quantize_values
    from inquant.triton_attention import PackedDecodeState
    from kvcase import oracle_decode
    import synth
    k = torch.from_numpy(synth.kv_like(5, 4, 256)).cuda().to(torch.bfloat16)
    v = torch.from_numpy(synth.kv_like(6, 4, 256, scale=40.0)).cuda().to(torch.bfloat16)
    q = (k[:, :, 77:78, :].repeat_interleave(7, dim=1) * 0.5).contiguous()
    kp, vp = quantize(k), quantize_values(v)
    state = PackedDecodeState([kp], [vp])
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    state.decode(q, output=out)
    exp = oracle_decode(q, [kp], [vp])
    np.testing.assert_allclose(to_np(out)[0, :, 0], exp, atol=ATOL, rtol=0)


def test_cfg2_full_context_matches_oracle_and_is_repeatable():
    # config 2 layer: 128 packed blocks (32768 tokens) + 4 sink + 128 tail;
    # 130 partitions merged by the reduction kernel
    from inquant.triton_attention import PackedDecodeState
    case = make_case(2, n_blocks=128, sink=4, tail=128)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    outs = [_decode_f32(state, case) for _ in range(4)]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])            # the merge order is fixed
    np.testing.assert_allclose(outs[0], case.expected(), atol=ATOL, rtol=0)


@pytest.mark.parametrize("value_bits,dtype", [(2, torch.bfloat16), (0, torch.bfloat16), (2, torch.float16)])
def test_cfg3_full_context_grid_above_resident_capacity_matches_oracle(value_bits, dtype):
    # config 3 layer: 8 KV heads x (128 packed blocks + 5 dense
    # slices) = 1064 workgroups, more than fit at once (256 compute units x 4,
    # or x 3 with K4-coded values), so the dense slices take the first grid
    # rows; outliers in 3-wide runs
    from inquant.triton_attention import PackedDecodeState
    case = make_case(3, H=8, G=4, n_blocks=128, sink=4, tail=128, groups=(3, 3, 3, 1), value_bits=value_bits,
                     dtype=dtype)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    outs = [_decode_f32(state, case) for _ in range(2)]
    assert np.array_equal(outs[1], outs[0])
    np.testing.assert_allclose(outs[0], case.expected(), atol=ATOL, rtol=0)


@pytest.mark.parametrize("G", [1, 2, 8, 16])
@pytest.mark.parametrize("value_bits", [2, 0])
def test_query_group_sizes(G, value_bits):
    # one query row per KV head (G = 1) up to the 16 the matrix-core tiles
    # hold (all 16 columns live; the combine takes two passes over its rows)
    from inquant.triton_attention import PackedDecodeState
    case = make_case(13 + G, H=2, G=G, n_blocks=3, sink=4, tail=40, value_bits=value_bits)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


@pytest.mark.parametrize("n_blocks,tail", [(300, 100), (0, 5000)])
def test_merge_over_more_partitions_than_one_round(n_blocks, tail):
    # 304 and 157 partitions: the merge takes 144 per round, so its running
    # (max, sum, output) state is rescaled across rounds
    from inquant.triton_attention import PackedDecodeState
    case = make_case(11, H=2, G=4, n_blocks=n_blocks, block=16, sink=4, tail=tail)
    state = PackedDecodeState(case.key_blocks, case.value_blocks)
    np.testing.assert_allclose(_decode_f32(state, case), case.expected(), atol=ATOL, rtol=0)


def test_extend_checks_every_appended_block_and_keeps_the_state_on_error():
    # triton_attention.py:257-269: every appended block must match the first
    # block's shape, salient count and value quantizer; a rejected extend
    # leaves the state as it was
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant.triton_attention import PackedDecodeState
    torch.manual_seed(832)
    mk = lambda t=32: torch.randn(1, 2, t, 128, device="cuda", dtype=torch.bfloat16)
    keys = [quantize(mk()) for _ in range(3)]
    values = [quantize_values(mk()) for _ in range(3)]
    q = torch.randn(1, 8, 1, 128, device="cuda", dtype=torch.bfloat16)
    state = PackedDecodeState(keys[:2], values[:2])
    ref = state.decode(q).clone()
    cases = [
        (keys[:2] + [quantize(mk(16))], values, "shape"),
        (keys[:2] + [quantize(mk(), CodecConfig(salient_fraction=0.25))], values, "salient-channel"),
        (keys, values[:2] + [quantize_values(mk(), bits=4)], "same quantizer"),
        (keys, values[:2] + [quantize(mk())], "same quantizer"),
        (keys[:2] + [values[2]], values, "shape and salient-channel"),
    ]
    for ks, vs, msg in cases:
        with pytest.raises(ValueError, match=msg):
            state.extend(ks, vs)
        assert state.key_blocks == tuple(keys[:2]) and state.value_blocks == tuple(values[:2])
        assert torch.equal(state.decode(q), ref)
    state.extend(keys, values)
    assert torch.equal(state.decode(q), PackedDecodeState(keys, values).decode(q))
