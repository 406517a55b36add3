"""Pins the CPU restatement (oracle/) before it is trusted as the GPU parity checker.

Each check is independent of the oracle's own formulas: golden vectors written
by the reference implementation, the reference tests' known answers, torch's
CPU reductions (whose order the reference inherits), numpy/torch format
conversions, closed forms and invariants.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from recipes import K4_CASES, build_input
import synth

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(GOLDEN_DIR, "k4_quantize.json")) as f:
        meta = json.load(f)["cases"]
    arrays = np.load(os.path.join(GOLDEN_DIR, "k4_quantize.npz"))
    return meta, arrays


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("name", sorted(K4_CASES))
def test_oracle_matches_reference_golden_vectors(golden, name):
    meta, arrays = golden
    recipe, cfg = K4_CASES[name]
    x = build_input(recipe)
    assert hashlib.sha256(x.tobytes()).hexdigest() == meta[name]["input_sha256"], "input generator drifted"
    out = oracle.k4_quantize(x, **cfg)
    assert hashlib.sha256(out["payload"].tobytes()).hexdigest() == meta[name]["payload_sha256"]
    for field in ("scales", "salient_channels", "donor_channels", "padding"):
        np.testing.assert_array_equal(_bits(out[field]), _bits(arrays[f"{name}/{field}"]), err_msg=field)


@pytest.mark.parametrize("D", [2, 6, 8, 16, 34, 66, 96, 128, 130, 258])
def test_stats_follow_torch_cpu_reduction_order(D):
    gen = torch.Generator().manual_seed(D)
    for T, stride in [(1, 8), (41, 8), (256, 8), (300, 7), (4100, 1)]:
        x = (torch.randn(T, D, generator=gen) * torch.exp(torch.randn(T, 1, generator=gen) * 3)).float()
        s = x[::stride]
        var, mean = torch.var_mean(x, 0, correction=0)
        smean = s.mean(0)
        expected = [s.abs().mean(0), smean, var + (mean - smean).square(), x.abs().amax(0)]
        got = oracle.k4_stats(x.numpy(), stride, True)
        for name, a, b in zip(("saliency", "sampled_mean", "error", "amax"), got, expected):
            np.testing.assert_array_equal(_bits(a), _bits(b.numpy()), err_msg=f"{name} T={T} stride={stride}")


def test_adjacent_run_known_answer():
    # test_codec.py:36-45: channels 6..9 are a salient run; the first source
    # takes its free left neighbour, the others need non-adjacent donors.
    x = synth.normal(29, (2, 3, 41, 16)) * np.float32(0.1)
    x[..., 6:10] *= 100
    out = oracle.k4_quantize(x, salient_fraction=0.25)
    src, don = out["salient_channels"], out["donor_channels"]
    assert (src == np.array([6, 7, 8, 9])).all()
    assert (np.diff(np.sort(don, -1), axis=-1) > 0).all()
    assert not (src[..., :, None] == don[..., None, :]).any()
    assert (np.abs(src - don) > 1).any()
    assert (don[..., 0] == 5).all()


def test_min_error_known_answer():
    # test_codec.py:150-162: neighbours picks the varying neighbour 1,
    # min_error picks channel 7, which its sampled mean reconstructs exactly.
    x = synth.normal(119, (1, 2, 128, 8))
    x[..., 0] = 100
    x[..., 1] *= 10
    x[..., 7] = 2
    local = oracle.k4_quantize(x, salient_fraction=0.125)
    chosen = oracle.k4_quantize(x, salient_fraction=0.125, donor_policy="min_error")
    assert (local["donor_channels"] == 1).all()
    assert (chosen["donor_channels"] == 7).all()
    assert (local["salient_channels"] == chosen["salient_channels"]).all()
    err_local = ((oracle.k4_dequantize(local) - x) ** 2).mean()
    err_chosen = ((oracle.k4_dequantize(chosen) - x) ** 2).mean()
    assert err_chosen < err_local


def test_sampled_positions_known_answer():
    # test_codec.py:101-106: unsampled outliers must not influence ranking
    x = np.ones((1, 1, 16, 8), np.float32)
    x[..., 1::2, 0] = 1000
    x[..., ::8, 6] = 10
    assert oracle.k4_quantize(x, sample_stride=8)["salient_channels"].tolist() == [[[6]]]


def test_sources_are_stable_top_k_and_pool_is_stable_bottom_k():
    gen = np.random.default_rng(5)
    sal = gen.integers(0, 6, size=(64, 128)).astype(np.float32)
    err = gen.integers(0, 4, size=(64, 128)).astype(np.float32)
    for count in (1, 8, 16, 64):
        src, don = oracle.reuse_map(sal, count, err)
        for r in range(sal.shape[0]):
            top = np.sort(np.argsort(-sal[r], kind="stable")[:count])
            assert (src[r] == top).all()
            masked = np.where(np.isin(np.arange(128), top), np.inf, err[r])
            pool = set(np.argsort(masked, kind="stable")[:count].tolist())
            assert set(don[r].tolist()) == pool          # every pool slot is used exactly once
        src, don = oracle.reuse_map(sal, count)
        assert not (don[:, :, None] == src[:, None, :]).any()
        assert all(len(set(row)) == count for row in don.tolist())


def test_neighbour_search_on_tiny_rows_matches_exhaustive_rule():
    # For single-source rows the rule reduces to: an available immediate
    # neighbour of least saliency, else the nearest available channel to the
    # run boundary.  Check every 6-channel saliency pattern over {0, 1, 2}.
    import itertools
    for values in itertools.product([0.0, 1.0, 2.0], repeat=6):
        sal = np.array(values, np.float32)
        src, don = oracle.reuse_map(sal[None], 1)
        s = int(np.argsort(-sal, kind="stable")[0])
        neigh = [p for p in (s - 1, s + 1) if 0 <= p < 6]
        best = min(neigh, key=lambda p: (sal[p], p))
        assert src[0, 0] == s and don[0, 0] == best


@pytest.mark.parametrize("bits", [2, 4])
def test_value_codec_known_answers(bits):
    # test_value_codec.py:14-27
    codes = np.tile(np.arange(1 << bits), 128 // (1 << bits)).astype(np.float32)
    x = np.broadcast_to(codes * 2 - 3, (2, 3, 7, 128)).copy()
    q = oracle.v_quantize(x, bits, 64)
    assert q["payload"][0, 0, 0, 0] == sum(i << (bits * i) for i in range(8 // bits))
    np.testing.assert_array_equal(oracle.v_dequantize(q, bits, 64), x)
    for constant in (0.0, 3.0, -7.0):
        y = np.full((1, 2, 17, 128), constant, np.float32)
        np.testing.assert_array_equal(oracle.v_dequantize(oracle.v_quantize(y, bits), bits, 64), y)


@pytest.mark.parametrize("bits,group", [(2, 32), (2, 64), (2, 128), (4, 64)])
def test_value_codec_parameters_and_nearest_level(bits, group):
    x = synth.kv_like(7, 2, 64, groups=(2, 2, 1))
    q = oracle.v_quantize(x, bits, group)
    levels = (1 << bits) - 1
    g = x.reshape(*x.shape[:-1], -1, group)
    lo, hi = g.min(-1), g.max(-1)
    np.testing.assert_array_equal(q["offsets"], lo.astype(np.float16))
    s = np.maximum((hi - lo) / np.float32(levels), np.float32(2.0 ** -14))
    np.testing.assert_array_equal(q["scales"], s.astype(np.float16))
    dec = oracle.v_dequantize(q, bits, group).reshape(g.shape)
    sc = q["scales"].astype(np.float32)[..., None]
    off = q["offsets"].astype(np.float32)[..., None]
    # each code is a nearest level (clamped to the code range)
    level_vals = off + np.arange(levels + 1, dtype=np.float32) * sc
    dist = np.abs(g[..., None] - level_vals[..., None, :])
    chosen = np.abs(g - dec)
    assert (chosen <= dist.min(-1) * (1 + 1e-6) + 1e-6).all()


@pytest.mark.parametrize("bits", [2, 4])
def test_value_codec_rounds_like_ieee_division_and_half_to_even(bits):
    # value_codec.py:66-67: torch.round (half to even) of the IEEE fp32
    # quotient.  Literal known answers: exact ties, and quotients one ulp
    # from k + 1/2 where a reciprocal product would round the other way.
    import vknown
    vknown.quotients_hold()
    x, codes = vknown.build(bits, "float32")
    q = oracle.v_quantize(x, bits, vknown.GROUP)
    np.testing.assert_array_equal(vknown.unpack_codes(q["payload"][0, 0], bits), codes)


def test_value_codec_rejects_unrepresentable_parameters():
    for value in (float("nan"), float("inf"), 1e6):
        with pytest.raises(ValueError, match="finite"):
            oracle.v_quantize(np.full((1, 1, 2, 128), value, np.float32))


def test_half_and_bfloat16_rounding_match_numpy_and_torch():
    vals = np.concatenate([synth.normal(3, (4096,)) * np.float32(10.0) ** synth.normal(4, (4096,)),
                           np.array([65504, 65519.99, 65520, 1e-8, 6e-8, 3e-8, 2.0 ** -24, 2.0 ** -25,
                                     -2.0 ** -14, 1.5 * 2.0 ** -24, 0.0, -0.0], np.float32)]).astype(np.float32)
    lib = oracle.lib()
    got16 = np.array([lib.iqo_f32_to_f16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got16, vals.astype(np.float16).view(np.uint16))
    gotbf = np.array([lib.iqo_f32_to_bf16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(gotbf, torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy()
                                  .view(np.uint16))


def test_k4_dequantize_exact_codes_padding_and_int4_bound():
    # test_codec.py:48-70
    x = synth.normal(29, (2, 3, 41, 16)) * np.float32(0.1)
    x[..., 6:10] *= 100
    q = oracle.k4_quantize(x, salient_fraction=0.25)
    r = oracle.k4_dequantize(q)
    src, don, sc = q["salient_channels"], q["donor_channels"], q["scales"]
    sampled_mean = torch.from_numpy(x)[..., ::8, :].mean(-2).numpy()   # torch's own reduction
    for b in range(2):
        for h in range(3):
            for s, d in zip(src[b, h], don[b, h]):
                exp = np.clip(np.rint(x[b, h, :, s] / sc[b, h, s]), -127, 127) * sc[b, h, s]
                np.testing.assert_array_equal(r[b, h, :, s], exp)
                np.testing.assert_array_equal(r[b, h, :, d], np.full(41, sampled_mean[b, h, d], np.float32))
            normal = np.setdiff1d(np.arange(16), np.concatenate([src[b, h], don[b, h]]))
            bound = sc[b, h, normal] / 2 + 1e-7
            assert (np.abs(r[b, h][:, normal] - x[b, h][:, normal]) <= bound).all()


def test_k4_uniform_int4_and_nibble_patterns():
    # test_codec.py:84-98: fraction 0 is plain symmetric INT4
    x = synth.normal(29, (2, 3, 41, 16))
    q = oracle.k4_quantize(x, salient_fraction=0)
    expected = np.clip(np.rint(x / q["scales"][:, :, None]), -7, 7) * q["scales"][:, :, None]
    np.testing.assert_array_equal(oracle.k4_dequantize(q), expected.astype(np.float32))
    y = np.broadcast_to(np.arange(-7, 8, dtype=np.float32).reshape(1, 1, 15, 1), (1, 1, 15, 16)).copy()
    np.testing.assert_array_equal(oracle.k4_dequantize(oracle.k4_quantize(y, salient_fraction=0)), y)
    z = np.zeros((1, 2, 17, 16), np.float32)
    for frac in (0.0, 0.125, 0.5):
        assert not oracle.k4_dequantize(oracle.k4_quantize(z, salient_fraction=frac)).any()


def test_role_map_encodes_sources_donors_and_padding_slots():
    gen = np.random.default_rng(3)
    src = np.stack([np.sort(gen.choice(128, 16, replace=False)) for _ in range(4)])
    don = np.stack([gen.permutation(np.setdiff1d(np.arange(128), s))[:16] for s in src])
    roles = oracle.role_map(src, don)
    for h in range(4):
        for c in range(128):
            if c in src[h]:
                assert roles[h, c] == don[h][list(src[h]).index(c)]
            elif c in don[h]:
                assert roles[h, c] == -2 - list(don[h]).index(c)
            else:
                assert roles[h, c] == -1


def test_attention_oracle_against_torch_sdpa_and_closed_forms():
    gen = torch.Generator().manual_seed(4)
    q = torch.randn(8, 128, generator=gen)
    k = torch.randn(2, 300, 128, generator=gen) * 3
    v = torch.randn(2, 300, 128, generator=gen)
    got = oracle.attend(q.numpy(), k.numpy(), v.numpy(), 0.125)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double().view(1, 8, 1, 128), k.double().view(1, 2, 300, 128), v.double().view(1, 2, 300, 128),
        scale=0.125, enable_gqa=True).view(8, 128).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # equal keys -> uniform weights -> mean of values
    kk = np.ones((1, 50, 128), np.float32)
    out = oracle.attend(q.numpy()[:2], kk, v.numpy()[:1, :50], 0.1)
    np.testing.assert_allclose(out, np.broadcast_to(v.numpy()[0, :50].astype(np.float64).mean(0), (2, 128)),
                               rtol=1e-12, atol=1e-12)


def test_tile_encoder_quotient_identity():
    # the GPU tile encoder's Welford step replaces delta / n by a reciprocal
    # product with one remainder correction; it must be the IEEE quotient
    assert oracle.check_recip_division(256, 20000, 11) == 0


def test_causal_attention_oracle_against_torch_sdpa():
    # the prefill oracle against torch's scaled_dot_product_attention in fp64
    # (is_causal, GQA expanded by repeat), and the first query's closed form
    # (it sees only key 0: its output is v[0])
    n, hq, h = 37, 6, 2
    q = synth.normal(501, (n, hq, 128))
    k = synth.normal(502, (n, h, 128))
    v = synth.normal(503, (n, h, 128))
    got = oracle.causal_attend(q, k, v, 0.1)
    qt = torch.from_numpy(q).double().transpose(0, 1)
    kt = torch.from_numpy(k).double().transpose(0, 1).repeat_interleave(hq // h, 0)
    vt = torch.from_numpy(v).double().transpose(0, 1).repeat_interleave(hq // h, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.1).transpose(0, 1)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(got[0], np.repeat(v[0], hq // h, 0), rtol=0, atol=1e-15)


def test_causal_attend_rows_equals_the_full_causal_oracle():
    # the chunked row/head evaluation that the long prefill checks use,
    # pinned against the whole-matrix fp64 oracle (itself pinned to SDPA)
    rng = np.random.default_rng(3)
    n, hq, h = 300, 6, 2
    q = rng.standard_normal((n, hq, 128))
    k = rng.standard_normal((n, h, 128))
    v = rng.standard_normal((n, h, 128))
    full = oracle.causal_attend(q, k, v, 0.1)
    rows = np.array([0, 1, 77, 128, 129, 299])
    got = oracle.causal_attend_rows(q, k, v, 0.1, rows, [0, 3, 5], chunk=4)
    np.testing.assert_allclose(got, full[rows][:, [0, 3, 5]], rtol=0, atol=1e-12)
