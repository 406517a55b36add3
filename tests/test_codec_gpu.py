"""GPU parity of the HIP codec kernels: bit-exact against the reference's
golden vectors and the pinned CPU oracle (tests/test_oracle.py)."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from recipes import K4_CASES, build_input
import synth

pytestmark = pytest.mark.gpu

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TORCH_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _dev(x: np.ndarray, dtype=torch.float32):
    t = torch.from_numpy(np.ascontiguousarray(x)).to("cuda")
    return t.to(dtype)


def _np(t):
    return t.detach().cpu().numpy()


def _same_bits(a, b, what=""):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.astype(np.float32).view(np.uint32)
    np.testing.assert_array_equal(a, b, err_msg=what)


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(GOLDEN_DIR, "k4_quantize.json")) as f:
        meta = json.load(f)["cases"]
    return meta, np.load(os.path.join(GOLDEN_DIR, "k4_quantize.npz"))


@pytest.mark.parametrize("name", sorted(K4_CASES))
def test_k4_quantize_matches_reference_golden(golden, name):
    from inquant.codec import CodecConfig, quantize
    meta, arrays = golden
    recipe, cfg = K4_CASES[name]
    x = build_input(recipe)
    dtype = TORCH_DTYPES.get(recipe.get("dtype", "float32"), torch.float32)
    packed = quantize(_dev(x, dtype), CodecConfig(**cfg))
    assert hashlib.sha256(_np(packed.payload).tobytes()).hexdigest() == meta[name]["payload_sha256"]
    assert str(packed.salient_channels.dtype).replace("torch.", "") == meta[name]["descriptor_dtype"]
    for field in ("scales", "salient_channels", "donor_channels", "padding"):
        _same_bits(_np(packed.tensors[field]).astype(arrays[f"{name}/{field}"].dtype), arrays[f"{name}/{field}"],
                   field)
    assert packed.shape == tuple(x.shape) and packed.original_dtype == dtype


@pytest.mark.parametrize("policy", ["neighbors", "min_error"])
def test_k4_blocked_strided_view_matches_golden(golden, policy):
    # the cache encodes a strided [nb, H, B, D] view of the prefill in place
    from inquant.codec import CodecConfig, quantize
    meta, arrays = golden
    name = f"cfg0_blocks_{policy}"
    recipe, cfg = K4_CASES[name]
    flat = build_input({k: v for k, v in recipe.items() if k != "block"})
    t = _dev(flat, torch.bfloat16)
    view = t[0].reshape(4, 16, 256, 128).permute(1, 0, 2, 3)
    assert not view.is_contiguous()
    packed = quantize(view, CodecConfig(**cfg))
    assert hashlib.sha256(_np(packed.payload).tobytes()).hexdigest() == meta[name]["payload_sha256"]
    _same_bits(_np(packed.padding), arrays[f"{name}/padding"])


@pytest.mark.parametrize("D,T,stride,policy,frac,dtype", [
    (128, 256, 8, "min_error", 0.125, torch.bfloat16),
    (128, 200, 8, "neighbors", 0.125, torch.float16),
    # LDS tile encoder (16-bit input, D = 128, T <= 256): edge lengths and counts
    (128, 256, 8, "min_error", 0.125, torch.float16),
    (128, 256, 16, "neighbors", 0.5, torch.bfloat16),
    (128, 256, 1, "min_error", 0.5, torch.bfloat16),
    (128, 255, 7, "min_error", 0.25, torch.bfloat16),
    (128, 17, 8, "min_error", 0.0, torch.bfloat16),
    (128, 1, 8, "min_error", 0.125, torch.float16),
    (128, 257, 8, "min_error", 0.125, torch.bfloat16),
    (64, 77, 5, "min_error", 0.25, torch.float32),
    (130, 33, 2, "neighbors", 0.5, torch.float32),
    (258, 9, 3, "min_error", 0.5, torch.bfloat16),
    (512, 16, 1, "neighbors", 0.125, torch.float32),
    (16, 4100, 1, "min_error", 0.25, torch.float32),
    (8, 16, 8, "neighbors", 0.125, torch.float64),
])
def test_k4_quantize_matches_oracle(D, T, stride, policy, frac, dtype):
    from inquant.codec import CodecConfig, quantize
    x = synth.normal(D * 1000 + T, (2, 3, T, D)) * np.exp(synth.normal(7, (2, 3, T, 1)))
    x[..., 1:3] *= 25
    xt = _dev(x, torch.float64).to(dtype)
    ref = oracle.k4_quantize(_np(xt.float()), stride, frac, policy)
    got = quantize(xt, CodecConfig(sample_stride=stride, salient_fraction=frac, donor_policy=policy))
    for field in ("payload", "scales", "salient_channels", "donor_channels", "padding"):
        _same_bits(_np(got.tensors[field]).astype(ref[field].dtype), ref[field], field)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k4_sealed_blocks_with_padded_rows(dtype):
    # sealed 256-token blocks whose rows are 192 elements apart (a view of
    # wider rows) and whose heads are not adjacent: the direct-to-LDS chunk
    # loads take the strides from the view
    from inquant.codec import CodecConfig, quantize
    x = synth.normal(91, (2, 3, 256, 192)) * np.exp(synth.normal(92, (2, 3, 256, 1)))
    x[..., 5:8] *= 30
    wide = _dev(x, torch.float64).to(dtype)
    view = wide[:, :, :, 32:160]
    assert view.stride(2) == 192 and not view.is_contiguous()
    for policy in ("neighbors", "min_error"):
        ref = oracle.k4_quantize(_np(view.float()), 8, 0.125, policy)
        got = quantize(view, CodecConfig(donor_policy=policy))
        for field in ("payload", "scales", "salient_channels", "donor_channels", "padding"):
            _same_bits(_np(got.tensors[field]).astype(ref[field].dtype), ref[field], field)


@pytest.mark.parametrize("fraction", [0.0, 0.125, 0.5])
def test_k4_all_zero_is_finite_and_exact(fraction):
    # test_codec.py:73-81; T = 256 takes the tile encoder, 17 the generic one
    from inquant.codec import CodecConfig, quantize
    for T, D in ((17, 16), (256, 128)):
        x = torch.zeros(1, 2, T, D, dtype=torch.bfloat16, device="cuda")
        packed = quantize(x, CodecConfig(salient_fraction=fraction))
        restored = packed.dequantize()
        assert restored.dtype == x.dtype and torch.isfinite(restored).all()
        assert torch.count_nonzero(restored) == 0
        assert packed.dequantize(torch.float32).dtype == torch.float32


def test_k4_zero_fraction_is_uniform_int4_and_nibble_patterns_stay_codes():
    # test_codec.py:84-99
    from inquant.codec import CodecConfig, quantize
    x = synth.normal(93, (1, 4, 256, 128)).astype(np.float32)
    xt = _dev(x)
    packed = quantize(xt, CodecConfig(salient_fraction=0))
    s = packed.scales.unsqueeze(-2)
    torch.testing.assert_close(packed.dequantize(), (xt / s).round().clamp(-7, 7) * s, rtol=0, atol=0)
    assert packed.salient_channels.numel() == packed.donor_channels.numel() == packed.padding.numel() == 0
    assert packed.metadata_nbytes == packed.scales.numel() * 4
    codes = torch.arange(-7, 8, dtype=torch.float32, device="cuda").view(1, 1, 15, 1).expand(1, 1, 15, 16)
    torch.testing.assert_close(quantize(codes, CodecConfig(salient_fraction=0)).dequantize(), codes, rtol=0, atol=0)


def test_k4_noncontiguous_input_and_detached_output():
    # test_codec.py:109-115
    from inquant.codec import quantize
    x = _dev(synth.normal(94, (1, 2, 16, 12))).requires_grad_(True).transpose(-2, -1)
    packed = quantize(x)
    assert packed.dequantize().shape == x.shape
    assert all(not t.requires_grad for t in packed.tensors.values())
    assert torch.isfinite(packed.dequantize()).all()


@pytest.mark.parametrize("channels", [2, 128, 258])
def test_k4_half_salient_fraction_always_has_enough_donors(channels):
    # test_codec.py:118-124
    from inquant.codec import CodecConfig, quantize
    packed = quantize(_dev(synth.normal(95 + channels, (1, 1, 3, channels))), CodecConfig(salient_fraction=0.5))
    assert packed.donor_channels.unique().numel() == channels // 2
    assert torch.isfinite(packed.dequantize()).all()
    if channels > 256:
        assert packed.donor_channels.dtype == torch.int32


def test_k4_rejects_nonfinite_values():
    from inquant.codec import quantize
    for bad in (float("nan"), float("inf")):
        with pytest.raises(ValueError, match="finite"):
            quantize(torch.full((1, 1, 8, 8), bad, device="cuda"))


@pytest.mark.parametrize("count", [0, 1, 8, 16, 32, 64])
@pytest.mark.parametrize("policy", ["neighbors", "min_error"])
def test_reuse_map_with_ties_and_adjacent_outliers(count, policy):
    # restates test_triton_selection.py:9-22 with the oracle as the expectation
    from inquant.codec import _reuse_map
    from inquant.triton_selection import reuse_map
    gen = np.random.default_rng(112)
    score = gen.random((3, 4, 128)).astype(np.float32)
    score[0] = 0
    score[1, :, 30:70] = 5
    score[2, :, 127] = 9
    error = gen.integers(0, 4, score.shape).astype(np.float32) if policy == "min_error" else None
    ref = oracle.reuse_map(score, count, error)
    for fn in (reuse_map, _reuse_map):
        got = fn(_dev(score), count, None if error is None else _dev(error))
        for a, b in zip(got, ref):
            assert a.dtype == torch.int64
            np.testing.assert_array_equal(_np(a), b)


def _check_values(got, ref):
    np.testing.assert_array_equal(_np(got.payload), ref["payload"])
    np.testing.assert_array_equal(_np(got.scales).view(np.uint16), ref["scales"].view(np.uint16))
    np.testing.assert_array_equal(_np(got.offsets).view(np.uint16), ref["offsets"].view(np.uint16))


@pytest.mark.parametrize("bits,group", [(2, 32), (2, 64), (2, 128), (4, 64), (4, 32), (4, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_value_codec_matches_oracle(bits, group, dtype):
    from inquant.value_codec import quantize_values
    x = synth.kv_like(11 + bits, 4, 300, groups=(2, 2, 1))
    xt = _dev(x).to(dtype)
    ref = oracle.v_quantize(_np(xt.float()), bits, group)
    got = quantize_values(xt, bits, group)
    _check_values(got, ref)
    for out in ("float32", "bfloat16", "float16"):
        dec = got.dequantize(TORCH_DTYPES[out])
        _same_bits(_np(dec.float()), oracle.v_dequantize(ref, bits, group, out), out)


@pytest.mark.parametrize("D,group", [(32, 32), (64, 32), (64, 64), (96, 32), (256, 64), (256, 128), (512, 128)])
@pytest.mark.parametrize("bits", [2, 4])
def test_value_codec_head_dims(D, group, bits):
    # D = 32..256 take the row kernel (16 channels per lane), 96 and 512 the
    # per-8-channel kernel; T = 1, 255 and 1000 end inside a token block
    from inquant.value_codec import quantize_values
    for T in (1, 255, 1000):
        x = synth.kv_like(40 + D + T, 3, T, D=D, groups=(1,))
        for dtype in (torch.bfloat16, torch.float16):
            xt = _dev(x).to(dtype)
            _check_values(quantize_values(xt, bits, group), oracle.v_quantize(_np(xt.float()), bits, group))


def test_value_codec_strided_blocks_and_many_rows():
    # the [blocks, H, B, D] view of a cache tensor (quantize_value_blocks) and
    # a batch*heads count above the row kernel's 65535 grid rows
    from inquant.value_codec import quantize_value_blocks, quantize_values
    x = _dev(synth.kv_like(77, 4, 1024), torch.bfloat16)
    blocks = quantize_value_blocks(x, 3, 256, 2, 64)
    for i, packed in enumerate(blocks):
        _check_values(packed, oracle.v_quantize(_np(x[:, :, 256 * i:256 * (i + 1)].float()), 2, 64))
    many = _dev(synth.normal(78, (256, 257, 1, 32)), torch.bfloat16)
    _check_values(quantize_values(many, 2, 32), oracle.v_quantize(_np(many.float()), 2, 32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_value_codec_rejects_one_nonfinite_value(dtype):
    from inquant.value_codec import quantize_values
    x = _dev(synth.kv_like(79, 2, 300), dtype)
    quantize_values(x, 2, 64)
    for value, where in ((float("nan"), (0, 1, 299, 127)), (float("inf"), (0, 0, 0, 5)),
                         (float("-inf"), (0, 1, 130, 64)), (float("nan"), (0, 0, 17, 0))):
        bad = x.clone()
        bad[where] = value
        with pytest.raises(ValueError, match="finite"):
            quantize_values(bad, 2, 64)


def test_value_codec_known_answers_and_rejections():
    from inquant.value_codec import quantize_values
    for bits in (2, 4):
        codes = torch.arange(1 << bits).repeat(128 // (1 << bits))
        x = (codes.float() * 2 - 3).view(1, 1, 1, 128).expand(2, 3, 7, 128).cuda()
        q = quantize_values(x, bits, 64)
        assert q.payload[0, 0, 0, 0].item() == sum(i << (bits * i) for i in range(8 // bits))
        assert q.payload_nbytes == x.numel() * bits // 8
        assert q.metadata_nbytes == x.numel() // 64 * 4
        assert torch.equal(q.dequantize(), x)
    for value in (float("nan"), float("inf"), 1e6):
        with pytest.raises(ValueError, match="finite"):
            quantize_values(torch.full((1, 1, 2, 128), value, device="cuda"))


@pytest.mark.parametrize("frac,policy,T", [(0.0, "neighbors", 96), (0.125, "min_error", 96), (0.5, "neighbors", 96),
                                           (0.125, "min_error", 300)])
def test_k4_dequantize_matches_oracle(frac, policy, T):
    from inquant.codec import CodecConfig, quantize
    x = synth.kv_like(21, 4, T)
    packed = quantize(_dev(x, torch.bfloat16), CodecConfig(salient_fraction=frac, donor_policy=policy))
    fields = {k: _np(v) for k, v in packed.tensors.items()}
    fields["salient_channels"] = fields["salient_channels"].astype(np.int64)
    fields["donor_channels"] = fields["donor_channels"].astype(np.int64)
    for out in ("float32", "bfloat16", "float16"):
        got = packed.dequantize(TORCH_DTYPES[out])
        assert got.dtype == TORCH_DTYPES[out]
        _same_bits(_np(got.float()), oracle.k4_dequantize(fields, out), out)
    assert packed.dequantize().dtype == torch.bfloat16


def test_k4_storage_accounting():
    # test_codec.py:18-33
    from inquant.codec import CodecConfig, quantize
    x = torch.randn(2, 3, 41, 16, device="cuda", dtype=torch.float16)
    packed = quantize(x, CodecConfig(salient_fraction=0.25))
    assert packed.payload.shape == (2, 3, 41, 8) and packed.payload.dtype == torch.uint8
    assert packed.payload_nbytes == x.numel() // 2
    assert packed.metadata_nbytes == 2 * 3 * (16 * 4 + 4 * (1 + 1 + 4))
    assert all(t.device == x.device and t.is_contiguous() for t in packed.tensors.values())
    stats = packed.storage_stats()
    assert stats["source_nbytes"] == x.numel() * 2 and stats["compression_ratio"] < 4
    big = quantize(torch.randn(1, 1, 3, 258, device="cuda"), CodecConfig(salient_fraction=0.5))
    assert big.donor_channels.dtype == torch.int32 and big.donor_channels.unique().numel() == 129


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_codecs_round_half_to_even_on_exact_ties(dtype):
    # quotients landing exactly on half-integers (and one ulp either side)
    # must round like the IEEE division followed by rint (half to even)
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    gen = np.random.default_rng(5)
    halves = gen.integers(-14, 15, (2, 4, 256, 128)).astype(np.float32) * 0.5
    halves[..., 0, :] = 7.0                      # amax 7 -> normal-channel scale exactly 1
    halves[..., 9:12] *= 16                      # salient run: scale 112 / 127
    k = _dev(halves, dtype)
    for policy in ("neighbors", "min_error"):
        ref = oracle.k4_quantize(_np(k.float()), 8, 0.125, policy)
        got = quantize(k, CodecConfig(donor_policy=policy))
        for field in ("payload", "scales", "salient_channels", "donor_channels", "padding"):
            _same_bits(_np(got.tensors[field]).astype(ref[field].dtype), ref[field], field)
    v = gen.integers(0, 7, (2, 4, 256, 128)).astype(np.float32) * 0.5   # groups span [0, 3]: scale 1
    v[..., ::64] = 0.0
    v[..., 1::64] = 3.0
    v[1, 1, 5, 7] = np.nextafter(np.float32(1.5), np.float32(2))
    vt = _dev(v, dtype)
    for bits in (2, 4):
        ref = oracle.v_quantize(_np(vt.float()), bits, 64)
        got = quantize_values(vt, bits, 64)
        np.testing.assert_array_equal(_np(got.payload), ref["payload"])


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_value_codes_match_ieee_division_known_answers(bits, dtype):
    # value_codec.py:66-67 pinned by literal codes (tests/vknown.py): exact
    # ties go to the even code; quotients one ulp from k + 1/2 follow the
    # IEEE division (fp32 rows: the generic encoder; bf16 rows: the row encoder)
    import vknown
    from inquant.value_codec import quantize_values
    x, codes = vknown.build(bits, dtype)
    got = quantize_values(_dev(x, TORCH_DTYPES[dtype]), bits, vknown.GROUP)
    np.testing.assert_array_equal(vknown.unpack_codes(_np(got.payload)[0, 0], bits), codes)
    ref = oracle.v_quantize(x, bits, vknown.GROUP)
    np.testing.assert_array_equal(_np(got.scales).view(np.uint16), ref["scales"].view(np.uint16))
    np.testing.assert_array_equal(_np(got.offsets).view(np.uint16), ref["offsets"].view(np.uint16))


def test_cfg3_full_layer_encode_matches_oracle():
    # config 3 at its real size: one Mistral-7B layer of 32768 tokens x 8 KV
    # heads in 256-token blocks (the cache's strided view of the prefill),
    # 8% outlier channels as three 3-wide runs plus one, K4 min_error and V2
    # g64, bit-exact against the oracle (codec.py:181-243, value_codec.py:51-72)
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    H, T, B = 8, 32768, 256
    print("cfg3 full-layer encode", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3003)
    kv = []
    for which in range(2):
        x = torch.randn((1, H, T, 128), generator=g, device="cuda")
        for h, chans in enumerate(synth.outlier_channels(3003 + which, H, 128, [3, 3, 3, 1])):
            x[0, h, :, chans] *= 20
        kv.append(x.to(torch.bfloat16))
    k, v = kv
    view = lambda t: t[0].reshape(H, T // B, B, 128).permute(1, 0, 2, 3)
    got_k = quantize(view(k), CodecConfig(donor_policy="min_error"))
    got_v = quantize_values(view(v), 2, 64)
    ref_k = oracle.k4_quantize(_np(view(k).float()), 8, 0.125, "min_error")
    for field in ("payload", "scales", "salient_channels", "donor_channels", "padding"):
        _same_bits(_np(got_k.tensors[field]).astype(ref_k[field].dtype), ref_k[field], field)
    ref_v = oracle.v_quantize(_np(view(v).float()), 2, 64)
    np.testing.assert_array_equal(_np(got_v.payload), ref_v["payload"])
    np.testing.assert_array_equal(_np(got_v.scales).view(np.uint16), ref_v["scales"].view(np.uint16))
    np.testing.assert_array_equal(_np(got_v.offsets).view(np.uint16), ref_v["offsets"].view(np.uint16))
