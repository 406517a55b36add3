"""GPU parity of the cache's paired key / value block encodes
(cache.py:288-295).  iq_kv_quantize (V2/V4 values): one launch for sealed
256-token blocks of 128 16-bit channels (K4 keys, the values encoded by the
same workgroups), the two encoders back to back otherwise; bit-identical to
iq_k4_quantize + iq_v_quantize (themselves pinned to the oracle and the
reference's goldens) and, at config 3's shape, to the oracle directly.
iq_k4_quantize_kv (K4-coded values): one launch over (blocks, 2 heads),
bit-identical to two iq_k4_quantize calls."""
import numpy as np
import pytest
import torch

from oracle import oracle
import synth

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _kv(seed, shape, dtype, runs=(3, 3, 1)):
    """[B, H, T, D] keys and values: N(0, 1) with x20 outlier channel runs."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = []
    for which in range(2):
        x = torch.randn(shape, generator=g, device="cuda")
        for h, chans in enumerate(synth.outlier_channels(seed + which, shape[1], shape[3], list(runs))):
            x[:, h, :, chans] *= 20
        out.append(x.to(dtype))
    return out


def _fused(k, v, fraction, policy, bits, group, stride=8):
    """iq_kv_quantize on [B, H, T, D] views; returns (key fields, value fields, flags)."""
    from inquant import _native as nat
    B, H, T, D = k.shape
    count = int(D * fraction)
    dev = k.device
    out = {
        "payload": torch.empty((B, H, T, D // 2), dtype=torch.uint8, device=dev),
        "scales": torch.empty((B, H, D), dtype=torch.float32, device=dev),
        "salient_channels": torch.empty((B, H, count), dtype=torch.uint8, device=dev),
        "donor_channels": torch.empty((B, H, count), dtype=torch.uint8, device=dev),
        "padding": torch.empty((B, H, count), dtype=torch.float32, device=dev),
    }
    vout = {
        "payload": torch.empty((B, H, T, D * bits // 8), dtype=torch.uint8, device=dev),
        "scales": torch.empty((B, H, T, D // group), dtype=torch.float16, device=dev),
        "offsets": torch.empty((B, H, T, D // group), dtype=torch.float16, device=dev),
    }
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    c = lambda name: out[name].data_ptr() if count else None
    nat.check(nat.lib().iq_kv_quantize(
        k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), nat.strides4(k), nat.strides4(v), B, H, T, D, count,
        stride, int(policy == "min_error"), out["payload"].data_ptr(), out["scales"].data_ptr(),
        c("salient_channels"), c("donor_channels"), 1, c("padding"), bits, group, vout["payload"].data_ptr(),
        vout["scales"].data_ptr(), vout["offsets"].data_ptr(), flags.data_ptr(), flags.data_ptr() + 4,
        nat.stream_handle(dev)))
    torch.cuda.synchronize()
    return out, vout, flags.tolist()


def _separate(k, v, fraction, policy, bits, group, stride=8):
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    pk = quantize(k, CodecConfig(sample_stride=stride, salient_fraction=fraction, donor_policy=policy))
    pv = quantize_values(v, bits, group)
    return pk.tensors, {"payload": pv.payload, "scales": pv.scales, "offsets": pv.offsets}


def _same(a: dict, b: dict):
    for name in b:
        x, y = _np(a[name]), _np(b[name])
        assert x.dtype == y.dtype and x.shape == y.shape, name
        np.testing.assert_array_equal(x.view(np.uint8), y.view(np.uint8), err_msg=name)


def _blocks(t, nb, B=256):
    """The cache's strided [blocks, H, B, D] view of [1, H, nb * B, D]."""
    return t[0, :, :nb * B].unflatten(1, (nb, B)).transpose(0, 1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,group", [(2, 64), (2, 32), (2, 128), (4, 64), (4, 32), (4, 128)])
@pytest.mark.parametrize("fraction,policy", [(0.125, "min_error"), (0.125, "neighbors"), (0.0, "min_error"),
                                             (0.5, "neighbors")])
def test_fused_sealed_blocks_equal_the_separate_encoders(dtype, bits, group, fraction, policy):
    print(f"fused kv {dtype} bits {bits} group {group} {fraction} {policy}", flush=True)
    k, v = _kv(11, (1, 3, 6 * 256, 128), dtype)
    kb, vb = _blocks(k, 6), _blocks(v, 6)
    fk, fv, flags = _fused(kb, vb, fraction, policy, bits, group)
    sk, sv = _separate(kb, vb, fraction, policy, bits, group)
    assert flags == [0, 0]
    _same(fk, sk)
    _same(fv, sv)


@pytest.mark.parametrize("shape,dtype", [((2, 3, 100, 128), torch.bfloat16), ((2, 2, 256, 64), torch.float16),
                                         ((1, 2, 256, 128), torch.float32), ((3, 1, 17, 32), torch.bfloat16)])
def test_other_shapes_run_the_two_encoders(shape, dtype):
    # T != 256, D != 128 or 32-bit rows: the back-to-back path, same bits
    print(f"kv fallback {shape} {dtype}", flush=True)
    k, v = _kv(21, shape, dtype, runs=(1,))
    fk, fv, flags = _fused(k, v, 0.125, "min_error", 2, 32)
    sk, sv = _separate(k, v, 0.125, "min_error", 2, 32)
    assert flags == [0, 0]
    _same(fk, sk)
    _same(fv, sv)


def test_fused_values_with_padded_rows_and_distinct_strides():
    # keys and values are different views (rows 192 and 256 elements apart):
    # each side takes its own strides
    print("fused kv strided views", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    kw = torch.randn((4, 2, 256, 192), generator=g, device="cuda").to(torch.bfloat16)
    vw = torch.randn((4, 2, 256, 256), generator=g, device="cuda").to(torch.bfloat16) * 3
    kw[..., 40:43] *= 25
    k, v = kw[..., 32:160], vw[..., 128:]
    assert k.stride(2) == 192 and v.stride(2) == 256
    fk, fv, flags = _fused(k, v, 0.125, "min_error", 4, 64)
    sk, sv = _separate(k, v, 0.125, "min_error", 4, 64)
    assert flags == [0, 0]
    _same(fk, sk)
    _same(fv, sv)


@pytest.mark.parametrize("where", ["key", "value", "both"])
def test_fused_nonfinite_flags(where):
    # a NaN key raises only the key flag, an inf value only the value flag
    print(f"fused kv nonfinite {where}", flush=True)
    k, v = _kv(31, (1, 2, 3 * 256, 128), torch.bfloat16)
    if where in ("key", "both"):
        k[0, 1, 300, 7] = float("nan")
    if where in ("value", "both"):
        v[0, 0, 600, 99] = float("inf")
    _, _, flags = _fused(_blocks(k, 3), _blocks(v, 3), 0.125, "min_error", 2, 64)
    assert flags == [int(where in ("key", "both")), int(where in ("value", "both"))]


def test_cfg3_layer_fused_encode_matches_oracle():
    # config 3 at its real size through the fused launch: one Mistral-7B
    # layer of 32768 tokens x 8 KV heads in 256-token blocks, 8% outlier
    # channels as three 3-wide runs plus one, K4 min_error and V2 g64,
    # bit-exact against the oracle (codec.py:181-243, value_codec.py:51-72)
    print("cfg3 fused encode", flush=True)
    H, T = 8, 32768
    k, v = _kv(3003, (1, H, T, 128), torch.bfloat16, runs=(3, 3, 3, 1))
    kb, vb = _blocks(k, T // 256), _blocks(v, T // 256)
    fk, fv, flags = _fused(kb, vb, 0.125, "min_error", 2, 64)
    assert flags == [0, 0]
    ref_k = oracle.k4_quantize(_np(kb.float()), 8, 0.125, "min_error")
    for name in ("payload", "scales", "salient_channels", "donor_channels", "padding"):
        got = _np(fk[name]).astype(ref_k[name].dtype)
        np.testing.assert_array_equal(got.view(np.uint8), np.ascontiguousarray(ref_k[name]).view(np.uint8), name)
    ref_v = oracle.v_quantize(_np(vb.float()), 2, 64)
    np.testing.assert_array_equal(_np(fv["payload"]), ref_v["payload"])
    np.testing.assert_array_equal(_np(fv["scales"]).view(np.uint16), ref_v["scales"].view(np.uint16))
    np.testing.assert_array_equal(_np(fv["offsets"]).view(np.uint16), ref_v["offsets"].view(np.uint16))


@pytest.mark.parametrize("bits,group", [(2, 64), (4, 128)])
def test_cache_seal_of_full_blocks_uses_the_fused_encode(bits, group):
    # a cache with 256-token blocks and V2/V4 values seals through
    # iq_kv_quantize's one launch: the stored blocks equal the separate
    # encoders' output for the same rows
    print(f"cache fused seal {bits} {group}", flush=True)
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    cfg = CacheConfig(CodecConfig(donor_policy="min_error"), block_size=256, residual_length=128, sink_tokens=4,
                      value_bits=bits, value_group_size=group)
    cache = InQuantCache(cfg)
    k, v = _kv(41, (1, 4, 4 + 3 * 256 + 200, 128), torch.bfloat16)
    cache.update(k, v, 0)
    layer = cache._layers[0]
    assert len(layer.key_blocks) == 3
    kb, vb = _blocks(k[:, :, 4:4 + 768], 3), _blocks(v[:, :, 4:4 + 768], 3)
    sk, sv = _separate(kb, vb, 0.125, "min_error", bits, group)
    for i, (kblock, vblock) in enumerate(zip(layer.key_blocks, layer.value_blocks)):
        for name, t in kblock.tensors.items():
            np.testing.assert_array_equal(_np(t[0]).view(np.uint8), _np(sk[name][i]).view(np.uint8), name)
        np.testing.assert_array_equal(_np(vblock.payload[0]), _np(sv["payload"][i]))
        np.testing.assert_array_equal(_np(vblock.scales[0]).view(np.uint16), _np(sv["scales"][i]).view(np.uint16))
        np.testing.assert_array_equal(_np(vblock.offsets[0]).view(np.uint16),
                                      _np(sv["offsets"][i]).view(np.uint16))


def _k4_pair(k, v, fraction, policy, stride=8):
    """iq_k4_quantize_kv on [B, H, T, D] views; returns (key fields, value fields, flags)."""
    from inquant import _native as nat
    B, H, T, D = k.shape
    count = int(D * fraction)
    dev = k.device

    def outputs():
        return {"payload": torch.empty((B, H, T, D // 2), dtype=torch.uint8, device=dev),
                "scales": torch.empty((B, H, D), dtype=torch.float32, device=dev),
                "salient_channels": torch.empty((B, H, count), dtype=torch.uint8, device=dev),
                "donor_channels": torch.empty((B, H, count), dtype=torch.uint8, device=dev),
                "padding": torch.empty((B, H, count), dtype=torch.float32, device=dev)}

    ko, vo = outputs(), outputs()
    ptrs = lambda o: [o["payload"].data_ptr(), o["scales"].data_ptr()] + [
        o[n].data_ptr() if count else None for n in ("salient_channels", "donor_channels", "padding")]
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    nat.check(nat.lib().iq_k4_quantize_kv(
        k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), nat.strides4(k), nat.strides4(v), B, H, T, D, count,
        stride, int(policy == "min_error"), *ptrs(ko), *ptrs(vo), 1, flags.data_ptr(), flags.data_ptr() + 4,
        nat.stream_handle(dev)))
    torch.cuda.synchronize()
    return ko, vo, flags.tolist()


def _k4_separate(k, v, fraction, policy, stride=8):
    from inquant.codec import CodecConfig, quantize
    cfg = CodecConfig(sample_stride=stride, salient_fraction=fraction, donor_policy=policy)
    return quantize(k, cfg).tensors, quantize(v, cfg).tensors


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [256, 100])
@pytest.mark.parametrize("fraction,policy", [(0.125, "min_error"), (0.125, "neighbors"), (0.0, "min_error"),
                                             (0.5, "neighbors")])
def test_k4_pair_equals_two_key_encodes(dtype, T, fraction, policy):
    # K4-coded values (the cache's default): one launch over (blocks, 2 H)
    # rows, bit-identical to two iq_k4_quantize calls (256-token blocks take
    # the direct-to-LDS variant, 100-token rows the other)
    print(f"k4 pair {dtype} T {T} {fraction} {policy}", flush=True)
    k, v = _kv(51, (1, 3, 5 * T, 128), dtype)
    kb, vb = _blocks(k, 5, T), _blocks(v, 5, T)
    fk, fv, flags = _k4_pair(kb, vb, fraction, policy)
    sk, sv = _k4_separate(kb, vb, fraction, policy)
    assert flags == [0, 0]
    _same(fk, sk)
    _same(fv, sv)


@pytest.mark.parametrize("shape,dtype", [((2, 2, 256, 64), torch.float16), ((1, 2, 256, 128), torch.float32)])
def test_k4_pair_other_shapes_run_two_encodes(shape, dtype):
    print(f"k4 pair fallback {shape} {dtype}", flush=True)
    k, v = _kv(61, shape, dtype, runs=(1,))
    fk, fv, flags = _k4_pair(k, v, 0.125, "min_error")
    sk, sv = _k4_separate(k, v, 0.125, "min_error")
    assert flags == [0, 0]
    _same(fk, sk)
    _same(fv, sv)


@pytest.mark.parametrize("where", ["key", "value"])
def test_k4_pair_nonfinite_flags(where):
    print(f"k4 pair nonfinite {where}", flush=True)
    k, v = _kv(71, (1, 2, 2 * 256, 128), torch.bfloat16)
    (k if where == "key" else v)[0, 1, 300, 50] = float("nan")
    _, _, flags = _k4_pair(_blocks(k, 2), _blocks(v, 2), 0.125, "min_error")
    assert flags == [int(where == "key"), int(where == "value")]


def test_cache_seal_with_k4_values_uses_one_launch():
    # value_bits None (K4-coded values): the cache's blocks equal two
    # separate encodes of the same rows, and one launch encodes them
    print("cache k4 pair seal", flush=True)
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    cfg = CacheConfig(CodecConfig(donor_policy="min_error"), block_size=256, residual_length=128, sink_tokens=4)
    cache = InQuantCache(cfg)
    k, v = _kv(81, (1, 4, 4 + 2 * 256 + 150, 128), torch.bfloat16)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        cache.update(k, v, 0)
        torch.cuda.synchronize()
    names = [e.name for e in prof.events()]
    assert sum("k4_encode_pair" in n for n in names) == 1 and not any("k4_encode_tile" in n for n in names)
    layer = cache._layers[0]
    assert len(layer.key_blocks) == 2
    kb, vb = _blocks(k[:, :, 4:4 + 512], 2), _blocks(v[:, :, 4:4 + 512], 2)
    sk, sv = _k4_separate(kb, vb, 0.125, "min_error")
    for i, (kblock, vblock) in enumerate(zip(layer.key_blocks, layer.value_blocks)):
        for name, t in kblock.tensors.items():
            np.testing.assert_array_equal(_np(t[0]).view(np.uint8), _np(sk[name][i]).view(np.uint8), name)
        for name, t in vblock.tensors.items():
            np.testing.assert_array_equal(_np(t[0]).view(np.uint8), _np(sv[name][i]).view(np.uint8), name)
