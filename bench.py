"""Benchmark of the InQuant packed-KV hot path on one MI355X.

Workload (config 2): Qwen2.5-7B-shaped decode, 28 query heads over 4
KV heads, head_dim 128, 32768 packed tokens (128 K4/V2 blocks of 256) + 4-token
BF16 sink + 128-token BF16 tail per layer, 28 layers with independent data.
One step = one decode token through all 28 layers (28 fused decode calls,
replayed as one HIP graph).  Inputs are resident in HBM; the 28 layers
(~400 MB) exceed the 256 MB Infinity Cache, so every step streams from HBM.

value  = algorithmic bytes (packed K/V, scales, role maps, padding, V params,
         pointer table, sink, tail, Q, O) per step / step time  [GB/s]
extras = codec encode Mtok/s (config 3: Mistral-7B layer, 32768
         tokens x 8 KV heads, K4 min_error + V2 g64), the config 3 decode
         (32 Mistral-7B layers), the config 2 append, the config 4 batched
         paged decode, the rows next to the decode path (materialize,
         encode into pages, causal prefill), roofline and the CPU oracle
         baseline on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "inquant-open-source_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0     # dense bf16 matrix-core peak
METRIC = "packed-KV decode attn GB/s (% HBM peak) @32K ctx; codec encode Mtok/s"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--rotate", type=int, default=2,
                    help="independent sets of `layers` layers replayed in turn (2 x 28 layers = 800 MB, "
                         "above the 512 MiB flush rule), so no step finds its layers in the Infinity Cache")
    ap.add_argument("--blocks", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="launch layer by layer instead of a HIP graph")
    ap.add_argument("--no-paged", action="store_true", help="skip the batched paged decode (config 4)")
    ap.add_argument("--no-cfg3", action="store_true", help="skip the Mistral-7B decode (config 3)")
    ap.add_argument("--no-encode", action="store_true", help="skip the config 3 encode")
    ap.add_argument("--no-k4-values", action="store_true", help="skip the config 2 decode with K4-coded values")
    ap.add_argument("--no-append", action="store_true", help="skip the config 2 append measurements")
    ap.add_argument("--no-next", action="store_true",
                    help="skip the rows next to the decode path (materialize, encode into pages, prefill)")
    ap.add_argument("--breakdown", action="store_true",
                    help="only the config 2 decode time split: full decode, the partition merge alone "
                         "(iq_decode_merge) and the launch floor of a one-element kernel, each replayed "
                         "28 x rotated sets in a graph")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device-to-device copy (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


COPY_PROBE_BYTES = 1 << 30
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_fast_cfg2_traffic.txt")


def copy_probe() -> None:
    """Three copies of 1 GiB with torch's elementwise copy kernel: the known
    byte count against which rocprofv3's FETCH_SIZE and WRITE_SIZE are scaled."""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "copies": 3}))


def measured_traffic():
    """HBM bytes per decode_fast launch from the committed rocprofv3 summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by the copy calibration), or None."""
    import re
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch\s*=\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


def kv_tensor(gen, heads, tokens, device, frac_groups=(2, 2, 1), scale=20.0):
    """bf16 N(0,1) KV with outlier channel runs scaled by `scale` (4% of channels per head)."""
    import torch
    x = torch.randn((1, heads, tokens, 128), generator=gen, device=device, dtype=torch.float32)
    for h in range(heads):
        perm = torch.randperm(120, generator=gen, device=device)[: len(frac_groups)].tolist()
        start = 0
        for w, p in zip(frac_groups, sorted(perm)):
            lo = max(start, p)
            lo = min(lo, 128 - w)
            x[0, h, :, lo:lo + w] *= scale
            start = lo + w + 1
    return x.to(torch.bfloat16)


def build_layer(seed, device, H=4, G=7, n_blocks=128, block=256, sink=4, tail=128, frac_groups=(2, 2, 1),
                k4_values=False):
    import torch
    from inquant.cache import _quantize_temporal_blocks
    from inquant.codec import CodecConfig
    from inquant.triton_attention import PackedDecodeState, SharedDecodeWorkspace
    from inquant.value_codec import quantize_value_blocks
    gen = torch.Generator(device=device).manual_seed(seed)
    k = kv_tensor(gen, H, n_blocks * block, device, frac_groups=frac_groups)
    v = kv_tensor(gen, H, n_blocks * block, device, frac_groups=frac_groups)
    cfg = CodecConfig(donor_policy="min_error")
    kb = _quantize_temporal_blocks(k, n_blocks, block, cfg)
    # K4-coded values (CacheConfig's default value_bits=None) or V2 with 64-channel groups
    vb = _quantize_temporal_blocks(v, n_blocks, block, cfg) if k4_values else quantize_value_blocks(v, n_blocks, block, 2, 64)
    del k, v
    layer = {
        "q": torch.randn((1, H * G, 1, 128), generator=gen, device=device).to(torch.bfloat16),
        "sink_k": kv_tensor(gen, H, sink, device), "sink_v": kv_tensor(gen, H, sink, device),
        "tail_k": kv_tensor(gen, H, tail, device), "tail_v": kv_tensor(gen, H, tail, device),
        "kb": kb, "vb": vb,
    }
    layer["state"] = PackedDecodeState(kb, vb, workspace_pool=None)
    return layer


def algorithmic_bytes(layer) -> int:
    H = layer["kb"][0].shape[1]
    n = len(layer["kb"])
    b = 0
    k4_values = not hasattr(layer["vb"][0], "offsets")
    for k, v in zip(layer["kb"], layer["vb"]):
        b += k.payload.numel() + k.scales.numel() * 4 + k.padding.numel() * 4
        if k4_values:
            b += v.payload.numel() + v.scales.numel() * 4 + v.padding.numel() * 4
        else:
            b += v.payload.numel() + (v.scales.numel() + v.offsets.numel()) * 2
    b += n * H * 128 * (2 if k4_values else 1)   # int8 role maps read per (block, head)
    b += n * 6 * 8            # pointer table
    for name in ("sink_k", "sink_v", "tail_k", "tail_v"):
        b += layer[name].numel() * 2
    b += 2 * layer["q"].numel() * 2   # Q read + O write (bf16)
    return b


def decode_all(layers, outs):
    for layer, out in zip(layers, outs):
        layer["state"].decode(layer["q"], sink_key=layer["sink_k"], sink_value=layer["sink_v"],
                              residual_key=layer["tail_k"], residual_value=layer["tail_v"], output=out)


def time_decode(layers, steps, warmup, use_graph):
    import torch
    outs = [torch.empty_like(l["q"]) for l in layers]
    stream = torch.cuda.current_stream()
    for _ in range(max(1, warmup)):
        decode_all(layers, outs)
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            decode_all(layers, outs)          # warm the capture stream
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                decode_all(layers, outs)
        torch.cuda.synchronize()
        for _ in range(max(1, warmup)):
            graph.replay()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        if graph is not None:
            graph.replay()
        else:
            decode_all(layers, outs)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    return ms, outs


def _graph_replay_us(device, launch, per_replay, steps=50):
    """Microseconds per unit of `launch` (per_replay units per call),
    captured once and replayed `steps` times."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launch()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            launch()
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1e3 / steps / per_replay


def decode_breakdown(layers, device):
    """Config 2 decode split into its launches, each timed as 28 x rotated
    sets of graph nodes: the full decode (partitions kernel + merge kernel),
    the merge kernel alone on the partials the decode left in each layer's
    workspace (it must reproduce the decode's outputs exactly), and a
    one-element fill kernel (the launch floor of one graph node)."""
    import torch
    from inquant import _native as nat
    lib = nat.lib()
    n = len(layers)
    ms, outs = time_decode(layers, 50, 5, True)
    full_us = ms * 1e3 / n
    q = layers[0]["q"]
    hq = q.shape[1]
    parts = lib.iq_decode_partitions(len(layers[0]["kb"]), layers[0]["sink_k"].shape[2],
                                     layers[0]["tail_k"].shape[2], 1)
    merged = [torch.empty_like(o) for o in outs]

    def merges():
        st = nat.stream_handle(q.device)
        for layer, out in zip(layers, merged):
            ws = layer["state"]._workspace
            nat.check(lib.iq_decode_merge(ws.data_ptr(), parts, hq, out.data_ptr(), nat.dtype_code(out.dtype), st))

    merge_us = _graph_replay_us(device, merges, n)
    assert all(torch.equal(a, b) for a, b in zip(merged, outs)), "the merge alone must reproduce the decode"
    cells = [torch.zeros(1, device=device) for _ in range(n)]

    def fills():
        for c in cells:
            c.fill_(1.0)

    floor_us = _graph_replay_us(device, fills, n)
    return {"decode_us_per_layer": round(full_us, 3), "merge_alone_us": round(merge_us, 3),
            "launch_floor_us": round(floor_us, 3), "partitions_kernel_us": round(full_us - merge_us, 3),
            "partitions": parts, "layers": n,
            "note": "full = partitions kernel + merge kernel; each figure includes its graph node's launch"}


def time_decode_k4_values(device, layers=28, steps=20, warmup=3):
    """Config 2 shape with K4-coded values (the reference CacheConfig default,
    value_bits=None): 28 layers of 32768 packed tokens + 4 sink + 128 tail."""
    import torch
    lay = [build_layer(5000 + i, device, k4_values=True) for i in range(layers)]
    torch.cuda.synchronize()
    per_layer = algorithmic_bytes(lay[0])
    ms, _ = time_decode(lay, steps, warmup, True)
    us = ms * 1e3 / layers
    out = {"layers": layers, "us_per_layer": round(us, 3), "bytes_per_layer": per_layer,
           "gbs": round(per_layer / (us * 1e-6) / 1e9, 2),
           "hbm_frac": round(per_layer / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del lay
    torch.cuda.empty_cache()
    return out


def time_decode_cfg3(device, layers=32, steps=20, warmup=3):
    """Config 3 decode: Mistral-7B shape, 32 query heads over 8 KV heads, 32768
    packed tokens (outliers at 8% of channels in 3-wide runs) + 4 sink + 128
    tail per layer, 32 layers replayed as one HIP graph."""
    import torch
    lay = [build_layer(3000 + i, device, H=8, G=4, frac_groups=(3, 3, 3, 1)) for i in range(layers)]
    torch.cuda.synchronize()
    per_layer = algorithmic_bytes(lay[0])
    ms, _ = time_decode(lay, steps, warmup, True)
    us = ms * 1e3 / layers
    out = {"layers": layers, "us_per_layer": round(us, 3), "bytes_per_layer": per_layer,
           "gbs": round(per_layer / (us * 1e-6) / 1e9, 2),
           "hbm_frac": round(per_layer / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del lay
    torch.cuda.empty_cache()
    return out


def time_encode(device, sets=4, cycles=3):
    """Mistral-7B layer encode (config 3): K4 min_error + V2 g64 of [1, 8, 32768, 128]
    bf16.  `sets` distinct layers (inputs and outputs, 4 x 162 MB = 648 MB,
    more than twice the 256 MB Infinity Cache) are encoded in turn, `cycles`
    times, in one HIP graph, so every encode reads its layer from HBM."""
    import torch
    from inquant import _native as nat
    H, T, B = 8, 32768, 256
    nb = T // B
    S = 16
    lib = nat.lib()
    bad = torch.zeros(2, dtype=torch.int32, device=device)
    work = []
    for i in range(sets):
        gen = torch.Generator(device=device).manual_seed(3 + i)
        k = kv_tensor(gen, H, T, device, frac_groups=(3, 3, 3, 1))
        v = kv_tensor(gen, H, T, device, frac_groups=(3, 3, 3, 1))
        w = {"k": k, "v": v,
             "kb": k[0].reshape(H, nb, B, 128).permute(1, 0, 2, 3),
             "vb": v[0].reshape(H, nb, B, 128).permute(1, 0, 2, 3),
             "pay": torch.empty((nb, H, B, 64), dtype=torch.uint8, device=device),
             "sc": torch.empty((nb, H, 128), dtype=torch.float32, device=device),
             "src": torch.empty((nb, H, S), dtype=torch.uint8, device=device),
             "don": torch.empty((nb, H, S), dtype=torch.uint8, device=device),
             "pad": torch.empty((nb, H, S), dtype=torch.float32, device=device),
             "vpay": torch.empty((nb, H, B, 32), dtype=torch.uint8, device=device),
             "vsc": torch.empty((nb, H, B, 2), dtype=torch.float16, device=device),
             "voff": torch.empty((nb, H, B, 2), dtype=torch.float16, device=device)}
        work.append(w)

    def once(w, st):
        # the cache's block encode (keys K4, values V2 in one launch)
        nat.check(lib.iq_kv_quantize(w["kb"].data_ptr(), w["vb"].data_ptr(), nat.IQ_BF16, nat.strides4(w["kb"]),
                                     nat.strides4(w["vb"]), nb, H, B, 128, S, 8, 1, w["pay"].data_ptr(),
                                     w["sc"].data_ptr(), w["src"].data_ptr(), w["don"].data_ptr(), 1,
                                     w["pad"].data_ptr(), 2, 64, w["vpay"].data_ptr(), w["vsc"].data_ptr(),
                                     w["voff"].data_ptr(), bad.data_ptr(), bad.data_ptr() + 4, st))

    def once_k4v(w, st):
        # the same layer with K4-coded values (the cache's default
        # value_bits=None): keys and values K4 in one launch (iq_k4_quantize_kv);
        # the value outputs reuse the V2 payload storage
        vk = w.setdefault("vk", [torch.empty_like(w[n]) for n in ("pay", "sc", "src", "don", "pad")])
        nat.check(lib.iq_k4_quantize_kv(w["kb"].data_ptr(), w["vb"].data_ptr(), nat.IQ_BF16, nat.strides4(w["kb"]),
                                        nat.strides4(w["vb"]), nb, H, B, 128, S, 8, 1, w["pay"].data_ptr(),
                                        w["sc"].data_ptr(), w["src"].data_ptr(), w["don"].data_ptr(),
                                        w["pad"].data_ptr(), *[t.data_ptr() for t in vk], 1, bad.data_ptr(),
                                        bad.data_ptr() + 4, st))

    def rotated(fn):
        def launch():
            st = nat.stream_handle(torch.device(device))
            for _ in range(cycles):
                for w in work:
                    fn(w, st)
        return launch

    def once_values(w, st):
        # quantize_values alone (a8): the layer's values, V2 g64 (v_encode_rows)
        nat.check(lib.iq_v_quantize(w["vb"].data_ptr(), nat.IQ_BF16, nat.strides4(w["vb"]), nb, H, B, 128, 2, 64,
                                    w["vpay"].data_ptr(), w["vsc"].data_ptr(), w["voff"].data_ptr(),
                                    bad.data_ptr() + 4, st))

    calls = sets * cycles
    ms = _graph_us(device, rotated(once), reps=1) * 1e-3 / calls
    assert bad.tolist() == [0, 0]
    ms_k4v = _graph_us(device, rotated(once_k4v), reps=1) * 1e-3 / calls
    assert bad.tolist() == [0, 0]
    ms_v = _graph_us(device, rotated(once_values), reps=1) * 1e-3 / calls
    assert bad.tolist() == [0, 0]
    w = work[0]
    enc_bytes = 2 * w["k"].numel() * 2 + w["pay"].numel() + w["sc"].numel() * 4 + w["src"].numel() * 2 \
        + w["pad"].numel() * 4 + w["vpay"].numel() + w["vsc"].numel() * 4
    v_bytes = w["v"].numel() * 2 + w["vpay"].numel() + w["vsc"].numel() * 4

    # reuse_map (a4/a5): sources and min_error donors of every (block, head)
    # row of the layer from its saliency and donor error (1024 rows of 128)
    g = torch.Generator(device=device).manual_seed(8)
    sal = torch.rand((nb * H, 128), generator=g, device=device)
    err = torch.rand((nb * H, 128), generator=g, device=device)
    rsrc = torch.empty((nb * H, S), dtype=torch.int64, device=device)
    rdon = torch.empty_like(rsrc)

    def reuse():
        nat.check(lib.iq_reuse_map(sal.data_ptr(), err.data_ptr(), nb * H, 128, S, rsrc.data_ptr(), rdon.data_ptr(),
                                   nat.stream_handle(torch.device(device))))

    us_reuse = _graph_us(device, reuse, reps=20)

    # quantize() of a whole layer's keys as one block ([1, 8, 32768, 128]: the
    # codec API on rows of any length, statistics over all 32768 tokens)
    from inquant.codec import CodecConfig, quantize
    long_ms = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        quantize(work[0]["k"], CodecConfig(donor_policy="min_error"))
        torch.cuda.synchronize()
        long_ms.append((time.perf_counter() - t0) * 1e3)
    del work
    torch.cuda.empty_cache()
    return {"encode_mtok_s": T / (ms * 1e-3) / 1e6, "encode_ms_per_layer": ms,
            "encode_gbs": enc_bytes / (ms * 1e-3) / 1e9, "encode_bytes_per_layer": enc_bytes,
            "k4_values_mtok_s": T / (ms_k4v * 1e-3) / 1e6, "k4_values_ms_per_layer": ms_k4v,
            "values_only_mtok_s": T / (ms_v * 1e-3) / 1e6, "values_only_ms_per_layer": ms_v,
            "values_only_gbs": v_bytes / (ms_v * 1e-3) / 1e9,
            "reuse_map_us": us_reuse, "reuse_map_rows": nb * H,
            "quantize_one_block_ms": sorted(long_ms)[1], "quantize_one_block_tokens": T, "quantize_one_block_heads": H,
            "rotated_layers": sets, "rotated_bytes": sets * enc_bytes}


def _graph_us(device, launch, reps=10, timed=5):
    """Microseconds per call of `launch` (native launches on the current
    stream), replayed `reps` times in one HIP graph: the median of `timed`
    timed replays after one untimed one (a single replay of a short graph
    moves with the clock state the previous work left)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launch()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(reps):
                launch()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(timed):
        start.record()
        graph.replay()
        stop.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop))
    return sorted(times)[len(times) // 2] * 1e3 / reps


def time_next_rows(device, sets=8):
    """The rows next to the decode path, inputs resident, launches replayed in
    a HIP graph: materialize (K4 keys and V2 g64 values of one config 2 layer,
    4 heads x 32768 tokens, dequantized to bf16), encode into 256- and
    16-token pages (keys K4 min_error + role map + values V2 of 32768 tokens
    x 4 heads, one launch), unpack those pages back to dense bf16 K and V,
    write codec outputs into pages (write_codec_pages), and causal prefill attention over exact K/V (one 8192-token Qwen2.5-7B
    sequence, 28 query heads over 4 KV heads, bf16).  Materialize and the
    page encodes run over `sets` distinct layers in turn (8 x ~81 MB =
    ~650 MB, above the 256 MB Infinity Cache), so each call reads its inputs
    from HBM; the unpacks read the `sets` page pools in turn (8 x 14 MB)."""
    import torch
    from inquant import _native as nat
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant_vllm import PageLayout
    lib = nat.lib()
    H, T, D = 4, 32768, 128
    gen = torch.Generator(device=device).manual_seed(6)
    kv = [(kv_tensor(gen, H, T, device), kv_tensor(gen, H, T, device)) for _ in range(sets)]
    k, v = kv[0]
    out = {}

    # materialize: both dequantizers into bf16 K and V
    mats = []
    for kk, vv in kv:
        pk = quantize(kk, CodecConfig(donor_policy="min_error"))
        pv = quantize_values(vv, 2, 64)
        mats.append((pk, pv, torch.empty_like(kk), torch.empty_like(vv)))
    S = mats[0][0].salient_channels.shape[-1]

    def materialize():
        st = nat.stream_handle(torch.device(device))
        for pk, pv, kd, vd in mats:
            nat.check(lib.iq_k4_dequantize(pk.payload.data_ptr(), pk.scales.data_ptr(),
                                           pk.salient_channels.data_ptr(), pk.donor_channels.data_ptr(), 1,
                                           pk.padding.data_ptr(), H, T, D, S, kd.data_ptr(), nat.IQ_BF16, st))
            nat.check(lib.iq_v_dequantize(pv.payload.data_ptr(), pv.scales.data_ptr(), pv.offsets.data_ptr(),
                                          H * T, D, 2, 64, vd.data_ptr(), nat.IQ_BF16, st))

    us = _graph_us(device, materialize, reps=2) / sets
    pk, pv, kd, vd = mats[-1]
    assert torch.equal(kd, pk.dequantize(torch.bfloat16)) and torch.equal(vd, pv.dequantize(torch.bfloat16))
    mat_bytes = sum(t.numel() * t.element_size() for t in pk.tensors.values()) \
        + sum(t.numel() * t.element_size() for t in (pv.payload, pv.scales, pv.offsets)) + 2 * k.numel() * 2
    out["materialize_cfg2"] = {"us_per_layer": round(us, 3), "bytes_per_layer": mat_bytes,
                               "gbs": round(mat_bytes / (us * 1e-6) / 1e9, 2),
                               "hbm_frac": round(mat_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                               "rotated_layers": sets}
    del mats, pk, pv, kd, vd

    # encode into pages (the plugin's seal of a prefill: 256-token pages, the
    # reference layout's largest, and the 16-token pages of config 4), flags
    # written on the device
    for B in (256, 16):
        layout = PageLayout(B, H)
        P = T // B
        jobs = []
        for kk, vv in kv:
            jobs.append((kk[0].reshape(H, P, B, D).transpose(0, 1), vv[0].reshape(H, P, B, D).transpose(0, 1),
                         torch.empty((P, layout.page_bytes), dtype=torch.uint8, device=device)))
        ids = torch.arange(P, dtype=torch.int32, device=device)
        flags = torch.zeros(8, dtype=torch.int32, device=device)     # two (key, value, page id) triples

        def encode_pages():
            st = nat.stream_handle(torch.device(device))
            for kp, vp, pool in jobs:
                nat.check(lib.iq_encode_pages(kp.data_ptr(), vp.data_ptr(), nat.IQ_BF16, nat.strides4(kp),
                                              nat.strides4(vp), P, H, B, pool.data_ptr(), P, ids.data_ptr(), 4,
                                              flags.data_ptr(), flags.data_ptr() + 16, st))

        us = _graph_us(device, encode_pages, reps=2) / sets
        assert flags[:3].tolist() == [0, 0, 0]
        enc_bytes = 2 * k.numel() * 2 + P * layout.page_bytes
        out[f"encode_pages_b{B}"] = {"tokens": T, "heads": H, "page_tokens": B, "us": round(us, 3),
                                     "mtok_s": round(T / us, 2), "bytes": enc_bytes,
                                     "gbs": round(enc_bytes / (us * 1e-6) / 1e9, 2),
                                     "hbm_frac": round(enc_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                     "rotated_layers": sets}

        # the pages just written, unpacked to dense bf16 K and V [P, H, B, 128]
        # (unpack_pages_reference): every page read once, both outputs written
        kd = torch.empty((P, H, B, D), dtype=torch.bfloat16, device=device)
        vd = torch.empty_like(kd)

        def unpack_pages():
            st = nat.stream_handle(torch.device(device))
            for _, _, pool in jobs:
                nat.check(lib.iq_unpack_pages(pool.data_ptr(), P, H, B, kd.data_ptr(), vd.data_ptr(), nat.IQ_BF16,
                                              st))

        us = _graph_us(device, unpack_pages, reps=2) / sets
        unp_bytes = P * layout.page_bytes + 2 * kd.numel() * 2
        out[f"unpack_pages_b{B}"] = {"tokens": T, "heads": H, "page_tokens": B, "us": round(us, 3),
                                     "bytes": unp_bytes, "gbs": round(unp_bytes / (us * 1e-6) / 1e9, 2),
                                     "hbm_frac": round(unp_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                     "rotated_layers": sets}
        del kd, vd

        # write_codec_pages: each set's codec outputs (K4 min_error, V2 g64 of
        # [P, H, B, 128]) scattered into its pool at a random permutation of ids
        codecs = []
        for kp, vp, _ in jobs:
            codecs.append((quantize(kp.contiguous(), CodecConfig(donor_policy="min_error")),
                           quantize_values(vp.contiguous(), 2, 64)))
        perm = torch.randperm(P, generator=gen, device=device).to(torch.int32)

        def write_pages():
            st = nat.stream_handle(torch.device(device))
            for (pk, pv), (_, _, pool) in zip(codecs, jobs):
                nat.check(lib.iq_write_pages(pk.payload.data_ptr(), pk.scales.data_ptr(), pk.padding.data_ptr(),
                                             pk.salient_channels.data_ptr(), pk.donor_channels.data_ptr(),
                                             pk.salient_channels.element_size(), pv.payload.data_ptr(),
                                             pv.scales.data_ptr(), pv.offsets.data_ptr(), P, H, B, pool.data_ptr(),
                                             P, perm.data_ptr(), 4, st))

        us = _graph_us(device, write_pages, reps=2) / sets
        pk, pv = codecs[0]
        wr_bytes = (sum(t.numel() * t.element_size() for t in pk.tensors.values())
                    + sum(t.numel() * t.element_size() for t in (pv.payload, pv.scales, pv.offsets))
                    + P * layout.page_bytes)
        out[f"write_codec_pages_b{B}"] = {"tokens": T, "heads": H, "page_tokens": B, "us": round(us, 3),
                                          "bytes": wr_bytes, "gbs": round(wr_bytes / (us * 1e-6) / 1e9, 2),
                                          "hbm_frac": round(wr_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                          "rotated_layers": sets}
        del jobs, codecs, pk, pv
    del kv
    torch.cuda.empty_cache()

    # causal prefill attention over exact K/V
    Sq, Hq = 8192, 28
    q = torch.randn((Sq, Hq, D), generator=gen, device=device).to(torch.bfloat16)
    kq = k[0, :, :Sq].transpose(0, 1).contiguous()
    vq = v[0, :, :Sq].transpose(0, 1).contiguous()
    o = torch.empty_like(q)
    cu = torch.tensor([0, Sq], dtype=torch.int32, device=device)

    def prefill():
        st = nat.stream_handle(torch.device(device))
        nat.check(lib.iq_prefill_attention(q.data_ptr(), kq.data_ptr(), vq.data_ptr(), nat.IQ_BF16, q.stride(0),
                                           q.stride(1), kq.stride(0), kq.stride(1), vq.stride(0), vq.stride(1),
                                           cu.data_ptr(), 1, Sq, Hq, H, D, 128 ** -0.5, o.data_ptr(), o.stride(0),
                                           o.stride(1), nat.IQ_BF16, st))

    us = _graph_us(device, prefill, reps=3)
    flops = 4 * Hq * D * Sq * (Sq + 1) / 2          # Q.K^T and P.V over the causal triangle
    out["prefill_qwen_8k"] = {"tokens": Sq, "us": round(us, 1), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                              "mfma_frac": round(flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    return out


def time_paged(device, layers=4, n_seq=16, block=16, H=4, G=7, seed=4, steps=20, lifecycle_steps=24):
    """Config 4: batched paged decode, 16 sequences with contexts ~ U{2048..32768}
    in 16-token pages of the vLLM layout, random physical page order, per-sequence
    BF16 sink (4) and open page.  Each of `layers` independent layers (rotated,
    so the working set exceeds the Infinity Cache) is built by the plugin's
    many-request lifecycle (InQuantBatchImpl: one prefill step of the 16
    requests seals their full pages and keeps sink and open page in their
    dense slots); the decode launches the lifecycle makes for the next token
    are then replayed back to back in a graph.  `lifecycle_steps` whole decode
    steps through InQuantBatchImpl.forward (new-token writes, the batched
    decode, the seals of filled pages, host included) are timed eagerly, and
    the causal prefill of the first layer's 16 sequences (one varlen launch)
    alone in a graph."""
    import torch
    import inquant_vllm.backend as backend
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode_batch, work_list
    gen = torch.Generator(device="cpu").manual_seed(seed)
    ctx = torch.randint(2048, 32769, (n_seq,), generator=gen).tolist()
    pages = [c // block for c in ctx]
    tails = [c % block for c in ctx]
    need_pages = [(c + lifecycle_steps) // block + 1 for c in ctx]
    max_pages = max(pages)
    backend.configure(block_size=block, max_model_len=max(ctx) + lifecycle_steps + block)
    work, impls = [], []
    g = torch.Generator(device=device).manual_seed(seed)
    qsl = [0]
    for c in ctx:
        qsl.append(qsl[-1] + c)
    for _ in range(layers):
        impl = backend.InQuantBatchImpl(H * G, 128, 128 ** -0.5, H, max_num_seqs=n_seq)
        pool = torch.empty((sum(need_pages), impl.layout.page_bytes), dtype=torch.uint8, device=device)
        perm = torch.randperm(sum(need_pages), generator=g, device=device).to(torch.int32)
        tables = torch.zeros((n_seq, max(need_pages)), dtype=torch.int32, device=device)
        first = 0
        for i, n in enumerate(need_pages):
            tables[i, :n] = perm[first:first + n]
            first += n
        ks = [kv_tensor(g, H, c, device)[0].transpose(0, 1) for c in ctx]
        vs = [kv_tensor(g, H, c, device)[0].transpose(0, 1) for c in ctx]
        k, v = torch.cat(ks), torch.cat(vs)
        del ks, vs
        q = torch.randn((qsl[-1], H * G, 128), generator=g, device=device).to(torch.bfloat16)
        meta = backend.InQuantBatchMetadata([f"seq{i}" for i in range(n_seq)],
                                            torch.tensor(qsl, dtype=torch.int32, device=device), qsl, list(ctx),
                                            tables, ())
        impl.forward(None, q, k, v, pool, meta, torch.empty_like(q))      # prefill: pools built by the lifecycle
        if not work:
            # the causal prefill of these 16 sequences alone (the lifecycle's
            # one varlen launch), replayed in a graph
            from inquant_vllm.kernels import prefill_attention
            cu = torch.tensor(qsl, dtype=torch.int32, device=device)
            pout = torch.empty_like(q)
            pf_us = _graph_us(device, lambda: prefill_attention(q, k, v, cu, max(ctx), 128 ** -0.5, pout), reps=2)
            pf_flops = sum(4 * H * G * 128 * c * (c + 1) / 2 for c in ctx)
            del pout
        del q, k, v
        slots = torch.tensor([impl.requests[f"seq{i}"].slot for i in range(n_seq)], dtype=torch.int32,
                             device=device)
        info = torch.tensor([[n, t + 1, 4] for n, t in zip(pages, tails)], dtype=torch.int32, device=device)
        qd = torch.randn((n_seq, H * G, 128), generator=g, device=device).to(torch.bfloat16)
        work.append((qd, pool, tables, info, impl.dense, slots, SharedDecodeWorkspace(), torch.empty_like(qd)))
        impls.append((impl, pool, tables))
    torch.cuda.synchronize()
    layout = impls[0][0].layout
    items = torch.tensor(work_list(pages, block), dtype=torch.int32, device=device)

    st = torch.cuda.Stream()                # the workspaces are pinned to the stream they first run on
    st.wait_stream(torch.cuda.current_stream())

    def graphed_us(listed):
        def step():
            for q, pool, tables, info, dense, slots, ws, out in work:
                paged_decode_batch(q, pool, tables, info, dense, max_pages, layout, ws, 128 ** -0.5, out,
                                   dense_slots=slots, work=items if listed else None)

        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=st):
                step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3 / steps / layers

    us_grid = graphed_us(False)
    us = graphed_us(True)
    # algorithmic bytes per layer: every page of every sequence, its block-table
    # entry, the live dense sink/open-page rows, Q and O
    bytes_layer = sum(pages) * (layout.page_bytes + 4) + sum(4 + t + 1 for t in tails) * 2 * H * 128 * 2 \
        + 2 * n_seq * H * G * 128 * 2
    # whole lifecycle decode steps of the first layer (host included, eager)
    impl, pool, tables = impls[0]
    qd = torch.randn((n_seq, H * G, 128), generator=g, device=device).to(torch.bfloat16)
    kd = torch.randn((n_seq, H, 128), generator=g, device=device).to(torch.bfloat16)
    out = torch.empty_like(qd)
    qsl1 = list(range(n_seq + 1))
    qsl1_dev = torch.tensor(qsl1, dtype=torch.int32, device=device)
    lens = list(ctx)
    seals0 = impl.seal_calls
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(lifecycle_steps):
        lens = [n + 1 for n in lens]
        meta = backend.InQuantBatchMetadata([f"seq{i}" for i in range(n_seq)], qsl1_dev, qsl1, lens, tables, ())
        impl.forward(None, qd, kd, kd, pool, meta, out)
    torch.cuda.synchronize()
    life_us = (time.perf_counter() - t0) * 1e6 / lifecycle_steps
    return {"sequences": n_seq, "page_tokens": block, "mean_ctx": round(sum(ctx) / n_seq, 1),
            "us_per_layer": round(us, 3), "bytes_per_layer": bytes_layer,
            "gbs": round(bytes_layer / (us * 1e-6) / 1e9, 2),
            "hbm_frac": round(bytes_layer / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(n_seq / (us * 1e-6), 1), "layers_rotated": layers,
            "work_items": int(items.numel()), "us_per_layer_full_grid": round(us_grid, 3),
            "built_by": "InQuantBatchImpl prefill of the 16 requests",
            "lifecycle_step_us": round(life_us, 1), "lifecycle_steps": lifecycle_steps,
            "lifecycle_seal_launches": impl.seal_calls - seals0,
            "prefill_varlen": {"sequences": n_seq, "tokens": sum(ctx), "max_seqlen": max(ctx),
                               "us": round(pf_us, 1), "tflops": round(pf_flops / (pf_us * 1e-6) / 1e12, 1),
                               "mfma_frac": round(pf_flops / (pf_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}}


def time_append(device, H=4, packed_tokens=32768, validate_positions=True, seals=7):
    """Config 2 append, through the cache API of one Qwen2.5-7B layer (32K packed
    context): 128 single-token appends (dense tail 128 -> 256, no seal), then
    `seals` times the append that seals one 256-token block (K4 + V2 encode)
    starting from a 383-token tail and the decode-state metadata append for
    that block (medians reported).  The sealing append synchronizes on its
    own flag read, so its wall clock to return covers its device work; the
    metadata append returns before its one launch finishes (host time).
    Last, the layer's dense K/V through materialize() (median wall clock)."""
    import torch
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.triton_attention import PackedDecodeState
    g = torch.Generator(device=device).manual_seed(11)
    cfg = CacheConfig(codec=CodecConfig(donor_policy="min_error"), value_bits=2, value_group_size=64,
                      validate_positions=validate_positions)
    cache = InQuantCache(cfg)
    n0 = 4 + packed_tokens + 128
    extra = 768 + 256 * seals
    k = kv_tensor(g, H, n0 + extra, device)
    v = kv_tensor(g, H, n0 + extra, device)
    cache.update(k[:, :, :n0], v[:, :, :n0], 0)
    layer = cache._layers[0]
    # one position tensor per decode step, shared by the layers in a model
    # (Transformers builds cache_position once per step): device slices, no
    # host-to-device copy inside the timed loop
    positions = torch.arange(n0 + extra, device=device)
    state = PackedDecodeState(list(layer.key_blocks), list(layer.value_blocks))
    pos = n0
    # one full cycle first (tail 128 -> 384 -> seal -> 128), so that the timed
    # window sees warm allocator blocks and loaded kernels
    for _ in range(256):
        cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                   {"cache_position": positions[pos:pos + 1]})
        pos += 1
    state.extend(list(layer.key_blocks), list(layer.value_blocks))
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
    ev[0].record()
    t0 = time.perf_counter()
    for _ in range(128):
        cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                   {"cache_position": positions[pos:pos + 1]})
        pos += 1
    ev[1].record()
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0) * 1e6 / 128
    seal_us, meta_us = [], []
    for _ in range(seals):
        while layer.tail.count < 383:    # tail up to 383 (no seal)
            cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                       {"cache_position": positions[pos:pos + 1]})
            pos += 1
        # wall clock of the call: the seal synchronizes once itself (its
        # position and non-finite checks), so its work is done on the device
        # when it returns (asserted: nothing left on the stream)
        torch.cuda.synchronize()
        blocks_before = len(layer.key_blocks)
        t0 = time.perf_counter()
        cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                   {"cache_position": positions[pos:pos + 1]})
        t1 = time.perf_counter()
        assert torch.cuda.current_stream().query(), "the sealing append returned with work queued"
        torch.cuda.synchronize()
        pos += 1
        assert len(layer.key_blocks) == blocks_before + 1
        kb, vb = list(layer.key_blocks), list(layer.value_blocks)
        # the metadata append is asynchronous (one ~3 us launch behind it):
        # host time to return
        t2 = time.perf_counter()
        state.extend(kb, vb)
        t3 = time.perf_counter()
        torch.cuda.synchronize()
        seal_us.append((t1 - t0) * 1e6)
        meta_us.append((t3 - t2) * 1e6)
    seal_bytes = 2 * H * 256 * 128 * 2 + (16384 + 512 + 32 + 64 + 8192 + 2048) * H + 64 + H * 128
    # the layer's dense K and V through the cache API (what update() returns to
    # a non-fused attention): wall clock of materialize() to its results
    mat_us = []
    for _ in range(10):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dense_k, dense_v = cache.materialize(0)
        torch.cuda.synchronize()
        mat_us.append((time.perf_counter() - t0) * 1e6)
    mat_tokens = dense_k.shape[2]
    del dense_k, dense_v
    return {"append_us_per_token": round(ev[0].elapsed_time(ev[1]) * 1e3 / 128, 2),
            "append_host_us_per_token": round(host_us, 2),
            "seal_us": round(sorted(seal_us)[len(seal_us) // 2], 2),
            "metadata_append_us": round(sorted(meta_us)[len(meta_us) // 2], 2),
            "seals_timed": seals, "seal_bytes": seal_bytes,
            "materialize_api_us": round(sorted(mat_us)[len(mat_us) // 2], 1), "materialize_api_tokens": mat_tokens}


def time_append_step(device, H=4, packed_tokens=32768, layers=28):
    """Config 2 append as a model makes it: every decode step appends one
    token to each layer of a 28-layer cache (32K packed context per layer),
    the layers sharing the step's cache_position tensor.  One full cycle of
    256 steps is timed (tail 128 -> 383, then the step on which all 28
    layers seal a 256-token block back to 128): the mean step, the mean of
    the steps that seal nothing, and the sealing step."""
    import torch
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    g = torch.Generator(device=device).manual_seed(12)
    cfg = CacheConfig(codec=CodecConfig(donor_policy="min_error"), value_bits=2, value_group_size=64)
    cache = InQuantCache(cfg)
    n0 = 4 + packed_tokens + 128
    steps = 256
    k = kv_tensor(g, H, n0 + 2 * steps, device)
    v = kv_tensor(g, H, n0 + 2 * steps, device)
    for i in range(layers):
        cache.update(k[:, :, :n0], v[:, :, :n0], i)
    positions = torch.arange(n0 + 2 * steps, device=device)
    times = []

    def step(pos):
        p = positions[pos:pos + 1]
        kk, vv = k[:, :, pos:pos + 1], v[:, :, pos:pos + 1]
        t0 = time.perf_counter()
        for i in range(layers):
            cache.append_for_attention(kk, vv, i, {"cache_position": p})
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    pos = n0
    for _ in range(steps):               # one warm cycle (allocator blocks, kernels, views)
        step(pos)
        pos += 1
    for _ in range(steps):
        times.append(step(pos))
        pos += 1
    blocks = len(cache._layers[0].key_blocks)
    seal_at = max(range(steps), key=lambda i: times[i])
    plain = [t for i, t in enumerate(times) if i != seal_at]
    assert cache.get_seq_length(layers - 1) == n0 + 2 * steps and blocks == packed_tokens // 256 + 2
    return {"layers": layers, "cycle_steps": steps,
            "append_step_us": round(sum(plain) / len(plain) * 1e6, 1),
            "append_us_per_layer_token": round(sum(plain) / len(plain) * 1e6 / layers, 2),
            "sealing_step_us": round(times[seal_at] * 1e6, 1),
            "cycle_mean_step_us": round(sum(times) / steps * 1e6, 1)}


def time_step_graph(device, H=4, HQ=28, packed_tokens=32768, layers=28, reps=50):
    """Config 2 decode step of a 28-layer model captured as one HIP graph:
    per layer, the one-token append (append_for_attention, one
    iq_tail_append_row launch) and the packed decode of the view it returns
    (sink + 128 blocks + tail, two launches).  The replays rewrite the same
    tail row and decode the same length, so they time the device work of one
    step without the host's per-call cost; the same step run eagerly is
    timed beside it, and the 28 appends alone as a second graph.  The
    captured appends take no cache_position: the
    position check reads a device flag back on the host, which a graph
    cannot do."""
    import torch
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    from inquant.triton_attention import PackedDecodeState
    g = torch.Generator(device=device).manual_seed(13)
    cfg = CacheConfig(codec=CodecConfig(donor_policy="min_error"), value_bits=2, value_group_size=64)
    cache = InQuantCache(cfg)
    n0 = 4 + packed_tokens + 128
    k = kv_tensor(g, H, n0 + 64, device)
    v = kv_tensor(g, H, n0 + 64, device)
    for i in range(layers):
        cache.update(k[:, :, :n0], v[:, :, :n0], i)
    states = [PackedDecodeState(list(cache._layers[i].key_blocks), list(cache._layers[i].value_blocks))
              for i in range(layers)]
    q = torch.randn((1, HQ, 1, 128), generator=g, device=device).to(torch.bfloat16)
    outs = [torch.empty_like(q) for _ in range(layers)]

    def step(pos):
        kk, vv = k[:, :, pos:pos + 1], v[:, :, pos:pos + 1]
        for i in range(layers):
            view = cache.append_for_attention(kk, vv, i)
            states[i].decode(q, sink_key=view.sink_key, sink_value=view.sink_value, residual_key=view.residual_key,
                             residual_value=view.residual_value, output=outs[i])

    pos = n0
    for _ in range(8):                   # warm: kernels loaded, views and workspaces built
        step(pos)
        pos += 1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(16):
        step(pos)
        pos += 1
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) * 1e6 / 16
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        step(pos)
        pos += 1
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            step(pos)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / reps
    # the 28 appends alone, captured the same way (one launch per layer)
    appends = torch.cuda.CUDAGraph()
    kk, vv = k[:, :, pos:pos + 1], v[:, :, pos:pos + 1]
    with torch.cuda.stream(s):
        with torch.cuda.graph(appends, stream=s):
            for i in range(layers):
                cache.append_for_attention(kk, vv, i)
    torch.cuda.synchronize()
    for _ in range(3):
        appends.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        appends.replay()
    stop.record()
    torch.cuda.synchronize()
    append_us = start.elapsed_time(stop) * 1e3 / reps
    assert cache._layers[0].tail.count < cfg.residual_length + cfg.block_size     # no seal inside the graphs
    return {"layers": layers, "graph_step_us": round(us, 1), "graph_us_per_layer": round(us / layers, 2),
            "eager_step_us": round(eager_us, 1), "eager_us_per_layer": round(eager_us / layers, 2),
            "launches_per_layer": 3, "graph_append_step_us": round(append_us, 1),
            "graph_append_us_per_layer": round(append_us / layers, 2)}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, budget_s: float, max_reps: int = 200) -> tuple[float, int]:
    """Seconds per call of fn, repeated until `budget_s` has passed (at least once)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or reps >= max_reps:
            return dt / reps, reps


def cpu_baseline(layer, device):
    """The C oracle (the CPU restatement of the reference's codec and of its
    dequantize-then-attend decode) timed on this host, on all cores and on
    one thread, on bounded samples of the benchmark's workloads:
      decode: one config-2 layer restricted to 16 of its 128 packed blocks
              (+ sink and tail): K4/V2 dequantize to bf16, fp64 attention;
      encode: K4 min_error + V2 g64 of 8 blocks x 8 heads of a config-3 layer
              (2048 tokens of the 32768)."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle import oracle
    from kvcase import oracle_dequant_k4, oracle_dequant_v, to_np
    from dataclasses import replace
    cores = len(os.sched_getaffinity(0))
    n = min(16, len(layer["kb"]))
    kb, vb = layer["kb"][:n], layer["vb"][:n]
    q = to_np(layer["q"])[0, :, 0]
    sink_k, sink_v = to_np(layer["sink_k"])[0], to_np(layer["sink_v"])[0]
    tail_k, tail_v = to_np(layer["tail_k"])[0], to_np(layer["tail_v"])[0]
    blocks = [(replace(k, **{f: t.cpu() for f, t in k.tensors.items()}),
               replace(v, **{f: t.cpu() for f, t in v.tensors.items()})) for k, v in zip(kb, vb)]

    def decode():
        ks = [sink_k] + [oracle_dequant_k4(k, "bfloat16") for k, _ in blocks] + [tail_k]
        vs = [sink_v] + [oracle_dequant_v(v, "bfloat16") for _, v in blocks] + [tail_v]
        oracle.attend(q, np.concatenate(ks, 1), np.concatenate(vs, 1), 128 ** -0.5)

    g = torch.Generator(device=device).manual_seed(33)
    enc_blocks, H, B = 8, 8, 256
    kx = kv_tensor(g, H, enc_blocks * B, device, frac_groups=(3, 3, 3, 1))
    vx = kv_tensor(g, H, enc_blocks * B, device, frac_groups=(3, 3, 3, 1))
    kx = np.ascontiguousarray(kx[0].float().reshape(H, enc_blocks, B, 128).transpose(0, 1).cpu().numpy())
    vx = np.ascontiguousarray(vx[0].float().reshape(H, enc_blocks, B, 128).transpose(0, 1).cpu().numpy())

    def encode():
        oracle.k4_quantize(kx, 8, 0.125, "min_error")
        oracle.v_quantize(vx, 2, 64)

    sample_bytes = algorithmic_bytes(layer) * n / len(layer["kb"])
    enc_tokens = enc_blocks * B
    result = {}
    for threads, tag in ((cores, ""), (1, "_1t")):
        oracle.set_threads(threads)
        dec_s, dec_reps = _timed(decode, 4.0)
        enc_s, enc_reps = _timed(encode, 4.0)
        result["decode_gbs" + tag] = sample_bytes / dec_s / 1e9
        result["encode_mtok_s" + tag] = enc_tokens / enc_s / 1e6
        result["reps" + tag] = [dec_reps, enc_reps]
    oracle.set_threads(cores)
    return {"value": round(result["decode_gbs"], 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"decode: 1 config-2 layer, {n} of {len(layer['kb'])} packed blocks + sink + tail, oracle "
                      f"K4/V2 dequantize to bf16 then fp64 attention; encode: K4 min_error + V2 g64 of "
                      f"{enc_blocks} blocks x {H} heads (config 3); ~4 s per leg per thread count",
            "cpu_model": _cpu_model(),
            "decode_gbs_1thread": round(result["decode_gbs_1t"], 4),
            "encode_mtok_s": round(result["encode_mtok_s"], 4),
            "encode_mtok_s_1thread": round(result["encode_mtok_s_1t"], 4),
            "reps": {"all_cores": result["reps"], "one_thread": result["reps_1t"]}}


def main():
    args = parse()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported on this single-GPU build "
              "(the decode shards over KV heads with no exchange: each GPU runs the same kernel on "
              "its share of heads)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    device = "cuda:0"
    torch.cuda.set_device(0)
    rotate = max(1, args.rotate)
    layers = [build_layer(1000 + i, device, n_blocks=args.blocks) for i in range(args.layers * rotate)]
    torch.cuda.synchronize()
    if args.breakdown:
        print(json.dumps({"breakdown": "cfg2 decode", **decode_breakdown(layers, device)}))
        return
    per_layer = algorithmic_bytes(layers[0])
    step_bytes = sum(algorithmic_bytes(l) for l in layers) / rotate
    # one replay runs `rotate` steps, each over its own set of layers
    ms_replay, _ = time_decode(layers, args.steps, args.warmup, not args.no_graph)
    ms = ms_replay / rotate
    gbs = step_bytes / (ms * 1e-3) / 1e9
    layer_us = ms * 1e3 / args.layers
    achieved = per_layer / (layer_us * 1e-6) / 1e9
    enc = None if args.no_encode else time_encode(device)
    paged = None if args.no_paged else time_paged(device)
    nxt = None if args.no_next else time_next_rows(device)
    append = None
    if not args.no_append:
        append = time_append(device)
        # a controlled runner may skip the position check and its synchronization (cache.py:30-32)
        append["append_us_per_token_unvalidated"] = time_append(device, validate_positions=False)[
            "append_us_per_token"]
        append["step"] = time_append_step(device)
        append["step_graph"] = time_step_graph(device)
    cfg3 = None if args.no_cfg3 else time_decode_cfg3(device)
    k4v = None if args.no_k4_values else time_decode_k4_values(device)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 KV with 4% x20 outlier channel runs, seeded per layer)",
        "config": {"workload": "cfg2: Qwen2.5-7B decode, 28 layers x (32768 packed K4/V2 tokens in 256-token "
                               "blocks + 4 BF16 sink + 128 BF16 tail), Hq=28, H_kv=4, D=128, batch 1",
                   "layers": args.layers, "packed_tokens": args.blocks * 256, "graph": not args.no_graph,
                   "rotated_sets": rotate, "rotated_bytes": int(step_bytes * rotate)},
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_us_per_layer": round(layer_us, 3),
        "decode_tokens_per_s": round(1e3 / ms, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "decode_fast + decode_reduce (matrix-core decode, then the partition merge)",
                     "bytes_per_launch": per_layer},
    }
    if enc is not None:
        result["encode_mtok_s"] = round(enc["encode_mtok_s"], 2)
        result["encode"] = {k: round(v, 3) for k, v in enc.items()}
    if append is not None:
        result["append_cfg2"] = append
    if cfg3 is not None:
        result["decode_cfg3"] = cfg3
    if k4v is not None:
        result["decode_cfg2_k4_values"] = k4v
    if paged is not None:
        result["paged_cfg4"] = paged
    if nxt is not None:
        result.update(nxt)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(layers[0], device)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
