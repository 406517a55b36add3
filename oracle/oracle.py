"""ctypes binding of the CPU restatement in iq_oracle.c.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU port,
never as part of the product path.  Inputs and outputs are numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libiq_oracle.so")
_lib = None

c_i64 = ctypes.c_int64
c_p = ctypes.c_void_p


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.iqo_f32_to_bf16.restype = ctypes.c_uint16
        _lib.iqo_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.iqo_f32_to_f16.restype = ctypes.c_uint16
        _lib.iqo_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.iqo_k4_quantize.restype = ctypes.c_int
        _lib.iqo_k4_quantize.argtypes = [c_p, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int,
                                         c_p, c_p, c_p, c_p, c_p]
        _lib.iqo_k4_stats.argtypes = [c_p, c_i64, c_i64, c_i64, ctypes.c_int, c_p, c_p, c_p, c_p]
        _lib.iqo_reuse_map.argtypes = [c_p, c_p, c_i64, c_i64, c_i64, c_p, c_p]
        _lib.iqo_k4_dequantize.argtypes = [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64,
                                           ctypes.c_int, c_p]
        _lib.iqo_v_quantize.restype = ctypes.c_int
        _lib.iqo_v_quantize.argtypes = [c_p, c_i64, c_i64, ctypes.c_int, ctypes.c_int, c_p, c_p, c_p]
        _lib.iqo_v_dequantize.argtypes = [c_p, c_p, c_p, c_i64, c_i64, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, c_p]
        _lib.iqo_role_map.argtypes = [c_p, c_p, c_i64, c_i64, c_i64, c_p]
        _lib.iqo_check_recip_division.argtypes = [c_i64, c_i64, ctypes.c_uint64]
        _lib.iqo_check_recip_division.restype = c_i64
        _lib.iqo_attend.argtypes = [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, ctypes.c_double, c_p]
        _lib.iqo_set_threads.argtypes = [ctypes.c_int]
    return _lib


def set_threads(n: int) -> None:
    """Thread count of the oracle's OpenMP loops."""
    lib().iqo_set_threads(int(n))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(c_p)


DTYPE_CODE = {"float32": 0, "bfloat16": 1, "float16": 2}


def k4_stats(x: np.ndarray, stride: int, min_error: bool):
    """x fp32 [T, D] -> (saliency, sampled_mean, err or None, amax)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, D = x.shape
    out = [np.empty(D, np.float32) for _ in range(4)]
    lib().iqo_k4_stats(_ptr(x), T, D, stride, int(min_error), *[_ptr(o) for o in out])
    return out[0], out[1], (out[2] if min_error else None), out[3]


def reuse_map(saliency: np.ndarray, count: int, donor_error: np.ndarray | None = None):
    """saliency fp32 [..., D] -> (sources, donors) int64 [..., count] (codec.py:137-178)."""
    sal = np.ascontiguousarray(saliency, dtype=np.float32)
    D = sal.shape[-1]
    rows = sal.size // D if D else 0
    err = None if donor_error is None else np.ascontiguousarray(donor_error, dtype=np.float32)
    src = np.zeros((*sal.shape[:-1], count), np.int64)
    don = np.zeros_like(src)
    if count and rows:
        lib().iqo_reuse_map(_ptr(sal), None if err is None else _ptr(err), rows, D, count,
                            _ptr(src), _ptr(don))
    return src, don


def k4_quantize(x: np.ndarray, sample_stride: int = 8, salient_fraction: float = 0.125,
                donor_policy: str = "neighbors"):
    """x fp32 [B, H, T, D] -> dict of payload/scales/src/don/padding (codec.py:181-243)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, H, T, D = x.shape
    count = int(np.floor(D * salient_fraction))
    rows = B * H
    payload = np.empty((B, H, T, D // 2), np.uint8)
    scales = np.empty((B, H, D), np.float32)
    src = np.empty((B, H, count), np.int64)
    don = np.empty((B, H, count), np.int64)
    padding = np.empty((B, H, count), np.float32)
    rc = lib().iqo_k4_quantize(_ptr(x), rows, T, D, count, sample_stride, int(donor_policy == "min_error"),
                               _ptr(payload), _ptr(scales), _ptr(src), _ptr(don), _ptr(padding))
    if rc:
        raise ValueError("x must contain finite values representable in float32")
    return {"payload": payload, "scales": scales, "salient_channels": src, "donor_channels": don,
            "padding": padding}


def k4_dequantize(packed: dict, dtype: str = "float32") -> np.ndarray:
    payload = np.ascontiguousarray(packed["payload"], np.uint8)
    B, H, T, half = payload.shape
    D = half * 2
    src = np.ascontiguousarray(packed["salient_channels"], np.int64)
    count = src.shape[-1]
    out = np.empty((B, H, T, D), np.float32)
    lib().iqo_k4_dequantize(_ptr(payload), _ptr(np.ascontiguousarray(packed["scales"], np.float32)),
                            _ptr(src), _ptr(np.ascontiguousarray(packed["donor_channels"], np.int64)),
                            _ptr(np.ascontiguousarray(packed["padding"], np.float32)),
                            B * H, T, D, count, DTYPE_CODE[dtype], _ptr(out))
    return out


def v_quantize(x: np.ndarray, bits: int = 2, group_size: int = 64):
    """x fp32 [..., D] -> payload u8, scales/offsets as float16 arrays (value_codec.py:51-72)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    payload = np.empty((*x.shape[:-1], D * bits // 8), np.uint8)
    scales = np.empty((*x.shape[:-1], D // group_size), np.uint16)
    offsets = np.empty_like(scales)
    rc = lib().iqo_v_quantize(_ptr(x), rows, D, bits, group_size, _ptr(payload), _ptr(scales), _ptr(offsets))
    if rc:
        raise ValueError("Values and stored FP16 quantization parameters must be finite")
    return {"payload": payload, "scales": scales.view(np.float16), "offsets": offsets.view(np.float16)}


def v_dequantize(packed: dict, bits: int, group_size: int, dtype: str = "float32") -> np.ndarray:
    payload = np.ascontiguousarray(packed["payload"], np.uint8)
    D = payload.shape[-1] * 8 // bits
    rows = payload.size // payload.shape[-1]
    out = np.empty((*payload.shape[:-1], D), np.float32)
    lib().iqo_v_dequantize(_ptr(payload), _ptr(np.ascontiguousarray(packed["scales"]).view(np.uint16)),
                           _ptr(np.ascontiguousarray(packed["offsets"]).view(np.uint16)),
                           rows, D, bits, group_size, DTYPE_CODE[dtype], _ptr(out))
    return out


def role_map(src: np.ndarray, don: np.ndarray, D: int = 128) -> np.ndarray:
    """src/don int64 [heads, count] -> int16 [heads, D] roles (triton_attention.py:301-309)."""
    src = np.ascontiguousarray(src, np.int64)
    don = np.ascontiguousarray(don, np.int64)
    heads, count = src.shape
    out = np.empty((heads, D), np.int16)
    lib().iqo_role_map(_ptr(src), _ptr(don), heads, D, count, _ptr(out))
    return out


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """fp64 attention: q [Hq, D], k/v [H, T, D] -> [Hq, D] float64 (qwen_fused.py:21-30)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    Hq, D = q.shape
    H, T, _ = k.shape
    out = np.empty((Hq, D), np.float64)
    lib().iqo_attend(_ptr(q), _ptr(k), _ptr(v), Hq, H, T, D, float(scale), _ptr(out))
    return out


def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (RNE) and return them as fp32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, (u | 0x400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32)


def to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def check_recip_division(n_max: int = 256, samples: int = 20000, seed: int = 1) -> int:
    """Mismatches of the GPU tile encoder's reciprocal-and-remainder quotient
    against IEEE division (test support, see iqo_check_recip_division)."""
    return int(lib().iqo_check_recip_division(n_max, samples, seed))


# ---------------------------------------------------------------- paged cache (vLLM page layout)

def page_fields(H: int, B: int):
    """Field order, dtypes and shapes of one page (layout.py:18-31)."""
    return (("key_payload", np.uint8, (H, B, 64)), ("key_scales", np.float32, (H, 128)),
            ("key_map", np.int16, (H, 128)), ("key_padding", np.float32, (H, 16)),
            ("value_payload", np.uint8, (H, B, 32)), ("value_scales", np.float16, (H, B, 2)),
            ("value_offsets", np.float16, (H, B, 2)))


def page_offsets(H: int, B: int):
    """Byte offset of every field and the page size (layout.py:33-45)."""
    off, result = 0, {}
    for name, dtype, shape in page_fields(H, B):
        result[name] = off
        off += int(np.prod(shape)) * np.dtype(dtype).itemsize
    return result, off


def page_views(pages: np.ndarray, H: int, B: int):
    offsets, size = page_offsets(H, B)
    assert pages.dtype == np.uint8 and pages.ndim == 2 and pages.shape[1] == size
    out = {}
    for name, dtype, shape in page_fields(H, B):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        out[name] = pages[:, offsets[name]:offsets[name] + n].view(dtype).reshape(-1, *shape)
    return out


def pack_pages(kq: dict, vq: dict, H: int, B: int) -> np.ndarray:
    """Codec outputs of [P, H, B, 128] pages -> [P, page_bytes] (layout.py:56-81):
    fields copied, role map -1 / donor channel for a source / -2 - j for donor j."""
    P = kq["payload"].shape[0]
    _, size = page_offsets(H, B)
    pages = np.zeros((P, size), np.uint8)
    f = page_views(pages, H, B)
    f["key_payload"][...] = kq["payload"]
    f["key_scales"][...] = kq["scales"]
    f["key_padding"][...] = kq["padding"]
    src = np.asarray(kq["salient_channels"], np.int64).reshape(P * H, -1)
    don = np.asarray(kq["donor_channels"], np.int64).reshape(P * H, -1)
    f["key_map"][...] = role_map(src, don).reshape(P, H, 128)
    f["value_payload"][...] = vq["payload"]
    f["value_scales"][...] = np.asarray(vq["scales"], np.float16)
    f["value_offsets"][...] = np.asarray(vq["offsets"], np.float16)
    return pages


def unpack_pages(pages: np.ndarray, H: int, B: int, dtype: str = "bfloat16"):
    """[P, page_bytes] -> K, V float32 [P, H, B, 128] rounded to dtype (layout.py:84-100)."""
    f = page_views(np.ascontiguousarray(pages), H, B)
    role = f["key_map"].astype(np.int64)                                    # [P, H, 128]
    kp = f["key_payload"]
    slots = np.stack((kp & 15, kp >> 4), -1).reshape(*kp.shape[:-1], 128).astype(np.int64)
    partner = np.take_along_axis(slots, np.broadcast_to(np.maximum(role, 0)[:, :, None, :], slots.shape), -1)
    code = np.where(role[:, :, None, :] >= 0, (slots << 4 | partner) - 128, slots - 8)
    keys = code.astype(np.float32) * f["key_scales"][:, :, None, :]
    pad = np.take_along_axis(f["key_padding"], np.maximum(-role - 2, 0), -1)  # [P, H, 128]
    keys = np.where(role[:, :, None, :] <= -2, pad[:, :, None, :], keys).astype(np.float32)
    vp = f["value_payload"]
    codes = np.stack([(vp >> i) & 3 for i in (0, 2, 4, 6)], -1).reshape(*vp.shape[:-1], 128)
    vals = codes.astype(np.float32).reshape(*codes.shape[:-1], 2, 64)
    vals = (vals * f["value_scales"].astype(np.float32)[..., None]
            + f["value_offsets"].astype(np.float32)[..., None]).reshape(*codes.shape[:-1], 128)
    rnd = to_bf16 if dtype == "bfloat16" else (to_f16 if dtype == "float16" else (lambda a: a))
    return rnd(keys), rnd(vals.astype(np.float32))


def paged_tokens(pool: np.ndarray, ids, dense: np.ndarray, n_pages: int, tail_t: int, sink_t: int,
                 H: int, B: int):
    """The K/V tokens paged decode attends to, in any order (kernels.py:29-59): packed
    tokens of the block table's pages whose global index is at least the sink
    length, dense slots below the sink length, and dense tail slots 4 .. 4 + tail
    whose global position n_pages * B + slot - 4 is at least the sink length.
    dense: float32 [2, H, B + 4, 128]."""
    ks, vs = [], []
    if n_pages:
        k, v = unpack_pages(pool[np.asarray(ids[:n_pages], np.int64)], H, B)     # [n, H, B, 128]
        k = k.transpose(1, 0, 2, 3).reshape(H, n_pages * B, 128)
        v = v.transpose(1, 0, 2, 3).reshape(H, n_pages * B, 128)
        live = np.arange(n_pages * B) >= sink_t
        ks.append(k[:, live])
        vs.append(v[:, live])
    slots = np.arange(B + 4)
    live = (slots < sink_t) | ((slots >= 4) & (slots < 4 + tail_t) & (n_pages * B + slots - 4 >= sink_t))
    ks.append(dense[0][:, live])
    vs.append(dense[1][:, live])
    return np.concatenate(ks, 1), np.concatenate(vs, 1)


def paged_attend(q: np.ndarray, pool: np.ndarray, ids, dense: np.ndarray, n_pages: int, tail_t: int,
                 sink_t: int, H: int, B: int, scale: float) -> np.ndarray:
    """fp64 paged decode of one sequence: q [Hq, 128] -> [Hq, 128]."""
    k, v = paged_tokens(pool, ids, dense, n_pages, tail_t, sink_t, H, B)
    return attend(q, k, v, scale)


def causal_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """fp64 causal self-attention of one sequence: q [n, Hq, D], k/v [n, H, D]
    -> [n, Hq, D]; query i sees keys 0..i of its KV head (query head h reads
    KV head h // (Hq / H)).  The semantics of the plugin's prefill call
    flash_attn_varlen_func(..., causal=True) (backend.py:139-144)."""
    q64, k64, v64 = (np.asarray(a, np.float64) for a in (q, k, v))
    n, hq, _ = q64.shape
    group = hq // k64.shape[1]
    out = np.empty_like(q64)
    future = np.triu(np.ones((n, n), bool), 1)
    for h in range(hq):
        s = q64[:, h] @ k64[:, h // group].T * scale
        s[future] = -np.inf
        s -= s.max(1, keepdims=True)
        p = np.exp(s)
        out[:, h] = (p @ v64[:, h // group]) / p.sum(1, keepdims=True)
    return out


def causal_attend_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, rows, heads,
                       chunk: int = 1024) -> np.ndarray:
    """fp64 causal attention of the query rows `rows` (ascending) and query
    heads `heads` of one sequence -> [len(rows), len(heads), D]; the same
    semantics as causal_attend (query i sees keys 0..i of KV head
    h // (Hq / H)), evaluated in row chunks so that long sequences need
    O(chunk * n) memory."""
    rows = np.asarray(rows, np.int64)
    group = q.shape[1] // k.shape[1]
    out = np.empty((rows.size, len(heads), q.shape[2]))
    for j, h in enumerate(heads):
        kh = np.asarray(k[:, h // group], np.float64)
        vh = np.asarray(v[:, h // group], np.float64)
        for a in range(0, rows.size, chunk):
            r = rows[a:a + chunk]
            n = int(r[-1]) + 1
            s = np.asarray(q[r, h], np.float64) @ kh[:n].T * scale
            s[np.arange(n)[None, :] > r[:, None]] = -np.inf
            s -= s.max(1, keepdims=True)
            p = np.exp(s)
            out[a:a + chunk, j] = (p @ vh[:n]) / p.sum(1, keepdims=True)
    return out
