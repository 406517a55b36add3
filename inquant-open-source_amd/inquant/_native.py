"""ctypes binding of libinquant_hip.so (the gfx950 kernels behind every module).

There is no fallback: if the library is missing or a tensor is not on a ROCm
GPU, the call raises.  Tensors cross the boundary as raw device pointers,
element strides and the current HIP stream handle.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libinquant_hip.so")

IQ_F32, IQ_BF16, IQ_F16, IQ_F64 = 0, 1, 2, 3
_DTYPE_CODE = {torch.float32: IQ_F32, torch.bfloat16: IQ_BF16, torch.float16: IQ_F16, torch.float64: IQ_F64}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_p = ctypes.c_void_p
_f32 = ctypes.c_float


class BlockPtrs(ctypes.Structure):
    """Mirror of iq_block_ptrs in include/inquant_hip.h."""
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "k_payload", "k_scales", "k_padding", "v_payload", "v_scales", "v_offsets",
        "k_src", "k_don", "v_src", "v_don")]


class BlockRun(ctypes.Structure):
    """Mirror of iq_block_run: field addresses of the first block of the
    fixed-stride run of a decode state's leading blocks, and their count."""
    _fields_ = [("base", ctypes.c_uint64 * 8), ("blocks", _i64)]


class TailDesc(ctypes.Structure):
    """Mirror of iq_tail_desc in include/inquant_hip.h: the fixed part of a
    cache layer's tail append (its [2, H, capacity, D] row buffer and the
    position flag word)."""
    _fields_ = [("buf", ctypes.c_uint64), ("buf_kv", _i64), ("buf_h", _i64), ("buf_t", _i64),
                ("heads", _i64), ("dim", _i64), ("capacity", _i64), ("elem_bytes", _int), ("pos_bytes", _int),
                ("flag", ctypes.c_uint64), ("k_sh", _i64), ("k_st", _i64), ("v_sh", _i64), ("v_st", _i64)]


_SIGNATURES = {
    "iq_abi_version": (_int, []),
    "iq_last_error": (ctypes.c_char_p, []),
    "iq_k4_quantize": (_int, [_p, _int, ctypes.POINTER(_i64), _i64, _i64, _i64, _i64, _i64, _i64, _int,
                              _p, _p, _p, _p, _int, _p, _p, _p]),
    "iq_reuse_map": (_int, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "iq_k4_dequantize": (_int, [_p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _i64, _p, _int, _p]),
    "iq_v_quantize": (_int, [_p, _int, ctypes.POINTER(_i64), _i64, _i64, _i64, _i64, _int, _int,
                             _p, _p, _p, _p, _p]),
    "iq_v_dequantize": (_int, [_p, _p, _p, _i64, _i64, _int, _int, _p, _int, _p]),
    "iq_kv_quantize": (_int, [_p, _p, _int, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64, _i64, _i64, _i64,
                              _i64, _i64, _int, _p, _p, _p, _p, _int, _p, _int, _int, _p, _p, _p, _p, _p, _p]),
    "iq_k4_quantize_kv": (_int, [_p, _p, _int, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64, _i64, _i64, _i64,
                                 _i64, _i64, _int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _int, _p, _p, _p]),
    "iq_decode_append": (_int, [_p, _p, _p, _i64, _i64, ctypes.POINTER(BlockPtrs), _i64, _i64, _int, _p]),
    "iq_decode_workspace_floats": (_i64, [_i64, _i64, _i64, _i64]),
    "iq_decode_merge": (_int, [_p, _i64, _i64, _p, _int, _p]),
    "iq_decode_partitions": (_i64, [_i64, _i64, _i64, _int]),
    "iq_decode_attention": (_int, [_p, _int, _i64, _i64, _p, _p, _p, ctypes.POINTER(BlockRun), _i64, _i64, _i64,
                                   _i64, _int, _int,
                                   _p, _p, _i64, _i64, _i64, _i64, _i64,
                                   _p, _p, _i64, _i64, _i64, _i64, _i64,
                                   _f32, _p, _i64, _p, _int, _p]),
    "iq_decode_attention_noalloc": (_int, [_p, _int, _i64, _i64, _p, _p, _p, ctypes.POINTER(BlockRun), _i64, _i64,
                                           _i64, _i64, _int, _int,
                                           _p, _p, _i64, _i64, _i64, _i64, _i64,
                                           _p, _p, _i64, _i64, _i64, _i64, _i64,
                                           _f32, _p, _int, _p]),
    "iq_prefill_attention": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                    _i64, _i64, _f32, _p, _i64, _i64, _int, _p]),
    "iq_page_bytes": (_i64, [_i64, _i64]),
    "iq_encode_pages": (_int, [_p, _p, _int, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64, _i64, _i64, _p, _i64,
                               _p, _int, _p, _p, _p]),
    "iq_encode_pages_at": (_int, [_p, _p, _int, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _p, _i64, _i64, _i64,
                                  _p, _i64, _p, _int, _p, _p, _p]),
    "iq_write_pages": (_int, [_p, _p, _p, _p, _p, _int, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _int, _p]),
    "iq_unpack_pages": (_int, [_p, _i64, _i64, _i64, _p, _p, _int, _p]),
    "iq_paged_workspace_floats": (_i64, [_i64, _i64, _i64, _i64]),
    "iq_paged_decode": (_int, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64,
                               _p, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _f32, _p, _i64, _p, _i64, _int, _p]),
    "iq_tail_append": (_int, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _p, _i64, _i64, _i64,
                              _i64, _i64, _i64, _i64, _p, _int, _i64, _p, _p]),
    "iq_tail_append_row": (_int, [ctypes.POINTER(TailDesc), _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
}

_lib = None
_tail_row = None


def tail_append_row(desc, *args) -> int:
    """iq_tail_append_row(desc, ...); kept as a module-level function bound once."""
    global _tail_row
    if _tail_row is None:
        lib()
        _tail_row = _lib.iq_tail_append_row
    return _tail_row(ctypes.byref(desc), *args)


class NativeError(RuntimeError):
    """A HIP kernel launch or argument check failed inside libinquant_hip.so."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libinquant_hip.so is not built ({LIB_PATH}); run `make -C inquant-open-source_amd` "
                "or __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int) -> None:
    if status != 0:
        raise NativeError(lib().iq_last_error().decode(errors="replace"))


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def require_gpu(*tensors: torch.Tensor, what: str = "InQuant HIP kernels") -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{what} require ROCm GPU tensors; got a {t.device.type} tensor")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must share one GPU")
    return device


def stream_handle(device: torch.device) -> int:
    """The current stream's raw handle (torch.cuda.current_stream(device).cuda_stream,
    without building a Stream object: ~0.3 against ~2 us per call)."""
    index = device.index
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device() if index is None else index)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def strides4(t: torch.Tensor):
    return (_i64 * 4)(*t.stride())
