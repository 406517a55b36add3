"""Versioned byte layout: every packed page owns all of its decoding metadata.

Same fields, order and sizes as the reference (layout.py:8-53): per page of
`block_size` tokens and `heads` KV heads, field-major,
key_payload u8 [H,B,64] | key_scales f32 [H,128] | key_map i16 [H,128] |
key_padding f32 [H,16] | value_payload u8 [H,B,32] | value_scales f16 [H,B,2] |
value_offsets f16 [H,B,2], so `page_bytes = H * (104 B + 832)`.  Block sizes
64/128/256 as in the reference, plus 16 and 32 for small-page pools.  Pages
are encoded by one launch of libinquant_hip.so (iq_encode_pages: K4
min_error, the role map and V2 group 64 written straight into the page).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from inquant import _native as nat

BLOCK_SIZES = (16, 32, 64, 128, 256)


@dataclass(frozen=True)
class PageLayout:
    block_size: int
    heads: int
    dim: int = 128

    def __post_init__(self):
        if self.block_size not in BLOCK_SIZES or self.dim != 128 or self.heads < 1:
            raise ValueError("Expected block_size 16/32/64/128/256, head_dim 128, positive KV heads")

    @property
    def fields(self):
        b, h, d = self.block_size, self.heads, self.dim
        return (
            ("key_payload", torch.uint8, (h, b, d // 2)),
            ("key_scales", torch.float32, (h, d)),
            ("key_map", torch.int16, (h, d)),
            ("key_padding", torch.float32, (h, d // 8)),
            ("value_payload", torch.uint8, (h, b, d // 4)),
            ("value_scales", torch.float16, (h, b, d // 64)),
            ("value_offsets", torch.float16, (h, b, d // 64)),
        )

    @property
    def offsets(self):
        offset, result = 0, {}
        for name, dtype, shape in self.fields:
            result[name] = offset
            offset += math.prod(shape) * dtype.itemsize
        return result

    @property
    def page_bytes(self):
        return self.heads * (104 * self.block_size + 832)

    def views(self, pages):
        if pages.dtype != torch.uint8 or pages.ndim != 2 or pages.shape[1] != self.page_bytes:
            raise ValueError("Expected [pages, page_bytes] uint8 storage")
        out = {}
        for name, dtype, shape in self.fields:
            offset = self.offsets[name]
            size = math.prod(shape) * dtype.itemsize
            out[name] = pages[:, offset:offset + size].view(dtype).view(-1, *shape)
        return out


def _check_pages(keys, values, layout):
    if keys.shape != values.shape or tuple(keys.shape[1:]) != (layout.heads, layout.block_size, 128):
        raise ValueError("Invalid full-page K/V shape")


class _Flags:
    """Two rows of device ints per (device, stream): a page launch raises
    (key non-finite, value non-finite, page id out of range) flags in one row
    and zeroes the other, which the next launch on that stream uses, so no
    separate clearing launch is needed."""

    def __init__(self, device):
        self.words = torch.zeros((2, 4), dtype=torch.int32, device=device)
        self.turn = 0


_FLAGS: dict = {}


def _encode_into(keys, values, layout, pool, page_ids):
    """One launch: K4 min_error (stride 8, 16 salient channels), the i16 role
    map and V2 g64 of every (page, head) written straight into pool[page_ids]."""
    nat.require_gpu(keys, values, pool, page_ids, what="pack_pages_into")
    if keys.dtype not in (torch.bfloat16, torch.float16) or values.dtype != keys.dtype:
        raise ValueError("Pages are encoded from BF16 or FP16 keys and values")
    keys = keys if _rows_ok(keys) else keys.contiguous()
    values = values if _rows_ok(values) else values.contiguous()
    _launch(keys.data_ptr(), values.data_ptr(), keys.dtype, nat.strides4(keys), nat.strides4(values), None,
            keys.shape[0], layout, pool, page_ids)


def _launch(k_ptr, v_ptr, dtype, k_strides, v_strides, page_rows, n, layout, pool, page_ids):
    """One page-encoder launch and its flag read (see _encode_into)."""
    ids = page_ids.contiguous()
    device = pool.device
    stream = nat.stream_handle(device)
    flags = _FLAGS.get((device, stream))
    if flags is None:
        flags = _FLAGS[(device, stream)] = _Flags(device)
    mine, other = flags.words[flags.turn], flags.words[1 - flags.turn]
    nat.check(nat.lib().iq_encode_pages_at(
        k_ptr, v_ptr, nat.dtype_code(dtype), k_strides, v_strides,
        None if page_rows is None else page_rows.data_ptr(), n, layout.heads, layout.block_size,
        pool.data_ptr(), pool.shape[0], ids.data_ptr(), ids.element_size(), mine.data_ptr(), other.data_ptr(),
        stream))
    if n == 0:
        return
    flags.turn = 1 - flags.turn
    bad_key, bad_value, bad_id, _ = mine.tolist()   # the one synchronization, as the codec's finite check
    if bad_id:
        raise ValueError("Physical page ID outside the destination pool")
    if bad_key:
        raise ValueError("x must contain finite values representable in float32")
    if bad_value:
        raise ValueError("Values and stored FP16 quantization parameters must be finite")


def _rows_ok(t) -> bool:
    """Rows the page encoder reads in place: unit channel stride, 16-byte aligned."""
    return (t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1])
            and t.data_ptr() % 16 == 0)


@torch.no_grad()
def pack_pages_at(keys, values, page_rows, layout, destination, page_ids):
    """Seal pages that start at arbitrary token rows, in one launch and one
    flag read (the batched seal of several requests, backend.py:106-116 per
    request in the reference).

    keys / values: [H, tokens, 128] views (any head and token strides that
    are multiples of 8 elements, unit channel stride, 16-byte aligned base)
    over the rows of every page; page n holds tokens page_rows[n] ..
    page_rows[n] + B - 1 (int64 device tensor, rows in range) and goes to
    physical page page_ids[n]."""
    if keys.shape != values.shape or keys.ndim != 3 or keys.shape[0] != layout.heads or keys.shape[2] != 128:
        raise ValueError("Expected key/value rows [kv_heads, tokens, 128]")
    if destination.dtype != torch.uint8 or destination.ndim != 2 or destination.shape[1] != layout.page_bytes \
            or not destination.is_contiguous():
        raise ValueError("Expected contiguous uint8 destination page pool")
    if page_rows.dtype != torch.int64 or page_rows.ndim != 1 or page_ids.ndim != 1 \
            or page_ids.numel() != page_rows.numel() or page_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("One int64 start row and one integer physical page ID are required per page")
    nat.require_gpu(keys, values, destination, page_rows, page_ids, what="pack_pages_at")
    if keys.dtype not in (torch.bfloat16, torch.float16) or values.dtype != keys.dtype:
        raise ValueError("Pages are encoded from BF16 or FP16 keys and values")
    strides = []
    for t in (keys, values):
        st = (0, t.stride(0), t.stride(1), t.stride(2))
        if st[3] != 1 or st[1] % 8 or st[2] % 8 or t.data_ptr() % 16:
            raise ValueError("key/value rows must be contiguous and 16-byte aligned")
        strides.append((nat._i64 * 4)(*st))
    _launch(keys.data_ptr(), values.data_ptr(), keys.dtype, strides[0], strides[1], page_rows.contiguous(),
            page_rows.numel(), layout, destination, page_ids)


@torch.no_grad()
def pack_pages(keys, values, layout):
    """Encode full temporal pages [P, H, B, 128] into fresh [P, page_bytes]
    storage (layout.py:56-81): K4 min_error, the role map and V2 group 64, in
    one launch."""
    _check_pages(keys, values, layout)
    result = torch.empty((keys.shape[0], layout.page_bytes), dtype=torch.uint8, device=keys.device)
    ids = torch.arange(keys.shape[0], dtype=torch.int32, device=keys.device)
    _encode_into(keys, values, layout, result, ids)
    return result


def unpack_pages_reference(pages, layout, dtype=torch.bfloat16):
    """Testing/inspection: dense K and V [P, H, B, 128] of `dtype` (layout.py:84-100)."""
    nat.require_gpu(pages, what="unpack_pages_reference")
    layout.views(pages)                       # shape / dtype validation
    pages = pages.contiguous()
    n = pages.shape[0]
    shape = (n, layout.heads, layout.block_size, 128)
    keys = torch.empty(shape, dtype=dtype, device=pages.device)
    values = torch.empty(shape, dtype=dtype, device=pages.device)
    nat.check(nat.lib().iq_unpack_pages(pages.data_ptr(), n, layout.heads, layout.block_size, keys.data_ptr(),
                                        values.data_ptr(), nat.dtype_code(dtype),
                                        nat.stream_handle(pages.device)))
    return keys, values


@torch.no_grad()
def pack_pages_into(keys, values, layout, destination, page_ids, *, donor_backend="torch"):
    """Seal fresh pages straight into their physical slots (layout.py:103-115)
    with one launch and one flag read; no codec temporaries.

    The page allocator owns unique in-range ids: an id outside the pool
    writes nothing and raises ValueError after the launch, as does a
    non-finite input (the other pages were then written; they belong to the
    caller's fresh allocation).  ``donor_backend`` is accepted for
    compatibility: every backend runs the same selector."""
    _check_pages(keys, values, layout)
    if destination.dtype != torch.uint8 or destination.ndim != 2 or destination.shape[1] != layout.page_bytes \
            or not destination.is_contiguous():
        raise ValueError("Expected contiguous uint8 destination page pool")
    if page_ids.ndim != 1 or page_ids.numel() != keys.shape[0] or page_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("One integer physical page ID is required per input page")
    _encode_into(keys, values, layout, destination, page_ids)
