"""Versioned byte layout: every packed page owns all of its decoding metadata.

Same fields, order and sizes as the reference (layout.py:8-53): per page of
`block_size` tokens and `heads` KV heads, field-major,
key_payload u8 [H,B,64] | key_scales f32 [H,128] | key_map i16 [H,128] |
key_padding f32 [H,16] | value_payload u8 [H,B,32] | value_scales f16 [H,B,2] |
value_offsets f16 [H,B,2], so `page_bytes = H * (104 B + 832)`.  Block sizes
64/128/256 as in the reference, plus 16 and 32 for small-page pools.  Encoding
runs in libinquant_hip.so (K4 min_error + V2 group 64, then one page writer).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from inquant import _native as nat
from inquant.codec import CodecConfig, quantize
from inquant.value_codec import quantize_values

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


@torch.no_grad()
def pack_pages(keys, values, layout):
    """Encode full temporal pages [P, H, B, 128] into fresh [P, page_bytes] storage
    (layout.py:56-81): K4 min_error and V2 group 64, written by the page writer."""
    from .packing import write_codec_pages
    _check_pages(keys, values, layout)
    k = quantize(keys, CodecConfig(donor_policy="min_error"))
    v = quantize_values(values, bits=2, group_size=64)
    result = torch.empty((keys.shape[0], layout.page_bytes), dtype=torch.uint8, device=keys.device)
    ids = torch.arange(keys.shape[0], dtype=torch.int32, device=keys.device)
    write_codec_pages(k, v, layout, result, ids)
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
    """Seal fresh pages directly into their physical slots (layout.py:103-115).

    The page allocator owns unique in-range ids; no staging page pool is
    created (codec temporaries are separately owned)."""
    from .packing import write_codec_pages
    _check_pages(keys, values, layout)
    k = quantize(keys, CodecConfig(donor_policy="min_error", donor_backend=donor_backend))
    v = quantize_values(values, bits=2, group_size=64)
    write_codec_pages(k, v, layout, destination, page_ids)
