"""Write codec outputs directly to physical pages (packing.py:7-55 of the reference).

One HIP launch copies every field of every (page, head) with 16-byte stores
and builds the i16 role map from the descriptors; ids outside the pool are
skipped by the kernel.
"""
from __future__ import annotations

import torch

from inquant import _native as nat


def write_codec_pages(keys, values, layout, pool, page_ids):
    """Caller owns allocation and supplies unique, in-range GPU page ids."""
    if pool.dtype != torch.uint8 or pool.ndim != 2 or pool.shape[1] != layout.page_bytes or not pool.is_contiguous():
        raise ValueError('Expected contiguous uint8 destination page pool')
    if page_ids.ndim != 1 or page_ids.numel() != keys.shape[0] or page_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError('One integer physical page ID is required per input page')
    if page_ids.device != pool.device or keys.payload.device != pool.device or values.payload.device != pool.device:
        raise ValueError('Codec tensors, page IDs and pool must share a CUDA device')
    n, h, b = keys.shape[0], layout.heads, layout.block_size
    if tuple(keys.shape) != (n, h, b, 128) or tuple(values.shape) != (n, h, b, 128):
        raise ValueError("Codec tensors do not match the page layout")
    if keys.salient_channels.shape[-1] != 16 or values.bits != 2 or values.group_size != 64:
        raise ValueError("Pages hold K4 with 16 salient channels and V2 with group 64")
    nat.require_gpu(pool, what="write_codec_pages")
    ids = page_ids.contiguous()
    t = [x.contiguous() for x in (keys.payload, keys.scales, keys.padding, keys.salient_channels,
                                  keys.donor_channels, values.payload, values.scales, values.offsets)]
    nat.check(nat.lib().iq_write_pages(
        t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(), t[4].data_ptr(), t[3].element_size(),
        t[5].data_ptr(), t[6].data_ptr(), t[7].data_ptr(), n, h, b, pool.data_ptr(), pool.shape[0],
        ids.data_ptr(), ids.element_size(), nat.stream_handle(pool.device)))
