"""Fused paged K4/V2 decode (kernels.py:8-88 of the reference): no dense history,
no host page lookup.

`paged_decode` keeps the reference's signature (one sequence per call);
`paged_decode_batch` decodes several sequences, each with its own block
table row, lengths and dense sink/tail buffer, in one launch.
"""
from __future__ import annotations

import torch

from inquant import _native as nat


def _check_query(query, hkv):
    if query.shape[-1] != 128 or query.dtype != torch.bfloat16:
        raise ValueError("Paged decode expects one BF16 query [1, heads, 128]")
    hq = query.shape[1]
    if hq % hkv or hq // hkv > 16:
        raise ValueError("Expected 1..16 query heads per KV head")
    return hq


def _check_pool(cache, layout):
    if cache.dtype != torch.uint8 or cache.ndim != 2 or cache.shape[1] != layout.page_bytes or not cache.is_contiguous():
        raise ValueError("Expected contiguous uint8 [pages, page_bytes] cache")


def paged_decode(query, cache, blocks, dense, num_pages, tail_tokens,
                 sink_tokens, layout, workspace, scale, output=None):
    if query.shape[0] != 1:
        raise ValueError("Paged decode expects one BF16 query [1, heads, 128]")
    hkv, b = layout.heads, layout.block_size
    hq = _check_query(query, hkv)
    _check_pool(cache, layout)
    if tuple(dense.shape) != (2, hkv, b + 4, 128) or dense.dtype != torch.bfloat16:
        raise ValueError("Expected dense BF16 [2, kv_heads, block_size + 4, 128]")
    if not 0 <= int(num_pages) <= blocks.numel() or not 0 <= int(tail_tokens) <= b or not 0 <= int(sink_tokens) <= 4:
        raise ValueError("Page, tail or sink count out of range")
    nat.require_gpu(query, cache, blocks, dense, what="paged_decode")
    query = query.contiguous()
    dense = dense.contiguous()
    table = blocks.reshape(-1)
    table = (table if table.dtype == torch.int32 else table.to(torch.int32)).contiguous()
    need = nat.lib().iq_paged_workspace_floats(hq, 1, int(num_pages), b)
    scratch = workspace.acquire((need,), query.device)
    if output is None:
        output = torch.empty_like(query)
    nat.check(nat.lib().iq_paged_decode(
        query.data_ptr(), 0, 128, hq, 1, cache.data_ptr(), cache.shape[0], hkv, b,
        table.data_ptr() if table.numel() else None, 0, int(num_pages), None, int(num_pages), int(tail_tokens),
        int(sink_tokens), dense.data_ptr(), 0, float(scale), scratch.data_ptr(), need,
        output.data_ptr(), 0, nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
    return output


def paged_decode_batch(query, cache, block_tables, seq_info, dense, max_pages, layout, workspace, scale,
                       output=None):
    """query bf16 [n, Hq, 128]; block_tables int32 [n, >= max_pages]; seq_info int32
    [n, 3] device tensor of (pages, tail tokens, sink tokens); dense bf16
    [n, 2, kv_heads, block_size + 4, 128].  Returns [n, Hq, 128]."""
    hkv, b = layout.heads, layout.block_size
    hq = _check_query(query, hkv)
    _check_pool(cache, layout)
    n = query.shape[0]
    if tuple(dense.shape) != (n, 2, hkv, b + 4, 128) or dense.dtype != torch.bfloat16:
        raise ValueError("Expected dense BF16 [sequences, 2, kv_heads, block_size + 4, 128]")
    if block_tables.ndim != 2 or block_tables.shape[0] != n or block_tables.shape[1] < max_pages \
            or block_tables.dtype != torch.int32:
        raise ValueError("Expected int32 block tables [sequences, >= max_pages]")
    if tuple(seq_info.shape) != (n, 3) or seq_info.dtype != torch.int32:
        raise ValueError("Expected int32 sequence lengths [sequences, 3]")
    nat.require_gpu(query, cache, block_tables, seq_info, dense, what="paged_decode_batch")
    query, dense = query.contiguous(), dense.contiguous()
    block_tables, seq_info = block_tables.contiguous(), seq_info.contiguous()
    need = nat.lib().iq_paged_workspace_floats(hq, n, int(max_pages), b)
    scratch = workspace.acquire((need,), query.device)
    if output is None:
        output = torch.empty_like(query)
    nat.check(nat.lib().iq_paged_decode(
        query.data_ptr(), hq * 128, 128, hq, n, cache.data_ptr(), cache.shape[0], hkv, b,
        block_tables.data_ptr(), block_tables.shape[1], int(max_pages), seq_info.data_ptr(), 0, 0, 0,
        dense.data_ptr(), dense[0].numel(), float(scale), scratch.data_ptr(), need,
        output.data_ptr(), hq * 128, nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
    return output
