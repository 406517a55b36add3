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
        int(sink_tokens), dense.data_ptr(), 0, None, None, 0, float(scale), scratch.data_ptr(), need,
        output.data_ptr(), 0, nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
    return output


def work_list(pages, block_size):
    """The compacted work list of a batch whose page counts the host knows:
    every (sequence, partition) the decode needs, as int32 sequence << 16 |
    partition: a sequence's packed partitions (256 tokens of pages each),
    then its dense ones (sink and open page); the sequences with the most
    partitions first, each sequence's partitions consecutive (as the grid
    without a list orders them)."""
    per_part = 256 // block_size
    dense = -(-(block_size + 4) // 256)
    parts = [(-(-int(n) // per_part)) + dense for n in pages]
    order = sorted(range(len(parts)), key=lambda i: -parts[i])
    return [(i << 16) | p for i in order for p in range(parts[i])]


def paged_decode_batch(query, cache, block_tables, seq_info, dense, max_pages, layout, workspace, scale,
                       output=None, dense_slots=None, work=None):
    """query bf16 [n, Hq, 128]; block_tables int32 [n, >= max_pages]; seq_info int32
    [n, 3] device tensor of (pages, tail tokens, sink tokens); dense bf16
    [n, 2, kv_heads, block_size + 4, 128], or [slots, 2, kv_heads, block_size + 4,
    128] with dense_slots an int32 [n] device tensor naming each sequence's
    slot (the caller keeps them in range).  ``work``: optional int32 device
    tensor from ``work_list`` (the partitions that exist, so no workgroup
    starts past a short sequence's end).  Returns [n, Hq, 128]."""
    hkv, b = layout.heads, layout.block_size
    hq = _check_query(query, hkv)
    _check_pool(cache, layout)
    n = query.shape[0]
    rows = n if dense_slots is None else dense.shape[0]
    if tuple(dense.shape) != (rows, 2, hkv, b + 4, 128) or dense.dtype != torch.bfloat16:
        raise ValueError("Expected dense BF16 [sequences, 2, kv_heads, block_size + 4, 128]")
    if dense_slots is not None and (tuple(dense_slots.shape) != (n,) or dense_slots.dtype != torch.int32):
        raise ValueError("Expected int32 dense slots [sequences]")
    if work is not None and (work.ndim != 1 or work.dtype != torch.int32 or not work.is_contiguous()
                             or work.numel() < n):
        raise ValueError("Expected a contiguous int32 work list with every partition of every sequence")
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
        dense.data_ptr(), dense[0].numel(), None if dense_slots is None else dense_slots.contiguous().data_ptr(),
        None if work is None else work.data_ptr(), 0 if work is None else work.numel(),
        float(scale), scratch.data_ptr(), need,
        output.data_ptr(), hq * 128, nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
    return output


def prefill_attention(query, key, value, cu_seqlens, max_seqlen, scale, output=None, *, check_lengths=False):
    """Causal self-attention of a prefill over its exact K/V (replaces the
    plugin's flash_attn_varlen_func(..., causal=True) call, backend.py:139-144).

    query [tokens, Hq, 128], key/value [tokens, H, 128] (bf16 or f16, rows
    16-byte aligned), cu_seqlens int32 [sequences + 1] on the device,
    max_seqlen >= every sequence length.  Returns (or fills) output
    [tokens, Hq, 128] of the query dtype or float32.

    Contract (as flash_attn_varlen_func's max_seqlen_q): the launch covers
    max_seqlen query rows per sequence, so the query rows of a sequence
    longer than max_seqlen past that count are not written.  cu_seqlens lives
    on the device and is not read back; with ``check_lengths=True`` the
    lengths are read (one synchronization) and a longer sequence raises."""
    if query.ndim != 3 or key.ndim != 3 or key.shape != value.shape or query.shape[-1] != 128 \
            or key.shape[-1] != 128 or query.shape[0] != key.shape[0]:
        raise ValueError("Expected query [tokens, Hq, 128] and key/value [tokens, H, 128]")
    if query.dtype not in (torch.bfloat16, torch.float16) or key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("Prefill attention expects BF16 or FP16 query, key and value")
    hq, h = query.shape[1], key.shape[1]
    if hq % h:
        raise ValueError("query heads must be a multiple of KV heads")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be an int32 [sequences + 1] tensor")
    nat.require_gpu(query, key, value, cu_seqlens, what="prefill_attention")
    if check_lengths and int((cu_seqlens[1:] - cu_seqlens[:-1]).max()) > int(max_seqlen):
        raise ValueError("a sequence is longer than max_seqlen")
    if any(t.stride(-1) != 1 for t in (query, key, value)):
        raise ValueError("head dimension must be contiguous")
    if output is None:
        output = torch.empty_like(query)
    elif tuple(output.shape) != tuple(query.shape) or output.stride(-1) != 1 \
            or output.dtype not in (query.dtype, torch.float32):
        raise ValueError("output must be [tokens, Hq, 128] of the query dtype or float32")
    cu = cu_seqlens.contiguous()
    nat.check(nat.lib().iq_prefill_attention(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), nat.dtype_code(query.dtype),
        query.stride(0), query.stride(1), key.stride(0), key.stride(1), value.stride(0), value.stride(1),
        cu.data_ptr(), cu.numel() - 1, int(max_seqlen), hq, h, 128, float(scale), output.data_ptr(),
        output.stride(0), output.stride(1), nat.dtype_code(output.dtype), nat.stream_handle(query.device)))
    return output
