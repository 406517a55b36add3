"""Paged InQuant cache in the vLLM plugin's page layout, on MI355X.

Mirrors the reference's extensions/vllm/src/inquant_vllm modules that carry
the packed-KV hot path: `layout` (PageLayout, pack_pages,
unpack_pages_reference, pack_pages_into), `packing` (write_codec_pages) and
`kernels` (paged_decode, plus paged_decode_batch for several sequences in
one launch, and prefill_attention for the prefill's causal attention) and
`backend` (the attention backend's page lifecycle: prefill, dense tail,
paged decode, seal after attention).  The vLLM platform and worker glue
(platform.py, worker.py) need vLLM itself and are not part of this package.
"""
from .layout import PageLayout, pack_pages, pack_pages_into, unpack_pages_reference
from .packing import write_codec_pages
from .kernels import paged_decode, paged_decode_batch, prefill_attention, work_list

__all__ = ["PageLayout", "pack_pages", "pack_pages_into", "unpack_pages_reference", "write_codec_pages",
           "paged_decode", "paged_decode_batch", "prefill_attention", "work_list"]
