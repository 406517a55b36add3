"""Page lifecycle of the InQuant vLLM attention backend, without vLLM (MI355X).

Restates extensions/vllm/src/inquant_vllm/backend.py:18-177 of the
reference for one active request per layer:

* prefill (context length 0): the first four tokens go to the dense sink
  slots, every query attends causally over the exact K/V
  (``prefill_attention``, the reference's flash_attn_varlen_func call),
  full pages are sealed into the physical pages of the block table with the
  one-launch page encoder, and the partial page stays dense;
* decode (one token): the token is written to its dense tail slot (and to
  its sink slot while fewer than four tokens exist), the paged decode
  attends over sealed pages + sink + tail, and a page that this token fills
  is sealed *after* attention, so the query that fills it sees exact values;
* a request whose id or length does not match the layer's state is refused
  ("state mismatch") instead of reusing a stale tail.

The classes keep the reference's names and call signatures so a vLLM
plugin can bind them: ``InQuantMetadata``, ``InQuantMetadataBuilder``,
``InQuantBackend`` (static backend description) and ``InQuantImpl``
(``forward(layer, query, key, value, kv_cache, attn_metadata, output)``).
Where the reference reads vLLM's current config, ``get_current_vllm_config``
returns vLLM's when vLLM is importable and otherwise the config set with
``configure(block_size=..., max_model_len=...)``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from inquant.triton_attention import SharedDecodeWorkspace
from .kernels import paged_decode, prefill_attention
from .layout import PageLayout, pack_pages_into

# Layers run in stream order and share one workspace (it checks stream identity).
WORKSPACE = SharedDecodeWorkspace()
_CONFIG = None
SINK = 4


def configure(*, block_size: int, max_model_len: int) -> None:
    """Page size and maximum request length used when vLLM is not present."""
    global _CONFIG
    _CONFIG = SimpleNamespace(cache_config=SimpleNamespace(block_size=block_size),
                              model_config=SimpleNamespace(max_model_len=max_model_len))


def get_current_vllm_config():
    try:
        from vllm.config import get_current_vllm_config as current
    except ImportError:
        if _CONFIG is None:
            raise RuntimeError("InQuant paged backend: call inquant_vllm.backend.configure() (vLLM is absent)")
        return _CONFIG
    return current()


@dataclass
class InQuantMetadata:
    num_actual_tokens: int
    seq_len: int
    context_len: int
    query_start_loc: torch.Tensor
    block_table: torch.Tensor
    request_id: str


class InQuantMetadataBuilder:
    """Per-step metadata of the single active request (backend.py:28-50)."""

    def __init__(self, runner, kv_cache_spec, block_table):
        self.runner, self.block_table = runner, block_table

    def reorder_batch(self, input_batch, scheduler_output):
        return False

    def use_cascade_attention(self, *args, **kwargs):
        return False

    def build(self, num_reqs, num_actual_tokens, max_query_len, common_prefix_len, common_attn_metadata):
        if num_reqs != 1 or common_prefix_len:
            raise RuntimeError("InQuant requires one active request and no shared prefix")
        seq_len = int(self.runner.seq_lens_np[0])
        context_len = seq_len - num_actual_tokens
        if context_len and num_actual_tokens != 1:
            raise RuntimeError("Chunked prefill/speculative multi-token decode is unsupported")
        return InQuantMetadata(num_actual_tokens, seq_len, context_len, common_attn_metadata.query_start_loc,
                               self.block_table.get_device_tensor()[0], self.runner.input_batch.req_ids[0])


class InQuantBackend:
    """Backend description: name, head size, classes and the packed page pool shape."""

    @staticmethod
    def get_name():
        return "INQUANT_PAGED_K4V2_V1"

    @staticmethod
    def get_supported_head_sizes():
        return [128]

    @staticmethod
    def get_impl_cls():
        return InQuantImpl

    @staticmethod
    def get_metadata_cls():
        return InQuantMetadata

    @staticmethod
    def get_builder_cls():
        return InQuantMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size):
        return (num_blocks, PageLayout(block_size, num_kv_heads, head_size).page_bytes)

    @staticmethod
    def get_kv_cache_stride_order():
        return (0, 1)


class _Request:
    """Dense rows and progress of the layer's active request."""

    __slots__ = ("request_id", "tokens", "sealed_pages")

    def __init__(self, request_id, tokens, sealed_pages):
        self.request_id, self.tokens, self.sealed_pages = request_id, tokens, sealed_pages


class InQuantImpl:
    """One attention layer over a packed page pool (backend.py:75-177)."""

    def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes=None, sliding_window=None,
                 kv_cache_dtype="auto", blocksparse_params=None, logits_soft_cap=None, attn_type=None,
                 kv_sharing_target_layer_name=None, use_irope=False, **_):
        if alibi_slopes is not None or sliding_window not in (None, (-1, -1)) or logits_soft_cap:
            raise ValueError("InQuant supports full causal attention without ALiBi/softcap")
        if kv_sharing_target_layer_name is not None or use_irope:
            raise ValueError("KV sharing and iRoPE are not implemented")
        if num_heads % num_kv_heads:
            raise ValueError("query heads must be a multiple of KV heads")
        if num_heads // num_kv_heads > 16:
            raise ValueError("At most 16 query heads per KV head")
        self.num_heads, self.head_size, self.scale = num_heads, head_size, float(scale)
        self.num_kv_heads = num_kv_heads
        self.num_queries_per_kv = num_heads // num_kv_heads
        config = get_current_vllm_config()
        self.layout = PageLayout(config.cache_config.block_size, num_kv_heads, head_size)
        self.max_pages = math.ceil(config.model_config.max_model_len / self.layout.block_size)
        self.dense = None           # [2, H, block + 4, 128]: slots 0..3 sink, 4.. the open page
        self.request: _Request | None = None
        self.max_tokens_seen = 0
        self.prefill_calls = self.decode_calls = self.seal_calls = 0

    # the reference's attribute names
    @property
    def request_id(self):
        return None if self.request is None else self.request.request_id

    @property
    def tokens(self):
        return 0 if self.request is None else self.request.tokens

    @property
    def sealed_pages(self):
        return 0 if self.request is None else self.request.sealed_pages

    def _buffers(self, query):
        if self.dense is None:
            self.dense = torch.empty((2, self.num_kv_heads, self.layout.block_size + SINK, 128),
                                     dtype=query.dtype, device=query.device)
            WORKSPACE.acquire((self.num_heads, self.max_pages + 1, 130), query.device)

    def _seal(self, keys, values, cache, block_table, first_page):
        """Encode full pages [n, H, B, 128] into the block table's physical pages."""
        pack_pages_into(keys, values, self.layout, cache, block_table[first_page:first_page + keys.shape[0]])
        self.seal_calls += 1

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None):
        if output is None:
            raise ValueError("vLLM must supply an output buffer")
        self._buffers(query)
        if attn_metadata is None:
            return output               # memory profiling: no request state is touched
        if kv_cache.dtype != torch.uint8 or kv_cache.ndim != 2 or kv_cache.shape[1] != self.layout.page_bytes:
            raise RuntimeError("InQuant cache spec was not installed; refusing dense fallback")
        m = attn_metadata
        if m.context_len == 0:
            self._prefill(query, key, value, kv_cache, m, output)
        else:
            self._decode(query, key, value, kv_cache, m, output)
        self.max_tokens_seen = max(self.max_tokens_seen, self.tokens)
        return output

    def _prefill(self, query, key, value, kv_cache, m, output):
        n, b = m.num_actual_tokens, self.layout.block_size
        full = n // b
        sink = min(SINK, n)
        # [tokens, H, 128] -> the dense buffer's [H, slot, 128]
        self.dense[0, :, :sink].copy_(key[:sink].transpose(0, 1))
        self.dense[1, :, :sink].copy_(value[:sink].transpose(0, 1))
        cu = m.query_start_loc[:2].to(torch.int32)
        prefill_attention(query[:n], key[:n], value[:n], cu, n, self.scale, output[:n])
        if full:
            pages = lambda t: t[:full * b].view(full, b, self.num_kv_heads, 128).transpose(1, 2)
            self._seal(pages(key), pages(value), kv_cache, m.block_table, 0)
        rest = n - full * b
        if rest:
            self.dense[0, :, SINK:SINK + rest].copy_(key[n - rest:n].transpose(0, 1))
            self.dense[1, :, SINK:SINK + rest].copy_(value[n - rest:n].transpose(0, 1))
        self.request = _Request(m.request_id, n, full)
        self.prefill_calls += 1

    def _decode(self, query, key, value, kv_cache, m, output):
        req = self.request
        if req is None or m.request_id != req.request_id or m.context_len != req.tokens \
                or m.num_actual_tokens != 1:
            raise RuntimeError("InQuant request state mismatch; refusing stale tail reuse")
        b = self.layout.block_size
        slot = req.tokens % b                      # this token's place in the open page
        self.dense[0, :, SINK + slot].copy_(key[0])
        self.dense[1, :, SINK + slot].copy_(value[0])
        if req.tokens < SINK:
            self.dense[0, :, req.tokens].copy_(key[0])
            self.dense[1, :, req.tokens].copy_(value[0])
        req.tokens += 1
        paged_decode(query[:1], kv_cache, m.block_table, self.dense, req.sealed_pages, slot + 1,
                     min(SINK, req.tokens), self.layout, WORKSPACE, self.scale, output[:1])
        if slot + 1 == b:
            # sealed after attention: only later queries see this page quantized
            self._seal(self.dense[0:1, :, SINK:], self.dense[1:2, :, SINK:], kv_cache, m.block_table,
                       req.sealed_pages)
            req.sealed_pages += 1
        self.decode_calls += 1
