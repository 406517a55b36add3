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

from inquant import _native as nat
from inquant.triton_attention import SharedDecodeWorkspace
from .kernels import paged_decode, paged_decode_batch, prefill_attention, work_list
from .layout import PageLayout, _launch, pack_pages_into

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


# ---------------------------------------------------------------- many requests
#
# The reference serves one active request (backend.py:39-40 refuses more).
# The classes below keep its page lifecycle per request and run a step of N
# requests with one launch per phase: one varlen prefill over every new
# request, one seal of every full prefill page, one batched paged decode over
# every decoding request, and one seal of every page this step's decode
# tokens filled (after attention, as the reference seals).


@dataclass
class InQuantBatchMetadata:
    """One scheduler step of several requests: batch order ``request_ids``,
    their query rows [query_start_loc_cpu[i], query_start_loc_cpu[i + 1])
    (host list; ``query_start_loc`` is the same on the device), their lengths
    after this step ``seq_lens`` (host list), their block-table rows
    ``block_table`` (int32 device tensor [N, >= pages]) and the requests that
    finished since the previous step (their dense slots are released first)."""
    request_ids: list
    query_start_loc: torch.Tensor
    query_start_loc_cpu: list
    seq_lens: list
    block_table: torch.Tensor
    finished_req_ids: tuple = ()

    @property
    def num_actual_tokens(self):
        return int(self.query_start_loc_cpu[-1])


class InQuantBatchMetadataBuilder(InQuantMetadataBuilder):
    """Per-step metadata of every scheduled request.  ``reorder_batch``
    receives the scheduler's output each step; its finished request ids are
    handed to the next metadata."""

    def __init__(self, runner, kv_cache_spec, block_table):
        super().__init__(runner, kv_cache_spec, block_table)
        self._finished = ()

    def reorder_batch(self, input_batch, scheduler_output):
        self._finished = tuple(getattr(scheduler_output, "finished_req_ids", ()) or ())
        return False

    def build(self, num_reqs, num_actual_tokens, max_query_len, common_prefix_len, common_attn_metadata):
        if common_prefix_len:
            raise RuntimeError("InQuant requires no shared prefix")
        qsl = common_attn_metadata.query_start_loc
        finished, self._finished = self._finished, ()
        return InQuantBatchMetadata(list(self.runner.input_batch.req_ids[:num_reqs]), qsl,
                                    [int(x) for x in self.runner.query_start_loc_np[:num_reqs + 1]],
                                    [int(x) for x in self.runner.seq_lens_np[:num_reqs]],
                                    self.block_table.get_device_tensor()[:num_reqs], finished)


class InQuantBatchBackend(InQuantBackend):
    """The backend description of the many-request lifecycle."""

    @staticmethod
    def get_name():
        return "INQUANT_PAGED_K4V2_BATCH_V1"

    @staticmethod
    def get_impl_cls():
        return InQuantBatchImpl

    @staticmethod
    def get_metadata_cls():
        return InQuantBatchMetadata

    @staticmethod
    def get_builder_cls():
        return InQuantBatchMetadataBuilder


class _Slot(_Request):
    """A request of the batch lifecycle and its row of the dense buffer."""

    __slots__ = ("slot",)

    def __init__(self, request_id, tokens, sealed_pages, slot):
        super().__init__(request_id, tokens, sealed_pages)
        self.slot = slot


class InQuantBatchImpl(InQuantImpl):
    """One attention layer serving up to ``max_num_seqs`` requests per step.

    Each request owns one slot of the dense buffer [slots, 2, H, B + 4, 128]
    (rows 0..3 its sink, 4.. its open page), as the single-request
    implementation owns its one buffer.  A step validates every request
    before anything changes: a decode request whose id or length does not
    match its state is refused ("state mismatch"), as are multi-token steps
    of a running request (chunked prefill, speculative decode)."""

    def __init__(self, *args, max_num_seqs=None, **kwargs):
        super().__init__(*args, **kwargs)
        if max_num_seqs is None:
            sched = getattr(get_current_vllm_config(), "scheduler_config", None)
            max_num_seqs = getattr(sched, "max_num_seqs", None) or 16
        self.max_num_seqs = int(max_num_seqs)
        self.requests: dict = {}
        self._free = list(range(self.max_num_seqs - 1, -1, -1))

    # the single-request attributes describe no request here
    @property
    def request_id(self):
        return None

    def _buffers(self, query):
        if self.dense is None:
            self.dense = torch.zeros((self.max_num_seqs, 2, self.num_kv_heads, self.layout.block_size + SINK, 128),
                                     dtype=query.dtype, device=query.device)

    def release(self, request_id):
        """Forget a finished request and free its dense slot (its pages belong
        to the caller's page allocator)."""
        req = self.requests.pop(request_id, None)
        if req is not None:
            self._free.append(req.slot)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None):
        if output is None:
            raise ValueError("vLLM must supply an output buffer")
        self._buffers(query)
        if attn_metadata is None:
            return output               # memory profiling: no request state is touched
        if kv_cache.dtype != torch.uint8 or kv_cache.ndim != 2 or kv_cache.shape[1] != self.layout.page_bytes:
            raise RuntimeError("InQuant cache spec was not installed; refusing dense fallback")
        m = attn_metadata
        for rid in m.finished_req_ids:
            self.release(rid)
        qsl, n = m.query_start_loc_cpu, len(m.request_ids)
        if len(qsl) != n + 1 or len(m.seq_lens) != n or m.block_table.shape[0] < n:
            raise ValueError("Batch metadata lengths disagree")
        prefills, decodes = [], []
        for i, rid in enumerate(m.request_ids):
            count, context = qsl[i + 1] - qsl[i], m.seq_lens[i] - (qsl[i + 1] - qsl[i])
            if context == 0:
                prefills.append(i)
                continue
            if count != 1:
                raise RuntimeError("Chunked prefill/speculative multi-token decode is unsupported")
            req = self.requests.get(rid)
            if req is None or req.tokens != context:
                raise RuntimeError(f"InQuant request state mismatch; refusing stale tail reuse ({rid})")
            decodes.append(i)
        fresh = sum(1 for i in prefills if m.request_ids[i] not in self.requests)
        if fresh > len(self._free):
            raise RuntimeError(f"InQuant batch holds at most {self.max_num_seqs} requests")
        if prefills:
            self._prefill_batch(prefills, query, key, value, kv_cache, m, output)
        if decodes:
            self._decode_batch(decodes, query, key, value, kv_cache, m, output)
        self.max_tokens_seen = max([self.max_tokens_seen] + [r.tokens for r in self.requests.values()])
        return output

    def _to_device(self, rows, dtype, device):
        return torch.tensor(rows, dtype=dtype).to(device, non_blocking=True)

    def _page_ids(self, m, table_index, dev):
        """Physical ids m.block_table[r, c] for flat indices r * stride + c."""
        bt = m.block_table
        if bt.is_contiguous():
            return bt.reshape(-1)[self._to_device(table_index, torch.int64, dev)]
        w = bt.stride(0)
        return bt[self._to_device([f // w for f in table_index], torch.int64, dev),
                  self._to_device([f % w for f in table_index], torch.int64, dev)]

    def _prefill_batch(self, rows, query, key, value, kv_cache, m, output):
        b, h, qsl = self.layout.block_size, self.num_kv_heads, m.query_start_loc_cpu
        dev = query.device
        lo, hi = qsl[rows[0]], qsl[rows[-1] + 1]
        lengths = [qsl[i + 1] - qsl[i] for i in rows]
        if sum(lengths) == hi - lo:      # the prefill rows are contiguous: attend over them only
            cu = [qsl[i] - lo for i in rows] + [hi - lo]
        else:                            # every request as a sequence; decode rows are overwritten later
            lo, hi, cu = 0, qsl[-1], list(qsl)
        prefill_attention(query[lo:hi], key[lo:hi], value[lo:hi], self._to_device(cu, torch.int32, dev),
                          max(lengths), self.scale, output[lo:hi])
        # the sink and open-page rows of every new request, one gather and one scatter
        src, slot_of, pos_of, page_rows, table_index = [], [], [], [], []
        states = []
        for i, n in zip(rows, lengths):
            rid = m.request_ids[i]
            req = self.requests.get(rid)
            slot = req.slot if req is not None else self._free.pop()
            full, start = n // b, qsl[i]
            for t in list(range(min(SINK, n))):
                src.append(start + t), slot_of.append(slot), pos_of.append(t)
            for t in range(full * b, n):
                src.append(start + t), slot_of.append(slot), pos_of.append(SINK + t - full * b)
            for p in range(full):
                page_rows.append(start + p * b)
                table_index.append(i * m.block_table.stride(0) + p)
            states.append((rid, _Slot(rid, n, full, slot)))
        if src:
            index = self._to_device(src, torch.int64, dev)
            rows_kv = torch.stack((key.index_select(0, index), value.index_select(0, index)), 1)
            self.dense[self._to_device(slot_of, torch.int64, dev), :, :, self._to_device(pos_of, torch.int64, dev)] \
                = rows_kv.to(self.dense.dtype)
        for rid, st in states:
            self.requests[rid] = st
        if page_rows:
            # every full page of every new request: one launch over the batch's rows
            ks = (nat._i64 * 4)(0, key.stride(1), key.stride(0), 1)
            vs = (nat._i64 * 4)(0, value.stride(1), value.stride(0), 1)
            _launch(key.data_ptr(), value.data_ptr(), key.dtype, ks, vs,
                    self._to_device(page_rows, torch.int64, dev), len(page_rows), self.layout, kv_cache,
                    self._page_ids(m, table_index, dev))
            self.seal_calls += 1
        self.prefill_calls += 1

    def _decode_batch(self, rows, query, key, value, kv_cache, m, output):
        b, h, qsl = self.layout.block_size, self.num_kv_heads, m.query_start_loc_cpu
        dev = query.device
        reqs = [self.requests[m.request_ids[i]] for i in rows]
        qrows = [qsl[i] for i in rows]
        leading = qrows == list(range(len(rows))) and list(rows) == list(range(len(rows)))
        # one host plan -> one copy: token rows, slots, write positions, seq_info
        slots = [r.slot for r in reqs]
        plan = [qrows, slots, [SINK + r.tokens % b for r in reqs],
                [r.sealed_pages for r in reqs], [r.tokens % b + 1 for r in reqs],
                [min(SINK, r.tokens + 1) for r in reqs]]
        sink_rows = [j for j, r in enumerate(reqs) if r.tokens < SINK]
        nd = len(rows)
        # the partitions the decode needs (no workgroup past a short sequence's end)
        items = work_list([r.sealed_pages for r in reqs], b)
        flat = self._to_device([x for row in plan for x in row] + items, torch.int32, dev)
        dplan, work = flat[:6 * nd].view(6, nd), flat[6 * nd:]
        idx = dplan[:3].long()
        if leading:
            new_kv = torch.stack((key[:nd], value[:nd]), 1)
        else:
            new_kv = torch.stack((key.index_select(0, idx[0]), value.index_select(0, idx[0])), 1)
        new_kv = new_kv.to(self.dense.dtype)
        self.dense[idx[1], :, :, idx[2]] = new_kv
        if sink_rows:
            sel = self._to_device(sink_rows, torch.int64, dev)
            self.dense[idx[1][sel], :, :, self._to_device([reqs[j].tokens for j in sink_rows], torch.int64, dev)] \
                = new_kv[sel]
        for r in reqs:
            r.tokens += 1
        seq_info = dplan[3:6].t().contiguous()
        max_pages = max(r.sealed_pages for r in reqs)
        tables = m.block_table[:nd] if leading else m.block_table.index_select(0, self._to_device(rows, torch.int64, dev))
        q = query[:nd] if leading else query.index_select(0, idx[0])
        out = output[:nd] if leading else torch.empty_like(q, dtype=output.dtype)
        paged_decode_batch(q, kv_cache, tables[:, :max(1, max_pages)].contiguous(), seq_info, self.dense, max_pages,
                           self.layout, WORKSPACE, self.scale, out, dense_slots=dplan[1].contiguous(), work=work)
        if not leading:
            output.index_copy_(0, idx[0], out)
        # pages the decode tokens filled, sealed after attention from their slots
        full = [j for j, r in enumerate(reqs) if r.tokens % b == 0]
        if full:
            row = self.dense.stride(0) // 128            # token rows per slot (the strides are in elements)
            page_rows = [reqs[j].slot * row + SINK for j in full]
            table_index = [rows[j] * m.block_table.stride(0) + reqs[j].sealed_pages for j in full]
            ks = (nat._i64 * 4)(0, self.dense.stride(2), 128, 1)
            v_base = self.dense.data_ptr() + self.dense.stride(1) * self.dense.element_size()
            _launch(self.dense.data_ptr(), v_base, self.dense.dtype, ks, ks,
                    self._to_device(page_rows, torch.int64, dev), len(full), self.layout, kv_cache,
                    self._page_ids(m, table_index, dev))
            self.seal_calls += 1
            for j in full:
                reqs[j].sealed_pages += 1
        self.decode_calls += 1
