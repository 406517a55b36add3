"""The many-request page lifecycle (``InQuantBatchImpl``): the reference's
single-request lifecycle (extensions/vllm/src/inquant_vllm/backend.py:106-177,
tests/test_backend.py:48-92) run for 16 requests per step, against the
oracle.  Every decode output is within 2e-3 (plus the bf16 output rounding)
of fp64 attention over the request's history (sealed pages dequantized, the
first four tokens and the open page exact); every sealed page is bit-exact
with the oracle's page; prefill outputs meet the causal prefill bound."""
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu
B, H, HQ = 16, 4, 28
SCALE = 128 ** -0.5


def _np(t):
    return t.detach().float().cpu().numpy()


def _pages(k, v, first, count):
    """Oracle pages first .. first + count - 1 of one request's K/V [tokens, H, 128]."""
    sl = slice(first * B, (first + count) * B)
    kp = k[sl].reshape(count, B, H, 128).transpose(0, 2, 1, 3)
    vp = v[sl].reshape(count, B, H, 128).transpose(0, 2, 1, 3)
    return oracle.pack_pages(oracle.k4_quantize(np.ascontiguousarray(kp), 8, 0.125, "min_error"),
                             oracle.v_quantize(np.ascontiguousarray(vp), 2, 64), H, B)


def _history(k, v, total):
    """K/V [H, total, 128] the decode of token total - 1 attends to: the pages
    sealed before it dequantized (except the exact first four tokens), the
    rest exact (backend.py:158-169)."""
    kh, vh = k[:total].transpose(1, 0, 2).copy(), v[:total].transpose(1, 0, 2).copy()
    sealed = (total - 1) // B
    if sealed:
        kd, vd = oracle.unpack_pages(_pages(k, v, 0, sealed), H, B, "bfloat16")
        kh[:, :sealed * B] = kd.transpose(1, 0, 2, 3).reshape(H, sealed * B, 128)
        vh[:, :sealed * B] = vd.transpose(1, 0, 2, 3).reshape(H, sealed * B, 128)
        kh[:, :4], vh[:, :4] = k[:4].transpose(1, 0, 2), v[:4].transpose(1, 0, 2)
    return kh, vh


class _Req:
    def __init__(self, rid, length, pages, g):
        self.rid, self.pages = rid, pages
        k = torch.randn((length, H, 128), generator=g, device="cuda")
        k[..., 40:42] *= 20
        self.k = k.to(torch.bfloat16)
        self.v = torch.randn((length, H, 128), generator=g, device="cuda").to(torch.bfloat16)
        self.q = torch.randn((length, HQ, 128), generator=g, device="cuda").to(torch.bfloat16)
        self.kn, self.vn, self.qn = _np(self.k), _np(self.v), _np(self.q)
        self.done = 0              # tokens already given to the cache


def _step(backend, impl, pool, reqs, counts, finished=(), order=None):
    """One scheduler step: request r contributes counts[r] tokens (its prefill
    when r.done == 0, else one decode token).  Decode requests come first, as
    vLLM orders them, unless `order` gives the batch order."""
    if order is None:
        order = sorted(range(len(reqs)), key=lambda i: reqs[i].done == 0)
    reqs = [reqs[i] for i in order]
    counts = [counts[i] for i in order]
    qsl = np.cumsum([0] + counts).tolist()
    cat = lambda name: torch.cat([getattr(r, name)[r.done:r.done + c] for r, c in zip(reqs, counts)])
    q, k, v = cat("q"), cat("k"), cat("v")
    width = max(len(r.pages) for r in reqs)
    table = torch.tensor([r.pages + [0] * (width - len(r.pages)) for r in reqs], dtype=torch.int32, device="cuda")
    meta = backend.InQuantBatchMetadata([r.rid for r in reqs], torch.tensor(qsl, dtype=torch.int32, device="cuda"),
                                        qsl, [r.done + c for r, c in zip(reqs, counts)], table, tuple(finished))
    out = torch.full_like(q, float("nan"))
    impl.forward(None, q, k, v, pool, meta, out)
    got = _np(out)
    for r, c, a in zip(reqs, counts, qsl[:-1]):
        if r.done == 0:        # prefill: causal over the exact K/V
            exp = oracle.causal_attend(r.qn[:c], r.kn[:c], r.vn[:c], SCALE)
            bound = 2 ** -8 * float(np.abs(r.vn[:c]).max()) + 1e-4 + 2 ** -8 * np.abs(exp)
            assert (np.abs(got[a:a + c] - exp) <= bound).all(), r.rid
        else:
            kh, vh = _history(r.kn, r.vn, r.done + 1)
            exp = oracle.attend(r.qn[r.done], kh, vh, SCALE)
            err = float(np.abs(got[a] - exp).max())
            assert err <= 2e-3 + np.abs(exp).max() * 2 ** -8, (r.rid, r.done, err)
        r.done += c


def _check_pages(pool, reqs):
    for r in reqs:
        sealed = r.done // B
        if r.done and sealed:
            ids = torch.tensor(r.pages[:sealed], dtype=torch.int64, device="cuda")
            np.testing.assert_array_equal(pool[ids].cpu().numpy(), _pages(r.kn, r.vn, 0, sealed), err_msg=r.rid)


def test_sixteen_requests_across_page_boundaries_finish_and_page_reuse(monkeypatch):
    import inquant_vllm.backend as backend
    from inquant.triton_attention import SharedDecodeWorkspace
    monkeypatch.setattr(backend, "WORKSPACE", SharedDecodeWorkspace())
    monkeypatch.setattr(backend, "get_current_vllm_config", lambda: NS(
        cache_config=NS(block_size=B), model_config=NS(max_model_len=512), scheduler_config=NS(max_num_seqs=16)))
    impl = backend.InQuantBatchImpl(HQ, 128, SCALE, H, None, None, "auto")
    g = torch.Generator(device="cuda").manual_seed(2024)
    free = torch.randperm(160, generator=g, device="cuda").tolist()
    pool = torch.full((160, impl.layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    lengths = [1, 3, 4, 5, 15, 16, 17, 31, 32, 33, 47, 50, 63, 64, 70, 90]
    steps = 20

    def request(rid, prefill):
        pages = [free.pop() for _ in range((prefill + steps) // B + 1)]
        return _Req(rid, prefill + steps, pages, g)

    reqs = [request(f"req-{i}", n) for i, n in enumerate(lengths)]
    print("batch lifecycle: prefill 16 requests", flush=True)
    _step(backend, impl, pool, reqs, lengths)
    assert impl.seal_calls == 1 and impl.prefill_calls == 1
    _check_pages(pool, reqs)
    finished, order = (), None
    for step in range(steps):
        counts = [1] * len(reqs)
        if step == 8:
            # requests 5 and 9 finish: their slots are released and their pages
            # go back to the allocator; two new requests prefill in the same
            # step as the other decodes, reusing those pages, placed in the
            # batch between decode requests (rows of neither kind contiguous)
            gone = [reqs.pop(9), reqs.pop(5)]
            for r in gone:
                free.extend(r.pages)
            finished = tuple(r.rid for r in gone)
            reqs += [request("new-a", 37), request("new-b", 5)]
            counts = [1] * (len(reqs) - 2) + [37, 5]
            order = [0, 1, 14, 2, 3, 15] + list(range(4, 14))
        print(f"batch lifecycle: step {step}", flush=True)
        _step(backend, impl, pool, reqs, counts, finished, order)
        finished, order = (), None
        assert len(impl.requests) == 16
    _check_pages(pool, reqs)
    assert all(impl.requests[r.rid].tokens == r.done for r in reqs)
    assert "req-5" not in impl.requests and "req-9" not in impl.requests


def test_stale_requests_are_refused_before_any_change(monkeypatch):
    import inquant_vllm.backend as backend
    from inquant.triton_attention import SharedDecodeWorkspace
    monkeypatch.setattr(backend, "WORKSPACE", SharedDecodeWorkspace())
    monkeypatch.setattr(backend, "get_current_vllm_config", lambda: NS(
        cache_config=NS(block_size=B), model_config=NS(max_model_len=256)))
    impl = backend.InQuantBatchImpl(HQ, 128, SCALE, H, None, None, "auto", max_num_seqs=3)
    g = torch.Generator(device="cuda").manual_seed(7)
    pool = torch.full((40, impl.layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    reqs = [_Req("a", 40, list(range(0, 4)), g), _Req("b", 40, list(range(4, 8)), g)]
    _step(backend, impl, pool, reqs, [20, 9])
    before = {rid: (r.tokens, r.sealed_pages, r.slot) for rid, r in impl.requests.items()}
    dense = impl.dense.clone()
    qsl = [0, 1, 2]
    table = torch.tensor([reqs[0].pages, reqs[1].pages], dtype=torch.int32, device="cuda")
    x = torch.zeros((2, HQ, 128), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((2, H, 128), dtype=torch.bfloat16, device="cuda")
    for ids, lens, match in ((["a", "b"], [21, 11], "state mismatch"),     # b's length is stale
                             (["a", "zzz"], [21, 10], "state mismatch"),   # unknown request
                             (["a", "b"], [21, 12], "multi-token")):       # b sends two tokens
        q_sl = qsl if match != "multi-token" else [0, 1, 3]
        xx = x if match != "multi-token" else torch.zeros((3, HQ, 128), dtype=torch.bfloat16, device="cuda")
        kk = kv if match != "multi-token" else torch.zeros((3, H, 128), dtype=torch.bfloat16, device="cuda")
        meta = backend.InQuantBatchMetadata(ids, torch.tensor(q_sl, dtype=torch.int32, device="cuda"), q_sl, lens,
                                            table, ())
        with pytest.raises(RuntimeError, match=match):
            impl.forward(None, xx, kk, kk, pool, meta, torch.empty_like(xx))
        assert {rid: (r.tokens, r.sealed_pages, r.slot) for rid, r in impl.requests.items()} == before
        assert torch.equal(impl.dense, dense)
    _step(backend, impl, pool, reqs, [1, 1])          # the valid step still runs
    reqs3 = [_Req(f"c{i}", 8, [20 + i], g) for i in range(2)]
    meta = backend.InQuantBatchMetadata(["c0", "c1"], torch.tensor([0, 8, 16], dtype=torch.int32, device="cuda"),
                                        [0, 8, 16], [8, 8], torch.tensor([[20], [21]], dtype=torch.int32,
                                                                          device="cuda"), ())
    with pytest.raises(RuntimeError, match="at most 3 requests"):
        impl.forward(None, torch.cat([r.q for r in reqs3]), torch.cat([r.k for r in reqs3]),
                     torch.cat([r.v for r in reqs3]), pool, meta, torch.empty_like(torch.cat([r.q for r in reqs3])))


@pytest.mark.parametrize("block,lengths", [(64, [1, 3, 60, 63, 64, 65, 100, 130]),
                                           (256, [4, 250, 255, 256, 257, 300, 20, 511])])
def test_batch_lifecycle_with_64_and_256_token_pages(monkeypatch, block, lengths):
    # the same lifecycle at the reference's page sizes 64 and 256: eight
    # requests, prefills and decodes crossing page boundaries, every output
    # against the oracle and every sealed page bit-exact
    import sys
    import inquant_vllm.backend as backend
    from inquant.triton_attention import SharedDecodeWorkspace
    monkeypatch.setattr(sys.modules[__name__], "B", block)
    monkeypatch.setattr(backend, "WORKSPACE", SharedDecodeWorkspace())
    monkeypatch.setattr(backend, "get_current_vllm_config", lambda: NS(
        cache_config=NS(block_size=block), model_config=NS(max_model_len=1024), scheduler_config=NS(max_num_seqs=8)))
    impl = backend.InQuantBatchImpl(HQ, 128, SCALE, H, None, None, "auto")
    g = torch.Generator(device="cuda").manual_seed(block)
    steps = 12
    npages = sum((n + steps) // block + 1 for n in lengths) + 8
    free = torch.randperm(npages, generator=g, device="cuda").tolist()
    pool = torch.full((npages, impl.layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    reqs = [_Req(f"r{i}", n + steps, [free.pop() for _ in range((n + steps) // block + 1)], g)
            for i, n in enumerate(lengths)]
    print(f"batch lifecycle, {block}-token pages: prefill", flush=True)
    _step(backend, impl, pool, reqs, lengths)
    _check_pages(pool, reqs)
    for step in range(steps):
        _step(backend, impl, pool, reqs, [1] * len(reqs))
    _check_pages(pool, reqs)
    assert all(impl.requests[r.rid].tokens == r.done for r in reqs)
