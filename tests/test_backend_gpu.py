"""The paged backend's page lifecycle without vLLM (restates
extensions/vllm/tests/test_backend.py:48-92 against the oracle): prefill
attends causally over exact K/V and seals full pages, decode writes the dense
tail, attends, then seals a page the token filled; the sealed pages are
bit-exact with the oracle's, outputs within tolerance of fp64 attention over
the dequantized history, and a stale request is refused."""
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu
B, H, HQ = 64, 4, 28


def _np(t):
    return t.detach().float().cpu().numpy()


def _pages(k, v, n_pages):
    """Oracle pages of the first n_pages * B tokens of k/v [tokens, H, 128]."""
    kp = k[:n_pages * B].reshape(n_pages, B, H, 128).transpose(0, 2, 1, 3)
    vp = v[:n_pages * B].reshape(n_pages, B, H, 128).transpose(0, 2, 1, 3)
    return oracle.pack_pages(oracle.k4_quantize(np.ascontiguousarray(kp), 8, 0.125, "min_error"),
                             oracle.v_quantize(np.ascontiguousarray(vp), 2, 64), H, B)


def _history(k, v, upto):
    """K/V [H, upto, 128] a decode attends to: sealed pages dequantized
    (first four tokens exact), the rest exact (backend.py:158-169)."""
    kh, vh = k[:upto].transpose(1, 0, 2).copy(), v[:upto].transpose(1, 0, 2).copy()
    sealed = (upto - 1) // B
    if sealed:
        kd, vd = oracle.unpack_pages(_pages(k, v, sealed), H, B, "bfloat16")
        kh[:, :sealed * B] = kd.transpose(1, 0, 2, 3).reshape(H, sealed * B, 128)
        vh[:, :sealed * B] = vd.transpose(1, 0, 2, 3).reshape(H, sealed * B, 128)
        kh[:, :4], vh[:, :4] = k[:4].transpose(1, 0, 2), v[:4].transpose(1, 0, 2)
    return kh, vh


def test_prefill_decode_page_boundary_request_reuse_and_stale_tail(monkeypatch):
    import inquant_vllm.backend as backend
    from inquant.triton_attention import SharedDecodeWorkspace
    monkeypatch.setattr(backend, "WORKSPACE", SharedDecodeWorkspace())
    monkeypatch.setattr(backend, "get_current_vllm_config", lambda: NS(
        cache_config=NS(block_size=B), model_config=NS(max_model_len=512)))
    impl = backend.InQuantImpl(HQ, 128, 128 ** -0.5, H, None, None, "auto")
    pool = torch.full((12, impl.layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    blocks = torch.tensor([7, 2, 9, 3, 5, 8, 6, 1], dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(99)
    for request, initial in [("one-token", 1), ("boundary", 63), ("reused-pages", 257)]:
        print(f"backend request {request}: prefill {initial} + 3 decode steps", flush=True)
        k = torch.randn((initial + 3, H, 128), generator=g, device="cuda")
        k[..., 40:42] *= 20
        k = k.to(torch.bfloat16)
        v = torch.randn((initial + 3, H, 128), generator=g, device="cuda").to(torch.bfloat16)
        q = torch.randn((initial + 3, HQ, 128), generator=g, device="cuda").to(torch.bfloat16)
        kn, vn, qn = _np(k), _np(v), _np(q)
        starts = torch.tensor([0, initial], dtype=torch.int32, device="cuda")
        meta = backend.InQuantMetadata(initial, initial, 0, starts, blocks, request)
        out = impl.forward(None, q[:initial], k[:initial], v[:initial], pool, meta, torch.empty_like(q[:initial]))
        exp = oracle.causal_attend(qn[:initial], kn[:initial], vn[:initial], 128 ** -0.5)
        assert (np.abs(_np(out) - exp) <= 0.02 + 0.02 * np.abs(exp)).all()
        assert impl.sealed_pages == initial // B and impl.tokens == initial
        for step in range(3):
            index = initial + step
            starts = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
            meta = backend.InQuantMetadata(1, index + 1, index, starts, blocks, request)
            out = impl.forward(None, q[index:index + 1], k[index:index + 1], v[index:index + 1], pool, meta,
                               torch.empty_like(q[:1]))
            kh, vh = _history(kn, vn, index + 1)
            exp = oracle.attend(qn[index], kh, vh, 128 ** -0.5)
            assert np.abs(_np(out)[0] - exp).max() <= 2e-3 + np.abs(exp).max() * 2 ** -8   # bf16 output
        sealed = impl.sealed_pages
        assert sealed == (initial + 3) // B
        if sealed:
            ids = blocks[:sealed].long()
            np.testing.assert_array_equal(pool[ids].cpu().numpy(), _pages(kn, vn, sealed))
    meta.request_id = "wrong-request"
    with pytest.raises(RuntimeError, match="state mismatch"):
        impl.forward(None, q[:1], k[:1], v[:1], pool, meta, torch.empty_like(q[:1]))
    # seals: the 63-token request fills page 0 on its first decode step; the
    # 257-token prefill seals its four full pages in one call
    assert impl.prefill_calls == 3 and impl.decode_calls == 9 and impl.seal_calls == 2


def test_backend_refusals_and_profile_call(monkeypatch):
    import inquant_vllm.backend as backend
    monkeypatch.setattr(backend, "_CONFIG", None)        # restored after the test
    backend.configure(block_size=16, max_model_len=256)
    with pytest.raises(ValueError, match="ALiBi"):
        backend.InQuantImpl(8, 128, 0.1, 2, torch.ones(8), None, "auto")
    with pytest.raises(ValueError, match="16 query heads"):
        backend.InQuantImpl(64, 128, 0.1, 2, None, None, "auto")
    impl = backend.InQuantImpl(8, 128, 0.1, 2, None, None, "auto")
    q = torch.zeros((1, 8, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    assert impl.forward(None, q, q[:, :2], q[:, :2], None, None, out) is out     # memory profiling call
    assert impl.request_id is None and impl.dense is not None
    with pytest.raises(RuntimeError, match="refusing dense fallback"):
        impl.forward(None, q, q[:, :2], q[:, :2], torch.empty((4, 8), device="cuda"),
                     backend.InQuantMetadata(1, 1, 0, torch.tensor([0, 1], device="cuda"), None, "r"), out)
    assert backend.InQuantBackend.get_kv_cache_shape(10, 16, 2, 128) == (10, 2 * (104 * 16 + 832))
