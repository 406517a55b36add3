"""GPU parity of the causal prefill attention (the plugin's
flash_attn_varlen_func call, backend.py:139-144) against the fp64 oracle.

Tolerance: the reference's own prefill bound against SDPA (atol 0.02,
rtol 0.02, extensions/vllm/tests/test_backend.py:73), since the kernel, like
flash attention, rounds the softmax weights to the K/V dtype before P.V; the
fp32 output of bf16 inputs is additionally held to 1e-2 max-abs."""
import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


def _qkv(seed, n, hq, h, dtype):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((n, hq, 128), generator=g, device="cuda").to(dtype)
    k = torch.randn((n, h, 128), generator=g, device="cuda")
    k[..., 17:19] *= 8
    v = torch.randn((n, h, 128), generator=g, device="cuda")
    return q, k.to(dtype), v.to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 130, 257, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_matches_causal_oracle(n, dtype):
    from inquant_vllm import prefill_attention
    print(f"prefill n={n} {dtype}", flush=True)
    hq, h = 28, 4
    q, k, v = _qkv(n + 7, n, hq, h, dtype)
    cu = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    out = prefill_attention(q, k, v, cu, n, 128 ** -0.5)
    out32 = prefill_attention(q, k, v, cu, n, 128 ** -0.5, torch.empty(q.shape, device="cuda"))
    exp = oracle.causal_attend(_np(q), _np(k), _np(v), 128 ** -0.5)
    got = _np(out)
    assert out.dtype == dtype and np.isfinite(got).all()
    assert (np.abs(got - exp) <= 0.02 + 0.02 * np.abs(exp)).all()
    assert np.abs(_np(out32) - exp).max() <= 1e-2
    assert torch.equal(out, out32.to(dtype))


def test_prefill_varlen_sequences_and_strided_views():
    # three sequences in one launch, q/k/v as views of a fused [tokens, heads, 128] projection
    from inquant_vllm import prefill_attention
    lens = [5, 300, 77]
    n, hq, h = sum(lens), 32, 8
    g = torch.Generator(device="cuda").manual_seed(9)
    qkv = torch.randn((n, hq + 2 * h, 128), generator=g, device="cuda").to(torch.bfloat16)
    q, k, v = qkv[:, :hq], qkv[:, hq:hq + h], qkv[:, hq + h:]
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32, device="cuda")
    out = torch.full((n, hq, 128), float("nan"), device="cuda")
    prefill_attention(q, k, v, cu, max(lens), 0.1, out)
    got = _np(out)
    for a, b in zip(np.cumsum([0] + lens)[:-1], np.cumsum(lens)):
        exp = oracle.causal_attend(_np(q[a:b]), _np(k[a:b]), _np(v[a:b]), 0.1)
        assert np.abs(got[a:b] - exp).max() <= 1e-2


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_prefill_unaligned_output_rows_take_the_element_path(out_dtype):
    # output rows 129 elements apart: the kernel cannot use 4-channel stores and
    # writes element by element; the values equal those of an aligned output
    from inquant_vllm import prefill_attention
    n, hq, h = 300, 28, 4
    q, k, v = _qkv(311, n, hq, h, torch.bfloat16)
    cu = torch.tensor([0, 137, n], dtype=torch.int32, device="cuda")
    aligned = prefill_attention(q, k, v, cu, 163, 128 ** -0.5, torch.empty((n, hq, 128), dtype=out_dtype, device="cuda"))
    pad = torch.full((n, hq, 129), float("nan"), dtype=out_dtype, device="cuda")
    prefill_attention(q, k, v, cu, 163, 128 ** -0.5, pad[..., :128])
    assert torch.equal(pad[..., :128], aligned)
    assert torch.isnan(pad[..., 128].float()).all()     # nothing written past the row


def _outlier_qkv(seed, n, hq, h):
    # the bench's prefill input: N(0, 1) bf16 with five of 128 key channels
    # (two adjacent pairs and one single channel, ~4%) scaled by 20
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((n, hq, 128), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((n, h, 128), generator=g, device="cuda")
    k[..., [17, 18, 60, 61, 127]] *= 20
    v = torch.randn((n, h, 128), generator=g, device="cuda")
    return q, k.to(torch.bfloat16), v.to(torch.bfloat16)


def _bound(v):
    """The bound the kernel meets: the softmax weights are rounded to bf16
    before P.V (as flash attention does), a relative change of at most 2^-8
    per weight, so an output moves by at most 2^-8 * max|V|; 1e-4 covers the
    fp32 accumulation.  (8K case: max|V| ~ 4.9, bound ~ 1.9e-2, measured
    ~ 4e-3.)"""
    return 2 ** -8 * float(np.abs(v).max()) + 1e-4


def test_prefill_qwen_8k_matches_causal_oracle():
    # the 8192-token Qwen2.5-7B causal prefill that the bench times (28 query
    # heads over 4 KV heads): every row of the first and last query heads,
    # and three row bands (first, middle, last 256 rows) of every head
    from inquant_vllm import prefill_attention
    n, hq, h = 8192, 28, 4
    q, k, v = _outlier_qkv(8192, n, hq, h)
    cu = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    out = prefill_attention(q, k, v, cu, n, 128 ** -0.5)
    out32 = prefill_attention(q, k, v, cu, n, 128 ** -0.5, torch.empty(q.shape, device="cuda"))
    assert torch.equal(out, out32.to(torch.bfloat16))
    qn, kn, vn, got = _np(q), _np(k), _np(v), _np(out32)
    bands = np.concatenate([np.arange(0, 256), np.arange(4000, 4256), np.arange(n - 256, n)])
    worst = 0.0
    for rows, heads in ((np.arange(n), [0, hq - 1]), (bands, list(range(hq)))):
        exp = oracle.causal_attend_rows(qn, kn, vn, 128 ** -0.5, rows, heads)
        err = np.abs(got[rows][:, heads] - exp)
        worst = max(worst, float(err.max()))
        bf = _np(out)[rows][:, heads]
        assert (np.abs(bf - exp) <= _bound(vn) + 2 ** -8 * np.abs(exp)).all()   # + bf16 output rounding
    print(f"8K prefill max-abs error {worst:.3e} (bound {_bound(vn):.3e})", flush=True)
    assert worst <= _bound(vn)


def test_prefill_varlen_batch_of_4k_tokens_matches_causal_oracle():
    # four sequences (4648 tokens) in one launch, every row of every head
    from inquant_vllm import prefill_attention
    lens = [1500, 37, 2600, 511]
    n, hq, h = sum(lens), 28, 4
    q, k, v = _outlier_qkv(4648, n, hq, h)
    starts = np.cumsum([0] + lens)
    cu = torch.tensor(starts, dtype=torch.int32, device="cuda")
    out = torch.full((n, hq, 128), float("nan"), device="cuda")
    prefill_attention(q, k, v, cu, max(lens), 128 ** -0.5, out)
    got, qn, kn, vn = _np(out), _np(q), _np(k), _np(v)
    worst = 0.0
    for a, b in zip(starts[:-1], starts[1:]):
        exp = oracle.causal_attend_rows(qn[a:b], kn[a:b], vn[a:b], 128 ** -0.5, np.arange(b - a), range(hq))
        worst = max(worst, float(np.abs(got[a:b] - exp).max()))
    print(f"varlen prefill max-abs error {worst:.3e} (bound {_bound(vn):.3e})", flush=True)
    assert worst <= _bound(vn)


def test_prefill_rejects_bad_arguments():
    from inquant_vllm import prefill_attention
    q, k, v = _qkv(1, 8, 4, 2, torch.bfloat16)
    cu = torch.tensor([0, 8], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="multiple"):
        prefill_attention(q[:, :3], k, v, cu, 8, 0.1)
    with pytest.raises(ValueError, match="int32"):
        prefill_attention(q, k, v, cu.long(), 8, 0.1)
    with pytest.raises(ValueError, match="BF16 or FP16"):
        prefill_attention(q.float(), k.float(), v.float(), cu, 8, 0.1)
