"""GPU parity of the paged cache: page bytes bit-exact against the oracle,
paged decode within 2e-3 of the fp64 oracle (restates the reference's
extensions/vllm/tests/test_pages.py and test_direct_packing.py)."""
import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _np(t):
    return t.detach().cpu().numpy()


def _kv(seed, shape, device="cuda"):
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(shape, generator=g, device=device)
    v = torch.randn(shape, generator=g, device=device)
    k[..., 17:19] *= 20
    return k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("block", [16, 64, 128, 256])
def test_page_layout_matches_existing_codecs(block):
    # test_pages.py:9-19, plus the page bytes against the oracle
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant_vllm import PageLayout, pack_pages, unpack_pages_reference
    layout = PageLayout(block, 2)
    k, v = _kv(7, (3, 2, block, 128))
    pages = pack_pages(k, v, layout)
    assert pages.shape == (3, layout.page_bytes)
    kq = oracle.k4_quantize(_np(k.float()), 8, 0.125, "min_error")
    vq = oracle.v_quantize(_np(v.float()), 2, 64)
    np.testing.assert_array_equal(_np(pages), oracle.pack_pages(kq, vq, 2, block))
    rk, rv = unpack_pages_reference(pages, layout)
    assert torch.equal(rk, quantize(k, CodecConfig(donor_policy="min_error")).dequantize())
    assert torch.equal(rv, quantize_values(v).dequantize())
    for dtype, name in ((torch.float32, "float32"), (torch.float16, "float16")):
        rk, rv = unpack_pages_reference(pages, layout, dtype)
        ok, ov = oracle.unpack_pages(_np(pages), 2, block, name)
        np.testing.assert_array_equal(_np(rk.float()).view(np.uint32), ok.view(np.uint32))
        np.testing.assert_array_equal(_np(rv.float()).view(np.uint32), ov.view(np.uint32))


@pytest.mark.parametrize("block", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("backend", ["torch", "triton"])
@pytest.mark.parametrize("heads", [4, 8])
def test_direct_scattered_pages_match_reference_and_reuse(block, backend, heads):
    # test_direct_packing.py:9-22
    from inquant_vllm import PageLayout, pack_pages, pack_pages_into
    layout = PageLayout(block, heads)
    pool = torch.full((7, layout.page_bytes), 173, device="cuda", dtype=torch.uint8)
    ids = torch.tensor([5, 0, 3], device="cuda", dtype=torch.int32)
    for r in range(2):
        k, v = _kv(915 + r, (3, heads, block, 128))
        reference = pack_pages(k, v, layout)
        pack_pages_into(k, v, layout, pool, ids, donor_backend=backend)
        assert torch.equal(pool[ids.long()], reference)
        assert (pool[torch.tensor([1, 2, 4, 6], device="cuda")] == 173).all()


@pytest.mark.parametrize("block,id_dtype", [(16, torch.int32), (64, torch.int64), (256, torch.int32)])
def test_write_codec_pages_scatters_codec_outputs_bit_exact(block, id_dtype):
    # packing.py:41-55 write_codec_pages: the codec's own outputs (quantize
    # with min_error, quantize_values V2 g64) scattered to random physical
    # ids; the page bytes, the int16 role map included, equal the oracle's
    # pages and every other page keeps its fill; a second write of other
    # pages to other ids leaves the first ones intact
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant_vllm import PageLayout, write_codec_pages
    layout = PageLayout(block, 4)
    pool = torch.full((23, layout.page_bytes), 173, device="cuda", dtype=torch.uint8)
    g = torch.Generator(device="cuda").manual_seed(5150 + block)
    perm = torch.randperm(23, generator=g, device="cuda").to(id_dtype)
    written, start = [], 0
    for r, n in enumerate((5, 3)):
        k, v = _kv(333 + 10 * block + r, (n, 4, block, 128))
        kq = quantize(k, CodecConfig(donor_policy="min_error"))
        vq = quantize_values(v, bits=2, group_size=64)
        ids = perm[start:start + n]
        start += n
        write_codec_pages(kq, vq, layout, pool, ids)
        ok = oracle.k4_quantize(_np(k.float()), 8, 0.125, "min_error")
        ov = oracle.v_quantize(_np(v.float()), 2, 64)
        written.append((ids.long(), oracle.pack_pages(ok, ov, 4, block)))
    torch.cuda.synchronize()
    used = torch.zeros(23, dtype=torch.bool, device="cuda")
    for ids, exp in written:
        np.testing.assert_array_equal(_np(pool[ids]), exp)
        role = _np(layout.views(pool[ids])["key_map"])
        np.testing.assert_array_equal(role, _np(layout.views(torch.from_numpy(exp))["key_map"]))
        assert (role >= -17).all() and ((role <= -2).sum(-1) == 16).all()      # 16 donors per (page, head)
        used[ids] = True
    assert (pool[~used] == 173).all()


def test_write_codec_pages_beyond_signed_32bit_byte_offset():
    # the physical page offset id * page_bytes past 2^31 bytes (packing.py:14
    # widens the id to int64): a 256-token page written there holds the same
    # bytes as one written at id 0
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    from inquant_vllm import PageLayout, write_codec_pages
    layout = PageLayout(256, 4)
    far = 2 ** 31 // layout.page_bytes + 2
    pool = torch.zeros((far + 1, layout.page_bytes), device="cuda", dtype=torch.uint8)
    k, v = _kv(919, (2, 4, 256, 128))
    kq = quantize(k, CodecConfig(donor_policy="min_error"))
    vq = quantize_values(v, bits=2, group_size=64)
    ids = torch.tensor([far, 0], device="cuda", dtype=torch.int64)
    assert far * layout.page_bytes > 2 ** 31
    write_codec_pages(kq, vq, layout, pool, ids)
    exp = oracle.pack_pages(oracle.k4_quantize(_np(k.float()), 8, 0.125, "min_error"),
                            oracle.v_quantize(_np(v.float()), 2, 64), 4, 256)
    np.testing.assert_array_equal(_np(pool[ids]), exp)
    assert not pool[1:far].any()


def _paged_case(seed, block, pages, tail, h=4, hq=28, spare=7):
    from inquant_vllm import PageLayout, pack_pages
    layout = PageLayout(block, h)
    g = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.full((pages + spare, layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    ids = torch.randperm(pages + spare, generator=g, device="cuda")[:pages].to(torch.int32)
    dense = torch.full((2, h, block + 4, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    k, v = _kv(seed + 1, (h, pages * block + tail, 128))
    sink = min(4, k.shape[1])
    dense[0, :, :sink], dense[1, :, :sink] = k[:, :sink], v[:, :sink]
    if tail:
        dense[0, :, 4:4 + tail], dense[1, :, 4:4 + tail] = k[:, -tail:], v[:, -tail:]
    if pages:
        kt = k[:, :pages * block].reshape(h, pages, block, 128).transpose(0, 1)
        vt = v[:, :pages * block].reshape(h, pages, block, 128).transpose(0, 1)
        pool.index_copy_(0, ids.long(), pack_pages(kt, vt, layout))
    q = torch.randn(1, hq, 128, generator=g, device="cuda").to(torch.bfloat16)
    return layout, pool, ids, dense, sink, q


def _expected(layout, pool, ids, dense, pages, tail, sink, q):
    d = _np(dense.float())
    return oracle.paged_attend(_np(q.float())[0], _np(pool), _np(ids), d, pages, tail, sink,
                               layout.heads, layout.block_size, 128 ** -0.5)


@pytest.mark.parametrize("block,pages,tail", [(64, 0, 1), (64, 0, 63), (64, 1, 0), (64, 1, 64), (128, 3, 17),
                                               (256, 128, 128), (256, 2, 256), (16, 1, 1), (16, 37, 9),
                                               (32, 9, 31), (16, 0, 3), (64, 600, 10)])
def test_paged_decode_random_page_order_and_reuse(block, pages, tail):
    # (64, 600, 10): 151 partitions, more than the merge's 144 per round
    # test_pages.py:22-58 (random physical order, unused pages full of 0xff,
    # NaN in dead dense slots, the workspace reused), against the fp64 oracle
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode
    workspace = SharedDecodeWorkspace()
    for reuse in range(2):
        layout, pool, ids, dense, sink, q = _paged_case(71 + reuse, block, pages, tail)
        actual = paged_decode(q, pool, ids, dense, pages, tail, sink, layout, workspace, 128 ** -0.5)
        assert actual.shape == q.shape and actual.dtype == torch.bfloat16
        got = _np(actual.float())[0]
        assert np.isfinite(got).all()
        exp = _expected(layout, pool, ids, dense, pages, tail, sink, q)
        assert np.abs(got - exp).max() <= ATOL + np.abs(exp).max() * 2 ** -8   # bf16 output rounding
        out32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
        paged_decode(q, pool, ids, dense, pages, tail, sink, layout, workspace, 128 ** -0.5, out32)
        assert np.abs(_np(out32)[0] - exp).max() <= ATOL


@pytest.mark.parametrize("block", [16, 64, 128, 256])
def test_paged_decode_reads_roles_as_the_role_map_states(block):
    # The decode takes every role from the page's int16 role map, as the
    # reference's _decode_tile does (kernels.py:34-35): role >= 0 is a source
    # whose low nibble comes from channel `role`, role <= -2 is donor
    # -2 - role (its padding), -1 a plain 4-bit channel.  Edited maps, decoded
    # by the oracle from the same bytes: a page with a source/donor pair made
    # plain (15 sources), a source whose partner is a plain channel, two
    # donors sharing one padding, a page with no salient channels at all.
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode
    pages, tail = 6, 5
    layout, pool, ids, dense, sink, q = _paged_case(97, block, pages, tail)
    roles = layout.views(pool)["key_map"]                       # [pool pages, H, 128] views of the pool
    pid = [int(i) for i in ids.tolist()]
    r = roles[pid[0], 0]
    s0 = int(torch.nonzero(r >= 0)[0])
    d0 = int(r[s0])
    r[s0], r[d0] = -1, -1                                       # a pair made plain
    r = roles[pid[1], 1]
    s1 = int(torch.nonzero(r >= 0)[0])
    plain = int(torch.nonzero(r == -1)[0])
    r[s1] = plain                                               # partner: a plain channel
    r = roles[pid[2], 2]
    donors = torch.nonzero(r <= -2).flatten()
    r[int(donors[0])] = r[int(donors[1])]                       # two donors, one padding
    roles[pid[3], 3] = -1                                       # no salient channels
    out32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    paged_decode(q, pool, ids, dense, pages, tail, sink, layout, SharedDecodeWorkspace(), 128 ** -0.5, out32)
    exp = _expected(layout, pool, ids, dense, pages, tail, sink, q)
    assert np.abs(_np(out32)[0] - exp).max() <= ATOL
    # the edits change the attended keys: the unedited pool decodes differently
    _, pool0, _, _, _, _ = _paged_case(97, block, pages, tail)
    assert np.abs(_expected(layout, pool0, ids, dense, pages, tail, sink, q) - exp).max() > 1e-4
    # unpacking reads the edited maps the same way, bit for bit
    from inquant_vllm import unpack_pages_reference
    edited = pool[ids.long()]
    rk, rv = unpack_pages_reference(edited, layout, torch.float32)
    ok, ov = oracle.unpack_pages(_np(edited), layout.heads, block, "float32")
    np.testing.assert_array_equal(_np(rk).view(np.uint32), ok.view(np.uint32))
    np.testing.assert_array_equal(_np(rv).view(np.uint32), ov.view(np.uint32))


@pytest.mark.parametrize("h,hq", [(4, 4), (2, 32)])
def test_paged_decode_query_group_sizes(h, hq):
    # one query row per KV head, and the 16 a matrix-core tile holds
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode
    layout, pool, ids, dense, sink, q = _paged_case(83, 16, 20, 5, h=h, hq=hq)
    out32 = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    paged_decode(q, pool, ids, dense, 20, 5, sink, layout, SharedDecodeWorkspace(), 128 ** -0.5, out32)
    exp = _expected(layout, pool, ids, dense, 20, 5, sink, q)
    assert np.abs(_np(out32)[0] - exp).max() <= ATOL


def test_paged_decode_batch_equals_single_sequences():
    # sequences of different lengths and pools in one launch (16-token pages)
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode, paged_decode_batch
    cases = [_paged_case(300 + i, 16, n, t) for i, (n, t) in enumerate([(5, 3), (0, 7), (40, 15), (13, 0)])]
    layout = cases[0][0]
    # one shared pool: append every case's pages, re-basing its ids
    pools, bases, tables, infos, dense, qs = [], 0, [], [], [], []
    max_pages = max(n for n, _ in [(5, 3), (0, 7), (40, 15), (13, 0)])
    for (lay, pool, ids, d, sink, q), (n, t) in zip(cases, [(5, 3), (0, 7), (40, 15), (13, 0)]):
        pools.append(pool)
        row = torch.zeros(max_pages, dtype=torch.int32, device="cuda")
        row[:n] = ids + bases
        tables.append(row)
        bases += pool.shape[0]
        infos.append([n, t, sink])
        dense.append(d)
        qs.append(q[0])
    pool = torch.cat(pools)
    out = paged_decode_batch(torch.stack(qs), pool, torch.stack(tables),
                             torch.tensor(infos, dtype=torch.int32, device="cuda"), torch.stack(dense),
                             max_pages, layout, SharedDecodeWorkspace(), 128 ** -0.5)
    for i, ((lay, p1, ids, d, sink, q), (n, t)) in enumerate(zip(cases, [(5, 3), (0, 7), (40, 15), (13, 0)])):
        single = paged_decode(q, p1, ids, d, n, t, sink, lay, SharedDecodeWorkspace(), 128 ** -0.5)
        assert torch.equal(out[i], single[0])


def test_page_ids_outside_the_pool_contribute_nothing():
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import paged_decode
    layout, pool, ids, dense, sink, q = _paged_case(5, 64, 3, 10)
    bad = ids.clone()
    bad[1] = pool.shape[0] + 100
    got = _np(paged_decode(q, pool, bad, dense, 3, 10, sink, layout, SharedDecodeWorkspace(), 128 ** -0.5)
              .float())[0]
    # expected: the same decode without page 1's tokens
    k, v = oracle.paged_tokens(_np(pool), _np(ids), _np(dense.float()), 3, 10, sink, 4, 64)
    live = np.ones(k.shape[1], bool)
    live[64 - sink:128 - sink] = False          # the token list starts after the first `sink` packed tokens
    exp = oracle.attend(_np(q.float())[0], k[:, live], v[:, live], 128 ** -0.5)
    assert np.abs(got - exp).max() <= ATOL + np.abs(exp).max() * 2 ** -8


def test_page_write_and_decode_beyond_signed_32bit_byte_offset():
    # test_direct_packing.py:25-46
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import PageLayout, pack_pages, pack_pages_into, paged_decode
    layout = PageLayout(64, 4)
    far = 2 ** 31 // layout.page_bytes + 1
    pool = torch.empty((far + 1, layout.page_bytes), device="cuda", dtype=torch.uint8)
    ids = torch.tensor([0, far], device="cuda", dtype=torch.int32)
    k, v = _kv(811, (1, 4, 64, 128))
    reference = pack_pages(k, v, layout)
    pack_pages_into(k.expand(2, -1, -1, -1), v.expand(2, -1, -1, -1), layout, pool, ids, donor_backend="triton")
    assert torch.equal(pool[ids.long()], reference.expand(2, -1))
    query = torch.randn(1, 28, 128, device="cuda", dtype=torch.bfloat16)
    tail = torch.randn(2, 4, 68, 128, device="cuda", dtype=torch.bfloat16)
    workspace = SharedDecodeWorkspace()
    near = paged_decode(query, pool, ids[:1], tail, 1, 1, 4, layout, workspace, 128 ** -0.5)
    far_out = paged_decode(query, pool, ids[1:], tail, 1, 1, 4, layout, workspace, 128 ** -0.5)
    assert torch.equal(near, far_out)


def test_paged_decode_batch_sixteen_sequences_against_oracle():
    # config 4 at its real shape: 16 sequences, contexts drawn from 2K..32K,
    # 16-token pages at random physical ids in one pool, per-sequence sink and
    # partial-page tail; every sequence within 2e-3 of the fp64 oracle
    # (kernels.py:8-88 semantics, batched over sequences in one launch)
    from inquant.triton_attention import SharedDecodeWorkspace
    from inquant_vllm import PageLayout, pack_pages, paged_decode_batch
    B, H, HQ, S = 16, 4, 28, 16
    layout = PageLayout(B, H)
    ctx = np.random.default_rng(404).integers(2048, 32769, S)
    pages = ctx // B
    tails = ctx % B
    total = int(pages.sum())
    print(f"cfg4 batch: contexts {ctx.tolist()}, {total} pages", flush=True)
    g = torch.Generator(device="cuda").manual_seed(404)
    perm = torch.randperm(total + 9, generator=g, device="cuda")[:total].to(torch.int32)
    pool = torch.full((total + 9, layout.page_bytes), 255, dtype=torch.uint8, device="cuda")
    max_pages = int(pages.max())
    tables = torch.zeros((S, max_pages), dtype=torch.int32, device="cuda")
    dense = torch.full((S, 2, H, B + 4, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    first = 0
    for i in range(S):
        n, t = int(pages[i]), int(tails[i])
        k, v = _kv(4040 + i, (H, int(ctx[i]), 128))
        ids = perm[first:first + n]
        first += n
        tables[i, :n] = ids
        kt = k[:, :n * B].reshape(H, n, B, 128).transpose(0, 1)
        vt = v[:, :n * B].reshape(H, n, B, 128).transpose(0, 1)
        pool.index_copy_(0, ids.long(), pack_pages(kt, vt, layout))
        dense[i, 0, :, :4], dense[i, 1, :, :4] = k[:, :4], v[:, :4]
        if t:
            dense[i, 0, :, 4:4 + t], dense[i, 1, :, 4:4 + t] = k[:, -t:], v[:, -t:]
    infos = torch.tensor([[int(pages[i]), int(tails[i]), 4] for i in range(S)], dtype=torch.int32, device="cuda")
    q = torch.randn(S, HQ, 128, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((S, HQ, 128), dtype=torch.float32, device="cuda")
    paged_decode_batch(q, pool, tables, infos, dense, max_pages, layout, SharedDecodeWorkspace(), 128 ** -0.5,
                       out)
    got = _np(out)
    pool_np, tables_np, dense_np, q_np = _np(pool), _np(tables), _np(dense.float()), _np(q.float())
    for i in range(S):
        exp = oracle.paged_attend(q_np[i], pool_np, tables_np[i], dense_np[i], int(pages[i]), int(tails[i]), 4,
                                  H, B, 128 ** -0.5)
        err = float(np.abs(got[i] - exp).max())
        assert err <= ATOL, (i, int(ctx[i]), err)
    # the compacted work list (only the partitions that exist, longest
    # sequences first) runs the same partitions: bit-identical outputs; a
    # list in another order, and items outside the batch, change nothing
    from inquant_vllm import work_list
    items = work_list(pages.tolist(), B)
    assert len(items) == sum(-(-int(n) // 16) + 1 for n in pages)
    for order in (items, items[::-1] + [(S << 16) | 0, (0 << 16) | 0xfff0]):
        listed = torch.full_like(out, float("nan"))
        paged_decode_batch(q, pool, tables, infos, dense, max_pages, layout, SharedDecodeWorkspace(), 128 ** -0.5,
                           listed, work=torch.tensor(order, dtype=torch.int32, device="cuda"))
        assert torch.equal(listed, out)


@pytest.mark.parametrize("block", [16, 32, 64, 256])
def test_pack_pages_into_is_one_launch_and_reports_non_finite_inputs(block):
    # the fused page encoder: K4 min_error, role map and V2 written straight
    # into the physical pages by one kernel, bit-exact with the oracle's
    # pages; a non-finite key or value raises the codec's message
    from inquant_vllm import PageLayout, pack_pages_into
    layout = PageLayout(block, 4)
    pool = torch.full((9, layout.page_bytes), 7, device="cuda", dtype=torch.uint8)
    ids = torch.tensor([8, 1, 4], device="cuda", dtype=torch.int64)
    k, v = _kv(977, (3, 4, block, 128))
    pack_pages_into(k, v, layout, pool, ids)           # warm (first-use allocations)
    torch.cuda.synchronize()
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        pack_pages_into(k, v, layout, pool, ids)
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA
               and "memcpy" not in e.name.lower() and "memset" not in e.name.lower()]
    assert len(kernels) == 1 and "k4_encode" in kernels[0], kernels
    kq = oracle.k4_quantize(_np(k.float()), 8, 0.125, "min_error")
    vq = oracle.v_quantize(_np(v.float()), 2, 64)
    np.testing.assert_array_equal(_np(pool[ids]), oracle.pack_pages(kq, vq, 4, block))
    assert (pool[torch.tensor([0, 2, 3, 5, 6, 7], device="cuda")] == 7).all()
    bad_k, bad_v = k.clone(), v.clone()
    bad_k[1, 2, 3, 4] = float("nan")
    bad_v[2, 0, 5, 6] = float("inf")
    with pytest.raises(ValueError, match="finite values"):
        pack_pages_into(bad_k, v, layout, pool, ids)
    with pytest.raises(ValueError, match="FP16 quantization parameters"):
        pack_pages_into(k, bad_v, layout, pool, ids)
    pack_pages_into(k, v, layout, pool, ids)           # flags cleared for the next call
    np.testing.assert_array_equal(_np(pool[ids]), oracle.pack_pages(kq, vq, 4, block))


@pytest.mark.parametrize("block", [16, 32])
def test_short_pages_half_inputs_partial_workgroups_and_skipped_ids(block):
    # 16- and 32-token pages are encoded one wavefront per (page, head), four
    # pages per workgroup: six pages leave the second workgroup half empty,
    # and ids outside the pool (negative or too large) write nothing and
    # raise after the launch; the next in-range call finds the flags cleared
    from inquant_vllm import PageLayout, pack_pages_into
    layout = PageLayout(block, 4)
    pool = torch.full((8, layout.page_bytes), 7, device="cuda", dtype=torch.uint8)
    ids = torch.tensor([3, -1, 8, 0, 5, 6], device="cuda", dtype=torch.int64)
    g = torch.Generator(device="cuda").manual_seed(4242 + block)
    k = torch.randn((6, 4, block, 128), generator=g, device="cuda")
    v = torch.randn((6, 4, block, 128), generator=g, device="cuda")
    k[..., 40:43] *= 30
    k, v = k.to(torch.float16), v.to(torch.float16)
    with pytest.raises(ValueError, match="outside the destination pool"):
        pack_pages_into(k, v, layout, pool, ids)
    live = [0, 3, 4, 5]
    kq = oracle.k4_quantize(_np(k[live].float()), 8, 0.125, "min_error")
    vq = oracle.v_quantize(_np(v[live].float()), 2, 64)
    np.testing.assert_array_equal(_np(pool[torch.tensor([3, 0, 5, 6], device="cuda")]),
                                  oracle.pack_pages(kq, vq, 4, block))
    assert (pool[torch.tensor([1, 2, 4, 7], device="cuda")] == 7).all()
    pack_pages_into(k[live], v[live], layout, pool, ids[live])      # flags cleared: no error
    np.testing.assert_array_equal(_np(pool[torch.tensor([3, 0, 5, 6], device="cuda")]),
                                  oracle.pack_pages(kq, vq, 4, block))
