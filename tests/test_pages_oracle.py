"""CPU checks of the page-layout oracle and the paged host API (no GPU)."""
import numpy as np
import pytest
import torch

from oracle import oracle


@pytest.mark.parametrize("B", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("H", [1, 4, 8])
def test_page_layout_closed_form(B, H):
    # layout.py:18-45: field-major page, H * (104 B + 832) bytes
    from inquant_vllm import PageLayout
    offsets, size = oracle.page_offsets(H, B)
    assert size == H * (104 * B + 832)
    expect = {"key_payload": 0, "key_scales": 64 * H * B, "key_map": 64 * H * B + 512 * H,
              "key_padding": 64 * H * B + 768 * H, "value_payload": 64 * H * B + 832 * H,
              "value_scales": 96 * H * B + 832 * H, "value_offsets": 100 * H * B + 832 * H}
    assert offsets == expect
    layout = PageLayout(B, H)
    assert layout.page_bytes == size and layout.offsets == expect
    assert all(v % 16 == 0 for v in expect.values()) and size % 16 == 0


def test_page_layout_validation():
    from inquant_vllm import PageLayout
    for bad in ((48, 4, 128), (64, 0, 128), (64, 4, 64)):
        with pytest.raises(ValueError, match="Expected block_size"):
            PageLayout(*bad)
    layout = PageLayout(64, 2)
    with pytest.raises(ValueError, match="uint8 storage"):
        layout.views(torch.zeros(3, layout.page_bytes + 1, dtype=torch.uint8))


@pytest.mark.parametrize("B", [16, 64, 128, 256])
def test_oracle_unpack_of_pack_is_dequantize_of_quantize(B):
    # test_pages.py:9-19: pages restore exactly what the codecs decode
    rng = np.random.default_rng(B)
    H, P = 2, 3
    k = oracle.to_bf16(rng.standard_normal((P, H, B, 128)).astype(np.float32))
    v = oracle.to_bf16(rng.standard_normal((P, H, B, 128)).astype(np.float32))
    k[..., 7:9] *= 20
    kq, vq = oracle.k4_quantize(k, 8, 0.125, "min_error"), oracle.v_quantize(v, 2, 64)
    pages = oracle.pack_pages(kq, vq, H, B)
    assert pages.shape == (P, oracle.page_offsets(H, B)[1])
    kr, vr = oracle.unpack_pages(pages, H, B, "bfloat16")
    np.testing.assert_array_equal(kr.view(np.uint32), oracle.k4_dequantize(kq, "bfloat16").view(np.uint32))
    np.testing.assert_array_equal(vr.view(np.uint32), oracle.v_dequantize(vq, 2, 64, "bfloat16").view(np.uint32))
    assert oracle.page_offsets(H, B)[1] < B * H * 128 * 4 * 0.8 or B < 64


def test_oracle_role_map_in_pages():
    # roles: -1 normal, donor channel for a source, -2 - j for donor j
    rng = np.random.default_rng(3)
    k = oracle.to_bf16(rng.standard_normal((1, 1, 64, 128)).astype(np.float32))
    k[..., 40:43] *= 30
    kq = oracle.k4_quantize(k, 8, 0.125, "min_error")
    vq = oracle.v_quantize(k, 2, 64)
    role = oracle.page_views(oracle.pack_pages(kq, vq, 1, 64), 1, 64)["key_map"][0, 0]
    src, don = kq["salient_channels"][0, 0], kq["donor_channels"][0, 0]
    assert (role[src] == don).all()
    assert (role[don] == -2 - np.arange(16)).all()
    assert (np.delete(role, np.concatenate([src, don])) == -1).all()


def test_paged_token_selection_known_answers():
    # kernels.py:37 (packed tokens before the sink length are skipped) and
    # :48 (dense slots: the sink, then tail slots whose position is past the sink)
    H, B = 1, 16
    rng = np.random.default_rng(9)
    k = oracle.to_bf16(rng.standard_normal((2, H, B, 128)).astype(np.float32))
    kq, vq = oracle.k4_quantize(k, 8, 0.125, "min_error"), oracle.v_quantize(k, 2, 64)
    pool = oracle.pack_pages(kq, vq, H, B)
    dense = np.arange(2 * H * (B + 4) * 128, dtype=np.float32).reshape(2, H, B + 4, 128)
    kt, _ = oracle.paged_tokens(pool, [1, 0], dense, 2, 5, 4, H, B)
    assert kt.shape[1] == 2 * B - 4 + 4 + 5
    np.testing.assert_array_equal(kt[0, 2 * B - 4:2 * B], dense[0, 0, :4])          # sink slots
    np.testing.assert_array_equal(kt[0, 2 * B:], dense[0, 0, 4:9])                 # tail slots
    # no pages: tail slots at positions 0 .. 4 overlap a 3-token sink
    kt, _ = oracle.paged_tokens(pool, [], dense, 0, 5, 3, H, B)
    assert kt.shape[1] == 3 + 2
    np.testing.assert_array_equal(kt[0, 3:], dense[0, 0, 7:9])


def test_paged_host_validation_without_gpu():
    from inquant_vllm import PageLayout, paged_decode, write_codec_pages
    from inquant.triton_attention import SharedDecodeWorkspace
    layout = PageLayout(64, 4)
    pool = torch.zeros(4, layout.page_bytes, dtype=torch.uint8)
    q = torch.zeros(1, 28, 128, dtype=torch.bfloat16)
    dense = torch.zeros(2, 4, 68, 128, dtype=torch.bfloat16)
    ids = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="one BF16 query"):
        paged_decode(q.float(), pool, ids, dense, 1, 1, 1, layout, SharedDecodeWorkspace(), 0.1)
    with pytest.raises(ValueError, match="1..16 query heads"):
        paged_decode(torch.zeros(1, 27, 128, dtype=torch.bfloat16), pool, ids, dense, 1, 1, 1, layout,
                     SharedDecodeWorkspace(), 0.1)
    with pytest.raises(ValueError, match="out of range"):
        paged_decode(q, pool, ids, dense, 3, 1, 1, layout, SharedDecodeWorkspace(), 0.1)
    with pytest.raises(RuntimeError, match="require ROCm GPU tensors"):
        paged_decode(q, pool, ids, dense, 1, 1, 1, layout, SharedDecodeWorkspace(), 0.1)
    with pytest.raises(ValueError, match="contiguous uint8 destination"):
        write_codec_pages(None, None, layout, pool[:, :-1], ids)


def test_work_list_names_every_partition_once_longest_first():
    # the paged decode's compacted work list: packed partitions of 256 tokens
    # of pages, then the dense partition(s) (sink and open page), per sequence
    from inquant_vllm import work_list
    items = work_list([0, 17, 33, 2], 16)
    seqs = [i >> 16 for i in items]
    parts = {}
    for i in items:
        parts.setdefault(i >> 16, []).append(i & 0xffff)
    assert parts == {0: [0], 1: [0, 1, 2], 2: [0, 1, 2, 3], 3: [0, 1]}
    assert seqs == sorted(seqs, key=lambda s: -len(parts[s]))          # longest first, consecutive
    assert work_list([3], 256) == [0, 1, 2, 3, 4]                       # 260-token dense buffer: two
