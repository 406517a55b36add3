"""InQuantCache behaviour on the GPU, restating the reference's cache tests
(tests/test_cache.py:15-158, test_value_codec.py:52-76) with ROCm tensors:
storage ownership and accounting, append chunking over seal boundaries,
immutable sealed blocks, sink accumulation, batched prefill equal to serial
per-block encodes, position checks, reset, a 32K-token layer, and the append
view against update() across seals.  Serial encodes are additionally pinned
to the CPU oracle, so the comparison is not only self-consistency."""
from unittest.mock import patch

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from inquant.cache import CacheConfig
    from inquant.codec import CodecConfig
    base = dict(block_size=8, residual_length=3, sink_tokens=2)
    base.update(kw)
    codec = base.pop("codec", CodecConfig(salient_fraction=0))
    return CacheConfig(codec, **base)


def _randn(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


def test_prefill_exact_small_tail_storage_and_accounting():
    # test_cache.py:15-31
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    key, value = _randn(1, 2, 37, 8, seed=1), _randn(1, 2, 37, 8, seed=2)
    returned_key, returned_value = cache.update(key, value, 0)
    assert returned_key is key and returned_value is value
    layer = cache._layers[0]
    # the exact rows live in the cache's own [2, H, rows, D] buffers (never a
    # view of the prefill input); accounting counts the live rows, and the
    # unfilled part of the preallocated tail is reported separately
    for item in (layer.sink_key, layer.sink_value, layer.residual_key, layer.residual_value):
        assert item.untyped_storage().data_ptr() != key.untyped_storage().data_ptr()
    assert cache.sink_nbytes == 2 * 2 * 2 * 8 * 4 and cache.residual_nbytes == 2 * 2 * 3 * 8 * 4
    assert torch.equal(layer.sink_key, key[:, :, :2]) and torch.equal(layer.residual_value, value[:, :, -3:])
    held = layer.tail.buf.untyped_storage().nbytes() + layer.sink.buf.untyped_storage().nbytes()
    assert cache.memory_stats()["dense_reserve_nbytes"] == held - cache.sink_nbytes - cache.residual_nbytes
    packed_bytes = sum(block.nbytes for block in layer.key_blocks + layer.value_blocks)
    assert cache.nbytes == packed_bytes + cache.sink_nbytes + cache.residual_nbytes
    assert cache.bf16_nbytes == 2 * key.numel() * 2
    assert cache.memory_stats()["quantized_layer_tokens"] == 32
    assert cache.get_seq_length() == 37 and cache.get_usable_length(2) == 37
    assert cache.get_max_cache_shape() is None


def test_multihead_append_chunking_and_old_blocks_immutable():
    # test_cache.py:33-59, with the serial blocks also checked against the oracle
    from inquant.cache import InQuantCache
    from inquant.codec import quantize
    cfg = _cfg()
    cache = InQuantCache(cfg)
    key, value = _randn(1, 3, 61, 8, seed=3), _randn(1, 3, 61, 8, seed=4)
    cache.update(key[:, :, :21], value[:, :, :21], 0)
    old_block = cache._layers[0].key_blocks[0]
    old_decoded = old_block.dequantize().clone()
    seen = 21
    for count in (1, 7, 12, 20):
        prior_key, prior_value = cache.materialize()
        out_key, out_value = cache.update(key[:, :, seen:seen + count], value[:, :, seen:seen + count], 0)
        torch.testing.assert_close(out_key, torch.cat((prior_key, key[:, :, seen:seen + count]), dim=2))
        torch.testing.assert_close(out_value, torch.cat((prior_value, value[:, :, seen:seen + count]), dim=2))
        seen += count
    layer = cache._layers[0]
    assert layer.key_blocks[0] is old_block
    torch.testing.assert_close(old_block.dequantize(), old_decoded, rtol=0, atol=0)
    blocks = (seen - cfg.sink_tokens - cfg.residual_length) // cfg.block_size
    for original, actual, sealed in ((key, cache.materialize()[0], layer.key_blocks),
                                     (value, cache.materialize()[1], layer.value_blocks)):
        pieces = [original[:, :, :2]]
        for index in range(blocks):
            start = 2 + index * 8
            serial = quantize(original[:, :, start:start + 8], cfg.codec)
            pieces.append(serial.dequantize(dtype=original.dtype))
            ref = oracle.k4_quantize(original[:, :, start:start + 8].cpu().numpy(), cfg.codec.sample_stride,
                                     cfg.codec.salient_fraction, cfg.codec.donor_policy)
            np.testing.assert_array_equal(sealed[index].payload.cpu().numpy(), ref["payload"])
            np.testing.assert_array_equal(sealed[index].scales.cpu().numpy().view(np.uint32),
                                          ref["scales"].view(np.uint32))
        pieces.append(original[:, :, 2 + blocks * 8:])
        torch.testing.assert_close(actual, torch.cat(pieces, dim=2), rtol=0, atol=0)
    assert seen == 61 and cache.get_seq_length() == 61
    assert layer.residual_key.shape[2] < cfg.residual_length + cfg.block_size


@pytest.mark.parametrize("value_bits", [None, 2])
def test_materialize_equals_per_block_dequantize_across_runs(value_bits):
    # materialize dequantizes a prefill's blocks (views of one batched encode)
    # in one launch per run and sealed blocks one by one: the result is the
    # reference's sink ++ [block.dequantize() for each block] ++ tail, bit for bit
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    cfg = CacheConfig(codec=CodecConfig(donor_policy="min_error"), block_size=32, residual_length=16, sink_tokens=4,
                      value_bits=value_bits, value_group_size=32)
    cache = InQuantCache(cfg)
    n0, extra = 4 + 32 * 6 + 16, 70
    key, value = _randn(1, 2, n0 + extra, 64, seed=41), _randn(1, 2, n0 + extra, 64, seed=42)
    key, value = key.to(torch.bfloat16), value.to(torch.bfloat16)
    cache.update(key[:, :, :n0], value[:, :, :n0], 0)
    for t in range(n0, n0 + extra):                 # two more blocks sealed one at a time
        cache.append_for_attention(key[:, :, t:t + 1], value[:, :, t:t + 1], 0)
    layer = cache._layers[0]
    assert layer.runs == [(0, 6), (6, 7), (7, 8)] and len(layer.key_blocks) == 8
    got_k, got_v = cache.materialize(0)
    for got, blocks, side in ((got_k, layer.key_blocks, key), (got_v, layer.value_blocks, value)):
        parts = [side[:, :, :4]] + [b.dequantize(dtype=torch.bfloat16) for b in blocks]
        parts.append(side[:, :, 4 + 32 * len(blocks):n0 + extra])
        expected = torch.cat(parts, 2)
        assert got.shape == expected.shape and torch.equal(got, expected)


def test_sink_accumulates_across_short_prefills():
    # test_cache.py:61-67
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    x = _randn(1, 2, 7, 8, seed=5)
    for pos in range(7):
        result, _ = cache.update(x[:, :, pos:pos + 1], x[:, :, pos:pos + 1], 0)
        torch.testing.assert_close(result, x[:, :, :pos + 1], rtol=0, atol=0)
    torch.testing.assert_close(cache.materialize()[0], x, rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batched_prefill_matches_serial_blocks_and_owns_compact_storage(dtype):
    # test_cache.py:69-108: heads and temporal blocks keep independent
    # statistics after the block axis moves into the batch; the reference
    # makes one encode call per tensor, this cache one library call for the
    # keys and values of all six blocks (iq_k4_quantize_kv over the strided
    # [6, 3, 8, 16] views); every field an owned compact tensor
    import inquant.cache as cache_mod
    from inquant.cache import InQuantCache
    from inquant.codec import CodecConfig, quantize
    cfg = _cfg(codec=CodecConfig(sample_stride=3, salient_fraction=.25))
    key = _randn(1, 3, 16, 55, seed=6, dtype=dtype).transpose(2, 3)
    value = _randn(1, 3, 16, 55, seed=7, dtype=dtype).transpose(2, 3)
    assert not key.is_contiguous()
    for index in range(6):
        key[:, index % 3, 2 + index * 8:10 + index * 8, index] *= 20
        value[:, (index + 1) % 3, 2 + index * 8:10 + index * 8, 15 - index] *= 17
    cache = InQuantCache(cfg)
    with patch.object(cache_mod, "_k4_pair_blocks", wraps=cache_mod._k4_pair_blocks) as observed, \
            patch.object(cache_mod, "quantize", wraps=quantize) as single:
        cache.update(key, value, 0)
    assert observed.call_count == 1 and single.call_count == 0
    assert observed.call_args.args[2:4] == (6, 8)
    layer = cache._layers[0]
    expected_bytes = 0
    ranges, storages = [], {}
    for original, blocks in ((key, layer.key_blocks), (value, layer.value_blocks)):
        assert len(blocks) == 6
        for index, actual in enumerate(blocks):
            start = 2 + index * 8
            serial = quantize(original[:, :, start:start + 8], cfg.codec)
            assert actual.shape == serial.shape and actual.original_dtype == dtype
            assert actual.nbytes == serial.nbytes
            expected_bytes += serial.nbytes
            for name, tensor in actual.tensors.items():
                torch.testing.assert_close(tensor, serial.tensors[name], rtol=0, atol=0)
                assert tensor.is_contiguous()
                if tensor.numel():
                    ranges.append((tensor.data_ptr(), tensor.data_ptr() + tensor.numel() * tensor.element_size()))
                    st = tensor.untyped_storage()
                    storages.setdefault(st.data_ptr(), [st.nbytes(), 0])[1] += tensor.numel() * tensor.element_size()
            torch.testing.assert_close(actual.dequantize(), serial.dequantize(), rtol=0, atol=0)
    # per-block fields are disjoint views of their seal's one allocation: the
    # counted bytes are every stored byte, once, apart from the alignment
    # (each field starts on a 16-byte boundary: at most 15 bytes per field)
    ranges.sort()
    assert all(a[1] <= b[0] for a, b in zip(ranges, ranges[1:]))
    assert all(0 <= held - counted <= 15 * 10 for held, counted in storages.values())
    assert cache.nbytes == expected_bytes + cache.sink_nbytes + cache.residual_nbytes


def test_positions_layers_reset_and_unsupported_operations():
    # test_cache.py:110-134
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    x = _randn(1, 2, 7, 8, seed=8)
    pos = torch.arange(7, device="cuda")
    cache.update(x, x, 0, {"cache_position": pos})
    cache.update(x, x, 1, {"cache_position": pos})
    assert len(cache) == 2 and cache.seen_tokens == 7
    assert cache.get_seq_length(5) == 0
    assert cache.get_mask_sizes(torch.arange(7, 9, device="cuda"), 1) == (9, 0)
    with pytest.raises(ValueError):
        cache.update(x, x, 0, {"cache_position": pos})
    assert cache.get_seq_length() == 7
    with pytest.raises(NotImplementedError):
        cache.update(x.expand(2, -1, -1, -1), x.expand(2, -1, -1, -1), 0)
    with pytest.raises(NotImplementedError):
        cache.reorder_cache(torch.tensor([0]))
    with pytest.raises(NotImplementedError):
        cache.crop(3)
    with pytest.raises(ValueError):
        cache.update(x[:, :, :, :7], x[:, :, :, :7], 2)
    assert len(cache) == 2
    cache.release()
    assert cache.nbytes == 0 and cache.get_seq_length() == 0 and len(cache) == 0


def test_controlled_position_validation_opt_out_keeps_shape_checks():
    # test_cache.py:136-148
    from inquant.cache import CacheConfig, InQuantCache
    cache = InQuantCache(CacheConfig(validate_positions=False))
    x = _randn(1, 2, 3, 8, seed=9)
    with patch("inquant.cache.torch.equal", side_effect=AssertionError("Unexpected value synchronization")):
        cache.update(x, x, 0, {"cache_position": torch.arange(3, device="cuda")})
        cache.append_for_attention(x[:, :, :1], x[:, :, :1], 0, {"cache_position": torch.tensor([3], device="cuda")})
    assert cache.get_seq_length() == 4
    for bad in (torch.tensor([[4]]), torch.tensor([4, 5]), torch.tensor([4.0]), [4]):
        with pytest.raises(ValueError):
            cache.append_for_attention(x[:, :, :1], x[:, :, :1], 0, {"cache_position": bad})
        assert cache.get_seq_length() == 4
    with pytest.raises(ValueError):
        CacheConfig(validate_positions="false")


def test_over_32k_cache_shape_and_persistent_bytes():
    # test_cache.py:150-158
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    cache = InQuantCache(CacheConfig(CodecConfig(salient_fraction=0), block_size=256, residual_length=128,
                                     sink_tokens=4))
    x = _randn(1, 2, 32768, 8, seed=10, dtype=torch.bfloat16)
    cache.update(x, x, 0)
    tail = _randn(1, 2, 3, 8, seed=11, dtype=torch.bfloat16)
    out, _ = cache.update(tail, tail, 0)
    assert tuple(out.shape) == (1, 2, 32771, 8)
    assert cache.get_seq_length() == 32771
    assert cache.nbytes < cache.bf16_nbytes * 0.8
    assert cache.metadata_nbytes > 0


def test_k4v2_append_semantics_and_owned_bytes_across_seal_boundary():
    # test_value_codec.py:52-76: the append view (sink, sealed blocks, tail)
    # equals what update() returns, token by token across seals, with the
    # same owned bytes and peak
    from inquant.cache import CacheConfig, InQuantCache
    from inquant.codec import CodecConfig
    cfg = CacheConfig(CodecConfig(donor_policy="min_error"), block_size=8, residual_length=3, sink_tokens=2,
                      value_bits=2, track_peak_bytes=True)
    a, b = InQuantCache(cfg), InQuantCache(cfg)
    k, v = _randn(1, 2, 51, 128, seed=12), _randn(1, 2, 51, 128, seed=13)
    for cache in (a, b):
        cache.update(k[:, :, :27], v[:, :, :27], 0)
    expected_peak = a.nbytes
    for step in range(27, 51):
        expected = a.update(k[:, :, step:step + 1], v[:, :, step:step + 1], 0)
        view = b.append_for_attention(k[:, :, step:step + 1], v[:, :, step:step + 1], 0)
        for wanted, sink, blocks, tail in zip(expected, (view.sink_key, view.sink_value),
                                              (view.key_blocks, view.value_blocks),
                                              (view.residual_key, view.residual_value)):
            actual = torch.cat([sink] + [block.dequantize() for block in blocks] + [tail], dim=2)
            torch.testing.assert_close(actual, wanted, rtol=0, atol=0)
        assert a.nbytes == b.nbytes
        expected_peak = max(expected_peak, a.nbytes)
        assert a.peak_nbytes == b.peak_nbytes == expected_peak
    stats = a.memory_stats()
    assert stats["nbytes"] == sum(stats[key] for key in ("payload_nbytes", "metadata_nbytes", "sink_nbytes",
                                                         "residual_nbytes", "auxiliary_nbytes"))


@pytest.mark.parametrize("value_bits", [None, 2])
def test_seal_nonfinite_raises_the_encoders_error_and_leaves_the_layer(value_bits):
    # codec.py:197 and value_codec.py:64 raise before anything is stored; the
    # cache reads both encoders' flags with one sync, the key error first
    from inquant.cache import InQuantCache
    cfg = _cfg(value_bits=value_bits, value_group_size=32) if value_bits else _cfg()
    cache = InQuantCache(cfg)
    key, value = _randn(1, 2, 5, 64, seed=30), _randn(1, 2, 5, 64, seed=31)
    cache.update(key, value, 0)
    before = (cache.get_seq_length(), len(cache._layers[0].key_blocks), cache.nbytes)
    v_msg = "FP16 quantization parameters" if value_bits else "finite values"
    for bad_k, bad_v, msg in ((True, False, "finite values"), (False, True, v_msg), (True, True, "finite values")):
        k, v = _randn(1, 2, 16, 64, seed=32), _randn(1, 2, 16, 64, seed=33)
        if bad_k:
            k[0, 1, 3, 7] = float("nan")
        if bad_v:
            v[0, 0, 9, 40] = float("inf")
        with pytest.raises(ValueError, match=msg):
            cache.update(k, v, 0)
        assert (cache.get_seq_length(), len(cache._layers[0].key_blocks), cache.nbytes) == before
    # a clean append after the failures seals normally
    cache.update(_randn(1, 2, 16, 64, seed=34), _randn(1, 2, 16, 64, seed=35), 0)
    assert len(cache._layers[0].key_blocks) == 2 and cache.get_seq_length() == 21


def test_single_token_position_check():
    # test_cache.py:110-134: a wrong one-token position raises and changes nothing
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    x = _randn(1, 2, 6, 8, seed=36)
    cache.update(x, x, 0, {"cache_position": torch.arange(6, device="cuda")})
    t = x[:, :, :1]
    for wrong in (5, 7, 0):
        for dtype in (torch.int64, torch.int32):
            with pytest.raises(ValueError, match="contiguous append positions"):
                cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([wrong], dtype=dtype, device="cuda")})
    assert cache.get_seq_length() == 6
    cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([6], dtype=torch.int32, device="cuda")})
    assert cache.get_seq_length() == 7


@pytest.mark.parametrize("value_bits", [None, 2])
def test_sealing_append_checks_its_position_in_the_seal_sync(value_bits):
    # An append that seals reads the position flag together with the
    # encoders' flags (one synchronization, position first): a wrong position
    # raises the reference's error and leaves every layer unchanged; the right
    # one seals, and a second layer given the same verified tensor seals too.
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg(value_bits=value_bits, value_group_size=32))
    k, v = _randn(1, 2, 21, 64, seed=60), _randn(1, 2, 21, 64, seed=61)
    for layer in (0, 1):
        cache.update(k[:, :, :12], v[:, :, :12], layer, {"cache_position": torch.arange(12, device="cuda")})
    before = (cache.get_seq_length(0), len(cache._layers[0].key_blocks), cache.nbytes,
              cache._layers[0].tail.count, cache._layers[0].tail.start)
    assert before[1] == 0 and before[3] == 10          # the next append fills the tail: 3 + 8 rows
    t, u = k[:, :, 12:13], v[:, :, 12:13]
    for wrong in (11, 13):
        with pytest.raises(ValueError, match="contiguous append positions"):
            cache.append_for_attention(t, u, 0, {"cache_position": torch.tensor([wrong], device="cuda")})
        assert (cache.get_seq_length(0), len(cache._layers[0].key_blocks), cache.nbytes,
                cache._layers[0].tail.count, cache._layers[0].tail.start) == before
        assert cache._position_checked is None and not any(cache._flags.tolist())
    p = torch.tensor([12], device="cuda")
    views = [cache.append_for_attention(t, u, layer, {"cache_position": p}) for layer in (0, 1)]
    assert cache._position_checked[0] is p and cache._position_checked[2] == 12
    for layer, view in enumerate(views):
        assert len(cache._layers[layer].key_blocks) == 1 and cache.get_seq_length(layer) == 13
        assert len(view.key_blocks) == 0                   # attended from the next step on
        assert torch.equal(view.residual_key, k[:, :, 2:13]) and torch.equal(view.residual_value, v[:, :, 2:13])
    # the next append, which does not seal, carves the next seal's outputs
    # (reported apart from nbytes); the seal after it encodes into them
    layer = cache._layers[0]
    assert layer.seal_out is None and cache.memory_stats()["seal_reserve_nbytes"] == 0
    nbytes = cache.nbytes
    cache.append_for_attention(k[:, :, 13:14], v[:, :, 13:14], 0, {"cache_position": torch.tensor([13], device="cuda")})
    carved = [t.data_ptr() for t in layer.seal_out]
    assert cache.memory_stats()["seal_reserve_nbytes"] == layer.seal_out[0].untyped_storage().nbytes() > 0
    assert cache.nbytes == nbytes + 2 * 2 * 64 * k.element_size()       # one more tail row only
    for pos in range(14, 21):
        cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                   {"cache_position": torch.tensor([pos], device="cuda")})
    assert len(layer.key_blocks) == 2 and cache.get_seq_length(0) == 21
    fields = list(layer.key_blocks[1].tensors.values()) + list(layer.value_blocks[1].tensors.values())
    assert [t.data_ptr() for t in fields] == carved
    # both sealed blocks equal the ones update() seals from the same tokens
    ref = InQuantCache(_cfg(value_bits=value_bits, value_group_size=32))
    ref.update(k[:, :, :21], v[:, :, :21], 0)
    assert len(ref._layers[0].key_blocks) == 2
    for i in range(2):
        for a, b in ((layer.key_blocks[i], ref._layers[0].key_blocks[i]),
                     (layer.value_blocks[i], ref._layers[0].value_blocks[i])):
            for name, x in a.tensors.items():
                assert torch.equal(x, b.tensors[name]), (i, name)
    assert sum(b.nbytes for b in layer.key_blocks + layer.value_blocks) == \
        sum(b.nbytes for b in ref._layers[0].key_blocks + ref._layers[0].value_blocks)


@pytest.mark.parametrize("inference", [False, True])
def test_shared_cache_position_checked_on_the_device(inference):
    # The layers of one step share one cache_position tensor.  The first
    # layer's append synchronizes and raises on a mismatch before anything
    # changes; the other layers rely on the append kernel's comparison while
    # the tensor is unchanged.  An in-place change between layers moves the
    # tensor's version counter, so that layer checks again and raises before
    # anything changes (cache.py:233-238 raises on every layer).  An
    # inference tensor has no version counter: its change is reported at the
    # next synchronizing check (the next step's first layer).
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    x = _randn(1, 2, 6, 8, seed=37)
    for layer in (0, 1):
        cache.update(x, x, layer, {"cache_position": torch.arange(6, device="cuda")})
    cache.update(x[:, :, :5], x[:, :, :5], 2, {"cache_position": torch.arange(5, device="cuda")})
    t = x[:, :, :1]
    with torch.inference_mode(inference):
        p = torch.tensor([6], device="cuda")
        for layer in (0, 1):
            cache.append_for_attention(t, t, layer, {"cache_position": p})
        assert cache._position_checked[0] is p and cache._position_checked[2] == 6
        with pytest.raises(ValueError, match="contiguous append positions"):
            cache.append_for_attention(t, t, 2, {"cache_position": p})   # layer 2 expects 5
        assert cache.get_seq_length(2) == 5
        q = torch.tensor([7], device="cuda")
        cache.append_for_attention(t, t, 0, {"cache_position": q})
        q.fill_(3)                                   # changed in place between layers
        if not inference:
            with pytest.raises(ValueError, match="contiguous append positions"):
                cache.append_for_attention(t, t, 1, {"cache_position": q})   # raised on this layer
            assert [cache.get_seq_length(i) for i in range(3)] == [8, 7, 5]
            q.fill_(7)
            cache.append_for_attention(t, t, 1, {"cache_position": q})
            assert [cache.get_seq_length(i) for i in range(3)] == [8, 8, 5]
            cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([8], device="cuda")})
            assert cache.get_seq_length(0) == 9
            return
        cache.append_for_attention(t, t, 1, {"cache_position": q})    # compared on the device only
        assert [cache.get_seq_length(i) for i in range(3)] == [8, 8, 5]
        with pytest.raises(ValueError, match="contiguous append positions"):
            cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([8], device="cuda")})
        cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([8], device="cuda")})
        assert cache.get_seq_length(0) == 9


def test_tail_rows_move_once_after_a_seal():
    # one-token appends write rows in place; after a seal the tail's first
    # rows are the survivors, moved by the next append; every append view
    # equals the exact tokens (sink 2, residual 3, blocks of 8)
    from inquant.cache import InQuantCache
    cache = InQuantCache(_cfg())
    k, v = _randn(1, 2, 40, 8, seed=38), _randn(1, 2, 40, 8, seed=39)
    cache.update(k[:, :, :5], v[:, :, :5], 0)
    seen = []
    for pos in range(5, 40):
        view = cache.append_for_attention(k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], 0,
                                          {"cache_position": torch.tensor([pos], device="cuda")})
        sealed = len(view.key_blocks)
        first = 2 + 8 * sealed
        assert torch.equal(view.residual_key, k[:, :, first:pos + 1])
        assert torch.equal(view.residual_value, v[:, :, first:pos + 1])
        seen.append(cache._layers[0].tail.start)
    assert 8 in seen and seen[-1] in (0, 8)
    assert len(cache._layers[0].key_blocks) == (40 - 2 - 3) // 8
