"""CPU checks of the drop-in boundary: the C-ABI library loads and exports what
include/inquant_hip.h declares, and host-side validation mirrors the reference."""
import ctypes
import math
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    with open(os.path.join(ROOT, "include", "inquant_hip.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(iq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from inquant import _native
    lib = _native.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.exported_symbols())
    assert lib.iq_abi_version() == 1


def test_invalid_arguments_return_errors_without_a_gpu():
    from inquant import _native
    lib = _native.lib()
    # argument checks run on the host before any launch
    assert lib.iq_reuse_map(None, None, 4, 2000, 4, None, None, None) == -1
    assert b"D=2000" in lib.iq_last_error()
    assert lib.iq_v_dequantize(None, None, None, 1, 128, 3, 64, None, 0, None) == -1
    # 128 blocks + one 32-token sink slice + four 32-token tail slices, 130 floats each
    assert lib.iq_decode_workspace_floats(28, 128, 4, 128) == 28 * 133 * 130
    assert lib.iq_decode_partitions(128, 4, 128, 1) == 133 and lib.iq_decode_partitions(128, 4, 128, 0) == 133
    assert lib.iq_decode_merge(None, 133, 28, None, 1, None) == -1 and b"null" in lib.iq_last_error()
    assert lib.iq_decode_merge(1 << 20, 0, 28, 1 << 20, 1, None) == -1 and b"sizes" in lib.iq_last_error()
    # the allocation-free decode refuses, on the host and before touching a
    # device, inputs whose partials exceed its static scratch (4 Mi floats)
    assert lib.iq_decode_attention_noalloc(
        None, 1, 128, 28, None, None, None, None, 1, 256, 4, 16, 2, 64, None, None, 0, 0, 0, 0, 0,
        None, None, 0, 0, 0, 0, 4700 * 256, 0.088, None, 0, None) == -1
    assert b"static scratch" in lib.iq_last_error()
    # prefill: key tiles are addressed by 32-bit offsets, so token strides of
    # 2^25 elements or more are refused (the pointers are never dereferenced)
    fake = 1 << 20
    st = 1 << 25
    assert lib.iq_prefill_attention(fake, fake, fake, _native.IQ_BF16, 28 * 128, 128, st, 128, 512, 128, fake, 1,
                                    8192, 28, 4, 128, 0.088, fake, 28 * 128, 128, _native.IQ_BF16, None) == -1
    assert b"token stride" in lib.iq_last_error()


@pytest.mark.parametrize("bad", [-0.1, 0.51, float("nan")])
def test_invalid_fraction_rejected(bad):
    from inquant.codec import CodecConfig
    with pytest.raises(ValueError, match="salient_fraction"):
        CodecConfig(salient_fraction=bad)


@pytest.mark.parametrize("bad", [0, -1, 1.5, True])
def test_invalid_sample_stride_rejected(bad):
    from inquant.codec import CodecConfig
    with pytest.raises(ValueError, match="sample_stride"):
        CodecConfig(sample_stride=bad)


def test_config_rejects_unknown_policy_and_backend():
    from inquant.codec import CodecConfig
    with pytest.raises(ValueError, match="donor_policy"):
        CodecConfig(donor_policy="nearest")
    with pytest.raises(ValueError, match="donor_backend"):
        CodecConfig(donor_backend="cuda")


def test_quantize_validation_precedes_device_dispatch():
    from inquant.codec import quantize
    with pytest.raises(ValueError, match="even"):
        quantize(torch.ones(1, 1, 8, 7))
    with pytest.raises(ValueError, match="nonempty"):
        quantize(torch.ones(1, 1, 0, 8))
    with pytest.raises(ValueError, match="floating"):
        quantize(torch.ones(1, 1, 8, 8, dtype=torch.int32))


def test_cpu_tensors_are_rejected_not_served_by_a_fallback():
    from inquant.codec import quantize
    from inquant.value_codec import quantize_values
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        quantize(torch.ones(1, 1, 8, 8))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        quantize_values(torch.ones(1, 1, 8, 128))


def test_value_codec_argument_validation():
    from inquant.value_codec import quantize_values
    with pytest.raises(ValueError, match="bits"):
        quantize_values(torch.zeros(1, 1, 2, 128), bits=3)
    with pytest.raises(ValueError, match="group"):
        quantize_values(torch.zeros(1, 1, 2, 128), group_size=16)
    with pytest.raises(ValueError):
        quantize_values(torch.zeros(1, 1, 2, 48))


def test_cache_config_validation():
    from inquant.cache import CacheConfig
    with pytest.raises(ValueError, match="block_size"):
        CacheConfig(block_size=0)
    with pytest.raises(ValueError, match="integer"):
        CacheConfig(residual_length=1.5)
    with pytest.raises(ValueError, match="value_bits"):
        CacheConfig(value_bits=3)
    with pytest.raises(ValueError, match="value_group_size"):
        CacheConfig(value_group_size=16)
    with pytest.raises(ValueError, match="boolean"):
        CacheConfig(shared_workspace=1)


def test_cache_update_validation_runs_on_host():
    from inquant.cache import CacheConfig, InQuantCache
    cache = InQuantCache(CacheConfig())
    with pytest.raises(NotImplementedError):
        cache.update(torch.zeros(2, 1, 3, 8), torch.zeros(2, 1, 3, 8), 0)
    with pytest.raises(ValueError, match="even"):
        cache.update(torch.zeros(1, 1, 3, 7), torch.zeros(1, 1, 3, 7), 0)
    with pytest.raises(ValueError, match="layer_idx"):
        cache.update(torch.zeros(1, 1, 3, 8), torch.zeros(1, 1, 3, 8), -1)
    with pytest.raises(ValueError, match="cache_position"):
        cache.update(torch.zeros(1, 1, 3, 8), torch.zeros(1, 1, 3, 8), 0, {"cache_position": torch.arange(2)})
    assert cache.get_seq_length() == 0 and cache.nbytes == 0


def test_cache_positions_and_dense_rows_on_the_host():
    # Host logic only (CPU tensors, no block sealed, so no codec call): a
    # wrong position raises and changes nothing, the sink and tail rows hold
    # the exact tokens, reset() forgets the checked position
    from inquant.cache import CacheConfig, InQuantCache
    cache = InQuantCache(CacheConfig())
    x = torch.arange(6 * 8, dtype=torch.float32).view(1, 1, 6, 8)
    for layer in (0, 1):
        cache.update(x, x, layer, {"cache_position": torch.arange(6)})
    t = x[:, :, :1] + 100
    with pytest.raises(ValueError, match="contiguous append positions"):
        cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([5])})
    assert cache.get_seq_length(0) == 6
    view = cache.append_for_attention(t, t, 0, {"cache_position": torch.tensor([6])})
    assert view.seq_length == 7 and torch.equal(view.residual_key[:, :, -1:], t)
    assert torch.equal(view.sink_key, x[:, :, :4]) and torch.equal(view.residual_key[:, :, :2], x[:, :, 4:])
    assert cache.residual_nbytes == 2 * (3 + 2) * 8 * 4 and cache.sink_nbytes == 2 * 2 * 4 * 8 * 4
    cache.reset()
    assert cache._position_checked is None and cache.nbytes == 0


def test_decode_state_validation_without_gpu():
    from inquant.triton_attention import PackedDecodeState
    state = PackedDecodeState([], [])
    with pytest.raises(ValueError, match="query must have shape"):
        state.decode(torch.zeros(1, 4, 2, 128))
    with pytest.raises(ValueError, match="CUDA"):
        state.decode(torch.zeros(1, 4, 1, 128))
    with pytest.raises(ValueError, match="counts must match"):
        PackedDecodeState([1], [])
    assert math.isclose(128 ** -0.5, 0.08838834764831845)
