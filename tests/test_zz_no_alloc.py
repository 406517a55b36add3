"""iq_decode_attention_noalloc (the decode with its partials in a static
device array) against iq_decode_attention with a caller workspace, through
the C ABI: two calls in a row, the second with a smaller input, each equal
to the workspace entry point's output and within 2e-3 of the fp64 oracle."""
import numpy as np
import pytest
import torch

from kvcase import make_case

pytestmark = pytest.mark.gpu


def _call(entry, case, state, out, workspace=None):
    from inquant import _native as nat
    q = case.query
    n = len(case.key_blocks)
    fmt = state._format
    sk, sv, tk, tv = case.sink_k, case.sink_v, case.tail_k, case.tail_v
    args = [q.data_ptr(), nat.dtype_code(q.dtype), q.stride(1), q.shape[1],
            state._tables.data_ptr() if n else None, state._key_map.data_ptr() if n else None, None,
            state._desc.run if n and state._desc.run.blocks else None, n,
            fmt.tokens if n else 256, sk.shape[1], fmt.salient if n else 0, 2, 64,
            sk.data_ptr(), sv.data_ptr(), sk.stride(1), sk.stride(2), sv.stride(1), sv.stride(2), sk.shape[2],
            tk.data_ptr(), tv.data_ptr(), tk.stride(1), tk.stride(2), tv.stride(1), tv.stride(2), tk.shape[2],
            128 ** -0.5]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel()]
    args += [out.data_ptr(), nat.dtype_code(out.dtype), nat.stream_handle(q.device)]
    return entry(*args)


def test_noalloc_decode_equals_workspace_decode_twice_then_smaller():
    from inquant import _native as nat
    from inquant.triton_attention import PackedDecodeState
    lib = nat.lib()
    for seed, blocks, tail in ((61, 24, 128), (62, 3, 17)):      # the second call is smaller
        print(f"noalloc decode: seed {seed}, {blocks} blocks, tail {tail}", flush=True)
        case = make_case(seed, n_blocks=blocks, tail=tail)
        state = PackedDecodeState(case.key_blocks, case.value_blocks)
        need = lib.iq_decode_workspace_floats(case.query.shape[1], blocks, 4, tail)
        workspace = torch.empty(need, dtype=torch.float32, device="cuda")
        ref = torch.empty(case.query.shape, dtype=torch.float32, device="cuda")
        got = torch.full(case.query.shape, float("nan"), dtype=torch.float32, device="cuda")
        nat.check(_call(lib.iq_decode_attention, case, state, ref, workspace))
        nat.check(_call(lib.iq_decode_attention_noalloc, case, state, got))
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        exp = case.expected()
        assert np.abs(got.cpu().numpy()[0, :, 0] - exp).max() <= 2e-3
