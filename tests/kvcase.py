"""Builds packed decode cases on the GPU and their fp64 dequantize-then-attend oracle."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import oracle
import synth

NP_DTYPE_NAME = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle_dequant_k4(block, dtype_name: str) -> np.ndarray:
    fields = {k: v.detach().cpu().numpy() for k, v in block.tensors.items()}
    fields["salient_channels"] = fields["salient_channels"].astype(np.int64)
    fields["donor_channels"] = fields["donor_channels"].astype(np.int64)
    return oracle.k4_dequantize(fields, dtype_name)[0]          # [H, T, D]


def oracle_dequant_v(block, dtype_name: str) -> np.ndarray:
    if hasattr(block, "bits"):
        fields = {"payload": block.payload.cpu().numpy(), "scales": block.scales.cpu().numpy(),
                  "offsets": block.offsets.cpu().numpy()}
        return oracle.v_dequantize(fields, block.bits, block.group_size, dtype_name)[0]
    return oracle_dequant_k4(block, dtype_name)


def oracle_decode(query, key_blocks, value_blocks, sink_k=None, sink_v=None, tail_k=None, tail_v=None,
                  scale=None) -> np.ndarray:
    """fp64 attention over K/V decoded by the oracle and rounded to the query dtype."""
    name = NP_DTYPE_NAME[query.dtype]
    ks, vs = [], []
    if sink_k is not None:
        ks.append(to_np(sink_k)[0])
        vs.append(to_np(sink_v)[0])
    ks += [oracle_dequant_k4(b, name) for b in key_blocks]
    vs += [oracle_dequant_v(b, name) for b in value_blocks]
    if tail_k is not None:
        ks.append(to_np(tail_k)[0])
        vs.append(to_np(tail_v)[0])
    k = np.concatenate(ks, axis=1)
    v = np.concatenate(vs, axis=1)
    q = to_np(query)[0, :, 0]
    return oracle.attend(q, k, v, 128 ** -0.5 if scale is None else scale)


@dataclass
class DecodeCase:
    query: torch.Tensor
    key_blocks: list
    value_blocks: list
    sink_k: torch.Tensor | None
    sink_v: torch.Tensor | None
    tail_k: torch.Tensor | None
    tail_v: torch.Tensor | None

    def kwargs(self):
        return dict(sink_key=self.sink_k, sink_value=self.sink_v, residual_key=self.tail_k,
                    residual_value=self.tail_v)

    def expected(self, scale=None):
        return oracle_decode(self.query, self.key_blocks, self.value_blocks, self.sink_k, self.sink_v,
                             self.tail_k, self.tail_v, scale)


def make_case(seed: int, *, H=4, G=7, n_blocks=2, block=256, sink=4, tail=128, dtype=torch.bfloat16,
              fraction=0.125, policy="min_error", value_bits=2, group=64, groups=(2, 2, 1)) -> DecodeCase:
    from inquant.codec import CodecConfig, quantize
    from inquant.value_codec import quantize_values
    cfg = CodecConfig(salient_fraction=fraction, donor_policy=policy)
    dev = "cuda"
    kb, vb = [], []
    for i in range(n_blocks):
        k = torch.from_numpy(synth.kv_like(seed * 101 + 2 * i, H, block, groups=groups)).to(dev, dtype)
        v = torch.from_numpy(synth.kv_like(seed * 101 + 2 * i + 1, H, block, groups=groups)).to(dev, dtype)
        kb.append(quantize(k, cfg))
        vb.append(quantize_values(v, value_bits, group) if value_bits else quantize(v, cfg))

    def dense(s, t):
        if t == 0:
            return None
        return torch.from_numpy(synth.kv_like(s, H, t, groups=groups)).to(dev, dtype)

    q = torch.from_numpy(synth.normal(seed * 7 + 3, (1, H * G, 1, 128))).to(dev, dtype)
    return DecodeCase(q, kb, vb, dense(seed * 13 + 1, sink), dense(seed * 13 + 2, sink),
                      dense(seed * 13 + 3, tail), dense(seed * 13 + 4, tail))
