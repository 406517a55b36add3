"""Deterministic synthetic KV inputs, identical on every machine.

Integer-only generator (splitmix64 -> Irwin-Hall sum of 12 uniforms - 6 ->
float32 -> bf16 round-to-nearest-even), so golden fixtures store seeds and
digests instead of megabytes of inputs.  Test infrastructure only.
"""
from __future__ import annotations

import hashlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN
        z = state
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, shape) -> np.ndarray:
    """Approximately N(0, 1) float32 values (exactly reproducible)."""
    n = int(np.prod(shape))
    acc = np.zeros(n, np.float64)
    raw = splitmix64(seed, 12 * n).reshape(12, n) if n else np.zeros((12, 0), np.uint64)
    for i in range(12):
        acc += (raw[i] >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
    return (acc - 6.0).astype(np.float32).reshape(shape)


def bf16_round(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def outlier_channels(seed: int, heads: int, D: int, groups: list[int], touch_last: bool = True) -> list[list[int]]:
    """Per-head outlier channel lists made of runs of the given widths."""
    out = []
    for h in range(heads):
        rng = splitmix64(seed * 7919 + h, 64)
        chans: set[int] = set()
        k = 0
        for width in groups:
            while True:
                start = int(rng[k % 64] % np.uint64(D - width + 1))
                k += 1
                if h == 0 and touch_last and width == groups[0] and not chans:
                    start = D - width  # one head reaches the last channel
                run = set(range(start, start + width))
                halo = set(range(start - 1, start + width + 1))
                if not (halo & chans):
                    chans |= run
                    break
        out.append(sorted(chans))
    return out


def kv_like(seed: int, heads: int, tokens: int, D: int = 128, groups=(2, 2, 1), scale: float = 20.0,
            dtype: str = "bfloat16") -> np.ndarray:
    """[1, heads, tokens, D] N(0,1) with outlier channel runs scaled by `scale`."""
    x = np.empty((1, heads, tokens, D), np.float32)
    chans = outlier_channels(seed, heads, D, list(groups))
    for h in range(heads):
        xh = normal(seed * 1000003 + h, (tokens, D))
        xh[:, chans[h]] *= np.float32(scale)
        x[0, h] = xh
    if dtype == "bfloat16":
        x = bf16_round(x)
    elif dtype == "float16":
        x = x.astype(np.float16).astype(np.float32)
    return x


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
