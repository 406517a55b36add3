"""Known answers for the value codec's code rounding (value_codec.py:59-67).

The reference computes codes as ``round((x - f32(offset)) / f32(scale))``:
an IEEE fp32 division followed by torch's round-half-to-even, then a clamp.
Each case below fixes one group's offset and scale exactly (its minimum is
``lo`` and its maximum ``hi``, with ``(hi - lo) / levels`` an fp16 number), so
the quotient of the probe value ``x`` is the documented ``quotient`` and the
expected code follows from the rounding rule alone:

* exact half-integer quotients go to the even code;
* the fp32 cases are quotients one ulp from k + 1/2 for which the product
  with the rounded reciprocal, ``(x - off) * fl(1 / scale)``, lands on the
  other side of (or exactly on) k + 1/2, so a reciprocal-multiply encoder
  gets them wrong;
* the bf16 cases are quotients within 2^-16 of k + 1/2 (inputs a GPU encoder
  must resolve with the exact division).

The probe values were found by a search over fp16 scales; the expected codes
are written out by hand from the quotients, not computed by any encoder.
"""
from __future__ import annotations

import numpy as np

# (bits, dtype, lo, hi, [(x, quotient, code), ...])
CASES = [
    # exact ties, scale 1: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    (2, "bfloat16", 0.0, 3.0, [(0.5, 0.5, 0), (1.5, 1.5, 2), (2.5, 2.5, 2), (1.0, 1.0, 1)]),
    # exact ties, scale 1/2
    (2, "bfloat16", 0.0, 1.5, [(0.25, 0.5, 0), (0.75, 1.5, 2), (1.25, 2.5, 2)]),
    # one ulp below 1.5; the reciprocal product is exactly 1.5 (-> 2)
    (2, "float32", 0.0, 3.9755859375, [(1.9877928495407104, 1.4999998807907104, 1)]),
    # one ulp above 0.5; the reciprocal product is exactly 0.5 (-> 0)
    (2, "float32", 0.0, 4.8544921875, [(0.8090820908546448, 0.5000000596046448, 1)]),
    # exactly 1.5 by division; the reciprocal product is one ulp below (-> 1)
    (2, "float32", 0.0, 9.041015625, [(4.5205078125, 1.5, 2)]),
    (2, "float32", 0.0, 3.38671875, [(1.6933592557907104, 1.4999998807907104, 1)]),
    # bf16 inputs whose quotients lie within 2^-16 of a half-integer
    (2, "bfloat16", 0.0162353515625, 146.0, [(73.0, 1.4999874830245972, 1)]),
    (2, "bfloat16", 0.2490234375, 1184.0, [(592.0, 1.5000025033950806, 2)]),
    (2, "bfloat16", 0.0019378662109375, 9.625, [(4.8125, 1.500004768371582, 2)]),
    (2, "bfloat16", 0.0029449462890625, 4.625, [(0.7734375, 0.4999901056289673, 0)]),
    # 4-bit codes: ties to even, and reciprocal-product disagreements
    (4, "bfloat16", 0.0, 15.0, [(0.5, 0.5, 0), (1.5, 1.5, 2), (2.5, 2.5, 2), (13.5, 13.5, 14),
                                (14.5, 14.5, 14)]),
    (4, "float32", 0.0, 52.44140625, [(15.732422828674316, 4.500000476837158, 5)]),
    (4, "float32", 0.0, 29.8828125, [(10.957030296325684, 5.499999523162842, 5)]),
    (4, "float32", 0.0, 49.833984375, [(1.6611329317092896, 0.5000000596046448, 1)]),
]

GROUP = 64
D = 128


def build(bits: int, dtype: str):
    """Rows of [1, 1, T, 128] (one case per 64-channel group) and the expected codes.

    Channel 0 of a group holds lo, channel 1 hi, channels 2.. the probe
    values; the rest hold lo (code 0).  Returns (x fp32, codes uint8 [T, 128]).
    """
    groups = [c for c in CASES if c[0] == bits and (dtype == "float32" or c[1] == dtype)]
    rows = (len(groups) + 1) // 2
    x = np.zeros((rows * 2, GROUP), np.float32)
    codes = np.zeros((rows * 2, GROUP), np.uint8)
    levels = (1 << bits) - 1
    for i, (_, _, lo, hi, probes) in enumerate(groups):
        x[i, :] = lo
        x[i, 1] = hi
        codes[i, 1] = levels
        for j, (value, _, code) in enumerate(probes):
            x[i, 2 + j] = value
            codes[i, 2 + j] = code
    if len(groups) % 2:
        x[-1, :] = 0.0
        x[-1, 1] = float(levels)       # scale 1, every other code 0
        codes[-1, 1] = levels
    return x.reshape(1, 1, rows, D), codes.reshape(rows, D)


def quotients_hold() -> None:
    """Every documented quotient is the IEEE fp32 quotient of its case."""
    for bits, _, lo, hi, probes in CASES:
        levels = np.float32((1 << bits) - 1)
        off = np.float32(np.float16(np.float32(lo)))
        scale = np.float32(np.float16(max(np.float32(np.float32(hi) - np.float32(lo)) / levels,
                                          np.float32(2.0 ** -14))))
        assert off == np.float32(lo)
        for value, quotient, _ in probes:
            q = np.float32(np.float32(np.float32(value) - off) / scale)
            assert q == np.float32(quotient), (bits, lo, hi, value, q, quotient)


def unpack_codes(payload: np.ndarray, bits: int) -> np.ndarray:
    """Codes of a [..., D * bits / 8] payload, LSB first (value_codec.py:68-71)."""
    per = 8 // bits
    shifts = (np.arange(per) * bits).astype(np.uint8)
    out = (payload[..., None] >> shifts) & np.uint8((1 << bits) - 1)
    return out.reshape(*payload.shape[:-1], payload.shape[-1] * per)
