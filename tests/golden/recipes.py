"""Input recipes shared by the golden-vector generator and the parity tests.

A recipe names how to rebuild a codec input from tests/synth.py, so the
committed fixtures hold seeds, small arrays and SHA-256 digests only.
"""
from __future__ import annotations

import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import synth  # noqa: E402


def build_input(recipe: dict) -> np.ndarray:
    """Return fp32 [B, H, T, D] holding exact values of recipe['dtype']."""
    kind = recipe["kind"]
    if kind == "kv_like":
        x = synth.kv_like(recipe["seed"], recipe["heads"], recipe["tokens"], recipe.get("D", 128),
                          tuple(recipe.get("groups", (2, 2, 1))), recipe.get("scale", 20.0),
                          recipe.get("dtype", "bfloat16"))
    elif kind == "normal":
        x = synth.normal(recipe["seed"], tuple(recipe["shape"])) * np.float32(recipe.get("mult", 1.0))
        for lo, hi, factor in recipe.get("boost", []):
            x[..., lo:hi] *= np.float32(factor)
        x = _round(x, recipe.get("dtype", "float32"))
    elif kind == "zeros":
        x = np.zeros(tuple(recipe["shape"]), np.float32)
    elif kind == "ties":
        # small integers -> many exactly equal saliencies and errors
        raw = synth.splitmix64(recipe["seed"], int(np.prod(recipe["shape"])))
        x = ((raw % np.uint64(5)).astype(np.float32) - 2.0).reshape(tuple(recipe["shape"]))
        for lo, hi, factor in recipe.get("boost", []):
            x[..., lo:hi] *= np.float32(factor)
    elif kind == "sampled_positions":
        # only rows 0, s, 2s, ... may influence the ranking (test_codec.py:101-106)
        x = np.ones((1, 1, 16, 8), np.float32)
        x[..., 1::2, 0] = 1000
        x[..., ::8, 6] = 10
    else:
        raise ValueError(kind)
    block = recipe.get("block")
    if block:
        _, heads, tokens, D = x.shape
        n = tokens // block
        x = np.ascontiguousarray(x[0, :, :n * block].reshape(heads, n, block, D).transpose(1, 0, 2, 3))
    return np.ascontiguousarray(x, np.float32)


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return synth.bf16_round(x)
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    return x.astype(np.float32)


# name -> (recipe, codec config)
K4_CASES = {
    "cfg0_s16_neighbors": ({"kind": "kv_like", "seed": 100, "heads": 4, "tokens": 4096},
                           {"sample_stride": 16, "salient_fraction": 0.125, "donor_policy": "neighbors"}),
    "cfg0_s16_min_error": ({"kind": "kv_like", "seed": 100, "heads": 4, "tokens": 4096},
                           {"sample_stride": 16, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "cfg0_blocks_neighbors": ({"kind": "kv_like", "seed": 100, "heads": 4, "tokens": 4096, "block": 256},
                              {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "neighbors"}),
    "cfg0_blocks_min_error": ({"kind": "kv_like", "seed": 100, "heads": 4, "tokens": 4096, "block": 256},
                              {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "cfg3_blocks_min_error": ({"kind": "kv_like", "seed": 300, "heads": 8, "tokens": 1024,
                               "groups": [3, 3, 3, 1], "block": 256},
                              {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "cfg3_blocks_neighbors": ({"kind": "kv_like", "seed": 300, "heads": 8, "tokens": 1024,
                               "groups": [3, 3, 3, 1], "block": 256},
                              {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "neighbors"}),
    "run_fp16_neighbors": ({"kind": "normal", "seed": 29, "shape": [2, 3, 41, 16], "mult": 0.1,
                            "boost": [[6, 10, 100.0]], "dtype": "float16"},
                           {"sample_stride": 8, "salient_fraction": 0.25, "donor_policy": "neighbors"}),
    "run_fp32_min_error": ({"kind": "normal", "seed": 29, "shape": [2, 3, 41, 16], "mult": 0.1,
                            "boost": [[6, 10, 100.0]]},
                           {"sample_stride": 8, "salient_fraction": 0.25, "donor_policy": "min_error"}),
    "stride3_fp32": ({"kind": "normal", "seed": 55, "shape": [1, 3, 55, 16], "boost": [[2, 5, 20.0]]},
                     {"sample_stride": 3, "salient_fraction": 0.25, "donor_policy": "neighbors"}),
    "stride7_t300": ({"kind": "normal", "seed": 7, "shape": [1, 2, 300, 32], "dtype": "bfloat16"},
                     {"sample_stride": 7, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "long_t4100": ({"kind": "normal", "seed": 41, "shape": [1, 1, 4100, 16], "boost": [[0, 3, 9.0]]},
                   {"sample_stride": 1, "salient_fraction": 0.25, "donor_policy": "min_error"}),
    "t1_bf16": ({"kind": "normal", "seed": 1, "shape": [1, 2, 1, 128], "dtype": "bfloat16"},
                {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "d258_half": ({"kind": "normal", "seed": 258, "shape": [1, 1, 3, 258]},
                  {"sample_stride": 8, "salient_fraction": 0.5, "donor_policy": "neighbors"}),
    "d2_half": ({"kind": "normal", "seed": 2, "shape": [1, 1, 3, 2]},
                {"sample_stride": 8, "salient_fraction": 0.5, "donor_policy": "neighbors"}),
    "d128_half_min_error": ({"kind": "normal", "seed": 64, "shape": [2, 2, 64, 128], "dtype": "bfloat16"},
                            {"sample_stride": 8, "salient_fraction": 0.5, "donor_policy": "min_error"}),
    "zeros_frac0": ({"kind": "zeros", "shape": [1, 2, 17, 16]},
                    {"sample_stride": 8, "salient_fraction": 0.0, "donor_policy": "neighbors"}),
    "zeros_half": ({"kind": "zeros", "shape": [1, 2, 17, 16]},
                   {"sample_stride": 8, "salient_fraction": 0.5, "donor_policy": "min_error"}),
    "ties_neighbors": ({"kind": "ties", "seed": 112, "shape": [3, 4, 32, 128], "boost": [[30, 70, 3.0]]},
                       {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "neighbors"}),
    "ties_min_error": ({"kind": "ties", "seed": 112, "shape": [3, 4, 32, 128], "boost": [[30, 70, 3.0]]},
                       {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "min_error"}),
    "ties_quarter_min_error": ({"kind": "ties", "seed": 113, "shape": [2, 2, 64, 128]},
                               {"sample_stride": 4, "salient_fraction": 0.25, "donor_policy": "min_error"}),
    "sampled_positions": ({"kind": "sampled_positions"},
                          {"sample_stride": 8, "salient_fraction": 0.125, "donor_policy": "neighbors"}),
}
