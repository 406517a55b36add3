"""Write golden vectors for K4 `quantize` from the reference CPU implementation.

Only `codec.quantize` is imported from the reference: the float bits of its
torch reductions (sampled saliency and mean, `var_mean`, codec.py:205-209)
decide rankings and the stored padding, and nothing but the reference itself
pins them.  Everything else in the path is pinned by closed forms, the
reference tests' known answers and invariants (see tests/test_oracle.py).

Run in the build container only (the reference is not on the GPU box):
    python tests/golden/make_golden.py /root/reference/src
Outputs tests/golden/k4_quantize.npz and tests/golden/k4_quantize.json.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from recipes import K4_CASES, build_input  # noqa: E402

PAYLOAD_INLINE_LIMIT = 65536


def main(reference_src: str) -> None:
    sys.path.insert(0, reference_src)
    import torch
    from inquant.codec import CodecConfig, quantize  # reference implementation

    torch.set_num_threads(8)
    arrays: dict[str, np.ndarray] = {}
    meta: dict[str, dict] = {}
    for name, (recipe, cfg) in K4_CASES.items():
        x = build_input(recipe)
        dtype = {"bfloat16": torch.bfloat16, "float16": torch.float16}.get(recipe.get("dtype"), torch.float32)
        xt = torch.from_numpy(x).to(dtype)
        assert torch.equal(xt.to(torch.float32), torch.from_numpy(x)), name
        packed = quantize(xt, CodecConfig(**cfg))
        entry = {"recipe": recipe, "config": cfg, "shape": list(x.shape),
                 "input_sha256": __import__("hashlib").sha256(x.tobytes()).hexdigest(),
                 "descriptor_dtype": str(packed.salient_channels.dtype).replace("torch.", "")}
        payload = packed.payload.numpy()
        entry["payload_sha256"] = __import__("hashlib").sha256(payload.tobytes()).hexdigest()
        if payload.nbytes <= PAYLOAD_INLINE_LIMIT:
            arrays[f"{name}/payload"] = payload
        arrays[f"{name}/scales"] = packed.scales.numpy()
        arrays[f"{name}/salient_channels"] = packed.salient_channels.to(torch.int64).numpy()
        arrays[f"{name}/donor_channels"] = packed.donor_channels.to(torch.int64).numpy()
        arrays[f"{name}/padding"] = packed.padding.numpy()
        meta[name] = entry
        print(name, tuple(x.shape), entry["payload_sha256"][:12])
    np.savez_compressed(os.path.join(HERE, "k4_quantize.npz"), **arrays)
    with open(os.path.join(HERE, "k4_quantize.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "torch": torch.__version__,
                   "cases": meta}, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
