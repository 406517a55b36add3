"""Fused donor selector entry point (module name kept from the reference).

reuse_map(saliency, count, donor_error=None) mirrors
src/inquant/triton_selection.py:46-60 of the reference, including its argument
checks; the selection itself is the wave-level HIP kernel in
libinquant_hip.so (one 64-lane wavefront per row).  No Triton is involved.
"""
from __future__ import annotations

import torch

from . import _native as nat


def reuse_map(saliency: torch.Tensor, count: int, donor_error: torch.Tensor | None = None):
    if saliency.device.type != "cuda" or saliency.dtype != torch.float32 or saliency.shape[-1] != 128:
        raise ValueError("Fused selector requires CUDA float32 saliency with 128 channels")
    if not 0 <= count <= 64:
        raise ValueError("Expected 0..64 selected channels")
    if donor_error is not None and (donor_error.shape != saliency.shape or donor_error.dtype != saliency.dtype
                                   or donor_error.device != saliency.device):
        raise ValueError("Donor error must match saliency shape, dtype and device")
    sources = torch.empty((*saliency.shape[:-1], count), dtype=torch.int64, device=saliency.device)
    donors = torch.empty_like(sources)
    rows = saliency.numel() // 128
    if count and rows:
        sal = saliency.contiguous()
        err = None if donor_error is None else donor_error.contiguous()
        nat.check(nat.lib().iq_reuse_map(sal.data_ptr(), nat.ptr(err), rows, 128, count, sources.data_ptr(),
                                         donors.data_ptr(), nat.stream_handle(saliency.device)))
    return sources, donors
