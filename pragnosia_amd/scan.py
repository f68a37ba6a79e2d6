"""The per-token-lambda complex diagonal scan that the forget-gated carrier (fspin) trains through.

`scan_hip` keeps the contract of the reference's `scan_triton` (`src/scan_kernel.py:143-148`): inputs (B, T, D),
optional h0 = (Re h0, Im h0) of shape (B, D); returns (Re h, (Re h_last, Im h_last)) in u's dtype, fp32 inside.
Forward and backward are the HIP kernels behind `torch.ops.pragnosia.diag_scan`."""
from __future__ import annotations

import torch

from . import ops  # noqa: F401  (registers torch.ops.pragnosia.*)


def scan_hip(u, logmag, ang, h0=None):
    h0r, h0i = (h0[0].float(), h0[1].float()) if h0 is not None else (None, None)
    y, hr_last, hi_last, _ = torch.ops.pragnosia.diag_scan(u.float(), logmag.float(), ang.float(), h0r, h0i)
    return y.to(u.dtype), (hr_last.to(u.dtype), hi_last.to(u.dtype))


scan_triton = scan_hip  # the reference's name for this entry point
