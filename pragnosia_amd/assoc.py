"""The associative carrier (aspin / dspin) on the HIP kernels: scan entry points and the AssocCarrier module.

Module and function signatures, parameter names and the state layout follow the reference (`src/assoc.py`), so
checkpoints and callers (LM, forward_carried, the trainer, the decode loop) use this as a drop-in. Every scan runs
on the hand-written gfx950 kernels; there is no PyTorch or CPU path."""
from __future__ import annotations

import torch

from . import ops  # noqa: F401  (registers torch.ops.pragnosia.*)
from ._lib import PragnosiaError


def assoc_scan_hip(q, k, v, logalpha, S0=None, need_sent=True):
    """Plain rule, chunk 64, head dim 64: the contract of the reference's `assoc_scan_kernel`
    (`src/assoc_kernel.py:302-323`). q, k, v (B, H, T, D) any float dtype (bf16 inside), logalpha (B, H, T),
    S0 (B, H, D, D) or None. Returns (o in q's dtype, S_final fp32, sent bf16 (B, H, NC, D, D) or None)."""
    grad = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, logalpha, S0))
    want = bool(need_sent or grad)
    o, S, sent = torch.ops.pragnosia.aspin_chunk(q, k, v, logalpha.float(), None if S0 is None else S0.float(), want)
    return o.to(q.dtype), S, (sent if need_sent else None)
