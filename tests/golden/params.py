"""Seeded parameters and inputs shared by the golden-fixture generator and the tests that read the fixtures.

Every floating parameter of a module is overwritten, in sorted name order, from one torch.Generator: matrices get
N(0, 1/fan_in), norm weights 1 + N(0, 0.1^2), the carrier's log decay scale A -3 + N(0, 0.1^2) (a few percent of
decay per token, the regime the carrier trains in; with A near 0 every output would be dominated by its last one or
two tokens), every other vector N(0, 0.1^2), independent of the module's own
initialisation, so the reference's modules and this build's (same parameter names and shapes) receive identical
values, and gates, decays and norms all differ from their defaults. Values are rounded to fp32 (the precision the modules train
in), so a run in either dtype starts from identical numbers."""
from __future__ import annotations

import math

import torch


def fill_(module: torch.nn.Module, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters(), key=lambda kv: kv[0]):
            r = torch.randn(p.shape, generator=g, dtype=torch.float64)
            if p.dim() >= 2:
                v = r / math.sqrt(p.shape[-1])
            elif name.endswith("weight"):   # LayerNorm / RMSNorm scales
                v = 1.0 + 0.1 * r
            elif name == "A" or name.endswith(".A"):   # AssocCarrier's per-head log decay scale
                v = -3.0 + 0.1 * r
            else:
                v = 0.1 * r
            p.copy_(v.float().to(p.dtype))


def inputs(seed: int, *shapes, scale: float = 1.0) -> list[torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(s, generator=g, dtype=torch.float64) * scale).float() for s in shapes]


def ids(seed: int, shape, vocab: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, shape, generator=g)


# the configurations the fixtures cover (small; every option at its benchmarked default)
ASSOC = dict(d=128, heads=2, B=2, T=96, p0=77)
SPIN = dict(d=96, B=2, T=45)
LMCFG = dict(vocab=64, d=128, layers=2, mlp_mult=1, ctx=32, B=2, T=80, window=32)
