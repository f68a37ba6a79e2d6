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

# AssocCarrier options (`src/assoc.py:280-282`, `:355-359`, `:406-410`, `:435-439`, `:469-479`), each on the
# reference's torch path with a carried state at position offset p0; "attrs" are attributes set after
# construction (pos_wrap, and beta_scale, a (B, H, T) tensor drawn U(0, 1) from seed 60 + index).
OPT = dict(B=1, T=96, p0=77)
OPTIONS = {
    "topk": dict(d=128, heads=2, delta=False, ctor=dict(key_topk=8)),
    "delta_topk": dict(d=128, heads=2, delta=True, ctor=dict(key_topk=8)),
    "hlfloor": dict(d=256, heads=4, delta=False, ctor=dict(hl_floor=True)),
    "delta_hlfloor": dict(d=256, heads=4, delta=True, ctor=dict(hl_floor=True)),
    "writeall": dict(d=128, heads=2, delta=False, ctor=dict(write_all=True)),
    "delta_writeall": dict(d=128, heads=2, delta=True, ctor=dict(write_all=True)),
    "poswrap": dict(d=128, heads=2, delta=False, ctor={}, attrs=dict(pos_wrap=40)),
    "delta_poswrap": dict(d=128, heads=2, delta=True, ctor={}, attrs=dict(pos_wrap=40)),
    "delta_betascale": dict(d=128, heads=2, delta=True, ctor={}, attrs=dict(beta_scale=True)),
    "wide": dict(d=128, heads=1, delta=False, ctor={}),
    "delta_wide": dict(d=128, heads=1, delta=True, ctor={}),
    "delta_wide_topk": dict(d=128, heads=1, delta=True, ctor=dict(key_topk=8)),
}


def option_inputs(name: str):
    """x (B, T, d), S0 (B, H, dk, dk) (scaled by 0.2), the upstream gradient on the output (B, T, d), and beta_scale
    (B, H, T) or None, for option case `name`; the module's parameters come from fill_(module, 50 + index)."""
    c = OPTIONS[name]
    n = list(OPTIONS).index(name)
    dk = c["d"] // c["heads"]
    x, S0, gy = inputs(70 + n, (OPT["B"], OPT["T"], c["d"]), (OPT["B"], c["heads"], dk, dk),
                       (OPT["B"], OPT["T"], c["d"]))
    bs = None
    if c.get("attrs", {}).get("beta_scale"):
        g = torch.Generator().manual_seed(60 + n)
        bs = torch.rand(OPT["B"], c["heads"], OPT["T"], generator=g, dtype=torch.float64).float()
    return x, S0 * 0.2, gy, bs


def option_seed(name: str) -> int:
    return 50 + list(OPTIONS).index(name)


def option_la_floor(name: str):
    """The hl_floor buffer (`src/assoc.py:340-344`): per-head floors -ln 2 / hl, hl geometric from 8 to 131072."""
    c = OPTIONS[name]
    if not c["ctor"].get("hl_floor"):
        return None
    hl = torch.logspace(math.log10(8.0), math.log10(131072.0), c["heads"], dtype=torch.float64)
    return -math.log(2.0) / hl
