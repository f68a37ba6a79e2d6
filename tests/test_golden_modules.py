"""The oracle's module compositions against the reference's own modules: tests/golden/modules.npz holds the outputs
of the reference's CPU AssocCarrier (plain, delta), SpinCarrier(rf) and LM (aspin, fspin; forward and
forward_carried) on seeded parameters and inputs (tests/golden/params.py; written by tests/golden/make_golden.py).

The reference computed them in fp32, its training precision; the oracle runs in fp64 from the same fp32
parameters and inputs, so the two differ by the reference's fp32 rounding only. A wrong composition (a norm, gate,
rotation or rebase in the wrong place) moves the outputs by O(1) relative. Tolerance: max |a - b| / max |b| <= 1e-4."""
import os

import numpy as np
import pytest
import torch

from oracle import modules as M

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "modules.npz"))
TOL = 1e-4


def rel(a, b):
    a = torch.as_tensor(np.asarray(a, dtype=np.float64)) if not torch.is_tensor(a) else a.detach().double()
    b = torch.as_tensor(np.asarray(b, dtype=np.float64))
    return ((a - b).abs().max() / b.abs().max()).item()


def _params():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import params as P
    return P


def _sd(mod):
    return {k: v.detach().double() for k, v in mod.state_dict().items()}


@pytest.mark.parametrize("delta", [False, True])
def test_assoc_carrier_matches_reference(delta):
    P = _params()
    from pragnosia_amd.assoc import AssocCarrier
    a = P.ASSOC
    m = AssocCarrier(a["d"], heads=a["heads"], delta=delta)
    P.fill_(m, 10 + delta)
    x, S0 = P.inputs(20 + delta, (a["B"], a["T"], a["d"]), (a["B"], a["heads"], 64, 64))
    S0 = S0 * 0.2
    y, (S, p) = M.assoc_carrier(_sd(m), x.double(), (S0.double(), a["p0"]), heads=a["heads"], delta=delta)
    tag = "assoc_delta" if delta else "assoc_plain"
    assert p == a["T"]
    assert rel(y - x.double(), G[tag + "_y"] - x.numpy()) < TOL
    assert rel(S, G[tag + "_S"]) < TOL


def test_spin_rf_matches_reference():
    P = _params()
    from pragnosia_amd.spin import SpinCarrier
    s = P.SPIN
    m = SpinCarrier(s["d"], gated="rf")
    P.fill_(m, 30)
    x, hr, hi = P.inputs(31, (s["B"], s["T"], s["d"]), (s["B"], s["d"]), (s["B"], s["d"]))
    y, (hr2, hi2) = M.spin_rf(_sd(m), x.double(), (hr.double(), hi.double()))
    assert rel(y - x.double(), G["spin_y"] - x.numpy()) < TOL
    assert rel(hr2, G["spin_hr"]) < TOL and rel(hi2, G["spin_hi"]) < TOL


@pytest.mark.parametrize("mixer", ["aspin", "fspin"])
def test_lm_matches_reference(mixer):
    P = _params()
    from pragnosia_amd.model import LM
    c = P.LMCFG
    lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer=mixer)
    P.fill_(lm, 40 + len(mixer))
    ids = P.ids(41, (c["B"], c["T"]), c["vocab"])
    heads = c["d"] // 64 if mixer == "aspin" else None
    sd = _sd(lm)
    logits = M.lm_forward(sd, ids[:, : c["ctx"]], layers=c["layers"], mixer=mixer, heads=heads)
    carried = M.lm_forward_carried(sd, ids, c["window"], layers=c["layers"], mixer=mixer, heads=heads)
    assert rel(logits, G[f"lm_{mixer}_logits"]) < TOL
    assert rel(carried, G[f"lm_{mixer}_carried"]) < TOL


OPT = np.load(os.path.join(HERE, "golden", "options.npz"))


def option_case(name, build):
    """(module built by `build(ctor kwargs)` and filled, x, S0, gy, beta_scale, la_floor, pos_wrap) for an option
    case of tests/golden/options.npz."""
    P = _params()
    c = P.OPTIONS[name]
    m = build(c)
    P.fill_(m, P.option_seed(name))
    x, S0, gy, bs = P.option_inputs(name)
    return m, c, x, S0, gy, bs, P.option_la_floor(name), c.get("attrs", {}).get("pos_wrap")


@pytest.mark.parametrize("name", list(_params().OPTIONS))
def test_assoc_options_match_reference(name):
    """The carrier's options (key_topk, hl_floor, write_all, pos_wrap, beta_scale, head dim 128, and the sparse wide
    delta carrier) against the reference's own module: output, final state, and the input gradient under a seeded
    upstream gradient (the reference's fp32 autograd), the oracle in fp64 autograd."""
    from pragnosia_amd.assoc import AssocCarrier
    m, c, x, S0, gy, bs, floor, wrap = option_case(
        name, lambda c: AssocCarrier(c["d"], heads=c["heads"], delta=c["delta"], **c["ctor"]))
    xd = x.double().requires_grad_(True)
    y, (S, p) = M.assoc_carrier(_sd(m), xd, (S0.double(), _params().OPT["p0"]), heads=c["heads"], delta=c["delta"],
                                write_all=c["ctor"].get("write_all", False), key_topk=c["ctor"].get("key_topk", 0),
                                la_floor=floor, pos_wrap=wrap, beta_scale=None if bs is None else bs.double())
    (y * gy.double()).sum().backward()
    assert p == _params().OPT["T"]
    assert rel(y - xd, OPT[name + "_y"] - x.numpy()) < TOL
    assert rel(S, OPT[name + "_S"]) < TOL
    assert rel(xd.grad - gy.double(), OPT[name + "_dx"] - gy.numpy()) < TOL


def test_option_fixtures_exercise_their_branches():
    """Each option changes the reference's output (so its fixture pins the branch, not the default path): the oracle
    with the option switched off misses the fixture by far more than the tolerance."""
    from pragnosia_amd.assoc import AssocCarrier
    for name in ("topk", "hlfloor", "writeall", "poswrap", "delta_betascale", "delta_writeall"):
        m, c, x, S0, gy, bs, floor, wrap = option_case(
            name, lambda c: AssocCarrier(c["d"], heads=c["heads"], delta=c["delta"], **c["ctor"]))
        y, _ = M.assoc_carrier(_sd(m), x.double(), (S0.double(), _params().OPT["p0"]), heads=c["heads"],
                               delta=c["delta"])
        assert rel(y - x.double(), OPT[name + "_y"] - x.numpy()) > 100 * TOL, name


def test_lm_dspin_matches_reference():
    """The delta-rule LM (mixer "dspin"): forward and forward_carried logits."""
    P = _params()
    from pragnosia_amd.model import LM
    c = P.LMCFG
    lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer="dspin")
    P.fill_(lm, 45)
    ids = P.ids(41, (c["B"], c["T"]), c["vocab"])
    sd = _sd(lm)
    logits = M.lm_forward(sd, ids[:, : c["ctx"]], layers=c["layers"], mixer="dspin", heads=c["d"] // 64)
    carried = M.lm_forward_carried(sd, ids, c["window"], layers=c["layers"], mixer="dspin", heads=c["d"] // 64)
    assert rel(logits, OPT["lm_dspin_logits"]) < TOL
    assert rel(carried, OPT["lm_dspin_carried"]) < TOL
