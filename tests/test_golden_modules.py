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
