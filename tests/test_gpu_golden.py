"""The HIP modules against the reference's own modules: the fixtures of tests/golden/modules.npz (reference CPU
modules in fp32 on their torch path, kernel=False; seeded parameters and inputs; see tests/test_golden_modules.py,
which pins the oracle to the same fixtures at 1e-4). Tolerances: the aspin kernel paths compute the scans on bf16
operands, max relative error <= 2e-2 on outputs and carried states (the north star's bound); the aspin torch path
(kernel=False: the exact fp32 scan) and the fspin paths are fp32 end to end, <= 1e-4."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "modules.npz"))


def rel(a, b):
    a = a.detach().double().cpu()
    b = torch.as_tensor(np.asarray(b, dtype=np.float64))
    return ((a - b).abs().max() / b.abs().max()).item()


def _params():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import params as P
    return P


@pytest.mark.parametrize("kernel,tol", [(True, 2e-2), (False, 1e-4)])
@pytest.mark.parametrize("delta", [False, True])
def test_assoc_carrier_matches_reference(delta, kernel, tol):
    P = _params()
    from pragnosia_amd.assoc import AssocCarrier
    a = P.ASSOC
    m = AssocCarrier(a["d"], heads=a["heads"], delta=delta, kernel=kernel)
    P.fill_(m, 10 + delta)
    m = m.cuda()
    x, S0 = P.inputs(20 + delta, (a["B"], a["T"], a["d"]), (a["B"], a["heads"], 64, 64))
    S0 = S0 * 0.2
    with torch.no_grad():
        y, (S, p) = m(x.cuda(), (S0.cuda(), a["p0"]))
    tag = "assoc_delta" if delta else "assoc_plain"
    assert p == a["T"]
    assert rel(y - x.cuda(), G[tag + "_y"] - x.numpy()) < tol
    assert rel(S, G[tag + "_S"]) < tol


def test_spin_rf_matches_reference():
    P = _params()
    from pragnosia_amd.spin import SpinCarrier
    s = P.SPIN
    m = SpinCarrier(s["d"], gated="rf")
    P.fill_(m, 30)
    m = m.cuda()
    x, hr, hi = P.inputs(31, (s["B"], s["T"], s["d"]), (s["B"], s["d"]), (s["B"], s["d"]))
    with torch.no_grad():
        y, (hr2, hi2) = m(x.cuda(), (hr.cuda(), hi.cuda()))
    assert rel(y - x.cuda(), G["spin_y"] - x.numpy()) < 1e-4
    assert rel(hr2, G["spin_hr"]) < 1e-4 and rel(hi2, G["spin_hi"]) < 1e-4


@pytest.mark.parametrize("mixer,kernel,tol", [("aspin", True, 2e-2), ("aspin", False, 1e-4), ("fspin", True, 1e-4)])
def test_lm_matches_reference(mixer, kernel, tol):
    P = _params()
    from pragnosia_amd.model import LM
    c = P.LMCFG
    lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer=mixer)
    for mod in lm.modules():
        if hasattr(mod, "kernel"):
            mod.kernel = kernel
    P.fill_(lm, 40 + len(mixer))
    lm = lm.cuda().eval()
    ids = P.ids(41, (c["B"], c["T"]), c["vocab"]).cuda()
    with torch.no_grad():
        logits = lm(ids[:, : c["ctx"]])
        carried = lm.forward_carried(ids, window=c["window"])
    assert rel(logits, G[f"lm_{mixer}_logits"]) < tol
    assert rel(carried, G[f"lm_{mixer}_carried"]) < tol


OPT = np.load(os.path.join(HERE, "golden", "options.npz"))


@pytest.mark.parametrize("kernel", [True, False])
@pytest.mark.parametrize("name", list(_params().OPTIONS))
def test_assoc_options_match_reference(name, kernel):
    """The carrier's options against the reference's own module (tests/golden/options.npz; the oracle is held to the
    same fixtures at 1e-4 in tests/test_golden_modules.py): output, final state and the input gradient under a seeded
    upstream gradient. Kernel path (bf16 scan operands): 2e-2 on outputs and states, 5e-2 on the gradient; exact
    path (kernel=False, fp32 scan): 1e-4."""
    P = _params()
    from pragnosia_amd.assoc import AssocCarrier
    c = P.OPTIONS[name]
    m = AssocCarrier(c["d"], heads=c["heads"], delta=c["delta"], kernel=kernel, **c["ctor"])
    P.fill_(m, P.option_seed(name))
    m = m.cuda()
    x, S0, gy, bs = P.option_inputs(name)
    if "pos_wrap" in c.get("attrs", {}):
        m.pos_wrap = c["attrs"]["pos_wrap"]
    if bs is not None:
        m.beta_scale = bs.cuda()
    xc = x.cuda().requires_grad_(True)
    y, (S, p) = m(xc, (S0.cuda(), P.OPT["p0"]))
    (y * gy.cuda()).sum().backward()
    tol, gtol = (2e-2, 5e-2) if kernel else (1e-4, 1e-4)
    assert p == P.OPT["T"]
    assert rel(y - xc, OPT[name + "_y"] - x.numpy()) < tol
    assert rel(S, OPT[name + "_S"]) < tol
    assert rel(xc.grad - gy.cuda(), OPT[name + "_dx"] - gy.numpy()) < gtol


@pytest.mark.parametrize("kernel,tol", [(True, 2e-2), (False, 1e-4)])
def test_lm_dspin_matches_reference(kernel, tol):
    """The delta-rule LM (mixer "dspin"): forward and forward_carried logits against the reference's."""
    P = _params()
    from pragnosia_amd.model import LM
    c = P.LMCFG
    lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer="dspin")
    for mod in lm.modules():
        if hasattr(mod, "kernel"):
            mod.kernel = kernel
    P.fill_(lm, 45)
    lm = lm.cuda().eval()
    ids = P.ids(41, (c["B"], c["T"]), c["vocab"]).cuda()
    with torch.no_grad():
        logits = lm(ids[:, : c["ctx"]])
        carried = lm.forward_carried(ids, window=c["window"])
    assert rel(logits, OPT["lm_dspin_logits"]) < tol
    assert rel(carried, OPT["lm_dspin_carried"]) < tol
