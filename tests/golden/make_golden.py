"""Writes tests/golden/modules.npz: outputs of the reference's own CPU modules (imported from the reference
checkout, in this container only) on seeded parameters and inputs (tests/golden/params.py).

    python tests/golden/make_golden.py [/path/to/reference]

What it pins: the composition of the modules around the scans, which no closed form pins -- AssocCarrier.forward
(plain and delta rule, torch path, with a carried state and position offset; `src/assoc.py:384-512`),
SpinCarrier(gated="rf").forward (`src/spin.py:229-246`), and LM.forward / LM.forward_carried (`src/model.py:820-864`)
with the aspin and fspin mixers. The reference runs in fp32, its training precision (its RMSNorm eps follows the
input dtype), on fp32 parameters and inputs. Only inputs' seeds and the outputs are stored."""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import params as P  # noqa: E402


def main(ref: str) -> None:
    sys.path.insert(0, ref)
    from src.assoc import AssocCarrier
    from src.model import LM
    from src.spin import SpinCarrier
    torch.manual_seed(0)
    out = {}
    a = P.ASSOC
    for delta in (False, True):
        tag = "assoc_delta" if delta else "assoc_plain"
        m = AssocCarrier(a["d"], heads=a["heads"], delta=delta, kernel=False)
        P.fill_(m, 10 + delta)
        x, S0 = P.inputs(20 + delta, (a["B"], a["T"], a["d"]), (a["B"], a["heads"], 64, 64), scale=1.0)
        S0 = S0 * 0.2
        with torch.no_grad():
            y, (S, p) = m(x, (S0, a["p0"]))
        assert p == a["T"]  # positions restart every call: the next call rebases by this length
        out[tag + "_y"], out[tag + "_S"] = y.numpy(), S.numpy()
    s = P.SPIN
    m = SpinCarrier(s["d"], gated="rf")
    P.fill_(m, 30)
    x, hr, hi = P.inputs(31, (s["B"], s["T"], s["d"]), (s["B"], s["d"]), (s["B"], s["d"]))
    with torch.no_grad():
        y, (hr2, hi2) = m(x, (hr, hi))
    out["spin_y"], out["spin_hr"], out["spin_hi"] = y.numpy(), hr2.numpy(), hi2.numpy()
    c = P.LMCFG
    for mixer in ("aspin", "fspin"):
        torch.manual_seed(0)
        lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer=mixer)
        for mod in lm.modules():
            if hasattr(mod, "kernel"):
                mod.kernel = False
        P.fill_(lm, 40 + len(mixer))
        ids = P.ids(41, (c["B"], c["T"]), c["vocab"])
        with torch.no_grad():
            logits = lm(ids[:, : c["ctx"]])
            carried = lm.forward_carried(ids, window=c["window"])
        out[f"lm_{mixer}_logits"] = logits.numpy()
        out[f"lm_{mixer}_carried"] = carried.numpy()
    out = {k: v.astype(np.float32) for k, v in out.items()}   # the reference computed them in fp32
    np.savez_compressed(os.path.join(HERE, "modules.npz"), **out)
    for k, v in out.items():
        print(k, v.shape, float(np.abs(v).max()))
    options(AssocCarrier, LM)


def options(AssocCarrier, LM) -> None:
    """tests/golden/options.npz: the carrier's options (key_topk, hl_floor, write_all, pos_wrap, beta_scale, head
    dim 128, alone or combined as the mixers combine them), each with a carried state at a position offset: the
    output, the final state and the input gradient under a seeded upstream gradient (the reference's fp32 autograd
    through its torch path); and the dspin LM's forward and forward_carried."""
    out = {}
    o = P.OPT
    for name, c in P.OPTIONS.items():
        m = AssocCarrier(c["d"], heads=c["heads"], delta=c["delta"], kernel=False, **c["ctor"])
        P.fill_(m, P.option_seed(name))
        x, S0, gy, bs = P.option_inputs(name)
        if "pos_wrap" in c.get("attrs", {}):
            m.pos_wrap = c["attrs"]["pos_wrap"]
        if bs is not None:
            m.beta_scale = bs
        x = x.clone().requires_grad_(True)
        y, (S, p) = m(x, (S0, o["p0"]))
        assert p == o["T"]
        (y * gy).sum().backward()
        out[name + "_y"], out[name + "_S"], out[name + "_dx"] = y.detach().numpy(), S.detach().numpy(), x.grad.numpy()
    c = P.LMCFG
    torch.manual_seed(0)
    lm = LM(vocab=c["vocab"], d=c["d"], layers=c["layers"], mlp_mult=c["mlp_mult"], ctx=c["ctx"], mixer="dspin")
    for mod in lm.modules():
        if hasattr(mod, "kernel"):
            mod.kernel = False
    P.fill_(lm, 45)
    ids = P.ids(41, (c["B"], c["T"]), c["vocab"])
    with torch.no_grad():
        out["lm_dspin_logits"] = lm(ids[:, : c["ctx"]]).numpy()
        out["lm_dspin_carried"] = lm.forward_carried(ids, window=c["window"]).numpy()
    out = {k: v.astype(np.float32) for k, v in out.items()}
    np.savez_compressed(os.path.join(HERE, "options.npz"), **out)
    for k, v in out.items():
        print(k, v.shape, float(np.abs(v).max()))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
