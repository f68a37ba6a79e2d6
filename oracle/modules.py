"""Functional CPU restatements of the modules around the carrier hot path, driven by a state_dict.
TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Parameter names are the reference modules' (`src/assoc.py:323-348`, `src/spin.py:69-94`, `src/model.py:629-702`),
so a state_dict of the product modules in `pragnosia_amd` loads here unchanged. Everything runs in the dtype of the
parameters passed in (fp64 for the truth).

Pinning: these are compositions of the pinned scans in `oracle.aspin` / `oracle.diag` with torch built-ins
(LayerNorm, Linear, RMSNorm, GELU, softplus, sigmoid). The compositions are pinned against the reference's own
modules by the golden fixtures in tests/golden/modules.npz (the reference's CPU AssocCarrier plain and delta,
SpinCarrier(rf), LM forward and forward_carried with the aspin and fspin mixers, fp32, seeded parameters; checked in
tests/test_golden_modules.py to 1e-4), and by invariants in tests/test_oracle_modules.py: causality, carried windows
== one pass (across a position restart through the rebase), token-at-a-time decode == one pass, forward_carried's
last window == the same window after a carried prefix. `greedy_decode` is pinned against `lm_forward_carried` at
every step across window boundaries and the position wrap. `short_conv`: identity initialisation == no convolution,
carried cache == one pass, and a single tap equals the input shifted by that many tokens.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import aspin as A_
from . import diag as D_


def _lin(x, sd, name):
    return F.linear(x, sd[name + ".weight"], sd.get(name + ".bias"))


def _ln(x, sd, name, eps=1e-5):
    return F.layer_norm(x, (x.shape[-1],), sd[name + ".weight"], sd[name + ".bias"], eps)


def _rms(x, weight, eps=torch.finfo(torch.float32).eps):
    """The carrier's per-head `nn.RMSNorm(dk)` (`src/assoc.py:347`). Its eps=None means finfo(input dtype).eps, and
    the reference model runs it on fp32 activations, so the restatement uses fp32's eps (1.19e-7) whatever dtype it
    computes in: with fp64's eps a head output row whose mean square is below 1e-7 would be normalised differently
    from the reference."""
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


def short_conv(sconv, qo, ko, vo, cc):
    """The carrier's causal depthwise convolution on q, k, v (B, T, d each) over the last K tokens
    (`src/assoc.py:374-382`): weight sconv (3 d, K), the current token on the last tap; cc the previous call's last
    K - 1 inputs (B, 3 d, K - 1) or None (zeros) at a sequence start. Returns q, k, v and the new cache."""
    D, K = qo.shape[-1], sconv.shape[1]
    x = torch.cat([qo, ko, vo], dim=-1).transpose(1, 2)
    pad = cc.to(x.dtype) if cc is not None else x.new_zeros(x.shape[0], 3 * D, K - 1)
    xp = torch.cat([pad, x], dim=-1)
    y = F.conv1d(xp, sconv.to(x.dtype).unsqueeze(1), groups=3 * D).transpose(1, 2)
    return y[..., :D], y[..., D:2 * D], y[..., 2 * D:], xp[..., -(K - 1):]


def assoc_carrier(sd, x, h0=None, pos0=0, *, heads, delta=False, write_all=False, key_topk=0, la_floor=None,
                  chunk=64, pos_wrap=None, beta_scale=None):
    """AssocCarrier.forward, torch path (`src/assoc.py:384-512`, kernel=False, no fused projections), with the short
    convolution when sd holds "sconv". h0 = (S, p0), (S, p0, cache) with the convolution, or None. Returns
    (out, (S, T)) or (out, (S, T, cache))."""
    B, T, D = x.shape
    H = heads
    dk = D // H
    z = _ln(x, sd, "ln")
    S0, p0 = (None, pos0) if h0 is None else (h0[0], h0[1])
    cc = h0[2] if (h0 is not None and len(h0) == 3) else None
    theta = sd["theta"]
    if S0 is not None and float(p0) != 0.0:
        S0 = A_.rebase(S0.to(x.dtype), theta.to(x.dtype), float(p0))
    pos = torch.arange(T)
    if pos_wrap:
        pos = pos % pos_wrap
    qo, ko, vo = _lin(z, sd, "q"), _lin(z, sd, "k"), _lin(z, sd, "v")
    if "sconv" in sd:
        qo, ko, vo, cc = short_conv(sd["sconv"], qo, ko, vo, cc)
    kp = ko.reshape(B, T, H, dk)
    if key_topk:
        keep = torch.zeros_like(kp).scatter_(-1, kp.abs().topk(key_topk, dim=-1).indices, 1.0)
        kp = kp * keep
    qp = qo.reshape(B, T, H, dk)
    vp = vo.reshape(B, T, H, dk)
    gate = None if (delta or write_all) else _lin(z, sd, "wi")
    q, k, v = A_.prep(qp, kp, vp, gate, theta, pos)
    la = A_.logalpha(_lin(z, sd, "wa"), sd["A"], la_floor).transpose(1, 2)
    beta = None
    if delta:
        beta = torch.sigmoid(_lin(z, sd, "wb")).transpose(1, 2)
        if beta_scale is not None:  # a diagnostic multiplier on the write strength, (B, H, T) (`src/assoc.py:469-472`)
            beta = beta * beta_scale.to(beta.dtype)
        if write_all:
            beta = beta.clamp(min=0.75)
    o, S = A_.assoc_scan(q, k, v, la, S0, chunk=chunk, beta=beta)
    o = _rms(o.to(x.dtype), sd["on.weight"]).transpose(1, 2).reshape(B, T, D)
    out = x + F.linear(o, sd["o.weight"] * torch.sigmoid(sd["gate"]))
    return out, ((S, T, cc) if "sconv" in sd else (S, T))


def spin_rf(sd, x, h0=None, gate_c=8.0, nu_min=1e-3):
    """SpinCarrier(gated="rf").forward (`src/spin.py:229-246`, `lam` at `:98-103`), through the chunked scan.
    Returns (out, (Re h_T, Im h_T))."""
    z = _ln(x, sd, "ln")
    nu = nu_min + F.softplus(sd["nu_raw"])
    logmag = -gate_c * torch.sigmoid(_lin(z, sd, "Wr")) * nu
    gam = torch.sqrt((1.0 - torch.exp(2.0 * logmag)).clamp_min(1e-6))
    u = _lin(z, sd, "B") * gam * torch.sigmoid(_lin(z, sd, "Wi"))
    y, h = D_.scan_gated(u, logmag, sd["theta"].expand_as(logmag), h0)
    return x + torch.sigmoid(sd["gate"]) * _lin(y.to(x.dtype), sd, "C"), h


# the carrier mixers of `src/model.py:632-660`: (delta rule, options); the head count is the caller's `heads`
# `src/model.py:632-660`: the rule and options of each carrier mixer (its head count is the caller's `heads`: wspin
# and xspin four, w2spin two)
ASSOC_MIXERS = {"aspin": (False, {}), "dspin": (True, {}), "hspin": (False, {}), "hspin1": (False, {"write_all": True}),
                "hdspin": (True, {}), "sdspin": (True, {"key_topk": 8}), "aspin1": (True, {"write_all": True}),
                "wspin": (False, {}), "w2spin": (False, {}), "xspin": (True, {})}


def _mixer(sd, prefix, mixer, heads, x, st):
    sub = {k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}
    if mixer in ASSOC_MIXERS:
        delta, opts = ASSOC_MIXERS[mixer]
        return assoc_carrier(sub, x, st, heads=heads, delta=delta, **opts)
    if mixer == "fspin":
        return spin_rf(sub, x, st)
    raise ValueError(mixer)


def _mlp(sd, prefix, x):
    h = _ln(x, sd, prefix + "n")
    return x + _lin(F.gelu(_lin(h, sd, prefix + "a")), sd, prefix + "b")


def lm_forward(sd, ids, *, layers, mixer, heads):
    """LM.forward (`src/model.py:820-840`): token + position (mod the table), per layer mixer then MLP, final LN,
    tied head."""
    ctx = sd["p.weight"].shape[0]
    T = ids.shape[1]
    h = F.embedding(ids, sd["e.weight"]) + F.embedding(torch.arange(T) % ctx, sd["p.weight"])
    for i in range(layers):
        h, _ = _mixer(sd, f"mix.{i}.", mixer, heads, h, None)
        h = _mlp(sd, f"mlp.{i}.", h)
    return F.linear(_ln(h, sd, "n"), sd["e.weight"])


def lm_forward_carried(sd, ids, window, *, layers, mixer, heads):
    """LM.forward_carried (`src/model.py:842-864`): windows of `window` tokens, positions restarting per window,
    every layer's state carried; returns the final window's logits."""
    states = [None] * layers
    logits = None
    for s in range(0, ids.shape[1], window):
        xw = ids[:, s:s + window]
        h = F.embedding(xw, sd["e.weight"]) + F.embedding(torch.arange(xw.shape[1]), sd["p.weight"])
        for i in range(layers):
            h, states[i] = _mixer(sd, f"mix.{i}.", mixer, heads, h, states[i])
            h = _mlp(sd, f"mlp.{i}.", h)
        logits = F.linear(_ln(h, sd, "n"), sd["e.weight"])
    return logits


def greedy_decode(sd, prompt, n, *, layers, mixer, heads, forced=None):
    """Greedy incremental generation (`src/bench.py:192-239`): the prompt is read in ctx-sized windows with the
    state carried, then each new token is one T=1 step through every layer; the position index is (prefill +
    i) mod ctx and each carrier rebases its state by the previous call's length. prompt (B, P) ids.
    `forced` (B, n) replaces the argmax by the given tokens (teacher forcing), so a device run can be compared step
    by step without a near-tie in the argmax sending the two runs down different continuations.
    Returns (tokens (B, n), logits of every step (B, n, V))."""
    ctx = sd["p.weight"].shape[0]
    states = [None] * layers
    lg = None
    pw = 0
    for s in range(0, prompt.shape[1], ctx):
        x = prompt[:, s:s + ctx]
        h = F.embedding(x, sd["e.weight"]) + F.embedding(torch.arange(x.shape[1]), sd["p.weight"])
        for i in range(layers):
            h, states[i] = _mixer(sd, f"mix.{i}.", mixer, heads, h, states[i])
            h = _mlp(sd, f"mlp.{i}.", h)
        lg = F.linear(_ln(h[:, -1:], sd, "n"), sd["e.weight"])[:, -1]
        pw = x.shape[1] % ctx
    toks, lgs = [], []
    for step in range(n):
        nxt = lg.argmax(-1) if forced is None else forced[:, step]
        toks.append(nxt)
        lgs.append(lg)
        h = F.embedding(nxt[:, None], sd["e.weight"]) + F.embedding(torch.tensor([pw]), sd["p.weight"])
        for i in range(layers):
            h, states[i] = _mixer(sd, f"mix.{i}.", mixer, heads, h, states[i])
            h = _mlp(sd, f"mlp.{i}.", h)
        lg = F.linear(_ln(h, sd, "n"), sd["e.weight"])[:, -1]
        pw = (pw + 1) % ctx
    return torch.stack(toks, 1), torch.stack(lgs, 1)
