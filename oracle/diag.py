"""CPU restatement of the per-token-lambda complex diagonal recurrence that fspin trains through.
TEST INFRASTRUCTURE ONLY (see oracle/__init__).

    h_t = lambda_t h_{t-1} + u_t,   lambda_t = exp(logmag_t + i ang_t),   logmag_t <= 0,   u_t real,
    y_t = Re h_t;   returns (y, (Re h_{T-1}, Im h_{T-1})).

Tensors are (B, T, D); h0 is a pair of (B, D) tensors or None.

What pins each function (tests/test_oracle_diag.py):
  recurrence  -- brute force; for a time-invariant lambda it equals the convolution with lambda^t computed by
                 torch.fft (a library routine); for logmag = 0, ang = 0 it is the cumulative sum.
  scan_gated  -- == recurrence for chunks 1, 8, T, with and without h0, across carried windows; autograd
                 gradients == those of the recurrence.
  adjoint     -- == autograd through the recurrence for every input, including h0 and the final (Re, Im) state.
"""
from __future__ import annotations

import torch


def recurrence(u, logmag, ang, h0=None):
    """The literal recurrence in the input dtype (`tests/test_spin.py:194-200`, `src/scan_kernel.py:37-50`)."""
    B, T, D = u.shape
    hr = torch.zeros(B, D, dtype=u.dtype) if h0 is None else h0[0].to(u.dtype)
    hi = torch.zeros(B, D, dtype=u.dtype) if h0 is None else h0[1].to(u.dtype)
    ys = []
    for t in range(T):
        mag = torch.exp(logmag[:, t])
        lr, li = mag * torch.cos(ang[:, t]), mag * torch.sin(ang[:, t])
        hr, hi = lr * hr - li * hi + u[:, t], li * hr + lr * hi
        ys.append(hr)
    return torch.stack(ys, 1), (hr, hi)


def scan_gated(u, logmag, ang, h0=None, chunk=16):
    """The chunked closed form of `src/spin.py:181-215`, the reference's CPU path for the gated scan.

    Within a chunk, with Lr, Li the cumulative sums of logmag and ang,
        h_t = sum_{s<=t} exp(Lr_t - Lr_s) e^{i (Li_t - Li_s)} u_s + exp(Lr_t) e^{i Li_t} h_prev,
    every real exponent <= 0. Only Re h is emitted per token; Im h is formed at chunk ends for the carry."""
    B, T, D = u.shape
    rt = torch.float64 if u.dtype == torch.float64 else torch.float32
    u, logmag, ang = u.to(rt), logmag.to(rt), ang.to(rt)
    hr = torch.zeros(B, D, dtype=rt) if h0 is None else h0[0].to(rt)
    hi = torch.zeros(B, D, dtype=rt) if h0 is None else h0[1].to(rt)
    ys = []
    for t0 in range(0, T, chunk):
        uc, lc, ac = u[:, t0:t0 + chunk], logmag[:, t0:t0 + chunk], ang[:, t0:t0 + chunk]
        C = uc.shape[1]
        Lr, Li = lc.cumsum(1), ac.cumsum(1)
        dr = (Lr.unsqueeze(2) - Lr.unsqueeze(1)).clamp(max=0.0)           # (B, t, s, D)
        di = Li.unsqueeze(2) - Li.unsqueeze(1)
        causal = torch.tril(torch.ones(C, C, dtype=torch.bool)).reshape(1, C, C, 1)
        mag = torch.where(causal, torch.exp(dr), torch.zeros((), dtype=rt))
        yr = (mag * torch.cos(di) * uc.unsqueeze(1)).sum(2)
        eLr = torch.exp(Lr)
        yr = yr + eLr * (torch.cos(Li) * hr.unsqueeze(1) - torch.sin(Li) * hi.unsqueeze(1))
        hi = (mag[:, -1] * torch.sin(di[:, -1]) * uc).sum(1) \
            + eLr[:, -1] * (torch.sin(Li[:, -1]) * hr + torch.cos(Li[:, -1]) * hi)
        hr = yr[:, -1]
        ys.append(yr)
    return torch.cat(ys, 1), (hr, hi)


def forward_states(u, logmag, ang, h0=None):
    """(Re h, Im h) for every t, by the literal recurrence: what the forward kernel saves for the backward."""
    B, T, D = u.shape
    hr = torch.zeros(B, D, dtype=u.dtype) if h0 is None else h0[0].to(u.dtype)
    hi = torch.zeros(B, D, dtype=u.dtype) if h0 is None else h0[1].to(u.dtype)
    HR, HI = [], []
    for t in range(T):
        mag = torch.exp(logmag[:, t])
        lr, li = mag * torch.cos(ang[:, t]), mag * torch.sin(ang[:, t])
        hr, hi = lr * hr - li * hi + u[:, t], li * hr + lr * hi
        HR.append(hr)
        HI.append(hi)
    return torch.stack(HR, 1), torch.stack(HI, 1)


def adjoint(g, g_last_r, g_last_i, logmag, ang, hr, hi, h0=None):
    """The hand-derived backward of `src/scan_kernel.py:12-17`, `:53-99`, `:121-140`, as a reverse loop.

    With R_t the 2x2 rotation-scaling of lambda_t and a the adjoint (real, imag):
        a_{T-1} = (g_{T-1} + g_last_r, g_last_i);  a_t = (g_t, 0) + R_{t+1}^T a_{t+1}
        du_t = a_t[0];  dlogmag_t = a_t . (R_t h_{t-1});  dang_t = a_t . (R'_t h_{t-1}),
        R' = mag [[-sin, -cos], [cos, -sin]];  dh0 = R_0^T a_0.
    Returns (du, dlogmag, dang, dh0r, dh0i)."""
    B, T, D = g.shape
    dt = g.dtype
    ar = torch.zeros(B, D, dtype=dt)
    ai = torch.zeros(B, D, dtype=dt) if g_last_i is None else g_last_i.to(dt).clone()
    gg = g.clone()
    if g_last_r is not None:
        gg[:, -1] = gg[:, -1] + g_last_r.to(dt)
    du, dlm, dan = torch.empty_like(gg), torch.empty_like(gg), torch.empty_like(gg)
    zero = torch.zeros(B, D, dtype=dt)
    for t in range(T - 1, -1, -1):
        ar = ar + gg[:, t]
        if t > 0:
            pr, pi = hr[:, t - 1], hi[:, t - 1]
        elif h0 is not None:
            pr, pi = h0[0].to(dt), h0[1].to(dt)
        else:
            pr, pi = zero, zero
        mag = torch.exp(logmag[:, t])
        c, s = mag * torch.cos(ang[:, t]), mag * torch.sin(ang[:, t])
        du[:, t] = ar
        dlm[:, t] = ar * (c * pr - s * pi) + ai * (s * pr + c * pi)
        dan[:, t] = ar * (-s * pr - c * pi) + ai * (c * pr - s * pi)
        ar, ai = c * ar + s * ai, -s * ar + c * ai
    return du, dlm, dan, ar, ai
