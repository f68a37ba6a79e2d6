"""The forget-gated diagonal carrier (fspin): SpinCarrier(d, gated="rf") on the HIP complex diagonal scan.

Constructor arguments and parameter names are the reference's (`src/spin.py:59-103`), so a reference state_dict
loads unchanged. Only the gated="rf" path (per-token recurrence gate, time-varying, `src/spin.py:229-246`) is on this
build's hot path; the time-invariant FFT carrier (gated=None or "io") is outside it and raises."""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from ._lib import PragnosiaError
from .ops import layer_norm, linear
from .scan import scan_hip


class SpinCarrier(nn.Module):
    NU_MIN = 1e-3

    def __init__(self, d: int, chunk: int = 128, nu_min: float = 1e-3, nu_max: float = 0.3,
                 gated: str | None = None):
        super().__init__()
        if gated not in (None, "io", "rf"):
            raise ValueError(f"SpinCarrier: gated={gated!r}")
        self.d, self.chunk, self.gated = d, chunk, gated
        # timescales through softplus so |lambda| < 1; frequencies spread over [0, pi]
        self.nu_raw = nn.Parameter(torch.linspace(math.log(math.expm1(nu_min)), math.log(math.expm1(nu_max)), d))
        self.theta = nn.Parameter(torch.linspace(0.0, math.pi, d))
        self.B = nn.Linear(d, d, bias=False)
        self.C = nn.Linear(d, d, bias=False)
        self.ln = nn.LayerNorm(d)
        self.gate = nn.Parameter(torch.zeros(()))
        if gated == "io":
            self.Wi = nn.Linear(d, d)
            self.Wo = nn.Linear(d, d)
        elif gated == "rf":
            self.Wi = nn.Linear(d, d)
            self.Wr = nn.Linear(d, d)
            self.gate_c = 8.0

    def lam(self):
        """(|lambda|, angle) per channel: |lambda| = exp(-(NU_MIN + softplus(nu_raw)))."""
        nu = self.NU_MIN + torch.nn.functional.softplus(self.nu_raw)
        return torch.exp(-nu), self.theta

    def spectral_parameters(self):
        return [self.nu_raw, self.theta, self.gate]

    def forward(self, x, h0=None):
        """x (B, T, d); h0 = (Re h, Im h) of shape (B, d) or None. Returns (x + sigmoid(gate) C(Re h),
        (Re h_T, Im h_T))."""
        if self.gated != "rf":
            raise PragnosiaError("SpinCarrier: only gated='rf' (the per-token recurrence gate) runs on this build's "
                                 "kernels; the FFT carrier is outside it")
        if not x.is_cuda:
            raise PragnosiaError("SpinCarrier runs on a ROCm GPU only; there is no CPU path")
        z = layer_norm(x, self.ln)  # self.ln(x), in the dtype the projections compute in
        mag, ang = self.lam()
        # per-token log-magnitude <= 0: the recurrence gate scales the channel's timescale
        logmag = -self.gate_c * torch.sigmoid(linear(z, self.Wr)) * (-torch.log(mag))
        # per-token input normalisation sqrt(1 - |lambda_t|^2), its argument clamped to bound the derivative
        gam = torch.sqrt((1.0 - torch.exp(2.0 * logmag)).clamp_min(1e-6))
        u = self.B(z) * gam * torch.sigmoid(linear(z, self.Wi))
        y, h = scan_hip(u, logmag, ang.expand_as(logmag), h0)
        return x + torch.sigmoid(self.gate) * self.C(y), h

    def forward_windows(self, x, window: int, h0=None):
        """Consecutive windows of `window` tokens with the state carried from each into the next: nothing in this
        carrier depends on positions, so that is one continuous scan over the whole sequence. Returns the same as
        `forward`."""
        return self.forward(x, h0)
