"""Pins the CPU oracle for the complex diagonal scan (oracle/diag.py).

Mirrors `tests/test_spin.py:184-223` of the reference and adds a library routine (FFT convolution for a
time-invariant lambda), the cumulative sum special case, and autograd for the hand-derived adjoint."""
import math

import pytest
import torch

from oracle import diag as O



@pytest.fixture(autouse=True)
def _fp64_default():
    """The oracle is pinned in fp64; the default dtype is restored after each test so other modules are unaffected."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(B=2, T=45, D=6, seed=5):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, T, D, generator=g)
    lm = -torch.rand(B, T, D, generator=g) * 8.0
    lm[:, :, 0] = -1e-3                                  # a slow channel
    an = torch.randn(B, T, D, generator=g)
    h0 = (torch.randn(B, D, generator=g), torch.randn(B, D, generator=g))
    return u, lm, an, h0


def test_recurrence_special_cases():
    g = torch.Generator().manual_seed(0)
    u = torch.randn(2, 17, 4, generator=g)
    zero = torch.zeros_like(u)
    y, (hr, hi) = O.recurrence(u, zero, zero)
    assert torch.allclose(y, u.cumsum(1), atol=1e-12)
    assert hi.abs().max() == 0
    # pure rotation by pi/2 per step on a single impulse: h_t = i^t
    imp = torch.zeros(1, 8, 1)
    imp[0, 0, 0] = 1.0
    y, (hr, hi) = O.recurrence(imp, torch.zeros_like(imp), torch.full_like(imp, math.pi / 2))
    expect = torch.tensor([1.0, 0, -1, 0, 1, 0, -1, 0])
    assert torch.allclose(y[0, :, 0], expect, atol=1e-12)
    assert abs(hi.item() - (-1.0)) < 1e-12                 # i^7 = -i


def test_recurrence_time_invariant_equals_fft_convolution():
    """Constant lambda: Re h_t = sum_s Re(lambda^(t-s)) u_s, a causal convolution evaluated with torch.fft."""
    g = torch.Generator().manual_seed(1)
    B, T, D = 2, 64, 5
    u = torch.randn(B, T, D, generator=g)
    mag = torch.rand(D, generator=g) * 0.5 + 0.45
    th = torch.rand(D, generator=g) * 3
    lm = torch.log(mag).expand(B, T, D)
    an = th.expand(B, T, D)
    y, (hr, hi) = O.recurrence(u, lm, an)
    t = torch.arange(T, dtype=torch.float64)[:, None]
    kr = mag ** t * torch.cos(t * th)
    n = 2 * T
    yf = torch.fft.irfft(torch.fft.rfft(u, n=n, dim=1) * torch.fft.rfft(kr, n=n, dim=0), n=n, dim=1)[:, :T]
    assert torch.allclose(y, yf, atol=1e-10)
    ki = (mag ** t * torch.sin(t * th)).flip(0)
    assert torch.allclose(hi, (u * ki).sum(1), atol=1e-10)


@pytest.mark.parametrize("chunk", [1, 8, 16, 45])
def test_scan_gated_matches_recurrence(chunk):
    u, lm, an, h0 = _inputs()
    yr, (rr, ri) = O.recurrence(u, lm, an, h0)
    yg, (gr, gi) = O.scan_gated(u, lm, an, h0, chunk=chunk)
    assert torch.allclose(yg, yr, atol=1e-12)
    assert torch.allclose(gr, rr, atol=1e-12) and torch.allclose(gi, ri, atol=1e-12)
    y0, _ = O.scan_gated(u, lm, an, None, chunk=chunk)
    yr0, _ = O.recurrence(u, lm, an, None)
    assert torch.allclose(y0, yr0, atol=1e-12)


def test_scan_gated_two_windows_carried_equal_one():
    u, lm, an, h0 = _inputs()
    yr, _ = O.recurrence(u, lm, an, h0)
    a, st = O.scan_gated(u[:, :20], lm[:, :20], an[:, :20], h0, chunk=8)
    b, _ = O.scan_gated(u[:, 20:], lm[:, 20:], an[:, 20:], st, chunk=8)
    assert torch.allclose(torch.cat([a, b], 1), yr, atol=1e-12)


def test_scan_gated_gradients_match_recurrence():
    u, lm, an, h0 = _inputs()
    w = torch.randn_like(u)
    grads = []
    for fn in (lambda *a: O.scan_gated(*a[:3], (a[3], a[4]), chunk=8), lambda *a: O.recurrence(*a[:3], (a[3], a[4]))):
        args = [t.clone().requires_grad_(True) for t in (u, lm, an, *h0)]
        y, (r, i) = fn(*args)
        ((y * w).sum() + r.sum() - 2 * i.sum()).backward()
        grads.append([a.grad for a in args])
    for x, y in zip(*grads):
        assert (x - y).abs().max() / y.abs().max() < 1e-9


@pytest.mark.parametrize("with_h0", [False, True])
def test_adjoint_matches_autograd(with_h0):
    """The hand-derived backward == autograd through the literal recurrence, for u, logmag, ang, h0 (real and
    imaginary) and with upstream gradients on y and on both parts of the final state
    (`tests/test_spin.py:237-246`)."""
    u, lm, an, h0 = _inputs(T=33, D=7, seed=11)
    h0 = h0 if with_h0 else None
    g = torch.Generator().manual_seed(12)
    gy = torch.randn(u.shape, generator=g)
    glr = torch.randn(u.shape[0], u.shape[2], generator=g)
    gli = torch.randn(u.shape[0], u.shape[2], generator=g)
    args = [t.clone().requires_grad_(True) for t in (u, lm, an)]
    hh = None if h0 is None else tuple(t.clone().requires_grad_(True) for t in h0)
    y, (r, i) = O.recurrence(*args, hh)
    ((y * gy).sum() + (r * glr).sum() + (i * gli).sum()).backward()
    hr, hi = O.forward_states(u, lm, an, h0)
    du, dlm, dan, dh0r, dh0i = O.adjoint(gy, glr, gli, lm, an, hr, hi, h0)
    for mine, ref in zip((du, dlm, dan), args):
        assert (mine - ref.grad).abs().max() / ref.grad.abs().max() < 1e-12
    if h0 is not None:
        assert (dh0r - hh[0].grad).abs().max() < 1e-12 and (dh0i - hh[1].grad).abs().max() < 1e-12


def test_forward_states_match_recurrence():
    u, lm, an, h0 = _inputs()
    hr, hi = O.forward_states(u, lm, an, h0)
    y, (rT, iT) = O.recurrence(u, lm, an, h0)
    assert torch.equal(hr, y) and torch.equal(hr[:, -1], rT) and torch.equal(hi[:, -1], iT)


def test_fp32_extreme_decay_is_finite():
    g = torch.Generator().manual_seed(0)
    u = torch.randn(2, 512, 8, generator=g, dtype=torch.float32)
    lm = -torch.rand(2, 512, 8, generator=g, dtype=torch.float32) * 30.0
    an = torch.randn(2, 512, 8, generator=g, dtype=torch.float32)
    y, _ = O.scan_gated(u, lm, an, None, chunk=16)
    assert torch.isfinite(y).all()
