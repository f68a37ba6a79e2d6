"""GPU parity of the complex diagonal scan (HIP, through the C ABI via torch.ops.pragnosia) against the CPU oracle.

Tolerance (fp32 path): max relative error max|x - ref| / max|ref| <= 1e-4 on every output and gradient, with the
final (Re, Im) state compared explicitly; the reference's own bound (`tests/test_spin.py:226-248`), 1e-5, is
checked as well where it applies."""
import pytest
import torch
import torch.nn.functional as F

from oracle import diag as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _cfg(B, T, D, seed, h0=True, lm_scale=None):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, T, D, generator=g)
    if lm_scale is None:
        lm = F.logsigmoid(torch.randn(B, T, D, generator=g) + 4.0)
    else:
        lm = -torch.rand(B, T, D, generator=g) * lm_scale
    an = torch.rand(B, T, D, generator=g) - 0.5
    h = (torch.randn(B, D, generator=g), torch.randn(B, D, generator=g)) if h0 else None
    return u, lm, an, h


@pytest.fixture(scope="module")
def scan():
    from pragnosia_amd.scan import scan_hip
    return scan_hip


@pytest.mark.parametrize("B,T,D,h0", [(2, 45, 300, True), (2, 45, 300, False), (3, 1, 64, True),
                                      (1, 128, 32, True), (2, 300, 40, False), (1, 1000, 96, True)])
def test_forward_matches_oracle(scan, B, T, D, h0):
    u, lm, an, h = _cfg(B, T, D, seed=B * 1000 + T, h0=h0, lm_scale=8.0)
    yr, (rr, ri) = O.recurrence(u.double(), lm.double(), an.double(), None if h is None else (h[0].double(), h[1].double()))
    dev = [t.cuda() for t in (u, lm, an)]
    yk, (kr, ki) = scan(*dev, None if h is None else (h[0].cuda(), h[1].cuda()))
    assert rel(yk, yr) < TOL and rel(kr, rr) < TOL and rel(ki, ri) < TOL
    assert (yk.cpu().double() - yr).abs().max() < 1e-5


@pytest.mark.parametrize("B,T,D,h0", [(2, 45, 300, True), (2, 45, 300, False), (1, 1, 40, True),
                                      (2, 257, 64, True)])
def test_backward_matches_oracle(scan, B, T, D, h0):
    """Gradients of u, logmag, ang, h0 (real and imaginary), with upstream gradients on y and on both parts of the
    final state, against autograd through the fp64 literal recurrence."""
    u, lm, an, h = _cfg(B, T, D, seed=7 + T, h0=h0, lm_scale=8.0)
    g = torch.Generator().manual_seed(99)
    w, wl, wi = torch.randn(B, T, D, generator=g), torch.randn(B, D, generator=g), torch.randn(B, D, generator=g)

    def loss(fn, args, hh):
        y, (r, i) = fn(*args, hh)
        return (y * w.to(y)).sum() + (r * wl.to(r)).sum() + (i * wi.to(i)).sum()

    a64 = [t.double().requires_grad_(True) for t in (u, lm, an)]
    h64 = None if h is None else tuple(t.double().requires_grad_(True) for t in h)
    loss(O.recurrence, a64, h64).backward()
    a32 = [t.cuda().requires_grad_(True) for t in (u, lm, an)]
    h32 = None if h is None else tuple(t.cuda().requires_grad_(True) for t in h)
    loss(scan, a32, h32).backward()
    for mine, ref in zip(a32, a64):
        assert rel(mine.grad, ref.grad) < TOL
    if h is not None:
        assert rel(h32[0].grad, h64[0].grad) < TOL and rel(h32[1].grad, h64[1].grad) < TOL


def test_cfg1_full_size_forward_backward(scan):
    """B16 T512 D768, |lambda| = sigmoid(N(4,1)), arg ~ U(-0.5, 0.5), u = gamma * N(0,1) with
    gamma ~ N(0, 0.1) per channel, upstream dL/dy ~ N(0,1) and N(0,1) on the final (Re, Im) state."""
    B, T, D = 16, 512, 768
    g = torch.Generator().manual_seed(1)
    u = torch.randn(B, T, D, generator=g)
    lm = F.logsigmoid(torch.randn(B, T, D, generator=g) + 4.0)
    an = torch.rand(B, T, D, generator=g) - 0.5
    gam = torch.randn(D, generator=g) * 0.1
    gy, glr, gli = torch.randn(B, T, D, generator=g), torch.randn(B, D, generator=g), torch.randn(B, D, generator=g)
    a64 = [t.double().requires_grad_(True) for t in (u, lm, an)]
    gam64 = gam.double().requires_grad_(True)
    y, (r, i) = O.recurrence(a64[0] * gam64, a64[1], a64[2])
    ((y * gy).sum() + (r * glr).sum() + (i * gli).sum()).backward()
    a32 = [t.cuda().requires_grad_(True) for t in (u, lm, an)]
    gam32 = gam.cuda().requires_grad_(True)
    yk, (rk, ik) = scan(a32[0] * gam32, a32[1], a32[2])
    ((yk * gy.cuda()).sum() + (rk * glr.cuda()).sum() + (ik * gli.cuda()).sum()).backward()
    assert rel(yk, y) < TOL and rel(rk, r) < TOL and rel(ik, i) < TOL
    for mine, ref in zip(a32 + [gam32], a64 + [gam64]):
        assert rel(mine.grad, ref.grad) < TOL


def test_extreme_decay_is_finite(scan):
    g = torch.Generator().manual_seed(0)
    lm = torch.full((2, 512, 8), -40.0)
    y, (r, i) = scan(torch.randn(2, 512, 8, generator=g).cuda(), lm.cuda(), torch.randn(2, 512, 8, generator=g).cuda())
    assert torch.isfinite(y).all() and torch.isfinite(r).all()


def test_rejects_cpu_tensors(scan):
    from pragnosia_amd import PragnosiaError
    with pytest.raises(PragnosiaError):
        scan(torch.randn(1, 4, 8), torch.zeros(1, 4, 8), torch.zeros(1, 4, 8))


def test_large_angles(scan):
    """Angles on both sides of the hardware sine's range guard (|x| < 64 rad uses the hardware sine/cosine, beyond
    it the precise routine), up to 1500 rad: forward and gradients still within 1e-4 of the fp64 recurrence on the
    same fp32 inputs."""
    g = torch.Generator().manual_seed(12)
    B, T, D = 2, 70, 64
    u = torch.randn(B, T, D, generator=g)
    lm = F.logsigmoid(torch.randn(B, T, D, generator=g) + 4.0)
    an = (torch.rand(B, T, D, generator=g) - 0.5) * 3000.0
    w = torch.randn(B, T, D, generator=g)
    a64 = [t.double().requires_grad_(True) for t in (u, lm, an)]
    y64, _ = O.recurrence(*a64)
    (y64 * w.double()).sum().backward()
    a32 = [t.cuda().requires_grad_(True) for t in (u, lm, an)]
    y32, _ = scan(*a32)
    (y32 * w.cuda()).sum().backward()
    assert rel(y32, y64) < TOL
    for mine, ref in zip(a32, a64):
        assert rel(mine.grad, ref.grad) < TOL


def test_empty_sequence_returns_h0_and_passes_its_gradient(scan):
    """T = 0: the final state is the initial one (zero without h0), as the reference's scan returns it, and the
    gradient on the final state is the gradient on h0."""
    B, D = 3, 40
    g = torch.Generator().manual_seed(11)
    h0r, h0i = (torch.randn(B, D, generator=g).cuda().requires_grad_(True) for _ in range(2))
    u, lm, an = (torch.zeros(B, 0, D, device="cuda", requires_grad=True) for _ in range(3))
    y, (hr, hi) = scan(u, lm, an, (h0r, h0i))
    assert y.shape == (B, 0, D) and torch.equal(hr, h0r) and torch.equal(hi, h0i)
    wr, wi = (torch.randn(B, D, generator=g).cuda() for _ in range(2))
    ((hr * wr).sum() + (hi * wi).sum()).backward()
    assert torch.equal(h0r.grad, wr) and torch.equal(h0i.grad, wi)
    with torch.no_grad():
        _, (zr, zi) = scan(u, lm, an)
    assert not zr.any() and not zi.any()
