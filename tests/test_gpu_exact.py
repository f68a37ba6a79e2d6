"""GPU parity of the exact scan (`aspin_exact`: fp32 / fp64 operands, no bf16 rounding) behind `assoc_scan`,
against the literal recurrence and the CPU oracle.

Tolerances: fp64 inputs are held to the reference's own bounds for its fp64 scan (`tests/test_assoc.py:18-44`:
outputs and states 1e-11 absolute, gradients 1e-9 relative); fp32 paths to the north star's 1e-4 max relative error
(max|x - ref| / max|ref|) against the fp64 oracle, on outputs, final states and every gradient."""
import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as O

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def recurrence(q, k, v, la, S, beta=None):
    """The literal per-token recurrence, as the reference's test writes it (`tests/test_assoc.py:22-27`), with the
    delta rule's decay inside the read (`src/assoc.py:238-241`)."""
    out = []
    for t in range(q.shape[2]):
        a = torch.exp(la[:, :, t])[..., None, None]
        kt, vt = k[:, :, t].unsqueeze(-1), v[:, :, t].unsqueeze(-2)
        if beta is None:
            S = a * S + kt @ vt
        else:
            P = a * S
            S = P + beta[:, :, t][..., None, None] * kt @ (vt - kt.transpose(-1, -2) @ P)
        out.append((q[:, :, t].unsqueeze(-2) @ S).squeeze(-2))
    return torch.stack(out, 2), S


@pytest.fixture(scope="module")
def scan():
    from pragnosia_amd.assoc import assoc_scan
    return assoc_scan


def test_fp64_matches_recurrence_like_the_reference_test(scan):
    """`tests/test_assoc.py:18-44` on the GPU: fp64, B2 H3 T45 D8, carried S0; outputs and final state at 1e-11;
    chunk size irrelevant; carried windows == one pass; gradients of q, k, v, la at 1e-9."""
    g = torch.Generator().manual_seed(0)
    B, H, T, D = 2, 3, 45, 8
    q = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    k, v = torch.randn_like(q), torch.randn_like(q)
    la = -torch.rand(B, H, T, generator=g, dtype=torch.float64) * 3.0
    S0 = torch.randn(B, H, D, D, generator=g, dtype=torch.float64)
    yr, Sr = recurrence(q, k, v, la, S0.clone())
    dev = [t.cuda() for t in (q, k, v, la, S0)]
    yc, Sc = scan(*dev, chunk=8)
    assert yc.dtype == torch.float64 and Sc.dtype == torch.float64
    assert (yc.cpu() - yr).abs().max() < 1e-11 and (Sc.cpu() - Sr).abs().max() < 1e-11
    y0, _ = scan(*dev[:4], None, chunk=8)
    yr0, _ = recurrence(q, k, v, la, torch.zeros_like(S0))
    assert (y0.cpu() - yr0).abs().max() < 1e-11
    a, st = scan(*(t[:, :, :20] for t in dev[:4]), dev[4], chunk=8)
    b, _ = scan(*(t[:, :, 20:] for t in dev[:4]), st, chunk=8)
    assert (torch.cat([a, b], 2).cpu() - yr).abs().max() < 1e-11
    qg, kg, vg, lg = (t.clone().requires_grad_(True) for t in dev[:4])
    (scan(qg, kg, vg, lg, None, chunk=8)[0] ** 2).sum().backward()
    qr, kr, vr, lr = (t.clone().requires_grad_(True) for t in (q, k, v, la))
    (recurrence(qr, kr, vr, lr, torch.zeros_like(S0))[0] ** 2).sum().backward()
    worst = max(rel(x.grad, y.grad) for x, y in zip((qg, kg, vg, lg), (qr, kr, vr, lr)))
    assert worst < 1e-9, worst


def test_fp64_delta_known_answer():
    """`tests/test_assoc.py:118-130`: a key written twice reads back the second value under the delta rule, and the
    sum under the plain rule, in fp64 to 1e-9."""
    from pragnosia_amd.assoc import assoc_scan
    g = torch.Generator().manual_seed(3)
    kk = F.normalize(torch.randn(1, 1, 1, 4, generator=g, dtype=torch.float64), dim=-1)
    va = torch.tensor([[[[1.0, 0, 0, 0]]]], dtype=torch.float64)
    vb = torch.tensor([[[[0.0, 1.0, 0, 0]]]], dtype=torch.float64)
    K, V = torch.cat([kk, kk, kk], 2).cuda(), torch.cat([va, vb, va], 2).cuda()
    la = torch.zeros(1, 1, 3, dtype=torch.float64, device="cuda")
    be = torch.ones(1, 1, 3, dtype=torch.float64, device="cuda")
    r1 = assoc_scan(K, K, V, la, None, chunk=1, beta=be)[0][0, 0, 1].cpu()
    rp = assoc_scan(K, K, V, la, None, chunk=3)[0][0, 0, 1].cpu()
    assert (r1 - vb[0, 0, 0]).abs().max() < 1e-9
    assert (rp - (va + vb)[0, 0, 0]).abs().max() < 1e-9


def _fp32_case(B, H, T, Dk, Dv, delta, seed, s0=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, Dk, generator=g)
    k = F.normalize(torch.randn(B, H, T, Dk, generator=g), dim=-1)
    v = torch.randn(B, H, T, Dv, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    be = torch.sigmoid(torch.randn(B, H, T, generator=g)) if delta else None
    S0 = torch.randn(B, H, Dk, Dv, generator=g) * 0.1 if s0 else None
    wo = torch.randn(B, H, T, Dv, generator=g)
    wS = torch.randn(B, H, Dk, Dv, generator=g)
    return q, k, v, la, be, S0, wo, wS


def _check_fp32(scan, q, k, v, la, be, S0, wo, wS):
    """Forward, final state and every gradient (q, k, v, la, beta, S0) of the fp32 exact path against the fp64
    oracle (`oracle.aspin.assoc_scan`, the reference's two-pass forms)."""
    ins = [q, k, v, la] + ([be] if be is not None else []) + ([S0] if S0 is not None else [])
    names = ["q", "k", "v", "la"] + (["beta"] if be is not None else []) + (["S0"] if S0 is not None else [])
    r = [t.double().requires_grad_(True) for t in ins]
    rd = dict(zip(names, r))
    yr, Sr = O.assoc_scan(rd["q"], rd["k"], rd["v"], rd["la"], rd.get("S0"), chunk=16, beta=rd.get("beta"))
    ((yr * wo.double()).sum() + (Sr * wS.double()).sum()).backward()
    d = [t.cuda().requires_grad_(True) for t in ins]
    dd = dict(zip(names, d))
    yk, Sk = scan(dd["q"], dd["k"], dd["v"], dd["la"], dd.get("S0"), beta=dd.get("beta"))
    assert yk.dtype == torch.float32 and Sk.dtype == torch.float32
    ((yk * wo.cuda()).sum() + (Sk * wS.cuda()).sum()).backward()
    errs = {"o": rel(yk, yr), "S": rel(Sk, Sr)}
    for n, a, b in zip(names, d, r):
        errs["d" + n] = rel(a.grad, b.grad)
    return errs


@pytest.mark.parametrize("delta", [False, True])
@pytest.mark.parametrize("B,H,T,Dk,Dv,s0", [(2, 3, 333, 64, 64, True), (1, 2, 77, 32, 96, True),
                                            (1, 2, 130, 128, 128, False), (2, 1, 1, 64, 64, True),
                                            (1, 1, 9, 6, 10, True)])
def test_fp32_matches_oracle(scan, delta, B, H, T, Dk, Dv, s0):
    """fp32 inputs, plain and delta rules: ragged T, T = 1, unequal and odd head dims, head dim 128, with and without
    a carried state; outputs, final state and every gradient within 1e-4 of the fp64 oracle."""
    e = _check_fp32(scan, *_fp32_case(B, H, T, Dk, Dv, delta, seed=T + Dk, s0=s0))
    assert max(e.values()) < 1e-4, e


@pytest.mark.parametrize("B,H,T,Dk,Dv", [(1, 2, 77, 176, 176), (1, 1, 40, 384, 200)])
def test_fp32_wide_heads_plain(scan, B, H, T, Dk, Dv):
    """Head dims above 128, plain rule (the reference's wspin / w2spin: four or two heads of 176-384): the exact scan
    over key and value blocks of at most 128, outputs, final state and every gradient within 1e-4 of the fp64
    oracle."""
    e = _check_fp32(scan, *_fp32_case(B, H, T, Dk, Dv, False, seed=T + Dk, s0=True))
    assert max(e.values()) < 1e-4, e


@pytest.mark.parametrize("B,H,T,Dk,Dv", [(1, 2, 45, 176, 176), (1, 1, 30, 384, 72), (2, 1, 17, 300, 40)])
def test_fp32_wide_heads_delta(scan, B, H, T, Dk, Dv):
    """Key dims above 128, delta rule (the reference's xspin at d 704-768: four heads of 176-192; and up to 384): the
    keys stay in one launch (48 or 96 rows a lane), the value columns split into blocks that fit the backward's LDS;
    outputs, final state and every gradient within 1e-4 of the fp64 oracle."""
    e = _check_fp32(scan, *_fp32_case(B, H, T, Dk, Dv, True, seed=T + Dk, s0=True))
    assert max(e.values()) < 1e-4, e


@pytest.mark.parametrize("delta,Dk,Dv", [(False, 128, 128), (True, 192, 96)])
def test_fp64_wide_value_blocks(scan, delta, Dk, Dv):
    """fp64 at widths whose backward does not fit one launch's LDS (128 x 128 plain, 192 keys with the delta rule):
    split into value blocks, forward, state and gradients within 1e-10 of the fp64 oracle."""
    q, k, v, la, be, S0, wo, wS = (None if t is None else t.double()
                                   for t in _fp32_case(1, 2, 37, Dk, Dv, delta, seed=Dk + Dv, s0=True))
    ins = [q, k, v, la] + ([be] if delta else []) + [S0]
    r = [t.clone().requires_grad_(True) for t in ins]
    yr, Sr = O.assoc_scan(r[0], r[1], r[2], r[3], r[-1], chunk=16, beta=r[4] if delta else None)
    ((yr * wo).sum() + (Sr * wS).sum()).backward()
    d = [t.cuda().requires_grad_(True) for t in ins]
    yk, Sk = scan(d[0], d[1], d[2], d[3], d[-1], beta=d[4] if delta else None)
    assert yk.dtype == torch.float64
    ((yk * wo.cuda()).sum() + (Sk * wS.cuda()).sum()).backward()
    errs = [rel(yk, yr), rel(Sk, Sr)] + [rel(a.grad, b.grad) for a, b in zip(d, r)]
    assert max(errs) < 1e-10, errs


def test_delta_keys_above_384_rejected(scan):
    """The delta rule couples every key row in each write, so its keys do not split: key dims above 384 are refused
    with an error before any launch."""
    from pragnosia_amd._lib import PragnosiaError
    q, k, v, la, be, S0, _, _ = _fp32_case(1, 1, 12, 400, 32, True, seed=5)
    with pytest.raises(PragnosiaError):
        scan(q.cuda(), k.cuda(), v.cuda(), la.cuda(), S0.cuda(), beta=be.cuda())


def test_cfg0_fp32(scan):
    """BASELINE configs[0], the reference's CPU-runnable case, at its fp32 bound: B1 H4 T256 D64; q, k, v ~ N(0,1),
    k L2-normalised; la = logsigmoid(N(3,1)); theta ~ U(0, 0.1) rotating q and k at positions 0..255; S0 = 0.
    Outputs y (1, 4, 256, 64), the final state and every gradient within 1e-4 of the fp64 oracle."""
    g = torch.Generator().manual_seed(0)
    B, H, T, D = 1, 4, 256, 64
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    pos = torch.arange(T)
    q, k = O.rotate(q, th, pos), O.rotate(k, th, pos)
    wo = torch.randn(B, H, T, D, generator=g)
    wS = torch.randn(B, H, D, D, generator=g)
    e = _check_fp32(scan, q, k, v, la, None, None, wo, wS)
    assert max(e.values()) < 1e-4, e
    print(f"cfg0 fp32 exact path: max rel err {max(e.values()):.2e}")


def test_fp32_long_decay_range_and_mm_switch(scan):
    """Decays down to exp(-40) stay finite (`tests/test_assoc.py:44`), and mm=bf16 (the reference's autocast
    matmuls) routes the same call to the bf16 MFMA kernels: within bf16 error of the fp32 result, not equal to it."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 4, 512, 64, generator=g).cuda()
    k, v = F.normalize(torch.randn_like(q), dim=-1), torch.randn_like(q)
    la = (-torch.rand(2, 4, 512, generator=g) * 40).cuda()
    y32, S32 = scan(q, k, v, la)
    assert torch.isfinite(y32).all() and torch.isfinite(S32).all()
    la2 = -F.softplus(torch.randn(2, 4, 512, generator=g)).cuda() * 0.01
    y32, S32 = scan(q, k, v, la2)
    y16, S16 = scan(q, k, v, la2, mm=torch.bfloat16)
    r = rel(y16, y32)
    assert 1e-6 < r < 3e-2 and rel(S16, S32) < 3e-2


def test_repeated_calls_are_deterministic(scan):
    q, k, v, la, be, S0, _, _ = _fp32_case(2, 4, 200, 64, 64, True, seed=9)
    dev = [t.cuda() for t in (q, k, v, la, be, S0)]
    y1, S1 = scan(*dev[:4], dev[5], beta=dev[4])
    y2, S2 = scan(*dev[:4], dev[5], beta=dev[4])
    assert torch.equal(y1, y2) and torch.equal(S1, S2)


@pytest.mark.parametrize("Dk,dtype", [(384, torch.float32), (128, torch.float64), (192, torch.float64),
                                      (384, torch.float64)])
def test_value_cap_is_the_library_limit(Dk, dtype):
    """`ops.exact_value_cap` is the library's own limit: one launch at exactly that many value columns runs forward
    and backward (delta rule, finite results), and one wave more is refused by the backward."""
    from pragnosia_amd import ops
    from pragnosia_amd._lib import PragnosiaError
    cap = ops.exact_value_cap(Dk, dtype, True)
    assert cap < 128
    q, k, v, la, be, S0, _, _ = _fp32_case(1, 1, 20, Dk, cap + 16, True, seed=Dk)
    dev = lambda t: t.to(dtype).cuda()
    q, k, la, be = dev(q), dev(k), dev(la), dev(be)
    o, S, ckpt, resid = ops.aspin_exact(q, k, dev(v[..., :cap]), la, be, None, True)
    g = ops.aspin_exact_bwd(q, k, dev(v[..., :cap]), la, be, ckpt, resid, torch.ones_like(o), None)
    assert all(torch.isfinite(t).all() for t in (o, S) + tuple(g))
    o2, S2, ckpt2, resid2 = ops.aspin_exact(q, k, dev(v), la, be, None, True)
    with pytest.raises(PragnosiaError):
        ops.aspin_exact_bwd(q, k, dev(v), la, be, ckpt2, resid2, torch.ones_like(o2), None)
