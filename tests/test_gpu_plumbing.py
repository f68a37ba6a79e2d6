"""GPU parity of the carrier's fused plumbing (one projection GEMM feeding pragnosia_aspin_prep_proj_fwd / _bwd, and
the fused output epilogue) against the composition it replaces: separate q, k, v, decay and gate projections, the
decay -softplus(W_a z + b) exp(A) (floored), the write gate, pragnosia_aspin_prep, transposes and nn.RMSNorm.

Both sides run the same HIP scan kernels; they differ in rounding order only (one GEMM instead of five, the decay in
the kernel). Tolerances, as max relative error max|x - ref| / max|ref|: the prep from the same P, q, k, v (bf16)
<= 2^-8, la <= 1e-5, gradients <= 1e-3 (fp32 P) or 2e-2 (bf16 P); the module, whose two paths also round their
projections differently before the bf16 scan, <= 2e-2 on outputs and 5e-2 on gradients (the north star's bf16
bounds), with and without autocast."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


@pytest.mark.parametrize("gated,floor,dtype", [(True, False, torch.float32), (True, True, torch.float32),
                                               (False, False, torch.float32), (True, True, torch.bfloat16)])
def test_prep_proj_matches_composition(gated, floor, dtype):
    import pragnosia_amd.ops  # noqa: F401
    op = torch.ops.pragnosia
    g = torch.Generator().manual_seed(int(gated) + 2 * int(floor) + 4 * (dtype == torch.bfloat16))
    B, T, H = 2, 150, 3
    d = 64 * H
    W = 3 * d + H + (H if gated else 0)
    P = (torch.randn(B, T, W, generator=g) * 0.5).to(dtype)
    la_b, A = torch.randn(H, generator=g), torch.randn(H, generator=g) - 2.0
    fl = -torch.rand(H, generator=g) * 0.05 if floor else None
    gb = torch.randn(H, generator=g) if gated else None
    th = torch.rand(H, 32, generator=g) * 0.1
    pos = torch.arange(T)
    dev = lambda t: None if t is None else t.cuda().requires_grad_(t.is_floating_point())
    ins = [dev(t) for t in (P, la_b, A, fl, gb, th)]
    Pd, lbd, Ad, fld, gbd, thd = ins
    if fld is not None:
        fld.requires_grad_(False)
    q, k, v, la = op.aspin_prep_proj(Pd, H, lbd, Ad, fld, gbd, thd, pos.cuda())
    gq, gk, gv, gl = (torch.randn(t.shape, generator=g) for t in (q, k, v, la))
    ((q.float() * gq.cuda()).sum() + (k.float() * gk.cuda()).sum() + (v.float() * gv.cuda()).sum()
     + (la * gl.cuda()).sum()).backward()
    # the composition: slices, elementwise decay and gate, the dense prep op
    ref = [None if t is None else t.detach().cuda().requires_grad_(t.is_floating_point() and t is not fl)
           for t in (P, la_b, A, fl, gb, th)]
    Pr, lbr, Ar, flr, gbr, thr = ref
    qp, kp, vp = (Pr[..., i * d:(i + 1) * d].reshape(B, T, H, 64) for i in range(3))
    lar = -F.softplus(Pr[..., 3 * d:3 * d + H].float() + lbr) * torch.exp(Ar)
    if flr is not None:
        lar = lar.clamp(min=flr)
    gate = (Pr[..., 3 * d + H:].float() + gbr) if gated else None
    q2, k2, v2 = op.aspin_prep(qp, kp, vp, gate, thr, pos.cuda())
    la2 = lar.transpose(1, 2)
    ((q2.float() * gq.cuda()).sum() + (k2.float() * gk.cuda()).sum() + (v2.float() * gv.cuda()).sum()
     + (la2 * gl.cuda()).sum()).backward()
    for a, b in ((q, q2), (k, k2), (v, v2)):
        assert rel(a, b) < 2 ** -8
    assert rel(la, la2) < 1e-5
    gtol = 1e-3 if dtype == torch.float32 else 2e-2
    assert rel(Pd.grad, Pr.grad) < gtol
    for a, b in ((lbd, lbr), (Ad, Ar), (thd, thr)) + (((gbd, gbr),) if gated else ()):
        assert rel(a.grad, b.grad) < gtol


@pytest.mark.parametrize("autocast", [False, True])
@pytest.mark.parametrize("write_all,hl_floor", [(False, False), (True, True)])
def test_module_fused_plumbing_equals_composition(autocast, write_all, hl_floor):
    """AssocCarrier forward and backward (every parameter's gradient, the input's, the carried state's) with the
    fused plumbing and with the reference's composition, from the same parameters."""
    from pragnosia_amd import assoc
    torch.manual_seed(11)
    m = assoc.AssocCarrier(256, write_all=write_all, hl_floor=hl_floor).cuda()
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.05)
    x = torch.randn(2, 300, 256, device="cuda")
    S0 = torch.randn(2, 4, 64, 64, device="cuda") * 0.1
    gy = torch.randn(2, 300, 256, device="cuda")
    gS = torch.randn(2, 4, 64, 64, device="cuda")
    res = {}
    prev = assoc.FUSED_PLUMBING
    try:
        for fused in (True, False):
            assoc.FUSED_PLUMBING = fused
            m.zero_grad(set_to_none=True)
            xi, Si = x.clone().requires_grad_(True), S0.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
                y, (S, _) = m(xi, (Si, 17))
            ((y.float() * gy).sum() + (S * gS).sum()).backward()
            res[fused] = (y.detach(), S.detach(), xi.grad, Si.grad,
                          {n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None})
    finally:
        assoc.FUSED_PLUMBING = prev
    a, b = res[True], res[False]
    otol, gtol = 2e-2, 5e-2  # both sides cast q, k, v and o to bf16: their roundings differ, and that propagates
    assert rel(a[0] - x, b[0] - x) < otol and rel(a[1], b[1]) < otol
    assert rel(a[2], b[2]) < gtol and rel(a[3], b[3]) < gtol
    assert set(a[4]) == set(b[4])
    for n in a[4]:
        assert rel(a[4][n], b[4][n]) < gtol, n
