"""GPU parity of the modules around the kernels (AssocCarrier plain/delta, SpinCarrier rf, LM, forward_carried, the
fused decode step and the graphed greedy decode) against the fp64 CPU oracle driven by the same state_dict.

Tolerances (bf16-input scan paths, from the north star): max relative error <= 2e-2 on outputs and carried states,
<= 5e-2 on gradients; 1e-4 for the fp32 diagonal-scan module (SpinCarrier rf runs fp32 end to end). Outputs of a
residual module are compared on the module's contribution (out - x), which is what the kernels compute."""
import math

import pytest
import torch

from oracle import aspin as OA
from oracle import modules as M

pytestmark = pytest.mark.gpu
TOL_OUT, TOL_GRAD = 2e-2, 5e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _randomise(mod, g):
    """Every parameter away from its initial value (gates and decays included) so each term is exercised."""
    with torch.no_grad():
        for name, p in mod.named_parameters():
            if name.endswith("theta"):
                p.mul_(1 + 0.1 * torch.rand(p.shape, generator=g))
            elif name.endswith("A") or name.endswith("nu_raw"):
                continue
            elif p.dim() >= 2:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[-1]))
            else:
                p.add_(0.1 * torch.randn(p.shape, generator=g))


def _sd64(mod):
    return {k: v.detach().double().cpu() for k, v in mod.state_dict().items()}


def _param_blocks(mod):
    """Parameter groups compared as one tensor each. A linear layer is one affine map [W | b] on [z; 1], so its
    weight and bias are one block; the decay scale A joins the decay gate's block (la = -softplus(wa z + b) e^A).
    Compared alone, a per-head bias (or A) has a gradient that is a sum over every token of the batch with heavy
    cancellation (two entries here): its max-relative error then measures the cancellation, not the kernels --
    over 16 random inits the per-token gradients behind it (the weight blocks) stay within 1%, while the bare
    2-entry sums range up to 10%."""
    params = dict(mod.named_parameters())
    blocks, used = {}, set()
    for name in params:
        if name.endswith(".weight") and name[:-7] + ".bias" in params:
            blocks[name[:-7]] = [name, name[:-7] + ".bias"] + (["A"] if name == "wa.weight" and "A" in params else [])
            used.update(blocks[name[:-7]])
    for name in params:
        if name not in used:
            blocks[name] = [name]
    return blocks


def _block_errors(mod, sd):
    errs = {}
    for blk, names in _param_blocks(mod).items():
        got = [dict(mod.named_parameters())[n].grad for n in names]
        ref = [sd[n].grad for n in names]
        if all(t is None for t in got):   # the write gate wi is unused by the delta rule, on both sides
            assert all(t is None for t in ref), blk
            continue
        errs[blk] = rel(torch.cat([t.flatten().cpu() for t in got]), torch.cat([t.flatten() for t in ref]))
    return errs


@pytest.mark.parametrize("delta", [False, True])
def test_assoc_carrier_forward_backward(delta):
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(10 + delta)   # default initialisation of the parameters _randomise leaves partly in place
    g = torch.Generator().manual_seed(10 + delta)
    mod = AssocCarrier(128, delta=delta)
    _randomise(mod, g)
    mod = mod.cuda()
    x = torch.randn(2, 150, 128, generator=g)
    S0 = torch.randn(2, 2, 64, 64, generator=g) * 0.2
    wo = torch.randn(2, 150, 128, generator=g)
    wS = torch.randn(2, 2, 64, 64, generator=g)
    # oracle, fp64, with autograd on x, S0 and every parameter
    sd = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in _sd64(mod).items()}
    xr, S0r = x.double().requires_grad_(True), S0.double().requires_grad_(True)
    yr, (Sr, Tr) = M.assoc_carrier(sd, xr, (S0r, 77), heads=2, delta=delta)
    ((yr - xr) * wo.double()).sum().add((Sr * wS.double()).sum()).backward()
    xk, S0k = x.cuda().requires_grad_(True), S0.cuda().requires_grad_(True)
    yk, (Sk, Tk) = mod(xk, (S0k, 77))
    assert Tk == Tr == 150
    ((yk - xk) * wo.cuda()).sum().add((Sk * wS.cuda()).sum()).backward()
    assert rel(yk - xk, yr - xr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    assert rel(xk.grad, xr.grad) < TOL_GRAD and rel(S0k.grad, S0r.grad) < TOL_GRAD
    for blk, e in _block_errors(mod, sd).items():
        assert e < TOL_GRAD, (blk, e)


@pytest.mark.parametrize("delta", [False, True])
def test_assoc_carrier_decode_step(delta):
    """T = 1 without autograd runs the fused decode kernel: rebase by p0 (host int and device scalar), normalise,
    gate, write, read. Against the oracle's T = 1 call."""
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(20 + delta)
    g = torch.Generator().manual_seed(20 + delta)
    mod = AssocCarrier(128, delta=delta)
    _randomise(mod, g)
    mod = mod.cuda()
    sd = _sd64(mod)
    x = torch.randn(3, 1, 128, generator=g)
    S0 = torch.randn(3, 2, 64, 64, generator=g) * 0.2
    yr, (Sr, _) = M.assoc_carrier(sd, x.double(), (S0.double(), 33), heads=2, delta=delta)
    with torch.no_grad():
        yk, (Sk, Tk) = mod(x.cuda(), (S0.cuda(), 33))
        yd, (Sd, Td) = mod(x.cuda(), (S0.cuda(), torch.tensor(33.0, device="cuda")))
    assert Tk == 1 and torch.is_tensor(Td) and float(Td) == 1.0
    assert rel(yk - x.cuda(), yr - x.double()) < 1e-4 and rel(Sk, Sr) < 1e-4
    assert torch.equal(Sk, Sd) and torch.equal(yk, yd)


@pytest.mark.parametrize("D", [64, 128])
def test_rebase_kernel_and_gradient(D):
    """The rebase kernel against the oracle's rotation of the key rows, and its backward against autograd, at head
    dims 64 and 128."""
    from pragnosia_amd import ops  # noqa: F401
    g = torch.Generator().manual_seed(3)
    S = torch.randn(2, 3, D, D, generator=g)
    th = torch.rand(3, D // 2, generator=g) * 0.1
    w = torch.randn(2, 3, D, D, generator=g)
    Sr, thr = S.double().requires_grad_(True), th.double().requires_grad_(True)
    (OA.rebase(Sr, thr, 300.0) * w.double()).sum().backward()
    Sk, thk = S.cuda().requires_grad_(True), th.cuda().requires_grad_(True)
    out = torch.ops.pragnosia.aspin_rebase(Sk, thk, None, 300.0)
    (out * w.cuda()).sum().backward()
    assert rel(out, OA.rebase(S.double(), th.double(), 300.0)) < 1e-4
    assert rel(Sk.grad, Sr.grad) < 1e-4 and rel(thk.grad, thr.grad) < 1e-4


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prep_kernel_forward_backward(dtype, D):
    """The fused prep against the oracle's normalise/gate/rotate (`tests/test_assoc.py:187-212` of the reference:
    prep kernel vs torch at position offsets up to 4096), with gradients of the projections, gate and theta, at head
    dims 64 and 128."""
    from pragnosia_amd import ops  # noqa: F401
    g = torch.Generator().manual_seed(5)
    B, T, H = 2, 200, 3
    qp, kp, vp = (torch.randn(B, T, H, D, generator=g).to(dtype).float() for _ in range(3))
    gate = torch.randn(B, T, H, generator=g)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    pos = torch.arange(T) + 4096
    w = [torch.randn(B, H, T, D, generator=g) for _ in range(3)]
    ref_in = [t.double().requires_grad_(True) for t in (qp, kp, vp, gate, th)]
    outs = OA.prep(*ref_in[:4], ref_in[4], pos)
    sum((o * wi.double()).sum() for o, wi in zip(outs, w)).backward()
    k_in = [t.cuda().to(dtype).requires_grad_(True) for t in (qp, kp, vp)] + \
           [t.cuda().requires_grad_(True) for t in (gate, th)]
    kouts = torch.ops.pragnosia.aspin_prep(*k_in[:4], k_in[4], pos.cuda())
    sum((o.float() * wi.cuda()).sum() for o, wi in zip(kouts, w)).backward()
    for o, r in zip(kouts, outs):
        assert rel(o, r) < 1e-2
    # the op's outputs are the bf16 operands of the scan, and their gradients arrive rounded to bf16 (2^-9 per
    # element): against the exact fp64 gradients that costs 1.4-3.2e-3 (measured over three seeds), so fp32 inputs are
    # held to 5e-3 there, and the kernel itself to the fp32 bound against the same fp64 composition fed the
    # bf16-rounded upstream gradients (measured <= 1.3e-5)
    for a, b in zip(k_in, ref_in):
        assert rel(a.grad, b.grad) < (5e-2 if dtype == torch.bfloat16 else 5e-3)
    if dtype == torch.float32:
        ref2 = [t.double().requires_grad_(True) for t in (qp, kp, vp, gate, th)]
        outs2 = OA.prep(*ref2[:4], ref2[4], pos)
        sum((o * wi.bfloat16().double()).sum() for o, wi in zip(outs2, w)).backward()
        for a, b in zip(k_in, ref2):
            assert rel(a.grad, b.grad) < 1e-4


def test_spin_rf_forward_backward():
    from pragnosia_amd.spin import SpinCarrier
    torch.manual_seed(7)
    g = torch.Generator().manual_seed(7)
    mod = SpinCarrier(96, gated="rf")
    _randomise(mod, g)
    mod = mod.cuda()
    sd = {k: v.clone().requires_grad_(True) for k, v in _sd64(mod).items()}
    x = torch.randn(2, 130, 96, generator=g)
    h0 = (torch.randn(2, 96, generator=g), torch.randn(2, 96, generator=g))
    w = torch.randn(2, 130, 96, generator=g)
    xr = x.double().requires_grad_(True)
    yr, hr = M.spin_rf(sd, xr, tuple(t.double() for t in h0))
    ((yr - xr) * w.double()).sum().add(hr[0].sum() + 2 * hr[1].sum()).backward()
    xk = x.cuda().requires_grad_(True)
    yk, hk = mod(xk, tuple(t.cuda() for t in h0))
    ((yk - xk) * w.cuda()).sum().add(hk[0].sum() + 2 * hk[1].sum()).backward()
    assert rel(yk - xk, yr - xr) < 1e-4 and rel(hk[0], hr[0]) < 1e-4 and rel(hk[1], hr[1]) < 1e-4
    assert rel(xk.grad, xr.grad) < 1e-4
    # parameter gradients are sums over B T tokens (the scalar gate's of mixed signs): measured <= 3e-5
    for name, p in mod.named_parameters():
        assert rel(p.grad, sd[name].grad) < 1e-4, name


def _lm(mixer, seed):
    from pragnosia_amd.model import LM
    torch.manual_seed(seed)
    m = LM(vocab=300, d=128, layers=2, ctx=64, mixer=mixer)
    g = torch.Generator().manual_seed(seed)
    for mx in m.mix:
        _randomise(mx, g)
    with torch.no_grad():
        m.e.weight.mul_(20)   # logits of order one, so the argmax is not a near tie everywhere
    return m.cuda().eval()


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_lm_forward_and_forward_carried(mixer):
    m = _lm(mixer, 30)
    sd = _sd64(m)
    g = torch.Generator().manual_seed(31)
    ids = torch.randint(0, 300, (2, 200), generator=g)
    with torch.no_grad():
        f = m(ids[:, :64].cuda())
        c = m.forward_carried(ids.cuda(), window=64)
    fr = M.lm_forward(sd, ids[:, :64], layers=2, mixer=mixer, heads=2)
    cr = M.lm_forward_carried(sd, ids, 64, layers=2, mixer=mixer, heads=2)
    tol = 1e-4 if mixer == "fspin" else TOL_OUT
    assert rel(f, fr) < tol and rel(c, cr) < tol


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_graphed_decode_equals_eager_and_oracle(mixer):
    """The graph-captured greedy decode (argmax on the device) gives the eager loop's tokens exactly; the eager
    loop's logits match the oracle's teacher-forced decode on the same tokens."""
    from pragnosia_amd.decode import GreedyDecoder, greedy_eager
    m = _lm(mixer, 40)
    g = torch.Generator().manual_seed(41)
    prompt = torch.randint(0, 300, (2, 100), generator=g)
    n = 21
    dec = GreedyDecoder(m, 2, steps_per_graph=4)
    toks_g = dec.generate(prompt.cuda(), n)
    toks_e, lgs_e = greedy_eager(m, prompt.cuda(), n)
    assert torch.equal(toks_g.cpu(), toks_e.cpu())
    _, lgs_r = M.greedy_decode(_sd64(m), prompt, n, layers=2, mixer=mixer, heads=2, forced=toks_e.cpu())
    tol = 1e-4 if mixer == "fspin" else TOL_OUT
    assert rel(lgs_e, lgs_r) < tol
    # a second generation reuses the captured graph with a new state
    toks_g2 = dec.generate(prompt[:, :70].cuda(), n)
    toks_e2, _ = greedy_eager(m, prompt[:, :70].cuda(), n)
    assert torch.equal(toks_g2.cpu(), toks_e2.cpu())
