"""The carrier's module switches against the fp64 oracle on the same state_dict: `fused_scan` (no entering states
kept, `src/assoc.py:518-532`; under autograd the delta carriers recompute them in the backward, `:481-492`), `FUSED_PROJ` (one GEMM for the delta carrier's five projections, `:272-276`,
`:415-427`), `key_topk` (`:438-442`), `pos_wrap` (`:406-410`), `beta_scale` (`:469-472`) and `hl_floor` (`:355-359`).

Tolerances: kernel path (bf16 operands) 2e-2 on outputs and states, 5e-2 on gradients; torch path (kernel=False,
fp32) 1e-4."""
import math

import pytest
import torch

from oracle import modules as M
from test_gpu_modules import _block_errors, _randomise, _sd64, rel

pytestmark = pytest.mark.gpu


def _carrier(seed, **kw):
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(seed)
    g = torch.Generator().manual_seed(seed)
    mod = AssocCarrier(128, **kw)
    _randomise(mod, g)
    return mod.cuda(), g


@pytest.mark.parametrize("delta", [False, True])
def test_fused_scan_context(delta):
    """Inside fused_scan the carriers keep no entering states (their `sent` is None) and their outputs are
    unchanged; on exit the previous setting returns."""
    from pragnosia_amd import assoc as A
    from pragnosia_amd.model import LM
    torch.manual_seed(100)
    lm = LM(vocab=300, d=128, layers=2, ctx=64, mixer="dspin" if delta else "aspin").cuda()
    ids = torch.randint(0, 300, (2, 64), device="cuda")
    with torch.no_grad():
        ref = lm(ids)
        assert all(mx.sent is not None for mx in lm.mix)
        with A.fused_scan(lm):
            assert A.FUSED_SCAN and all(not mx.need_sent for mx in lm.mix)
            got = lm(ids)
            assert all(mx.sent is None for mx in lm.mix) or not delta
        assert not A.FUSED_SCAN and all(mx.need_sent for mx in lm.mix)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("D", [64, 128])
def test_delta_fused_recomputes_in_backward(D):
    """`aspin_delta_fused` (the FUSED_SCAN training path) equals the stored-state op bit for bit, outputs and every
    gradient (its backward recomputes X, W and the entering states with the same kernels), and what it keeps for the
    backward is its inputs: the saved bytes drop by exactly the entering states, W and X, less the S0 it keeps."""
    import torch.nn.functional as F
    from pragnosia_amd import ops  # noqa: F401
    op = torch.ops.pragnosia
    g = torch.Generator().manual_seed(5 + D)
    B, H, T = 2, 3, 200
    q = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16().cuda()
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16().cuda()
    v = torch.randn(B, H, T, D, generator=g).bfloat16().cuda()
    la = (-0.1 * torch.rand(B, H, T, generator=g)).cuda()
    beta = (0.2 + 0.6 * torch.rand(B, H, T, generator=g)).cuda()
    S0 = (0.1 * torch.randn(B, H, D, D, generator=g)).cuda()
    do = torch.randn(B, H, T, D, generator=g).bfloat16().cuda()
    dS = torch.randn(B, H, D, D, generator=g).cuda()

    def run(fused):
        ins = [t.clone().requires_grad_(True) for t in (q, k, v, la, beta, S0)]
        saved = []

        def pack(t):
            saved.append(t.numel() * t.element_size())
            return t
        with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
            o, S = op.aspin_delta_fused(*ins) if fused else op.aspin_delta(*ins, True)[:2]
        torch.autograd.backward([o, S], [do, dS])
        return o, S, [t.grad for t in ins], sum(saved)
    o1, S1, g1, b1 = run(False)
    o2, S2, g2, b2 = run(True)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    NC = (T + 63) // 64
    assert b1 - b2 == 2 * (B * H * NC * D * D + B * H * T * D + B * H * NC * 64 * 64) - 4 * B * H * D * D


def test_fused_scan_training_step():
    """A training step of a delta LM inside fused_scan: the carriers keep no entering states, and the loss and every
    parameter gradient equal the stored-state path's bit for bit."""
    from pragnosia_amd import assoc as A
    from pragnosia_amd.model import LM
    torch.manual_seed(101)
    lm = LM(vocab=300, d=128, layers=2, ctx=160, mixer="dspin").cuda()
    ids = torch.randint(0, 300, (2, 160), device="cuda")

    def step():
        lm.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = lm(ids)
        loss = torch.nn.functional.cross_entropy(logits.float().reshape(-1, 300), ids.reshape(-1))
        loss.backward()
        return loss.detach(), [None if p.grad is None else p.grad.clone() for p in lm.parameters()]
    ref_loss, ref_grads = step()
    with A.fused_scan(lm):
        loss, grads = step()
        assert all(mx.sent is None for mx in lm.mix)
    assert torch.equal(loss, ref_loss)
    assert sum(a is not None for a in grads) > 10
    for a, b in zip(grads, ref_grads):
        assert (a is None and b is None) or torch.equal(a, b)


@pytest.mark.parametrize("kernel", [True, False])
def test_fused_proj_delta(kernel, monkeypatch):
    """FUSED_PROJ (with this build's own fused plumbing off, so the reference's composition runs): one GEMM for q,
    k, v, the decay and the write strength; output, state and gradients against the oracle."""
    from pragnosia_amd import assoc as A
    monkeypatch.setattr(A, "FUSED_PROJ", True)
    monkeypatch.setattr(A, "FUSED_PLUMBING", False)
    mod, g = _carrier(110 + kernel, delta=True, kernel=kernel)
    _check(mod, g, delta=True, tol=(2e-2, 5e-2) if kernel else (1e-4, 1e-4))


def _check(mod, g, delta, tol, T=100, p0=21, **oracle_kw):
    x = torch.randn(2, T, 128, generator=g)
    S0 = torch.randn(2, mod.h, 64, 64, generator=g) * 0.2
    wo, wS = torch.randn(2, T, 128, generator=g), torch.randn(2, mod.h, 64, 64, generator=g)
    sd = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in _sd64(mod).items()}
    xr, S0r = x.double().requires_grad_(True), S0.double().requires_grad_(True)
    yr, (Sr, _) = M.assoc_carrier(sd, xr, (S0r, p0), heads=mod.h, delta=delta, key_topk=mod.key_topk,
                                  write_all=mod.write_all, **oracle_kw)
    ((yr - xr) * wo.double()).sum().add((Sr * wS.double()).sum()).backward()
    xk, S0k = x.cuda().requires_grad_(True), S0.cuda().requires_grad_(True)
    yk, (Sk, _) = mod(xk, (S0k, p0))
    ((yk - xk) * wo.cuda()).sum().add((Sk * wS.cuda()).sum()).backward()
    t_out, t_grad = tol
    assert rel(yk - xk, yr - xr) < t_out and rel(Sk, Sr) < t_out
    assert rel(xk.grad, xr.grad) < t_grad and rel(S0k.grad, S0r.grad) < t_grad
    for blk, e in _block_errors(mod, sd).items():
        assert e < t_grad, (blk, e)


@pytest.mark.parametrize("kernel", [True, False])
@pytest.mark.parametrize("delta", [False, True])
def test_key_topk(delta, kernel):
    """Sparse keys: only the key_topk largest coordinates of each projected key survive (straight-through)."""
    mod, g = _carrier(120 + delta + 2 * kernel, delta=delta, key_topk=8, kernel=kernel)
    _check(mod, g, delta, (2e-2, 5e-2) if kernel else (1e-4, 1e-4))


@pytest.mark.parametrize("kernel", [True, False])
def test_pos_wrap(kernel):
    """Rotation positions modulo pos_wrap (T = 100 > pos_wrap = 32): the plain carrier against the oracle."""
    mod, g = _carrier(130 + kernel, kernel=kernel)
    mod.pos_wrap = 32
    _check(mod, g, False, (2e-2, 5e-2) if kernel else (1e-4, 1e-4), pos_wrap=32)


@pytest.mark.parametrize("kernel", [True, False])
def test_beta_scale_and_hl_floor(kernel):
    """The delta carrier with a per-token write-strength multiplier (beta_scale, (B, H, T)) and the half-life floor
    under each head's decay."""
    mod, g = _carrier(140 + kernel, delta=True, hl_floor=True, kernel=kernel)
    bs = torch.rand(2, mod.h, 100, generator=g)
    mod.beta_scale = bs.cuda()
    floor = (-math.log(2.0) / torch.logspace(math.log10(8.0), math.log10(131072.0), mod.h)).double()
    assert torch.allclose(mod.la_floor.cpu().double(), floor)
    _check(mod, g, True, (2e-2, 5e-2) if kernel else (1e-4, 1e-4), la_floor=floor, beta_scale=bs.double())


def test_delta_chunk128_entering_states():
    """A delta carrier built with chunk=128 (the reference's 128-token delta kernel, `src/assoc.py:494-495`) returns
    the same output and final state as at chunk 64 (the result does not depend on the chunk) and exposes the states
    entering every 128-token chunk: those of every other 64-token chunk, ceil(T / 128) of them, each against the
    fp64 oracle's chunk-128 entering states (bf16 kernel tolerance)."""
    from oracle import aspin as OA
    m64, g = _carrier(91, delta=True)
    m128, _ = _carrier(91, delta=True, chunk=128)
    x = torch.randn(2, 300, 128, generator=g).cuda()
    with torch.no_grad():
        y64, (S64, _) = m64(x)
        y128, (S128, _) = m128(x)
    assert torch.equal(y64, y128) and torch.equal(S64, S128)
    s64, s128 = m64.sent, m128.sent
    assert s128.shape == (2, m64.h, 3, 64, 64) and torch.equal(s128, s64[:, :, ::2])
    # the oracle's chunk-128 scan on the kernel's own inputs (its prep), entering states of every 128-token chunk
    with torch.no_grad():
        from pragnosia_amd.assoc import _positions
        z = m64._norm_in(x)
        q, k, v, la, bt, _, _ = m64._scan_inputs(z, _positions(300, x.device, None), None)
    _, _, ent, _ = OA.scan_twopass_delta(q.double().cpu(), k.double().cpu(), v.double().cpu(), la.double().cpu(),
                                         bt.double().cpu(), torch.zeros(2, m64.h, 64, 64, dtype=torch.float64), 128)
    assert rel(s128.float(), ent.float()) < 2e-2
