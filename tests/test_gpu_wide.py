"""GPU parity of the plain rule at head dim 128 (the reference's `hspin` carrier, `src/model.py:650`), which runs as
four 64 x 64 kernel scans per head (key half x value half) summed: the scan against the fp64 oracle's chunked scan,
forward (o, final state, entering states) and backward; AssocCarrier(d, head_dim=128) forward and backward and its
T = 1 step against the oracle's module; an LM with 128-dim heads, forward_carried and graphed greedy decode.

Tolerances as for the 64-dim paths: bf16 operands, max relative error max|x - ref| / max|ref| <= 2e-2 on outputs and
states, 5e-2 on gradients; the T = 1 step is fp32 throughout (1e-4)."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as OA
from oracle import modules as M
from test_gpu_modules import TOL_GRAD, TOL_OUT, _block_errors, _randomise, _sd64, rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,s0", [(200, True), (64, False), (1, True)])
def test_wide_plain_scan_matches_oracle(T, s0):
    from pragnosia_amd.assoc import assoc_scan
    g = torch.Generator().manual_seed(T)
    B, H, D = 2, 3, 128
    q = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, H, T, D, generator=g).bfloat16()
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3)
    S0 = torch.randn(B, H, D, D, generator=g) * 0.2 if s0 else None
    wo, wS = torch.randn(B, H, T, D, generator=g), torch.randn(B, H, D, D, generator=g)
    ref = [t.double().requires_grad_(True) for t in (q, k, v, la)] + [S0.double().requires_grad_(True) if s0 else None]
    o_r, S_r, sent_r = OA.scan_twopass(*ref[:4], ref[4] if s0 else torch.zeros(B, H, D, D, dtype=torch.float64), 64)
    ((o_r * wo.double()).sum() + (S_r * wS.double()).sum()).backward()
    dev = [t.cuda().requires_grad_(True) for t in (q, k, v, la)] + [S0.cuda().requires_grad_(True) if s0 else None]
    o, S, sent = assoc_scan(*dev, need_sent=True)
    assert o.shape == (B, H, T, D) and S.shape == (B, H, D, D) and sent.shape == sent_r.shape
    ((o.float() * wo.cuda()).sum() + (S * wS.cuda()).sum()).backward()
    assert rel(o, o_r) < TOL_OUT and rel(S, S_r) < TOL_OUT and rel(sent.float(), sent_r) < TOL_OUT
    for a, b in zip(dev, ref):
        if a is not None:
            assert rel(a.grad, b.grad) < TOL_GRAD


def _wide_inputs(B, H, T, seed):
    g = torch.Generator().manual_seed(seed)
    D = 128
    q = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, H, T, D, generator=g).bfloat16()
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3)
    S0 = torch.randn(B, H, D, D, generator=g) * 0.2
    wo, wS = torch.randn(B, H, T, D, generator=g), torch.randn(B, H, D, D, generator=g)
    return q, k, v, la, S0, wo, wS


def test_wide_plain_scan_segmented_matches_oracle():
    """Few heads over a long sequence (B1 H1 T1000: 4 scans) take the segment-parallel passes in both directions;
    forward and backward against the fp64 oracle."""
    from pragnosia_amd import ops
    from pragnosia_amd.assoc import assoc_scan
    B, H, T = 1, 1, 1000
    NC = (T + 63) // 64
    assert ops.seg_chunks(4 * B * H, NC, range(1, NC + 1)) < NC
    assert ops.seg_chunks(4 * B * H, NC, range(1, NC + 1), "bwd") < NC
    q, k, v, la, S0, wo, wS = _wide_inputs(B, H, T, 70)
    ref = [t.double().requires_grad_(True) for t in (q, k, v, la, S0)]
    o_r, S_r, _ = OA.scan_twopass(*ref, 64)
    ((o_r * wo.double()).sum() + (S_r * wS.double()).sum()).backward()
    dev = [t.cuda().requires_grad_(True) for t in (q, k, v, la, S0)]
    o, S = assoc_scan(*dev)
    ((o.float() * wo.cuda()).sum() + (S * wS.cuda()).sum()).backward()
    assert rel(o, o_r) < TOL_OUT and rel(S, S_r) < TOL_OUT
    for a, b in zip(dev, ref):
        assert rel(a.grad, b.grad) < TOL_GRAD


def test_wide_abi_segment_lengths_agree():
    """The C ABI at head dim 128 over segment lengths 1, 3 (ragged: 11 chunks) and whole (one workgroup per scan):
    the segmented forward and backward agree with the one-pass result, which matches the oracle; sent is the same
    in every case (each chunk's entering state is the one-pass scan's up to fp32 summation order)."""
    from pragnosia_amd import ops
    from pragnosia_amd._lib import lib
    L = lib()
    B, H, T, D = 2, 1, 700, 128
    NC = 11
    q, k, v, la, S0, wo, wS = _wide_inputs(B, H, T, 71)
    ref = [t.double().requires_grad_(True) for t in (q, k, v, la, S0)]
    o_r, S_r, _ = OA.scan_twopass(*ref, 64)
    ((o_r * wo.double()).sum() + (S_r * wS.double()).sum()).backward()
    q, k, v, la, S0 = (t.cuda().contiguous() for t in (q, k, v, la, S0))
    do = wo.bfloat16().cuda()
    dS = wS.cuda()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    for seg in (NC, 3, 1):
        o = torch.empty(B, H, T, D, device="cuda", dtype=torch.bfloat16)
        S = torch.empty(B, H, D, D, device="cuda")
        sent = torch.empty(B, H, 4, NC, 64, 64, device="cuda", dtype=torch.bfloat16)
        ws = torch.empty(L.pragnosia_aspin_chunk_wide_workspace_bytes(B, H, T, D, 64, seg, 0), device="cuda",
                         dtype=torch.uint8)
        print(f"wide fwd B{B} H{H} T{T} seg {seg}", flush=True)
        assert L.pragnosia_aspin_chunk_fwd_wide(P(q), P(k), P(v), P(la), P(S0), P(o), P(S), P(sent), P(ws),
                                                ws.numel(), B, H, T, D, 64, seg, s) == 0
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        dla = torch.empty_like(la)
        dS0 = torch.empty_like(S0)
        wb = torch.empty(L.pragnosia_aspin_chunk_wide_workspace_bytes(B, H, T, D, 64, seg, 1), device="cuda",
                         dtype=torch.uint8)
        print(f"wide bwd B{B} H{H} T{T} seg {seg}", flush=True)
        assert L.pragnosia_aspin_chunk_bwd_wide(P(q), P(k), P(v), P(la), P(sent), P(do), P(dS), P(dq), P(dk), P(dv),
                                                P(dla), P(dS0), P(wb), wb.numel(), B, H, T, D, 64, seg, s) == 0
        torch.cuda.synchronize()
        res[seg] = (o, S, sent, dq, dk, dv, dla, dS0)
    o, S, sent, dq, dk, dv, dla, dS0 = res[NC]
    assert rel(o, o_r) < TOL_OUT and rel(S, S_r) < TOL_OUT
    for a, b in zip((dq, dk, dv, dla, dS0), ref):
        assert rel(a, b.grad) < TOL_GRAD
    for seg in (3, 1):
        for a, b in zip(res[seg], res[NC]):
            assert rel(a.float(), b.float()) < 1e-2, seg
    # the whole states assembled from the per-scan blocks, against the oracle's entering states
    _, _, sent_r = OA.scan_twopass(*(t.detach() for t in ref), 64)
    assert rel(ops.wide_sent(res[NC][2]).float(), sent_r) < TOL_OUT


def test_wide_carrier_forward_backward():
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(60)
    g = torch.Generator().manual_seed(60)
    mod = AssocCarrier(256, head_dim=128)
    assert mod.h == 2 and mod.dk == 128
    _randomise(mod, g)
    mod = mod.cuda()
    x = torch.randn(2, 150, 256, generator=g)
    S0 = torch.randn(2, 2, 128, 128, generator=g) * 0.2
    wo = torch.randn(2, 150, 256, generator=g)
    wS = torch.randn(2, 2, 128, 128, generator=g)
    sd = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in _sd64(mod).items()}
    xr, S0r = x.double().requires_grad_(True), S0.double().requires_grad_(True)
    yr, (Sr, Tr) = M.assoc_carrier(sd, xr, (S0r, 77), heads=2)
    ((yr - xr) * wo.double()).sum().add((Sr * wS.double()).sum()).backward()
    xk, S0k = x.cuda().requires_grad_(True), S0.cuda().requires_grad_(True)
    yk, (Sk, Tk) = mod(xk, (S0k, 77))
    assert Tk == Tr == 150
    ((yk - xk) * wo.cuda()).sum().add((Sk * wS.cuda()).sum()).backward()
    assert rel(yk - xk, yr - xr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    assert rel(xk.grad, xr.grad) < TOL_GRAD and rel(S0k.grad, S0r.grad) < TOL_GRAD
    for blk, e in _block_errors(mod, sd).items():
        assert e < TOL_GRAD, (blk, e)


def test_wide_carrier_decode_step():
    """T = 1 without autograd: rebase by p0 (host int and device scalar), normalise, gate, write, read, in fp32,
    against the oracle's T = 1 call; the delta rule at head dim 128 (hdspin) likewise, on the exact fp32 scan."""
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(61)
    g = torch.Generator().manual_seed(61)
    mod = AssocCarrier(256, head_dim=128)
    _randomise(mod, g)
    mod = mod.cuda()
    sd = _sd64(mod)
    x = torch.randn(3, 1, 256, generator=g)
    S0 = torch.randn(3, 2, 128, 128, generator=g) * 0.2
    yr, (Sr, _) = M.assoc_carrier(sd, x.double(), (S0.double(), 33), heads=2)
    with torch.no_grad():
        yk, (Sk, Tk) = mod(x.cuda(), (S0.cuda(), 33))
        yd, (Sd, Td) = mod(x.cuda(), (S0.cuda(), torch.tensor(33.0, device="cuda")))
    assert Tk == 1 and float(Td) == 1.0
    assert rel(yk - x.cuda(), yr - x.double()) < 1e-4 and rel(Sk, Sr) < 1e-4
    assert rel(yd, yk) < 1e-6 and rel(Sd, Sk) < 1e-6
    mod_d = AssocCarrier(256, delta=True, head_dim=128)
    _randomise(mod_d, g)
    mod_d = mod_d.cuda()
    yr2, (Sr2, _) = M.assoc_carrier(_sd64(mod_d), x.double(), (S0.double(), 33), heads=2, delta=True)
    with torch.no_grad():
        yk2, (Sk2, _) = mod_d(x.cuda(), (S0.cuda(), 33))
    assert rel(yk2 - x.cuda(), yr2 - x.double()) < 1e-4 and rel(Sk2, Sr2) < 1e-4


def _lm_wide(seed):
    from pragnosia_amd.model import LM
    torch.manual_seed(seed)
    m = LM(vocab=300, d=256, layers=2, ctx=64, mixer="hspin")
    g = torch.Generator().manual_seed(seed)
    for mx in m.mix:
        _randomise(mx, g)
    with torch.no_grad():
        m.e.weight.mul_(20)
    return m.cuda().eval()


def test_wide_lm_forward_carried_and_graphed_decode():
    from pragnosia_amd.decode import GreedyDecoder, greedy_eager
    m = _lm_wide(62)
    sd = _sd64(m)
    g = torch.Generator().manual_seed(62)
    ids = torch.randint(0, 300, (2, 200), generator=g)
    with torch.no_grad():
        f = m(ids[:, :64].cuda())
        c = m.forward_carried(ids.cuda(), window=64)
    assert rel(f, M.lm_forward(sd, ids[:, :64], layers=2, mixer="hspin", heads=2)) < TOL_OUT
    assert rel(c, M.lm_forward_carried(sd, ids, 64, layers=2, mixer="hspin", heads=2)) < TOL_OUT
    prompt = ids[:, :100]
    dec = GreedyDecoder(m, 2, steps_per_graph=4)
    assert dec.fused  # the raw-output step at 128, the RMSNorm in the o-projection's GEMV
    toks_g = dec.generate(prompt.cuda(), 13)
    toks_u = GreedyDecoder(m, 2, steps_per_graph=4, fused=False).generate(prompt.cuda(), 13)
    toks_e, lgs_e = greedy_eager(m, prompt.cuda(), 13)
    assert torch.equal(toks_g.cpu(), toks_e.cpu()) and torch.equal(toks_u.cpu(), toks_e.cpu())
    _, lgs_r = M.greedy_decode(sd, prompt, 13, layers=2, mixer="hspin", heads=2, forced=toks_e.cpu())
    assert rel(lgs_e, lgs_r) < TOL_OUT


def test_wide_native_forward_full_shape():
    """The native 128-key forward (one workgroup per head and value half, the pair numbered 8 apart) at configs[2]'s
    width, B16 H6 T512 with an entering state, through the C ABI with whole-sequence segments: o, the final state and
    every entering state against the fp64 oracle (2e-2)."""
    from pragnosia_amd import ops
    from pragnosia_amd._lib import lib
    L = lib()
    B, H, T, D = 16, 6, 512, 128
    NC = T // 64
    q, k, v, la, S0, _, _ = _wide_inputs(B, H, T, 128)
    o_r, S_r, sent_r = OA.scan_twopass(*(t.double() for t in (q, k, v, la, S0)), 64)
    q, k, v, la, S0 = (t.cuda().contiguous() for t in (q, k, v, la, S0))
    o = torch.empty(B, H, T, D, device="cuda", dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device="cuda")
    sent = torch.empty(B, H, 4, NC, 64, 64, device="cuda", dtype=torch.bfloat16)
    ws = torch.empty(L.pragnosia_aspin_chunk_wide_workspace_bytes(B, H, T, D, 64, NC, 0), device="cuda",
                     dtype=torch.uint8)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    print(f"wide native fwd B{B} H{H} T{T}", flush=True)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.pragnosia_aspin_chunk_fwd_wide(P(q), P(k), P(v), P(la), P(S0), P(o), P(S), P(sent), P(ws), ws.numel(),
                                            B, H, T, D, 64, NC, st) == 0
    torch.cuda.synchronize()
    assert rel(o, o_r) < TOL_OUT and rel(S, S_r) < TOL_OUT
    assert rel(ops.wide_sent(sent).float(), sent_r) < TOL_OUT
