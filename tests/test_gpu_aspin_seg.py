"""GPU parity of the segment-parallel plain forward (pragnosia_aspin_chunk_fwd_seg through the C ABI) and of the
windowed carried scan built on it, against the CPU oracle and against the one-workgroup-per-head kernel.

The segmented forward computes each segment's entering state from per-segment sums instead of walking the chunks in
order, so it agrees with the sequential kernel to rounding, not bit for bit. Tolerances are the plain rule's: max
relative error max|x - ref| / max|ref| <= 2e-2 on outputs, entering states and the final state against the fp64
oracle; against the sequential kernel the same bound holds (both are within it of the oracle)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as O

pytestmark = pytest.mark.gpu
TOL_OUT = 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _inputs(B, H, T, seed, s0=True, la_scale=0.02):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, H, T, 64, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, H, T, 64, generator=g), dim=-1)
    v = torch.randn(B, H, T, 64, generator=g)
    la = -F.softplus(torch.randn(B, H, T, generator=g)) * la_scale
    S0 = torch.randn(B, H, 64, 64, generator=g) * 0.1 if s0 else None
    return q, k, v, la, S0


def _seg_forward(q, k, v, la, S0, P, theta=None, window=0):
    """The segmented forward with segments of P chunks, called directly (no policy)."""
    from pragnosia_amd import ops
    q, k, v = (t.cuda().bfloat16().contiguous() for t in (q, k, v))
    la = la.cuda().float().contiguous()
    S0 = None if S0 is None else S0.cuda().float().contiguous()
    th = None if theta is None else theta.cuda().float().contiguous()
    B, H, T, D = q.shape
    NC = (T + 63) // 64
    o = torch.empty(B, H, T, D, device="cuda", dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device="cuda")
    sent = torch.empty(B, H, NC, D, D, device="cuda", dtype=torch.bfloat16)
    ops._aspin_fwd_seg(q, k, v, la, S0, th, window, o, S, sent, P)
    return o, S, sent


def _sequential_forward(q, k, v, la, S0):
    """The one-workgroup-per-head kernel, called through the C ABI directly."""
    from pragnosia_amd._lib import check, lib
    from pragnosia_amd.ops import _ptr, _stream
    q, k, v = (t.cuda().bfloat16().contiguous() for t in (q, k, v))
    la = la.cuda().float().contiguous()
    S0 = None if S0 is None else S0.cuda().float().contiguous()
    B, H, T, D = q.shape
    NC = (T + 63) // 64
    o = torch.empty(B, H, T, D, device="cuda", dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device="cuda")
    sent = torch.empty(B, H, NC, D, D, device="cuda", dtype=torch.bfloat16)
    check(lib().pragnosia_aspin_chunk_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(S0), _ptr(o), _ptr(S), _ptr(sent),
                                          B, H, T, D, 64, _stream(q)), "pragnosia_aspin_chunk_fwd")
    return o, S, sent


def _oracle(q, k, v, la, S0):
    """fp64 two-pass form: outputs, final state and the state entering every chunk."""
    B, H, T, D = q.shape
    r = [t.double() for t in (q.bfloat16(), k.bfloat16(), v.bfloat16(), la)]
    S = torch.zeros(B, H, D, D, dtype=torch.float64) if S0 is None else S0.double()
    return O.scan_twopass(*r, S, 64, None)


@pytest.mark.parametrize("B,H,T,P", [(1, 2, 70 * 64 - 17, 8), (1, 2, 70 * 64 - 17, 1), (2, 3, 333, 2),
                                     (2, 3, 333, 5), (1, 1, 64 * 9, 4), (3, 1, 64 * 9, 9), (1, 2, 40, 1)])
def test_segmented_matches_oracle_and_sequential(B, H, T, P):
    """Segments of P chunks (ragged last segment and last chunk, P = 1, P = NC, a single short chunk) with and
    without an initial state: o, the final state and every chunk's entering state against the oracle and against
    the sequential kernel."""
    for s0 in (True, False):
        q, k, v, la, S0 = _inputs(B, H, T, seed=T + P + s0, s0=s0)
        with torch.no_grad():
            o, S, sent = _seg_forward(q, k, v, la, S0, P)
            o1, S1, sent1 = _sequential_forward(q, k, v, la, S0)
        yr, Sr, Sent = _oracle(q, k, v, la, S0)
        errs = {"o": rel(o, yr), "S": rel(S, Sr), "sent": rel(sent.float(), Sent),
                "o_vs_seq": rel(o, o1), "S_vs_seq": rel(S, S1), "sent_vs_seq": rel(sent.float(), sent1.float())}
        assert max(errs.values()) < TOL_OUT, errs


def test_segmented_deterministic_and_long_decay():
    """Repeated calls agree bit for bit; with strong decay (most of a segment's tokens decayed to nothing by its
    end) the segment sums stay finite and the result still matches the oracle."""
    q, k, v, la, S0 = _inputs(2, 2, 64 * 24 + 5, seed=3, la_scale=2.0)
    with torch.no_grad():
        a = _seg_forward(q, k, v, la, S0, 3)
        b = _seg_forward(q, k, v, la, S0, 3)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert all(torch.isfinite(t.float()).all() for t in a)
    yr, Sr, _ = _oracle(q, k, v, la, S0)
    assert rel(a[0], yr) < TOL_OUT and rel(a[1], Sr) < TOL_OUT


def test_policy_routes_few_heads_to_segments():
    """aspin_chunk (the autograd op) uses the segmented forward for few heads over many chunks and keeps the
    sequential kernel for configs[2]'s 192 heads x 8 chunks; either way its forward and backward match the
    oracle (the backward reads the segmented forward's entering states)."""
    from pragnosia_amd.ops import seg_chunks
    assert seg_chunks(192, 8, range(1, 9)) == 8
    assert seg_chunks(2, 70, range(1, 71)) < 70
    from pragnosia_amd.assoc import assoc_scan_kernel
    q, k, v, la, S0 = _inputs(1, 2, 70 * 64 - 17, seed=9, la_scale=0.01)
    g = torch.Generator().manual_seed(10)
    wo = torch.randn(q.shape, generator=g)
    r = [t.double().requires_grad_(True) for t in (q.bfloat16(), k.bfloat16(), v.bfloat16(), la, S0)]
    yr, Sr = O.assoc_scan(*r, chunk=64)
    ((yr * wo.double()).sum() + Sr.sum()).backward()
    kk = [t.cuda().requires_grad_(True) for t in (q, k, v, la, S0)]
    yk, Sk, _ = assoc_scan_kernel(*kk)
    ((yk.float() * wo.cuda()).sum() + Sk.sum()).backward()
    assert rel(yk, yr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    for a, b in zip(kk, r):
        assert rel(a.grad, b.grad) < 5e-2


def _bwd(q, k, v, la, sent, do, dS, P):
    """The backward through the C ABI: sequential kernel (P = None) or segments of P chunks."""
    from pragnosia_amd import ops
    from pragnosia_amd._lib import check, lib
    from pragnosia_amd.ops import _ptr, _stream
    B, H, T, D = q.shape
    dq, dk, dv = (torch.empty(B, H, T, D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    dla = torch.empty(B, H, T, device="cuda")
    dS0 = torch.empty(B, H, D, D, device="cuda")
    if P is None:
        check(lib().pragnosia_aspin_chunk_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(sent), _ptr(do), _ptr(dS),
                                              _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla), _ptr(dS0), B, H, T, D, 64,
                                              _stream(q)), "pragnosia_aspin_chunk_bwd")
    else:
        ops._aspin_bwd_seg(q, k, v, la, sent, do, dS, dq, dk, dv, dla, dS0, P)
    return dq, dk, dv, dla, dS0


@pytest.mark.parametrize("B,H,T,P", [(1, 2, 70 * 64 - 17, 8), (1, 2, 70 * 64 - 17, 1), (2, 3, 333, 2),
                                     (1, 1, 64 * 9, 4), (3, 1, 64 * 9, 9), (1, 2, 40, 1)])
def test_segmented_backward_matches_oracle_and_sequential(B, H, T, P):
    """Every gradient (q, k, v, la, S0) of the segmented backward, with and without an upstream gradient on the
    final state, against the fp64 oracle's autograd and against the sequential backward on the same saved states."""
    for with_dS in (True, False):
        q, k, v, la, S0 = _inputs(B, H, T, seed=3 * T + P + with_dS)
        g = torch.Generator().manual_seed(T + P)
        wo = torch.randn(q.shape, generator=g)
        wS = torch.randn(B, H, 64, 64, generator=g) if with_dS else None
        r = [t.double().requires_grad_(True) for t in (q.bfloat16(), k.bfloat16(), v.bfloat16(), la, S0)]
        yr, Sr = O.assoc_scan(*r, chunk=64)
        ((yr * wo.double()).sum() + ((Sr * wS.double()).sum() if with_dS else 0)).backward()
        with torch.no_grad():
            dev = [t.cuda().bfloat16().contiguous() for t in (q, k, v)] + [la.cuda(), S0.cuda()]
            _, _, sent = _sequential_forward(q, k, v, la, S0)
            do = wo.cuda().bfloat16().contiguous()
            dS = wS.cuda() if with_dS else None
            seg = _bwd(*dev[:4], sent, do, dS, P)
            seq = _bwd(*dev[:4], sent, do, dS, None)
        errs = {}
        for n, a, b, c in zip(("dq", "dk", "dv", "dla", "dS0"), seg, seq, r):
            errs[n] = rel(a, c.grad)
            errs[n + "_vs_seq"] = rel(a, b)
        assert max(errs.values()) < 5e-2, errs


def _window_loop_oracle(q, k, v, la, S0, theta, W):
    """The reference's carried windows on the oracle: one two-pass scan per window, the state rebased by -W theta
    between windows (q and k already rotated with positions restarting per window)."""
    B, H, T, D = q.shape
    S = torch.zeros(B, H, D, D, dtype=torch.float64) if S0 is None else S0.double()
    outs = []
    for s in range(0, T, W):
        if s:
            S = O.rebase(S, theta.double(), W)
        sl = slice(s, s + W)
        o, S, _ = O.scan_twopass(*[t[:, :, sl].double() for t in (q.bfloat16(), k.bfloat16(), v.bfloat16())],
                                 la[:, :, sl].double(), S, 64, None)
        outs.append(o)
    return torch.cat(outs, 2), S


@pytest.mark.parametrize("B,H,T,W", [(2, 3, 64 * 10 + 7, 128), (1, 2, 64 * 12, 192), (1, 1, 300, 64),
                                     (2, 2, 100, 128)])
def test_windows_match_window_loop(B, H, T, W):
    """aspin_chunk_windows against the oracle's window-by-window scan with rebases, and against this build's own
    window loop (aspin_chunk per window, aspin_rebase between); q and k rotated with per-window positions."""
    g = torch.Generator().manual_seed(T + W)
    q, k, v, la, S0 = _inputs(B, H, T, seed=T + W)
    theta = torch.rand(H, 32, generator=g) * 0.2
    pos = torch.arange(T) % W
    q, k = O.rotate(q, theta, pos), O.rotate(k, theta, pos)
    yr, Sr = _window_loop_oracle(q, k, v, la, S0, theta, W)
    op = torch.ops.pragnosia
    dev = [t.cuda() for t in (q, k, v, la, S0, theta)]
    with torch.no_grad():
        o, S, sent = op.aspin_chunk_windows(*dev, W, True)
        St, outs = dev[4], []
        for s in range(0, T, W):
            if s:
                St = op.aspin_rebase(St, dev[5], None, float(W))
            ow, St, _ = op.aspin_chunk(*(t[:, :, s:s + W] for t in dev[:4]), St, False)
            outs.append(ow)
    errs = {"o": rel(o, yr), "S": rel(S, Sr), "o_vs_loop": rel(o, torch.cat(outs, 2)), "S_vs_loop": rel(S, St)}
    assert max(errs.values()) < TOL_OUT, errs
    assert sent.shape[2] == (T + 63) // 64 and torch.isfinite(sent.float()).all()


@pytest.mark.parametrize("delta", [False, True])
def test_windows_carrier_module_matches_window_calls(delta):
    """AssocCarrier.forward_windows (one pass; the delta rule from the windows' affine state maps, its ragged last
    window zero-padded) against calling forward on each window with the carried state."""
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(12)
    m = AssocCarrier(128, delta=delta).cuda().eval()
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.05)
        x = torch.randn(2, 64 * 7 + 9, 128, device="cuda")
        S0 = torch.randn(2, 2, 64, 64, device="cuda") * 0.1
        y, (S, last) = m.forward_windows(x, 128, (S0, 40))
        outs, st = [], (S0, 40)
        for s in range(0, x.shape[1], 128):
            o, st = m(x[:, s:s + 128], st)
            outs.append(o)
    assert last == st[1] == 64 * 7 + 9 - 3 * 128
    assert rel(y - x, torch.cat(outs, 1) - x) < TOL_OUT and rel(S, st[0]) < TOL_OUT
