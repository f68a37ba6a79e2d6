"""GPU parity of the fused decode step: the batched dense-layer kernel (pragnosia_decode_gemv) against torch's
LayerNorm + Linear (+ GELU, + residual), the step kernel reading one projection GEMV's output
(pragnosia_aspin_decode_proj) against the module's own T = 1 path, and whole greedy generations of the fused graphed
decoder against the unfused one and the eager loop.

Everything is fp32, as the reference decodes. Tolerances: max relative error max|x - ref| / max|ref| <= 1e-5 for a
dense layer (fp32 sums in another order) and 1e-4 for a whole carrier layer step; generated tokens must be equal."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


@pytest.mark.parametrize("B", [1, 2, 3, 4, 5, 13, 64])
@pytest.mark.parametrize("K,N,ln,act,res", [(768, 2328, True, 0, False), (768, 768, False, 0, True),
                                            (768, 3072, True, 1, False), (3072, 768, False, 0, True),
                                            (128, 8192, True, 0, False), (1000, 300, True, 1, True),
                                            (4100, 200, False, 0, False), (768, 8192, True, 0, False),
                                            (512, 1025, True, 1, True), (1024, 4097, True, 0, False),
                                            (2048, 300, False, 1, True), (4096, 5000, False, 0, True)])
def test_decode_gemv_matches_torch(B, K, N, ln, act, res):
    import pragnosia_amd.ops  # noqa: F401
    g = torch.Generator(device="cuda").manual_seed(B + K + N)
    x = torch.randn(B, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * 0.05
    lw, lb = torch.randn(K, device="cuda", generator=g), torch.randn(K, device="cuda", generator=g)
    bias = torch.randn(N, device="cuda", generator=g) if act else None
    scale = torch.rand(1, device="cuda", generator=g) if res else None
    resid = torch.randn(B, N, device="cuda", generator=g) if res else None
    y = torch.ops.pragnosia.decode_gemv(x, W, lw if ln else None, lb if ln else None, 1e-5, bias, scale, act, resid)
    xd, Wd = x.double(), W.double()
    z = F.layer_norm(xd, (K,), lw.double(), lb.double(), 1e-5) if ln else xd
    r = z @ Wd.t()
    if scale is not None:
        r = r * scale.double()
    if bias is not None:
        r = r + bias.double()
    if act == 1:
        r = F.gelu(r)
    if resid is not None:
        r = r + resid.double()
    assert rel(y, r) < 1e-5


@pytest.mark.parametrize("delta,write_all,hl_floor", [(False, False, False), (False, True, True),
                                                      (True, False, False), (True, True, True)])
def test_decode_proj_matches_module_step(delta, write_all, hl_floor):
    """One carrier step through the projection GEMV + the fused step kernel against the module's T = 1 path (its
    projections, aspin_decode_step, nn.RMSNorm), from a rebased carried state, twice in a row (in-place state). Also
    the step with the o-projection in the same launch (aspin_decode_oproj_, state into the other of two buffers,
    output added into the residual with atomics): its new state bit-identical to the split step's (the raw-output
    aspin_decode_proj_: the same operations), its output within 1e-5 of the two-launch result (the heads summed in
    another order)."""
    from pragnosia_amd.assoc import AssocCarrier
    op = torch.ops.pragnosia
    torch.manual_seed(3)
    m = AssocCarrier(256, delta=delta, write_all=write_all, hl_floor=hl_floor).cuda().eval()
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.05)
        B = 3
        S = torch.randn(B, 4, 64, 64, device="cuda") * 0.1
        S_f, S_r = S.clone(), S.clone()
        S_o = [S.clone(), torch.full_like(S, float("nan"))]  # the one-launch form's two state buffers
        p0 = torch.tensor([7.0], device="cuda")
        gated = not (delta or write_all)
        extra = [m.wi.weight] if gated else ([m.wb.weight] if delta else [])
        W = torch.cat([m.q.weight, m.k.weight, m.v.weight, m.wa.weight] + extra)
        st = (S, 7)
        for step in range(2):
            x = torch.randn(B, 1, 256, device="cuda")
            y_mod, st = m(x, st)
            P = op.decode_gemv(x.reshape(B, 256), W, m.ln.weight, m.ln.bias, m.ln.eps, None, None, 0, None)
            o = op.aspin_decode_proj_(S_f, P, 4, m.wa.bias, m.A, m.la_floor if hl_floor else None,
                                      m.wi.bias if gated else None, m.wb.bias if delta else None,
                                      0.75 if (delta and write_all) else 0.0, gated, m.theta, p0, 0.0, m.on.weight,
                                      torch.finfo(torch.float32).eps)
            y_f = op.decode_gemv(o, m.o.weight, None, None, 0.0, None, torch.sigmoid(m.gate).reshape(1), 0,
                                 x.reshape(B, 256))
            # the raw output (four workgroups per head) with the RMSNorm in the o-projection's GEMV
            o_r = op.aspin_decode_proj_(S_r, P, 4, m.wa.bias, m.A, m.la_floor if hl_floor else None,
                                        m.wi.bias if gated else None, m.wb.bias if delta else None,
                                        0.75 if (delta and write_all) else 0.0, gated, m.theta, p0, 0.0, None,
                                        torch.finfo(torch.float32).eps)
            y_r = op.decode_gemv_rms(o_r, m.o.weight, m.on.weight, torch.finfo(torch.float32).eps, None,
                                     torch.sigmoid(m.gate).reshape(1), 0, x.reshape(B, 256))
            y_o = x.reshape(B, 256).clone()
            op.aspin_decode_oproj_(S_o[step % 2], S_o[1 - step % 2], P, 4, m.wa.bias, m.A,
                                   m.la_floor if hl_floor else None, m.wi.bias if gated else None,
                                   m.wb.bias if delta else None, 0.75 if (delta and write_all) else 0.0, gated,
                                   m.theta, p0, 0.0, m.on.weight, torch.finfo(torch.float32).eps, m.o.weight,
                                   torch.sigmoid(m.gate).reshape(1), y_o)
            p0.fill_(1.0)
            assert torch.equal(S_o[1 - step % 2], S_r), step
            assert rel(y_o - x.reshape(B, 256), y_f - x.reshape(B, 256)) < 1e-5, step
            assert rel(y_f - x.reshape(B, 256), y_mod.reshape(B, 256) - x.reshape(B, 256)) < 1e-4, step
            assert rel(S_f, st[0]) < 1e-4, step
            assert rel(y_r - x.reshape(B, 256), y_mod.reshape(B, 256) - x.reshape(B, 256)) < 1e-4, step
            assert rel(S_r, st[0]) < 1e-4, step


@pytest.mark.parametrize("delta,write_all", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dk,B", [(128, 2), (128, 40), (128, 80), (64, 40), (64, 80)])
def test_decode_proj_raw_matches_module_step(delta, write_all, dk, B):
    """The step with the raw output and its RMSNorm in the consumer (the o-projection's GEMV up to 4 sequences, else
    decode_gemm's 64- or 128-channel RMS mode with the weight folded in) against the module's own T = 1 path (its
    projections, the step, nn.RMSNorm), from a rebased carried state, twice in a row. d 512: at dk 128 the step runs
    split (B 2, 40: 8 or 160 heads) or one workgroup a head (B 80: 320 heads); at dk 64 one workgroup a head (320 and
    640 heads)."""
    from pragnosia_amd import ops
    from pragnosia_amd.assoc import AssocCarrier
    op = torch.ops.pragnosia
    torch.manual_seed(5)
    d = 512
    m = AssocCarrier(d, delta=delta, write_all=write_all, head_dim=dk).cuda().eval()
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.05)
        H = m.h
        S = torch.randn(B, H, dk, dk, device="cuda") * 0.1
        S_f = S.clone()
        p0 = torch.tensor([7.0], device="cuda")
        gated = not (delta or write_all)
        extra = [m.wi.weight] if gated else ([m.wb.weight] if delta else [])
        W = torch.cat([m.q.weight, m.k.weight, m.v.weight, m.wa.weight] + extra)
        eps = torch.finfo(torch.float32).eps
        sig = torch.sigmoid(m.gate).reshape(1)
        Wt = ops.decode_gemm_tile(m.o.weight, m.on.weight)
        st = (S, 7)
        for step in range(2):
            x = torch.randn(B, 1, d, device="cuda")
            y_mod, st = m(x, st)
            P = F.linear(F.layer_norm(x.reshape(B, d), (d,), m.ln.weight, m.ln.bias, m.ln.eps), W)
            o = op.aspin_decode_proj_(S_f, P, H, m.wa.bias, m.A, None, m.wi.bias if gated else None,
                                      m.wb.bias if delta else None, 0.75 if (delta and write_all) else 0.0, gated,
                                      m.theta, p0, 0.0, None, eps)
            if B <= 4:
                y = op.decode_gemv_rms(o, m.o.weight, m.on.weight, eps, None, sig, 0, x.reshape(B, d))
            else:
                y = op.decode_gemm(o, Wt, d, 2 if dk == 64 else 3, None, eps, None, sig, 0, x.reshape(B, d))
            p0.fill_(1.0)
            assert rel(y - x.reshape(B, d), y_mod.reshape(B, d) - x.reshape(B, d)) < 1e-4, step
            assert rel(S_f, st[0]) < 1e-4, step


@pytest.mark.parametrize("B", [1, 3, 4])
@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("K,N,bias,act", [(768, 768, False, 0), (512, 300, True, 1), (1024, 1500, True, 0)])
def test_decode_gemv_rms_matches_torch(B, K, N, bias, act, G):
    """The o-projection GEMV with the carrier's per-head (64-channel) RMSNorm on its input, against fp64 torch."""
    import pragnosia_amd.ops  # noqa: F401
    g = torch.Generator(device="cuda").manual_seed(B + K + N)
    x = torch.randn(B, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * 0.05
    w64 = 1 + 0.1 * torch.randn(G, device="cuda", generator=g)
    b = torch.randn(N, device="cuda", generator=g) if bias else None
    scale = torch.rand(1, device="cuda", generator=g)
    resid = torch.randn(B, N, device="cuda", generator=g)
    eps = torch.finfo(torch.float32).eps
    y = torch.ops.pragnosia.decode_gemv_rms(x, W, w64, eps, b, scale, act, resid)
    z = F.rms_norm(x.double().view(B, K // G, G), (G,), w64.double(), eps).view(B, K)
    r = (z @ W.double().t()) * scale.double()
    if b is not None:
        r = r + b.double()
    if act == 1:
        r = F.gelu(r)
    r = r + resid.double()
    assert rel(y, r) < 1e-5


@pytest.mark.parametrize("d,mixer", [(128, "aspin"), (128, "dspin"), (256, "aspin"), (256, "dspin"),
                                     (256, "hspin"), (256, "hdspin"), (512, "hspin1")])
@pytest.mark.parametrize("B", [1, 3, 40, 64])  # 1, 3: GEMV dense layers; 40, 64: decode_gemm or torch GEMMs
# (at 64 and d >= 256 the step runs one workgroup a head)
def test_fused_graphed_decode_equals_unfused_and_eager(mixer, B, d):
    """d 256 and 64-dim heads: the per-head RMSNorm inside the o-projection's GEMV at B <= 4; 128-dim heads (hspin,
    hdspin, hspin1): the raw-output step with the RMSNorm in the GEMV or in decode_gemm's 128-channel mode."""
    from pragnosia_amd.decode import GreedyDecoder, greedy_eager
    from pragnosia_amd.model import LM
    torch.manual_seed(50 + B)
    m = LM(vocab=300, d=d, layers=2, mlp_mult=2, ctx=64, mixer=mixer).cuda().eval()
    with torch.no_grad():
        for mx in m.mix:
            for p in mx.parameters():
                p.add_(torch.randn_like(p) * 0.05)
        m.e.weight.mul_(20)
    g = torch.Generator().manual_seed(51)
    prompt = torch.randint(0, 300, (B, 100), generator=g).cuda()
    n = 25
    fused = GreedyDecoder(m, B, steps_per_graph=4)
    assert fused.fused
    plain = GreedyDecoder(m, B, steps_per_graph=4, fused=False)
    t_f = fused.generate(prompt, n)
    t_p = plain.generate(prompt, n)
    t_e, _ = greedy_eager(m, prompt, n)
    assert torch.equal(t_f.cpu(), t_p.cpu()) and torch.equal(t_f.cpu(), t_e.cpu())
    # a second generation through the same captured graph, after a parameter change the copied weights must follow
    with torch.no_grad():
        m.mix[0].q.weight.mul_(1.5)
    t_f2 = fused.generate(prompt[:, :70], n)
    t_e2, _ = greedy_eager(m, prompt[:, :70], n)
    assert torch.equal(t_f2.cpu(), t_e2.cpu())


@pytest.mark.parametrize("B,V", [(1, 8192), (3, 1000), (64, 8192)])
def test_decode_tail_matches_torch(B, V):
    """The step tail kernel against torch: argmax with ties (the first index of the maximum), a NaN row (NaN above
    every number, as torch.argmax), the output row and token buffer, the next input embedding at the advanced and
    wrapped position, the counter and position written to their other slots, p0 reset, the recorded logits."""
    from pragnosia_amd.ops import decode_tail
    g = torch.Generator(device="cuda").manual_seed(B + V)
    d, ctx, n_rows, L = 96, 7, 5, 12
    lg = torch.randn(B, V, device="cuda", generator=g)
    lg[0, 10] = lg[0, 700] = lg[0].max() + 1.0  # a tie: index 10 must win
    if B > 1:
        lg[1, 333] = float("nan")
        lg[1, 900] = float("nan")
    emb = torch.randn(V, d, device="cuda", generator=g)
    pemb = torch.randn(ctx, d, device="cuda", generator=g)
    ctr = torch.tensor([3, -1], device="cuda")
    pos = torch.tensor([6, -1], device="cuda")
    out = torch.zeros(n_rows, B, dtype=torch.long, device="cuda")
    tok = torch.zeros(B, 1, dtype=torch.long, device="cuda")
    h = torch.zeros(B, d, device="cuda")
    p0s = torch.zeros(L, device="cuda")
    rec = torch.zeros(n_rows, B, V, device="cuda")
    decode_tail(lg, emb, pemb, ctr[0], ctr[1], pos[0], pos[1], out, tok, h, p0s, rec)
    want = lg.argmax(-1)
    assert torch.equal(tok.view(-1), want) and torch.equal(out[3], want)
    assert int(want[0]) == 10 and (B == 1 or int(want[1]) == 333)
    assert int(ctr[1]) == 4 and int(pos[1]) == 0 and int(ctr[0]) == 3 and int(pos[0]) == 6
    assert torch.equal(h, emb[want] + pemb[0])
    assert bool((p0s == 1).all()) and int(out[[0, 1, 2, 4]].abs().sum()) == 0
    assert torch.allclose(rec[3], lg, rtol=0, atol=0, equal_nan=True)  # the NaN row copied as is
    # the counter past the buffer's rows: nothing is written there
    ctr[0] = n_rows
    decode_tail(lg, emb, pemb, ctr[0], ctr[1], pos[1], pos[0], out, tok, h, None, None)
    assert int(ctr[1]) == n_rows + 1 and int(pos[0]) == 1 and torch.equal(out[3], want)


@pytest.mark.parametrize("B", [1, 3, 4])
@pytest.mark.parametrize("K,N", [(3072, 768), (2816, 704), (1024, 300), (256, 64), (4096, 100)])
def test_decode_gemv_acc_adds_into_residual(B, K, N):
    """decode_gemv_acc_ (y += scale * W x + bias in place, K split over one-wave workgroups adding with atomics)
    against fp64 torch at 1e-5 (3072: two splits of 1536; 2816: one; 1024: one; 4096: two of 2048)."""
    g = torch.Generator(device="cuda").manual_seed(B + K + N)
    x = torch.randn(B, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * 0.05
    bias = torch.randn(N, device="cuda", generator=g)
    scale = torch.rand(1, device="cuda", generator=g)
    resid = torch.randn(B, N, device="cuda", generator=g)
    y = resid.clone()
    torch.ops.pragnosia.decode_gemv_acc_(x, W, bias, scale, y)
    ref = resid.double() + scale.double() * (x.double() @ W.double().t()) + bias.double()
    assert rel(y, ref) < 1e-5, (B, K, N)
    y2 = resid.clone()
    torch.ops.pragnosia.decode_gemv_acc_(x, W, None, None, y2)
    assert rel(y2, resid.double() + x.double() @ W.double().t()) < 1e-5
