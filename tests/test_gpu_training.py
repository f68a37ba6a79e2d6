"""Training integration on the GPU: every `pragnosia::*` op passes torch.library.opcheck (schema, autograd
registration, fake tensors, AOT dispatch with dynamic shapes), the LM's trunk traces whole under torch.compile and
matches eager, and a bf16-autocast forward + loss + backward micro-step captured in a HIP graph replays equal to
eager, as the reference's trainer captures it (`src/train.py:352`, `:494-517`).

torch.compile runs with the "aot_eager" backend: dynamo's graph capture, fake-tensor propagation through the ops'
fake implementations and AOT autograd (what the reference's trainer needs from the ops), executed eagerly, so no
code is generated around the HIP kernels."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _samples():
    """(op name, args) for every op, small shapes, on cuda; differentiable inputs require grad."""
    dev = "cuda"
    g = torch.Generator().manual_seed(0)
    r = lambda *s, dt=torch.float32, grad=False: torch.randn(*s, generator=g).to(dev, dt).requires_grad_(grad)
    B, H, T, D = 2, 2, 70, 64
    NC = (T + 63) // 64
    q, k, v = (F.normalize(r(B, H, T, D), dim=-1).bfloat16().requires_grad_(True) for _ in range(3))
    la = F.logsigmoid(r(B, H, T) + 3).requires_grad_(True)
    be = torch.sigmoid(r(B, H, T)).requires_grad_(True)
    S0 = (r(B, H, D, D) * 0.1).requires_grad_(True)
    th = (torch.rand(H, 32, generator=g) * 0.1).to(dev)
    pos = torch.arange(T, device=dev)
    op = torch.ops.pragnosia
    with torch.no_grad():
        _, _, sent = op.aspin_chunk(q, k, v, la, S0, True)
        _, _, sentd, W, X = op.aspin_delta(q, k, v, la, be, S0, True)
        o32 = r(B, H, T, D)
        _, _, ck, rs = op.aspin_exact(o32, o32, o32, la, be, S0, True)
    u, lm_, an = r(B, T, 40, grad=True), (F.logsigmoid(r(B, T, 40) + 4)).requires_grad_(True), r(B, T, 40, grad=True)
    h0r, h0i = r(B, 40, grad=True), r(B, 40, grad=True)
    with torch.no_grad():
        hr, _, _, hi = op.diag_scan(u, lm_, an, h0r, h0i)
    P = r(B, T, 3 * H * D + 2 * H, grad=True)
    qp, kp, vp = (r(B, T, H, D, grad=True) for _ in range(3))
    gate = r(B, T, H, grad=True)
    bias_h, A = r(H, grad=True), r(H, grad=True)
    wrms = (1 + 0.1 * r(64)).requires_grad_(True)
    ob = r(B, H, T, D).bfloat16().requires_grad_(True)
    with torch.no_grad():
        _, rstd = op.aspin_out(ob, wrms, 1e-6, True)
    x = r(3, 96)
    qw, kw, vw = (F.normalize(r(B, 1, T, 128), dim=-1).bfloat16().requires_grad_(True) for _ in range(3))
    law = F.logsigmoid(r(B, 1, T) + 3).requires_grad_(True)
    S0w = (r(B, 1, 128, 128) * 0.1).requires_grad_(True)
    bew = torch.sigmoid(r(B, 1, T)).requires_grad_(True)
    with torch.no_grad():
        _, _, sentw = op.aspin_chunk_wide(qw, kw, vw, law, S0w, True)
        _, _, sentdw, Ww, Xw = op.aspin_delta(qw, kw, vw, law, bew, S0w, True)
    xl = r(3, 40, 768, grad=True)
    wl, bl = (1 + 0.1 * r(768)).requires_grad_(True), (0.1 * r(768)).requires_grad_(True)
    with torch.no_grad():
        _, ml, rl = op.layer_norm(xl, wl, bl, 1e-5, True)
    return [
        ("wgrad", (r(200, 24).bfloat16(), r(200, 40).bfloat16())),
        ("layer_norm", (xl, wl, bl, 1e-5, True)),
        ("layer_norm", (xl, wl, bl, 1e-5, False)),
        ("layer_norm_bwd", (r(3, 40, 768).bfloat16(), xl.detach(), wl.detach(), ml, rl)),
        ("aspin_delta", (qw, kw, vw, law, bew, S0w, True)),
        ("aspin_delta_fused", (qw, kw, vw, law, bew, S0w)),
        ("aspin_delta_bwd", (qw.detach(), kw.detach(), vw.detach(), law.detach(), bew.detach(), sentdw, Ww, Xw,
                             r(B, 1, T, 128).bfloat16(), r(B, 1, 128, 128))),
        ("aspin_chunk_wide", (qw, kw, vw, law, S0w, True)),
        ("aspin_chunk_wide_bwd", (qw.detach(), kw.detach(), vw.detach(), law.detach(), sentw,
                                  r(B, 1, T, 128).bfloat16(), r(B, 1, 128, 128))),
        ("diag_scan", (u, lm_, an, h0r, h0i)),
        ("diag_scan_bwd", (r(B, T, 40), r(B, 40), r(B, 40), lm_.detach(), an.detach(), hr, hi, h0r.detach(),
                           h0i.detach())),
        ("aspin_out", (ob, wrms, 1e-6, True)),
        ("aspin_out_bwd", (r(B, T, H * D).bfloat16(), ob.detach(), wrms.detach(), rstd)),
        ("aspin_chunk", (q, k, v, la, S0, True)),
        ("aspin_chunk_windows", (q.detach(), k.detach(), v.detach(), la.detach(), S0.detach(), th, 64, False)),
        ("aspin_chunk_bwd", (q.detach(), k.detach(), v.detach(), la.detach(), sent, r(B, H, T, D).bfloat16(),
                             r(B, H, D, D))),
        ("aspin_delta", (q, k, v, la, be, S0, True)),
        ("aspin_delta_bwd", (q.detach(), k.detach(), v.detach(), la.detach(), be.detach(), sentd, W, X,
                             r(B, H, T, D).bfloat16(), r(B, H, D, D))),
        ("aspin_exact", (o32.clone().requires_grad_(True), o32.clone().requires_grad_(True),
                         o32.clone().requires_grad_(True), la, be, S0, True)),
        ("aspin_exact_bwd", (o32, o32, o32, la.detach(), be.detach(), ck, rs, r(B, H, T, D), r(B, H, D, D))),
        ("aspin_prep", (qp, kp, vp, gate, th.clone().requires_grad_(True), pos)),
        ("aspin_prep_bwd", (qp.detach(), kp.detach(), vp.detach(), gate.detach(), th, pos,
                            r(B, H, T, D).bfloat16(), r(B, H, T, D).bfloat16(), r(B, H, T, D).bfloat16())),
        ("aspin_prep_proj", (P, H, bias_h, A, None, None, r(H), 0.0, False, th.clone().requires_grad_(True), pos)),
        ("aspin_prep_proj_bwd", (P.detach(), H, bias_h.detach(), A.detach(), None, r(H), None, 0.0, True, th, pos,
                                 r(B, H, T, D).bfloat16(), r(B, H, T, D).bfloat16(), r(B, H, T, D).bfloat16(),
                                 r(B, H, T), None)),
        ("aspin_rebase", (S0, th.clone().requires_grad_(True), None, 17.0)),
        ("aspin_rebase_bwd", (S0.detach(), th, None, 17.0, r(B, H, D, D))),
        ("aspin_decode_step", (r(B, H, D, D), r(B, H, D), r(B, H, D), r(B, H, D), r(B, H), la[:, :, 0].detach(),
                               None, th, torch.tensor(3.0, device=dev), 0.0)),
        ("decode_gemv", (x, r(50, 96), 1 + 0.1 * r(96), r(96), 1e-5, r(50), r(1), 1, r(3, 50))),
        ("aspin_decode_proj_", (r(B, H, D, D), r(B, 3 * H * D + 2 * H), H, r(H), r(H), None, r(H), None, 0.0, True,
                                th, torch.tensor(1.0, device=dev), 0.0, 1 + 0.1 * r(64), 1e-6)),
        ("aspin_decode_proj_", (r(B, H, D, D), r(B, 3 * H * D + 2 * H), H, r(H), r(H), None, r(H), None, 0.0, True,
                                th, torch.tensor(1.0, device=dev), 0.0, None, 1e-6)),
        ("aspin_decode_oproj_", (r(B, H, D, D), r(B, H, D, D), r(B, 3 * H * D + 2 * H), H, r(H), r(H), None, r(H),
                                 None, 0.0, True, th, torch.tensor(1.0, device=dev), 0.0, 1 + 0.1 * r(64), 1e-6,
                                 r(100, H * D), r(1), r(B, 100))),
        ("decode_gemv_rms", (r(3, 256), r(50, 256), 1 + 0.1 * r(64), 1e-6, r(50), r(1), 1, r(3, 50))),
        ("decode_gemm", (r(20, 256), r(64 * 256), 50, 1, r(50), 1e-5, r(50), None, 1, r(20, 50))),
        ("decode_gemm", (r(20, 256), r(64 * 256), 50, 2, None, 1e-6, None, r(1), 0, None)),
        ("decode_gemm_acc_", (r(20, 1024), r(64 * 1024), 0, 0.0, r(50), r(1), r(20, 50))),   # two K splits of 512
        ("decode_gemv_acc_", (r(2, 1536), r(50, 1536), r(50), r(1), r(2, 50))),   # two K splits of 768
        ("decode_gemm_acc_", (r(20, 768), r(64 * 768), 2, 1e-6, None, r(1), r(20, 50))),     # three splits of 4 heads
        ("aspin_delta_windows", (q.detach(), k.detach(), v.detach(), la.detach(), be.detach(), S0.detach(), th, 64)),
    ]


def test_every_op_passes_opcheck():
    from pragnosia_amd import ops  # noqa: F401
    registered = {n for n in dir(torch.ops.pragnosia) if not n.startswith("_") and
                  isinstance(getattr(torch.ops.pragnosia, n), torch._ops.OpOverloadPacket)}
    samples = _samples()
    assert {n for n, _ in samples} == registered
    for name, args in samples:
        print(f"opcheck {name}", flush=True)
        torch.library.opcheck(getattr(torch.ops.pragnosia, name), args)


def _lm(mixer, seed):
    from pragnosia_amd.model import LM
    torch.manual_seed(seed)
    m = LM(vocab=512, d=128, layers=2, mlp_mult=4, ctx=128, mixer=mixer).cuda()
    with torch.no_grad():
        m.e.weight.mul_(10)
    return m


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_compiled_trunk_matches_eager(mixer):
    """torch.compile(m.trunk) (`src/train.py:352`) traces the whole trunk as one graph (fullgraph) under bf16
    autocast, and its output and parameter gradients equal the eager trunk's to bf16 rounding (AOT autograd
    re-derives the backward of the torch ops around the kernels, so bf16 sums may round differently: 1e-3 on the
    output, 1e-2 on each gradient; the kernels' own outputs are bit-identical)."""
    torch._dynamo.reset()
    m = _lm(mixer, 90)
    g = torch.Generator().manual_seed(91)
    ids = torch.randint(0, 512, (2, 129), generator=g).cuda()
    trunk = torch.compile(m.trunk, backend="aot_eager", fullgraph=True)

    def step(fn):
        for p in m.parameters():
            p.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            h = fn(ids[:, :128])
        loss = m.loss(h.float(), ids[:, 1:])
        loss.backward()
        return h.detach(), loss.detach(), [None if p.grad is None else p.grad.detach().clone()
                                           for p in m.parameters()]

    he, le, ge = step(m.trunk)
    hc, lc, gc = step(trunk)
    assert rel(hc, he) < 1e-3 and abs(lc.item() - le.item()) < 1e-3
    for (name, _), a, b in zip(m.named_parameters(), gc, ge):
        assert (a is None) == (b is None), name
        if a is not None:
            assert rel(a, b) < 1e-2, (name, rel(a, b))


def _memset_nodes(graph) -> int:
    """Memset nodes in a captured graph (hipGraphNodeTypeMemset = 2), through the HIP runtime."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    hip.hipGraphNodeGetType.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    gr, n = ctypes.c_void_p(graph.raw_cuda_graph()), ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(gr, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(gr, nodes, ctypes.byref(n)) == 0 and n.value > 0
    count = 0
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) == 0
        count += t.value == 2
    return count


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_graph_captured_training_micro_step(mixer):
    """The reference trainer's captured micro-step (`src/train.py:494-517`): bf16 autocast trunk forward, loss,
    backward, warmed on a side stream, then captured into one HIP graph over a static input buffer. The graph holds
    no memset node (torch's multi-block column sums record one; the modules form their bias gradients as GEMMs,
    `ops.linear`, and the ops their partial sums, `ops.colsum`). Three replays on new batches, with eager work and
    synchronisations between them, each against the eager micro-step on the same batch: loss and every parameter
    gradient."""
    m = _lm(mixer, 92)
    B, T = 4, 128
    xs = torch.zeros(B, T + 1, dtype=torch.long, device="cuda")
    for p in m.parameters():
        p.grad = torch.zeros_like(p)
    out = {}

    def micro():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            h = m.trunk(xs[:, :T])
        loss = m.loss(h.float(), xs[:, 1:T + 1])
        loss.backward()
        out["loss"] = loss.detach()

    g = torch.Generator().manual_seed(93)
    xs.copy_(torch.randint(0, 512, (B, T + 1), generator=g))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            micro()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    for p in m.parameters():
        p.grad.zero_()
    with torch.cuda.graph(graph):
        micro()
    assert _memset_nodes(graph) == 0
    loss_static = out["loss"]
    for it in range(3):
        batch = torch.randint(0, 512, (B, T + 1), generator=g)
        for p in m.parameters():
            p.grad.zero_()
        xs.copy_(batch)
        graph.replay()
        torch.cuda.synchronize()
        lg, gg = loss_static.clone(), [p.grad.clone() for p in m.parameters()]
        for p in m.parameters():
            p.grad.zero_()
        micro()                      # eager on the same batch
        torch.cuda.synchronize()
        assert abs(lg.item() - out["loss"].item()) < 1e-5 * max(1.0, abs(out["loss"].item())), it
        for a, p in zip(gg, m.parameters()):
            assert rel(a, p.grad) < 1e-4, (it, rel(a, p.grad))
