"""GPU checks at the full sizes of BASELINE.json configs[3] (carried long context) and configs[4] (78M-class LM
decode), against the CPU oracle (fp32) and against size-independent properties.

Tolerance: max relative error <= 2e-2 (bf16-input scan path) on outputs, logits and the carried state."""
import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as OA
from oracle import modules as M

pytestmark = pytest.mark.gpu
TOL = 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def test_cfg3_carried_windows_equal_unsplit_pass():
    """B2 T8192 H12 D64, la = logsigmoid(N(4,1)) so memory spans far. (i) 16 windows of 512, positions
    restarting per window, the fp32 state carried and rebased by -512 theta between windows; (ii) one T = 8192 pass
    with global positions. Both on the GPU, and (ii) against the fp32 oracle. The carried final state is expressed
    in the last window's positions, so the unsplit one is rebased by -(8192 - 512) theta before comparing."""
    from pragnosia_amd import ops  # noqa: F401
    from pragnosia_amd.assoc import rotate
    B, H, T, D, W = 2, 12, 8192, 64, 512
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 4.0)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    op = torch.ops.pragnosia
    qd, kd, vd, lad, thd = (t.cuda() for t in (q, k, v, la, th))
    loc = torch.arange(T, device="cuda") % W
    glob = torch.arange(T, device="cuda")
    qw, kw = rotate(qd, thd, loc).bfloat16(), rotate(kd, thd, loc).bfloat16()
    qg, kg = rotate(qd, thd, glob).bfloat16(), rotate(kd, thd, glob).bfloat16()
    vb = vd.bfloat16()
    with torch.no_grad():
        S, outs = None, []
        for s in range(0, T, W):
            if S is not None:
                S = op.aspin_rebase(S, thd, None, float(W))
            o, S, _ = op.aspin_chunk(qw[:, :, s:s + W], kw[:, :, s:s + W], vb[:, :, s:s + W], lad[:, :, s:s + W],
                                     S, False)
            outs.append(o)
        oc = torch.cat(outs, 2)
        ou, Su, _ = op.aspin_chunk(qg, kg, vb, lad, None, False)
        Su_loc = op.aspin_rebase(Su, thd, None, float(T - W))
    assert rel(oc, ou) < TOL and rel(S, Su_loc) < TOL
    # the unsplit pass against the oracle on the same bf16 inputs
    o_r, S_r = OA.assoc_scan(qg.float().cpu(), kg.float().cpu(), vb.float().cpu(), la, None, chunk=64)
    assert rel(ou, o_r) < TOL and rel(Su, S_r) < TOL
    assert torch.isfinite(S).all()


def test_cfg3_one_pass_windows_full_size():
    """configs[3] through the path `LM.forward_carried` and bench.py time: `aspin_chunk_windows`, the 16 windows of
    512 carried in ONE segment-parallel pass (state rebased by -512 theta at every window boundary inside the
    kernels). Against (i) the window-by-window loop on the GPU (aspin_chunk + aspin_rebase per window) and (ii) the
    CPU oracle's window loop (`oracle.aspin.assoc_scan` per window, `oracle.aspin.rebase` between), outputs and the
    final state, on the same bf16 inputs."""
    from pragnosia_amd import ops  # noqa: F401
    from pragnosia_amd.assoc import rotate
    B, H, T, D, W = 2, 12, 8192, 64, 512
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 4.0)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    op = torch.ops.pragnosia
    qd, kd, vd, lad, thd = (t.cuda() for t in (q, k, v, la, th))
    loc = torch.arange(T, device="cuda") % W
    qw, kw, vb = rotate(qd, thd, loc).bfloat16(), rotate(kd, thd, loc).bfloat16(), vd.bfloat16()
    with torch.no_grad():
        o1, S1, _ = op.aspin_chunk_windows(qw, kw, vb, lad, None, thd, W, False)
        S, outs = None, []
        for s in range(0, T, W):
            if S is not None:
                S = op.aspin_rebase(S, thd, None, float(W))
            o, S, _ = op.aspin_chunk(qw[:, :, s:s + W], kw[:, :, s:s + W], vb[:, :, s:s + W], lad[:, :, s:s + W],
                                     S, False)
            outs.append(o)
        oloop = torch.cat(outs, 2)
    torch.cuda.synchronize()
    assert rel(o1, oloop) < TOL and rel(S1, S) < TOL
    qc, kc, vc = qw.float().cpu(), kw.float().cpu(), vb.float().cpu()
    Sr, outs = None, []
    for s in range(0, T, W):
        if Sr is not None:
            Sr = OA.rebase(Sr, th, float(W))
        o, Sr = OA.assoc_scan(qc[:, :, s:s + W], kc[:, :, s:s + W], vc[:, :, s:s + W], la[:, :, s:s + W], Sr, chunk=64)
        outs.append(o)
    o_r = torch.cat(outs, 2)
    assert rel(o1, o_r) < TOL and rel(S1, Sr) < TOL
    print(f"cfg3 one pass vs loop {rel(o1, oloop):.2e}, vs oracle out {rel(o1, o_r):.2e} state {rel(S1, Sr):.2e}")


def test_cfg3_delta_windows_full_size():
    """configs[3]'s shape with the delta write rule (beta = sigmoid(N(0, 1)) per token and head): the 16 windows of 512
    through `aspin_delta_windows` (every window at once from its affine state map: two state passes, the prefix of
    the maps with the -512 theta rebase, one output pass) against (i) the window-by-window loop on the GPU
    (aspin_delta + aspin_rebase per window) and (ii) the CPU oracle's window loop (`oracle.aspin.assoc_scan` with
    beta per window, `oracle.aspin.rebase` between), outputs and the final state, on the same bf16 inputs; also with
    an entering state."""
    from pragnosia_amd import ops  # noqa: F401
    from pragnosia_amd.assoc import rotate
    B, H, T, D, W = 2, 12, 8192, 64, 512
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 4.0)
    be = torch.sigmoid(torch.randn(B, H, T, generator=g))
    th = torch.rand(H, D // 2, generator=g) * 0.1
    S0 = torch.randn(B, H, D, D, generator=g) * 0.1
    op = torch.ops.pragnosia
    qd, kd, vd, lad, bed, thd, S0d = (t.cuda() for t in (q, k, v, la, be, th, S0))
    loc = torch.arange(T, device="cuda") % W
    qw, kw, vb = rotate(qd, thd, loc).bfloat16(), rotate(kd, thd, loc).bfloat16(), vd.bfloat16()
    qc, kc, vc = qw.float().cpu(), kw.float().cpu(), vb.float().cpu()
    for s0 in (None, S0d):
        with torch.no_grad():
            o1, S1 = op.aspin_delta_windows(qw, kw, vb, lad, bed, s0, thd, W)
            S, outs = s0, []
            for s in range(0, T, W):
                if s:
                    S = op.aspin_rebase(S, thd, None, float(W))
                o, S, _, _, _ = op.aspin_delta(qw[:, :, s:s + W], kw[:, :, s:s + W], vb[:, :, s:s + W],
                                               lad[:, :, s:s + W], bed[:, :, s:s + W], S, False)
                outs.append(o)
            oloop = torch.cat(outs, 2)
        torch.cuda.synchronize()
        e_loop = (rel(o1, oloop), rel(S1, S))
        Sr, outs = (None if s0 is None else S0.double()), []
        for s in range(0, T, W):
            if s:
                Sr = OA.rebase(Sr, th.double(), float(W))
            o, Sr = OA.assoc_scan(qc[:, :, s:s + W].double(), kc[:, :, s:s + W].double(), vc[:, :, s:s + W].double(),
                                  la[:, :, s:s + W].double(), Sr, chunk=64, beta=be[:, :, s:s + W].double())
            outs.append(o)
        e_ref = (rel(o1, torch.cat(outs, 2)), rel(S1, Sr))
        print(f"cfg3 delta one pass (S0 {'given' if s0 is not None else 'none'}): vs loop {e_loop}, vs oracle {e_ref}")
        assert max(e_loop + e_ref) < TOL


@pytest.mark.parametrize("batch", [1, 64])
def test_cfg4_decode_matches_oracle(batch):
    """LM(vocab 8192, d 768, 12 layers, 12 heads of 64, ctx 512, aspin), weights N(0, 0.02), a 512-token
    prefill then all 1,024 greedy steps through the captured graph, at batch 1 (the GEMV dense layers) and batch 64
    (the dense layers on the fp32 matrix cores, decode_gemm, the branch above GEMV_MAX_BATCH). The prefill fills one
    window, so the first step starts a new window with every state rebased by 512, and the position index wraps mod
    512 at step 512: both happen inside the run. The graph records the logits of every step (record_logits).
    (i) Every graphed token is the argmax of the graphed step's own logits.
    (ii) The graphed logits equal the CPU oracle's decode teacher-forced with the graphed tokens
    (`oracle.modules.greedy_decode`, pinned against forward_carried across window boundaries and the wrap) at every
    one of the 1,024 steps, for sequence 0 and, at batch 64, sequence 63.
    (iii) The eager step loop (the modules' own T = 1 path, no fused kernels), teacher-forced with the graphed tokens,
    gives the same logits for every sequence."""
    from pragnosia_amd.decode import GEMV_MAX_BATCH, GreedyDecoder, greedy_eager
    from pragnosia_amd.model import LM
    torch.manual_seed(4)
    m = LM(vocab=8192, d=768, layers=12, mlp_mult=4, ctx=512, mixer="aspin")
    assert sum(p.numel() for p in m.parameters()) == 91_930_812
    sd = {k_: v_.detach().clone() for k_, v_ in m.state_dict().items()}
    m = m.cuda().eval()
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, 8192, (batch, 512), generator=g)
    n = 1024
    dec = GreedyDecoder(m, batch, steps_per_graph=8, record_logits=True)
    assert dec.fused and (batch > GEMV_MAX_BATCH) == (batch == 64)
    toks_g = dec.generate(prompt.cuda(), n)
    assert dec.gemm == (batch == 64)
    lgs_g = dec.logits(n)
    assert bool((lgs_g.argmax(-1) == toks_g).all())
    rows = [0] if batch == 1 else [0, batch - 1]
    _, lgs_r = M.greedy_decode(sd, prompt[rows], n, layers=12, mixer="aspin", heads=12, forced=toks_g[rows].cpu())
    err = rel(lgs_g[rows], lgs_r)
    _, lgs_e = greedy_eager(m, prompt.cuda(), n, forced=toks_g)
    err_e = rel(lgs_g, lgs_e)
    print(f"cfg4 batch {batch}: {n} graphed steps, logits vs oracle {err:.2e}, vs eager {err_e:.2e}")
    assert err < TOL and err_e < TOL
