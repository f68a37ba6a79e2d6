"""Benchmark of the carrier hot path on one MI355X: prints ONE JSON line.

Headline workload (the configuration the metric is quoted on): the aspin chunked scan,
forward + backward, B16 T512 H12 D64, chunk 64, bf16 q/k/v, fp32 log-decays and state, synthetic seeded inputs
resident in HBM. One step = one forward (o, the final state and the bf16 entering states) and one backward
(dq, dk, dv, dla, dS0 from dO and dS_final) through the HIP kernels, on one stream. `--rule` picks the write rule of
the headline (plain by default); the other rule, the complex diagonal scan of configs[1] and the decode step are
measured too and reported under "secondary".

    python bench.py [--steps K] [--warmup W] [--rule plain|delta] [--no-cpu-baseline] [--no-secondary]

`value` is tokens (B * T) per second over the K timed steps, between two device synchronisations. `roofline` is the
dominant kernel of the headline step: algorithmic HBM bytes per launch (every input read once, every output written
once) over its average launch time, timed with HIP events on the stream the kernel is launched on. `cpu_baseline` is
the CPU oracle (this repository's restatement of the reference's two-pass fp32 path, forward + autograd backward)
timed on this host's cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "aspin fwd+bwd Mtok/s (B16 T512 H12 d64 bf16); decode ms/token 78M bs1"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rule", choices=("plain", "delta"), default="plain")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-kernels", action="store_true",
                    help="run each hot kernel a fixed number of times (for rocprofv3 counter passes) and exit")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the configs[4] decode measurement (batch 1 and 64), print its JSON and exit")
    ap.add_argument("--profile-workload", choices=("layer", "layer_delta", "lm", "lm_delta", "wgrad", "head128"),
                    help="run one workload a fixed number of times for a tracer (rocprofv3 --kernel-trace or "
                         "--pmc) and exit: the carrier layer step (graph replays), the LM training micro-step "
                         "(graph replays), the weight-gradient kernel at the layer's two shapes, or the head-dim-128 "
                         "scan steps of `wide_bench`")
    ap.add_argument("--phase-rates", action="store_true",
                    help="measure the MFMA rate inside the scan kernels' per-chunk phases from the instrumented "
                         "build (libpragnosia_stamps.so), print its JSON and exit")
    return ap.parse_args()


def aspin_inputs(B, H, T, D, seed, rule, device):
    """Seeded synthetic inputs following BASELINE.json configs[2]: q, k, v ~ N(0,1) with k L2-normalised per head,
    la = logsigmoid(N(3,1)), theta ~ U(0, 0.1) rotating q and k (interleaved pairs) at positions 0..T-1; delta rule:
    beta = sigmoid(N(0,1)). Upstream dO ~ N(0,1) and dS_final ~ N(0,1)."""
    import torch
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    ang = torch.arange(T).reshape(1, 1, T, 1).float() * th.reshape(1, H, 1, D // 2)
    c, s = torch.cos(ang), torch.sin(ang)

    def rot(x):
        e, o = x[..., 0::2], x[..., 1::2]
        return torch.stack((e * c - o * s, e * s + o * c), -1).flatten(-2)

    q, k = rot(q), rot(k)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g)) if rule == "delta" else None
    do = torch.randn(B, H, T, D, generator=g)
    dS = torch.randn(B, H, D, D, generator=g)
    out = dict(q=q, k=k, v=v, la=la, beta=beta, do=do, dS=dS)
    if device != "cpu":
        bf16 = ("q", "k", "v", "do")
        out = {n: (None if t is None else t.to(device, torch.bfloat16 if n in bf16 else torch.float32))
               for n, t in out.items()}
    return out


def _time_ops(fns, n, stream):
    """Average device seconds per call of each fn. Each fn is captured n times into one HIP graph, and the graph is
    replayed between two HIP events recorded on `stream`, the stream the replay launches the kernels on, so a
    kernel shorter than the host's per-call dispatch time is not charged for the gaps between launches. The ops
    allocate their outputs from the graph's pool and record no memset nodes."""
    import torch
    out = []
    for fn in fns:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(n):
                fn()
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / (n * reps) * 1e-3)
        del g
    return out


def aspin_bench(rule, steps, warmup):
    """The cfg2 step for one write rule: wall-clock time per step of `steps` steps captured in one HIP graph (and of
    `steps` eager calls, reported beside it), plus per-op event timings."""
    import torch
    from pragnosia_amd import ops  # noqa: F401
    B, H, T, D, C = 16, 12, 512, 64, 64
    NC = T // C
    dev = torch.device("cuda:0")
    x = aspin_inputs(B, H, T, D, 2, rule, dev)
    op = torch.ops.pragnosia
    stream = torch.cuda.current_stream(dev)
    if rule == "plain":
        fwd = lambda: op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
        saved = fwd()
        bwd = lambda: op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], saved[2], x["do"], x["dS"])

        def step():
            o, S, sent = op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
            return op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sent, x["do"], x["dS"])
    else:
        fwd = lambda: op.aspin_delta(x["q"], x["k"], x["v"], x["la"], x["beta"], None, True)
        saved = fwd()
        bwd = lambda: op.aspin_delta_bwd(x["q"], x["k"], x["v"], x["la"], x["beta"], saved[2], saved[3], saved[4],
                                         x["do"], x["dS"])

        def step():
            o, S, sent, W, X = op.aspin_delta(x["q"], x["k"], x["v"], x["la"], x["beta"], None, True)
            return op.aspin_delta_bwd(x["q"], x["k"], x["v"], x["la"], x["beta"], sent, W, X, x["do"], x["dS"])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager = (time.perf_counter() - t0) / steps
    # The same `steps` steps captured into one HIP graph and replayed once: every step runs both kernels over the
    # full batch, and the timed region is bound by the device rather than by Python's per-op dispatch (which for
    # this step is comparable to the kernels' own time) or by a per-replay launch cost.
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            step()
    graph.replay()  # untimed: first replay
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    del graph
    t_fwd, t_bwd = _time_ops([fwd, bwd], max(20, min(steps, 200)), stream)

    elem, ht, state, sent_n = B * H * T * D, B * H * T, B * H * D * D, B * H * NC * D * D
    if rule == "plain":
        # forward: q, k, v read, o written (bf16); la read; S_final and sent written
        fwd_bytes = 4 * 2 * elem + 4 * ht + 4 * state + 2 * sent_n
        # backward: q, k, v, dO, sent read; dq, dk, dv written; la read, dla written; dS_final read, dS0 written
        bwd_bytes = 7 * 2 * elem + 2 * sent_n + 8 * ht + 8 * state
        fwd_flops = 4 * D * (C + D) * ht
        bwd_flops = 10 * D * (C + D) * ht
        names = ("aspin_plain_fwd", "aspin_plain_bwd")
        counted = names
        impl_fwd, impl_bwd = fwd_bytes, bwd_bytes
    else:
        # the minimal I/O of the delta rule (the algorithmic bytes): forward q, k, v, la, beta read, o written, the
        # final state and the bf16 entering states written; backward q, k, v, dO, la, beta and the entering states
        # read, dq, dk, dv, dla, dbeta written, dS_final read, dS0 written
        fwd_bytes = 4 * 2 * elem + 8 * ht + 4 * state + 2 * sent_n
        bwd_bytes = 7 * 2 * elem + 2 * sent_n + 16 * ht + 8 * state
        # what this implementation moves besides, as a formula (the counter-measured bytes, where the traffic table
        # has them, replace it in op_roofline): in the forward (one kernel, the inverses formed on chip; the inverse
        # waves' key reads hit L2) X (bf16 C x C per chunk) and W written for the backward; in the backward (one
        # kernel, the chain and the chunk-local work passing drhs and the per-chunk dS through LDS) X and W read
        x_n = B * H * NC * C * C
        impl_fwd = fwd_bytes + 2 * x_n + 2 * elem
        impl_bwd = bwd_bytes + 2 * x_n + 2 * elem
        fwd_flops = (4 * D * (C + D) + 2 * C * D + 2 * D * D + 2 * C * C) * ht
        bwd_flops = (10 * D * (C + D) + 6 * C * D + 4 * D * D + 4 * C * C) * ht
        names = ("aspin_delta_fwd_inv (one kernel, inverses on chip)",
                 "aspin_delta_bwd_fused (one kernel: the chain and the chunk-local work)")
        counted = ("aspin_delta_fwd_inv", "aspin_delta_bwd_fused")
    cold = _rotating_bwd(rule, stream, x)
    return dict(B=B, H=H, T=T, D=D, C=C, wall=wall, eager=eager, t_fwd=t_fwd, t_bwd=t_bwd, fwd_bytes=fwd_bytes,
                bwd_bytes=bwd_bytes, impl_fwd_bytes=impl_fwd, impl_bwd_bytes=impl_bwd, fwd_flops=fwd_flops,
                bwd_flops=bwd_flops, names=names, counted=counted, cold=cold)


ROTATE_SETS = 8


def _rotating_bwd(rule, stream, bwd_args):
    """The backward (and forward) kernels timed over ROTATE_SETS different input sets in turn, each set the full
    cfg2 inputs plus the forward's saved tensors (~63 MB for the plain rule), ~500 MB in all, twice the 256 MB
    last-level cache: no launch finds its inputs in that cache from an earlier one. Returns the average launch times
    (us) of the forward and backward under rotation."""
    import torch
    op = torch.ops.pragnosia
    sets = []
    for i in range(ROTATE_SETS):
        x = {n: (None if t is None else t.clone()) for n, t in bwd_args.items()}
        with torch.no_grad():
            sv = (op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True) if rule == "plain" else
                  op.aspin_delta(x["q"], x["k"], x["v"], x["la"], x["beta"], None, True))
        sets.append((x, sv))
    it = {"f": 0, "b": 0}

    def fwd_cycle():
        x, _ = sets[it["f"] % ROTATE_SETS]
        it["f"] += 1
        return (op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True) if rule == "plain" else
                op.aspin_delta(x["q"], x["k"], x["v"], x["la"], x["beta"], None, True))

    def bwd_cycle():
        x, sv = sets[it["b"] % ROTATE_SETS]
        it["b"] += 1
        if rule == "plain":
            return op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sv[2], x["do"], x["dS"])
        return op.aspin_delta_bwd(x["q"], x["k"], x["v"], x["la"], x["beta"], sv[2], sv[3], sv[4], x["do"], x["dS"])

    t_f, t_b = _time_ops([fwd_cycle, bwd_cycle], 8 * ROTATE_SETS, stream)
    footprint = sum(t.numel() * t.element_size() for x, sv in sets for t in list(x.values()) + list(sv)
                    if t is not None)
    del sets
    return {"sets": ROTATE_SETS, "input_footprint_MB": round(footprint / 1e6, 1), "fwd_us": round(t_f * 1e6, 2),
            "bwd_us": round(t_b * 1e6, 2)}


def diag_bench(steps):
    """the per-token-lambda complex diagonal scan, fwd + bwd, B16 T512 D768 fp32."""
    import torch
    import torch.nn.functional as F
    from pragnosia_amd import ops  # noqa: F401
    B, T, D = 16, 512, 768
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    u = (torch.randn(B, T, D, generator=g) * (torch.randn(D, generator=g) * 0.1)).to(dev)
    lm = F.logsigmoid(torch.randn(B, T, D, generator=g) + 4.0).to(dev)
    an = (torch.rand(B, T, D, generator=g) - 0.5).to(dev)
    gy = torch.randn(B, T, D, generator=g).to(dev)
    glr, gli = torch.randn(B, D, generator=g).to(dev), torch.randn(B, D, generator=g).to(dev)
    op = torch.ops.pragnosia
    hr, _, _, hi = op.diag_scan(u, lm, an, None, None)
    fwd = lambda: op.diag_scan(u, lm, an, None, None)
    bwd = lambda: op.diag_scan_bwd(gy, glr, gli, lm, an, hr, hi, None, None)
    for _ in range(5):
        fwd()
        bwd()
    t_fwd, t_bwd = _time_ops([fwd, bwd], max(20, min(steps, 200)), torch.cuda.current_stream(dev))
    n = B * T * D
    fb, bb = 20 * n, 32 * n
    return {"workload": "complex diagonal scan fwd+bwd, B16 T512 D768 fp32 (configs[1])",
            "Mtok_s": round(B * T / (t_fwd + t_bwd) / 1e6, 3),
            "fwd_us": round(t_fwd * 1e6, 2), "bwd_us": round(t_bwd * 1e6, 2),
            "fwd_GBs": round(fb / t_fwd / 1e9, 1), "bwd_GBs": round(bb / t_bwd / 1e9, 1),
            "fwd_bwd_GBs": round((fb + bb) / (t_fwd + t_bwd) / 1e9, 1),
            "hbm_frac": round((fb + bb) / (t_fwd + t_bwd) / 1e9 / HBM_PEAK_GBS, 4)}


def wide_bench(steps=30):
    """Head dim 128 (the reference's `hspin` / `hdspin` carriers) at configs[2]'s width: B16 T512, d 768 as 6 heads
    of 128, bf16 q/k/v; one forward + backward through `assoc_scan` with bf16 matmuls (mm=bf16, the kernel path: for
    the plain rule four 64 x 64 scans per head reading the halves in place and the sums of their partial outputs, for
    the delta rule two 128 x 64 scans per head over its value halves), one step captured in a HIP graph (forward and
    autograd backward, leaf-gradient accumulation included) and replayed `steps` times between HIP events, beside
    the 64-dim path at the same width timed the same way."""
    import torch
    import torch.nn.functional as F
    from pragnosia_amd.assoc import assoc_scan
    g = torch.Generator().manual_seed(9)
    out = {"workload": "plain and delta rule fwd+bwd at head dim 128 vs 64, B16 T512 d768 (configs[2] width), "
                       "graph-replayed"}
    for rule in ("plain", "delta"):
        for H, D in ((6, 128), (12, 64)):
            q = F.normalize(torch.randn(16, H, 512, D, generator=g), dim=-1).bfloat16().cuda().requires_grad_(True)
            k = F.normalize(torch.randn(16, H, 512, D, generator=g), dim=-1).bfloat16().cuda().requires_grad_(True)
            v = torch.randn(16, H, 512, D, generator=g).bfloat16().cuda().requires_grad_(True)
            la = F.logsigmoid(torch.randn(16, H, 512, generator=g) + 3).cuda().requires_grad_(True)
            be = (torch.sigmoid(torch.randn(16, H, 512, generator=g)).cuda().requires_grad_(True)
                  if rule == "delta" else None)
            do = torch.randn(16, H, 512, D, generator=g).bfloat16().cuda()

            def step():
                o, _ = assoc_scan(q, k, v, la, mm=torch.bfloat16, beta=be)
                torch.autograd.backward([o], [do])
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(steps):
                graph.replay()
            t1.record()
            torch.cuda.synchronize()
            ms = t0.elapsed_time(t1) / steps
            out[f"{rule}_head_dim_{D}"] = {"ms_per_step": round(ms, 4), "Mtok_s": round(16 * 512 / ms / 1e3, 2)}
    return out


def carried_bench():
    """B2 T8192 H12 D64 bf16 inputs, la = logsigmoid(N(4,1)); (i) 16 windows of 512 with the
    fp32 state carried and rebased by -512 theta between windows (positions restart per window, as successive
    AssocCarrier.forward calls do), in one segment-parallel pass (aspin_chunk_windows); (ii) one unsplit T = 8192
    pass (aspin_chunk, which takes the segment-parallel forward for these few heads); device time per call from graph
    replays. Also the window-by-window loop (16 x (rebase + aspin_chunk)) the carried path replaces, a forward +
    backward step over the unsplit sequence (segment-parallel, and through the one-workgroup-per-head kernels), and
    the carried-vs-unsplit error on the outputs and on the final state."""
    import torch
    import torch.nn.functional as F
    from pragnosia_amd import ops  # noqa: F401
    from pragnosia_amd.assoc import rotate
    B, H, T, D, W = 2, 12, 8192, 64, 512
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 4.0)
    th = torch.rand(H, D // 2, generator=g) * 0.1
    q, k, v, la, th = (t.to(dev) for t in (q, k, v, la, th))
    loc = torch.arange(T, device=dev) % W
    glob = torch.arange(T, device=dev)
    qw, kw = rotate(q, th, loc).bfloat16(), rotate(k, th, loc).bfloat16()
    qg, kg = rotate(q, th, glob).bfloat16(), rotate(k, th, glob).bfloat16()
    vb = v.bfloat16()
    op = torch.ops.pragnosia

    def loop():
        S, outs = None, []
        for s in range(0, T, W):
            if S is not None:
                S = op.aspin_rebase(S, th, None, float(W))
            o, S, _ = op.aspin_chunk(qw[:, :, s:s + W], kw[:, :, s:s + W], vb[:, :, s:s + W], la[:, :, s:s + W],
                                     S, False)
            outs.append(o)
        return torch.cat(outs, 2), S

    carried = lambda: op.aspin_chunk_windows(qw, kw, vb, la, None, th, W, False)
    unsplit = lambda: op.aspin_chunk(qg, kg, vb, la, None, False)
    # a training step over the long sequence: forward (entering states kept) and backward, segment-parallel, and
    # the same through the one-workgroup-per-head kernels
    do = torch.randn(qg.shape, generator=torch.Generator(device=dev).manual_seed(33), device=dev).bfloat16()

    def step():
        o, S, sent = op.aspin_chunk(qg, kg, vb, la, None, True)
        return op.aspin_chunk_bwd(qg, kg, vb, la, sent, do, None)

    def step_sequential():
        from pragnosia_amd._lib import check, lib
        from pragnosia_amd.ops import _ptr, _stream
        NC = T // 64
        o, sent = torch.empty_like(qg), torch.empty(B, H, NC, D, D, device=dev, dtype=torch.bfloat16)
        S, dS0 = torch.empty(B, H, D, D, device=dev), torch.empty(B, H, D, D, device=dev)
        dq, dk, dv = torch.empty_like(qg), torch.empty_like(qg), torch.empty_like(qg)
        dla = torch.empty(B, H, T, device=dev)
        check(lib().pragnosia_aspin_chunk_fwd(_ptr(qg), _ptr(kg), _ptr(vb), _ptr(la), None, _ptr(o), _ptr(S),
                                              _ptr(sent), B, H, T, D, 64, _stream(qg)), "fwd")
        check(lib().pragnosia_aspin_chunk_bwd(_ptr(qg), _ptr(kg), _ptr(vb), _ptr(la), _ptr(sent), _ptr(do), None,
                                              _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla), _ptr(dS0), B, H, T, D, 64,
                                              _stream(qg)), "bwd")

    # the delta rule over the same windows (beta = sigmoid(N(0, 1))): every window at once from its affine state map,
    # and the window-by-window loop it replaces
    be = torch.sigmoid(torch.randn(B, H, T, generator=g)).to(dev)

    def loop_delta():
        S, outs = None, []
        for s in range(0, T, W):
            if S is not None:
                S = op.aspin_rebase(S, th, None, float(W))
            o, S, _, _, _ = op.aspin_delta(qw[:, :, s:s + W], kw[:, :, s:s + W], vb[:, :, s:s + W], la[:, :, s:s + W],
                                           be[:, :, s:s + W], S, False)
            outs.append(o)
        return torch.cat(outs, 2), S

    carried_delta = lambda: op.aspin_delta_windows(qw, kw, vb, la, be, None, th, W)
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        t_c, t_u, t_l, t_s, t_q, t_cd, t_ld = _time_ops([carried, unsplit, loop, step, step_sequential, carried_delta,
                                                         loop_delta], 10, stream)
        ocd, Scd = carried_delta()
        old, Sld = loop_delta()
        oc, Sc, _ = carried()
        ol, Sl = loop()
        ou, Su, _ = unsplit()
        Su_loc = op.aspin_rebase(Su, th, None, float(T - W))
    rel = lambda a, b: ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()
    P = ops.seg_chunks(B * H, T // 64, [p for p in range(1, W // 64 + 1) if (W // 64) % p == 0])
    Pu = ops.seg_chunks(B * H, T // 64, range(1, T // 64 + 1))
    return {"workload": "aspin carried long context, 16 windows x 512 vs one T8192 pass, B2 H12 D64 (configs[3])",
            "carried_Mtok_s": round(B * T / t_c / 1e6, 3), "carried_us": round(t_c * 1e6, 2),
            "carried_segment_chunks": P,
            "unsplit_Mtok_s": round(B * T / t_u / 1e6, 3), "unsplit_us": round(t_u * 1e6, 2),
            "unsplit_segment_chunks": Pu,
            "window_loop_Mtok_s": round(B * T / t_l / 1e6, 3), "window_loop_us": round(t_l * 1e6, 2),
            "long_fwd_bwd_Mtok_s": round(B * T / t_s / 1e6, 3), "long_fwd_bwd_us": round(t_s * 1e6, 2),
            "long_fwd_bwd_sequential_us": round(t_q * 1e6, 2),
            "carried_vs_window_loop_rel_err_o": round(rel(oc, ol), 6),
            "carried_vs_window_loop_rel_err_S": round(rel(Sc, Sl), 6),
            "carried_vs_unsplit_rel_err_o": round(rel(oc, ou), 6),
            "carried_vs_unsplit_rel_err_S": round(rel(Sc, Su_loc), 6),
            "delta": {"carried_Mtok_s": round(B * T / t_cd / 1e6, 3), "carried_us": round(t_cd * 1e6, 2),
                      "window_loop_Mtok_s": round(B * T / t_ld / 1e6, 3), "window_loop_us": round(t_ld * 1e6, 2),
                      "carried_vs_window_loop_rel_err_o": round(rel(ocd, old), 6),
                      "carried_vs_window_loop_rel_err_S": round(rel(Scd, Sld), 6)}}


def lm_train_bench(mixer="aspin", updates=4, micro_per_update=4):
    """Whole-model training at the reference's own context configuration (`PROGRESS.md:428`: 78M, d704, 12 layers,
    mlp 4, ctx 2048, micro-batch 4, 32k tokens per update; 351 ktok/s plain and 335 delta on an H100 NVL): each
    micro-step is the trainer's (`src/train.py:494-517`: bf16 autocast trunk, the chunked tied-head loss, backward,
    gradients accumulated) captured in one HIP graph, and every `micro_per_update` micro-steps one fused AdamW update
    and a gradient reset run eagerly. Random-init weights, synthetic token ids. Reported: tokens/s over whole updates
    and the micro-step's own time."""
    import torch
    from pragnosia_amd.model import LM
    torch.manual_seed(11)
    B, T, V = 4, 2048, 8192
    m = LM(vocab=V, d=704, layers=12, mlp_mult=4, ctx=T, mixer=mixer).cuda()
    opt = torch.optim.AdamW(m.parameters(), lr=1e-4, fused=True)
    for p in m.parameters():
        p.grad = torch.zeros_like(p)
    xs = torch.randint(0, V, (B, T + 1), device="cuda")

    def micro():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            h = m.trunk(xs[:, :T])
        m.loss(h.float(), xs[:, 1:T + 1]).backward()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            micro()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        micro()
    opt.step()
    opt.zero_grad(set_to_none=False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(updates):
        for _ in range(micro_per_update):
            xs.random_(0, V)
            graph.replay()
        opt.step()
        opt.zero_grad(set_to_none=False)
    e1.record()
    torch.cuda.synchronize()
    per_update = e0.elapsed_time(e1) / updates * 1e-3
    e0.record()
    for _ in range(micro_per_update):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    micro_s = e0.elapsed_time(e1) / micro_per_update * 1e-3
    n = sum(p.numel() for p in m.parameters())
    return {"workload": f"LM({mixer}, d704 L12 mlp4 V8192 ctx2048) training, micro-batch 4, {micro_per_update} "
                        f"micro-steps ({micro_per_update * B * T} tokens) per fused AdamW update, bf16 autocast, "
                        "micro-step graph-captured", "params": n,
            "ktok_s": round(micro_per_update * B * T / per_update / 1e3, 1),
            "micro_step_ms": round(micro_s * 1e3, 3)}


def carrier_layer_bench(steps=20, delta=False):
    """The carrier layer around the scan at configs[2]'s shape: AssocCarrier(768) (12 heads of 64; plain rule, or the
    delta rule) forward + backward on x (B16, T512, 768) under bf16 autocast, fp32 parameters: LayerNorm, the q/k/v
    and gate (or write-strength) projections, the decay, prep, the chunked scan, the output epilogue and the gated
    o-projection with its residual. Reported eagerly (host dispatch included) and as HIP-graph replays of the whole
    step (device time), with this build's fused plumbing (one projection GEMM feeding one prep kernel, fused output
    epilogue) and as the reference's torch composition around the same scan kernels."""
    import torch
    from pragnosia_amd import assoc
    torch.manual_seed(7)
    B, T, d = 16, 512, 768
    m = assoc.AssocCarrier(d, delta=delta).cuda()
    x = torch.randn(B, T, d, device="cuda", requires_grad=True)
    gy = torch.randn(B, T, d, device="cuda")

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, _ = m(x)
        y.backward(gy)

    out = {"workload": f"AssocCarrier(768{', delta=True' if delta else ''}) layer fwd+bwd, B16 T512, bf16 autocast "
                       "(configs[2] shape)"}
    prev = assoc.FUSED_PLUMBING
    try:
        for name, fused in (("fused_plumbing", True), ("torch_plumbing", False)):
            assoc.FUSED_PLUMBING = fused
            for p in list(m.parameters()) + [x]:
                p.grad = None
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            for _ in range(2):
                step()  # the caching allocator keeps blocks per stream: the timed stream's own, allocated untimed
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            eager = (time.perf_counter() - t0) / steps
            for p in list(m.parameters()) + [x]:
                p.grad = None
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            dev = e0.elapsed_time(e1) / steps * 1e-3
            out[name] = {"graph_ms_per_step": round(dev * 1e3, 4), "graph_Mtok_s": round(B * T / dev / 1e6, 3),
                         "eager_ms_per_step": round(eager * 1e3, 4)}
            del g
    finally:
        assoc.FUSED_PLUMBING = prev
    return out


def decode_bench(n_tokens=1024):
    """LM(vocab 8192, d 768, 12 layers, 12 heads of 64, ctx 512, aspin), random-init weights
    N(0, 0.02) (fp32), prefill of 512 random ids, then greedy decode through the graph-captured recurrent step, at
    batch 1 and batch 64. ms/token = wall time of the decode loop / decode steps."""
    import torch
    from pragnosia_amd.decode import GreedyDecoder
    from pragnosia_amd.model import LM
    torch.manual_seed(4)
    m = LM(vocab=8192, d=768, layers=12, mlp_mult=4, ctx=512, mixer="aspin").cuda().eval()
    n_params = sum(p.numel() for p in m.parameters())
    weight_bytes = 4 * (n_params - m.p.weight.numel())
    state_bytes = 12 * 12 * 64 * 64 * 4
    out = {"workload": "78M-class aspin LM greedy decode (d768 L12 H12x64 V8192 ctx512, fp32), prefill 512 "
                       "(configs[4])", "params": n_params}
    g = torch.Generator().manual_seed(4)
    for B in (1, 64):
        prompt = torch.randint(0, 8192, (B, 512), generator=g).cuda()
        dec = GreedyDecoder(m, B, steps_per_graph=8)
        with torch.no_grad():
            states, pw, lg = dec.prefill(prompt)
            dec.start(states, pw, lg, n_tokens)
            dec.replay(65)
            torch.cuda.synchronize()
            dec.start(states, pw, lg, n_tokens)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            dec.replay(n_tokens)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
        steps = -(-(n_tokens - 1) // dec.K) * dec.K
        per = dt / steps
        step_bytes = weight_bytes + 2 * state_bytes * B
        out[f"bs{B}"] = {"ms_per_step": round(per * 1e3, 4), "tok_s": round(B / per, 1),
                         "GBs": round(step_bytes / per / 1e9, 1), "hbm_frac": round(step_bytes / per / 1e9 / HBM_PEAK_GBS, 4)}
    out["ms_per_token_bs1"] = out["bs1"]["ms_per_step"]
    return out


TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "pmc_traffic_configs.md")


def measured_traffic(kernel, launch="configs[2]"):
    """HBM bytes per launch of `kernel` at the named launch as measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes recorded in profiles/pmc_traffic_configs.md (copy-calibrated), or None when the table has no such row."""
    try:
        col = None
        for line in open(TRAFFIC_TABLE):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if col is None and "traffic_bytes (calibrated)" in cells:
                col = cells.index("traffic_bytes (calibrated)")
            elif col is not None and len(cells) > col and cells[0] == kernel and launch in cells[1]:
                return int(cells[col])
    except (OSError, ValueError):
        return None
    return None


def summarize(r, rule):
    tokens = r["B"] * r["T"]
    dom = (r["names"][1], r["t_bwd"], r["bwd_bytes"], r["bwd_flops"]) if r["t_bwd"] >= r["t_fwd"] else \
          (r["names"][0], r["t_fwd"], r["fwd_bytes"], r["fwd_flops"])
    achieved = dom[2] / dom[1] / 1e9
    return tokens, dom, achieved


def lds_contraction_bench():
    """LDS-resident contraction microbenchmark (csrc/microbench/contract.hip): bf16 MFMA throughput of the scan
    kernels' operand patterns with every operand on chip, at 8 and 16 waves per CU, on the 16 x 16 x 32 MFMA the
    kernels use and on the 32 x 32 x 16 one (half the operand bytes per flop). Bounds what the contraction phases
    could reach with no HBM traffic and no chunk chain."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "pragnosia_amd",
                                   "libpragnosia_microbench.so"))
    fn = lib.pragnosia_microbench_contract
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    stream = torch.cuda.current_stream()
    iters, waves = 2000, 8
    names = {0: "registers only", 1: "one LDS operand per MFMA", 2: "LDS operand + accumulator->operand chain",
             3: "32x32x16: registers only", 4: "32x32x16: one LDS operand per MFMA",
             5: "32x32x16: LDS operand + accumulator->operand chain"}
    out = {}
    for per_cu, nwg in ((8, 256), (16, 512)):
        buf = torch.empty(nwg * 64 * waves, device="cuda")
        for var in range(6):
            call = lambda: fn(var, waves, iters, nwg, ctypes.c_void_p(buf.data_ptr()),
                              ctypes.c_void_p(stream.cuda_stream))
            assert call() == 0
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(5):
                call()
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) / 5 * 1e-3
            tfl = nwg * waves * iters * 16 * 16384 / t / 1e12
            out[f"{names[var]}, {per_cu} waves/CU"] = {"tflops": round(tfl, 1), "frac": round(tfl / BF16_PEAK_TFLOPS, 4)}
    return out


def counter_ratio(r):
    """HBM bytes the rocprofv3 counters measured for the op's kernels at configs[2], summed, over its algorithmic
    bytes; None when any of them has no row in the traffic table."""
    got = [measured_traffic(k) for k in r["counted"]]
    if any(v is None for v in got):
        return None
    return round(sum(got) / (r["fwd_bytes"] + r["bwd_bytes"]), 3)


def op_roofline(r):
    """The whole fwd+bwd op against both rooflines, from the algorithmic bytes and flops over the two kernels' summed
    durations: the HBM fraction, the bf16 MFMA fraction, and the larger of the two (the op's roofline position)."""
    t = r["t_fwd"] + r["t_bwd"]
    gbs = (r["fwd_bytes"] + r["bwd_bytes"]) / t / 1e9
    tfl = (r["fwd_flops"] + r["bwd_flops"]) / t / 1e12
    measured = counter_ratio(r)
    impl = (measured * (r["fwd_bytes"] + r["bwd_bytes"]) if measured is not None
            else r["impl_fwd_bytes"] + r["impl_bwd_bytes"])
    tc = (r["cold"]["fwd_us"] + r["cold"]["bwd_us"]) * 1e-6
    return {"hbm_GBs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_tflops": round(tfl, 2),
            "mfma_frac": round(tfl / BF16_PEAK_TFLOPS, 4),
            "achieved_frac": round(max(gbs / HBM_PEAK_GBS, tfl / BF16_PEAK_TFLOPS), 4),
            "ai_flop_per_byte": round((r["fwd_flops"] + r["bwd_flops"]) / (r["fwd_bytes"] + r["bwd_bytes"]), 1),
            # this implementation's bytes (its own intermediates included) against the algorithmic ones: as the
            # FETCH_SIZE / WRITE_SIZE counters measured them for the same kernels (profiles/pmc_traffic_configs.md),
            # or from the formula in aspin_bench when a kernel has no row there (then counter_bytes_ratio is null)
            "impl_bytes_ratio": round(impl / (r["fwd_bytes"] + r["bwd_bytes"]), 3),
            "counter_bytes_ratio": measured,
            "impl_GBs": round(impl / t / 1e9, 1),
            # the same kernels with every launch's inputs out of the last-level cache (rotating input sets)
            "cold": dict(r["cold"], hbm_frac=round((r["fwd_bytes"] + r["bwd_bytes"]) / tc / 1e9 / HBM_PEAK_GBS, 4))}


def gpu_bench(args):
    r = aspin_bench(args.rule, args.steps, args.warmup)
    tokens, dom, achieved = summarize(r, args.rule)
    res = {
        "metric": METRIC,
        "value": round(tokens / r["wall"] / 1e6, 3),
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall"] * 1e3, 5),
        "eager_ms_per_step": round(r["eager"] * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json configs[2] distributions)",
        "config": {"workload": f"aspin chunked scan fwd+bwd, {args.rule} rule, B16 T512 H12 D64 chunk64 (configs[2])",
                   "B": r["B"], "T": r["T"], "H": r["H"], "D": r["D"], "chunk": r["C"], "rule": args.rule},
        "roofline": {"bound": "hbm", "kernel": dom[0], "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom[0]),
                     "algorithmic_bytes": dom[2], "avg_launch_us": round(dom[1] * 1e6, 2),
                     "mfma_tflops": round(dom[3] / dom[1] / 1e12, 2),
                     "mfma_frac": round(dom[3] / dom[1] / 1e12 / BF16_PEAK_TFLOPS, 4),
                     "cold_avg_launch_us": r["cold"]["bwd_us" if dom[0] == r["names"][1] else "fwd_us"],
                     "cold_frac": round(dom[2] / (r["cold"]["bwd_us" if dom[0] == r["names"][1] else "fwd_us"] * 1e-6)
                                        / 1e9 / HBM_PEAK_GBS, 4)},
        "kernels_us": {r["names"][0]: round(r["t_fwd"] * 1e6, 2), r["names"][1]: round(r["t_bwd"] * 1e6, 2)},
        "op": op_roofline(r),
    }
    if not args.no_secondary:
        other = "delta" if args.rule == "plain" else "plain"
        o = aspin_bench(other, max(20, args.steps // 4), 5)
        ot, odom, oach = summarize(o, other)
        sec = {f"aspin_{other}": {
            "workload": f"aspin chunked scan fwd+bwd, {other} rule, B16 T512 H12 D64 (configs[2])",
            "Mtok_s": round(ot / o["wall"] / 1e6, 3), "ms_per_step": round(o["wall"] * 1e3, 5),
            "eager_ms_per_step": round(o["eager"] * 1e3, 5),
            "fwd_us": round(o["t_fwd"] * 1e6, 2), "bwd_us": round(o["t_bwd"] * 1e6, 2),
            "fwd_bwd_GBs": round((o["fwd_bytes"] + o["bwd_bytes"]) / (o["t_fwd"] + o["t_bwd"]) / 1e9, 1),
            "fwd_bwd_mfma_tflops": round((o["fwd_flops"] + o["bwd_flops"]) / (o["t_fwd"] + o["t_bwd"]) / 1e12, 2),
            "op": op_roofline(o)}}
        sec["diag_scan"] = diag_bench(args.steps)
        sec["carried"] = carried_bench()
        sec["carrier_layer"] = carrier_layer_bench()
        sec["carrier_layer_delta"] = carrier_layer_bench(delta=True)
        sec["lm_train"] = {"plain": lm_train_bench("aspin"), "delta": lm_train_bench("dspin"),
                           "reference_h100_nvl_ktok_s": {"plain": 351, "delta": 335}}
        sec["decode"] = decode_bench()
        sec["head_dim_128"] = wide_bench()
        sec["lds_contraction"] = lds_contraction_bench()
        res["decode_ms_per_token_bs1"] = sec["decode"]["ms_per_token_bs1"]
        res["secondary"] = sec
    return res


def cpu_baseline(args):
    """The CPU oracle (two-pass fp32 form, autograd backward) on B = 1 sequence of the cfg2 shape, repeated for
    about `cpu_seconds`; median per-iteration rate, in the metric's unit."""
    import torch
    from oracle import aspin as O
    torch.set_num_threads(os.cpu_count() if not os.environ.get("OMP_NUM_THREADS") else
                          int(os.environ["OMP_NUM_THREADS"]))
    B, H, T, D = 1, 12, 512, 64
    x = aspin_inputs(B, H, T, D, 2, args.rule, "cpu")
    S0 = torch.zeros(B, H, D, D)

    def it():
        a = [x[n].clone().requires_grad_(True) for n in ("q", "k", "v", "la")]
        if args.rule == "plain":
            o, S, _ = O.scan_twopass(*a, S0, 64, None)
        else:
            o, S, _, _ = O.scan_twopass_delta(*a, x["beta"], S0, 64, None)
        ((o * x["do"]).sum() + (S * x["dS"]).sum()).backward()

    for _ in range(3):
        it()
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while time.perf_counter() < t_end or len(times) < 10:
        t0 = time.perf_counter()
        it()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    form = "src/assoc.py:118-165" if args.rule == "plain" else "src/assoc.py:168-251"
    return {"value": round(B * T / med / 1e6, 5), "unit": "Mtok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"CPU oracle ({args.rule} rule, two-pass fp32 restatement of {form}, autograd backward), "
                      f"B=1 x T512 H12 D64 per iteration, {len(times)} iterations (~{args.cpu_seconds:.0f} s), "
                      "median"}


def _host_cpu():
    """The host CPU's model name (from /proc/cpuinfo) and logical core count."""
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": name, "logical_cores": os.cpu_count()}


def _median_rate(fn, seconds, units):
    for _ in range(2):
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return units / med, med, len(times)


def cpu_baselines_more(args, seconds=5.0):
    """The CPU oracle on the other workloads, each on a bounded sample of its config (about `seconds` each): the
    delta rule of configs[2] (two-pass fp32 with the chunk inverse, autograd backward), the diagonal scan of
    configs[1] (`scan_gated`, chunk 16, autograd backward, the reference's CPU path `src/spin.py:181-215`), and the
    eager fp32 decode of configs[4] (the oracle's T = 1 steps through the 12-layer d768 LM)."""
    import torch
    from oracle import aspin as O
    from oracle import diag as OD
    from oracle import modules as OM
    out = {"host_cpu": _host_cpu(), "threads": torch.get_num_threads()}
    B, H, T, D = 1, 12, 512, 64
    x = aspin_inputs(B, H, T, D, 2, "delta", "cpu")
    S0 = torch.zeros(B, H, D, D)

    def delta_it():
        a = [x[n].clone().requires_grad_(True) for n in ("q", "k", "v", "la", "beta")]
        o, S, _, _ = O.scan_twopass_delta(*a, S0, 64, None)
        ((o * x["do"]).sum() + (S * x["dS"]).sum()).backward()

    rate, med, n = _median_rate(delta_it, seconds, B * T)
    out["aspin_delta_cfg2"] = {"value": round(rate / 1e6, 5), "unit": "Mtok/s", "kind": "port",
                               "sample": f"B=1 x T512 H12 D64, fwd + autograd bwd, {n} iterations, median"}
    g = torch.Generator().manual_seed(1)
    Tb, Db = 512, 768
    u = torch.randn(1, Tb, Db, generator=g)
    lm = torch.nn.functional.logsigmoid(torch.randn(1, Tb, Db, generator=g) + 4.0)
    an = torch.rand(1, Tb, Db, generator=g) - 0.5
    gy = torch.randn(1, Tb, Db, generator=g)

    def diag_it():
        a = [t.clone().requires_grad_(True) for t in (u, lm, an)]
        y, (hr, hi) = OD.scan_gated(*a, None, 16)
        (y * gy).sum().add(hr.sum() + hi.sum()).backward()

    rate, med, n = _median_rate(diag_it, seconds, Tb)
    out["diag_scan_cfg1"] = {"value": round(rate / 1e6, 5), "unit": "Mtok/s", "kind": "port",
                             "sample": f"B=1 x T512 D768 (one of 16 sequences), scan_gated chunk 16 fwd + autograd "
                                       f"bwd, {n} iterations, median; GPU reference point: configs[1] B16"}
    from pragnosia_amd.model import LM
    torch.manual_seed(4)
    sd = {k: v.detach() for k, v in LM(vocab=8192, d=768, layers=12, mlp_mult=4, ctx=512,
                                         mixer="aspin").state_dict().items()}
    prompt = torch.randint(0, 8192, (1, 64), generator=g)
    n1, n2 = 8, 72

    def decode_run(steps):
        with torch.inference_mode():
            t0 = time.perf_counter()
            OM.greedy_decode(sd, prompt, steps, layers=12, mixer="aspin", heads=12)
            return time.perf_counter() - t0

    decode_run(n1)
    t1 = sorted(decode_run(n1) for _ in range(3))[1]
    t2 = sorted(decode_run(n2) for _ in range(3))[1]
    # the same prefill in both runs: the difference of the medians is the cost of n2 - n1 steps, prefill excluded
    out["decode_cfg4_bs1"] = {"value": round((t2 - t1) / (n2 - n1) * 1e3, 3), "unit": "ms/token", "kind": "port",
                              "sample": f"92M LM at batch 1, fp32, oracle (torch CPU) T=1 steps: median time of "
                                        f"prefill 64 + {n2} greedy steps minus that of prefill 64 + {n1} steps, "
                                        f"over {n2 - n1} steps (3 runs each)"}
    return out


def profile_workload(name, reps=10):
    """The workloads behind the layer, LM and weight-gradient traces in profiles/: `reps` graph replays of the
    carrier layer step (AssocCarrier(768), B16 T512, bf16 autocast, fused plumbing) or of the LM training micro-step
    (d704 L12 mlp4 ctx2048 micro-batch 4, as lm_train_bench), after three eager warm-up steps on a side stream;
    `reps` calls of the weight-gradient kernel at 8192 x 2328 x 768 and 8192 x 768 x 768; or `wide_bench` as it
    runs in the secondary measurements (head128)."""
    import torch
    from pragnosia_amd import assoc, ops
    torch.manual_seed(7)
    if name == "head128":
        print(json.dumps(wide_bench()), flush=True)
        return
    if name == "wgrad":
        for M in (2328, 768):
            A = torch.randn(8192, M, device="cuda").bfloat16()
            Bm = torch.randn(8192, 768, device="cuda").bfloat16()
            for _ in range(reps):
                ops.wgrad(A, Bm)
        torch.cuda.synchronize()
        return
    if name.startswith("layer"):
        m = assoc.AssocCarrier(768, delta=name == "layer_delta").cuda()
        x = torch.randn(16, 512, 768, device="cuda", requires_grad=True)
        gy = torch.randn(16, 512, 768, device="cuda")

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y, _ = m(x)
            y.backward(gy)
        params = list(m.parameters()) + [x]
    else:
        from pragnosia_amd.model import LM
        m = LM(vocab=8192, d=704, layers=12, mlp_mult=4, ctx=2048, mixer="dspin" if name == "lm_delta" else "aspin")
        m = m.cuda()
        xs = torch.randint(0, 8192, (4, 2049), device="cuda")

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                h = m.trunk(xs[:, :2048])
            m.loss(h, xs[:, 1:]).backward()
        params = list(m.parameters())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    for p in params:
        # as carrier_layer_bench (gradients assigned by the captured step) and lm_train_bench (accumulated into
        # allocated gradients over the micro-steps of an update)
        p.grad = torch.zeros_like(p) if name.startswith("lm") else None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()


def profile_kernels(reps=10):
    """For counter runs under rocprofv3 (--pmc FETCH_SIZE, then WRITE_SIZE): each hot kernel `reps` times at its
    configs shape, plus a calibration copy of exactly COPY_BYTES read and COPY_BYTES written (a torch copy_ of a
    contiguous fp32 tensor), so that the counters' bytes per dispatch can be scaled against a known transfer."""
    import torch
    from pragnosia_amd import ops  # noqa: F401
    dev = torch.device("cuda:0")
    op = torch.ops.pragnosia
    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    for rule in ("plain", "delta"):
        x = aspin_inputs(16, 12, 512, 64, 2, rule, dev)
        for _ in range(reps):
            if rule == "plain":
                o, S, sent = op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
                op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sent, x["do"], x["dS"])
            else:
                o, S, sent, W, X = op.aspin_delta(x["q"], x["k"], x["v"], x["la"], x["beta"], None, True)
                op.aspin_delta_bwd(x["q"], x["k"], x["v"], x["la"], x["beta"], sent, W, X, x["do"], x["dS"])
        if rule == "delta":
            # the same forward kernel writing only o and the final state (the recomputing path's forward), then its
            # state pass (entering states, W and X; no output products), each `reps` times after the stored form's
            args = [x["q"].bfloat16(), x["k"].bfloat16(), x["v"].bfloat16(), x["la"].float(), x["beta"].float(), None]
            for _ in range(reps):
                ops._delta_pass(*args, True, False)
            for _ in range(reps):
                ops._delta_pass(*args, False, True)
    # the plain rule at head dim 128 (configs[2]'s width as 6 heads of 128): the native forward
    x = aspin_inputs(16, 6, 512, 128, 3, "plain", dev)
    for _ in range(reps):
        op.aspin_chunk_wide(x["q"], x["k"], x["v"], x["la"], None, True)
    B, T, D = 16, 512, 768
    u, lm, an, gy = (torch.randn(B, T, D, device=dev) for _ in range(4))
    lm = -lm.abs()
    hr, _, _, hi = op.diag_scan(u, lm, an, None, None)
    for _ in range(reps):
        op.diag_scan(u, lm, an, None, None)
        op.diag_scan_bwd(gy, None, None, lm, an, hr, hi, None, None)
    # the segment-parallel forward and backward at configs[3]'s unsplit shape (B2 H12 T8192)
    x = aspin_inputs(2, 12, 8192, 64, 3, "plain", dev)
    for _ in range(reps):
        o, S, sent = op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
        op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sent, x["do"], x["dS"])
    # the carrier's plumbing at configs[2]'s shape: the prep from one projection GEMM's bf16 output (q, k, v, decay and
    # gate columns) and the output epilogue, each way
    H = 12
    g = torch.Generator(device=dev).manual_seed(5)
    P = torch.randn(16, 512, 3 * H * 64 + 2 * H, device=dev, generator=g).bfloat16()
    lb, A, gb = (torch.randn(H, device=dev, generator=g) for _ in range(3))
    th = torch.rand(H, 32, device=dev, generator=g) * 0.1
    pos = torch.arange(512, device=dev)
    o = x_o = torch.randn(16, H, 512, 64, device=dev, generator=g).bfloat16()
    w = torch.randn(64, device=dev, generator=g)
    gyo = torch.randn(16, 512, H * 64, device=dev, generator=g).bfloat16()
    for _ in range(reps):
        q, k, v, la, _ = op.aspin_prep_proj(P, H, lb, A, None, gb, None, 0.0, True, th, pos)
        op.aspin_prep_proj_bwd(P, H, lb, A, None, gb, None, 0.0, True, th, pos, q, k, v, la, None)
        y, rstd = op.aspin_out(x_o, w, ops.RMS_EPS, True)
        op.aspin_out_bwd(gyo, o, w, rstd)
    torch.cuda.synchronize()
    print(json.dumps({"profile_kernels": reps, "copy_bytes": COPY_BYTES}), flush=True)


COPY_BYTES = 256 << 20

# MFMAs (16x16x32 bf16, 16384 flops each) per 64-token chunk of one workgroup, counted from the kernels' code.
# Plain forward: output waves 88 (per t block TB and value half: O^T = V^T A^T + S^T (Q o eL)^T, 3 or 4 a column
# tile (2 A operands from TB 2 on), 2 column tiles, and the state update 2 x 2), score waves 20 (2 per s block at or
# below the diagonal). Plain backward: group K 152 (P and dA 4 per block WL..3, then 4 dV^T and 4 dK^T tiles of 3 or
# 4), group D 128 (P^T and dA^T 4 per block 0..WL, 4 dQ^T tiles of 3 or 4, the dS update 4 x 2). Delta forward
# chain: 4 chain waves x 36 (U = K S 8, W = X rhs 6, O 14, state update 8) and the scores 20 (the inverse waves' bf16
# products, 20 a chunk, run in other phases and are not counted). Delta backward chain (the chain and service waves
# of the one-kernel backward; its eight chunk-local waves' products are not counted):
# 4 chain waves x 44 (K dS 8, K S_c 8, (Q o eL)^T dO 8, dW 6, drhs 6, dS update 8) and the transposed scores 20.
PHASE_MFMAS = {"plain_fwd": {"output": 88, "score": 20}, "plain_bwd": 280, "delta_fwd": 164, "delta_bwd_chain": 196}
MFMA_FLOPS = 16 * 16 * 32 * 2


def _rel32(x, ref):
    """uint32 clock readings relative to ref, as signed int64 (differences within a kernel never wrap twice)."""
    import numpy as np
    d = (x.astype(np.int64) - ref.astype(np.int64)) % (1 << 32)
    return np.where(d >= (1 << 31), d - (1 << 32), d)


def _phase_stats(buf, nwg, nw, NC, waves_of, flops_of):
    """Per-chunk phase windows from one stamp buffer ((workgroups, waves, 4 + 2 NC) uint32; entries 0-3 the clocks
    at the role's start and the kernel's end, then each chunk's phase start and end): the shader clock's rate from
    the 100 MHz clock beside it, each chunk's window (earliest start to latest end over waves_of(c)), and the MFMA
    rate over the windows against the per-CU share of the bf16 peak."""
    import numpy as np
    s = buf.cpu().numpy().view(np.uint32).reshape(nwg, nw, 4 + 2 * NC)
    mt_b, rt_b, mt_e, rt_e = (s[:, :, j].astype(np.int64) for j in range(4))
    clk = float(np.median(((mt_e - mt_b) % (1 << 32)) / ((rt_e - rt_b) % (1 << 32)))) * 1e8
    ref = s[:, :1, 0]
    start, end = _rel32(s[:, :, 4::2], ref[..., None]), _rel32(s[:, :, 5::2], ref[..., None])
    life = (_rel32(s[:, :, 2], ref).max(1) - _rel32(s[:, :, 0], ref).min(1)).astype(np.float64)
    win = np.stack([(end[:, waves_of(c), c].max(1) - start[:, waves_of(c), c].min(1)).astype(np.float64)
                    for c in range(NC)], 1)
    fl = np.array([flops_of(c) for c in range(NC)], dtype=np.float64)
    rate = fl.sum() * nwg / (win.sum() / clk)
    peak_cu = BF16_PEAK_TFLOPS * 1e12 / 256
    return {"shader_clock_GHz": round(clk / 1e9, 3),
            "phase_us_median": round(float(np.median(win)) / clk * 1e6, 3),
            "phase_TFLOPs_per_CU": round(rate / 1e12, 3),
            "phase_frac_of_peak": round(rate / peak_cu, 4),
            "phase_share_of_workgroup_life": round(float(win.sum(1).mean() / life.mean()), 4)}, fl.sum() * nwg


def phase_rates(reps=50):
    """MFMA rate inside the scan kernels' per-chunk phases at configs[2] (B16 T512 H12 D64), from the instrumented
    build (libpragnosia_stamps.so: the same kernels, every wave writing its shader clock where its role's branch
    starts, at the start and end of each chunk's phase, and at the kernel's end). A chunk's phase on a workgroup runs
    from the earliest phase start to the latest phase end over the waves that contract in that barrier interval
    (plain forward: the 8 output waves on chunk c and the 4 score waves on chunk c + 1; plain backward and the delta
    chain kernels: all 8 waves), so it covers the operand reads, the MFMAs, the result stores and, in the delta
    chain, its mid-chunk barrier. Rate = the chunk's MFMA flops (counted from the code, PHASE_MFMAS) / its window,
    per CU, against the per-CU share of the dense bf16 peak (2.5 PFLOP/s / 256 CUs). The shader clock's rate comes
    from the 100 MHz clock read beside it. Also reported: the share of each workgroup's lifetime spent in phases,
    and the stamped entry points' times against the product library's (the stamps' own cost)."""
    import ctypes
    import torch
    from pragnosia_amd._lib import SIGNATURES, lib as product_lib
    dev = torch.device("cuda:0")
    st = ctypes.CDLL(os.path.join(ROOT, "pragnosia_amd", "libpragnosia_stamps.so"))
    libs = {"stamped": st, "product": product_lib()}
    names = ("pragnosia_aspin_chunk_fwd", "pragnosia_aspin_chunk_bwd", "pragnosia_aspin_delta_fwd",
             "pragnosia_aspin_delta_bwd")
    for L in libs.values():
        for name in names:
            getattr(L, name).argtypes = SIGNATURES[name]
            getattr(L, name).restype = ctypes.c_int
    for unit in ("chunk", "delta"):
        getattr(st, "pragnosia_stamps_set_" + unit).argtypes = [ctypes.c_void_p]
        getattr(st, "pragnosia_stamps_set_" + unit).restype = ctypes.c_int
    B, H, T, D = 16, 12, 512, 64
    NC, nwg = T // 64, B * H
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    xp = aspin_inputs(B, H, T, D, 0, "plain", dev)
    xd = aspin_inputs(B, H, T, D, 0, "delta", dev)
    e = lambda *shape, dt=torch.float32: torch.empty(*shape, device=dev, dtype=dt)
    bf = torch.bfloat16
    o, dq, dk, dv, W = (e(B, H, T, D, dt=bf) for _ in range(5))
    S, dS0 = e(B, H, D, D), e(B, H, D, D)
    sent, X = e(B, H, NC, D, D, dt=bf), e(B, H, NC, 64, 64, dt=bf)
    dla, dbeta = e(B, H, T), e(B, H, T)
    wsb = product_lib().pragnosia_aspin_delta_bwd_workspace_bytes(B, H, T, D, 64)
    ws = e(wsb, dt=torch.uint8)
    run = {
        "plain_fwd": lambda L: L.pragnosia_aspin_chunk_fwd(
            P(xp["q"]), P(xp["k"]), P(xp["v"]), P(xp["la"]), None, P(o), P(S), P(sent), B, H, T, D, 64, sp),
        "plain_bwd": lambda L: L.pragnosia_aspin_chunk_bwd(
            P(xp["q"]), P(xp["k"]), P(xp["v"]), P(xp["la"]), P(sent), P(xp["do"]), P(xp["dS"]), P(dq), P(dk),
            P(dv), P(dla), P(dS0), B, H, T, D, 64, sp),
        "delta_fwd": lambda L: L.pragnosia_aspin_delta_fwd(
            P(xd["q"]), P(xd["k"]), P(xd["v"]), P(xd["la"]), P(xd["beta"]), None, P(o), P(S), P(sent), P(W), P(X),
            B, H, T, D, 64, sp),
        "delta_bwd_chain": lambda L: L.pragnosia_aspin_delta_bwd(
            P(xd["q"]), P(xd["k"]), P(xd["v"]), P(xd["la"]), P(xd["beta"]), P(sent), P(W), P(X), P(xd["do"]),
            P(xd["dS"]), P(dq), P(dk), P(dv), P(dla), P(dbeta), P(dS0), P(ws), wsb, B, H, T, D, 64, sp)}
    unit = {"plain_fwd": "chunk", "plain_bwd": "chunk", "delta_fwd": "delta", "delta_bwd_chain": "delta"}
    waves = {"plain_fwd": 16, "plain_bwd": 8, "delta_fwd": 8, "delta_bwd_chain": 8}
    pf = PHASE_MFMAS["plain_fwd"]
    waves_of = {"plain_fwd": lambda c: list(range(8)) + (list(range(8, 12)) if c + 1 < NC else []),
                "plain_bwd": lambda c: list(range(8)), "delta_fwd": lambda c: list(range(8)),
                "delta_bwd_chain": lambda c: list(range(8))}
    flops_of = {"plain_fwd": lambda c: (pf["output"] + (pf["score"] if c + 1 < NC else 0)) * MFMA_FLOPS,
                "plain_bwd": lambda c: PHASE_MFMAS["plain_bwd"] * MFMA_FLOPS,
                "delta_fwd": lambda c: PHASE_MFMAS["delta_fwd"] * MFMA_FLOPS,
                "delta_bwd_chain": lambda c: PHASE_MFMAS["delta_bwd_chain"] * MFMA_FLOPS}

    def timed(fn, L):
        for _ in range(5):
            assert fn(L) == 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn(L)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    out = {"workload": "plain and delta chunked scans, B16 T512 H12 D64 bf16 (configs[2]), phase stamps"}
    # the delta inverse at head dim 64 (formed on chip by the forward's three inverse waves, one chunk each over three
    # iterations in six phases): each phase's duration from the unit's second stamp buffer, 16 entries per (head,
    # chunk): clocks at the inverse's start (0, 1), each phase's start and end (2 + 2p, 3 + 2p), clocks at its end
    # (14, 15); the span from start to end includes the barriers between the phases
    import numpy as np
    st.pragnosia_stamps_set_delta_aux.argtypes = [ctypes.c_void_p]
    st.pragnosia_stamps_set_delta_aux.restype = ctypes.c_int
    ninv = nwg * NC
    ibuf = torch.zeros(ninv * 16, device=dev, dtype=torch.int32)
    assert st.pragnosia_stamps_set_delta_aux(P(ibuf)) == 0
    for _ in range(3):
        assert run["delta_fwd"](st) == 0
    torch.cuda.synchronize()
    assert st.pragnosia_stamps_set_delta_aux(None) == 0
    si = ibuf.cpu().numpy().view(np.uint32).reshape(ninv, 16)
    clk = float(np.median(((si[:, 14].astype(np.int64) - si[:, 0]) % (1 << 32)) /
                          ((si[:, 15].astype(np.int64) - si[:, 1]) % (1 << 32)))) * 1e8
    # differences within a wave only (the shader clocks of different XCDs are not synchronised)
    t = _rel32(si, si[:, :1]).astype(np.float64) / clk * 1e6  # us from the inverse's start
    names = ("keys staged, decay scan, N blocks", "diagonal blocks", "level 1", "level 2", "level 3",
             "store X, next keys' loads")
    out["delta_inverse_phases"] = {
        "chunks": ninv, "shader_clock_GHz": round(clk / 1e9, 3),
        "median_us": {n: round(float(np.median(t[:, 3 + 2 * j] - t[:, 2 + 2 * j])), 3) for j, n in enumerate(names)},
        "span_median_us": round(float(np.median(t[:, 14])), 3)}
    for kern in ("plain_fwd", "plain_bwd", "delta_fwd", "delta_bwd_chain"):
        setter = getattr(st, "pragnosia_stamps_set_" + unit[kern])
        buf = torch.zeros(nwg * waves[kern] * (4 + 2 * NC), device=dev, dtype=torch.int32)
        if kern == "delta_bwd_chain":  # its inputs: the forward's entering states, W and X
            assert run["delta_fwd"](libs["product"]) == 0
        assert setter(None) == 0
        t = {"product_us": timed(run[kern], libs["product"]), "stamped_off_us": timed(run[kern], st)}
        assert setter(P(buf)) == 0
        t["stamped_on_us"] = timed(run[kern], st)
        torch.cuda.synchronize()
        assert setter(None) == 0
        stats, total_flops = _phase_stats(buf, nwg, waves[kern], NC, waves_of[kern], flops_of[kern])
        stats["mfma_per_chunk"] = (pf["output"] + pf["score"]) if kern == "plain_fwd" else PHASE_MFMAS[kern]
        if kern.startswith("plain"):  # one kernel per entry point: the kernel's whole-run rate
            stats["kernel_TFLOPs"] = round(total_flops / (t["product_us"] * 1e-6) / 1e12, 1)
            stats["kernel_frac_of_peak"] = round(total_flops / (t["product_us"] * 1e-6) /
                                                 (BF16_PEAK_TFLOPS * 1e12), 4)
        out[kern] = {**stats, **{k_ + ("" if kern.startswith("plain") else "_entry_point"): round(v_, 2)
                                 for k_, v_ in t.items()}}
    return out


def main():
    args = parse()
    if args.profile_kernels:
        profile_kernels()
        return
    if args.decode_only:
        print(json.dumps(decode_bench()), flush=True)
        return
    if args.phase_rates:
        print(json.dumps(phase_rates()), flush=True)
        return
    if args.profile_workload:
        profile_workload(args.profile_workload)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the carrier path has no "
              "multi-GPU exchange to measure here.", file=sys.stderr)
        raise SystemExit(2)
    res = gpu_bench(args)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args)
        res["cpu_baseline"]["host_cpu"] = _host_cpu()
        if not args.no_secondary:
            res["cpu_baselines_more"] = cpu_baselines_more(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
