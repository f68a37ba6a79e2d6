"""Benchmark of the carrier hot path on one MI355X: prints ONE JSON line.

Workload (the configuration the headline metric is quoted on): the aspin chunked scan,
forward + backward, B16 T512 H12 D64, chunk 64, bf16 q/k/v, fp32 log-decays and state, synthetic seeded inputs
resident in HBM. One step = one forward (writing o, the final state and the bf16 entering states) and one backward
(dq, dk, dv, dla, dS0 from dO and dS_final) through the HIP kernels, on one stream.

    python bench.py [--steps K] [--warmup W] [--rule plain|delta] [--no-cpu-baseline]

`value` is tokens (B * T) per second over the K timed steps. `roofline` is the dominant kernel's algorithmic HBM
bytes per launch over its average launch time, timed with HIP events on the stream it runs on. `cpu_baseline` is
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
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def inputs(B, H, T, D, seed, rule, device):
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


def gpu_bench(args):
    import torch
    from pragnosia_amd import ops  # noqa: F401
    B, H, T, D, C = 16, 12, 512, 64, 64
    NC = T // C
    dev = torch.device("cuda:0")
    x = inputs(B, H, T, D, 2, args.rule, dev)
    op = torch.ops.pragnosia
    if args.rule != "plain":
        raise SystemExit("bench.py: --rule delta is not built yet")

    stream = torch.cuda.current_stream(dev)

    def step():
        o, S, sent = op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
        grads = op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sent, x["do"], x["dS"])
        return o, grads

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1e3

    # per-kernel averages with HIP events on the launch stream
    n_ev = max(20, min(args.steps, 200))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    o, S, sent = op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
    ev[0].record(stream)
    for _ in range(n_ev):
        op.aspin_chunk(x["q"], x["k"], x["v"], x["la"], None, True)
    ev[1].record(stream)
    for _ in range(n_ev):
        op.aspin_chunk_bwd(x["q"], x["k"], x["v"], x["la"], sent, x["do"], x["dS"])
    ev[2].record(stream)
    torch.cuda.synchronize()
    t_fwd = ev[0].elapsed_time(ev[1]) / n_ev * 1e-3     # seconds per launch
    t_bwd = ev[1].elapsed_time(ev[2]) / n_ev * 1e-3

    elem = B * H * T * D
    ht = B * H * T
    state = B * H * D * D
    # algorithmic HBM bytes per launch: every tensor read or written once
    fwd_bytes = 3 * 2 * elem + 2 * elem + 4 * ht + 4 * state + 2 * (B * H * NC * D * D)   # q,k,v in; o, la, S, sent
    bwd_bytes = 4 * 2 * elem + 2 * (B * H * NC * D * D) + 4 * ht + 4 * state + 3 * 2 * elem + 4 * ht + 4 * state
    fwd_flops = 4 * D * (C + D) * ht
    bwd_flops = 10 * D * (C + D) * ht
    dom = ("aspin_plain_bwd", t_bwd, bwd_bytes, bwd_flops) if t_bwd >= t_fwd else \
          ("aspin_plain_fwd", t_fwd, fwd_bytes, fwd_flops)
    achieved = dom[2] / dom[1] / 1e9
    tokens = B * T
    res = {
        "metric": METRIC,
        "value": round(tokens / (wall / args.steps) / 1e6, 3),
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json configs[2] distributions)",
        "config": {"workload": f"aspin chunked scan fwd+bwd, {args.rule} rule, B16 T512 H12 D64 chunk64",
                   "B": B, "T": T, "H": H, "D": D, "chunk": C, "rule": args.rule},
        "roofline": {"bound": "hbm", "kernel": dom[0], "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": dom[2], "avg_launch_us": round(dom[1] * 1e6, 2),
                     "mfma_tflops": round(dom[3] / dom[1] / 1e12, 2)},
        "kernels_us": {"aspin_plain_fwd": round(t_fwd * 1e6, 2), "aspin_plain_bwd": round(t_bwd * 1e6, 2)},
    }
    return res


def cpu_baseline(args):
    """The CPU oracle (two-pass fp32 form, autograd backward) on B = 1 sequence of the cfg2 shape, repeated for
    about `cpu_seconds`; median per-iteration rate, in the metric's unit."""
    import torch
    from oracle import aspin as O
    torch.set_num_threads(os.cpu_count() if not os.environ.get("OMP_NUM_THREADS") else
                          int(os.environ["OMP_NUM_THREADS"]))
    B, H, T, D = 1, 12, 512, 64
    x = inputs(B, H, T, D, 2, "plain", "cpu")
    S0 = torch.zeros(B, H, D, D)

    def it():
        a = [x[n].clone().requires_grad_(True) for n in ("q", "k", "v", "la")]
        o, S, _ = O.scan_twopass(*a, S0, 64, None)
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
    return {"value": round(B * T / med / 1e6, 5), "unit": "Mtok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"CPU oracle (two-pass fp32 restatement of src/assoc.py:118-165, autograd backward), "
                      f"B=1 x T512 H12 D64 per iteration, {len(times)} iterations (~{args.cpu_seconds:.0f} s), "
                      "median"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the carrier path has no "
              "multi-GPU exchange to measure here.", file=sys.stderr)
        raise SystemExit(2)
    res = gpu_bench(args)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
