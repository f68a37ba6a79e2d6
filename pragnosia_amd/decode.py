"""Greedy incremental generation with the decode step captured in a HIP graph (`src/bench.py:192-317`).

The prompt is read once, window by window, through the chunked kernels with the state carried; then each new token
is one recurrent step through every layer (the fused `aspin_decode_step` kernel for the carriers). The step is
captured once into a graph whose every input is a static device buffer: the token, the position index (which wraps
modulo the position table on the device) and each layer's state, which the step updates in place. Unlike the
reference, the argmax also runs inside the graph and writes the next token straight into the token buffer, so
consecutive replays need no host round trip; the generated ids accumulate in a device buffer read once at the end.
`steps_per_graph` steps are captured back to back into one graph to amortise its launch.

For an LM of associative carriers (aspin or dspin, LayerNorm) the step is fused: per layer one LayerNorm +
projection kernel (q, k, v, decay and gate or strength in one concatenated weight), one recurrent-step kernel that
forms the decay, gate or strength itself and writes the per-head RMS-normalised output, one kernel for the gated
output projection with the residual, and two for the MLP (LayerNorm + first layer + GELU; second layer + residual):
five kernels a layer instead of about twenty-five, the same fp32 arithmetic. Above GEMV_MAX_BATCH sequences the dense
layers run on the fp32 matrix cores (decode_gemm, the norms, biases, GELU and residuals inside), still five kernels
a layer (LayerNorm kernel and torch GEMMs where a width is not covered). Other mixers
run the modules' own T = 1 path. The concatenated weights are copied from the parameters at every `start`, so the
graph always sees the current parameters.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .assoc import AssocCarrier
from .ops import decode_gemm_ln, decode_gemm_ok, decode_gemm_tile, decode_tail, ln_supported


# The fused step's dense layers run as the batched GEMV kernel (each weight read once a step) up to this many
# sequences; beyond it on the fp32 matrix cores (decode_gemm: the LayerNorm, the per-head RMSNorm, the bias, GELU and
# the residual inside, weights tiled and the norms' weights folded in once per `start`), the carrier step fused and
# split four workgroups a head. Measured on the 12-layer d768 LM with the earlier 256-thread GEMV, ms a step (GEMV /
# torch GEMMs, both with the fused step): batch 1 0.45 / 0.77, 4 0.71 / 0.75, 8 1.06 / 0.76, 32 1.18 / 0.85, 64 2.05
# / 0.83; the unfused step with torch GEMMs: 1.45-1.57. The one-wave GEMV (up to 4 sequences) and the split carrier
# step bring batch 1 to 0.31.
GEMV_MAX_BATCH = 4
# On the decode_gemm path, a dense layer with a residual and at least this input width (the MLP's second layer, K =
# 4 d) runs as decode_gemm_acc_: its K split over groups of workgroups adding into the residual in place, so its
# column tiles' workgroups fill more compute units.
GEMM_ACC_MIN_K = 1024
# ... and the carrier's RMSNorm + gated o-projection adds into the residual in place, its K split over head groups.
OPROJ_ACC = True
# Up to GEMV_MAX_BATCH sequences, the MLP's second layer as the accumulating one-wave GEMV (decode_gemv_acc_: K split
# over workgroups adding into the residual in place).
GEMV_ACC = True


def _rms_gemv_ok(K: int) -> bool:
    """Whether decode_gemv_rms covers the carrier output of width K (B <= GEMV_MAX_BATCH)."""
    return K % 256 == 0 and K <= 1024


def fused_decode_ok(model, batch: int = 1) -> bool:
    """Whether `model`'s decode step can run fused at this batch size: every mixer an AssocCarrier with 64- or
    128-dim heads and no key_topk, beta_scale or short convolution, LayerNorms throughout and the standard MLP. The
    128-dim step writes its output raw, so its per-head RMSNorm must fit the consumer: the o-projection's GEMV up to
    GEMV_MAX_BATCH sequences, decode_gemm's 128-channel RMS mode past it."""
    import torch.nn as nn
    if not (isinstance(model.n, nn.LayerNorm) and getattr(model, "short_conv", 0) == 0):
        return False
    for mx, mp in zip(model.mix, model.mlp):
        if not (isinstance(mx, AssocCarrier) and mx.dk in (64, 128) and not mx.key_topk
                and getattr(mx, "beta_scale", None) is None and isinstance(mx.ln, nn.LayerNorm)
                and mx.on.weight is not None and isinstance(mp.n, nn.LayerNorm)):
            return False
        if mx.dk == 128:
            K = mx.h * mx.dk
            if not (_rms_gemv_ok(K) if batch <= GEMV_MAX_BATCH else _gemm_layers_ok(model)):
                return False
    return True


def _gemm_layers_ok(model) -> bool:
    """Whether decode_gemm covers every dense layer's input width of `model`'s step (the LayerNorm'd d-wide inputs,
    the per-head RMSNorm'd carrier outputs, the MLP's hidden width)."""
    hid = model.mlp[0].a.weight.shape[0]
    if not (decode_gemm_ok(model.d, 1) and decode_gemm_ok(hid, 0)):
        return False
    return all(decode_gemm_ok(mx.h * mx.dk, 2 if mx.dk == 64 else 3) for mx in model.mix)


class GreedyDecoder:
    def __init__(self, model, batch: int, steps_per_graph: int = 8, fused: bool | None = None,
                 record_logits: bool = False):
        """record_logits: the captured step also writes each step's logits (fp32) into a device buffer of
        (n + steps_per_graph, batch, vocab), read with `logits(n)`; for checking the graphed path itself against a
        reference decode, at the cost of one (batch, vocab) copy a step."""
        self.m = model
        self.B = batch
        self.K = steps_per_graph
        self.record = record_logits
        self.lgs = None
        self.graph = None
        self.fused = fused_decode_ok(model, batch) if fused is None else fused
        if self.fused and not fused_decode_ok(model, batch):
            raise ValueError("GreedyDecoder: this model's decode step cannot run fused")
        if self.fused and steps_per_graph % 2:
            raise ValueError("GreedyDecoder: the fused step captures an even number of steps per graph (its tail "
                             "alternates two counter slots)")

    @torch.no_grad()
    def prefill(self, ids):
        """ids (B, P) on the device. Returns (states, pw, last logits (B, V)); pw is the position index of the next
        token (P mod ctx), as the reference's generate() computes it."""
        m, w = self.m, self.m.ctx
        states = [None] * m.layers
        lg, pw = None, 0
        for s in range(0, ids.shape[1], w):
            x = ids[:, s:s + w]
            h = m.e(x) + m.p(torch.arange(x.shape[1], device=x.device))
            for i, (mx, mp) in enumerate(zip(m.mix, m.mlp)):
                h, states[i] = mx(h, states[i])
                h = mp(h)
            lg = F.linear(m.n(h[:, -1:]), m.e.weight)[:, -1].float()
            pw = x.shape[1] % w
        return states, pw, lg

    def _static_states(self, states):
        out = []
        for st in states:
            if isinstance(st[1], (int, float)) or (torch.is_tensor(st[1]) and st[1].dim() == 0):
                p0 = st[1] if torch.is_tensor(st[1]) else torch.tensor(float(st[1]), device=st[0].device)
                # (S, position) or, with a short convolution, (S, position, cache)
                out.append((st[0].clone().contiguous(), p0.float().clone(),
                            *(t.clone().contiguous() for t in st[2:])))
            else:
                out.append(tuple(t.clone().contiguous() for t in st))
        return out

    def _one_step(self, par=0):
        m = self.m
        h = m.e(self.tok) + m.p(self.pos)
        for i, (mx, mp) in enumerate(zip(m.mix, m.mlp)):
            h, new = mx(h, self.st[i])
            h = mp(h)
            for a, b in zip(self.st[i], new):
                if torch.is_tensor(b):
                    a.copy_(b)
                else:
                    a.fill_(float(b))
        self.pos.copy_((self.pos + 1) % m.ctx)
        lg = F.linear(m.n(h), m.e.weight)[:, -1]
        nxt = lg.argmax(-1)
        if self.lgs is not None:
            self.lgs.index_copy_(0, self.ctr, lg.float().view(1, self.B, -1))
        self.out.index_copy_(0, self.ctr, nxt.view(1, -1))
        self.ctr.add_(1)
        self.tok.copy_(nxt.view(-1, 1))

    def _gemm_ok(self) -> bool:
        """Whether the dense layers run on decode_gemm: past the GEMV's batch sizes, every layer's input width
        covered."""
        return self.B > GEMV_MAX_BATCH and _gemm_layers_ok(self.m)

    def _fused_weights(self):
        """Per layer: the concatenated input projection (q, k, v, decay, then the gate or strength), the output gate
        sigmoid(g) as a device scalar and the output projection pre-scaled by it (for the GEMM form), written into
        the same buffers every time (the graph reads them). On the decode_gemm path, instead of the GEMM form: each
        dense layer's weight tiled, its input LayerNorm's (or the carrier's RMSNorm's) weight folded into the tiled
        columns, the LayerNorm's bias into the layer's bias, with the folded weights' row sums."""
        m = self.m
        fresh = []
        for mx, mp in zip(m.mix, m.mlp):
            gated = not (mx.delta or mx.write_all)
            extra = [mx.wi.weight] if gated else ([mx.wb.weight] if mx.delta else [])
            sig = torch.sigmoid(mx.gate.detach().float()).reshape(1)
            wcat = torch.cat([mx.q.weight, mx.k.weight, mx.v.weight, mx.wa.weight] + extra).detach().float()
            if self.gemm:
                tp, cp, bp = decode_gemm_ln(wcat, mx.ln.weight, mx.ln.bias, None)
                ta, ca, ba = decode_gemm_ln(mp.a.weight, mp.n.weight, mp.n.bias, mp.a.bias)
                fresh.append((tp, cp, bp, sig, decode_gemm_tile(mx.o.weight, mx.on.weight), ta, ca, ba,
                              decode_gemm_tile(mp.b.weight)))
            else:
                fresh.append((wcat, sig, mx.o.weight.detach().float() * sig))
        if self.gemm:
            fresh.append(decode_gemm_ln(m.e.weight, m.n.weight, m.n.bias, None))
        if getattr(self, "wbuf", None) is None:
            self.wbuf = [tuple(t.contiguous() for t in f) for f in fresh]
        else:
            for dst, src in zip(self.wbuf, fresh):
                for d, t in zip(dst, src):
                    d.copy_(t)
        if not self.gemm:
            self.wcat = [f[0] for f in self.wbuf]
            self.sig = [f[1] for f in self.wbuf]
            self.wos = [f[2] for f in self.wbuf]

    def _dense(self, x, W, ln, bias=None, scale=None, act=0, resid=None):
        """act(scale * (W LayerNorm(x)) + bias) + resid: the batched GEMV kernel up to GEMV_MAX_BATCH sequences,
        else the LayerNorm kernel and torch's GEMM (matrix cores) with the same epilogue."""
        if self.B <= GEMV_MAX_BATCH:
            return torch.ops.pragnosia.decode_gemv(x, W, None if ln is None else ln.weight,
                                                   None if ln is None else ln.bias, 0.0 if ln is None else ln.eps,
                                                   bias, scale, act, resid)
        if ln is None:
            z = x
        elif ln_supported(x, ln):
            z = torch.ops.pragnosia.layer_norm(x, ln.weight, ln.bias, ln.eps, False)[0]  # the LayerNorm kernel
        else:
            z = F.layer_norm(x, (x.shape[-1],), ln.weight, ln.bias, ln.eps)
        y = F.linear(z, W, bias)
        if act == 1:
            y = F.gelu(y)
        if scale is not None:
            return torch.addcmul(resid, y, scale) if resid is not None else y * scale
        return y + resid if resid is not None else y

    def _one_step_gemm(self, par=0):
        """The fused step past GEMV batch sizes: five kernels a layer, all on the fp32 matrix cores but the carrier
        step (LayerNorm + projection; the step, split dk / 16 workgroups a head, raw output; per-head RMSNorm + gated
        o-projection + residual; LayerNorm + MLP in + GELU; MLP out + residual), then LayerNorm + head and the step's
        tail (argmax, next input)."""
        m, op = self.m, torch.ops.pragnosia
        h = self.h
        for i, (mx, mp) in enumerate(zip(m.mix, m.mlp)):
            gated = not (mx.delta or mx.write_all)
            tp, cp, bp, sig, to, ta, ca, ba, tb = self.wbuf[i]
            P = op.decode_gemm(h, tp, cp.shape[0], 1, cp, mx.ln.eps, bp, None, 0, None)
            on_eps = mx.on.eps if mx.on.eps is not None else torch.finfo(torch.float32).eps
            o = op.aspin_decode_proj_(self.st[i][0], P, mx.h, mx.wa.bias, mx.A,
                                      mx.la_floor if mx.hl_floor else None, mx.wi.bias if gated else None,
                                      mx.wb.bias if mx.delta else None, 0.75 if (mx.delta and mx.write_all) else 0.0,
                                      gated, mx.theta, self.p0s[i:i + 1], 0.0, None, on_eps)
            if OPROJ_ACC:
                # h += sigmoid(g) W_o RMSNorm(o): the residual in place (h is not read again this step: the
                # projection above has consumed it, and the tail rewrites the step's input)
                op.decode_gemm_acc_(o, to, 2 if mx.dk == 64 else 3, on_eps, None, sig, h)
                x1 = h
            else:
                x1 = op.decode_gemm(o, to, m.d, 2 if mx.dk == 64 else 3, None, on_eps, None, sig, 0, h)
            hm = op.decode_gemm(x1, ta, ca.shape[0], 1, ca, mp.n.eps, ba, None, 1, None)
            if hm.shape[1] >= GEMM_ACC_MIN_K:
                op.decode_gemm_acc_(hm, tb, 0, 0.0, mp.b.bias, None, x1)  # x1 += W hm + bias: the residual in place
                h = x1
            else:
                h = op.decode_gemm(hm, tb, m.d, 0, None, 0.0, mp.b.bias, None, 0, x1)
        th, ch, bh = self.wbuf[-1]
        self._tail(op.decode_gemm(h, th, ch.shape[0], 1, ch, m.n.eps, bh, None, 0, None), par)

    def _tail(self, lg, par):
        """The step's end in one kernel (decode_tail): argmax, the token written to the output row and the token
        buffer, the position advanced, the next step's input embedding into `self.h`, every carried state's position
        offset reset to 1 (one-token calls from here on), the logits recorded when asked. The row counter and the
        position alternate between two int64 slots (read slot `par`, write the other), so a captured graph of an even
        number of steps replays where the last replay ended."""
        m = self.m
        decode_tail(lg, m.e.weight, m.p.weight, self.ctrb[par], self.ctrb[1 - par], self.posb[par],
                    self.posb[1 - par], self.out, self.tok, self.h, self.p0s, self.lgs)

    def _one_step_fused(self, par=0):
        m, op = self.m, torch.ops.pragnosia
        h = self.h
        for i, (mx, mp) in enumerate(zip(m.mix, m.mlp)):
            gated = not (mx.delta or mx.write_all)
            P = self._dense(h, self.wcat[i], mx.ln)
            on_eps = mx.on.eps if mx.on.eps is not None else torch.finfo(torch.float32).eps
            if self.st2[i] is not None:
                # 64-wide heads at small batches: the step, the per-head RMSNorm and the gated o-projection in one
                # launch, added into h in place (h becomes x1); the state alternates between two buffers by step
                # parity (every workgroup of a head reads the old state), ending in st[i][0] after an even count
                src, dst = (self.st[i][0], self.st2[i]) if par == 0 else (self.st2[i], self.st[i][0])
                op.aspin_decode_oproj_(src, dst, P, mx.h, mx.wa.bias, mx.A, mx.la_floor if mx.hl_floor else None,
                                       mx.wi.bias if gated else None, mx.wb.bias if mx.delta else None,
                                       0.75 if (mx.delta and mx.write_all) else 0.0, gated, mx.theta,
                                       self.p0s[i:i + 1], 0.0, mx.on.weight, on_eps, mx.o.weight, self.sig[i], h)
                x1 = h
                hm = self._dense(x1, mp.a.weight, mp.n, bias=mp.a.bias, act=1)
                if GEMV_ACC and hm.shape[1] % 256 == 0 and hm.shape[1] <= 4096:
                    op.decode_gemv_acc_(hm, mp.b.weight, mp.b.bias, None, x1)  # x1 += W hm + bias, in place
                    h = x1
                else:
                    h = self._dense(hm, mp.b.weight, None, bias=mp.b.bias, resid=x1)
                continue
            # at small batches the per-head RMSNorm moves into the o-projection's GEMV, so the carrier step can run
            # dk / 16 workgroups per head (always so for 128-dim heads, whose step writes only the raw output)
            rms_in_gemv = self.B <= GEMV_MAX_BATCH and _rms_gemv_ok(mx.h * mx.dk)
            o = op.aspin_decode_proj_(self.st[i][0], P, mx.h, mx.wa.bias, mx.A,
                                      mx.la_floor if mx.hl_floor else None, mx.wi.bias if gated else None,
                                      mx.wb.bias if mx.delta else None, 0.75 if (mx.delta and mx.write_all) else 0.0,
                                      gated, mx.theta, self.p0s[i:i + 1], 0.0,
                                      None if rms_in_gemv else mx.on.weight, on_eps)
            if rms_in_gemv:
                x1 = op.decode_gemv_rms(o, mx.o.weight, mx.on.weight, on_eps, None, self.sig[i], 0, h)
            elif self.B <= GEMV_MAX_BATCH:
                x1 = self._dense(o, mx.o.weight, None, scale=self.sig[i], resid=h)
            else:  # h + o (sigmoid(g) W_o)^T in one GEMM
                x1 = torch.addmm(h, o, self.wos[i].t())
            hm = self._dense(x1, mp.a.weight, mp.n, bias=mp.a.bias, act=1)
            h = self._dense(hm, mp.b.weight, None, bias=mp.b.bias, resid=x1)
        self._tail(self._dense(h, m.e.weight, m.n), par)

    def _capture(self, states, n_max):
        dev = self.m.e.weight.device
        self.st = self._static_states(states)
        if self.fused:
            self.gemm = self._gemm_ok()
            self._fused_weights()
            self.p0s = torch.stack([st[1].reshape(()) for st in self.st]).float().contiguous()
            # the one-launch step + o-projection (64-wide heads, GEMV batch sizes) writes the new state to a second
            # buffer, the two swapping roles every step
            self.st2 = [torch.empty_like(st[0]) if (not self.gemm and self.B <= GEMV_MAX_BATCH and mx.dk == 64)
                        else None for st, mx in zip(self.st, self.m.mix)]
        self.tok = torch.zeros(self.B, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.out = torch.zeros(n_max + self.K, self.B, dtype=torch.long, device=dev)
        self.ctr = torch.zeros(1, dtype=torch.long, device=dev)
        if self.fused:  # the fused step's input and the tail kernel's alternating counter and position slots
            self.h = torch.zeros(self.B, self.m.d, device=dev)
            self.ctrb = torch.zeros(2, dtype=torch.long, device=dev)
            self.posb = torch.zeros(2, dtype=torch.long, device=dev)
        if self.record:
            self.lgs = torch.zeros(n_max + self.K, self.B, self.m.e.weight.shape[0], dtype=torch.float32, device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        step = (self._one_step if not self.fused else self._one_step_gemm if self.gemm else self._one_step_fused)
        with torch.cuda.stream(side):
            for i in range(2):
                step(i % 2)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for i in range(self.K):
                step(i % 2)
        self.n_max = n_max

    @torch.no_grad()
    def start(self, states, pw, lg, n):
        """Load a prefilled state into the static buffers (capturing the graph on first use)."""
        if self.graph is None or n > self.n_max:
            self._capture(states, n)
        for a_, b_ in zip(self.st, self._static_states(states)):
            for a, b in zip(a_, b_):
                a.copy_(b)
        if self.fused:
            self._fused_weights()
            self.p0s.copy_(torch.stack([st[1].reshape(()) for st in self.st]).float())
        self.pos.fill_(pw)
        first = lg.argmax(-1)
        self.out.zero_()
        self.out[0].copy_(first)
        if self.lgs is not None:
            self.lgs.zero_()
            self.lgs[0].copy_(lg.float())
        self.ctr.fill_(1)
        self.tok.copy_(first.view(-1, 1))
        if self.fused:
            self.ctrb.fill_(1)
            self.posb.fill_(pw)
            self.h.copy_((self.m.e(self.tok) + self.m.p(self.pos)).reshape(self.B, -1))

    @torch.no_grad()
    def replay(self, n):
        """Run ceil((n - 1) / steps_per_graph) graph replays (the first token came from the prefill's logits)."""
        for _ in range(-(-(n - 1) // self.K)):
            self.graph.replay()

    def logits(self, n):
        """With record_logits: the logits each of the last run's first n tokens was chosen from, (batch, n, vocab)
        (step 0's are the prefill's)."""
        if self.lgs is None:
            raise ValueError("GreedyDecoder: constructed without record_logits")
        return self.lgs[:n].transpose(0, 1)

    @torch.no_grad()
    def generate(self, prompt, n):
        """prompt (B, P) ids on the device; returns the n greedy tokens (B, n)."""
        states, pw, lg = self.prefill(prompt)
        self.start(states, pw, lg, n)
        self.replay(n)
        return self.out[:n].t().clone()


@torch.no_grad()
def greedy_eager(model, prompt, n, forced=None):
    """The same generation without a graph, one eager step per token (the reference's generate() with temp 0).
    `forced` (B, n) replaces each argmax by the given token (teacher forcing), so the logits of another run's tokens
    can be compared step by step. Returns (tokens (B, n), logits of every step (B, n, V))."""
    dec = GreedyDecoder(model, prompt.shape[0])
    states, pw, lg = dec.prefill(prompt)
    toks, lgs = [], []
    for step in range(n):
        nxt = lg.argmax(-1) if forced is None else forced[:, step]
        toks.append(nxt)
        lgs.append(lg)
        h = model.e(nxt[:, None]) + model.p(torch.full((1,), pw, device=prompt.device, dtype=torch.long))
        for i, (mx, mp) in enumerate(zip(model.mix, model.mlp)):
            h, states[i] = mx(h, states[i])
            h = mp(h)
        lg = F.linear(model.n(h), model.e.weight)[:, -1].float()
        pw = (pw + 1) % model.ctx
    return torch.stack(toks, 1), torch.stack(lgs, 1)
