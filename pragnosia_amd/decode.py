"""Greedy incremental generation with the decode step captured in a HIP graph (`src/bench.py:192-317`).

The prompt is read once, window by window, through the chunked kernels with the state carried; then each new token
is one recurrent step through every layer (the fused `aspin_decode_step` kernel for the carriers). The step is
captured once into a graph whose every input is a static device buffer: the token, the position index (which wraps
modulo the position table on the device) and each layer's state, which the step updates in place. Unlike the
reference, the argmax also runs inside the graph and writes the next token straight into the token buffer, so
consecutive replays need no host round trip; the generated ids accumulate in a device buffer read once at the end.
`steps_per_graph` steps are captured back to back into one graph to amortise its launch.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


class GreedyDecoder:
    def __init__(self, model, batch: int, steps_per_graph: int = 8):
        self.m = model
        self.B = batch
        self.K = steps_per_graph
        self.graph = None

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
                out.append((st[0].clone().contiguous(), p0.float().clone()))
            else:
                out.append(tuple(t.clone().contiguous() for t in st))
        return out

    def _one_step(self):
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
        self.out.index_copy_(0, self.ctr, nxt.view(1, -1))
        self.ctr.add_(1)
        self.tok.copy_(nxt.view(-1, 1))

    def _capture(self, states, n_max):
        dev = self.m.e.weight.device
        self.st = self._static_states(states)
        self.tok = torch.zeros(self.B, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.out = torch.zeros(n_max + self.K, self.B, dtype=torch.long, device=dev)
        self.ctr = torch.zeros(1, dtype=torch.long, device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                self._one_step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for _ in range(self.K):
                self._one_step()
        self.n_max = n_max

    @torch.no_grad()
    def start(self, states, pw, lg, n):
        """Load a prefilled state into the static buffers (capturing the graph on first use)."""
        if self.graph is None or n > self.n_max:
            self._capture(states, n)
        for a_, b_ in zip(self.st, self._static_states(states)):
            for a, b in zip(a_, b_):
                a.copy_(b)
        self.pos.fill_(pw)
        first = lg.argmax(-1)
        self.out.zero_()
        self.out[0].copy_(first)
        self.ctr.fill_(1)
        self.tok.copy_(first.view(-1, 1))

    @torch.no_grad()
    def replay(self, n):
        """Run ceil((n - 1) / steps_per_graph) graph replays (the first token came from the prefill's logits)."""
        for _ in range(-(-(n - 1) // self.K)):
            self.graph.replay()

    @torch.no_grad()
    def generate(self, prompt, n):
        """prompt (B, P) ids on the device; returns the n greedy tokens (B, n)."""
        states, pw, lg = self.prefill(prompt)
        self.start(states, pw, lg, n)
        self.replay(n)
        return self.out[:n].t().clone()


@torch.no_grad()
def greedy_eager(model, prompt, n):
    """The same generation without a graph, one eager step per token (the reference's generate() with temp 0).
    Returns (tokens (B, n), logits of every step (B, n, V))."""
    dec = GreedyDecoder(model, prompt.shape[0])
    states, pw, lg = dec.prefill(prompt)
    toks, lgs = [], []
    for _ in range(n):
        nxt = lg.argmax(-1)
        toks.append(nxt)
        lgs.append(lg)
        h = model.e(nxt[:, None]) + model.p(torch.full((1,), pw, device=prompt.device, dtype=torch.long))
        for i, (mx, mp) in enumerate(zip(model.mix, model.mlp)):
            h, states[i] = mx(h, states[i])
            h = mp(h)
        lg = F.linear(model.n(h), model.e.weight)[:, -1].float()
        pw = (pw + 1) % model.ctx
    return torch.stack(toks, 1), torch.stack(lgs, 1)
