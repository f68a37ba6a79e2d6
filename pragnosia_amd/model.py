"""The carrier language model around the hot path: LM with forward, trunk and forward_carried (`src/model.py`).

Constructor arguments, module names and initialisation follow the reference (`src/model.py:552-560`, `:621-738`), so
`LM(**cfg).load_state_dict(sd)` takes a reference checkpoint of a supported mixer:

    "aspin"   AssocCarrier(d)                                      plain write rule, 64-dim heads
    "dspin"   AssocCarrier(d, delta=True)                          delta write rule
    "hspin"   AssocCarrier(d, head_dim=128)                        plain rule, 128-dim heads (four 64 x 64 scans)
    "hspin1"  AssocCarrier(d, head_dim=128, write_all=True)        ... with no write gate
    "hdspin"  AssocCarrier(d, delta=True, head_dim=128)            delta rule, 128-dim heads
    "sdspin"  ... + key_topk=8;  "tspin" ... + hl_floor=True;  "aspin1" ... + write_all=True
    "wspin"   AssocCarrier(d, heads=4)                             plain rule, four wide heads (d / 4)
    "w2spin"  AssocCarrier(d, heads=2)                             plain rule, two wide heads (d / 2)
    "xspin"   AssocCarrier(d, delta=True, heads=4)                 delta rule, four heads (up to 384 wide)
    "fspin"   SpinCarrier(d, gated="rf")                           forget-gated complex diagonal carrier

(`src/model.py:632-660`.) The mixers run on the HIP kernels: heads of 64 and 128 on the bf16 MFMA scans, other head
widths on the exact fp32 scan (the plain rule at any width, in key blocks of at most 128; the delta rule with keys up
to 384; value columns split to fit the LDS). Embeddings, LayerNorms, the MLPs and the tied head are torch. Attention, the hybrid stacks and the other
reference mixers are outside this build and raise. `short_conv=K` adds every carrier's short causal convolution
(`src/model.py:717-726`).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

from ._lib import PragnosiaError
from .assoc import AssocCarrier
from .ops import layer_norm, linear
from .spin import SpinCarrier

MIXERS = {
    "aspin": lambda d: AssocCarrier(d),
    "dspin": lambda d: AssocCarrier(d, delta=True),
    "hspin": lambda d: AssocCarrier(d, head_dim=128),
    "hspin1": lambda d: AssocCarrier(d, head_dim=128, write_all=True),
    "hdspin": lambda d: AssocCarrier(d, delta=True, head_dim=128),
    "sdspin": lambda d: AssocCarrier(d, delta=True, head_dim=128, key_topk=8),
    "tspin": lambda d: AssocCarrier(d, delta=True, head_dim=128, hl_floor=True),
    "aspin1": lambda d: AssocCarrier(d, delta=True, head_dim=128, write_all=True),
    "wspin": lambda d: AssocCarrier(d, heads=4),
    "w2spin": lambda d: AssocCarrier(d, heads=2),
    "xspin": lambda d: AssocCarrier(d, delta=True, heads=4),
    "fspin": lambda d: SpinCarrier(d, gated="rf"),
}


class MLP(nn.Module):
    def __init__(self, d: int, mult: int = 4):
        super().__init__()
        self.n = nn.LayerNorm(d)
        self.a = nn.Linear(d, mult * d)
        self.b = nn.Linear(mult * d, d)

    def forward(self, x):
        # the biases' gradients as GEMMs, so a captured training step records no memset (ops.linear); the norm on
        # its kernel, in the dtype the first matmul computes in (ops.layer_norm)
        return x + linear(F.gelu(linear(layer_norm(x, self.n), self.a)), self.b)


class LM(nn.Module):
    def __init__(self, vocab=8192, d=768, layers=12, mlp_mult=4, ctx=512, mixer="aspin", norm="ln", short_conv=0,
                 **unused):
        super().__init__()
        if mixer not in MIXERS:
            raise PragnosiaError(f"LM: mixer {mixer!r} is outside this build (supported: {sorted(MIXERS)})")
        self.vocab, self.d, self.layers, self.ctx, self.mixer, self.norm = vocab, d, layers, ctx, mixer, norm
        self.e = nn.Embedding(vocab, d)
        self.p = nn.Embedding(ctx, d)
        self.mix = nn.ModuleList([MIXERS[mixer](d) for _ in range(layers)])
        self.mlp = nn.ModuleList([MLP(d, mlp_mult) for _ in range(layers)])
        self.n = nn.LayerNorm(d)
        if norm == "rms":
            for mod in list(self.modules()):
                for name, child in list(mod.named_children()):
                    if isinstance(child, nn.LayerNorm):
                        setattr(mod, name, nn.RMSNorm(child.normalized_shape[0]))
        self.apply(self._init)
        self.short_conv = 0
        if short_conv:
            self.add_short_conv(short_conv)

    def add_short_conv(self, K: int):
        """A short causal convolution over the last K tokens on every carrier's q, k and v, initialised as the
        identity (`src/model.py:721-726`); the carriers' states then carry the convolution's cache."""
        for mx in self.mix:
            if hasattr(mx, "add_short_conv"):
                mx.add_short_conv(K)
        self.short_conv = K
        return self

    @staticmethod
    def _init(m):
        """N(0, 0.02) for every embedding and Linear weight, zero biases (`src/model.py:729-738`); applied after the
        mixers' own constructors, so it overrides their initialisation of Linear layers."""
        if isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, 0.0, 0.02)
        elif isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, 0.0, 0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)

    def _embed(self, x, positions):
        return self.e(x) + self.p(positions)

    def trunk(self, x, states=None, carry=False):
        """The normalised final representation (B, T, d); with carry=True, `states` are the layers' states from the
        previous window (None at a stream's start) and the new ones are returned too (`src/model.py:759-789`)."""
        h = self._embed(x, torch.arange(x.shape[1], device=x.device) % self.p.num_embeddings)
        new = []
        for i, (mx, mp) in enumerate(zip(self.mix, self.mlp)):
            st = states[i] if states is not None else None
            o, st = mx(h, st) if st is not None else mx(h)
            h = mp(o)
            new.append(st)
        return (self.n(h), new) if carry else self.n(h)

    def forward(self, x, return_hidden=False, hidden_layer=None):
        h = self._embed(x, torch.arange(x.shape[1], device=x.device) % self.p.num_embeddings)
        grab = None
        for i, (mx, mp) in enumerate(zip(self.mix, self.mlp)):
            h = mp(mx(h)[0])
            if hidden_layer is not None and i == hidden_layer:
                grab = h
        h = self.n(h)
        logits = F.linear(h, self.e.weight)
        if not return_hidden:
            return logits
        return logits, (h if grab is None else grab)

    def loss(self, h, y, chunks=4):
        """Mean cross-entropy of the tied head over (B, T) targets, the logits formed chunk by chunk under
        activation checkpointing so at most one chunk's logits exist at a time."""
        hf, yf = h.reshape(-1, h.shape[-1]), y.reshape(-1)
        n = hf.shape[0]

        def piece(hc, yc, E):
            # the logits as the reference forms them (`src/model.py:563-567`): bf16 under autocast on the GPU,
            # the cross-entropy in fp32
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=hc.is_cuda):
                lg = F.linear(hc, E)
            return F.cross_entropy(lg.float(), yc, reduction="sum")

        total = 0.0
        for i in range(chunks):
            sl = slice(i * n // chunks, (i + 1) * n // chunks)
            total = total + torch.utils.checkpoint.checkpoint(piece, hf[sl], yf[sl], self.e.weight,
                                                              use_reentrant=False)
        return total / n

    @torch.no_grad()
    def forward_carried(self, x, window=None):
        """A sequence longer than one window: windows of `window` tokens with every layer's state carried across the
        boundary and position embeddings restarting per window; returns the final window's logits
        (`src/model.py:842-864`). Computed layer by layer over the whole sequence (the same function as window by
        window: a layer's windows depend on each other only through its carried state, which each mixer's
        forward_windows threads through one pass)."""
        window = window or self.ctx
        T = x.shape[1]
        h = self._embed(x, torch.arange(T, device=x.device) % window)
        for mx, mp in zip(self.mix, self.mlp):
            h = mp(mx.forward_windows(h, window)[0])
        return F.linear(self.n(h[:, window * ((T - 1) // window):]), self.e.weight)
