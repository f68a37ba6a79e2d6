"""The associative carrier (aspin / dspin) on the HIP kernels: the scan entry points and the AssocCarrier module.

Signatures, parameter names, initialisation and the state layout follow the reference (`src/assoc.py`), so a
reference state_dict loads unchanged and the callers (LM, forward_carried, the trainer, the decode loop) use this as
a drop-in. Every scan runs on the hand-written gfx950 kernels behind `torch.ops.pragnosia.*`:

    kernel path (T > 1):        aspin_rebase -> aspin_prep_proj / aspin_prep -> aspin_chunk / aspin_delta (bf16 MFMA)
    decode (T = 1, no autograd): aspin_decode_step (rebase, normalise, gate, write and read fused, fp32)
    torch path (kernel=False, T = 1 under autograd, other head dims): torch prep -> assoc_scan -> aspin_exact
                                (fp32 / fp64 operands; bf16 MFMA kernels under autocast)

The projections, LayerNorm, the decay and write-strength gates, the per-head RMSNorm and the gated output projection
are torch GEMMs and elementwise ops around them, as in the reference. There is no CPU path: a CPU tensor raises.
"""
from __future__ import annotations

import math
from contextlib import contextmanager

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops as _op_mod  # registers torch.ops.pragnosia.*
from ._lib import PragnosiaError

_op = torch.ops.pragnosia

# Module switches kept from the reference (`src/assoc.py:272-276`). FUSED_SCAN: delta carriers whose per-chunk
# entering states no later layer reads keep nothing from forward to backward but the scan's inputs (the reference
# switched to a third-party fused kernel there, which keeps the state on chip and recomputes chunk states in the
# backward; here `aspin_delta_fused` runs the same delta kernels and recomputes X, W and the entering states in its
# backward). FUSED_PROJ: one GEMM for the delta carrier's five input projections.
FUSED_SCAN = False
FUSED_PROJ = False
# This build's own switch for the plumbing around the plain-rule scan. True: one GEMM for the q, k, v, decay and
# write-gate projections, one kernel from its output to the scan's inputs (normalise, gate, rotate, decay, cast,
# transpose), and the per-head RMSNorm and transpose after the scan as one kernel, each with its own backward.
# False: the torch composition the reference uses (separate projections, elementwise decay and gate, nn.RMSNorm,
# transposes), kept for comparison.
FUSED_PLUMBING = True

HEAD_DIM_KERNEL = 64
_POS_CACHE: dict = {}


def rotate(x, theta, pos):
    """Rotation of interleaved channel pairs (x[..., 2i], x[..., 2i+1]) by angle pos * theta[h, i]
    (`src/assoc.py:34-39`): x (B, H, T, dk), theta (H, dk/2), pos (T,). A utility with the reference's signature;
    the module's own rotations run inside the prep, rebase and decode kernels."""
    ang = pos.reshape(1, 1, -1, 1).to(theta.dtype) * theta.reshape(1, theta.shape[0], 1, theta.shape[1])
    c, s = torch.cos(ang), torch.sin(ang)
    even, odd = x[..., 0::2], x[..., 1::2]
    return torch.stack((even * c - odd * s, even * s + odd * c), dim=-1).flatten(-2)


HEAD_DIM_WIDE = 128


def _plain_scan_wide(q, k, v, la, S0, want):
    """The plain rule at head dim 128 (the reference's `hspin` carrier, `src/model.py:650`, on its kernel path,
    `src/assoc.py:411`). The state's key rows evolve independently and o_t = S_t^T q_t sums over them, so with q = (q1,
    q2), k = (k1, k2), v = (v1, v2) in halves of 64,
        o[..., half vh] = scan(q1, k1, v_vh) + scan(q2, k2, v_vh),   S[half kh, half vh] = final state of
        scan(q_kh, k_kh, v_vh):
    four 64 x 64 scans per head in one launch over 4 H scans that read the halves in place (`aspin_chunk_wide`).
    Returns (o bf16 (B, H, T, 128), S_final fp32, sent per scan (B, H, 4, NC, 64, 64) bf16, or empty when not
    `want`; `ops.wide_sent` gives the whole states)."""
    return _op.aspin_chunk_wide(q, k, v, la.float(), S0, want)


def _rebase_wide(S, theta, p_dev, p_host):
    """Key rows (2i, 2i+1) of S rotated by -p0 theta[h, i] (`src/assoc.py:399-402`) as torch on the GPU, for states
    the rebase kernel does not take (heads other than 64 and 128 wide, fp64); p0 the device scalar p_dev when given,
    else p_host."""
    Dv = S.shape[-1]
    p = p_dev.float() if p_dev is not None else torch.tensor(p_host, device=S.device, dtype=torch.float32)
    return rotate(S.transpose(-1, -2), theta.float(), (-p).expand(Dv)).transpose(-1, -2).contiguous()


def _positions(T, device, wrap=None):
    if torch.compiler.is_compiling():  # traced code builds the tensor in the graph rather than caching it
        pos = torch.arange(T, device=device, dtype=torch.int64)
        return pos % wrap if wrap else pos
    key = (T, str(device), wrap)
    pos = _POS_CACHE.get(key)
    if pos is None:
        pos = torch.arange(T, device=device, dtype=torch.int64)
        if wrap:
            pos = pos % wrap
        _POS_CACHE[key] = pos
    return pos


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t is not None and torch.is_tensor(t) and t.requires_grad for t in ts)


def _kernel_ok(dk: int, dv: int, delta: bool) -> bool:
    """Whether the bf16-operand MFMA kernels take these heads: 64 or 128 wide, either rule."""
    return dk == dv and dk in (HEAD_DIM_KERNEL, HEAD_DIM_WIDE)


def assoc_scan(q, k, v, logalpha, S0=None, chunk: int = 64, recompute: bool = False, mm=None, beta=None,
               kernel=False, need_sent: bool = False):
    """The reference's dispatcher (`src/assoc.py:254-269`): o_t = S_t^T q_t with S_t = a_t S_{t-1} + k_t v_t^T (plain)
    or the delta rule when `beta` is given. q, k (B, H, T, Dk); v (B, H, T, Dv); logalpha, beta (B, H, T); S0
    (B, H, Dk, Dv) or None. Returns (o in q's dtype, S_final).

    As in the reference, the arithmetic is fp32, or fp64 for fp64 inputs (`rt`, `src/assoc.py:259-261`), with no
    operand rounding: the exact kernels (any head dims for the plain rule, keys up to 384 for the delta rule; wide heads
    run in blocks), S_final in that type. With `mm` a 16-bit type (the
    reference's bf16 matmuls under autocast, `:149-153`) the bf16-operand MFMA kernels run instead (fp32 accumulation
    and state; head dim 64 or 128), S_final fp32. The result does not depend on `chunk` (the
    reference's own test), and both paths recompute in the backward what they do not save, so `chunk`, `recompute`
    and `kernel` are accepted for the signature. need_sent (this build's): also return the bf16 entering state of
    every 64-token chunk, from the MFMA kernels."""
    lowp = mm in (torch.bfloat16, torch.float16)
    if need_sent or (lowp and _kernel_ok(q.shape[-1], v.shape[-1], beta is not None)):
        return _kernel_scan(q, k, v, logalpha, S0, beta, need_sent)
    rt = torch.float64 if q.dtype == torch.float64 else torch.float32
    want = _needs_grad(q, k, v, logalpha, S0, beta)
    cv = lambda t: None if t is None else t.to(rt)
    o, S = _exact_scan(cv(q), cv(k), cv(v), cv(logalpha), cv(beta), cv(S0), want)
    return o.to(q.dtype), S


def _dim_blocks(n: int, cap: int) -> list[tuple[int, int]]:
    """[start, end) ranges splitting n into the fewest near-equal blocks of at most cap."""
    nb = (n + cap - 1) // cap
    edges = [round(i * n / nb) for i in range(nb + 1)]
    return list(zip(edges[:-1], edges[1:]))


def _exact_scan(q, k, v, logalpha, beta, S0, want):
    """The exact scan (`ops.aspin_exact`) at the reference's wide head dims (`src/model.py:636-643`: four or two
    heads of 176-384). Value columns never mix (each is its own recurrence over the key rows), so every rule splits
    them into blocks that fit one launch's LDS (`exact_value_cap`). The plain rule's key rows evolve independently
    too and its read sums over them: with keys in blocks of at most 128, o[.., vb] = sum over key blocks kb of
    scan(q[.., kb], k[.., kb], v[.., vb]) and S[kb, vb] is that scan's state. The delta rule couples all key rows in
    every write (r = v - P^T k), so its keys stay in one launch, up to EXACT_MAX_DK = 384."""
    Dk, Dv = q.shape[-1], v.shape[-1]
    dt = torch.float64 if q.dtype == torch.float64 else torch.float32
    if beta is not None and Dk > _op_mod.EXACT_MAX_DK:
        raise PragnosiaError(f"assoc_scan: the delta rule takes key dims up to {_op_mod.EXACT_MAX_DK} (got {Dk}): "
                             "its state does not split into key blocks")
    kblocks = [(0, Dk)] if beta is not None else _dim_blocks(Dk, 128)
    vcap = min(_op_mod.exact_value_cap(k1 - k0, dt, bool(want)) for k0, k1 in kblocks)
    if len(kblocks) == 1 and Dv <= vcap:
        o, S, _, _ = _op.aspin_exact(q, k, v, logalpha, beta, S0, want)
        return o, S
    outs, cols = [], []
    for v0, v1 in _dim_blocks(Dv, vcap):
        o_vb, rows = None, []
        for k0, k1 in kblocks:
            S0b = None if S0 is None else S0[..., k0:k1, v0:v1]
            o_b, S_b, _, _ = _op.aspin_exact(q[..., k0:k1], k[..., k0:k1], v[..., v0:v1], logalpha, beta, S0b, want)
            o_vb = o_b if o_vb is None else o_vb + o_b
            rows.append(S_b)
        outs.append(o_vb)
        cols.append(rows[0] if len(rows) == 1 else torch.cat(rows, dim=-2))
    return torch.cat(outs, dim=-1), torch.cat(cols, dim=-1)


def _kernel_scan(q, k, v, logalpha, S0, beta, need_sent):
    """The bf16-operand MFMA kernels: q, k, v (B, H, T, 64 or 128), operands rounded to bf16,
    accumulation and state fp32. Returns (o in q's dtype, S_final fp32) and, when need_sent, the bf16 state entering
    every 64-token chunk."""
    wide = q.shape[-1] == HEAD_DIM_WIDE and beta is None
    if not _kernel_ok(q.shape[-1], v.shape[-1], beta is not None):
        raise PragnosiaError(f"assoc_scan: head dim {q.shape[-1]} is not supported by the bf16 kernels (64 or 128)")
    want = bool(need_sent or _needs_grad(q, k, v, logalpha, S0, beta))
    S0 = None if S0 is None else S0.float()
    if wide:
        o, S, sent = _plain_scan_wide(q, k, v, logalpha, S0, want)
        sent = _op_mod.wide_sent(sent) if need_sent else sent
    elif beta is None:
        o, S, sent = _op.aspin_chunk(q, k, v, logalpha.float(), S0, want)
    else:
        o, S, sent, _, _ = _op.aspin_delta(q, k, v, logalpha.float(), beta.float(), S0, want)
        sent = sent.transpose(-1, -2) if need_sent else sent  # the op stores each state transposed
    o = o.to(q.dtype) if q.dtype != torch.bfloat16 else o
    if need_sent:
        return o, S, sent
    return o, S


def assoc_scan_kernel(q, k, v, logalpha, S0=None, bv: int = 16):
    """Plain rule; the contract of the reference's `assoc_scan_kernel` (`src/assoc_kernel.py:302-323`):
    returns (o in q's dtype, S_final fp32, sent bf16 (B, H, NC, 64, 64))."""
    return _kernel_scan(q, k, v, logalpha, S0, None, True)


def delta_scan_kernel(q, k, v, logalpha, beta, S0=None, chunk: int = 64, bv: int = 32, bv_bwd: int = 16):
    """Delta rule; the contract of the reference's `delta_scan_kernel` (`src/assoc_kernel.py:512-546`)."""
    return _kernel_scan(q, k, v, logalpha, S0, beta, True)


def prep_kernel(qp, kp, vp, gate_logits, theta, pos):
    """The reference's `prep_kernel` (`src/assoc_kernel.py:888-891`): (B, T, H, D) projections -> bf16 q, k, v in
    (B, H, T, D), unit-normalised, k gated, q and k rotated by pos * theta."""
    return _op.aspin_prep(qp, kp, vp, gate_logits, theta, pos)


class AssocCarrier(nn.Module):
    """Per-head key-value outer-product memory with per-token forgetting, learned rotation frequencies and an
    optional delta write rule (`src/assoc.py:279-512`). Constructor arguments, parameters and paths are the
    reference's: with `kernel` (and T > 1, head dim 64 or 128) the bf16-operand MFMA kernels with
    the fused prep; otherwise (kernel=False, a T = 1 call under autograd, other head dims: any width for the plain
    rule, up to 384 for the delta rule) the reference's torch composition around the exact fp32 scan (bf16 MFMA kernels under autocast, as the reference's bf16 matmuls);
    a T = 1 call without autograd (decode) the fused fp32 step kernel. Options: key_topk, hl_floor, write_all,
    beta_scale, FUSED_PROJ, pos_wrap, and the short causal convolution with its carried cache (add_short_conv)."""

    def __init__(self, d: int, heads: int | None = None, chunk: int = 64, recompute: bool = False,
                 delta: bool = False, head_dim: int | None = None, kernel: bool = True, key_topk: int = 0,
                 hl_floor: bool = False, write_all: bool = False):
        super().__init__()
        self.d, self.recompute, self.delta = d, recompute, delta
        self.key_topk, self.hl_floor, self.write_all = key_topk, hl_floor, write_all
        self.need_sent = True
        self.kernel = kernel
        self.bv = 32
        self.h = heads or max(1, d // (head_dim or 64))
        if d % self.h or (d // self.h) % 2:
            raise ValueError(f"AssocCarrier: d={d} must split into {self.h} heads of even width")
        self.dk = d // self.h
        self.chunk = chunk
        self.ln = nn.LayerNorm(d)
        self.q = nn.Linear(d, d, bias=False)
        self.k = nn.Linear(d, d, bias=False)
        self.v = nn.Linear(d, d, bias=False)
        self.o = nn.Linear(d, d, bias=False)
        self.wa = nn.Linear(d, self.h)
        nn.init.zeros_(self.wa.weight)
        nn.init.zeros_(self.wa.bias)
        self.wi = nn.Linear(d, self.h)
        if delta:
            self.wb = nn.Linear(d, self.h)
        # per-head timescales spread geometrically at init: softplus(0) * exp(A) from 0.1 down to 1e-4
        self.A = nn.Parameter(torch.linspace(math.log(0.1 / 0.69), math.log(1e-4 / 0.69), self.h))
        if hl_floor:
            half_lives = torch.logspace(math.log10(8.0), math.log10(131072.0), self.h)
            self.register_buffer("la_floor", -math.log(2.0) / half_lives, persistent=False)
        inv_freq = 10000.0 ** (-torch.arange(0, self.dk, 2).float() / self.dk)
        self.theta = nn.Parameter(inv_freq.unsqueeze(0).repeat(self.h, 1))
        self.on = nn.RMSNorm(self.dk)
        self.gate = nn.Parameter(torch.zeros(()))
        self.sent = None

    @property
    def sent(self):
        """The bf16 state entering every chunk of the last kernel-path call, (B, H, NC, dk, dk), or None (the
        reference's `self.sent`, `src/assoc.py:349,510`, which its retrieval layers read). The kernels run 64-token
        chunks; a delta carrier built with chunk=128 (the reference's 128-token delta kernel, `src/assoc.py:494-495`)
        gets the states entering every 128-token chunk, those of every other 64-token one (the result does not depend
        on the chunk). The 128-wide scan keeps it per 64 x 64 block; it is assembled on first read."""
        s = self.__dict__.get("_sent")
        if s is not None and s.dim() == 6:
            s = _op_mod.wide_sent(s)
            self.__dict__["_sent"] = s
        if s is not None and self.delta and self.chunk == 128:
            s = s[:, :, ::2]
        return s

    @sent.setter
    def sent(self, value):
        self.__dict__["_sent"] = value

    def spectral_parameters(self):
        return [self.A, self.theta, self.gate]

    def logalpha(self, z):
        """la = -softplus(W_a z + b) exp(A_h) <= 0 per (b, t, h), floored per head when hl_floor
        (`src/assoc.py:355-359`)."""
        la = -F.softplus(_op_mod.linear(z, self.wa)) * torch.exp(self.A)
        return la.clamp(min=self.la_floor) if self.hl_floor else la

    def add_short_conv(self, K: int):
        """A depthwise causal convolution over the last K tokens on q, k and v (`src/assoc.py:361-372`): weight
        (3 d, K), initialised as the identity (all weight on the current token). The carried state becomes
        (S, position, cache) with the cache the last K - 1 inputs, (B, 3 d, K - 1)."""
        w = torch.zeros(3 * self.d, K, device=self.q.weight.device, dtype=self.q.weight.dtype)
        w[:, -1] = 1.0
        self.sconv = nn.Parameter(w)
        return self

    def _sconv(self, qo, ko, vo, cc):
        """The causal depthwise convolution on q, k, v (B, T, d each) continuing the cache cc ((B, 3 d, K - 1) or None
        at a sequence start) (`src/assoc.py:374-382`). Returns q, k, v and the new cache."""
        D, K = self.d, self.sconv.shape[1]
        x = torch.cat([qo, ko, vo], dim=-1).transpose(1, 2)
        pad = cc.to(x.dtype) if cc is not None else x.new_zeros(x.shape[0], 3 * D, K - 1)
        xp = torch.cat([pad, x], dim=-1)
        y = F.conv1d(xp, self.sconv.to(x.dtype).unsqueeze(1), groups=3 * D).transpose(1, 2)
        return y[..., :D].contiguous(), y[..., D:2 * D].contiguous(), y[..., 2 * D:].contiguous(), xp[..., -(K - 1):]

    def _projections(self, z, cc=None):
        """q, k, v projections (B, T, H, dk) (short convolution and key_topk applied), the write-gate logits (plain
        rule, else None), la (B, T, H), beta (B, T, H) or None, and the convolution's new cache."""
        B, T, _ = z.shape
        fused = FUSED_PROJ and self.delta and not self.key_topk
        if fused:
            W = torch.cat([self.q.weight, self.k.weight, self.v.weight, self.wa.weight, self.wb.weight])
            qo, ko, vo, ao, bo = F.linear(z, W).split([self.d, self.d, self.d, self.h, self.h], dim=-1)
            la = -F.softplus(ao + self.wa.bias) * torch.exp(self.A)
            if self.hl_floor:
                la = la.clamp(min=self.la_floor)
            bt = torch.sigmoid(bo + self.wb.bias)
            qo, ko, vo = qo.contiguous(), ko.contiguous(), vo.contiguous()
        else:
            qo, ko, vo = self.q(z), self.k(z), self.v(z)
            la = self.logalpha(z)
            bt = torch.sigmoid(_op_mod.linear(z, self.wb)) if self.delta else None
        if getattr(self, "sconv", None) is not None:
            qo, ko, vo, cc = self._sconv(qo, ko, vo, cc)
        kp = ko.view(B, T, self.h, self.dk)
        if self.key_topk:
            keep = torch.zeros_like(kp).scatter_(-1, kp.abs().topk(self.key_topk, dim=-1).indices, 1.0)
            kp = kp * keep
        gate = None if (self.delta or self.write_all) else _op_mod.linear(z, self.wi)
        if bt is not None:
            if getattr(self, "beta_scale", None) is not None:
                bt = bt * self.beta_scale.transpose(1, 2).to(bt.dtype)
            if self.write_all:
                bt = bt.clamp(min=0.75)
        return qo.view(B, T, self.h, self.dk), kp, vo.view(B, T, self.h, self.dk), gate, la, bt, cc

    def _torch_inputs(self, z, pos, cc=None):
        """The reference's torch path to the scan's inputs (`src/assoc.py:436-444`, used when the kernels are not):
        unit-normalise q, k, v per head, gate k (plain rule), rotate q and k at `pos`, all in the projections' dtype.
        Returns q, k, v (B, H, T, dk), la and beta (B, H, T) (beta None for the plain rule), the projections' dtype
        and the convolution's new cache."""
        qp, kp, vp, gate, la, bt, cc = self._projections(z, cc)
        q, k, v = (F.normalize(t.transpose(1, 2), dim=-1) for t in (qp, kp, vp))
        if gate is not None:
            k = k * torch.sigmoid(gate).transpose(1, 2).unsqueeze(-1)
        q, k = rotate(q, self.theta, pos), rotate(k, self.theta, pos)
        return q, k, v, la.transpose(1, 2), (None if bt is None else bt.transpose(1, 2)), qp.dtype, cc

    def _scan_inputs(self, z, pos, cc=None):
        """The bf16 kernels' inputs from the normalised layer input z (B, T, d): q, k, v (B, H, T, dk) bf16, la and
        beta (B, H, T) fp32 (beta None for the plain rule), the projections' dtype and the short convolution's new
        cache. With FUSED_PLUMBING (no key_topk, beta_scale or short convolution): one GEMM for the q, k, v, decay and
        write-gate (plain) or write-strength (delta) projections and one kernel from its output; otherwise the
        reference's composition: separate projections (one GEMM under FUSED_PROJ), convolution, elementwise decay,
        gate and strength, prep."""
        if (FUSED_PLUMBING and not self.key_topk and self.dk in (HEAD_DIM_KERNEL, HEAD_DIM_WIDE)
                and getattr(self, "beta_scale", None) is None and getattr(self, "sconv", None) is None):
            gated = not (self.delta or self.write_all)
            extra = [self.wi.weight] if gated else ([self.wb.weight] if self.delta else [])
            W = torch.cat([self.q.weight, self.k.weight, self.v.weight, self.wa.weight] + extra)
            P = _op_mod.linear_w(z, W)
            q, k, v, la, beta = _op.aspin_prep_proj(
                P, self.h, self.wa.bias, self.A, self.la_floor if self.hl_floor else None,
                self.wi.bias if gated else None, self.wb.bias if self.delta else None,
                0.75 if (self.delta and self.write_all) else 0.0, gated, self.theta, pos, self.dk)
            return q, k, v, la, (beta if self.delta else None), P.dtype, cc
        qp, kp, vp, gate, la, bt, cc = self._projections(z, cc)
        q, k, v = _op.aspin_prep(qp, kp, vp, gate, self.theta, pos)
        bt = None if bt is None else bt.transpose(1, 2).float()
        return q, k, v, la.transpose(1, 2).float(), bt, qp.dtype, cc

    def _norm_in(self, x):
        """`self.ln(x)` (`src/assoc.py:388`); with FUSED_PLUMBING one kernel each way that writes the result in the
        dtype the projections compute in."""
        return _op_mod.layer_norm(x, self.ln) if FUSED_PLUMBING else self.ln(x)

    def _epilogue(self, o, dtype):
        """`self.on(o.to(dtype)).transpose(1, 2).reshape(B, T, D)` (`src/assoc.py:500-505`) for the scan's bf16 output
        o (B, H, T, dk): one kernel each way (per-head RMSNorm in fp32, rounded once to `dtype`, written
        token-major)."""
        B, H, T, Dk = o.shape
        if (FUSED_PLUMBING and dtype in (torch.bfloat16, torch.float32) and self.on.weight is not None
                and Dk in (HEAD_DIM_KERNEL, HEAD_DIM_WIDE)):
            eps = self.on.eps if self.on.eps is not None else _op_mod.RMS_EPS
            return _op.aspin_out(o, self.on.weight, eps, dtype == torch.bfloat16)[0]
        return self.on(o.to(dtype)).transpose(1, 2).reshape(B, T, H * Dk)

    def forward(self, x, h0=None, pos0: int = 0):
        """x (B, T, d); h0 = (S (B, H, dk, dk), p0) from a previous call, (S, p0, cache) with the short convolution, or
        None. Returns (x + gated output, (S, T) or (S, T, cache)); positions restart at 0 every call and the carried
        state is rebased by -p0 (`src/assoc.py:384-512`)."""
        if self.delta and self.dk > _op_mod.EXACT_MAX_DK:
            raise PragnosiaError(f"AssocCarrier: the delta rule takes head dims up to {_op_mod.EXACT_MAX_DK} (got "
                                 f"{self.dk})")
        if not x.is_cuda:
            raise PragnosiaError("AssocCarrier runs on a ROCm GPU only; there is no CPU path")
        B, T, D = x.shape
        sc = getattr(self, "sconv", None) is not None
        cc = None
        if h0 is None:
            S0, p0 = None, pos0
        elif len(h0) == 3:
            S0, p0, cc = h0
        else:
            S0, p0 = h0
        z = self._norm_in(x)
        p_dev = p0.float().reshape(()) if torch.is_tensor(p0) else None
        p_host = 0.0 if torch.is_tensor(p0) else float(p0)
        shifted = S0 is not None and (p_dev is not None or p_host != 0.0)
        decode = T == 1 and not _needs_grad(x, S0, *self.parameters())
        kern = self.kernel and T > 1 and _kernel_ok(self.dk, self.dk, self.delta)
        sent = None
        if decode and self.dk == HEAD_DIM_KERNEL:
            # the fused fp32 step: rebase, normalise, gate, decay, write, read
            qp, kp, vp, gate, la, bt, cc = self._projections(z, cc)
            S_prev = S0 if S0 is not None else torch.zeros(B, self.h, self.dk, self.dk, device=x.device)
            S, o = _op.aspin_decode_step(S_prev, qp.reshape(B, self.h, self.dk), kp.reshape(B, self.h, self.dk),
                                         vp.reshape(B, self.h, self.dk),
                                         None if gate is None else gate.reshape(B, self.h),
                                         la.reshape(B, self.h), None if bt is None else bt.reshape(B, self.h),
                                         self.theta, p_dev, p_host)
            o = self.on(o.unsqueeze(2).to(qp.dtype)).transpose(1, 2).reshape(B, T, D)
        elif kern:
            wide = self.dk == HEAD_DIM_WIDE
            if shifted:
                S0 = _op.aspin_rebase(S0, self.theta, p_dev, p_host)
            pos = _positions(T, x.device, getattr(self, "pos_wrap", None))
            q, k, v, la, bt, dtype, cc = self._scan_inputs(z, pos, cc)
            fused = FUSED_SCAN and self.delta and not self.need_sent
            want = bool(self.need_sent or not (FUSED_SCAN and self.delta) or
                        _needs_grad(x, S0, *self.parameters()))
            if fused:
                # nothing kept for the backward but the scan's inputs: it recomputes X, W and the entering states
                o, S = _op.aspin_delta_fused(q, k, v, la, bt, S0)
                sent = None
            elif self.delta:
                o, S, sent, _, _ = _op.aspin_delta(q, k, v, la, bt, S0, want)
                sent = sent.transpose(-1, -2) if want else sent  # the op stores each state transposed
            elif wide:
                o, S, sent = _plain_scan_wide(q, k, v, la, S0, want)
            else:
                o, S, sent = _op.aspin_chunk(q, k, v, la, S0, want)
            sent = sent if want else None
            o = self._epilogue(o, dtype)
        else:
            # the reference's torch path (kernel=False, a T = 1 call under autograd, a decode step at a head dim
            # other than 64): normalise, gate and rotate in torch, then assoc_scan, fp32 (bf16 MFMA kernels under
            # autocast, as the reference's bf16 matmuls)
            if shifted:
                S0 = (_op.aspin_rebase(S0, self.theta, p_dev, p_host)
                      if self.dk in (HEAD_DIM_KERNEL, HEAD_DIM_WIDE) and S0.dtype == torch.float32
                      else _rebase_wide(S0, self.theta, p_dev, p_host))
            pos = _positions(T, x.device, getattr(self, "pos_wrap", None))
            q, k, v, la, bt, dtype, cc = self._torch_inputs(z, pos, cc)
            mm = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
            o, S = assoc_scan(q, k, v, la, S0, chunk=self.chunk, recompute=self.recompute, mm=mm, beta=bt)
            o = self.on(o).transpose(1, 2).reshape(B, T, D)
        self.sent = sent
        if _needs_grad(x, o, self.o.weight, self.gate):
            # gate on the weight, as the reference does for training (it keeps the backward's saved tensor small)
            Wg = self.o.weight * torch.sigmoid(self.gate)
            out = x + (_op_mod.linear_w(o, Wg) if FUSED_PLUMBING else F.linear(o, Wg))
        else:
            # the same function without materialising a gated d x d weight on every call (decode, inference)
            out = x + F.linear(o, self.o.weight) * torch.sigmoid(self.gate)
        # the state is now expressed in this call's positions 0..T-1: the next call rebases it by T
        p_out = p0 * 0 + T if torch.is_tensor(p0) else T
        return out, ((S, p_out, cc) if sc else (S, p_out))

    def forward_windows(self, x, window: int, h0=None, pos0: int = 0):
        """Consecutive windows of `window` tokens of x (B, T, d), the state carried from each window into the next:
        the same function as calling `forward` on x[:, s:s + window] for s = 0, window, ... in turn, handing each
        call the state the previous one returned (`src/model.py:842-864` drives the reference's carrier so). A
        carrier without autograd, with `window` a multiple of 64, runs every window in one pass: the projections over
        the whole sequence, then for the plain rule one segment-parallel scan that rebases the state at window
        boundaries, for the delta rule every window at once from its affine state map (`ops.aspin_delta_windows`);
        otherwise the windows run one call each. Returns (x + gated output, (S, length of the last window)); `sent`
        is not kept."""
        B, T, D = x.shape
        fused = (window % 64 == 0 and T > window and x.is_cuda and self.dk == HEAD_DIM_KERNEL
                 and self.kernel and getattr(self, "sconv", None) is None
                 and not _needs_grad(x, *(h0[:1] if h0 is not None else ()), *self.parameters()))
        if not fused:
            outs, st = [], h0
            for s in range(0, T, window):
                o, st = self.forward(x[:, s:s + window], st, pos0)
                outs.append(o)
            return torch.cat(outs, 1), st
        S0, p0 = (None, pos0) if h0 is None else h0[:2]
        z = self._norm_in(x)
        p_dev = p0.float().reshape(()) if torch.is_tensor(p0) else None
        p_host = 0.0 if torch.is_tensor(p0) else float(p0)
        if S0 is not None and (p_dev is not None or p_host != 0.0):
            S0 = _op.aspin_rebase(S0, self.theta, p_dev, p_host)
        pos = _positions(T, x.device, window)
        wrap = getattr(self, "pos_wrap", None)
        if wrap:
            pos = pos % wrap
        q, k, v, la, bt, dtype, _ = self._scan_inputs(z, pos)
        if self.delta:
            o, S = _op.aspin_delta_windows(q, k, v, la, bt, S0, self.theta, window)
        else:
            o, S, _ = _op.aspin_chunk_windows(q, k, v, la, S0, self.theta, window, False)
        self.sent = None
        o = self._epilogue(o, dtype)
        out = x + F.linear(o, self.o.weight) * torch.sigmoid(self.gate)
        last = T - window * ((T - 1) // window)
        return out, (S, p0 * 0 + last if torch.is_tensor(p0) else last)


@contextmanager
def fused_scan(model):
    """Within the block, carriers skip the per-chunk entering states no later layer reads (`src/assoc.py:518-532`);
    restores the previous setting on exit."""
    global FUSED_SCAN
    prev = FUSED_SCAN
    saved = [(m, m.need_sent) for m in model.modules() if isinstance(m, AssocCarrier)]
    FUSED_SCAN = True
    for m, _ in saved:
        m.need_sent = False
    try:
        yield
    finally:
        FUSED_SCAN = prev
        for m, v in saved:
            m.need_sent = v
