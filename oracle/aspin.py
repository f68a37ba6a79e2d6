"""CPU restatement of the reference's associative-carrier (aspin) scan. TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Conventions, as in the reference (`src/assoc.py:11-24`): per (batch, head) the memory S is (dk, dv) with KEYS on
rows; the plain rule is S_t = a_t S_{t-1} + k_t v_t^T and the read is o_t = S_t^T q_t, with a_t = exp(la_t),
la_t <= 0. Tensors are (B, H, T, D); la and beta are (B, H, T); S is (B, H, D, D).

What pins each function (tests/test_oracle_aspin.py):
  recurrence          -- brute force; the delta known-answer test (`tests/test_assoc.py:118-130`); the delta
                         rule's rotation equivariance.
  scan_twopass        -- == recurrence for chunks 1, 8, T (chunk 1 reduces every matrix to a scalar), with and
                         without S0, across carried windows; autograd gradients == those of the recurrence.
  unit_lower_inverse  -- X (I + N) == I against torch.linalg.solve_triangular.
  scan_twopass_delta  -- == the delta recurrence; chunk 16 == chunk 256; bounded under 256 correlated writes.
  prep                -- unit norm per row; rotation is orthogonal; q.k depends on t - s only.
  rebase              -- carrying a state across a position restart == global positions (rotation equivariance).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def rotate(x, theta, pos):
    """Rotate interleaved channel pairs (x[2i], x[2i+1]) by angle pos * theta[h, i].

    Follows `src/assoc.py:34-39`: x (B, H, T, D); theta (H, D/2); pos (T,). The angle is formed in theta's
    dtype (fp32 in the module), then cos/sin; the pair is (x1 c - x2 s, x1 s + x2 c)."""
    ang = pos.reshape(1, 1, -1, 1).to(theta.dtype) * theta.reshape(1, theta.shape[0], 1, theta.shape[1])
    c, s = torch.cos(ang), torch.sin(ang)
    even, odd = x[..., 0::2], x[..., 1::2]
    return torch.stack((even * c - odd * s, even * s + odd * c), dim=-1).flatten(-2)


def recurrence(q, k, v, la, S0=None, beta=None):
    """The literal per-token recurrence, in the dtype of q (use fp64 as the truth).

    Plain rule (`tests/test_assoc.py:22-27`): S_t = a_t S_{t-1} + k_t v_t^T, o_t = S_t^T q_t.
    Delta rule: the decay applies inside the read, S_t = a_t S_{t-1} + b_t k_t (v_t - (a_t S_{t-1})^T k_t)^T.
    That form is what the chunk equations give at chunk size 1 (`src/assoc.py:93-97`, `:238-241`); the docstring
    at `src/assoc.py:210` omits a_t inside the read and is not followed. Returns (o, S_final)."""
    B, H, T, D = q.shape
    S = torch.zeros(B, H, D, v.shape[-1], dtype=q.dtype) if S0 is None else S0.to(q.dtype).clone()
    outs = []
    for t in range(T):
        a = torch.exp(la[:, :, t]).to(q.dtype)[..., None, None]
        kt, vt = k[:, :, t], v[:, :, t]
        S = a * S
        if beta is None:
            S = S + kt.unsqueeze(-1) * vt.unsqueeze(-2)
        else:
            read = torch.einsum("bhd,bhdj->bhj", kt, S)
            S = S + beta[:, :, t].to(q.dtype)[..., None, None] * kt.unsqueeze(-1) * (vt - read).unsqueeze(-2)
        outs.append(torch.einsum("bhd,bhdj->bhj", q[:, :, t], S))
    o = torch.stack(outs, 2) if outs else q.new_zeros(B, H, 0, v.shape[-1])
    return o, S


def _chunk_views(x, la, C, extra=()):
    """Pad T up to a multiple of C with zero tokens (la = 0: no decay; beta = 0: no write), as
    `src/assoc.py:131-135` and `:219-221` do, and view as chunks."""
    B, H, T, D = x[0].shape
    pad = (-T) % C
    if pad:
        x = [F.pad(t, (0, 0, 0, pad)) for t in x]
        la = F.pad(la, (0, pad))
        extra = [F.pad(e, (0, pad)) for e in extra]
    NC = (T + pad) // C
    xs = [t.reshape(B, H, NC, C, t.shape[-1]) for t in x]
    return xs, la.reshape(B, H, NC, C), [e.reshape(B, H, NC, C) for e in extra], NC


def _decays(lc):
    """Within-chunk decay statistics from the chunked log-decays lc (B, H, NC, C): every exponent is <= 0.
    dec[t, s] = exp(L_t - L_s) for s <= t (0 above the diagonal); eL = exp(L); w = exp(L_C - L); a = exp(L_C)."""
    C = lc.shape[-1]
    L = lc.cumsum(-1)
    diff = (L.unsqueeze(-1) - L.unsqueeze(-2)).clamp(max=0.0)
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool))
    dec = torch.where(causal, torch.exp(diff), torch.zeros((), dtype=L.dtype))
    eL = torch.exp(L).unsqueeze(-1)
    w = torch.exp((L[..., -1:] - L).clamp(max=0.0)).unsqueeze(-1)
    a = torch.exp(L[..., -1])
    return dec, eL, w, a


def _mm(x, y, mm):
    """Matrix product in the reference's matmul dtype: exact when mm is None, else operands rounded to mm with the
    product returned in x's dtype (the bf16-autocast rounding points of `src/assoc.py:149-153`)."""
    if mm is None:
        return x @ y
    return (x.to(mm) @ y.to(mm)).to(x.dtype)


def scan_twopass(q, k, v, la, S, chunk, mm=None):
    """Plain rule, chunked: `src/assoc.py:118-165`.

    Pass 0 (all chunks): A = (Q K^T) o dec, intra = A V, KV_c = (K o w)^T V, a_c = exp(L_C).
    Pass 1 (the only sequential step): S_ent[c] = S; S <- a_c S + KV_c.
    Pass 2: O = intra + (Q o eL) S_ent. Returns (o, S_final, S_ent)."""
    B, H, T, D = q.shape
    C = min(chunk, T)
    (qc, kc, vc), lc, _, NC = _chunk_views([q, k, v], la, C)
    dec, eL, w, a = _decays(lc)
    A = _mm(qc, kc.transpose(-1, -2), mm) * dec
    intra = _mm(A, vc, mm)
    KV = _mm((kc * w).transpose(-1, -2), vc, mm)
    ent = []
    for c in range(NC):
        ent.append(S)
        S = a[:, :, c, None, None] * S + KV[:, :, c]
    Sent = torch.stack(ent, 2)
    o = intra + _mm(qc * eL, Sent, mm)
    return o.reshape(B, H, NC * C, v.shape[-1])[:, :, :T], S, Sent


def unit_lower_inverse(N, b=16):
    """X = (I + N)^-1 for strictly-lower N (..., C, C): `src/assoc.py:168-204`.

    b x b diagonal blocks are inverted by summing the (finite, nilpotent) Neumann series by doubling, then block
    forward substitution across block rows; every intermediate stays bounded. b = C when C is not a multiple of b."""
    C = N.shape[-1]
    if C % b:
        b = C
    nb = C // b
    eye_b = torch.eye(b, dtype=N.dtype)
    inv_diag = []
    for i in range(nb):
        R = -N[..., i * b:(i + 1) * b, i * b:(i + 1) * b]
        X = eye_b.expand_as(R).clone()
        m = 1
        while m < b:
            X = X + R @ X
            R = R @ R
            m *= 2
        inv_diag.append(X)
    eye = torch.eye(C, dtype=N.dtype).expand(*N.shape[:-2], C, C)
    rows = []
    for i in range(nb):
        rhs = eye[..., i * b:(i + 1) * b, :]
        if i:
            rhs = rhs - N[..., i * b:(i + 1) * b, :i * b] @ torch.cat(rows, -2)
        rows.append(inv_diag[i] @ rhs)
    return torch.cat(rows, -2)


def delta_inverse(kc, bc, dec):
    """X_c = (I + diag(beta) strictly_lower((K K^T) o dec))^-1 per chunk (`src/assoc.py:231-232`)."""
    KK = (kc @ kc.transpose(-1, -2)) * dec
    return unit_lower_inverse(bc.unsqueeze(-1) * torch.tril(KK, -1))


def scan_twopass_delta(q, k, v, la, be, S, chunk, mm=None):
    """Delta rule, chunked: `src/assoc.py:207-251`.

    X for every chunk first (it does not depend on the state); then per chunk rhs = beta (V - eL o (K S)),
    W = X rhs, S <- a S + (K o w)^T W; finally O = ((Q K^T) o dec) W + (Q o eL) S_ent. Padded tokens get beta = 0.
    Returns (o, S_final, S_ent, W)."""
    B, H, T, D = q.shape
    C = min(chunk, T)
    (qc, kc, vc), lc, (bc,), NC = _chunk_views([q, k, v], la, C, extra=(be,))
    dec, eL, w, a = _decays(lc)
    X = delta_inverse(kc, bc, dec)
    kw = (kc * w).transpose(-1, -2)
    ent, Ws = [], []
    for c in range(NC):
        ent.append(S)
        rhs = bc[:, :, c].unsqueeze(-1) * (vc[:, :, c] - eL[:, :, c] * (kc[:, :, c] @ S))
        Wc = X[:, :, c] @ rhs
        Ws.append(Wc)
        S = a[:, :, c, None, None] * S + kw[:, :, c] @ Wc
    Sent, W = torch.stack(ent, 2), torch.stack(Ws, 2)
    A = _mm(qc, kc.transpose(-1, -2), mm) * dec
    o = _mm(A, W, mm) + _mm(qc * eL, Sent, mm)
    return o.reshape(B, H, NC * C, v.shape[-1])[:, :, :T], S, Sent, W.reshape(B, H, NC * C, -1)[:, :, :T]


def assoc_scan(q, k, v, logalpha, S0=None, chunk=64, beta=None, mm=None):
    """The dispatcher of `src/assoc.py:254-269`: fp64 stays fp64, anything else runs in fp32; S0 None = zeros.
    Returns (o in the compute dtype, S_final)."""
    B, H, T, D = q.shape
    rt = torch.float64 if q.dtype == torch.float64 else torch.float32
    q, k, v, la = q.to(rt), k.to(rt), v.to(rt), logalpha.to(rt)
    S = torch.zeros(B, H, D, v.shape[-1], dtype=rt) if S0 is None else S0.to(rt)
    if beta is None:
        o, S, _ = scan_twopass(q, k, v, la, S, chunk, mm)
    else:
        o, S, _, _ = scan_twopass_delta(q, k, v, la, beta.to(rt), S, chunk, mm)
    return o, S


def normalize_rows(x, eps=1e-12):
    """F.normalize semantics (`src/assoc.py:457`): x / max(|x|, eps) over the last dimension."""
    return x / x.norm(dim=-1, keepdim=True).clamp_min(eps)


def prep(qp, kp, vp, gate_logits, theta, pos):
    """The plumbing between the projections and the scan (`src/assoc.py:453-460`, kernel form
    `src/assoc_kernel.py:740-769`, torch form used by the reference test `tests/test_assoc.py:189-193`):
    unit-normalise q, k, v per head; scale k by sigmoid(gate) when a gate is given (plain rule); rotate q and k
    by pos * theta. Inputs (B, T, H, D) and gate (B, T, H); outputs (B, H, T, D) in fp32 (fp64 if the input is)."""
    rt = torch.float64 if qp.dtype == torch.float64 else torch.float32
    q, k, v = [normalize_rows(t.transpose(1, 2).to(rt)) for t in (qp, kp, vp)]
    if gate_logits is not None:
        k = k * torch.sigmoid(gate_logits.to(rt)).transpose(1, 2).unsqueeze(-1)
    th = theta.to(rt)
    return rotate(q, th, pos), rotate(k, th, pos), v


def rebase(S, theta, p0):
    """Rotate the KEY rows of a carried state by -p0 * theta (`src/assoc.py:399-402`): the state written at
    positions ..p0-1 becomes the state a window whose positions restart at 0 reads correctly. S (B, H, Dk, Dv)."""
    Dv = S.shape[-1]
    sh = torch.full((Dv,), -float(p0), dtype=theta.dtype)
    return rotate(S.transpose(-1, -2), theta, sh).transpose(-1, -2).contiguous()


def logalpha(wa_out, A, floor=None):
    """la = -softplus(W_a z + b) * exp(A_h) <= 0, optionally floored (`src/assoc.py:355-359`)."""
    la = -F.softplus(wa_out) * torch.exp(A)
    if floor is not None:
        la = la.clamp(min=floor)
    return la
