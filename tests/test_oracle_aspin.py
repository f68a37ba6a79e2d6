"""Pins the CPU oracle for the aspin scan (oracle/aspin.py) against the definition, known answers and invariants.

Mirrors the reference's own checks (`tests/test_assoc.py:17-46`, `:113-139`) and adds brute-force closed forms and
library routines, chosen so a dropped decay term, a wrong sign, an off-by-one in the cumulative sum or a transposed
state fails at least one of them."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as O



@pytest.fixture(autouse=True)
def _fp64_default():
    """The oracle is pinned in fp64; the default dtype is restored after each test so other modules are unaffected."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(B=2, H=3, T=45, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, D, generator=g)
    k = torch.randn(B, H, T, D, generator=g)
    v = torch.randn(B, H, T, D, generator=g)
    la = -torch.rand(B, H, T, generator=g) * 3.0
    S0 = torch.randn(B, H, D, D, generator=g)
    return q, k, v, la, S0


def _brute(q, k, v, la, S0):
    """o_t = sum_{s<=t} exp(sum_{s<r<=t} la_r) (q_t . k_s) v_s + exp(sum_{r<=t} la_r) S0^T q_t, term by term."""
    B, H, T, D = q.shape
    o = torch.zeros(B, H, T, v.shape[-1])
    for b in range(B):
        for h in range(H):
            for t in range(T):
                acc = math.exp(float(la[b, h, :t + 1].sum())) * (S0[b, h].T @ q[b, h, t])
                for s in range(t + 1):
                    acc = acc + math.exp(float(la[b, h, s + 1:t + 1].sum())) * float(q[b, h, t] @ k[b, h, s]) * v[b, h, s]
                o[b, h, t] = acc
    return o


def test_recurrence_matches_brute_force():
    q, k, v, la, S0 = _inputs(B=1, H=2, T=7, D=3)
    o, _ = O.recurrence(q, k, v, la, S0)
    assert torch.allclose(o, _brute(q, k, v, la, S0), atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 8, 45, 64])
def test_twopass_matches_recurrence(chunk):
    q, k, v, la, S0 = _inputs()
    yr, Sr = O.recurrence(q, k, v, la, S0)
    yc, Sc = O.assoc_scan(q, k, v, la, S0, chunk=chunk)
    assert torch.allclose(yc, yr, atol=1e-11)
    assert torch.allclose(Sc, Sr, atol=1e-11)
    y0, _ = O.assoc_scan(q, k, v, la, None, chunk=chunk)
    yr0, _ = O.recurrence(q, k, v, la, torch.zeros_like(S0))
    assert torch.allclose(y0, yr0, atol=1e-11)


def test_twopass_entering_states_are_the_recurrence_states():
    q, k, v, la, S0 = _inputs(T=40)
    _, _, Sent = O.scan_twopass(q, k, v, la, S0, 8, None)
    for c in range(5):
        _, S_c = O.recurrence(q[:, :, :8 * c], k[:, :, :8 * c], v[:, :, :8 * c], la[:, :, :8 * c], S0)
        assert torch.allclose(Sent[:, :, c], S_c, atol=1e-11)


def test_two_windows_carried_equal_one():
    q, k, v, la, S0 = _inputs()
    yr, _ = O.recurrence(q, k, v, la, S0)
    a, st = O.assoc_scan(q[:, :, :20], k[:, :, :20], v[:, :, :20], la[:, :, :20], S0, chunk=8)
    b, _ = O.assoc_scan(q[:, :, 20:], k[:, :, 20:], v[:, :, 20:], la[:, :, 20:], st, chunk=8)
    assert torch.allclose(torch.cat([a, b], 2), yr, atol=1e-11)


def test_twopass_gradients_match_recurrence():
    q, k, v, la, S0 = _inputs(T=30)
    w = torch.randn_like(q)
    wS = torch.randn_like(S0)
    grads = []
    for fn in (lambda *a: O.assoc_scan(*a, chunk=8), O.recurrence):
        args = [t.clone().requires_grad_(True) for t in (q, k, v, la, S0)]
        y, S = fn(*args)
        ((y * w).sum() + (S * wS).sum()).backward()
        grads.append([a.grad for a in args])
    for x, y in zip(*grads):
        assert (x - y).abs().max() / y.abs().max() < 1e-9


def test_fp32_extreme_decay_is_finite():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 512, 64, generator=g, dtype=torch.float32)
    y, S = O.assoc_scan(q, torch.randn_like(q), torch.randn_like(q),
                        -torch.rand(2, 4, 512, generator=g, dtype=torch.float32) * 40, chunk=64)
    assert torch.isfinite(y).all() and torch.isfinite(S).all()


def test_bf16_matmul_rounding_stays_within_bf16_precision():
    """The mm=bf16 rounding points agree with the exact form to bf16 precision and not to less
    (`tests/test_assoc.py:86-97`)."""
    g = torch.Generator().manual_seed(7)
    q = F.normalize(torch.randn(2, 4, 256, 64, generator=g, dtype=torch.float32), dim=-1)
    k = F.normalize(torch.randn_like(q), dim=-1)
    v = F.normalize(torch.randn_like(q), dim=-1)
    la = -F.softplus(torch.randn(2, 4, 256, generator=g, dtype=torch.float32)) * 0.01
    o32, S32 = O.assoc_scan(q, k, v, la, None, chunk=64)
    o16, S16 = O.assoc_scan(q, k, v, la, None, chunk=64, mm=torch.bfloat16)
    ro = ((o16 - o32).abs().max() / o32.abs().max()).item()
    assert 1e-5 < ro < 0.03


# ------------------------------------------------------------------------------------------------ delta rule
def _kat():
    g = torch.Generator().manual_seed(0)
    kk = F.normalize(torch.randn(1, 1, 1, 4, generator=g), dim=-1)
    va = torch.tensor([[[[1.0, 0, 0, 0]]]])
    vb = torch.tensor([[[[0.0, 1.0, 0, 0]]]])
    K = torch.cat([kk, kk, kk], 2)
    V = torch.cat([va, vb, va], 2)
    return K, V, torch.zeros(1, 1, 3), torch.ones(1, 1, 3), va, vb


@pytest.mark.parametrize("chunk", [1, 2, 3])
def test_delta_known_answer(chunk):
    """`tests/test_assoc.py:118-130`: a key written twice reads back the SECOND value under the delta rule, and the
    plain rule reads back the sum."""
    K, V, la, be, va, vb = _kat()
    r = O.assoc_scan(K, K, V, la, None, chunk=chunk, beta=be)[0][0, 0, 1]
    assert torch.allclose(r, vb[0, 0, 0], atol=1e-9)
    rp = O.assoc_scan(K, K, V, la, None, chunk=chunk)[0][0, 0, 1]
    assert torch.allclose(rp, (va + vb)[0, 0, 0], atol=1e-9)
    rr = O.recurrence(K, K, V, la, None, beta=be)[0][0, 0, 1]
    assert torch.allclose(rr, vb[0, 0, 0], atol=1e-9)


def test_delta_single_token_closed_form():
    """One token into a carried state: S' = a S + b k (v - a S^T k)^T, o = S'^T q, written out by hand."""
    q, k, v, la, S0 = _inputs(B=1, H=1, T=1, D=5)
    be = torch.tensor([[[0.6]]])
    a = math.exp(float(la))
    S = a * S0[0, 0]
    res = v[0, 0, 0] - S.T @ k[0, 0, 0]
    Sn = S + 0.6 * torch.outer(k[0, 0, 0], res)
    o, Sf = O.recurrence(q, k, v, la, S0, beta=be)
    assert torch.allclose(Sf[0, 0], Sn, atol=1e-12)
    assert torch.allclose(o[0, 0, 0], Sn.T @ q[0, 0, 0], atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 8, 16, 45])
def test_delta_twopass_matches_recurrence(chunk):
    q, k, v, la, S0 = _inputs()
    k = F.normalize(k, dim=-1)
    be = torch.sigmoid(torch.randn(*la.shape, generator=torch.Generator().manual_seed(9)))
    yr, Sr = O.recurrence(q, k, v, la, S0, beta=be)
    yc, Sc = O.assoc_scan(q, k, v, la, S0, chunk=chunk, beta=be)
    assert torch.allclose(yc, yr, atol=1e-10)
    assert torch.allclose(Sc, Sr, atol=1e-10)


def test_delta_gradients_match_recurrence():
    q, k, v, la, S0 = _inputs(T=20)
    k = F.normalize(k, dim=-1)
    be = torch.sigmoid(torch.randn(*la.shape, generator=torch.Generator().manual_seed(4)))
    w = torch.randn_like(q)
    grads = []
    for fn in (lambda q, k, v, la, b, S: O.assoc_scan(q, k, v, la, S, chunk=8, beta=b),
               lambda q, k, v, la, b, S: O.recurrence(q, k, v, la, S, beta=b)):
        args = [t.clone().requires_grad_(True) for t in (q, k, v, la, be, S0)]
        y, S = fn(*args)
        ((y * w).sum() + S.sum()).backward()
        grads.append([a.grad for a in args])
    for x, y in zip(*grads):
        assert (x - y).abs().max() / y.abs().max() < 1e-9


def test_delta_chunk_invariance_and_boundedness_fp32():
    """`tests/test_assoc.py:131-139`: 256 correlated writes at beta = 1 stay bounded; chunk 16 == chunk 256."""
    g = torch.Generator().manual_seed(1)
    K = F.normalize(torch.randn(2, 4, 256, 64, generator=g, dtype=torch.float32), dim=-1)
    V = F.normalize(torch.randn(2, 4, 256, 64, generator=g, dtype=torch.float32), dim=-1)
    la = torch.zeros(2, 4, 256, dtype=torch.float32)
    be = torch.ones(2, 4, 256, dtype=torch.float32)
    y16, S16 = O.assoc_scan(K, K, V, la, None, chunk=16, beta=be)
    y256, _ = O.assoc_scan(K, K, V, la, None, chunk=256, beta=be)
    assert S16.abs().max() < 2.0
    assert (y16 - y256).abs().max() < 1e-5


@pytest.mark.parametrize("C", [16, 45, 64])
def test_unit_lower_inverse_against_triangular_solve(C):
    g = torch.Generator().manual_seed(C)
    N = torch.tril(torch.randn(3, C, C, generator=g) * 0.3, -1)
    X = O.unit_lower_inverse(N)
    I = torch.eye(C).expand(3, C, C)
    ref = torch.linalg.solve_triangular(I + N, I, upper=False, unitriangular=True)
    assert torch.allclose(X, ref, atol=1e-10)
    assert torch.allclose(X @ (I + N), I, atol=1e-10)


def test_unit_lower_inverse_repeated_keys_fp32():
    """Near-identical keys at beta ~ 1 (the repeated-token case of `src/assoc_kernel.py:577-582`): the true inverse
    has entries of magnitude <= 1 and the fp32 blocked form must keep them."""
    k = F.normalize(torch.ones(1, 1, 1, 64, 64, dtype=torch.float32) +
                    1e-3 * torch.randn(1, 1, 1, 64, 64, generator=torch.Generator().manual_seed(2), dtype=torch.float32), dim=-1)
    be = torch.full((1, 1, 1, 64), 0.99999, dtype=torch.float32)
    dec = torch.tril(torch.ones(64, 64, dtype=torch.float32))
    X = O.delta_inverse(k, be, dec)
    X64 = O.delta_inverse(k.double(), be.double(), dec.double())
    assert X.abs().max() < 1.5
    assert (X.double() - X64).abs().max() < 1e-3


# ------------------------------------------------------------------------------------------------ rotation, prep
def test_rotation_is_relative_position_code():
    """`tests/test_assoc.py:68-72`: q_t . k_s depends on t - s only."""
    g = torch.Generator().manual_seed(0)
    th = torch.rand(1, 4, generator=g) * 0.3
    qq, kk = torch.randn(1, 1, 1, 8, generator=g), torch.randn(1, 1, 1, 8, generator=g)
    s1 = (O.rotate(qq, th, torch.tensor([10])) * O.rotate(kk, th, torch.tensor([3]))).sum()
    s2 = (O.rotate(qq, th, torch.tensor([107])) * O.rotate(kk, th, torch.tensor([100]))).sum()
    assert abs(s1.item() - s2.item()) < 1e-12
    s3 = (O.rotate(qq, th, torch.tensor([11])) * O.rotate(kk, th, torch.tensor([3]))).sum()
    assert abs(s1.item() - s3.item()) > 1e-6


def test_rotation_is_orthogonal_and_pairs_are_interleaved():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 5, 8, generator=g)
    th = torch.rand(3, 4, generator=g)
    pos = torch.arange(5) * 7
    r = O.rotate(x, th, pos)
    assert torch.allclose(r.norm(dim=-1), x.norm(dim=-1), atol=1e-12)
    assert torch.allclose(O.rotate(r, th, -pos), x, atol=1e-12)
    # a unit vector on channel 0 rotates into channels 0 and 1 only: (cos, sin) of pos * theta[h, 0]
    e0 = torch.zeros(1, 3, 5, 8)
    e0[..., 0] = 1.0
    re0 = O.rotate(e0, th, pos)
    ang = pos[None, :] * th[:, :1]
    assert torch.allclose(re0[0, :, :, 0], torch.cos(ang), atol=1e-12)
    assert torch.allclose(re0[0, :, :, 1], torch.sin(ang), atol=1e-12)
    assert re0[..., 2:].abs().max() == 0


def test_prep_norms_and_gate():
    g = torch.Generator().manual_seed(2)
    B, T, H, D = 2, 9, 3, 8
    qp, kp, vp = (torch.randn(B, T, H, D, generator=g) * 3 for _ in range(3))
    gl = torch.randn(B, T, H, generator=g)
    th = torch.rand(H, D // 2, generator=g)
    pos = torch.arange(T) + 100
    q, k, v = O.prep(qp, kp, vp, gl, th, pos)
    assert q.shape == (B, H, T, D)
    assert torch.allclose(q.norm(dim=-1), torch.ones(B, H, T), atol=1e-12)
    assert torch.allclose(v.norm(dim=-1), torch.ones(B, H, T), atol=1e-12)
    assert torch.allclose(k.norm(dim=-1), torch.sigmoid(gl).transpose(1, 2), atol=1e-12)
    # v is not rotated: its direction is the projection's
    assert torch.allclose(v * vp.transpose(1, 2).norm(dim=-1, keepdim=True), vp.transpose(1, 2), atol=1e-12)
    # rotation by angle 0 at pos 0 leaves the normalised q unchanged
    q0, _, _ = O.prep(qp, kp, vp, None, th, torch.zeros(T, dtype=torch.long))
    assert torch.allclose(q0, qp.transpose(1, 2) / qp.transpose(1, 2).norm(dim=-1, keepdim=True), atol=1e-12)


@pytest.mark.parametrize("delta", [False, True])
def test_rebase_carry_equals_global_positions(delta):
    """A window read with positions restarting at 0 and the carried state rebased by -T1 theta gives exactly the
    outputs of one pass at global positions (`src/assoc.py:394-405`): rotation equivariance of both rules."""
    g = torch.Generator().manual_seed(5)
    B, T, H, D, T1 = 1, 30, 2, 8, 17
    qp, kp, vp = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    th = torch.rand(H, D // 2, generator=g) * 0.5
    la = -torch.rand(B, H, T, generator=g)
    be = torch.sigmoid(torch.randn(B, H, T, generator=g)) if delta else None
    q, k, v = O.prep(qp, kp, vp, None, th, torch.arange(T))
    y_full, S_full = O.assoc_scan(q, k, v, la, None, chunk=8, beta=be)
    q1, k1, v1 = O.prep(qp[:, :T1], kp[:, :T1], vp[:, :T1], None, th, torch.arange(T1))
    y1, S1 = O.assoc_scan(q1, k1, v1, la[..., :T1], None, chunk=8, beta=None if be is None else be[..., :T1])
    q2, k2, v2 = O.prep(qp[:, T1:], kp[:, T1:], vp[:, T1:], None, th, torch.arange(T - T1))
    S1r = O.rebase(S1, th, T1)
    y2, S2 = O.assoc_scan(q2, k2, v2, la[..., T1:], S1r, chunk=8, beta=None if be is None else be[..., T1:])
    assert torch.allclose(torch.cat([y1, y2], 2), y_full, atol=1e-10)
    # the final states differ by the rotation of the key rows by the second window's start
    assert torch.allclose(O.rebase(S_full, th, T1), S2, atol=1e-10)


def test_logalpha_is_nonpositive_and_floored():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 7, 3, generator=g) * 5
    A = torch.tensor([0.0, -2.0, -9.0])
    la = O.logalpha(x, A)
    assert (la <= 0).all()
    assert torch.allclose(la, -torch.log1p(torch.exp(x)) * torch.exp(A), atol=1e-12)
    fl = torch.tensor([-0.1, -0.01, -0.001])
    assert (O.logalpha(x, A, fl) >= fl).all()
