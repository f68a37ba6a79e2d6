"""GPU parity of the aspin chunked scan, DELTA rule (HIP kernels through the C ABI) against the CPU oracle.

Tolerances (bf16-input paths, from the north star): max relative error max|x - ref| / max|ref| <= 2e-2 on outputs and
on the final carried state, <= 5e-2 on every gradient (q, k, v, la, beta, S0). The oracle runs the exact two-pass
delta form (`oracle.aspin.scan_twopass_delta`, pinned in tests/test_oracle_aspin.py) in fp64, with autograd for the
gradients."""
import pytest
import torch
import torch.nn.functional as F

from oracle import aspin as O

pytestmark = pytest.mark.gpu
TOL_OUT, TOL_GRAD = 2e-2, 5e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


@pytest.fixture(scope="module")
def delta():
    from pragnosia_amd import ops  # noqa: F401
    return torch.ops.pragnosia.aspin_delta


def _inputs(B, H, T, D, seed, s0=True, rot=True):
    """configs[2]-style inputs: q, v ~ N(0,1), k L2-normalised, la = logsigmoid(N(3,1)), beta = sigmoid(N(0,1)),
    q and k rotated by pos * theta with theta ~ U(0, 0.1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, D, generator=g)
    k = F.normalize(torch.randn(B, H, T, D, generator=g), dim=-1)
    v = torch.randn(B, H, T, D, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    be = torch.sigmoid(torch.randn(B, H, T, generator=g))
    if rot:
        th = torch.rand(H, D // 2, generator=g) * 0.1
        q, k = O.rotate(q, th, torch.arange(T)), O.rotate(k, th, torch.arange(T))
    S0 = torch.randn(B, H, D, D, generator=g) * 0.3 if s0 else None
    q, k, v = q.bfloat16().float(), k.bfloat16().float(), v.bfloat16().float()
    return q, k, v, la, be, S0


def _check(delta, q, k, v, la, be, S0, seed=0):
    g = torch.Generator().manual_seed(seed + 1)
    wo = torch.randn(q.shape, generator=g)
    wS = torch.randn(q.shape[0], q.shape[1], q.shape[3], q.shape[3], generator=g)
    ins = [q, k, v, la, be] + ([S0] if S0 is not None else [])
    r = [t.detach().double().clone().requires_grad_(True) for t in ins]
    yr, Sr, _, _ = O.scan_twopass_delta(*r[:5], r[5] if S0 is not None else torch.zeros(
        q.shape[0], q.shape[1], q.shape[3], q.shape[3], dtype=torch.float64), 64)
    ((yr * wo.double()).sum() + (Sr * wS.double()).sum()).backward()
    kk = [t.detach().cuda().requires_grad_(True) for t in ins]
    yk, Sk, _, _, _ = delta(*kk[:5], kk[5] if S0 is not None else None, True)
    ((yk.float() * wo.cuda()).sum() + (Sk * wS.cuda()).sum()).backward()
    errs = {"o": rel(yk, yr), "S": rel(Sk, Sr)}
    for n, a, b in zip(("q", "k", "v", "la", "beta", "S0"), kk, r):
        errs["d" + n] = rel(a.grad, b.grad)
    return errs


def _assert(e):
    assert e["o"] < TOL_OUT and e["S"] < TOL_OUT, e
    assert max(v_ for n, v_ in e.items() if n.startswith("d")) < TOL_GRAD, e


@pytest.mark.parametrize("T,s0", [(64, False), (333, True), (1, True), (130, True), (512, False), (65, True)])
def test_delta_matches_oracle(delta, T, s0):
    q, k, v, la, be, S0 = _inputs(2, 3, T, 64, seed=T, s0=s0)
    _assert(_check(delta, q, k, v, la, be, S0, seed=T))


def test_delta_intermediates(delta):
    """X (the per-chunk inverse, computed in fp32 and stored bf16) and W (the residuals written) against the
    oracle's, and X (I + N) = I checked on the kernel's own X."""
    q, k, v, la, be, S0 = _inputs(1, 2, 200, 64, seed=4)
    with torch.no_grad():
        _, _, Sent, Wr = O.scan_twopass_delta(*(t.double() for t in (q, k, v, la, be, S0)), 64)
        o, S, sent, W, X = delta(*(t.cuda() for t in (q, k, v, la, be, S0)), True)
    (qc, kc, vc), lc, (bc,), NC = O._chunk_views([q.double(), k.double(), v.double()], la.double(), 64,
                                                  extra=(be.double(),))
    dec, _, _, _ = O._decays(lc)
    Xr = O.delta_inverse(kc, bc, dec)
    assert rel(X.float(), Xr) < 1e-2
    assert rel(W.float(), Wr) < TOL_OUT
    assert rel(sent.transpose(-1, -2).float(), Sent) < TOL_OUT  # stored transposed per chunk
    N = bc.unsqueeze(-1) * torch.tril((kc @ kc.transpose(-1, -2)) * dec, -1)
    eye = torch.eye(64, dtype=torch.float64)
    assert ((X.double().cpu() @ (eye + N)) - eye).abs().max() < 2e-2


def test_delta_known_answer(delta):
    """`tests/test_assoc.py:118-130` of the reference: the same key written with value e0 then e1 reads back e1
    under the delta rule (beta = 1, no decay), where the plain rule would read back e0 + e1."""
    B, H, T, D = 1, 1, 2, 64
    k = torch.zeros(B, H, T, D)
    k[..., 0] = 1.0
    v = torch.zeros(B, H, T, D)
    v[0, 0, 0, 0] = 1.0
    v[0, 0, 1, 1] = 1.0
    la = torch.zeros(B, H, T)
    be = torch.ones(B, H, T)
    with torch.no_grad():
        o, S, _, _, _ = delta(k.cuda(), k.cuda(), v.cuda(), la.cuda(), be.cuda(), None, False)
    assert torch.allclose(o[0, 0, 1].float().cpu(), v[0, 0, 1], atol=1e-3)
    assert torch.allclose(S[0, 0, 0].cpu(), v[0, 0, 1], atol=1e-3)


def test_cfg2_full_shape_delta(delta):
    """BASELINE configs[2], delta rule: B16 T512 H12 D64 bf16 q/k/v, fp32 state, beta = sigmoid(N(0,1));
    dO ~ N(0,1), dS_final ~ N(0,1). Oracle in fp32 (the full shape in fp64 is slow on the host)."""
    B, H, T, D = 16, 12, 512, 64
    q, k, v, la, be, _ = _inputs(B, H, T, D, seed=2, s0=False)
    g = torch.Generator().manual_seed(22)
    do = torch.randn(B, H, T, D, generator=g)
    dSf = torch.randn(B, H, D, D, generator=g)
    r = [t.clone().requires_grad_(True) for t in (q, k, v, la, be)]
    yr, Sr, _, _ = O.scan_twopass_delta(*r, torch.zeros(B, H, D, D), 64)
    ((yr * do).sum() + (Sr * dSf).sum()).backward()
    kk = [t.cuda().requires_grad_(True) for t in (q, k, v, la, be)]
    yk, Sk, _, _, _ = delta(*kk, None, True)
    ((yk.float() * do.cuda()).sum() + (Sk * dSf.cuda()).sum()).backward()
    assert rel(yk, yr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    for a, b in zip(kk, r):
        assert rel(a.grad, b.grad) < TOL_GRAD


def _fused(*a):
    """aspin_delta_fused (the FUSED_SCAN path: nothing kept but the inputs; at head dim 64 a forward that writes only o
    and S_final, X formed on chip) in aspin_delta's calling convention."""
    o, S = torch.ops.pragnosia.aspin_delta_fused(*a[:6])
    return o, S, None, None, None


def test_cfg2_full_shape_delta_fused():
    """The FUSED_SCAN path at BASELINE configs[2]'s full shape with an entering state: outputs, the final state and all
    six gradients (q, k, v, la, beta, S0) against the oracle in fp32 (as test_cfg2_full_shape_delta)."""
    from pragnosia_amd import ops  # noqa: F401
    B, H, T, D = 16, 12, 512, 64
    q, k, v, la, be, S0 = _inputs(B, H, T, D, seed=3, s0=True)
    g = torch.Generator().manual_seed(23)
    do = torch.randn(B, H, T, D, generator=g)
    dSf = torch.randn(B, H, D, D, generator=g)
    r = [t.clone().requires_grad_(True) for t in (q, k, v, la, be, S0)]
    yr, Sr, _, _ = O.scan_twopass_delta(*r, 64)
    ((yr * do).sum() + (Sr * dSf).sum()).backward()
    kk = [t.cuda().requires_grad_(True) for t in (q, k, v, la, be, S0)]
    yk, Sk, _, _, _ = _fused(*kk)
    ((yk.float() * do.cuda()).sum() + (Sk * dSf.cuda()).sum()).backward()
    assert rel(yk, yr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    for n, a, b in zip(("q", "k", "v", "la", "beta", "S0"), kk, r):
        assert rel(a.grad, b.grad) < TOL_GRAD, n


@pytest.mark.parametrize("D,T", [(64, 333), (64, 1), (128, 200), (128, 64)])
def test_delta_fused_matches_oracle(D, T):
    """The FUSED_SCAN path against the fp64 oracle, with an entering state and a final-state gradient, at head dims
    64 and 128, ragged and one-token sequences."""
    from pragnosia_amd import ops  # noqa: F401
    q, k, v, la, be, S0 = _inputs(2, 3, T, D, seed=500 + D + T, s0=True)
    print(f"delta fused: D {D} T {T}", flush=True)
    _assert(_check(_fused, q, k, v, la, be, S0, seed=500 + T))


def test_delta_repeated_keys_bounded(delta):
    """256 writes of nearly the same key at beta near 1 with no forgetting (the case that breaks a bf16 or tf32
    inverse, `src/assoc_kernel.py:577-582`): the state stays finite and bounded, and matches the fp64 oracle within
    5e-2. The looser bound is for this adversarial input only: the residuals cancel across 64 near-identical
    writes, which amplifies the bf16 rounding of the operands that the reference's kernel also rounds (X, W and the
    scores in bf16 dots, `src/assoc_kernel.py:354-359`); emulating those rounding points on the CPU in fp64 gives
    2.7e-2 on this input, and 1.3e-2 from the score rounding alone."""
    g = torch.Generator().manual_seed(9)
    B, H, T, D = 1, 2, 256, 64
    base = F.normalize(torch.randn(B, H, 1, D, generator=g), dim=-1)
    k = F.normalize(base + 0.01 * torch.randn(B, H, T, D, generator=g), dim=-1).bfloat16().float()
    v = torch.randn(B, H, T, D, generator=g).bfloat16().float()
    q = torch.randn(B, H, T, D, generator=g).bfloat16().float()
    la = torch.zeros(B, H, T)
    be = torch.full((B, H, T), 0.95)
    with torch.no_grad():
        yr, Sr, _, _ = O.scan_twopass_delta(*(t.double() for t in (q, k, v, la, be)),
                                            torch.zeros(B, H, D, D, dtype=torch.float64), 64)
        yk, Sk, _, _, _ = delta(*(t.cuda() for t in (q, k, v, la, be)), None, False)
    assert torch.isfinite(Sk).all() and Sk.abs().max() < 50
    assert rel(Sk, Sr) < 5e-2 and rel(yk, yr) < 5e-2


def test_delta_carried_windows_equal_one_pass(delta):
    q, k, v, la, be, S0 = _inputs(2, 2, 300, 64, seed=11)
    with torch.no_grad():
        dev = [t.cuda() for t in (q, k, v, la, be, S0)]
        y, S, *_ = delta(*dev, False)
        a, Sa, *_ = delta(*(t[:, :, :130] for t in dev[:5]), dev[5], False)
        b, Sb, *_ = delta(*(t[:, :, 130:] for t in dev[:5]), Sa, False)
    assert rel(torch.cat([a, b], 2), y) < TOL_OUT and rel(Sb, S) < TOL_OUT


@pytest.mark.parametrize("N,T", [(5, 192), (3, 130)])
def test_delta_window_maps_equal_state_passes(delta, N, T):
    """pragnosia_aspin_delta_window_maps (through the C ABI) writes, for N sequences, R (the final state from a zero
    entering state) then M (from the identity with zero values) in one launch: bit-identical to the forward's state
    pass run twice, once with no entering state and once with identity states and a zero value tensor (the same
    kernel and the same operations, the identity and the zero values formed on chip instead of read). Also M's meaning
    on a ragged length: M S0 + R is the final state from S0, to the scan's tolerance."""
    from pragnosia_amd._lib import lib, check
    q, k, v, la, be, S0 = _inputs(1, N, T, 64, seed=17)
    q, k, v = (t.cuda().bfloat16().contiguous() for t in (q, k, v))
    la, be, S0 = (t.cuda().float().contiguous() for t in (la, be, S0))
    RM = torch.full((2, N, 64, 64), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    check(lib().pragnosia_aspin_delta_window_maps(q.data_ptr(), k.data_ptr(), v.data_ptr(), la.data_ptr(),
                                                  be.data_ptr(), RM.data_ptr(), N, T, st),
          "pragnosia_aspin_delta_window_maps")
    with torch.no_grad():
        _, R, *_ = delta(q, k, v, la, be, None, False)
        eye = torch.eye(64, device="cuda").expand(1, N, 64, 64).contiguous()
        _, M, *_ = delta(q, k, torch.zeros_like(v), la, be, eye, False)
        _, S, *_ = delta(q, k, v, la, be, S0, False)
    torch.cuda.synchronize()
    assert torch.equal(RM[0], R[0]) and torch.equal(RM[1], M[0])
    assert rel(RM[1] @ S0[0] + RM[0], S[0]) < TOL_OUT


# ---- head dim 128 (the reference's hdspin / sdspin / tspin / aspin1 carriers, `src/model.py:651-660`): each head runs
# as two scans over its value halves sharing X; dq, dk, dla and dbeta are the sums of the two scans' parts.
@pytest.mark.parametrize("T,s0", [(64, False), (200, True), (1, True), (130, True)])
def test_delta_128_matches_oracle(delta, T, s0):
    q, k, v, la, be, S0 = _inputs(2, 2, T, 128, seed=300 + T, s0=s0)
    print(f"delta 128: T {T} s0 {s0}", flush=True)
    _assert(_check(delta, q, k, v, la, be, S0, seed=300 + T))


def test_delta_128_intermediates(delta):
    """At head dim 128: X (shared by the head's two value-half scans) against the oracle's inverse and X (I + N) = I;
    W and the entering states (stored transposed per chunk) against the oracle's."""
    q, k, v, la, be, S0 = _inputs(1, 2, 200, 128, seed=41)
    with torch.no_grad():
        _, _, Sent, Wr = O.scan_twopass_delta(*(t.double() for t in (q, k, v, la, be, S0)), 64)
        o, S, sent, W, X = delta(*(t.cuda() for t in (q, k, v, la, be, S0)), True)
    (qc, kc, vc), lc, (bc,), NC = O._chunk_views([q.double(), k.double(), v.double()], la.double(), 64,
                                                  extra=(be.double(),))
    dec, _, _, _ = O._decays(lc)
    Xr = O.delta_inverse(kc, bc, dec)
    assert X.shape == (1, 2, NC, 64, 64) and sent.shape == (1, 2, NC, 128, 128) and W.shape == (1, 2, 200, 128)
    assert rel(X.float(), Xr) < 1e-2
    assert rel(W.float(), Wr) < TOL_OUT
    assert rel(sent.transpose(-1, -2).float(), Sent) < TOL_OUT
    N = bc.unsqueeze(-1) * torch.tril((kc @ kc.transpose(-1, -2)) * dec, -1)
    eye = torch.eye(64, dtype=torch.float64)
    assert ((X.double().cpu() @ (eye + N)) - eye).abs().max() < 2e-2


def test_delta_128_known_answer(delta):
    """The reference's overwrite test (`tests/test_assoc.py:118-130`) at head dim 128, with the key in the second key
    half and the values in the second value half: the second write replaces the first."""
    B, H, T, D = 1, 1, 2, 128
    k = torch.zeros(B, H, T, D)
    k[..., 100] = 1.0
    v = torch.zeros(B, H, T, D)
    v[0, 0, 0, 70] = 1.0
    v[0, 0, 1, 71] = 1.0
    la = torch.zeros(B, H, T)
    be = torch.ones(B, H, T)
    with torch.no_grad():
        o, S, _, _, _ = delta(k.cuda(), k.cuda(), v.cuda(), la.cuda(), be.cuda(), None, False)
    assert torch.allclose(o[0, 0, 1].float().cpu(), v[0, 0, 1], atol=1e-3)
    assert torch.allclose(S[0, 0, 100].cpu(), v[0, 0, 1], atol=1e-3)
    assert S[0, 0].abs().sum().item() == pytest.approx(1.0, abs=1e-3)


def test_delta_128_long_sequence(delta):
    """B2 H3 T512 at head dim 128 with S0, forward and backward against the fp32 oracle (fp64 at this size is slow
    on the host)."""
    q, k, v, la, be, S0 = _inputs(2, 3, 512, 128, seed=51)
    g = torch.Generator().manual_seed(52)
    do = torch.randn(q.shape, generator=g)
    dSf = torch.randn(2, 3, 128, 128, generator=g)
    r = [t.clone().requires_grad_(True) for t in (q, k, v, la, be, S0)]
    yr, Sr, _, _ = O.scan_twopass_delta(*r, 64)
    ((yr * do).sum() + (Sr * dSf).sum()).backward()
    kk = [t.cuda().requires_grad_(True) for t in (q, k, v, la, be, S0)]
    yk, Sk, _, _, _ = delta(*kk, True)
    ((yk.float() * do.cuda()).sum() + (Sk * dSf.cuda()).sum()).backward()
    assert rel(yk, yr) < TOL_OUT and rel(Sk, Sr) < TOL_OUT
    for a, b in zip(kk, r):
        assert rel(a.grad, b.grad) < TOL_GRAD
