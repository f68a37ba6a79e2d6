"""GPU parity of the decode step's dense layers on the fp32 matrix cores (pragnosia_decode_gemm, the batches past the
one-wave GEMV) against fp64 torch: LayerNorm + Linear (+ bias, GELU, residual), the per-head RMSNorm + gated output
projection, and the long-row layer whose waves each run several chunks of K.

Everything is fp32, as the reference decodes. Tolerance: max relative error max|y - ref| / max|ref| <= 1e-5 (fp32
sums in another order). Results must be bit-identical from call to call, and a captured graph must replay correctly
with new inputs."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def reference(x, W, mode, nw, nb, eps, bias, scale, act, resid):
    xd, Wd = x.double(), W.double()
    B, K = x.shape
    if mode == 1:
        z = F.layer_norm(xd, (K,), nw.double(), None if nb is None else nb.double(), eps)
    elif mode in (2, 3):
        G = 64 if mode == 2 else 128
        z = F.rms_norm(xd.view(B, K // G, G), (G,), nw.double(), eps).view(B, K)
    else:
        z = xd
    r = z @ Wd.t()
    if scale is not None:
        r = r * scale.double()
    if bias is not None:
        r = r + bias.double()
    if act == 1:
        r = F.gelu(r)
    if resid is not None:
        r = r + resid.double()
    return r


def inputs(B, K, N, mode, act, res, seed, mean=0.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(B, K, device="cuda", generator=g) + mean
    W = torch.randn(N, K, device="cuda", generator=g) * 0.05
    nw = (1 + 0.1 * torch.randn({2: 64, 3: 128}.get(mode, K), device="cuda", generator=g)) if mode else None
    nb = torch.randn(K, device="cuda", generator=g) if mode == 1 else None
    bias = torch.randn(N, device="cuda", generator=g) if act else None
    scale = torch.rand(1, device="cuda", generator=g) if res else None
    resid = torch.randn(B, N, device="cuda", generator=g) if res else None
    return x, W, nw, nb, bias, scale, resid


def run(x, W, mode, nw, nb, eps, bias, scale, act, resid):
    """The layer through decode_gemm: mode 1 folds the LayerNorm's weight and bias (decode_gemm_ln), modes 2 and 3
    the RMSNorm's weight into the tiled weight's columns."""
    from pragnosia_amd import ops
    N = W.shape[0]
    if mode == 1:
        Wt, csum, b = ops.decode_gemm_ln(W, nw, nb, bias, scale)
        return torch.ops.pragnosia.decode_gemm(x, Wt, N, 1, csum, eps, b, scale, act, resid)
    Wt = ops.decode_gemm_tile(W, nw if mode in (2, 3) else None)
    return torch.ops.pragnosia.decode_gemm(x, Wt, N, mode, None, eps, bias, scale, act, resid)


SHAPES = [(768, 2328, 1, 0, False),   # the carrier's projections (LayerNorm)
          (768, 768, 2, 0, True),     # RMSNorm + gated o-projection + residual (12 waves, one head each)
          (768, 3072, 1, 1, False),   # MLP in: LayerNorm + bias + GELU
          (3072, 768, 0, 0, True),    # MLP out: bias-free here, residual; 2 chunks a wave
          (768, 8192, 1, 0, False),   # the tied head
          (256, 200, 1, 1, True),     # a ragged column tile, small K
          (128, 1000, 0, 1, False),   # fewer than four waves
          (512, 300, 2, 1, True),     # RMS over 8 groups
          (768, 768, 3, 0, True),     # 128-dim heads: RMSNorm over 6 groups of 128 + gated o-projection
          (2048, 300, 3, 1, True),    # 16 groups of 128
          (1024, 640, 1, 0, False),   # LayerNorm over 16 waves of 4 steps
          (3072, 520, 1, 0, True),    # LayerNorm moments merged over 2 chunks a wave
          (4096, 300, 1, 1, True),    # ... and over 4 chunks a wave
          (768, 4000, 0, 1, True),    # no normalisation, three column tiles a workgroup from 64 rows (a partial last group)
          (4096, 520, 0, 0, True)]    # 16 waves of 4 chunks of 4 steps


@pytest.mark.parametrize("B", [5, 13, 32, 64, 100])
@pytest.mark.parametrize("K,N,mode,act,res", SHAPES)
def test_decode_gemm_matches_torch(B, K, N, mode, act, res):
    x, W, nw, nb, bias, scale, resid = inputs(B, K, N, mode, act, res, B + K + N + mode)
    eps = 1e-5 if mode == 1 else torch.finfo(torch.float32).eps
    y = run(x, W, mode, nw, nb, eps, bias, scale, act, resid)
    r = reference(x, W, mode, nw, nb, eps, bias, scale, act, resid)
    assert rel(y, r) < 1e-5, (B, K, N, mode)
    assert torch.equal(y, run(x, W, mode, nw, nb, eps, bias, scale, act, resid))


@pytest.mark.parametrize("mean,spread", [(40.0, 1.0), (0.0, 1e-3), (-300.0, 20.0)])
def test_layer_norm_with_offset_rows(mean, spread):
    """LayerNorm input rows far from zero or of small spread: the moments are exact two-pass ones merged pairwise and
    the products run on the row shifted by its first entry, so neither cancels."""
    B, K, N = 64, 768, 2328
    x, W, nw, nb, _, _, _ = inputs(B, K, N, 1, 0, False, 7)
    x = x * spread + mean
    y = run(x, W, 1, nw, nb, 1e-5, None, None, 0, None)
    assert rel(y, reference(x, W, 1, nw, nb, 1e-5, None, None, 0, None)) < 1e-5


def test_tile_layout():
    """decode_gemm_tile against the layout stated in the header, element by element on a small weight."""
    from pragnosia_amd import ops
    N, K = 21, 32
    W = torch.arange(N * K, dtype=torch.float32).reshape(N, K)
    Wt = ops.decode_gemm_tile(W)
    assert Wt.numel() == 32 * K
    KS = K // 16
    for t in range(2):
        for s in range(KS):
            for lane in range(64):
                for e in range(4):
                    n, k = 16 * t + lane % 16, 16 * s + 4 * (lane // 16) + e
                    want = W[n, k].item() if n < N else 0.0
                    assert Wt[((t * KS + s) * 64 + lane) * 4 + e].item() == want


def test_graph_replay_with_new_inputs():
    """Three dependent layers (each mode) captured into one graph and replayed with new inputs copied into the captured
    buffers, eager work and synchronisations between replays: every replay equals the eager calls bit for bit."""
    from pragnosia_amd import ops
    op = torch.ops.pragnosia
    B, d = 64, 768
    g = torch.Generator(device="cuda").manual_seed(11)
    W1 = torch.randn(3072, d, device="cuda", generator=g) * 0.05
    W2 = torch.randn(d, 3072, device="cuda", generator=g) * 0.05
    W3 = torch.randn(d, d, device="cuda", generator=g) * 0.05
    lw, lb = 1 + 0.1 * torch.randn(d, device="cuda", generator=g), torch.randn(d, device="cuda", generator=g)
    w64 = 1 + 0.1 * torch.randn(64, device="cuda", generator=g)
    b1 = torch.randn(3072, device="cuda", generator=g)
    sc = torch.rand(1, device="cuda", generator=g)
    T1, c1, b1f = ops.decode_gemm_ln(W1, lw, lb, b1)
    T2, T3 = ops.decode_gemm_tile(W2), ops.decode_gemm_tile(W3, w64)
    x = torch.randn(B, d, device="cuda", generator=g)
    eps = torch.finfo(torch.float32).eps

    def chain(x):
        h = op.decode_gemm(x, T1, 3072, 1, c1, 1e-5, b1f, None, 1, None)
        y = op.decode_gemm(h, T2, d, 0, None, 0.0, None, None, 0, x)
        return op.decode_gemm(y, T3, d, 2, None, eps, None, sc, 0, y)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = chain(x)
    for rep in range(4):
        x.copy_(torch.randn(B, d, device="cuda", generator=g))
        graph.replay()
        torch.cuda.synchronize()
        want = chain(x.clone())
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep


ACC_SHAPES = [(3072, 768),   # the MLP's second layer at d 768: four splits of 768
              (2816, 704),   # d 704: four splits of 704
              (1024, 300),   # two splits of 512, a ragged last column tile
              (4096, 2048),  # four splits of 1024, three column tiles a workgroup
              (768, 520)]    # one split: a plain atomic add into the residual


@pytest.mark.parametrize("B", [5, 64, 100])
@pytest.mark.parametrize("K,N", ACC_SHAPES)
def test_decode_gemm_acc_adds_into_residual(B, K, N):
    """decode_gemm_acc_ (y += scale * W x + bias, K split over workgroups that add with atomics) against fp64 torch
    and against decode_gemm's residual epilogue at the same tolerance; the adds' order varies, so two calls agree to
    the tolerance, not bit for bit."""
    from pragnosia_amd import ops
    x, W, _, _, bias, scale, resid = inputs(B, K, N, 0, 1, True, 3 * B + K + N)
    Wt = ops.decode_gemm_tile(W)
    r = reference(x, W, 0, None, None, 0.0, bias, scale, 0, resid)
    y = resid.clone()
    torch.ops.pragnosia.decode_gemm_acc_(x, Wt, 0, 0.0, bias, scale, y)
    assert rel(y, r) < 1e-5, (B, K, N)
    y2 = resid.clone()
    torch.ops.pragnosia.decode_gemm_acc_(x, Wt, 0, 0.0, None, None, y2)
    assert rel(y2, reference(x, W, 0, None, None, 0.0, None, None, 0, resid)) < 1e-5
    full = torch.ops.pragnosia.decode_gemm(x, Wt, N, 0, None, 0.0, bias, scale, 0, resid)
    assert rel(y, full) < 1e-5


RMS_ACC_SHAPES = [(768, 768, 2),    # the o-projection at d 768, heads of 64: three splits of four heads
                  (1536, 768, 2),   # 24 heads of 64: four splits of six
                  (1024, 300, 2),   # 16 heads: four splits of four, a ragged last column tile
                  (1536, 520, 3),   # 12 heads of 128: three splits of four
                  (768, 768, 3),    # 6 heads of 128: one split
                  (640, 300, 2)]    # 10 heads of 64: two splits of five


@pytest.mark.parametrize("B", [5, 64, 100])
@pytest.mark.parametrize("K,N,mode", RMS_ACC_SHAPES)
def test_decode_gemm_acc_rms_groups(B, K, N, mode):
    """The accumulating form in the RMS modes (the carrier's per-head RMSNorm + gated o-projection added into the
    residual, K split at head boundaries) against fp64 torch and against decode_gemm's residual epilogue, 1e-5."""
    from pragnosia_amd import ops
    x, W, nw, _, _, scale, resid = inputs(B, K, N, mode, 0, True, 5 * B + K + N + mode)
    eps = torch.finfo(torch.float32).eps
    Wt = ops.decode_gemm_tile(W, nw)
    r = reference(x, W, mode, nw, None, eps, None, scale, 0, resid)
    y = resid.clone()
    torch.ops.pragnosia.decode_gemm_acc_(x, Wt, mode, eps, None, scale, y)
    assert rel(y, r) < 1e-5, (B, K, N, mode)
    if ops.decode_gemm_ok(K, mode):  # 24 heads of 64 exceed the unsplit form's 16 waves; each split holds six
        full = torch.ops.pragnosia.decode_gemm(x, Wt, N, mode, None, eps, None, scale, 0, resid)
        assert rel(y, full) < 1e-5


def test_decode_gemm_acc_graph_replay():
    """The MLP's two layers with the second added into the residual in place, captured and replayed with new inputs
    and eager work between replays: every replay within 1e-5 of the eager result."""
    from pragnosia_amd import ops
    op = torch.ops.pragnosia
    B, d = 64, 768
    g = torch.Generator(device="cuda").manual_seed(12)
    W1 = torch.randn(3072, d, device="cuda", generator=g) * 0.05
    W2 = torch.randn(d, 3072, device="cuda", generator=g) * 0.05
    lw, lb = 1 + 0.1 * torch.randn(d, device="cuda", generator=g), torch.randn(d, device="cuda", generator=g)
    b1, b2 = torch.randn(3072, device="cuda", generator=g), torch.randn(d, device="cuda", generator=g)
    T1, c1, b1f = ops.decode_gemm_ln(W1, lw, lb, b1)
    T2 = ops.decode_gemm_tile(W2)
    x = torch.randn(B, d, device="cuda", generator=g)

    def mlp(x):
        h = op.decode_gemm(x, T1, 3072, 1, c1, 1e-5, b1f, None, 1, None)
        y = x.clone()
        op.decode_gemm_acc_(h, T2, 0, 0.0, b2, None, y)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = mlp(x)
    for i in range(3):
        x.copy_(torch.randn(B, d, device="cuda", generator=g) * (1 + i))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = mlp(x.clone())
        torch.cuda.synchronize()
        assert rel(out, want) < 1e-5, i
