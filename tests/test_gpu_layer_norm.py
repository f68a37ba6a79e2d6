"""GPU parity of the LayerNorm kernels (`pragnosia::layer_norm`, the carrier's and the MLP's `nn.LayerNorm(d)`,
src/assoc.py:323,388, src/model.py:555) against torch in fp64.

Tolerances: fp32 outputs and every gradient 1e-4 (max |x - ref| / max |ref|; the fp32 bound); the bf16 output within
2^-8 (one rounding of the fp32 value); with a bf16 upstream gradient the reference is fed the same bf16-rounded
gradient, so the bound stays 1e-4."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _inputs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    D = shape[-1]
    x = torch.randn(*shape, generator=g) * 2.0 + 0.5
    w = 1.0 + 0.3 * torch.randn(D, generator=g)
    b = 0.2 * torch.randn(D, generator=g)
    dy = torch.randn(*shape, generator=g)
    return x, w, b, dy


@pytest.mark.parametrize("shape", [(3, 200, 768), (1000, 256), (7, 2048), (1, 1, 1024), (5, 512), (33, 1280),
                                   (4, 257, 704), (9, 100), (50, 68), (6, 2044), (37, 4)])
@pytest.mark.parametrize("dy_bf16", [False, True])
def test_layer_norm_forward_backward(shape, dy_bf16):
    from pragnosia_amd import ops  # noqa: F401
    x, w, b, dy = _inputs(shape, seed=shape[-1] + len(shape))
    if dy_bf16:
        dy = dy.bfloat16().float()  # the reference sees the gradient the kernel sees
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    yr = F.layer_norm(xr, (shape[-1],), wr, br, 1e-5)
    (yr * dy.double()).sum().backward()
    xk, wk, bk = (t.cuda().requires_grad_(True) for t in (x, w, b))
    y, mean, rstd = torch.ops.pragnosia.layer_norm(xk, wk, bk, 1e-5, False)
    y.backward(dy.cuda().bfloat16() if dy_bf16 else dy.cuda())
    assert y.dtype == torch.float32 and rel(y, yr) < 1e-4
    x2 = x.double().reshape(-1, shape[-1])
    assert rel(mean, x2.mean(-1)) < 1e-5
    assert rel(rstd, 1.0 / torch.sqrt(x2.var(-1, unbiased=False) + 1e-5)) < 1e-5
    for a, r in ((xk, xr), (wk, wr), (bk, br)):
        assert rel(a.grad, r.grad) < 1e-4


def test_layer_norm_bf16_output():
    from pragnosia_amd import ops  # noqa: F401
    x, w, b, _ = _inputs((4, 300, 768), seed=9)
    y, _, _ = torch.ops.pragnosia.layer_norm(x.cuda(), w.cuda(), b.cuda(), 1e-5, True)
    ref = F.layer_norm(x.double(), (768,), w.double(), b.double(), 1e-5)
    assert y.dtype == torch.bfloat16 and rel(y.float(), ref) < 2 ** -8


def test_layer_norm_helper_dtype_and_fallback():
    """The module helper: fp32 output without autocast, bf16 under bf16 autocast (the dtype of the matmul after it),
    and nn.LayerNorm itself for a shape the kernels do not take (D = 90, not a multiple of 4)."""
    from pragnosia_amd.ops import layer_norm
    torch.manual_seed(3)
    mod = torch.nn.LayerNorm(768).cuda()
    x = torch.randn(2, 50, 768, device="cuda")
    assert layer_norm(x, mod).dtype == torch.float32 and rel(layer_norm(x, mod), mod(x)) < 1e-5
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yb = layer_norm(x, mod)
    assert yb.dtype == torch.bfloat16 and rel(yb.float(), mod(x)) < 2 ** -8
    small = torch.nn.LayerNorm(90).cuda()
    xs = torch.randn(3, 90, device="cuda")
    assert torch.equal(layer_norm(xs, small), small(xs))


def test_layer_norm_graph_replays():
    """Forward and backward captured in a HIP graph: no memset node (the weight and bias gradients are GEMM column
    sums), and three replays on new inputs, with eager work between them, equal to the eager call."""
    from pragnosia_amd import ops  # noqa: F401
    from test_gpu_training import _memset_nodes
    torch.manual_seed(4)
    mod = torch.nn.LayerNorm(768).cuda()
    xs = torch.randn(16, 64, 768, device="cuda", requires_grad=True)
    gs = torch.randn(16, 64, 768, device="cuda")

    def step():
        y, _, _ = torch.ops.pragnosia.layer_norm(xs, mod.weight, mod.bias, 1e-5, True)
        y.backward(gs.bfloat16())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in (xs, mod.weight, mod.bias):
        t.grad = torch.zeros_like(t)  # the captured backward accumulates into these buffers
    g = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(g):
        step()
    assert _memset_nodes(g) == 0
    for i in range(3):
        with torch.no_grad():
            xs.copy_(torch.randn(16, 64, 768, device="cuda"))
            gs.copy_(torch.randn(16, 64, 768, device="cuda"))
        for t in (xs, mod.weight, mod.bias):
            t.grad.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = [t.grad.clone() for t in (xs, mod.weight, mod.bias)]
        xe = xs.detach().clone().requires_grad_(True)
        wr = mod.weight.detach().clone().requires_grad_(True)
        br = mod.bias.detach().clone().requires_grad_(True)
        ye, _, _ = torch.ops.pragnosia.layer_norm(xe, wr, br, 1e-5, True)
        ye.backward(gs.bfloat16())
        assert torch.equal(got[0], xe.grad), i
        assert rel(got[1], wr.grad) < 1e-6 and rel(got[2], br.grad) < 1e-6, i


@pytest.mark.parametrize("shape", [(1, 5), (512, 768), (37, 36), (1000, 384), (4096, 64), (129, 2048)])
def test_colsum_kernel(shape):
    """`pragnosia_colsum_f32` (the sum of the kernels' partial rows) against an fp64 column sum, and repeatable bit
    for bit; a tensor past COLSUM_MAX_ROWS takes the GEMM form."""
    from pragnosia_amd import ops
    g = torch.Generator().manual_seed(shape[0] * 7 + shape[1])
    x = torch.randn(*shape, generator=g)
    got = ops.colsum(x.cuda())
    assert got.shape == (shape[1],) and rel(got, x.double().sum(0)) < 1e-6
    assert torch.equal(got, ops.colsum(x.cuda()))
    big = torch.randn(ops.COLSUM_MAX_ROWS + 3, 40, generator=g)
    assert rel(ops.colsum(big.cuda()), big.double().sum(0)) < 1e-5
