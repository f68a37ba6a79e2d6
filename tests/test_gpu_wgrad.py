"""GPU parity of the split-K weight-gradient kernel (`pragnosia::wgrad`, C ABI `pragnosia_wgrad_bf16`): dW = dYᵀ X
over token rows for the linear layers around the carrier and the MLP (src/assoc.py:384-512, src/model.py:552-560).

The operands are bf16 and their products exact in fp32, so the reference is the fp64 product of the same bf16
values; the kernel sums in fp32 in another order: bound 1e-5 of max |C| (fp32 rounding over K terms). Against
autograd's own bf16 GEMM (rounded to bf16, then cast) the bound is one bf16 rounding, 2^-8."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _ab(K, M, N, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(K, M, generator=g).bfloat16().cuda(), torch.randn(K, N, generator=g).bfloat16().cuda())


@pytest.mark.parametrize("K,M,N", [(8192, 768, 768), (8192, 2328, 768), (8192, 3072, 768), (8192, 768, 3072),
                                   (1000, 24, 40), (64, 8, 8), (130, 136, 264), (1, 16, 8), (70000, 8, 16)])
def test_wgrad_matches_fp64(K, M, N):
    from pragnosia_amd import ops
    A, B = _ab(K, M, N, seed=K + M + N)
    got = ops.wgrad(A, B)
    ref = A.double().t() @ B.double()
    assert got.dtype == torch.float32 and got.shape == (M, N)
    assert rel(got, ref) < 1e-5
    assert torch.equal(got, ops.wgrad(A, B))  # deterministic: fixed split and summation order


def test_wgrad_c_abi_strided_and_accumulate():
    """Row pitches wider than the matrices (column slices of wider tensors) and C += AᵀB."""
    from pragnosia_amd._lib import lib
    from pragnosia_amd.ops import _ptr
    K, M, N = 3000, 136, 200
    Aw, Bw = _ab(K, M + 24, N + 40, seed=3)
    A, B = Aw[:, 8:8 + M], Bw[:, 16:16 + N]
    Cw = torch.randn(M, N + 12, device="cuda")
    C0 = Cw.clone()
    nbytes = lib().pragnosia_wgrad_workspace_bytes(M, N, K)
    ws = torch.empty(max(nbytes, 1), device="cuda", dtype=torch.uint8)
    rc = lib().pragnosia_wgrad_bf16(_ptr(A), Aw.stride(0), _ptr(B), Bw.stride(0), _ptr(Cw), Cw.stride(0), 1,
                                    _ptr(ws), nbytes, M, N, K, None)
    torch.cuda.synchronize()
    assert rc == 0
    ref = C0[:, :N].double().cpu() + A.double().t().cpu() @ B.double().cpu()
    assert rel(Cw[:, :N], ref) < 1e-5
    assert torch.equal(Cw[:, N:], C0[:, N:])  # columns past N untouched


def test_linear_weight_gradient_under_autocast():
    """`linear_w` (the carrier's projections, the MLP) under bf16 autocast: output as F.linear's, input and bias
    gradients as autograd's, the weight gradient the fp32 sum of the bf16 products (fp64 reference) and within one
    bf16 rounding of autograd's."""
    from pragnosia_amd import ops
    torch.manual_seed(5)
    x = torch.randn(4, 300, 768, device="cuda", requires_grad=True)
    W = torch.randn(2328, 768, device="cuda", requires_grad=True)
    b = torch.randn(2328, device="cuda", requires_grad=True)
    gy = torch.randn(4, 300, 2328, device="cuda").bfloat16()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = ops.linear_w(x, W, b)
    y.backward(gy)
    xr, Wr, br = (t.detach().clone().requires_grad_(True) for t in (x, W, b))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yr = torch.nn.functional.linear(xr, Wr, br)
    yr.backward(gy)
    assert y.dtype == yr.dtype == torch.bfloat16 and torch.equal(y, yr)
    assert torch.equal(x.grad, xr.grad)
    assert W.grad.dtype == torch.float32
    ref = gy.reshape(-1, 2328).double().t() @ x.detach().bfloat16().reshape(-1, 768).double()
    assert rel(W.grad, ref) < 1e-5 and rel(W.grad, Wr.grad) < 2 ** -8
    assert rel(b.grad, br.grad) < 2 ** -7  # both bf16 column sums (a ones GEMM here), each rounded once


def test_wgrad_graph_replays():
    """wgrad captured in a HIP graph: no memset node, and replays on new inputs equal the eager call bit for bit."""
    from pragnosia_amd import ops
    from test_gpu_training import _memset_nodes
    A, B = _ab(4096, 768, 768, seed=11)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.wgrad(A, B)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(g):
        C = ops.wgrad(A, B)
    assert _memset_nodes(g) == 0
    for i in range(3):
        A2, B2 = _ab(4096, 768, 768, seed=20 + i)
        A.copy_(A2)
        B.copy_(B2)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, ops.wgrad(A2, B2)), i
