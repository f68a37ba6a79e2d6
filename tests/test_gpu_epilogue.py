"""GPU parity of the carrier's output epilogue (pragnosia_aspin_out_fwd / _bwd through the C ABI): the per-head
RMSNorm of the scan output written token-major, against an fp64 restatement of nn.RMSNorm(dk) (eps=None: fp32
epsilon) followed by the transpose, and against the torch expression it replaces in the module.

Tolerances: the forward rounds once to the output dtype, so max relative error max|x - ref| / max|ref| <= 2^-8 for
bf16 output and 1e-6 for fp32; gradients (dO rounded to bf16) <= 1e-2, the weight gradient (fp32 sums) <= 1e-5."""
import pytest
import torch

pytestmark = pytest.mark.gpu
EPS = torch.finfo(torch.float32).eps


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _ref(o, w):
    """fp64: y[b, t, h*D + d] = o[b, h, t, d] r w[d], r = (mean_d o^2 + eps)^-1/2."""
    x = o.double()
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + EPS)
    B, H, T, D = o.shape
    return (x * r * w.double()).transpose(1, 2).reshape(B, T, H * D)


@pytest.mark.parametrize("B,H,T,scale,D", [(2, 3, 333, 1.0, 64), (1, 12, 64, 1e-3, 64), (3, 2, 1, 10.0, 64),
                                           (2, 12, 512, 0.05, 64), (2, 3, 333, 1.0, 128), (2, 6, 512, 0.05, 128),
                                           (1, 2, 7, 10.0, 128)])
@pytest.mark.parametrize("out_bf16", [True, False])
def test_epilogue_forward_and_backward_match_fp64(B, H, T, scale, D, out_bf16):
    import pragnosia_amd.ops  # noqa: F401
    g = torch.Generator().manual_seed(B * T + H)
    o = (torch.randn(B, H, T, D, generator=g) * scale).bfloat16()
    w = torch.randn(D, generator=g)
    gy = torch.randn(B, T, H * D, generator=g)
    od = o.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    y, rstd = torch.ops.pragnosia.aspin_out(od, wd, EPS, out_bf16)
    assert y.dtype == (torch.bfloat16 if out_bf16 else torch.float32) and y.shape == (B, T, H * D)
    gyd = gy.cuda().to(y.dtype)
    (y.float() * gyd.float()).sum().backward()
    orr = o.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    yr = _ref(orr, wr)
    (yr * gyd.double().cpu()).sum().backward()
    tol = 2 ** -8 if out_bf16 else 1e-6
    assert rel(y, yr) < tol
    assert rel(od.grad, orr.grad) < 1e-2
    assert rel(wd.grad, wr.grad) < 1e-5


def test_module_epilogue_equals_torch_expression():
    """AssocCarrier._epilogue against `self.on(o.to(dtype)).transpose(1, 2).reshape(B, T, D)` on the GPU, forward and
    backward, under autocast (bf16) and without (fp32)."""
    from pragnosia_amd.assoc import AssocCarrier
    torch.manual_seed(5)
    m = AssocCarrier(256).cuda()
    with torch.no_grad():
        m.on.weight.add_(torch.randn_like(m.on.weight) * 0.3)
    o = (torch.randn(2, 4, 200, 64, device="cuda") * 0.2).bfloat16()
    for dtype in (torch.bfloat16, torch.float32):
        gy = torch.randn(2, 200, 256, device="cuda")
        a = o.clone().requires_grad_(True)
        y = m._epilogue(a, dtype)
        (y.float() * gy).sum().backward()
        ga, gw = a.grad.clone(), m.on.weight.grad.clone()
        m.on.weight.grad = None
        b = o.clone().requires_grad_(True)
        yr = m.on(b.to(dtype)).transpose(1, 2).reshape(2, 200, 256)
        (yr.float() * gy).sum().backward()
        tol = 2 ** -7 if dtype == torch.bfloat16 else 1e-5
        assert y.dtype == yr.dtype and rel(y, yr) < tol
        assert rel(ga, b.grad) < 2e-2 and rel(gw, m.on.weight.grad) < 1e-3
        m.on.weight.grad = None
