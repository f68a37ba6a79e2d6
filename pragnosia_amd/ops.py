"""torch custom ops (namespace `pragnosia`) over the C ABI of libpragnosia_hip.so.

Every op allocates its outputs with torch on the input's device, makes its inputs contiguous, launches on the
current HIP stream and returns; nothing synchronises, so the ops are hipGraph-capturable once shapes are fixed.
Each op has a fake (meta) implementation for torch.compile and, where differentiable, a registered backward that is
itself a custom op. There is no CPU path: a CPU tensor raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from ._lib import PragnosiaError, check, lib


def _ptr(t: Optional[Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_gpu(*ts: Optional[Tensor]) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise PragnosiaError("pragnosia_amd runs on a ROCm GPU only: got a tensor on "
                                 f"{t.device}; there is no CPU fallback")


def _f32(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.to(torch.float32).contiguous()


COLSUM_MAX_ROWS = 4096  # above this many rows the GEMM form (more workgroups per column) is the faster one


def colsum(x: Tensor) -> Tensor:
    """Sum over the first dimension. torch's column sum over many rows is a multi-block reduction that zeroes its
    semaphores with a memset, and memset nodes captured in a HIP graph have given wrong results on replays after the
    first on this ROCm stack. A contiguous fp32 GPU tensor of at most COLSUM_MAX_ROWS rows (the kernels' partial
    rows) is summed by `pragnosia_colsum_f32` (one launch, a fixed order); anything else as a GEMM against a ones
    vector. Neither records a memset. Same function, the terms summed in another order."""
    rows = x.shape[0]
    x2 = x.reshape(rows, -1)
    if x2.is_cuda and x2.dtype == torch.float32 and x2.is_contiguous() and 0 < rows <= COLSUM_MAX_ROWS and x2.numel():
        out = torch.empty(x2.shape[1], device=x.device, dtype=torch.float32)
        check(lib().pragnosia_colsum_f32(_ptr(x2), rows, x2.shape[1], _ptr(out), _stream(x2)), "pragnosia_colsum_f32")
        return out.reshape(x.shape[1:])
    return (torch.ones(1, rows, device=x.device, dtype=x2.dtype) @ x2).reshape(x.shape[1:])


@torch.library.custom_op("pragnosia::wgrad", mutates_args=())
def wgrad(dy: Tensor, x: Tensor) -> Tensor:
    """The weight gradient of y = x Wᵀ over token rows, dy (K, M) and x (K, N) bf16 → dW = dyᵀ x (M, N) fp32: the
    split-K MFMA kernel `pragnosia_wgrad_bf16`, the fp32 accumulator being the result (autograd's form is a bf16 GEMM
    whose result is cast to the fp32 parameter). M and N multiples of 8."""
    _require_gpu(dy, x)
    if dy.dim() != 2 or x.dim() != 2 or dy.shape[0] != x.shape[0]:
        raise PragnosiaError(f"wgrad: dy (K, M) and x (K, N) expected, got {tuple(dy.shape)} and {tuple(x.shape)}")
    _expect("wgrad", dy.device, x=(x, (dy.shape[0], None)))
    dy, x = _bf16(dy), _bf16(x)
    K, M = dy.shape
    N = x.shape[1]
    nbytes = lib().pragnosia_wgrad_workspace_bytes(M, N, K)
    if nbytes < 0:
        raise PragnosiaError(f"wgrad: shape M={M} N={N} K={K} rejected (M and N must be multiples of 8)")
    out = torch.empty(M, N, device=dy.device, dtype=torch.float32)
    ws = torch.empty(nbytes, device=dy.device, dtype=torch.uint8) if nbytes else None
    check(lib().pragnosia_wgrad_bf16(_ptr(dy), M, _ptr(x), N, _ptr(out), N, 0, _ptr(ws), nbytes, M, N, K,
                                     _stream(dy)), "pragnosia_wgrad_bf16")
    return out


@wgrad.register_fake
def _(dy, x):
    return dy.new_empty(dy.shape[1], x.shape[1], dtype=torch.float32)


def weight_grad(g2: Tensor, x2: Tensor) -> Tensor:
    """g2ᵀ x2 over token rows (the weight gradient of F.linear): `wgrad` in fp32 for bf16 GPU operands whose widths
    are multiples of 8 (autocast's case), a matmul in the operands' dtype otherwise."""
    if (g2.is_cuda and g2.dtype == torch.bfloat16 and x2.dtype == torch.bfloat16 and g2.shape[0] > 0
            and g2.shape[1] % 8 == 0 and x2.shape[1] % 8 == 0):
        return wgrad(g2, x2)
    return g2.t() @ x2


class _Linear(torch.autograd.Function):
    """F.linear(x, W, b) whose backward forms the weight gradient with `weight_grad` (the split-K kernel under bf16
    autocast) and the bias gradient with `colsum` instead of torch's column sum, so a backward captured in a HIP graph
    records no memset node; the input gradient is the usual GEMM. Runs in the autocast dtype like F.linear."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, W, b):
        # under autocast the operands are cast once here, as F.linear would, and the casts are what the backward
        # reads (no second cast of W there)
        ctx.dtypes = (x.dtype, W.dtype)  # the gradients' dtypes
        ctx.b_dtype = None if b is None else b.dtype
        low = (torch.float32, torch.float16, torch.bfloat16)  # the dtypes autocast casts (fp64 stays as it is)
        if (torch.is_autocast_enabled("cuda") and x.is_cuda and x.dtype in low and W.dtype in low
                and (b is None or b.dtype in low)):
            dt = torch.get_autocast_dtype("cuda")
            x, W, b = x.to(dt), W.to(dt), (None if b is None else b.to(dt))
        ctx.save_for_backward(x, W)
        return F.linear(x, W, b)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, g):
        x, W = ctx.saved_tensors
        x_dtype, W_dtype = ctx.dtypes
        g2 = g.reshape(-1, g.shape[-1])
        cdt = g2.dtype
        gx = (g2 @ W.to(cdt)).reshape(x.shape).to(x_dtype) if ctx.needs_input_grad[0] else None
        gW = weight_grad(g2, x.reshape(-1, x.shape[-1]).to(cdt)).to(W_dtype) if ctx.needs_input_grad[1] else None
        gb = colsum(g2).to(ctx.b_dtype) if (ctx.b_dtype is not None and ctx.needs_input_grad[2]) else None
        return gx, gW, gb


def linear(x: Tensor, mod) -> Tensor:
    """`mod(x)` for an nn.Linear `mod`, with the split-K weight gradient and a graph-capturable bias gradient (see
    _Linear)."""
    return linear_w(x, mod.weight, mod.bias)


def linear_w(x: Tensor, W: Tensor, b: Optional[Tensor] = None) -> Tensor:
    """F.linear(x, W, b), under autograd through _Linear."""
    if not torch.is_grad_enabled():
        return F.linear(x, W, b)
    return _Linear.apply(x, W, b)


def _expect(op: str, dev, **shapes) -> None:
    """Reject, before anything is launched, an argument whose shape differs from the one the kernels assume or that
    lives on another device than `dev`: the C ABI takes raw pointers and sizes, so a mismatch there would read or
    write past a buffer instead of raising. `shapes` maps an argument name to (tensor or None, expected shape), a
    shape entry None matching any size; a shape of () for a scalar accepts any one-element tensor."""
    for name, (t, shape) in shapes.items():
        if t is None:
            continue
        if shape == ():
            ok = t.numel() == 1
        else:
            ok = t.dim() == len(shape) and all(s is None or t.shape[i] == s for i, s in enumerate(shape))
        if not ok:
            want = "one element" if shape == () else str(tuple("*" if s is None else s for s in shape))
            raise PragnosiaError(f"{op}: {name} has shape {tuple(t.shape)}, expected {want}")
        if t.device != dev:
            raise PragnosiaError(f"{op}: {name} is on {t.device}, expected {dev}")


# ---------------------------------------------------------------------------------------------------------------
# complex diagonal scan (fspin): replaces src/scan_kernel.py:105-148
@torch.library.custom_op("pragnosia::diag_scan", mutates_args=())
def diag_scan(u: Tensor, logmag: Tensor, ang: Tensor, h0r: Optional[Tensor],
              h0i: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """h_t = exp(logmag_t + i ang_t) h_{t-1} + u_t over (B, T, D) fp32. Returns (Re h, Re h_last, Im h_last, Im h);
    the last output is the saved imaginary part for the backward (not differentiable)."""
    _require_gpu(u, logmag, ang, h0r, h0i)
    if u.dim() != 3 or (h0r is None) != (h0i is None):
        raise PragnosiaError("diag_scan: u must be (B, T, D), and h0r and h0i given together")
    B, T, D = u.shape
    _expect("diag_scan", u.device, logmag=(logmag, (B, T, D)), ang=(ang, (B, T, D)), h0r=(h0r, (B, D)),
            h0i=(h0i, (B, D)))
    u, logmag, ang, h0r, h0i = _f32(u), _f32(logmag), _f32(ang), _f32(h0r), _f32(h0i)
    hr = torch.empty(B, T, D, device=u.device, dtype=torch.float32)
    hi = torch.empty_like(hr)
    hrl = torch.empty(B, D, device=u.device, dtype=torch.float32)
    hil = torch.empty_like(hrl)
    check(lib().pragnosia_diag_scan_fwd(_ptr(u), _ptr(logmag), _ptr(ang), _ptr(h0r), _ptr(h0i), _ptr(hr), _ptr(hi),
                                        _ptr(hrl), _ptr(hil), B, T, D, _stream(u)), "pragnosia_diag_scan_fwd")
    return hr, hrl, hil, hi


@diag_scan.register_fake
def _(u, logmag, ang, h0r, h0i):
    B, T, D = u.shape
    e = lambda *s: u.new_empty(*s, dtype=torch.float32)
    return e(B, T, D), e(B, D), e(B, D), e(B, T, D)


@torch.library.custom_op("pragnosia::diag_scan_bwd", mutates_args=())
def diag_scan_bwd(g: Tensor, g_last_r: Optional[Tensor], g_last_i: Optional[Tensor], logmag: Tensor, ang: Tensor,
                  hr: Tensor, hi: Tensor, h0r: Optional[Tensor],
                  h0i: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The adjoint recurrence. Returns (du, dlogmag, dang, dh0r, dh0i); dh0r/dh0i are empty when h0 was None."""
    _require_gpu(g, logmag, ang, hr, hi)
    if g.dim() != 3 or (h0r is None) != (h0i is None):
        raise PragnosiaError("diag_scan_bwd: g must be (B, T, D), and h0r and h0i given together")
    B, T, D = g.shape
    _expect("diag_scan_bwd", g.device, g_last_r=(g_last_r, (B, D)), g_last_i=(g_last_i, (B, D)),
            logmag=(logmag, (B, T, D)), ang=(ang, (B, T, D)), hr=(hr, (B, T, D)), hi=(hi, (B, T, D)),
            h0r=(h0r, (B, D)), h0i=(h0i, (B, D)))
    g, g_last_r, g_last_i = _f32(g), _f32(g_last_r), _f32(g_last_i)
    logmag, ang, hr, hi, h0r, h0i = _f32(logmag), _f32(ang), _f32(hr), _f32(hi), _f32(h0r), _f32(h0i)
    du, dlm, dan = (torch.empty(B, T, D, device=g.device, dtype=torch.float32) for _ in range(3))
    has = h0r is not None
    dh0r = torch.empty(B, D, device=g.device) if has else g.new_empty(0)
    dh0i = torch.empty(B, D, device=g.device) if has else g.new_empty(0)
    check(lib().pragnosia_diag_scan_bwd(_ptr(g), _ptr(g_last_r), _ptr(g_last_i), _ptr(logmag), _ptr(ang), _ptr(hr),
                                        _ptr(hi), _ptr(h0r), _ptr(h0i), _ptr(du), _ptr(dlm), _ptr(dan),
                                        _ptr(dh0r) if has else None, _ptr(dh0i) if has else None,
                                        B, T, D, _stream(g)), "pragnosia_diag_scan_bwd")
    return du, dlm, dan, dh0r, dh0i


@diag_scan_bwd.register_fake
def _(g, g_last_r, g_last_i, logmag, ang, hr, hi, h0r, h0i):
    B, T, D = g.shape
    e = lambda *s: g.new_empty(*s, dtype=torch.float32)
    has = h0r is not None
    return e(B, T, D), e(B, T, D), e(B, T, D), e(B, D) if has else e(0), e(B, D) if has else e(0)


def _diag_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    u, logmag, ang, h0r, h0i = inputs
    hr, _, _, hi = output
    ctx.has_h0 = h0r is not None
    ctx.save_for_backward(logmag, ang, hr, hi, h0r, h0i)
    ctx.mark_non_differentiable(hi)


def _diag_backward(ctx, gy, glr, gli, _ghi):
    logmag, ang, hr, hi, h0r, h0i = ctx.saved_tensors
    if gy is None:
        gy = torch.zeros_like(hr)
    du, dlm, dan, dh0r, dh0i = diag_scan_bwd(gy.contiguous(), glr, gli, logmag, ang, hr, hi, h0r, h0i)
    return du, dlm, dan, (dh0r if ctx.has_h0 else None), (dh0i if ctx.has_h0 else None)


diag_scan.register_autograd(_diag_backward, setup_context=_diag_setup)


# ---------------------------------------------------------------------------------------------------------------
# the carrier's output epilogue: replaces `self.on(o).transpose(1, 2).reshape(B, T, D)`, src/assoc.py:505
RMS_EPS = torch.finfo(torch.float32).eps  # nn.RMSNorm(eps=None) computes in fp32 with fp32's epsilon


@torch.library.custom_op("pragnosia::aspin_out", mutates_args=())
def aspin_out(o: Tensor, weight: Tensor, eps: float, out_bf16: bool) -> tuple[Tensor, Tensor]:
    """Per-head RMSNorm of the scan output o (B, H, T, D), D = 64 or 128 (cast to bf16), with `weight` (D,), written
    token-major as (B, T, H * D) in bf16 (out_bf16) or fp32. Returns (y, rstd (B, H, T) fp32, saved for the
    backward)."""
    _require_gpu(o, weight)
    Dw = o.shape[-1] if o.dim() == 4 and o.shape[-1] in (64, 128) else 64
    _expect("aspin_out", o.device, o=(o, (None, None, None, Dw)), weight=(weight, (Dw,)))
    o, weight = _bf16(o), _f32(weight)
    B, H, T, D = o.shape
    y = torch.empty(B, T, H * D, device=o.device, dtype=torch.bfloat16 if out_bf16 else torch.float32)
    rstd = torch.empty(B, H, T, device=o.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_out_fwd(_ptr(o), _ptr(weight), float(eps), _ptr(y), int(out_bf16), _ptr(rstd),
                                        B, H, T, D, _stream(o)), "pragnosia_aspin_out_fwd")
    return y, rstd


@aspin_out.register_fake
def _(o, weight, eps, out_bf16):
    B, H, T, D = o.shape
    return (o.new_empty(B, T, H * D, dtype=torch.bfloat16 if out_bf16 else torch.float32),
            o.new_empty(B, H, T, dtype=torch.float32))


@torch.library.custom_op("pragnosia::aspin_out_bwd", mutates_args=())
def aspin_out_bwd(gy: Tensor, o: Tensor, weight: Tensor, rstd: Tensor) -> tuple[Tensor, Tensor]:
    """Backward of aspin_out. gy (B, T, H * D) bf16 or fp32. Returns (dO (B, H, T, D) bf16, dweight (D,) fp32)."""
    _require_gpu(gy, o, weight, rstd)
    Dw = o.shape[-1] if o.dim() == 4 and o.shape[-1] in (64, 128) else 64
    _expect("aspin_out_bwd", o.device, o=(o, (None, None, None, Dw)), weight=(weight, (Dw,)))
    B, H, T, D = o.shape
    _expect("aspin_out_bwd", o.device, gy=(gy, (B, T, H * D)), rstd=(rstd, (B, H, T)))
    gy = gy.contiguous() if gy.dtype in (torch.bfloat16, torch.float32) else gy.float().contiguous()
    o, weight, rstd = _bf16(o), _f32(weight), _f32(rstd)
    dO = torch.empty(B, H, T, D, device=o.device, dtype=torch.bfloat16)
    n = lib().pragnosia_aspin_out_weight_partials(B, H, T)
    part = torch.empty(n, D, device=o.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_out_bwd(_ptr(gy), int(gy.dtype == torch.bfloat16), _ptr(o), _ptr(weight), _ptr(rstd),
                                        _ptr(dO), _ptr(part), B, H, T, D, _stream(o)), "pragnosia_aspin_out_bwd")
    return dO, colsum(part)


@aspin_out_bwd.register_fake
def _(gy, o, weight, rstd):
    return o.new_empty(o.shape, dtype=torch.bfloat16), o.new_empty(o.shape[-1], dtype=torch.float32)


def _out_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    o, weight, eps, out_bf16 = inputs
    _, rstd = output
    ctx.save_for_backward(o, weight, rstd)
    ctx.mark_non_differentiable(rstd)


def _out_backward(ctx, gy, _grstd):
    o, weight, rstd = ctx.saved_tensors
    if gy is None:
        return None, None, None, None
    dO, dw = aspin_out_bwd(gy, o, weight, rstd)
    return dO.to(o.dtype), dw.to(weight.dtype), None, None


aspin_out.register_autograd(_out_backward, setup_context=_out_setup)


# ---------------------------------------------------------------------------------------------------------------
# LayerNorm before the carrier's projections and the MLP: replaces nn.LayerNorm(d) (src/assoc.py:323,388;
# src/model.py:555) together with autocast's cast of its fp32 output to bf16 for the matmul after it
LN_MAX_D = 2048


def ln_supported(x: Tensor, mod) -> bool:
    """Whether the LayerNorm kernels take `mod(x)`: fp32 x on the GPU, the last dim a multiple of 4 up to 2048, an
    affine nn.LayerNorm over that dim."""
    D = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.float32 and D % 4 == 0 and D <= LN_MAX_D and x.numel() > 0
            and isinstance(mod, torch.nn.LayerNorm) and tuple(mod.normalized_shape) == (D,)
            and mod.weight is not None and mod.bias is not None
            and mod.weight.dtype == torch.float32 and mod.bias.dtype == torch.float32)


@torch.library.custom_op("pragnosia::layer_norm", mutates_args=())
def layer_norm_op(x: Tensor, weight: Tensor, bias: Tensor, eps: float,
                  out_bf16: bool) -> tuple[Tensor, Tensor, Tensor]:
    """LayerNorm of x (..., D) fp32 over its last dim with fp32 statistics. Returns (y (..., D), bf16 if out_bf16 else
    fp32; mean and rstd (rows,) fp32, kept for the backward)."""
    _require_gpu(x, weight, bias)
    D = x.shape[-1]
    _expect("layer_norm", x.device, weight=(weight, (D,)), bias=(bias, (D,)))
    if x.dtype != torch.float32 or weight.dtype != torch.float32 or bias.dtype != torch.float32:
        raise PragnosiaError("layer_norm: x, weight and bias must be fp32")
    x = x.contiguous()
    rows = x.numel() // D
    y = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16 if out_bf16 else torch.float32)
    mean = torch.empty(rows, device=x.device, dtype=torch.float32)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    check(lib().pragnosia_layer_norm_fwd(_ptr(x), _ptr(weight.contiguous()), _ptr(bias.contiguous()), float(eps),
                                         _ptr(y), int(out_bf16), _ptr(mean), _ptr(rstd), rows, D, _stream(x)),
          "pragnosia_layer_norm_fwd")
    return y, mean, rstd


@layer_norm_op.register_fake
def _(x, weight, bias, eps, out_bf16):
    rows = x.numel() // x.shape[-1]
    return (x.new_empty(x.shape, dtype=torch.bfloat16 if out_bf16 else torch.float32),
            x.new_empty(rows, dtype=torch.float32), x.new_empty(rows, dtype=torch.float32))


@torch.library.custom_op("pragnosia::layer_norm_bwd", mutates_args=())
def layer_norm_bwd(dy: Tensor, x: Tensor, weight: Tensor, mean: Tensor,
                   rstd: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Backward of layer_norm from dy (bf16 or fp32, x's shape). Returns (dx fp32, dweight fp32, dbias fp32)."""
    _require_gpu(dy, x, weight, mean, rstd)
    D = x.shape[-1]
    rows = x.numel() // D
    _expect("layer_norm_bwd", x.device, dy=(dy, tuple(x.shape)), weight=(weight, (D,)), mean=(mean, (rows,)),
            rstd=(rstd, (rows,)))
    if dy.dtype not in (torch.bfloat16, torch.float32):
        dy = dy.float()
    dy, x = dy.contiguous(), x.contiguous()
    P = lib().pragnosia_layer_norm_partials(rows, D)
    if P < 0:
        raise PragnosiaError(f"layer_norm_bwd: shape {tuple(x.shape)} rejected")
    dx = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    dwp = torch.empty(P, D, device=x.device, dtype=torch.float32)
    dbp = torch.empty(P, D, device=x.device, dtype=torch.float32)
    check(lib().pragnosia_layer_norm_bwd(_ptr(dy), int(dy.dtype == torch.bfloat16), _ptr(x), _ptr(weight.contiguous()),
                                         _ptr(mean), _ptr(rstd), _ptr(dx), _ptr(dwp), _ptr(dbp), rows, D, _stream(x)),
          "pragnosia_layer_norm_bwd")
    with torch.autocast("cuda", enabled=False):  # the partial rows summed in fp32
        return dx, colsum(dwp), colsum(dbp)


@layer_norm_bwd.register_fake
def _(dy, x, weight, mean, rstd):
    D = x.shape[-1]
    return (x.new_empty(x.shape, dtype=torch.float32), x.new_empty(D, dtype=torch.float32),
            x.new_empty(D, dtype=torch.float32))


def _ln_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    x, weight, bias, eps, out_bf16 = inputs
    _, mean, rstd = output
    ctx.save_for_backward(x, weight, mean, rstd)
    ctx.mark_non_differentiable(mean, rstd)


def _ln_backward(ctx, dy, _dmean, _drstd):
    if dy is None:
        return None, None, None, None, None
    x, weight, mean, rstd = ctx.saved_tensors
    dx, dw, db = layer_norm_bwd(dy, x, weight, mean, rstd)
    return dx, dw, db, None, None


layer_norm_op.register_autograd(_ln_backward, setup_context=_ln_setup)


def layer_norm(x: Tensor, mod) -> Tensor:
    """`mod(x)` for an nn.LayerNorm `mod` feeding a matmul: on the LayerNorm kernels when they take the shape
    (ln_supported), with the output in bf16 under bf16 autocast (the dtype that matmul computes in, so its own cast
    is skipped) and fp32 otherwise; `mod(x)` itself elsewhere."""
    if not ln_supported(x, mod):
        return mod(x)
    bf16 = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
    return layer_norm_op(x, mod.weight, mod.bias, float(mod.eps), bf16)[0]


# ---------------------------------------------------------------------------------------------------------------
# aspin chunked scan, plain rule: replaces assoc_scan_kernel and its ops, src/assoc_kernel.py:128-323
CHUNK = 64


def _bf16(t: Tensor) -> Tensor:
    return t.to(torch.bfloat16).contiguous()


def _expect_scan(op: str, q: Tensor, k, v, la, beta=None, S0=None, theta=None, widths=(64,)) -> None:
    """q, k, v (B, H, T, D) with D in `widths`; la and beta (B, H, T); S0 (B, H, D, D); theta (H, D / 2); all on q's
    device."""
    if q.dim() == 4 and q.shape[-1] in widths:
        _expect(op, q.device, q=(q, (None, None, None, q.shape[-1])))
    else:
        _expect(op, q.device, q=(q, (None, None, None, widths[0])))
    B, H, T, D = q.shape
    _expect(op, q.device, k=(k, (B, H, T, D)), v=(v, (B, H, T, D)), la=(la, (B, H, T)), beta=(beta, (B, H, T)),
            S0=(S0, (B, H, D, D)), theta=(theta, (H, D // 2)))


@torch.library.custom_op("pragnosia::aspin_chunk", mutates_args=())
def aspin_chunk(q: Tensor, k: Tensor, v: Tensor, la: Tensor, S0: Optional[Tensor],
                want_sent: bool) -> tuple[Tensor, Tensor, Tensor]:
    """Plain-rule chunked scan. q, k, v (B, H, T, 64) (cast to bf16), la (B, H, T) fp32, S0 (B, H, 64, 64) fp32 or
    None. Returns (o bf16, S_final fp32, sent bf16 (B, H, NC, 64, 64), or an empty tensor if not wanted)."""
    _require_gpu(q, k, v, la, S0)
    _expect_scan("aspin_chunk", q, k, v, la, S0=S0)
    q, k, v, la, S0 = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(S0)
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    o = torch.empty(B, H, T, D, device=q.device, dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    sent = (torch.empty(B, H, NC, D, D, device=q.device, dtype=torch.bfloat16) if want_sent
            else q.new_empty(0, dtype=torch.bfloat16))
    P = seg_chunks(B * H, NC, range(1, NC + 1))
    if P < NC:
        _aspin_fwd_seg(q, k, v, la, S0, None, 0, o, S, sent if want_sent else None, P)
        return o, S, sent
    check(lib().pragnosia_aspin_chunk_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(S0), _ptr(o), _ptr(S),
                                          _ptr(sent) if want_sent else None, B, H, T, D, CHUNK, _stream(q)),
          "pragnosia_aspin_chunk_fwd")
    return o, S, sent


COMPUTE_UNITS = 256  # MI355X


SEG_MIN_CHUNKS = 2   # shorter segments cost more in start-up than they save (measured)
# what the segment sums and prefix add, in chunk steps of the kernel they feed: per chunk summed, and fixed
# (measured; the backward's chunk step is about twice the forward's, so its sums weigh less)
SEG_COST = {"fwd": (1.0, 6.0), "bwd": (0.4, 3.0)}


def seg_chunks(heads: int, NC: int, candidates, kind: str = "fwd") -> int:
    """Chunks per segment for the plain forward (or backward) over `heads` (batch x head) sequences of NC chunks.
    Segments are sized so that one round of workgroups covers the compute units (several rounds of shorter segments
    measured slower), at least SEG_MIN_CHUNKS long, and taken only when the walk they save exceeds what the segment
    sums add. Returns the largest candidate not above that size, or NC (one workgroup per head, no segments)."""
    per_chunk, fixed = SEG_COST[kind]
    nseg = max(1, COMPUTE_UNITS // max(heads, 1))
    want = max(SEG_MIN_CHUNKS, -(-NC // nseg))
    fit = [c for c in candidates if c <= want]
    if not fit:
        return NC
    P = max(fit)
    if -(-NC // P) < 2 or NC <= P * (1.0 + per_chunk) + fixed:
        return NC
    return P


def _aspin_fwd_seg(q, k, v, la, S0, theta, window, o, S, sent, P):
    B, H, T, D = q.shape
    nbytes = lib().pragnosia_aspin_chunk_seg_workspace_bytes(B, H, T, D, CHUNK, P)
    if nbytes < 0:
        raise PragnosiaError(f"aspin segmented forward: shape rejected (B={B} H={H} T={T} D={D} segment={P})")
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    check(lib().pragnosia_aspin_chunk_fwd_seg(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(S0), _ptr(theta), window,
                                              _ptr(o), _ptr(S), _ptr(sent), _ptr(ws), nbytes, B, H, T, D, CHUNK, P,
                                              _stream(q)), "pragnosia_aspin_chunk_fwd_seg")


def _aspin_bwd_seg(q, k, v, la, sent, do, dS, dq, dk, dv, dla, dS0, P):
    B, H, T, D = q.shape
    nbytes = lib().pragnosia_aspin_chunk_seg_workspace_bytes(B, H, T, D, CHUNK, P)
    if nbytes < 0:
        raise PragnosiaError(f"aspin segmented backward: shape rejected (B={B} H={H} T={T} D={D} segment={P})")
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    check(lib().pragnosia_aspin_chunk_bwd_seg(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(sent), _ptr(do), _ptr(dS),
                                              _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla), _ptr(dS0), _ptr(ws), nbytes,
                                              B, H, T, D, CHUNK, P, _stream(q)), "pragnosia_aspin_chunk_bwd_seg")


@torch.library.custom_op("pragnosia::aspin_chunk_windows", mutates_args=())
def aspin_chunk_windows(q: Tensor, k: Tensor, v: Tensor, la: Tensor, S0: Optional[Tensor], theta: Tensor,
                        window: int, want_sent: bool) -> tuple[Tensor, Tensor, Tensor]:
    """Forward only. The plain-rule scan over consecutive windows of `window` tokens (a multiple of 64) whose q and k
    were rotated with positions restarting at 0 in every window, the state carried across window boundaries and
    rebased by -window * theta there: what aspin_chunk over each window in turn, with aspin_rebase between, computes
    (the reference's carried windows, `src/model.py:842-864` over `src/assoc.py:391-405`), as one segment-parallel
    pass. S0 enters the first window. Returns (o bf16, S after the last window fp32 (in its positions), sent bf16
    (B, H, NC, 64, 64) or an empty tensor)."""
    _require_gpu(q, k, v, la, S0, theta)
    _expect_scan("aspin_chunk_windows", q, k, v, la, S0=S0, theta=theta)
    if window <= 0 or window % CHUNK:
        raise PragnosiaError(f"aspin_chunk_windows: window {window} must be a positive multiple of {CHUNK}")
    q, k, v, la, S0, theta = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(S0), _f32(theta)
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    o = torch.empty(B, H, T, D, device=q.device, dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    sent = (torch.empty(B, H, NC, D, D, device=q.device, dtype=torch.bfloat16) if want_sent
            else q.new_empty(0, dtype=torch.bfloat16))
    W = window // CHUNK
    divisors = [p for p in range(1, W + 1) if W % p == 0]
    P = seg_chunks(B * H, NC, divisors)
    _aspin_fwd_seg(q, k, v, la, S0, theta, window, o, S, sent if want_sent else None, P if P in divisors else W)
    return o, S, sent


@aspin_chunk_windows.register_fake
def _(q, k, v, la, S0, theta, window, want_sent):
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    sent = q.new_empty(B, H, NC, D, D, dtype=torch.bfloat16) if want_sent else q.new_empty(0, dtype=torch.bfloat16)
    return q.new_empty(B, H, T, D, dtype=torch.bfloat16), q.new_empty(B, H, D, D, dtype=torch.float32), sent


@aspin_chunk.register_fake
def _(q, k, v, la, S0, want_sent):
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    sent = q.new_empty(B, H, NC, D, D, dtype=torch.bfloat16) if want_sent else q.new_empty(0, dtype=torch.bfloat16)
    return q.new_empty(B, H, T, D, dtype=torch.bfloat16), q.new_empty(B, H, D, D, dtype=torch.float32), sent


@torch.library.custom_op("pragnosia::aspin_chunk_bwd", mutates_args=())
def aspin_chunk_bwd(q: Tensor, k: Tensor, v: Tensor, la: Tensor, sent: Tensor, do: Tensor,
                    dS: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of aspin_chunk. Returns (dq, dk, dv bf16, dla fp32, dS0 fp32)."""
    _require_gpu(q, k, v, la, sent, do, dS)
    _expect_scan("aspin_chunk_bwd", q, k, v, la)
    B, H, T, D = q.shape
    _expect("aspin_chunk_bwd", q.device, sent=(sent, (B, H, (T + CHUNK - 1) // CHUNK, D, D)), do=(do, (B, H, T, D)),
            dS=(dS, (B, H, D, D)))
    q, k, v, la, sent, do, dS = _bf16(q), _bf16(k), _bf16(v), _f32(la), _bf16(sent), _bf16(do), _f32(dS)
    dq, dk, dv = (torch.empty(B, H, T, D, device=q.device, dtype=torch.bfloat16) for _ in range(3))
    dla = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    dS0 = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    NC = (T + CHUNK - 1) // CHUNK
    P = seg_chunks(B * H, NC, range(1, NC + 1), "bwd")
    if P < NC:
        _aspin_bwd_seg(q, k, v, la, sent, do, dS, dq, dk, dv, dla, dS0, P)
        return dq, dk, dv, dla, dS0
    check(lib().pragnosia_aspin_chunk_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(sent), _ptr(do), _ptr(dS),
                                          _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla), _ptr(dS0),
                                          B, H, T, D, CHUNK, _stream(q)), "pragnosia_aspin_chunk_bwd")
    return dq, dk, dv, dla, dS0


@aspin_chunk_bwd.register_fake
def _(q, k, v, la, sent, do, dS):
    B, H, T, D = q.shape
    b = lambda *s: q.new_empty(*s, dtype=torch.bfloat16)
    f = lambda *s: q.new_empty(*s, dtype=torch.float32)
    return b(B, H, T, D), b(B, H, T, D), b(B, H, T, D), f(B, H, T), f(B, H, D, D)


def _aspin_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    q, k, v, la, S0, want_sent = inputs
    _, _, sent = output
    if sent.numel() == 0 and any(ctx.needs_input_grad[:5]):
        raise PragnosiaError("aspin_chunk: the backward needs the entering states; call with want_sent=True")
    ctx.has_s0 = S0 is not None
    ctx.save_for_backward(q, k, v, la, sent)
    ctx.mark_non_differentiable(sent)


def _aspin_backward(ctx, do, dS, _dsent):
    q, k, v, la, sent = ctx.saved_tensors
    if do is None:
        do = torch.zeros(q.shape, device=q.device, dtype=torch.bfloat16)
    dq, dk, dv, dla, dS0 = aspin_chunk_bwd(q, k, v, la, sent, do.contiguous(), dS)
    return dq, dk, dv, dla, (dS0 if ctx.has_s0 else None), None


aspin_chunk.register_autograd(_aspin_backward, setup_context=_aspin_setup)


# ---------------------------------------------------------------------------------------------------------------
# the plain rule at head dim 128: assoc_scan_kernel at D = 128 (src/assoc_kernel.py:21,302-323) and its backward
HEAD_DIM_WIDE = 128


def _expect_wide(op: str, q: Tensor, k, v, la) -> None:
    _expect(op, q.device, q=(q, (None, None, None, HEAD_DIM_WIDE)))
    B, H, T, D = q.shape
    _expect(op, q.device, k=(k, (B, H, T, D)), v=(v, (B, H, T, D)), la=(la, (B, H, T)))


def _wide_workspace(op: str, B: int, H: int, T: int, P: int, backward: bool, dev) -> Tensor:
    nbytes = lib().pragnosia_aspin_chunk_wide_workspace_bytes(B, H, T, HEAD_DIM_WIDE, CHUNK, P, int(backward))
    if nbytes < 0:
        raise PragnosiaError(f"{op}: shape rejected (B={B} H={H} T={T} segment={P})")
    return torch.empty(nbytes, device=dev, dtype=torch.uint8)


@torch.library.custom_op("pragnosia::aspin_chunk_wide", mutates_args=())
def aspin_chunk_wide(q: Tensor, k: Tensor, v: Tensor, la: Tensor, S0: Optional[Tensor],
                     want_sent: bool) -> tuple[Tensor, Tensor, Tensor]:
    """Plain-rule chunked scan at head dim 128: one pass per (head, value half) over all 128 keys where each head is
    one segment, else four 64 x 64 scans per head (key half x value half) that read the 128-wide rows in place. q, k, v (B, H, T, 128) (cast to bf16), la (B, H, T) fp32, S0 (B, H, 128, 128) fp32 or
    None. Returns (o bf16 (B, H, T, 128), S_final fp32 (B, H, 128, 128), sent bf16 (B, H, 4, NC, 64, 64): the state
    entering every chunk per scan, scan 2 kh + vh holding block (rows 64 kh.., columns 64 vh..); or an empty tensor
    if not wanted). `wide_sent` turns sent into (B, H, NC, 128, 128)."""
    _require_gpu(q, k, v, la, S0)
    _expect_wide("aspin_chunk_wide", q, k, v, la)
    B, H, T, D = q.shape
    _expect("aspin_chunk_wide", q.device, S0=(S0, (B, H, D, D)))
    q, k, v, la, S0 = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(S0)
    NC = (T + CHUNK - 1) // CHUNK
    o = torch.empty(B, H, T, D, device=q.device, dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    sent = (torch.empty(B, H, 4, NC, CHUNK, CHUNK, device=q.device, dtype=torch.bfloat16) if want_sent
            else q.new_empty(0, dtype=torch.bfloat16))
    P = seg_chunks(4 * B * H, NC, range(1, NC + 1))
    ws = _wide_workspace("aspin_chunk_wide", B, H, T, P, False, q.device)
    check(lib().pragnosia_aspin_chunk_fwd_wide(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(S0), _ptr(o), _ptr(S),
                                               _ptr(sent) if want_sent else None, _ptr(ws), ws.numel(),
                                               B, H, T, D, CHUNK, P, _stream(q)), "pragnosia_aspin_chunk_fwd_wide")
    return o, S, sent


@aspin_chunk_wide.register_fake
def _(q, k, v, la, S0, want_sent):
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    sent = (q.new_empty(B, H, 4, NC, CHUNK, CHUNK, dtype=torch.bfloat16) if want_sent
            else q.new_empty(0, dtype=torch.bfloat16))
    return q.new_empty(B, H, T, D, dtype=torch.bfloat16), q.new_empty(B, H, D, D, dtype=torch.float32), sent


def wide_sent(sent: Tensor) -> Tensor:
    """aspin_chunk_wide's per-scan entering states (B, H, 4, NC, 64, 64) as whole states (B, H, NC, 128, 128)."""
    B, H, _, NC, h, _ = sent.shape
    return sent.view(B, H, 2, 2, NC, h, h).permute(0, 1, 4, 2, 5, 3, 6).reshape(B, H, NC, 2 * h, 2 * h)


@torch.library.custom_op("pragnosia::aspin_chunk_wide_bwd", mutates_args=())
def aspin_chunk_wide_bwd(q: Tensor, k: Tensor, v: Tensor, la: Tensor, sent: Tensor, do: Tensor,
                         dS: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of aspin_chunk_wide. Returns (dq, dk, dv bf16, dla fp32, dS0 fp32)."""
    _require_gpu(q, k, v, la, sent, do, dS)
    _expect_wide("aspin_chunk_wide_bwd", q, k, v, la)
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    _expect("aspin_chunk_wide_bwd", q.device, sent=(sent, (B, H, 4, NC, CHUNK, CHUNK)), do=(do, (B, H, T, D)),
            dS=(dS, (B, H, D, D)))
    q, k, v, la, sent, do, dS = _bf16(q), _bf16(k), _bf16(v), _f32(la), _bf16(sent), _bf16(do), _f32(dS)
    dq, dk, dv = (torch.empty(B, H, T, D, device=q.device, dtype=torch.bfloat16) for _ in range(3))
    dla = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    dS0 = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    P = seg_chunks(4 * B * H, NC, range(1, NC + 1), "bwd")
    ws = _wide_workspace("aspin_chunk_wide_bwd", B, H, T, P, True, q.device)
    check(lib().pragnosia_aspin_chunk_bwd_wide(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(sent), _ptr(do), _ptr(dS),
                                               _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla), _ptr(dS0), _ptr(ws),
                                               ws.numel(), B, H, T, D, CHUNK, P, _stream(q)),
          "pragnosia_aspin_chunk_bwd_wide")
    return dq, dk, dv, dla, dS0


@aspin_chunk_wide_bwd.register_fake
def _(q, k, v, la, sent, do, dS):
    B, H, T, D = q.shape
    b = lambda *s: q.new_empty(*s, dtype=torch.bfloat16)
    f = lambda *s: q.new_empty(*s, dtype=torch.float32)
    return b(B, H, T, D), b(B, H, T, D), b(B, H, T, D), f(B, H, T), f(B, H, D, D)


def _wide_backward(ctx, do, dS, _dsent):
    q, k, v, la, sent = ctx.saved_tensors
    if do is None:
        do = torch.zeros(q.shape, device=q.device, dtype=torch.bfloat16)
    dq, dk, dv, dla, dS0 = aspin_chunk_wide_bwd(q, k, v, la, sent, do.contiguous(), dS)
    return dq, dk, dv, dla, (dS0 if ctx.has_s0 else None), None


aspin_chunk_wide.register_autograd(_wide_backward, setup_context=_aspin_setup)


# ---------------------------------------------------------------------------------------------------------------
# aspin chunked scan, delta rule: replaces delta_scan_kernel and its ops, src/assoc_kernel.py:332-704
@torch.library.custom_op("pragnosia::aspin_delta", mutates_args=())
def aspin_delta(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Tensor, S0: Optional[Tensor],
                want_sent: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Delta-rule chunked scan. q, k, v (B, H, T, D), D = 64 or 128 (cast to bf16), la and beta (B, H, T) fp32, S0
    (B, H, D, D) fp32 or None. Returns (o bf16, S_final fp32, sent bf16 (B, H, NC, D, D) or empty, W bf16 (B, H, T, D),
    X bf16 (B, H, NC, 64, 64)); W and X are the intermediates the backward reads (not differentiable). Each entering
    state in sent is stored transposed (sent[..., c, j, d] = S_c[d, j]); `.transpose(-1, -2)` gives the states.
    D = 128 runs each head as two scans over its value halves (the rule is independent per value column given X),
    sharing X."""
    _require_gpu(q, k, v, la, beta, S0)
    _expect_scan("aspin_delta", q, k, v, la, beta=beta, S0=S0, widths=(64, 128))
    q, k, v, la, beta, S0 = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(beta), _f32(S0)
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    dev = q.device
    o = torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16)
    S = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    sent = (torch.empty(B, H, NC, D, D, device=dev, dtype=torch.bfloat16) if want_sent
            else q.new_empty(0, dtype=torch.bfloat16))
    W = torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16)
    X = torch.empty(B, H, NC, CHUNK, CHUNK, device=dev, dtype=torch.bfloat16)
    check(lib().pragnosia_aspin_delta_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(beta), _ptr(S0), _ptr(o),
                                          _ptr(S), _ptr(sent) if want_sent else None, _ptr(W), _ptr(X),
                                          B, H, T, D, CHUNK, _stream(q)), "pragnosia_aspin_delta_fwd")
    return o, S, sent, W, X


@aspin_delta.register_fake
def _(q, k, v, la, beta, S0, want_sent):
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    b = lambda *s: q.new_empty(*s, dtype=torch.bfloat16)
    sent = b(B, H, NC, D, D) if want_sent else b(0)
    return b(B, H, T, D), q.new_empty(B, H, D, D, dtype=torch.float32), sent, b(B, H, T, D), b(B, H, NC, CHUNK, CHUNK)


@torch.library.custom_op("pragnosia::aspin_delta_bwd", mutates_args=())
def aspin_delta_bwd(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Tensor, sent: Tensor, W: Tensor, X: Tensor,
                    do: Tensor, dS: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of aspin_delta. Returns (dq, dk, dv bf16, dla fp32, dbeta fp32, dS0 fp32)."""
    _require_gpu(q, k, v, la, beta, sent, W, X, do, dS)
    _expect_scan("aspin_delta_bwd", q, k, v, la, beta=beta, widths=(64, 128))
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    _expect("aspin_delta_bwd", q.device, sent=(sent, (B, H, NC, D, D)), W=(W, (B, H, T, D)),
            X=(X, (B, H, NC, CHUNK, CHUNK)), do=(do, (B, H, T, D)), dS=(dS, (B, H, D, D)))
    q, k, v, la, beta = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(beta)
    sent, W, X, do, dS = _bf16(sent), _bf16(W), _bf16(X), _bf16(do), _f32(dS)
    B, H, T, D = q.shape
    dev = q.device
    dq, dk, dv = (torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16) for _ in range(3))
    dla = torch.empty(B, H, T, device=dev, dtype=torch.float32)
    dbeta = torch.empty(B, H, T, device=dev, dtype=torch.float32)
    dS0 = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    nbytes = lib().pragnosia_aspin_delta_bwd_workspace_bytes(B, H, T, D, CHUNK)
    if nbytes < 0:
        raise PragnosiaError(f"aspin_delta_bwd: shape {tuple(q.shape)} rejected")
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    check(lib().pragnosia_aspin_delta_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(beta), _ptr(sent), _ptr(W),
                                          _ptr(X), _ptr(do), _ptr(dS), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla),
                                          _ptr(dbeta), _ptr(dS0), _ptr(ws), nbytes, B, H, T, D, CHUNK, _stream(q)),
          "pragnosia_aspin_delta_bwd")
    return dq, dk, dv, dla, dbeta, dS0


@aspin_delta_bwd.register_fake
def _(q, k, v, la, beta, sent, W, X, do, dS):
    B, H, T, D = q.shape
    b = lambda *s: q.new_empty(*s, dtype=torch.bfloat16)
    f = lambda *s: q.new_empty(*s, dtype=torch.float32)
    return b(B, H, T, D), b(B, H, T, D), b(B, H, T, D), f(B, H, T), f(B, H, T), f(B, H, D, D)


def _delta_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    q, k, v, la, beta, S0, want_sent = inputs
    _, _, sent, W, X = output
    if sent.numel() == 0 and any(ctx.needs_input_grad[:6]):
        raise PragnosiaError("aspin_delta: the backward needs the entering states; call with want_sent=True")
    ctx.has_s0 = S0 is not None
    ctx.save_for_backward(q, k, v, la, beta, sent, W, X)
    ctx.mark_non_differentiable(sent, W, X)


def _delta_backward(ctx, do, dS, _dsent, _dW, _dX):
    q, k, v, la, beta, sent, W, X = ctx.saved_tensors
    if do is None:
        do = torch.zeros(q.shape, device=q.device, dtype=torch.bfloat16)
    dq, dk, dv, dla, dbeta, dS0 = aspin_delta_bwd(q, k, v, la, beta, sent, W, X, do.contiguous(), dS)
    return dq, dk, dv, dla, dbeta, (dS0 if ctx.has_s0 else None), None


aspin_delta.register_autograd(_delta_backward, setup_context=_delta_setup)


def _delta_pass(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Tensor, S0: Optional[Tensor], want_o: bool,
                want_saved: bool) -> tuple[Optional[Tensor], Tensor, Optional[Tensor], Optional[Tensor],
                                            Optional[Tensor]]:
    """One 64-wide delta forward through the C ABI writing only what is asked for: o when want_o; the entering
    states, W and X when want_saved (the state pass of a recomputing backward, want_o False, skips the output
    products). Returns (o, S_final, sent, W, X), None for what was not written. Inputs already cast."""
    B, H, T, D = q.shape
    NC = (T + CHUNK - 1) // CHUNK
    dev = q.device
    o = torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16) if want_o else None
    S = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    sent = W = X = None
    if want_saved:
        sent = torch.empty(B, H, NC, D, D, device=dev, dtype=torch.bfloat16)
        W = torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16)
        X = torch.empty(B, H, NC, CHUNK, CHUNK, device=dev, dtype=torch.bfloat16)
    check(lib().pragnosia_aspin_delta_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(beta), _ptr(S0), _ptr(o),
                                          _ptr(S), _ptr(sent), _ptr(W), _ptr(X), B, H, T, D, CHUNK, _stream(q)),
          "pragnosia_aspin_delta_fwd")
    return o, S, sent, W, X


@torch.library.custom_op("pragnosia::aspin_delta_fused", mutates_args=())
def aspin_delta_fused(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Tensor,
                      S0: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """The delta-rule scan keeping nothing for its backward but its inputs: (o bf16, S_final fp32). At head dim 64
    the forward is one kernel that forms each chunk's inverse X on chip and writes only o and S_final: X, W and the
    per-chunk entering states never reach memory. Its backward first runs the state pass of the same kernel (no
    output products), which writes the entering states, W and X (the same operations on the same inputs, so
    bit-identical to what the forward formed), then the stored-state backward. At head dim 128, X, W and o come from
    the two-kernel forward into temporaries freed on return. This is the trait of the third-party fused kernel the
    reference's FUSED_SCAN switches to (`src/assoc.py:481-492`: state on chip, chunk states recomputed in the backward
    instead of written per chunk and read back): the activation memory kept from forward to backward drops by 2 B/elem
    of W, 2 B per entering-state element and 2 B per X element, for one more forward pass in the backward."""
    _require_gpu(q, k, v, la, beta, S0)
    _expect_scan("aspin_delta_fused", q, k, v, la, beta=beta, S0=S0, widths=(64, 128))
    if q.shape[-1] == 128:
        o, S, _, _, _ = aspin_delta(q, k, v, la, beta, S0, False)
        return o, S
    q, k, v, la, beta, S0 = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(beta), _f32(S0)
    o, S, _, _, _ = _delta_pass(q, k, v, la, beta, S0, True, False)
    return o, S


@torch.library.custom_op("pragnosia::aspin_delta_windows", mutates_args=())
def aspin_delta_windows(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Tensor, S0: Optional[Tensor],
                        theta: Tensor, window: int) -> tuple[Tensor, Tensor]:
    """Forward only. The delta-rule scan over consecutive windows of `window` tokens (a multiple of 64) whose q and k
    were rotated with positions restarting at 0 in every window, the state carried across window boundaries and
    rebased by -window * theta there: what aspin_delta over each window in turn, with aspin_rebase between, computes
    (the reference's carried windows, `src/model.py:842-864` over `src/assoc.py:391-405`), with every window at once.
    Given X the rule is linear in the state and independent per value column, so each window maps its entering state
    affinely, S_out = M S_in + R: the state passes over all windows (R from zero entering states; M from identity
    states with zero values) in one launch (`pragnosia_aspin_delta_window_maps`), the entering states chained by
    `pragnosia_aspin_delta_window_prefix`, then one pass with outputs from the true entering states. A partial last window runs zero-padded (zero keys, values, decay and
    strength leave the state unchanged). Head dim 64. S0 enters the first window. Returns (o bf16, S after the last
    window fp32, in its positions)."""
    _require_gpu(q, k, v, la, beta, S0, theta)
    _expect_scan("aspin_delta_windows", q, k, v, la, beta=beta, S0=S0, theta=theta)
    if window <= 0 or window % CHUNK:
        raise PragnosiaError(f"aspin_delta_windows: window {window} must be a positive multiple of {CHUNK}")
    if q.shape[-1] != 64:
        raise PragnosiaError(f"aspin_delta_windows: head dim {q.shape[-1]}; the window maps are built for 64")
    q, k, v, la, beta, S0, theta = _bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(beta), _f32(S0), _f32(theta)
    B, H, T, D = q.shape
    NW = (T + window - 1) // window
    Tp = NW * window
    if Tp != T:
        pad = lambda t: F.pad(t, (0, 0, 0, Tp - T)) if t.dim() == 4 else F.pad(t, (0, Tp - T))
        q, k, v, la, beta = (pad(t) for t in (q, k, v, la, beta))
    BW = B * H * NW  # every window of every (batch, head) a sequence of its own: contiguous views
    qw, kw, vw = (t.view(BW, 1, window, D) for t in (q, k, v))
    lw, bw = la.view(BW, 1, window), beta.view(BW, 1, window)
    RM = torch.empty(2, BW, D, D, device=q.device, dtype=torch.float32)  # R, then M: both state passes, one launch
    check(lib().pragnosia_aspin_delta_window_maps(_ptr(qw), _ptr(kw), _ptr(vw), _ptr(lw), _ptr(bw), _ptr(RM), BW, window,
                                                  _stream(q)), "pragnosia_aspin_delta_window_maps")
    Sin = torch.empty(BW, 1, D, D, device=q.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_delta_window_prefix(_ptr(RM[1]), _ptr(RM[0]), _ptr(S0), _ptr(theta), float(window),
                                                    _ptr(Sin), B * H, H, NW, _stream(q)),
          "pragnosia_aspin_delta_window_prefix")
    o, Sf, _, _, _ = _delta_pass(qw, kw, vw, lw, bw, Sin, True, False)
    o = o.view(B, H, Tp, D)[:, :, :T]
    return (o if Tp == T else o.contiguous()), Sf.view(B, H, NW, D, D)[:, :, -1].contiguous()


@aspin_delta_windows.register_fake
def _(q, k, v, la, beta, S0, theta, window):
    B, H, T, D = q.shape
    return q.new_empty(B, H, T, D, dtype=torch.bfloat16), q.new_empty(B, H, D, D, dtype=torch.float32)


@aspin_delta_fused.register_fake
def _(q, k, v, la, beta, S0):
    B, H, T, D = q.shape
    return q.new_empty(B, H, T, D, dtype=torch.bfloat16), q.new_empty(B, H, D, D, dtype=torch.float32)


def _delta_fused_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    q, k, v, la, beta, S0 = inputs
    ctx.has_s0 = S0 is not None
    ctx.save_for_backward(q, k, v, la, beta, S0)


def _delta_fused_backward(ctx, do, dS):
    q, k, v, la, beta, S0 = ctx.saved_tensors
    if q.shape[-1] == 128:
        _, _, sent, W, X = aspin_delta(q, k, v, la, beta, S0, True)  # the forward's intermediates, recomputed
    else:  # the state pass: entering states, W and X, no output
        _, _, sent, W, X = _delta_pass(_bf16(q), _bf16(k), _bf16(v), _f32(la), _f32(beta), _f32(S0), False, True)
    if do is None:
        do = torch.zeros(q.shape, device=q.device, dtype=torch.bfloat16)
    dq, dk, dv, dla, dbeta, dS0 = aspin_delta_bwd(q, k, v, la, beta, sent, W, X, do.contiguous(), dS)
    return dq, dk, dv, dla, dbeta, (dS0 if ctx.has_s0 else None)


aspin_delta_fused.register_autograd(_delta_fused_backward, setup_context=_delta_fused_setup)


# ---------------------------------------------------------------------------------------------------------------
# the scan with fp32 / fp64 operands (no bf16 rounding): replaces assoc_scan's fp32/fp64 torch forms and their
# autograd backward, src/assoc.py:118-165, :207-269
EXACT_CKPT = 8  # tokens per checkpointed state (PRAGNOSIA_EXACT_CKPT_TOKENS)
EXACT_MAX_DK = 384  # key rows (kMaxDk)
EXACT_MAX_DV = 128  # value columns (kMaxDv)
EXACT_MAX_LDS = 160 * 1024


def exact_rows_per_lane(Dk: int) -> int:
    """Key rows each lane holds in the exact scan (rows_per_lane): the smallest of 2 .. 96 with 4 R >= Dk."""
    for r in (2, 4, 8, 16, 32, 48, 96):
        if 4 * r >= Dk:
            return r
    raise PragnosiaError(f"exact scan: Dk={Dk} exceeds {EXACT_MAX_DK}")


def exact_value_cap(Dk: int, dtype: torch.dtype, backward: bool) -> int:
    """The most value columns one exact-scan launch takes at key width Dk: a multiple of 16 (one wave each) whose
    LDS (fwd_lds / bwd_lds of the kernel) fits 160 KiB."""
    R, es = exact_rows_per_lane(Dk), (8 if dtype == torch.float64 else 4)
    for nw in range(EXACT_MAX_DV // 16, 0, -1):
        if backward:
            n = 2 * EXACT_CKPT * 4 * R + 3 * EXACT_CKPT * 16 * nw + 2 * EXACT_CKPT + 2 * nw * EXACT_CKPT * 4 * R \
                + 2 * nw * EXACT_CKPT
        else:
            n = 2 * EXACT_CKPT * 4 * R + EXACT_CKPT * 16 * nw + 2 * EXACT_CKPT
        if n * es <= EXACT_MAX_LDS:
            return 16 * nw
    raise PragnosiaError(f"exact scan: no value block fits the LDS at Dk={Dk}")


def _exact_dtype(t: Tensor) -> torch.dtype:
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def _dtype_code(dt: torch.dtype) -> int:
    return 1 if dt == torch.float64 else 0


def _expect_exact(op: str, q: Tensor, k, v, la, beta=None, S0=None) -> None:
    """q, k (B, H, T, Dk); v (B, H, T, Dv); la, beta (B, H, T); S0 (B, H, Dk, Dv); Dk <= 384, Dv <= 128."""
    if q.dim() != 4 or v is None or v.dim() != 4:
        raise PragnosiaError(f"{op}: q and v must be (B, H, T, D)")
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    if not (0 < Dk <= EXACT_MAX_DK and 0 < Dv <= EXACT_MAX_DV):
        raise PragnosiaError(f"{op}: head dims Dk={Dk}, Dv={Dv} must be in 1..{EXACT_MAX_DK} x 1..{EXACT_MAX_DV}")
    _expect(op, q.device, k=(k, (B, H, T, Dk)), v=(v, (B, H, T, Dv)), la=(la, (B, H, T)), beta=(beta, (B, H, T)),
            S0=(S0, (B, H, Dk, Dv)))


@torch.library.custom_op("pragnosia::aspin_exact", mutates_args=())
def aspin_exact(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Optional[Tensor], S0: Optional[Tensor],
                want_ckpt: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The scan with fp32 operands (fp64 when q is fp64), plain rule, or the delta rule when beta is given.
    q, k (B, H, T, Dk), v (B, H, T, Dv), la and beta (B, H, T), S0 (B, H, Dk, Dv) or None; Dk <= 384, Dv <= 128
    (wide keys take fewer value columns: exact_value_cap; the library refuses what does not fit its LDS). Returns
    (o (B, H, T, Dv), S_final (B, H, Dk, Dv), ckpt, resid) in the compute dtype; ckpt (the state entering every 8
    tokens) and resid (the delta rule's residuals) are what the backward reads, empty unless want_ckpt."""
    _require_gpu(q, k, v, la, beta, S0)
    _expect_exact("aspin_exact", q, k, v, la, beta, S0)
    dt = _exact_dtype(q)
    cv = lambda t: None if t is None else t.to(dt).contiguous()
    q, k, v, la, beta, S0 = cv(q), cv(k), cv(v), cv(la), cv(beta), cv(S0)
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    dev = q.device
    o = torch.empty(B, H, T, Dv, device=dev, dtype=dt)
    S = torch.empty(B, H, Dk, Dv, device=dev, dtype=dt)
    NB = (T + EXACT_CKPT - 1) // EXACT_CKPT
    ckpt = torch.empty(B, H, NB, Dk, Dv, device=dev, dtype=dt) if want_ckpt else q.new_empty(0)
    resid = (torch.empty(B, H, T, Dv, device=dev, dtype=dt) if (want_ckpt and beta is not None)
             else q.new_empty(0))
    check(lib().pragnosia_aspin_exact_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(beta), _ptr(S0), _ptr(o), _ptr(S),
                                          _ptr(ckpt) if want_ckpt else None,
                                          _ptr(resid) if resid.numel() else None, B, H, T, Dk, Dv, _dtype_code(dt),
                                          _stream(q)), "pragnosia_aspin_exact_fwd")
    return o, S, ckpt, resid


@aspin_exact.register_fake
def _(q, k, v, la, beta, S0, want_ckpt):
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    dt = _exact_dtype(q)
    NB = (T + EXACT_CKPT - 1) // EXACT_CKPT
    ckpt = q.new_empty(B, H, NB, Dk, Dv, dtype=dt) if want_ckpt else q.new_empty(0, dtype=dt)
    resid = q.new_empty(B, H, T, Dv, dtype=dt) if (want_ckpt and beta is not None) else q.new_empty(0, dtype=dt)
    return q.new_empty(B, H, T, Dv, dtype=dt), q.new_empty(B, H, Dk, Dv, dtype=dt), ckpt, resid


@torch.library.custom_op("pragnosia::aspin_exact_bwd", mutates_args=())
def aspin_exact_bwd(q: Tensor, k: Tensor, v: Tensor, la: Tensor, beta: Optional[Tensor], ckpt: Tensor,
                    resid: Optional[Tensor], do: Tensor,
                    dS: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of aspin_exact. Returns (dq, dk, dv, dla, dbeta (empty for the plain rule), dS0) in the compute
    dtype."""
    _require_gpu(q, k, v, la, beta, ckpt, resid, do, dS)
    _expect_exact("aspin_exact_bwd", q, k, v, la, beta)
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    NB = (T + EXACT_CKPT - 1) // EXACT_CKPT
    _expect("aspin_exact_bwd", q.device, ckpt=(ckpt, (B, H, NB, Dk, Dv)), do=(do, (B, H, T, Dv)),
            dS=(dS, (B, H, Dk, Dv)), resid=(resid if beta is not None else None, (B, H, T, Dv)))
    dt = _exact_dtype(q)
    cv = lambda t: None if t is None else t.to(dt).contiguous()
    q, k, v, la, beta, ckpt, do, dS = cv(q), cv(k), cv(v), cv(la), cv(beta), cv(ckpt), cv(do), cv(dS)
    resid = cv(resid) if beta is not None else None
    dev = q.device
    dq, dk = torch.empty(B, H, T, Dk, device=dev, dtype=dt), torch.empty(B, H, T, Dk, device=dev, dtype=dt)
    dv = torch.empty(B, H, T, Dv, device=dev, dtype=dt)
    dla = torch.empty(B, H, T, device=dev, dtype=dt)
    dbeta = torch.empty(B, H, T, device=dev, dtype=dt) if beta is not None else q.new_empty(0)
    dS0 = torch.empty(B, H, Dk, Dv, device=dev, dtype=dt)
    check(lib().pragnosia_aspin_exact_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(la), _ptr(beta), _ptr(ckpt), _ptr(resid),
                                          _ptr(do), _ptr(dS), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla),
                                          _ptr(dbeta) if beta is not None else None, _ptr(dS0), B, H, T, Dk, Dv,
                                          _dtype_code(dt), _stream(q)), "pragnosia_aspin_exact_bwd")
    return dq, dk, dv, dla, dbeta, dS0


@aspin_exact_bwd.register_fake
def _(q, k, v, la, beta, ckpt, resid, do, dS):
    B, H, T, Dk = q.shape
    Dv = v.shape[-1]
    dt = _exact_dtype(q)
    e = lambda *s: q.new_empty(*s, dtype=dt)
    return e(B, H, T, Dk), e(B, H, T, Dk), e(B, H, T, Dv), e(B, H, T), e(B, H, T) if beta is not None else e(0), \
        e(B, H, Dk, Dv)


def _exact_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    q, k, v, la, beta, S0, want_ckpt = inputs
    _, _, ckpt, resid = output
    if ckpt.numel() == 0 and any(ctx.needs_input_grad[:6]):
        raise PragnosiaError("aspin_exact: the backward needs the checkpoints; call with want_ckpt=True")
    ctx.has_s0, ctx.has_beta = S0 is not None, beta is not None
    ctx.dtypes = tuple(None if t is None else t.dtype for t in (q, k, v, la, beta, S0))
    ctx.save_for_backward(q, k, v, la, beta, ckpt, resid)
    ctx.mark_non_differentiable(ckpt, resid)


def _exact_backward(ctx, do, dS, _dckpt, _dresid):
    q, k, v, la, beta, ckpt, resid = ctx.saved_tensors
    if do is None:
        do = torch.zeros(*q.shape[:3], v.shape[-1], device=q.device, dtype=_exact_dtype(q))
    dq, dk, dv, dla, dbeta, dS0 = aspin_exact_bwd(q, k, v, la, beta, ckpt, resid if ctx.has_beta else None,
                                                  do.contiguous(), dS)
    dt = ctx.dtypes
    return (dq.to(dt[0]), dk.to(dt[1]), dv.to(dt[2]), dla.to(dt[3]), dbeta.to(dt[4]) if ctx.has_beta else None,
            dS0.to(dt[5]) if ctx.has_s0 else None, None)


aspin_exact.register_autograd(_exact_backward, setup_context=_exact_setup)


# ---------------------------------------------------------------------------------------------------------------
# prep (normalise, gate, rotate, cast, transpose): replaces prep_kernel and its ops, src/assoc_kernel.py:740-891
def _proj(t: Tensor) -> Tensor:
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return t.contiguous()


def _expect_prep(op: str, qp: Tensor, kp, vp, gate, theta, pos) -> None:
    """qp, kp, vp (B, T, H, D), D = 64 or 128; gate (B, T, H); theta (H, D / 2); pos (T,); all on qp's device."""
    Dw = qp.shape[-1] if qp.dim() == 4 and qp.shape[-1] in (64, 128) else 64
    _expect(op, qp.device, qp=(qp, (None, None, None, Dw)))
    B, T, H, D = qp.shape
    _expect(op, qp.device, kp=(kp, (B, T, H, D)), vp=(vp, (B, T, H, D)), gate=(gate, (B, T, H)),
            theta=(theta, (H, D // 2)), pos=(pos, (T,)))


@torch.library.custom_op("pragnosia::aspin_prep", mutates_args=())
def aspin_prep(qp: Tensor, kp: Tensor, vp: Tensor, gate: Optional[Tensor], theta: Tensor,
               pos: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """qp, kp, vp (B, T, H, D) fp32 or bf16 projections, D = 64 or 128; gate (B, T, H) logits or None; theta
    (H, D / 2); pos (T,) int64. Returns bf16 q, k, v in (B, H, T, D)."""
    _require_gpu(qp, kp, vp, gate, theta, pos)
    _expect_prep("aspin_prep", qp, kp, vp, gate, theta, pos)
    qp, kp, vp = _proj(qp), _proj(kp).to(qp.dtype), _proj(vp).to(qp.dtype)
    gate, theta, pos = _f32(gate), _f32(theta), pos.to(torch.int64).contiguous()
    B, T, H, D = qp.shape
    q, k, v = (torch.empty(B, H, T, D, device=qp.device, dtype=torch.bfloat16) for _ in range(3))
    check(lib().pragnosia_aspin_prep_fwd(_ptr(qp), _ptr(kp), _ptr(vp), _ptr(gate), _ptr(theta), _ptr(pos), _ptr(q),
                                         _ptr(k), _ptr(v), B, T, H, D, H * D, int(qp.dtype == torch.bfloat16),
                                         _stream(qp)), "pragnosia_aspin_prep_fwd")
    return q, k, v


@aspin_prep.register_fake
def _(qp, kp, vp, gate, theta, pos):
    B, T, H, D = qp.shape
    return tuple(qp.new_empty(B, H, T, D, dtype=torch.bfloat16) for _ in range(3))


@torch.library.custom_op("pragnosia::aspin_prep_bwd", mutates_args=())
def aspin_prep_bwd(qp: Tensor, kp: Tensor, vp: Tensor, gate: Optional[Tensor], theta: Tensor, pos: Tensor,
                   dq: Tensor, dk: Tensor, dv: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Returns (dqp, dkp, dvp in the projections' dtype, dgate fp32 (B, T, H) or empty, dtheta fp32 (H, D / 2))."""
    _require_gpu(qp, kp, vp, gate, theta, pos, dq, dk, dv)
    _expect_prep("aspin_prep_bwd", qp, kp, vp, gate, theta, pos)
    B, T, H, D = qp.shape
    _expect("aspin_prep_bwd", qp.device, dq=(dq, (B, H, T, D)), dk=(dk, (B, H, T, D)), dv=(dv, (B, H, T, D)))
    qp, kp, vp = _proj(qp), _proj(kp).to(qp.dtype), _proj(vp).to(qp.dtype)
    gate, theta, pos = _f32(gate), _f32(theta), pos.to(torch.int64).contiguous()
    dq, dk, dv = _bf16(dq), _bf16(dk), _bf16(dv)
    B, T, H, D = qp.shape
    dqp, dkp, dvp = torch.empty_like(qp), torch.empty_like(qp), torch.empty_like(qp)
    dgate = torch.empty(B, T, H, device=qp.device) if gate is not None else qp.new_empty(0, dtype=torch.float32)
    rows = lib().pragnosia_aspin_prep_theta_partials(B, T)
    dth = torch.empty(rows, H, D // 2, device=qp.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_prep_bwd(_ptr(qp), _ptr(kp), _ptr(vp), _ptr(gate), _ptr(theta), _ptr(pos), _ptr(dq),
                                         _ptr(dk), _ptr(dv), _ptr(dqp), _ptr(dkp), _ptr(dvp),
                                         _ptr(dgate) if gate is not None else None, _ptr(dth), B, T, H, D, H * D,
                                         int(qp.dtype == torch.bfloat16), _stream(qp)), "pragnosia_aspin_prep_bwd")
    return dqp, dkp, dvp, dgate, colsum(dth)


@aspin_prep_bwd.register_fake
def _(qp, kp, vp, gate, theta, pos, dq, dk, dv):
    B, T, H, D = qp.shape
    dg = qp.new_empty(B, T, H, dtype=torch.float32) if gate is not None else qp.new_empty(0, dtype=torch.float32)
    return (torch.empty_like(qp), torch.empty_like(qp), torch.empty_like(qp), dg,
            qp.new_empty(H, D // 2, dtype=torch.float32))


def _prep_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    qp, kp, vp, gate, theta, pos = inputs
    ctx.has_gate = gate is not None
    ctx.dtypes = (qp.dtype, kp.dtype, vp.dtype, None if gate is None else gate.dtype, theta.dtype)
    ctx.save_for_backward(qp, kp, vp, gate, theta, pos)


def _prep_backward(ctx, dq, dk, dv):
    qp, kp, vp, gate, theta, pos = ctx.saved_tensors
    z = lambda t, ref: torch.zeros(ref.shape[0], ref.shape[2], ref.shape[1], ref.shape[3], device=ref.device,
                                   dtype=torch.bfloat16) if t is None else t
    dq, dk, dv = z(dq, qp), z(dk, qp), z(dv, qp)
    dqp, dkp, dvp, dgate, dth = aspin_prep_bwd(qp, kp, vp, gate, theta, pos, dq, dk, dv)
    dt = ctx.dtypes
    return (dqp.to(dt[0]), dkp.to(dt[1]), dvp.to(dt[2]), (dgate.to(dt[3]) if ctx.has_gate else None),
            dth.to(dt[4]), None)


aspin_prep.register_autograd(_prep_backward, setup_context=_prep_setup)


def _proj_cols(H: int, gated: bool, has_beta: bool, D: int = 64) -> tuple[int, int, int]:
    """Column offsets (decay, gate, strength; -1 = absent) in the projection GEMM's output rows."""
    base = 3 * H * D
    return base, (base + H if gated else -1), (base + H if has_beta else -1)


def _expect_proj(op: str, P: Tensor, H: int, gated: bool, la_bias, A, la_floor, gate_bias, beta_bias, theta,
                 pos=None, D: int = 64) -> None:
    """P (B, T, W) (or (B, W) for the decode step) with W at least the columns the kernels read; the per-head
    vectors (H,); theta (H, D / 2); pos (T,); all on P's device. D = 64 or 128."""
    if D not in (64, 128):
        raise PragnosiaError(f"{op}: head dim {D} (the prep kernels take 64 and 128)")
    if H <= 0 or P.dim() not in (2, 3) or P.shape[-1] < 3 * H * D + (2 if gated else 1) * H:
        raise PragnosiaError(f"{op}: P has shape {tuple(P.shape)}, expected (B, [T,] >= {3 * H * D + H}) columns "
                             f"for {H} heads of {D}")
    _expect(op, P.device, la_bias=(la_bias, (H,)), A=(A, (H,)), la_floor=(la_floor, (H,)),
            gate_bias=(gate_bias, (H,)), beta_bias=(beta_bias, (H,)), theta=(theta, (H, D // 2)))
    if pos is not None:
        _expect(op, P.device, pos=(pos, (P.shape[1] if P.dim() == 3 else None,)))


@torch.library.custom_op("pragnosia::aspin_prep_proj", mutates_args=())
def aspin_prep_proj(P: Tensor, H: int, la_bias: Tensor, A: Tensor, la_floor: Optional[Tensor],
                    gate_bias: Optional[Tensor], beta_bias: Optional[Tensor], beta_min: float, gated: bool,
                    theta: Tensor, pos: Tensor, D: int = 64) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The carrier's inputs to the scan from ONE GEMM's output P (B, T, 3 H D + 2 H) (fp32 or bf16), head dim D = 64
    or 128: the q, k, v projections in the first 3 H D columns, then the decay logits, then either the plain rule's
    write-gate logits (gated) or the delta rule's write-strength logits (beta_bias given, or beta_min > 0), all before
    their biases. Returns bf16 q, k, v (B, H, T, D) (normalised, k gated, q and k rotated by pos * theta), la (B, H,
    T) fp32 = -softplus(logit + la_bias) exp(A) (floored at la_floor when given) and beta (B, H, T) fp32 =
    max(sigmoid(logit + beta_bias), beta_min) for the delta rule (else an empty tensor)."""
    _require_gpu(P, la_bias, A, la_floor, gate_bias, beta_bias, theta, pos)
    _expect_proj("aspin_prep_proj", P, H, gated, la_bias, A, la_floor, gate_bias, beta_bias, theta, pos, D)
    if P.dim() != 3:
        raise PragnosiaError(f"aspin_prep_proj: P must be (B, T, W), got {tuple(P.shape)}")
    P = _proj(P)
    la_bias, A, la_floor, theta = _f32(la_bias), _f32(A), _f32(la_floor), _f32(theta)
    gate_bias, beta_bias = _f32(gate_bias), _f32(beta_bias)
    pos = pos.to(torch.int64).contiguous()
    B, T, W = P.shape
    has_beta = not gated and W > 3 * H * D + H
    q, k, v = (torch.empty(B, H, T, D, device=P.device, dtype=torch.bfloat16) for _ in range(3))
    la = torch.empty(B, H, T, device=P.device, dtype=torch.float32)
    beta = (torch.empty(B, H, T, device=P.device, dtype=torch.float32) if has_beta
            else P.new_empty(0, dtype=torch.float32))
    acol, gcol, bcol = _proj_cols(H, gated, has_beta, D)
    check(lib().pragnosia_aspin_prep_proj_fwd(_ptr(P), W, acol, gcol, bcol, _ptr(la_bias), _ptr(A), _ptr(la_floor),
                                              _ptr(gate_bias), _ptr(beta_bias), float(beta_min), _ptr(theta),
                                              _ptr(pos), _ptr(q), _ptr(k), _ptr(v), _ptr(la),
                                              _ptr(beta) if has_beta else None, B, T, H, D,
                                              int(P.dtype == torch.bfloat16), _stream(P)),
          "pragnosia_aspin_prep_proj_fwd")
    return q, k, v, la, beta


@aspin_prep_proj.register_fake
def _(P, H, la_bias, A, la_floor, gate_bias, beta_bias, beta_min, gated, theta, pos, D=64):
    B, T, W = P.shape
    b = lambda: P.new_empty(B, H, T, D, dtype=torch.bfloat16)
    has_beta = not gated and W > 3 * H * D + H
    beta = P.new_empty(B, H, T, dtype=torch.float32) if has_beta else P.new_empty(0, dtype=torch.float32)
    return b(), b(), b(), P.new_empty(B, H, T, dtype=torch.float32), beta


@torch.library.custom_op("pragnosia::aspin_prep_proj_bwd", mutates_args=())
def aspin_prep_proj_bwd(P: Tensor, H: int, la_bias: Tensor, A: Tensor, la_floor: Optional[Tensor],
                        gate_bias: Optional[Tensor], beta_bias: Optional[Tensor], beta_min: float, gated: bool,
                        theta: Tensor, pos: Tensor, dq: Tensor, dk: Tensor, dv: Tensor, dla: Tensor,
                        dbeta: Optional[Tensor], D: int = 64) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of aspin_prep_proj. Returns (dP in P's dtype and layout, d la_bias, dA, d gate_bias or d beta_bias
    (the one in use; empty when neither), dtheta), the per-head sums reduced from the kernel's partials."""
    _require_gpu(P, dq, dk, dv, dla, dbeta)
    _expect_proj("aspin_prep_proj_bwd", P, H, gated, la_bias, A, la_floor, gate_bias, beta_bias, theta, pos, D)
    if P.dim() != 3:
        raise PragnosiaError(f"aspin_prep_proj_bwd: P must be (B, T, W), got {tuple(P.shape)}")
    _expect("aspin_prep_proj_bwd", P.device, dq=(dq, (P.shape[0], H, P.shape[1], D)),
            dk=(dk, (P.shape[0], H, P.shape[1], D)), dv=(dv, (P.shape[0], H, P.shape[1], D)),
            dla=(dla, (P.shape[0], H, P.shape[1])), dbeta=(dbeta, (P.shape[0], H, P.shape[1])))
    P = _proj(P)
    la_bias, A, la_floor, theta = _f32(la_bias), _f32(A), _f32(la_floor), _f32(theta)
    gate_bias, beta_bias = _f32(gate_bias), _f32(beta_bias)
    pos = pos.to(torch.int64).contiguous()
    dq, dk, dv, dla = _bf16(dq), _bf16(dk), _bf16(dv), _f32(dla)
    B, T, W = P.shape
    has_beta = not gated and W > 3 * H * D + H
    if has_beta:
        dbeta = torch.zeros(B, H, T, device=P.device) if dbeta is None else _f32(dbeta)
    dP = torch.empty_like(P)
    if W > 3 * H * D + (2 if (gated or has_beta) else 1) * H:
        dP.zero_()  # columns the kernel does not write
    rows = lib().pragnosia_aspin_prep_theta_partials(B, T)
    dth = torch.empty(rows, H, D // 2, device=P.device, dtype=torch.float32)
    part = torch.empty(lib().pragnosia_aspin_prep_proj_partials(B, T, H), 3, device=P.device, dtype=torch.float32)
    acol, gcol, bcol = _proj_cols(H, gated, has_beta, D)
    check(lib().pragnosia_aspin_prep_proj_bwd(_ptr(P), W, acol, gcol, bcol, _ptr(la_bias), _ptr(A), _ptr(la_floor),
                                              _ptr(gate_bias), _ptr(beta_bias), float(beta_min), _ptr(theta),
                                              _ptr(pos), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dla),
                                              _ptr(dbeta) if has_beta else None, _ptr(dP), _ptr(dth), _ptr(part),
                                              B, T, H, D, int(P.dtype == torch.bfloat16), _stream(P)),
          "pragnosia_aspin_prep_proj_bwd")
    sums = colsum(part.view(-1, H, 3))  # partials laid out (B, T blocks, H, 3)
    dxb = sums[:, 0].clone() if (gated or has_beta) else P.new_empty(0, dtype=torch.float32)
    return dP, sums[:, 1].clone(), sums[:, 2].clone(), dxb, colsum(dth)


@aspin_prep_proj_bwd.register_fake
def _(P, H, la_bias, A, la_floor, gate_bias, beta_bias, beta_min, gated, theta, pos, dq, dk, dv, dla, dbeta, D=64):
    f = lambda *s: P.new_empty(*s, dtype=torch.float32)
    has_beta = not gated and P.shape[-1] > 3 * H * D + H
    return (torch.empty_like(P), f(H), f(H), f(H) if (gated or has_beta) else f(0), f(H, D // 2))


def _prep_proj_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
    P, H, la_bias, A, la_floor, gate_bias, beta_bias, beta_min, gated, theta, pos, D = inputs
    ctx.H, ctx.beta_min, ctx.gated, ctx.D = H, beta_min, gated, D
    ctx.bias_dtype = (gate_bias if gated else beta_bias)
    ctx.bias_dtype = None if ctx.bias_dtype is None else ctx.bias_dtype.dtype
    ctx.dtypes = (P.dtype, la_bias.dtype, A.dtype, theta.dtype)
    ctx.save_for_backward(P, la_bias, A, la_floor, gate_bias, beta_bias, theta, pos)
    ctx.mark_non_differentiable(*[t for t in output[4:] if t.numel() == 0])


def _prep_proj_backward(ctx, dq, dk, dv, dla, dbeta):
    P, la_bias, A, la_floor, gate_bias, beta_bias, theta, pos = ctx.saved_tensors
    B, T, _ = P.shape
    zb = lambda t: torch.zeros(B, ctx.H, T, ctx.D, device=P.device, dtype=torch.bfloat16) if t is None else t
    dla = torch.zeros(B, ctx.H, T, device=P.device) if dla is None else dla
    dP, dlb, dA, dxb, dth = aspin_prep_proj_bwd(P, ctx.H, la_bias, A, la_floor, gate_bias, beta_bias, ctx.beta_min,
                                                ctx.gated, theta, pos, zb(dq), zb(dk), zb(dv), dla,
                                                dbeta if (dbeta is not None and dbeta.numel()) else None, ctx.D)
    dt = ctx.dtypes
    dgb = dxb.to(ctx.bias_dtype) if (ctx.gated and gate_bias is not None) else None
    dbb = dxb.to(ctx.bias_dtype) if (not ctx.gated and beta_bias is not None) else None
    return (dP.to(dt[0]), None, dlb.to(dt[1]), dA.to(dt[2]), None, dgb, dbb, None, None, dth.to(dt[3]), None, None)


aspin_prep_proj.register_autograd(_prep_proj_backward, setup_context=_prep_proj_setup)


# ---------------------------------------------------------------------------------------------------------------
# carried-state rebase: replaces the rotate() of S0's key rows at src/assoc.py:399-402
@torch.library.custom_op("pragnosia::aspin_rebase", mutates_args=())
def aspin_rebase(S: Tensor, theta: Tensor, p0_dev: Optional[Tensor], p0: float) -> Tensor:
    """Key rows (2i, 2i+1) of S (B, H, D, D), D = 64 or 128, rotated by -p0 * theta[h, i]; p0 from the device scalar
    p0_dev when given, else the float p0."""
    _require_gpu(S, theta, p0_dev)
    Dw = S.shape[-1] if S.dim() == 4 and S.shape[-1] in (64, 128) else 64
    _expect("aspin_rebase", S.device, S=(S, (None, None, Dw, Dw)))
    _expect("aspin_rebase", S.device, theta=(theta, (S.shape[1], Dw // 2)), p0_dev=(p0_dev, ()))
    S, theta, p0_dev = _f32(S), _f32(theta), _f32(p0_dev)
    B, H, D, _ = S.shape
    out = torch.empty_like(S)
    check(lib().pragnosia_aspin_rebase_fwd(_ptr(S), _ptr(theta), _ptr(p0_dev), float(p0), _ptr(out), B, H, D,
                                           _stream(S)), "pragnosia_aspin_rebase_fwd")
    return out


@aspin_rebase.register_fake
def _(S, theta, p0_dev, p0):
    return torch.empty_like(S, dtype=torch.float32)


@torch.library.custom_op("pragnosia::aspin_rebase_bwd", mutates_args=())
def aspin_rebase_bwd(S: Tensor, theta: Tensor, p0_dev: Optional[Tensor], p0: float,
                     g: Tensor) -> tuple[Tensor, Tensor]:
    _require_gpu(S, theta, p0_dev, g)
    Dw = S.shape[-1] if S.dim() == 4 and S.shape[-1] in (64, 128) else 64
    _expect("aspin_rebase_bwd", S.device, S=(S, (None, None, Dw, Dw)))
    _expect("aspin_rebase_bwd", S.device, theta=(theta, (S.shape[1], Dw // 2)), p0_dev=(p0_dev, ()),
            g=(g, tuple(S.shape)))
    S, theta, p0_dev, g = _f32(S), _f32(theta), _f32(p0_dev), _f32(g)
    B, H, D, _ = S.shape
    dS = torch.empty_like(S)
    dth = torch.empty(B, H, D // 2, device=S.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_rebase_bwd(_ptr(S), _ptr(theta), _ptr(p0_dev), float(p0), _ptr(g), _ptr(dS),
                                           _ptr(dth), B, H, D, _stream(S)), "pragnosia_aspin_rebase_bwd")
    return dS, colsum(dth)


@aspin_rebase_bwd.register_fake
def _(S, theta, p0_dev, p0, g):
    B, H, D, _ = S.shape
    return torch.empty_like(S, dtype=torch.float32), S.new_empty(H, D // 2, dtype=torch.float32)


def _rebase_setup(ctx, inputs, output):
    S, theta, p0_dev, p0 = inputs
    ctx.p0 = p0
    ctx.dtypes = (S.dtype, theta.dtype)
    ctx.save_for_backward(S, theta, p0_dev)


def _rebase_backward(ctx, g):
    S, theta, p0_dev = ctx.saved_tensors
    dS, dth = aspin_rebase_bwd(S, theta, p0_dev, ctx.p0, g.contiguous())
    return dS.to(ctx.dtypes[0]), dth.to(ctx.dtypes[1]), None, None


aspin_rebase.register_autograd(_rebase_backward, setup_context=_rebase_setup)


# ---------------------------------------------------------------------------------------------------------------
# the single-token recurrent step (decode): replaces the T = 1 torch path of src/assoc.py:391-411, :502
@torch.library.custom_op("pragnosia::aspin_decode_step", mutates_args=())
def aspin_decode_step(S: Tensor, qp: Tensor, kp: Tensor, vp: Tensor, gate: Optional[Tensor], la: Tensor,
                      beta: Optional[Tensor], theta: Tensor, p0_dev: Optional[Tensor],
                      p0: float) -> tuple[Tensor, Tensor]:
    """S (B, H, 64, 64) fp32 carried state; qp, kp, vp (B, H, 64) the T = 1 projections; gate (B, H) write-gate
    logits (plain rule) or None; la (B, H) log-decay; beta (B, H) write strength (delta rule) or None; theta (H, 32).
    Returns (S_new fp32, o (B, H, 64) fp32). Not differentiable (decode runs without autograd)."""
    _require_gpu(S, qp, kp, vp, gate, la, beta, theta, p0_dev)
    _expect("aspin_decode_step", S.device, S=(S, (None, None, 64, 64)))
    B_, H_ = S.shape[0], S.shape[1]
    _expect("aspin_decode_step", S.device, qp=(qp, (B_, H_, 64)), kp=(kp, (B_, H_, 64)), vp=(vp, (B_, H_, 64)),
            gate=(gate, (B_, H_)), la=(la, (B_, H_)), beta=(beta, (B_, H_)), theta=(theta, (H_, 32)),
            p0_dev=(p0_dev, ()))
    S, qp, kp, vp, gate = _f32(S), _f32(qp), _f32(kp), _f32(vp), _f32(gate)
    la, beta, theta, p0_dev = _f32(la), _f32(beta), _f32(theta), _f32(p0_dev)
    B, H, D, _ = S.shape
    S_new = torch.empty_like(S)
    o = torch.empty(B, H, D, device=S.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_decode_step(_ptr(S), _ptr(S_new), _ptr(qp), _ptr(kp), _ptr(vp), _ptr(gate), _ptr(la),
                                            _ptr(beta), _ptr(theta), _ptr(p0_dev), float(p0), _ptr(o), B, H, D,
                                            _stream(S)), "pragnosia_aspin_decode_step")
    return S_new, o


@aspin_decode_step.register_fake
def _(S, qp, kp, vp, gate, la, beta, theta, p0_dev, p0):
    B, H, D, _ = S.shape
    return torch.empty_like(S, dtype=torch.float32), S.new_empty(B, H, D, dtype=torch.float32)


# ---------------------------------------------------------------------------------------------------------------
# the fused decode step's kernels: replace the torch calls of one LM layer's T = 1 step inside the graphed decode
@torch.library.custom_op("pragnosia::decode_gemv", mutates_args=())
def decode_gemv(x: Tensor, W: Tensor, ln_weight: Optional[Tensor], ln_bias: Optional[Tensor], ln_eps: float,
                bias: Optional[Tensor], scale: Optional[Tensor], act: int, resid: Optional[Tensor]) -> Tensor:
    """y (B, N) = act(scale * (W LayerNorm(x)) + bias) + resid for x (B, K), W (N, K), all fp32; LayerNorm only when
    ln_weight is given; act 0 identity, 1 GELU (erf form); scale a device scalar. Not differentiable."""
    _require_gpu(x, W, ln_weight, ln_bias, bias, scale, resid)
    if x.dim() != 2 or W.dim() != 2 or W.shape[1] != x.shape[1]:
        raise PragnosiaError(f"decode_gemv: x {tuple(x.shape)} and W {tuple(W.shape)} must be (B, K) and (N, K)")
    B_, K_, N_ = x.shape[0], x.shape[1], W.shape[0]
    _expect("decode_gemv", x.device, W=(W, (N_, K_)), ln_weight=(ln_weight, (K_,)), ln_bias=(ln_bias, (K_,)),
            bias=(bias, (N_,)), scale=(scale, ()), resid=(resid, (B_, N_)))
    x, W = _f32(x), _f32(W)
    ln_weight, ln_bias, bias, scale, resid = _f32(ln_weight), _f32(ln_bias), _f32(bias), _f32(scale), _f32(resid)
    B, K = x.shape
    N = W.shape[0]
    y = torch.empty(B, N, device=x.device, dtype=torch.float32)
    check(lib().pragnosia_decode_gemv(_ptr(x), B, K, _ptr(ln_weight), _ptr(ln_bias), float(ln_eps), _ptr(W), N,
                                      _ptr(bias), _ptr(scale), int(act), _ptr(resid), _ptr(y), _stream(x)),
          "pragnosia_decode_gemv")
    return y


@decode_gemv.register_fake
def _(x, W, ln_weight, ln_bias, ln_eps, bias, scale, act, resid):
    return x.new_empty(x.shape[0], W.shape[0], dtype=torch.float32)


@torch.library.custom_op("pragnosia::decode_gemv_rms", mutates_args=())
def decode_gemv_rms(x: Tensor, W: Tensor, rms_weight: Tensor, rms_eps: float, bias: Optional[Tensor],
                    scale: Optional[Tensor], act: int, resid: Optional[Tensor]) -> Tensor:
    """y (B, N) = act(scale * (W z) + bias) + resid with z the per-head RMSNorm of x (B, K) with rms_weight (G,),
    heads of G = 64 or 128 channels: the carrier's per-head RMSNorm and gated o-projection of one decode step, for
    B <= 4 and K a multiple of 256 up to 1024. All fp32. Not differentiable."""
    _require_gpu(x, W, rms_weight, bias, scale, resid)
    if x.dim() != 2 or W.dim() != 2 or W.shape[1] != x.shape[1]:
        raise PragnosiaError(f"decode_gemv_rms: x {tuple(x.shape)} and W {tuple(W.shape)} must be (B, K) and (N, K)")
    B_, K_, N_ = x.shape[0], x.shape[1], W.shape[0]
    G = rms_weight.numel()
    if G not in (64, 128) or K_ % G:
        raise PragnosiaError(f"decode_gemv_rms: RMSNorm weight of {G} channels over rows of {K_} (heads of 64 or 128)")
    _expect("decode_gemv_rms", x.device, W=(W, (N_, K_)), rms_weight=(rms_weight, (G,)), bias=(bias, (N_,)),
            scale=(scale, ()), resid=(resid, (B_, N_)))
    x, W, rms_weight = _f32(x), _f32(W), _f32(rms_weight)
    bias, scale, resid = _f32(bias), _f32(scale), _f32(resid)
    y = torch.empty(B_, N_, device=x.device, dtype=torch.float32)
    check(lib().pragnosia_decode_gemv_rms(_ptr(x), B_, K_, _ptr(rms_weight), G, float(rms_eps), _ptr(W), N_,
                                          _ptr(bias), _ptr(scale), int(act), _ptr(resid), _ptr(y), _stream(x)),
          "pragnosia_decode_gemv_rms")
    return y


@decode_gemv_rms.register_fake
def _(x, W, rms_weight, rms_eps, bias, scale, act, resid):
    return x.new_empty(x.shape[0], W.shape[0], dtype=torch.float32)


def decode_gemm_tile(W: Tensor, col_scale: Optional[Tensor] = None) -> Tensor:
    """The tiled copy of a dense layer's weight W (N, K) fp32 that `decode_gemm` reads (K a multiple of 16), its
    columns scaled by col_scale when given (a normalisation's weight folded in: (K,), or (G,) repeated over the
    G-channel groups), flat: Wt[((t KS + s) 64 + l) 4 + e] = W[16 t + l % 16][16 s + 4 (l / 16) + e] for column tile
    t, 16-wide step s of KS = K / 16, lane l, entry e; columns past N padded with zeros. So each wave's weight piece
    of a step is one contiguous 1 KiB read, laid out as the fp32 matrix cores take their operand."""
    N, K = W.shape
    if K % 16:
        raise PragnosiaError(f"decode_gemm_tile: K = {K} is not a multiple of 16")
    Wp = W.detach().to(torch.float32)
    if col_scale is not None:
        cs = col_scale.detach().to(torch.float32)
        Wp = Wp * (cs.repeat(K // cs.numel()) if cs.numel() != K else cs)
    NT = (N + 15) // 16
    if NT * 16 != N:
        Wp = torch.cat([Wp, Wp.new_zeros(NT * 16 - N, K)])
    return Wp.reshape(NT, 16, K // 16, 4, 4).permute(0, 2, 3, 1, 4).contiguous().reshape(-1)


def decode_gemm_ln(W: Tensor, ln_weight: Tensor, ln_bias: Optional[Tensor], bias: Optional[Tensor],
                   scale: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """A LayerNorm + linear layer folded for `decode_gemm` mode 1: (the tiled W diag(ln_weight), the row sums of that
    fp32 product (summed in fp64), bias + scale W ln_bias (in fp64)). Then decode_gemm(x, Wt, N, 1, csum, eps, bias',
    scale, ...) = scale (W LayerNorm(x)) + bias. With a scale, the folded bias holds its value at fold time."""
    Wf = W.detach().to(torch.float32) * ln_weight.detach().to(torch.float32)
    csum = Wf.double().sum(1).float()
    b = torch.zeros(W.shape[0], device=W.device, dtype=torch.float64) if bias is None else bias.detach().double()
    if ln_bias is not None:
        wb = W.detach().double() @ ln_bias.detach().double()
        b = b + (wb if scale is None else scale.detach().double() * wb)
    return decode_gemm_tile(Wf), csum, b.float()


def decode_gemm_ok(K: int, mode: int) -> bool:
    """Whether `decode_gemm` covers a dense layer of input width K in this mode."""
    return lib().pragnosia_decode_gemm_waves(K, mode) > 0


@torch.library.custom_op("pragnosia::decode_gemm", mutates_args=())
def decode_gemm(x: Tensor, Wt: Tensor, N: int, mode: int, csum: Optional[Tensor], eps: float,
                bias: Optional[Tensor], scale: Optional[Tensor], act: int, resid: Optional[Tensor]) -> Tensor:
    """y (B, N) = act(scale * (W z) + bias) + resid on the fp32 matrix cores, W given tiled (`decode_gemm_tile`), with
    z = x (mode 0), the row standardised (mode 1: a LayerNorm folded by `decode_gemm_ln`, csum its row sums) or each
    64-channel (mode 2) or 128-channel (mode 3) group RMS-scaled (the RMSNorm's weight folded into the tiled W). The
    dense layers of the decode step past GEMV batch sizes. Not differentiable."""
    _require_gpu(x, Wt, csum, bias, scale, resid)
    if x.dim() != 2:
        raise PragnosiaError(f"decode_gemm: x must be (B, K), got {tuple(x.shape)}")
    B_, K_ = x.shape
    if K_ % 16 or Wt.numel() != ((N + 15) // 16) * 16 * K_:
        raise PragnosiaError(f"decode_gemm: tiled weight of {Wt.numel()} values does not fit N {N} and K {K_}")
    if (mode == 1) != (csum is not None):
        raise PragnosiaError("decode_gemm: mode 1 takes the folded weight's row sums, the other modes none")
    _expect("decode_gemm", x.device, csum=(csum, (N,)), bias=(bias, (N,)), scale=(scale, ()), resid=(resid, (B_, N)))
    x, Wt, csum, bias, scale, resid = _f32(x), _f32(Wt), _f32(csum), _f32(bias), _f32(scale), _f32(resid)
    y = torch.empty(B_, N, device=x.device, dtype=torch.float32)
    check(lib().pragnosia_decode_gemm(_ptr(x), B_, K_, int(mode), _ptr(csum), float(eps), _ptr(Wt), N, _ptr(bias),
                                      _ptr(scale), int(act), _ptr(resid), _ptr(y), _stream(x)),
          "pragnosia_decode_gemm")
    return y


@decode_gemm.register_fake
def _(x, Wt, N, mode, csum, eps, bias, scale, act, resid):
    return x.new_empty(x.shape[0], N, dtype=torch.float32)


@torch.library.custom_op("pragnosia::decode_gemv_acc_", mutates_args=("y",))
def decode_gemv_acc_(x: Tensor, W: Tensor, bias: Optional[Tensor], scale: Optional[Tensor], y: Tensor) -> None:
    """y (B, N) += scale * (W x) + bias in place for B <= 4, W (N, K) fp32 row-major, K a multiple of 256 up to 4096:
    the one-wave GEMV with its K split over workgroups that add their partial sums into y (which holds the residual).
    Adds in varying order: not bit-deterministic. Not differentiable."""
    _require_gpu(x, W, bias, scale, y)
    if x.dim() != 2 or y.dim() != 2 or y.shape[0] != x.shape[0] or not 1 <= x.shape[0] <= 4:
        raise PragnosiaError(f"decode_gemv_acc_: x (B, K) and y (B, N) with B <= 4 expected, got {tuple(x.shape)}, "
                             f"{tuple(y.shape)}")
    B_, K_ = x.shape
    N = y.shape[1]
    if K_ % 256 or K_ > 4096:
        raise PragnosiaError(f"decode_gemv_acc_: K = {K_} must be a multiple of 256 up to 4096")
    if y.dtype != torch.float32 or not y.is_contiguous():
        raise PragnosiaError("decode_gemv_acc_: y must be contiguous fp32 (it is added into in place)")
    _expect("decode_gemv_acc_", x.device, W=(W, (N, K_)), bias=(bias, (N,)), scale=(scale, ()), y=(y, (B_, N)))
    x, W, bias, scale = _f32(x), _f32(W), _f32(bias), _f32(scale)
    check(lib().pragnosia_decode_gemv_acc(_ptr(x), B_, K_, _ptr(W), N, _ptr(bias), _ptr(scale), _ptr(y),
                                          _stream(x)), "pragnosia_decode_gemv_acc")


@decode_gemv_acc_.register_fake
def _(x, W, bias, scale, y):
    return None


@torch.library.custom_op("pragnosia::decode_gemm_acc_", mutates_args=("y",))
def decode_gemm_acc_(x: Tensor, Wt: Tensor, group_mode: int, eps: float, bias: Optional[Tensor],
                     scale: Optional[Tensor], y: Tensor) -> None:
    """y (B, N) += scale * (W z) + bias in place, W given tiled (`decode_gemm_tile`): `decode_gemm` mode 0 (z = x) or
    2 / 3 (z = x RMS-scaled per 64- / 128-channel group, the RMSNorm's weight folded into the tiled W) with its K split
    over groups of workgroups that add their partial products into y (which holds the residual), so the layer spreads
    over more compute units. Adds in varying order: not bit-deterministic. Not differentiable."""
    _require_gpu(x, Wt, bias, scale, y)
    if x.dim() != 2 or y.dim() != 2 or y.shape[0] != x.shape[0]:
        raise PragnosiaError(f"decode_gemm_acc_: x (B, K) and y (B, N) expected, got {tuple(x.shape)}, "
                             f"{tuple(y.shape)}")
    B_, K_ = x.shape
    N = y.shape[1]
    if K_ % 16 or Wt.numel() != ((N + 15) // 16) * 16 * K_:
        raise PragnosiaError(f"decode_gemm_acc_: tiled weight of {Wt.numel()} values does not fit N {N} and K {K_}")
    if y.dtype != torch.float32 or not y.is_contiguous():
        raise PragnosiaError("decode_gemm_acc_: y must be contiguous fp32 (it is added into in place)")
    if group_mode not in (0, 2, 3):
        raise PragnosiaError(f"decode_gemm_acc_: group_mode {group_mode} (0, 2 or 3 expected)")
    _expect("decode_gemm_acc_", x.device, bias=(bias, (N,)), scale=(scale, ()), y=(y, (B_, N)))
    x, Wt, bias, scale = _f32(x), _f32(Wt), _f32(bias), _f32(scale)
    check(lib().pragnosia_decode_gemm_acc(_ptr(x), B_, K_, int(group_mode), float(eps), _ptr(Wt), N, _ptr(bias),
                                          _ptr(scale), _ptr(y), _stream(x)), "pragnosia_decode_gemm_acc")


@decode_gemm_acc_.register_fake
def _(x, Wt, group_mode, eps, bias, scale, y):
    return None


def decode_tail(logits: Tensor, emb: Tensor, pemb: Tensor, ctr_in: Tensor, ctr_out: Tensor, pos_in: Tensor,
                pos_out: Tensor, out: Tensor, tok: Tensor, h: Tensor, p0s: Optional[Tensor],
                logits_rec: Optional[Tensor]) -> None:
    """The end of one graphed greedy decode step, in place (`pragnosia_decode_tail`): tok = argmax of logits (B, V)
    per row (torch.argmax's rule), out[*ctr_in] = tok, h = emb[tok] + pemb[(*pos_in + 1) mod ctx], *pos_out and
    *ctr_out advanced, p0s set to 1, and the logits copied to logits_rec[*ctr_in] when given. ctr and pos are int64
    device scalars, each read from one and written to another. All on one device, fp32 / int64 contiguous."""
    _require_gpu(logits, emb, pemb, ctr_in, ctr_out, pos_in, pos_out, out, tok, h, p0s, logits_rec)
    B, V = logits.shape
    d = emb.shape[1]
    ok = (logits.dtype == torch.float32 and logits.is_contiguous() and emb.shape[0] == V and pemb.shape[1] == d
          and out.dtype == torch.int64 and out.dim() == 2 and out.shape[1] == B and tok.numel() == B
          and tok.dtype == torch.int64 and h.shape == (B, d) and h.dtype == torch.float32
          and all(t.dtype == torch.int64 and t.numel() == 1 for t in (ctr_in, ctr_out, pos_in, pos_out))
          and all(t.is_contiguous() for t in (emb, pemb, out, tok, h))
          and (logits_rec is None or (logits_rec.shape == (out.shape[0], B, V) and logits_rec.is_contiguous()
                                      and logits_rec.dtype == torch.float32))
          and (p0s is None or (p0s.dtype == torch.float32 and p0s.is_contiguous())))
    if not ok or emb.dtype != torch.float32 or pemb.dtype != torch.float32:
        raise PragnosiaError("decode_tail: buffers do not have the documented shapes, dtypes or layout")
    check(lib().pragnosia_decode_tail(_ptr(logits), B, V, _ptr(emb), _ptr(pemb), d, pemb.shape[0], _ptr(ctr_in),
                                      _ptr(ctr_out), _ptr(pos_in), _ptr(pos_out), _ptr(out), out.shape[0], _ptr(tok),
                                      _ptr(h), _ptr(p0s), 0 if p0s is None else p0s.numel(), _ptr(logits_rec),
                                      _stream(logits)), "pragnosia_decode_tail")


@torch.library.custom_op("pragnosia::aspin_decode_proj_", mutates_args=("S",))
def aspin_decode_proj_(S: Tensor, P: Tensor, H: int, la_bias: Tensor, A: Tensor, la_floor: Optional[Tensor],
                       gate_bias: Optional[Tensor], beta_bias: Optional[Tensor], beta_min: float, gated: bool,
                       theta: Tensor, p0_dev: Optional[Tensor], p0: float, on_weight: Optional[Tensor],
                       on_eps: float) -> Tensor:
    """The carrier's recurrent step from one projection GEMV's output P (B, 3 H D + H [+ H]) (q, k, v, decay
    logits, then the write-gate (gated) or write-strength logits), updating the carried state S (B, H, D, D) fp32 in
    place. Returns the output token-major, (B, H * D) fp32: RMS-normalised per head with on_weight (D = 64), or raw
    when on_weight is None (D = 64 or 128; D / 16 workgroups per head below 256 heads, one past it; decode_gemv_rms
    or decode_gemm then applies the RMSNorm)."""
    _require_gpu(S, P, la_bias, A, theta, on_weight)
    if not (S.is_contiguous() and S.dtype == torch.float32):
        raise PragnosiaError("aspin_decode_proj_: the state must be a contiguous fp32 tensor (it is updated in place)")
    if P.dim() != 2:
        raise PragnosiaError(f"aspin_decode_proj_: P must be (B, W), got {tuple(P.shape)}")
    D = S.shape[-1] if S.dim() == 4 else 64
    if D not in (64, 128) or (D == 128 and on_weight is not None):
        raise PragnosiaError(f"aspin_decode_proj_: heads of {D} (64, or 128 with the raw output)")
    _expect_proj("aspin_decode_proj_", P, H, gated, la_bias, A, la_floor, gate_bias, beta_bias, theta, D=D)
    _expect("aspin_decode_proj_", P.device, S=(S, (P.shape[0], H, D, D)), p0_dev=(p0_dev, ()),
            on_weight=(on_weight, (64,)))
    P, la_bias, A, la_floor, theta = _f32(P), _f32(la_bias), _f32(A), _f32(la_floor), _f32(theta)
    gate_bias, beta_bias, p0_dev, on_weight = _f32(gate_bias), _f32(beta_bias), _f32(p0_dev), _f32(on_weight)
    B, np_ = P.shape
    has_beta = not gated and np_ > 3 * H * D + H
    acol, gcol, bcol = _proj_cols(H, gated, has_beta, D)
    o = torch.empty(B, H * D, device=P.device, dtype=torch.float32)
    check(lib().pragnosia_aspin_decode_proj(_ptr(S), _ptr(S), _ptr(P), np_, acol, gcol, bcol, _ptr(la_bias), _ptr(A),
                                            _ptr(la_floor), _ptr(gate_bias), _ptr(beta_bias), float(beta_min),
                                            _ptr(theta), _ptr(p0_dev), float(p0), _ptr(on_weight), float(on_eps),
                                            _ptr(o), B, H, D, _stream(P)), "pragnosia_aspin_decode_proj")
    return o


@aspin_decode_proj_.register_fake
def _(S, P, H, la_bias, A, la_floor, gate_bias, beta_bias, beta_min, gated, theta, p0_dev, p0, on_weight, on_eps):
    return P.new_empty(P.shape[0], H * S.shape[-1], dtype=torch.float32)


@torch.library.custom_op("pragnosia::aspin_decode_oproj_", mutates_args=("S_out", "y"))
def aspin_decode_oproj_(S: Tensor, S_out: Tensor, P: Tensor, H: int, la_bias: Tensor, A: Tensor,
                        la_floor: Optional[Tensor], gate_bias: Optional[Tensor], beta_bias: Optional[Tensor],
                        beta_min: float, gated: bool, theta: Tensor, p0_dev: Optional[Tensor], p0: float,
                        on_weight: Tensor, on_eps: float, Wo: Tensor, scale: Optional[Tensor], y: Tensor) -> None:
    """aspin_decode_proj_ with the per-head RMSNorm, then the gated o-projection and residual, in one launch (64-wide
    heads): reads the carried state S (B, H, 64, 64), writes the new state to S_out (a different buffer: every
    workgroup reads the old state) and adds scale * (Wo o_n) to y (B, N), which holds the residual on entry; Wo (N,
    H 64), scale a one-element tensor (the gate's sigmoid) or None. The heads' contributions are added with atomics in
    arrival order: y equals the two-launch result to fp32 rounding, not bit for bit, and not the same bits from run
    to run."""
    _require_gpu(S, S_out, P, la_bias, A, theta, on_weight, Wo, scale, y)
    for name, t in (("S", S), ("S_out", S_out), ("y", y)):
        if not (t.is_contiguous() and t.dtype == torch.float32):
            raise PragnosiaError(f"aspin_decode_oproj_: {name} must be a contiguous fp32 tensor")
    if P.dim() != 2:
        raise PragnosiaError(f"aspin_decode_oproj_: P must be (B, W), got {tuple(P.shape)}")
    if S.data_ptr() == S_out.data_ptr():
        raise PragnosiaError("aspin_decode_oproj_: S_out must be another buffer than S")
    B = P.shape[0]
    N = Wo.shape[0] if Wo.dim() == 2 else -1
    _expect_proj("aspin_decode_oproj_", P, H, gated, la_bias, A, la_floor, gate_bias, beta_bias, theta, D=64)
    _expect("aspin_decode_oproj_", P.device, S=(S, (B, H, 64, 64)), S_out=(S_out, (B, H, 64, 64)),
            p0_dev=(p0_dev, ()), on_weight=(on_weight, (64,)), Wo=(Wo, (N, H * 64)), y=(y, (B, N)),
            scale=(scale, ()))
    P, la_bias, A, la_floor, theta = _f32(P), _f32(la_bias), _f32(A), _f32(la_floor), _f32(theta)
    gate_bias, beta_bias, p0_dev, on_weight = _f32(gate_bias), _f32(beta_bias), _f32(p0_dev), _f32(on_weight)
    Wo, scale = _f32(Wo), _f32(scale)
    np_ = P.shape[1]
    has_beta = not gated and np_ > 3 * H * 64 + H
    acol, gcol, bcol = _proj_cols(H, gated, has_beta, 64)
    check(lib().pragnosia_aspin_decode_oproj(_ptr(S), _ptr(S_out), _ptr(P), np_, acol, gcol, bcol, _ptr(la_bias),
                                             _ptr(A), _ptr(la_floor), _ptr(gate_bias), _ptr(beta_bias),
                                             float(beta_min), _ptr(theta), _ptr(p0_dev), float(p0), _ptr(on_weight),
                                             float(on_eps), _ptr(Wo), N, _ptr(scale), _ptr(y), B, H, 64, _stream(P)),
          "pragnosia_aspin_decode_oproj")


@aspin_decode_oproj_.register_fake
def _(S, S_out, P, H, la_bias, A, la_floor, gate_bias, beta_bias, beta_min, gated, theta, p0_dev, p0, on_weight,
      on_eps, Wo, scale, y):
    return None
