// The carrier's output epilogue: the per-head RMSNorm of the scan's output and the move back to the projections'
// token-major layout, in one pass each way.
//
// Forward, per (batch, head, token) row x of D = 64 or 128 channels (the scan output o, (B, H, T, D) bf16):
//     r = 1 / sqrt(mean(x^2) + eps),   y[b, t, h D + d] = (x_d r) w_d,
// rounded once to the output dtype (bf16 under autocast, fp32 otherwise) and written in (B, T, H D): the
// reference's `self.on(o).transpose(1, 2).reshape(B, T, D)` (`src/assoc.py:505`, nn.RMSNorm(dk) with eps=None, which
// computes in fp32 with fp32's epsilon). r is saved per row for the backward.
// Backward, with g the gradient on y (either dtype):
//     dx_d = r w_d g_d - x_d r^3 (1/D) sum_e x_e w_e g_e     (written as the scan's dO, (B, H, T, D) bf16)
//     dw_d = sum over rows of g_d x_d r                        (one partial per workgroup, reduced by the caller)
//
// One workgroup of 256 threads per (batch, head, 64-token block): D / 4 threads per row (4 channels each), 1024 / D
// rows per pass. HBM-bound: forward reads 2 B and writes 2 or 4 B per element, backward reads 4-6 B and writes 2 B.
#include "common.h"

namespace {

constexpr int TB = 64;    // tokens per workgroup

// sum over the L lanes that share a row (lane bits 0 .. log2 L - 1)
template <int L>
PGN_DEVICE float sum_lanes(float x) {
#pragma unroll
  for (int o = 1; o < L; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

PGN_DEVICE f32x4 load4(const __bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
PGN_DEVICE f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

PGN_DEVICE void store4(__bf16* p, f32x4 x) {
  bf16x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (__bf16)x[e];
  *reinterpret_cast<bf16x4*>(p) = v;
}
PGN_DEVICE void store4(float* p, f32x4 x) { *reinterpret_cast<f32x4*>(p) = x; }

template <typename Out, int D>
__global__ __launch_bounds__(256) void out_fwd(const __bf16* __restrict__ o, const float* __restrict__ w, float eps,
                                               Out* __restrict__ y, float* __restrict__ rstd, int T, int H,
                                               int ntb) {
  constexpr int L = D / 4, ROWS = 256 / L;
  const int blk = blockIdx.x;
  const int bh = blk / ntb, tb = blk - bh * ntb;
  const int b = bh / H, h = bh - b * H;
  const int j = threadIdx.x & (L - 1), rs = threadIdx.x / L;
  const f32x4 wv = *reinterpret_cast<const f32x4*>(w + 4 * j);
#pragma unroll
  for (int p = 0; p < TB / ROWS; ++p) {
    const int t = tb * TB + p * ROWS + rs;
    if (t >= T) break;
    const f32x4 x = load4(o + ((size_t)bh * T + t) * D + 4 * j);
    const float ss = sum_lanes<L>(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float r = 1.f / sqrtf(ss * (1.f / D) + eps);
    f32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (x[e] * r) * wv[e];
    store4(y + (((size_t)b * T + t) * H + h) * D + 4 * j, out);
    if (j == 0) rstd[(size_t)bh * T + t] = r;
  }
}

template <typename G, int D>
__global__ __launch_bounds__(256) void out_bwd(const G* __restrict__ gy, const __bf16* __restrict__ o,
                                               const float* __restrict__ w, const float* __restrict__ rstd,
                                               __bf16* __restrict__ dO, float* __restrict__ dw_part, int T, int H,
                                               int ntb) {
  constexpr int L = D / 4, ROWS = 256 / L;
  __shared__ f32x4 red[ROWS][L];
  const int blk = blockIdx.x;
  const int bh = blk / ntb, tb = blk - bh * ntb;
  const int b = bh / H, h = bh - b * H;
  const int j = threadIdx.x & (L - 1), rs = threadIdx.x / L;
  const f32x4 wv = *reinterpret_cast<const f32x4*>(w + 4 * j);
  f32x4 dw = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < TB / ROWS; ++p) {
    const int t = tb * TB + p * ROWS + rs;
    if (t >= T) break;
    const size_t row = ((size_t)bh * T + t) * D + 4 * j;
    const f32x4 x = load4(o + row);
    const f32x4 g = load4(gy + (((size_t)b * T + t) * H + h) * D + 4 * j);
    const float r = rstd[(size_t)bh * T + t];
    const float s = sum_lanes<L>(x[0] * wv[0] * g[0] + x[1] * wv[1] * g[1] + x[2] * wv[2] * g[2] +
                                 x[3] * wv[3] * g[3]);
    const float c = r * r * r * s * (1.f / D);
    f32x4 dx;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dx[e] = r * wv[e] * g[e] - x[e] * c;
      dw[e] += g[e] * x[e] * r;
    }
    store4(dO + row, dx);
  }
  red[rs][j] = dw;
  __syncthreads();
  if (threadIdx.x < D) {
    const int jj = threadIdx.x >> 2, e = threadIdx.x & 3;
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc += red[r][jj][e];
    dw_part[(size_t)blk * D + threadIdx.x] = acc;
  }
}

bool shape_ok(int64_t B, int64_t H, int64_t T) {
  return B > 0 && H > 0 && T > 0 && B * H * ((T + TB - 1) / TB) < ((int64_t)1 << 31) &&
         B * T * H < ((int64_t)1 << 40);
}

}  // namespace

namespace {

template <int D>
int out_fwd_launch(const void* o, const float* weight, float eps, void* y, int y_bf16, float* rstd, int64_t B,
                   int64_t H, int64_t T, hipStream_t st) {
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  if (y_bf16)
    hipLaunchKernelGGL((out_fwd<__bf16, D>), grid, dim3(256), 0, st, (const __bf16*)o, weight, eps, (__bf16*)y, rstd,
                       (int)T, (int)H, ntb);
  else
    hipLaunchKernelGGL((out_fwd<float, D>), grid, dim3(256), 0, st, (const __bf16*)o, weight, eps, (float*)y, rstd,
                       (int)T, (int)H, ntb);
  PGN_RETURN_LAUNCH();
}

template <int D>
int out_bwd_launch(const void* gy, int gy_bf16, const void* o, const float* weight, const float* rstd, void* dO,
                   float* dw_partials, int64_t B, int64_t H, int64_t T, hipStream_t st) {
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  if (gy_bf16)
    hipLaunchKernelGGL((out_bwd<__bf16, D>), grid, dim3(256), 0, st, (const __bf16*)gy, (const __bf16*)o, weight,
                       rstd, (__bf16*)dO, dw_partials, (int)T, (int)H, ntb);
  else
    hipLaunchKernelGGL((out_bwd<float, D>), grid, dim3(256), 0, st, (const float*)gy, (const __bf16*)o, weight, rstd,
                       (__bf16*)dO, dw_partials, (int)T, (int)H, ntb);
  PGN_RETURN_LAUNCH();
}

}  // namespace

extern "C" int pragnosia_aspin_out_fwd(const void* o, const float* weight, float eps, void* y, int y_bf16,
                                       float* rstd, int64_t B, int64_t H, int64_t T, int64_t D_, void* stream) {
  if (D_ != 64 && D_ != 128) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T));
  PGN_CHECK_ARG(o && weight && y && rstd && eps >= 0.f);
  hipStream_t st = (hipStream_t)stream;
  return D_ == 64 ? out_fwd_launch<64>(o, weight, eps, y, y_bf16, rstd, B, H, T, st)
                  : out_fwd_launch<128>(o, weight, eps, y, y_bf16, rstd, B, H, T, st);
}

extern "C" int64_t pragnosia_aspin_out_weight_partials(int64_t B, int64_t H, int64_t T) {
  if (!shape_ok(B, H, T)) return -1;
  return B * H * ((T + TB - 1) / TB);
}

extern "C" int pragnosia_aspin_out_bwd(const void* gy, int gy_bf16, const void* o, const float* weight,
                                       const float* rstd, void* dO, float* dw_partials, int64_t B, int64_t H,
                                       int64_t T, int64_t D_, void* stream) {
  if (D_ != 64 && D_ != 128) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T));
  PGN_CHECK_ARG(gy && o && weight && rstd && dO && dw_partials);
  hipStream_t st = (hipStream_t)stream;
  return D_ == 64 ? out_bwd_launch<64>(gy, gy_bf16, o, weight, rstd, dO, dw_partials, B, H, T, st)
                  : out_bwd_launch<128>(gy, gy_bf16, o, weight, rstd, dO, dw_partials, B, H, T, st);
}
