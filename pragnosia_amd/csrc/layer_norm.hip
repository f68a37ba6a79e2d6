// LayerNorm over the last dimension, fp32 statistics, for the carrier's input norm and the MLP's (the reference's
// `nn.LayerNorm(d)`, src/assoc.py:323,388, src/model.py:555): forward writing its output in the dtype of the matmul
// that consumes it (bf16 under autocast, where the reference's fp32 LayerNorm output is cast to bf16 by that matmul;
// fp32 otherwise), and backward taking that matmul's input gradient in either dtype.
//
//     mu = mean(x),  var = mean((x - mu)^2),  r = 1 / sqrt(var + eps),  xh = (x - mu) r,  y = xh w + b
//     dx = r (g - mean(g) - xh mean(g xh)),  g = dy w;   dw = sum_rows dy xh,  db = sum_rows dy
//
// One wave per row, D a multiple of 4 up to 256 V: lane l holds elements 4 (l + 64 k) .. +3, k < V (groups at or past
// D are inactive: nothing is loaded or stored there and they add zero to every sum), so every load and store of a
// row is one contiguous wave access per k; the row's sums are wave totals on DPP row shifts (no LDS round trips).
// The backward runs 8 waves of R rows each per workgroup (R = 2 for D <= 1024, else 1), every wave loading all its
// rows before the first reduction; the waves' column sums of dy xh and dy are added in LDS and written as one partial
// row of each per workgroup, for the caller to sum (a fixed-order column sum, so nothing records a memset). Memory
// per row: forward reads 4 D bytes and writes 2 D (bf16) or 4 D; backward reads 2 D or 4 D and 4 D, writes 4 D.
#include "common.h"
#include "mfma_tile.h"

namespace {

using pgn::lane_value;
using pgn::row_total16;

constexpr int kBwdWaves = 8;

constexpr int rows_per_wave(int V) { return V <= 4 ? 2 : 1; }

// The total over the wave's 64 lanes, in every lane: sums within each row of 16 lanes on DPP row shifts (lane 15 of a
// row ends holding its row's total), then the four row totals read as scalars.
PGN_DEVICE float ln_wave_total(float x) {
  x = row_total16(x);
  return (lane_value(x, 15) + lane_value(x, 31)) + (lane_value(x, 47) + lane_value(x, 63));
}

PGN_DEVICE float4 zero_f4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

PGN_DEVICE float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

PGN_DEVICE float4 ld4_dy(const void* dy, size_t e, bool bf16) {
  if (bf16) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const __bf16*>(dy) + e);
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
  }
  return ld4(reinterpret_cast<const float*>(dy) + e);
}

template <int V>
__global__ __launch_bounds__(256) void ln_fwd(const float* __restrict__ x, const float* __restrict__ w,
                                              const float* __restrict__ b, float eps, void* __restrict__ y,
                                              int y_bf16, float* __restrict__ mean, float* __restrict__ rstd,
                                              int64_t rows, int D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // a whole wave
  const int l = threadIdx.x & 63;
  const float* xr = x + row * D;
  float4 v[V], wv[V], bv[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int e = 4 * (l + 64 * k);
    const bool on = e < D;
    v[k] = on ? ld4(xr + e) : zero_f4();
    wv[k] = on ? ld4(w + e) : zero_f4();
    bv[k] = on ? ld4(b + e) : zero_f4();
  }
  const float inv_d = 1.f / (float)D;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < V; ++k) s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  const float mu = ln_wave_total(s) * inv_d;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const float a = v[k].x - mu, bb = v[k].y - mu, c = v[k].z - mu, d = v[k].w - mu;
    const float t = (a * a + bb * bb) + (c * c + d * d);
    q += 4 * (l + 64 * k) < D ? t : 0.f;
  }
  const float r = rsqrtf(ln_wave_total(q) * inv_d + eps);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int e = 4 * (l + 64 * k);
    if (e >= D) continue;
    const float4 o = make_float4((v[k].x - mu) * r * wv[k].x + bv[k].x, (v[k].y - mu) * r * wv[k].y + bv[k].y,
                                 (v[k].z - mu) * r * wv[k].z + bv[k].z, (v[k].w - mu) * r * wv[k].w + bv[k].w);
    if (y_bf16) {
      bf16x4 ob;
      ob[0] = (__bf16)o.x;
      ob[1] = (__bf16)o.y;
      ob[2] = (__bf16)o.z;
      ob[3] = (__bf16)o.w;
      *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(y) + row * D + e) = ob;
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + row * D + e) = o;
    }
  }
  if (l == 0) {
    mean[row] = mu;
    rstd[row] = r;
  }
}

// Adds the kBwdWaves waves' float4 column sums a[V] in LDS (buffer red, one 256 V-float row per wave) and writes the
// first D columns of the total row to dst. Every thread of the workgroup takes part (two barriers).
template <int V>
PGN_DEVICE void ln_reduce_waves(float (*red)[256 * V], const float4 (&a)[V], float* __restrict__ dst, int D) {
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < V; ++k) *reinterpret_cast<float4*>(&red[wv][4 * (l + 64 * k)]) = a[k];
  __syncthreads();
  for (int c4 = threadIdx.x; c4 < D / 4; c4 += 64 * kBwdWaves) {
    float4 s = *reinterpret_cast<const float4*>(&red[0][4 * c4]);
#pragma unroll
    for (int i = 1; i < kBwdWaves; ++i) {
      const float4 t = *reinterpret_cast<const float4*>(&red[i][4 * c4]);
      s.x += t.x;
      s.y += t.y;
      s.z += t.z;
      s.w += t.w;
    }
    *reinterpret_cast<float4*>(dst + 4 * c4) = s;
  }
  __syncthreads();
}

template <int V>
__global__ __launch_bounds__(64 * kBwdWaves) void ln_bwd(const void* __restrict__ dy, int dy_bf16,
                                                         const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ mean,
                                                         const float* __restrict__ rstd, float* __restrict__ dx,
                                                         float* __restrict__ dwp, float* __restrict__ dbp,
                                                         int64_t rows, int D) {
  constexpr int R = rows_per_wave(V);
  __shared__ float red[kBwdWaves][256 * V];
  const int l = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * kBwdWaves + (threadIdx.x >> 6)) * R;
  float4 wv[V], xv[R][V], d[R][V];
  float mu[R], rs[R];
#pragma unroll
  for (int k = 0; k < V; ++k) wv[k] = 4 * (l + 64 * k) < D ? ld4(w + 4 * (l + 64 * k)) : zero_f4();
  // every row's loads first; a row past the end, or an element past D, reads nothing and has dy = 0, so it adds
  // nothing to the sums
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int64_t row = r0 + rr;
    const bool in = row < rows;
    mu[rr] = in ? mean[row] : 0.f;
    rs[rr] = in ? rstd[row] : 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int e = 4 * (l + 64 * k);
      const bool on = in && e < D;
      xv[rr][k] = on ? ld4(x + row * D + e) : zero_f4();
      d[rr][k] = on ? ld4_dy(dy, (size_t)(row * D + e), dy_bf16 != 0) : zero_f4();
    }
  }
  const float inv_d = 1.f / (float)D;
  float4 dwa[V], dba[V];
#pragma unroll
  for (int k = 0; k < V; ++k) dwa[k] = dba[k] = zero_f4();
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int64_t row = r0 + rr;
    float4 xh[V], g[V];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      // an inactive group has x = dy = 0: its xh = -mu r is finite and meets g = 0 and dy = 0 in every product below
      xh[k] = make_float4((xv[rr][k].x - mu[rr]) * rs[rr], (xv[rr][k].y - mu[rr]) * rs[rr],
                          (xv[rr][k].z - mu[rr]) * rs[rr], (xv[rr][k].w - mu[rr]) * rs[rr]);
      g[k] = make_float4(d[rr][k].x * wv[k].x, d[rr][k].y * wv[k].y, d[rr][k].z * wv[k].z, d[rr][k].w * wv[k].w);
      s1 += (g[k].x + g[k].y) + (g[k].z + g[k].w);
      s2 += (g[k].x * xh[k].x + g[k].y * xh[k].y) + (g[k].z * xh[k].z + g[k].w * xh[k].w);
    }
    const float m1 = ln_wave_total(s1) * inv_d, m2 = ln_wave_total(s2) * inv_d;
    const float r = rs[rr];
    if (row < rows) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const int e = 4 * (l + 64 * k);
        if (e >= D) continue;
        *reinterpret_cast<float4*>(dx + row * D + e) =
            make_float4(r * (g[k].x - m1 - xh[k].x * m2), r * (g[k].y - m1 - xh[k].y * m2),
                        r * (g[k].z - m1 - xh[k].z * m2), r * (g[k].w - m1 - xh[k].w * m2));
      }
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      dwa[k].x += d[rr][k].x * xh[k].x;
      dwa[k].y += d[rr][k].y * xh[k].y;
      dwa[k].z += d[rr][k].z * xh[k].z;
      dwa[k].w += d[rr][k].w * xh[k].w;
      dba[k].x += d[rr][k].x;
      dba[k].y += d[rr][k].y;
      dba[k].z += d[rr][k].z;
      dba[k].w += d[rr][k].w;
    }
  }
  ln_reduce_waves<V>(red, dwa, dwp + (int64_t)blockIdx.x * D, D);
  ln_reduce_waves<V>(red, dba, dbp + (int64_t)blockIdx.x * D, D);
}

bool ln_shape_ok(int64_t rows, int64_t D) {
  return rows > 0 && rows < ((int64_t)1 << 31) && D > 0 && D % 4 == 0 && D <= 2048 && rows * D < ((int64_t)1 << 40);
}

int ln_width(int64_t D) { return (int)((D + 255) / 256); }  // V: the 256-element blocks a row spans

// Backward workgroups, one partial row each: kBwdWaves waves of rows_per_wave(V) rows.
int64_t partial_rows(int64_t rows, int64_t D) {
  const int64_t per = (int64_t)kBwdWaves * rows_per_wave(ln_width(D));
  return (rows + per - 1) / per;
}

template <int V>
int launch_fwd(const float* x, const float* w, const float* b, float eps, void* y, int y_bf16, float* mean,
               float* rstd, int64_t rows, int D, hipStream_t st) {
  hipLaunchKernelGGL(ln_fwd<V>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, eps, y, y_bf16, mean,
                     rstd, rows, D);
  PGN_RETURN_LAUNCH();
}

template <int V>
int launch_bwd(const void* dy, int dy_bf16, const float* x, const float* w, const float* mean, const float* rstd,
               float* dx, float* dwp, float* dbp, int64_t rows, int D, hipStream_t st) {
  hipLaunchKernelGGL(ln_bwd<V>, dim3((unsigned)partial_rows(rows, D)), dim3(64 * kBwdWaves), 0, st, dy, dy_bf16, x,
                     w, mean, rstd, dx, dwp, dbp, rows, D);
  PGN_RETURN_LAUNCH();
}

}  // namespace

extern "C" int64_t pragnosia_layer_norm_partials(int64_t rows, int64_t D) {
  if (!ln_shape_ok(rows, D)) return -1;
  return partial_rows(rows, D);
}

extern "C" int pragnosia_layer_norm_fwd(const float* x, const float* weight, const float* bias, float eps, void* y,
                                        int y_bf16, float* mean, float* rstd, int64_t rows, int64_t D,
                                        void* stream) {
  if (D % 4 != 0 || D > 2048) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(ln_shape_ok(rows, D));
  PGN_CHECK_ARG(x && weight && bias && y && mean && rstd);
  PGN_CHECK_ARG(eps >= 0.f);
  hipStream_t st = (hipStream_t)stream;
  const int d = (int)D;
  switch (ln_width(D)) {
    case 1: return launch_fwd<1>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 2: return launch_fwd<2>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 3: return launch_fwd<3>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 4: return launch_fwd<4>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 5: return launch_fwd<5>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 6: return launch_fwd<6>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    case 7: return launch_fwd<7>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
    default: return launch_fwd<8>(x, weight, bias, eps, y, y_bf16, mean, rstd, rows, d, st);
  }
}

extern "C" int pragnosia_layer_norm_bwd(const void* dy, int dy_bf16, const float* x, const float* weight,
                                        const float* mean, const float* rstd, float* dx, float* dw_partials,
                                        float* db_partials, int64_t rows, int64_t D, void* stream) {
  if (D % 4 != 0 || D > 2048) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(ln_shape_ok(rows, D));
  PGN_CHECK_ARG(dy && x && weight && mean && rstd && dx && dw_partials && db_partials);
  hipStream_t st = (hipStream_t)stream;
  const int d = (int)D;
  switch (ln_width(D)) {
    case 1: return launch_bwd<1>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 2: return launch_bwd<2>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 3: return launch_bwd<3>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 4: return launch_bwd<4>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 5: return launch_bwd<5>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 6: return launch_bwd<6>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    case 7: return launch_bwd<7>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
    default: return launch_bwd<8>(dy, dy_bf16, x, weight, mean, rstd, dx, dw_partials, db_partials, rows, d, st);
  }
}
