// The dense layers of the carrier LM's single-token decode step, batched over B sequences, fp32 (the reference
// decodes in fp32 without autocast): y = act(scale * (W z) + bias) + resid, with z = LayerNorm(x) (weight, bias,
// eps) or z = x, act = identity or GELU (erf form), all optional parts NULL. One call per dense layer of the step:
// the carrier's input projections (LayerNorm + one concatenated projection), its gated output projection with the
// residual, the MLP's first layer (LayerNorm + bias + GELU) and second (bias + residual), and the tied head
// (LayerNorm). Replaces the torch calls of `src/model.py:552-560` and `src/assoc.py:384-512` inside the graphed
// decode of `src/bench.py:241-317`, one kernel each instead of three to six.
//
// At decode batch sizes the weight read is the whole cost (each weight read once per step). Up to 4 sequences (and K
// a multiple of 256) the one-wave kernel gemv_wave below runs; beyond, a workgroup owns a few output rows and all B
// sequences: thread (r, l) reads 16-byte pieces 4 l + 4 LANES i of weight row r (a row
// is read by LANES consecutive lanes, 16 * LANES contiguous bytes per instruction), twelve pieces at a time held in
// registers (all issued before the first is used), and accumulates 8 sequences at a time; the LayerNorm'd inputs of
// those 8 sequences sit in LDS. The first weight pieces are loaded before the LayerNorm, whose row is held in
// registers (one read of x). Each group of 8 sequences is its own row of workgroups (the weight is then read once
// from HBM and again from the last-level cache). LANES = 64 for narrow outputs (more workgroups) or long rows, 16
// otherwise.
#include <algorithm>

#include "common.h"

namespace {

constexpr int BT = 8;            // sequences per pass
constexpr int LNMAX = 1024;      // LayerNorm'd inputs are staged in LDS for K <= LNMAX

template <int LANES>
__global__ __launch_bounds__(256) void gemv(const float* __restrict__ x, int B, int K, const float* __restrict__ lnw,
                                            const float* __restrict__ lnb, float eps, const float* __restrict__ W,
                                            int N, const float* __restrict__ bias,
                                            const float* __restrict__ scale, int act,
                                            const float* __restrict__ resid, float* __restrict__ y) {
  constexpr int ROWS = 256 / LANES;
  constexpr int NW = 12;                 // 16-byte weight pieces per thread held in registers per K chunk
  constexpr int KC = NW * 4 * LANES;     // K chunk
  constexpr int LV = LNMAX / 128;        // 16-byte pieces of one LayerNorm row per lane (32 lanes a row)
  __shared__ __align__(16) float zs[BT * LNMAX];  // the LayerNorm'd inputs of one pass
  const int tid = threadIdx.x, r = tid / LANES, l = tid % LANES;
  const int n = blockIdx.x * ROWS + r;
  const bool ln = lnw != nullptr;
  const float* wr = W + (size_t)min(n, N - 1) * K;
  f32x4 w4[NW];
  auto load_w = [&](int kc) {
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const int k = kc + 4 * l + 4 * LANES * u;
      w4[u] = k < K ? *reinterpret_cast<const f32x4*>(wr + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // the first chunk's weights are in flight while the LayerNorm below runs
  load_w(0);
  const float sc = scale ? *scale : 1.f;
  for (int b0 = blockIdx.y * BT; b0 < B; b0 += BT * gridDim.y) {
    const int nb = min(BT, B - b0);
    if (ln) {
      // row rr of the pass by 32 lanes, held in registers: mean, then the variance about it, then z into LDS
      __syncthreads();
      const int rr = tid / 32, ll = tid % 32;
      if (rr < nb) {
        const float* xr = x + (size_t)(b0 + rr) * K;
        f32x4 xv[LV];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < LV; ++i) {
          const int k = 4 * ll + 128 * i;
          xv[i] = k < K ? *reinterpret_cast<const f32x4*>(xr + k) : f32x4{0.f, 0.f, 0.f, 0.f};
          s += (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);
        }
        for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
        const float mean = s / K;
        float s2 = 0.f;
#pragma unroll
        for (int i = 0; i < LV; ++i) {
          if (4 * ll + 128 * i < K) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float d = xv[i][e] - mean;
              s2 += d * d;
            }
          }
        }
        for (int o = 16; o > 0; o >>= 1) s2 += __shfl_xor(s2, o, 32);
        const float rs = 1.f / sqrtf(s2 / K + eps);
#pragma unroll
        for (int i = 0; i < LV; ++i) {
          const int k = 4 * ll + 128 * i;
          if (k < K) {
            const f32x4 g = *reinterpret_cast<const f32x4*>(lnw + k);
            const f32x4 c = lnb ? *reinterpret_cast<const f32x4*>(lnb + k) : f32x4{0.f, 0.f, 0.f, 0.f};
            f32x4 z;
#pragma unroll
            for (int e = 0; e < 4; ++e) z[e] = (xv[i][e] - mean) * rs * g[e] + c[e];
            *reinterpret_cast<f32x4*>(zs + rr * K + k) = z;
          }
        }
      }
      __syncthreads();
    }
    float acc[BT];
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[b] = 0.f;
    for (int kc = 0; kc < K; kc += KC) {
      if (kc > 0 || b0 != (int)blockIdx.y * BT) load_w(kc);
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        if (b < nb) {
          const float* zr = ln ? zs + b * K : x + (size_t)(b0 + b) * K;
          float a = 0.f;
#pragma unroll
          for (int u = 0; u < NW; ++u) {
            const int k = kc + 4 * l + 4 * LANES * u;
            if (k < K) {
              const f32x4 z4 = *reinterpret_cast<const f32x4*>(zr + k);
              a += w4[u][0] * z4[0] + w4[u][1] * z4[1] + w4[u][2] * z4[2] + w4[u][3] * z4[3];
            }
          }
          acc[b] += a;
        }
      }
    }
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      float v = acc[b];
      for (int o = LANES / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LANES);
      acc[b] = v;
    }
    if (l == 0 && n < N) {
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        if (b < nb) {
          float v = sc * acc[b] + (bias ? bias[n] : 0.f);
          if (act == 1) v = pgn_gelu_erf(v);
          const size_t off = (size_t)(b0 + b) * N + n;
          if (resid) v += resid[off];
          y[off] = v;
        }
      }
    }
  }
}

// The decode GEMV for B <= 4 sequences and K = 256 KV: one wave per RPW output rows (a one-wave workgroup, so
// hundreds to thousands of them cover the chip and one round of loads covers the whole weight). Lane l reads the
// 16-byte pieces 4 l + 256 u of each of its rows, so one load instruction reads 1 KiB contiguous; all RPW KV pieces
// are issued before the inputs are read. The input is used as is (MODE 0), LayerNorm'd (MODE 1: the wave computes
// the LayerNorm of every input row itself, the row in registers, two wave reductions), or RMS-normalised per group
// of 64 or 128 channels (MODE 2 or 3: the carrier's per-head RMSNorm; a group's channels sit on 16 or 32 consecutive
// lanes of one piece, so its sum of squares is a four- or five-step exchange). No LDS, no barrier. NB = 1 (B = 1) or 4 (B <= 4, rows past
// B masked).
template <int RPW, int NB, int KV, int MODE>
__global__ __launch_bounds__(64) void gemv_wave(const float* __restrict__ x, int B, const float* __restrict__ lnw,
                                                const float* __restrict__ lnb, float eps, const float* __restrict__ W,
                                                int N, const float* __restrict__ bias,
                                                const float* __restrict__ scale, int act,
                                                const float* __restrict__ resid, float* __restrict__ y) {
  constexpr int K = 256 * KV;
  const int l = threadIdx.x;
  const int n0 = blockIdx.x * RPW;
  f32x4 w[RPW][KV];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float* wr = W + (size_t)min(n0 + r, N - 1) * K + 4 * l;
#pragma unroll
    for (int u = 0; u < KV; ++u) w[r][u] = *reinterpret_cast<const f32x4*>(wr + 256 * u);
  }
  float acc[RPW * NB];
#pragma unroll
  for (int m = 0; m < RPW * NB; ++m) acc[m] = 0.f;
  if constexpr (MODE != 0) {
    f32x4 z[NB][KV];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int u = 0; u < KV; ++u)
        z[b][u] = b < B ? *reinterpret_cast<const f32x4*>(x + (size_t)b * K + 4 * l + 256 * u)
                        : f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == 1) {
      f32x4 g[KV], c[KV];
#pragma unroll
      for (int u = 0; u < KV; ++u) {
        g[u] = *reinterpret_cast<const f32x4*>(lnw + 4 * l + 256 * u);
        c[u] = lnb ? *reinterpret_cast<const f32x4*>(lnb + 4 * l + 256 * u) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < KV; ++u) s += (z[b][u][0] + z[b][u][1]) + (z[b][u][2] + z[b][u][3]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        const float mean = s * (1.f / K);
        float s2 = 0.f;
#pragma unroll
        for (int u = 0; u < KV; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d = z[b][u][e] - mean;
            s2 += d * d;
          }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s2 += __shfl_xor(s2, o);
        const float rs = 1.f / sqrtf(s2 * (1.f / K) + eps);
#pragma unroll
        for (int u = 0; u < KV; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) z[b][u][e] = (z[b][u][e] - mean) * rs * g[u][e] + c[u][e];
      }
    } else {
      // channels 4 (l mod GL) .. + 3 of a G-channel group: the group weight piece is the same for every u
      constexpr int G = MODE == 3 ? 128 : 64, GL = G / 4;
      const f32x4 g = *reinterpret_cast<const f32x4*>(lnw + 4 * (l & (GL - 1)));
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int u = 0; u < KV; ++u) {
          float s = (z[b][u][0] * z[b][u][0] + z[b][u][1] * z[b][u][1]) +
                    (z[b][u][2] * z[b][u][2] + z[b][u][3] * z[b][u][3]);
#pragma unroll
          for (int o = 1; o < GL; o <<= 1) s += __shfl_xor(s, o);
          const float rs = 1.f / sqrtf(s * (1.f / G) + eps);
#pragma unroll
          for (int e = 0; e < 4; ++e) z[b][u][e] = (z[b][u][e] * rs) * g[e];
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int u = 0; u < KV; ++u)
          acc[r * NB + b] += w[r][u][0] * z[b][u][0] + w[r][u][1] * z[b][u][1] + w[r][u][2] * z[b][u][2] +
                             w[r][u][3] * z[b][u][3];
  } else {
#pragma unroll
    for (int u = 0; u < KV; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const f32x4 z = b < B ? *reinterpret_cast<const f32x4*>(x + (size_t)b * K + 4 * l + 256 * u)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < RPW; ++r)
          acc[r * NB + b] += w[r][u][0] * z[0] + w[r][u][1] * z[1] + w[r][u][2] * z[2] + w[r][u][3] * z[3];
      }
  }
  constexpr int NV = RPW * NB;
  wave_sum_many<NV>(acc, l);
  constexpr int sh = 6 - log2_of<NV>();
  if ((l & ((1 << sh) - 1)) == 0) {
    const int m = l >> sh, r = m / NB, b = m % NB;
    const int n = n0 + r;
    if (n < N && b < B) {
      float v = (scale ? *scale : 1.f) * acc[0] + (bias ? bias[n] : 0.f);
      if (act == 1) v = pgn_gelu_erf(v);
      const size_t off = (size_t)b * N + n;
      if (resid) v += resid[off];
      y[off] = v;
    }
  }
}

// The accumulating GEMV (no normalisation) for B <= 4: y[b][n] += scale * (W x_b)[n] + bias[n], K = 256 KV split
// SK ways: workgroup (n, ks) of one wave reads the pieces 4 l + 256 u, u in [ks KV, ks KV + KV), of row n and of each
// input row, sums them over the wave and adds into y (which holds the residual) with an fp32 atomic, the bias with the
// first split. SK times the workgroups of gemv_wave, each a 1 / SK share of the row.
template <int NB, int KV>
__global__ __launch_bounds__(64) void gemv_wave_acc(const float* __restrict__ x, int B, int K,
                                                    const float* __restrict__ W, int N,
                                                    const float* __restrict__ bias,
                                                    const float* __restrict__ scale, float* __restrict__ y) {
  const int l = threadIdx.x;
  const int n = blockIdx.x % N, ks = blockIdx.x / N;
  const float* wr = W + (size_t)n * K + 256 * KV * ks + 4 * l;
  f32x4 w[KV];
#pragma unroll
  for (int u = 0; u < KV; ++u) w[u] = *reinterpret_cast<const f32x4*>(wr + 256 * u);
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.f;
#pragma unroll
  for (int u = 0; u < KV; ++u)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const f32x4 z = b < B ? *reinterpret_cast<const f32x4*>(x + (size_t)b * K + 256 * KV * ks + 4 * l + 256 * u)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
      acc[b] += w[u][0] * z[0] + w[u][1] * z[1] + w[u][2] * z[2] + w[u][3] * z[3];
    }
  wave_sum_many<NB>(acc, l);
  constexpr int sh = 6 - log2_of<NB>();
  if ((l & ((1 << sh) - 1)) == 0) {
    const int b = l >> sh;
    if (b < B) atomicAdd(y + (size_t)b * N + n, (scale ? *scale : 1.f) * acc[0] + (bias && ks == 0 ? bias[n] : 0.f));
  }
}

template <int RPW, int NB, int KV, int MODE>
int launch_wave(const float* x, int B, const float* lnw, const float* lnb, float eps, const float* W, int N,
                const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
  hipLaunchKernelGGL((gemv_wave<RPW, NB, KV, MODE>), dim3((unsigned)((N + RPW - 1) / RPW)), dim3(64), 0, st, x, B,
                     lnw, lnb, eps, W, N, bias, scale, act, resid, y);
  PGN_RETURN_LAUNCH();
}

template <int RPW, int NB, int MODE>
int dispatch_kv(int KV, const float* x, int B, const float* lnw, const float* lnb, float eps, const float* W, int N,
                const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
#define PGN_KV(V) return launch_wave<RPW, NB, V, MODE>(x, B, lnw, lnb, eps, W, N, bias, scale, act, resid, y, st)
  if constexpr (MODE != 0) {
    switch (KV) {
      case 1: PGN_KV(1);
      case 2: PGN_KV(2);
      case 3: PGN_KV(3);
      default: PGN_KV(4);
    }
  } else {
    switch (KV) {
      case 1: PGN_KV(1);
      case 2: PGN_KV(2);
      case 3: PGN_KV(3);
      case 4: PGN_KV(4);
      case 8: PGN_KV(8);
      case 12: PGN_KV(12);
      default: PGN_KV(16);
    }
  }
#undef PGN_KV
}

template <int RPW, int MODE>
int dispatch_nb(int KV, const float* x, int B, const float* lnw, const float* lnb, float eps, const float* W, int N,
                const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
  return B == 1 ? dispatch_kv<RPW, 1, MODE>(KV, x, B, lnw, lnb, eps, W, N, bias, scale, act, resid, y, st)
                : dispatch_kv<RPW, 4, MODE>(KV, x, B, lnw, lnb, eps, W, N, bias, scale, act, resid, y, st);
}

template <int MODE>
int dispatch_rpw(int KV, const float* x, int B, const float* lnw, const float* lnb, float eps, const float* W,
                 int N, const float* bias, const float* scale, int act, const float* resid, float* y,
                 hipStream_t st) {
  // one row a wave up to 4096 rows (768-4096 one-wave workgroups), 4 beyond: batch-1 step 0.2783 -> 0.2766 ms against
  // 2 rows a wave from 1025 rows (A/B twice on one box; 2 rows a wave past 4096 rows measured the same)
  if (N <= 4096) return dispatch_nb<1, MODE>(KV, x, B, lnw, lnb, eps, W, N, bias, scale, act, resid, y, st);
  return dispatch_nb<4, MODE>(KV, x, B, lnw, lnb, eps, W, N, bias, scale, act, resid, y, st);
}

bool wave_shape_ok(int64_t B, int64_t K, bool ln) {
  if (B > 4 || K % 256) return false;
  const int64_t KV = K / 256;
  if (ln) return KV >= 1 && KV <= 4;
  return (KV >= 1 && KV <= 4) || KV == 8 || KV == 12 || KV == 16;
}

}  // namespace

extern "C" int pragnosia_decode_gemv(const float* x, int64_t B, int64_t K, const float* ln_weight,
                                     const float* ln_bias, float ln_eps, const float* W, int64_t N,
                                     const float* bias, const float* scale, int act, const float* resid, float* y,
                                     void* stream) {
  PGN_CHECK_ARG(x && W && y && B > 0 && K > 0 && N > 0 && K % 4 == 0);
  PGN_CHECK_ARG(B * N < ((int64_t)1 << 31) && B * K < ((int64_t)1 << 31));
  PGN_CHECK_ARG(act == 0 || act == 1);
  PGN_CHECK_ARG(ln_weight == nullptr || K <= LNMAX);
  PGN_CHECK_ARG(y != x && (resid == nullptr || resid != y));
  PGN_CHECK_ARG(((uintptr_t)x | (uintptr_t)W | (uintptr_t)ln_weight | (uintptr_t)ln_bias) % 16 == 0);
  hipStream_t st = (hipStream_t)stream;
  const bool ln = ln_weight != nullptr;
  if (wave_shape_ok(B, K, ln))
    return ln ? dispatch_rpw<1>((int)(K / 256), x, (int)B, ln_weight, ln_bias, ln_eps, W, (int)N, bias, scale, act,
                                resid, y, st)
              : dispatch_rpw<0>((int)(K / 256), x, (int)B, ln_weight, ln_bias, ln_eps, W, (int)N, bias, scale, act,
                                resid, y, st);
  const unsigned tiles = (unsigned)std::min<int64_t>((B + BT - 1) / BT, 65535);  // one workgroup row per 8 sequences
  if (N < 2048 || K > 768) {  // 64 lanes a row: more workgroups for narrow outputs, fewer chunks for long rows
    hipLaunchKernelGGL(gemv<64>, dim3((unsigned)((N + 3) / 4), tiles), dim3(256), 0, st, x, (int)B, (int)K, ln_weight,
                       ln_bias, ln_eps, W, (int)N, bias, scale, act, resid, y);
  } else {
    hipLaunchKernelGGL(gemv<16>, dim3((unsigned)((N + 15) / 16), tiles), dim3(256), 0, st, x, (int)B, (int)K, ln_weight,
                       ln_bias, ln_eps, W, (int)N, bias, scale, act, resid, y);
  }
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_decode_gemv_rms(const float* x, int64_t B, int64_t K, const float* rms_weight, int64_t group,
                                         float rms_eps, const float* W, int64_t N, const float* bias,
                                         const float* scale, int act, const float* resid, float* y, void* stream) {
  PGN_CHECK_ARG(x && W && y && rms_weight && B > 0 && K > 0 && N > 0 && (group == 64 || group == 128));
  PGN_CHECK_ARG(B * N < ((int64_t)1 << 31) && B * K < ((int64_t)1 << 31));
  PGN_CHECK_ARG(act == 0 || act == 1);
  PGN_CHECK_ARG(y != x && (resid == nullptr || resid != y));
  PGN_CHECK_ARG(((uintptr_t)x | (uintptr_t)W | (uintptr_t)rms_weight) % 16 == 0);
  if (!wave_shape_ok(B, K, true)) return PRAGNOSIA_ERR_UNSUPPORTED;
  if (group == 128)
    return dispatch_rpw<3>((int)(K / 256), x, (int)B, rms_weight, nullptr, rms_eps, W, (int)N, bias, scale, act,
                           resid, y, (hipStream_t)stream);
  return dispatch_rpw<2>((int)(K / 256), x, (int)B, rms_weight, nullptr, rms_eps, W, (int)N, bias, scale, act, resid,
                         y, (hipStream_t)stream);
}

// K split of the accumulating GEMV: two when that keeps at least 3 pieces a lane (768 of K), else none. At batch 1 on
// the d 768 LM (K 3072), step 0.2653 ms with the residual-epilogue GEMV, 0.2612-0.2624 unsplit in place, 0.2612-0.2615
// with two splits, 0.2648 with three, 0.2687-0.2691 with four (variant builds, one box, A/B twice).
extern "C" int pragnosia_decode_gemv_acc(const float* x, int64_t B, int64_t K, const float* W, int64_t N,
                                         const float* bias, const float* scale, float* y, void* stream) {
  PGN_CHECK_ARG(x && W && y && B > 0 && B <= 4 && K > 0 && N > 0 && K % 256 == 0 && K <= 4096);
  PGN_CHECK_ARG(N * 4 < ((int64_t)1 << 31) && B * K < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31));
  PGN_CHECK_ARG(((uintptr_t)x | (uintptr_t)W) % 16 == 0);
  // the atomics into y run while other workgroups still read x
  const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
  PGN_CHECK_ARG(xa + (uintptr_t)(B * K * 4) <= ya || ya + (uintptr_t)(B * N * 4) <= xa);
  const int KV = (int)(K / 256);
  const int SK = KV % 2 == 0 && KV / 2 >= 3 ? 2 : 1;
  const int kv = KV / SK;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(N * SK));
#define PGN_ACC_KV(V)                                                                                              \
  if (kv == V) {                                                                                                   \
    if (B == 1)                                                                                                    \
      hipLaunchKernelGGL((gemv_wave_acc<1, V>), grid, dim3(64), 0, st, x, (int)B, (int)K, W, (int)N, bias, scale, y); \
    else                                                                                                           \
      hipLaunchKernelGGL((gemv_wave_acc<4, V>), grid, dim3(64), 0, st, x, (int)B, (int)K, W, (int)N, bias, scale, y); \
    PGN_RETURN_LAUNCH();                                                                                           \
  }
  PGN_ACC_KV(1)
  PGN_ACC_KV(2)
  PGN_ACC_KV(3)
  PGN_ACC_KV(4)
  PGN_ACC_KV(5)
  PGN_ACC_KV(6)
  PGN_ACC_KV(7)
  PGN_ACC_KV(8)
  PGN_ACC_KV(9)
  PGN_ACC_KV(10)
  PGN_ACC_KV(11)
  PGN_ACC_KV(12)
  PGN_ACC_KV(13)
  PGN_ACC_KV(14)
  PGN_ACC_KV(15)
  PGN_ACC_KV(16)
#undef PGN_ACC_KV
  return PRAGNOSIA_ERR_UNSUPPORTED;
}
