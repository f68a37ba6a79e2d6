// The dense layers of the carrier LM's decode step for batches past the one-wave GEMV (5 sequences and more), fp32
// on the matrix cores (v_mfma_f32_16x16x4f32): y = act(scale * (W z) + bias) + resid with z the row standardised,
// (x - mean) / sqrt(var + eps) (MODE 1: a LayerNorm whose weight the caller folds into W's columns and whose bias
// into `bias` as W ln_bias), the per-group RMS scaling x / sqrt(mean x^2 + eps) over groups of 64 or 128 channels
// (MODE 2, mode 2 or 3 at the boundary: the carrier's per-head RMSNorm of its raw step output, its weight folded into
// W's columns) or x (MODE 0). Replaces, inside the graphed decode of `src/bench.py:241-317`, the LayerNorm +
// nn.Linear (+ GELU, + residual) calls of `src/model.py:552-560` and `src/assoc.py:384-512`, one kernel per dense
// layer, as decode_gemv.hip does for at most 4 sequences.
//
// At 64 sequences every weight element is used 64 times a step (32 flop per byte read), so the fp32 matrix-core rate
// matters as much as HBM, and at these sizes a workgroup's own latency (its loads, then its products, then its
// reduction) sets the kernel's time. Work split: a workgroup owns NC column tiles of 16 output columns (NC = 1, or 3
// where that still leaves 192 workgroups: each input piece then feeds three products, a third fewer operand bytes
// per CU from L2) of 16 rows (one row block), all of K: its KW waves (at most 16) split K into 16-wide steps, S
// consecutive steps a chunk and C chunks a wave. So a layer at 64 rows is 4 x ceil(N / 16 NC) workgroups; those of
// one column group are numbered 8 apart, so they run on one XCD (workgroup i goes to XCD i mod 8) and read the
// group's weight from one L2. A wave issues its
// first chunk's loads before any product and each next chunk's loads before the current chunk's products (register
// double buffering): S weight pieces, each one contiguous 1 KiB, and S input pieces. The weight (N, K) comes
// pre-tiled: Wt[((t KS + s) 64 + l) 4 + e] = W[16 t + l % 16][16 s + 4 (l / 16) + e] for column tile t, 16-wide step
// s (KS = K / 16 of them), lane l and entry e, zero for columns past N (tiled once by the caller; ops.decode_gemm_tile).
// MODE 1 needs the row's moments only in the epilogue: the products run on x - x0 (x0 the row's first entry, so the
// subtraction of mean(x - x0) csum below cancels no more than the row's spread; csum[n] = sum_k W[n][k]) while each
// wave forms, per chunk, the mean and the sum of squared deviations of its entries (exact two-pass in registers) and
// merges them (Chan, Golub and LeVeque's pairwise update); the waves' pairs meet in the epilogue, in wave order, with
// the products' partials. MODE 2 (S = 4 or 8, C = 1) has each wave own one group of 16 S channels, so the group's
// sum of squares is a two-step lane exchange before its products. The wave partials are summed through LDS in wave
// order: deterministic, no atomics, nothing shared between workgroups, no workspace. The accumulating form (ACC) splits
// K over groups of workgroups instead (whole channel groups in the RMS mode) and adds each split's sums into the
// output, which holds the residual, with fp32 atomics: more workgroups for the deep layers, not bit-deterministic.
//
// Operand layout of v_mfma_f32_16x16x4f32: A[r][k] in lane r + 16 k, B[k][c] in lane c + 16 k, D[4 g + e][c] in
// lane c + 16 g, e = 0..3. A lane holds four consecutive K entries of a row (one 16-byte piece): product e of a
// 16-wide step contracts entry e of every lane's piece, i.e. k = 16 s + 4 (l / 16) + e; the weight pieces are tiled
// with the same pairing, so every k is contracted exactly once.
#include "common.h"

namespace {

constexpr int MAXW = 16;  // waves per workgroup

// ACC: the K split over SK groups of workgroups (split ks over K range ks K .. ks K + K - 1 of rows of ldx = SK K
// entries), each adding its partial products (and, for split 0, the bias) to y with atomics: y holds the residual.
template <int S, int C, int MODE, int NC, bool ACC>
__global__ __launch_bounds__(1024) void decode_gemm_k(const float* __restrict__ x, int B, int K,
                                                      const float* __restrict__ csum, float eps,
                                                      const float* __restrict__ Wt, int N, int NT, int ZB,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ scale, int act,
                                                      const float* __restrict__ resid, float* __restrict__ y,
                                                      int SK) {
  static_assert(MODE != 2 || C == 1, "the RMS mode holds one channel group per wave");
  static_assert(!ACC || MODE != 1, "the split-K form needs no whole-row statistics");
  __shared__ __align__(16) float red[NC * MAXW * 256];
  __shared__ float2 stat[MAXW][16];
  const int KW = blockDim.x >> 6;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, r16 = l & 15, k4 = l >> 4;
  // workgroup i -> (K split, column group of NC tiles, row block): the ZB row blocks of a group are 8 apart (one XCD)
  const int per_split = (int)(gridDim.x / SK);
  const int ks = ACC ? (int)blockIdx.x / per_split : 0;
  const int i = (int)blockIdx.x - ks * per_split;
  const int ng = (i / (8 * ZB)) * 8 + (i & 7), zb = (i >> 3) % ZB;
  if (ng * NC >= NT) return;  // padding workgroups of the last group of 8
  const int nt0 = ng * NC;    // the group's first column tile
  const int KS = K >> 4, KSt = KS * SK;  // 16-wide steps of this workgroup's K range, of the whole row
  const int s0 = w * S * C;  // the wave's first 16-wide step
  const int row = 16 * zb + r16;
  const bool live = row < B;
  const float* xrow = x + (size_t)min(row, B - 1) * K * SK + (size_t)ks * K;
  const float* xr = xrow + 16 * s0 + 4 * k4;
  const float* wp[NC];  // tiles past the last are read from the last one and not written
#pragma unroll
  for (int t = 0; t < NC; ++t) wp[t] = Wt + ((size_t)min(nt0 + t, NT - 1) * KSt + ks * KS + s0) * 256 + 4 * l;

  f32x4 wv[2][S][NC], z[2][S];
  auto load = [&](int c, int b) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int t = 0; t < NC; ++t) wv[b][s][t] = *reinterpret_cast<const f32x4*>(wp[t] + 256 * (c * S + s));
      const f32x4 v = *reinterpret_cast<const f32x4*>(xr + 16 * (c * S + s));
      z[b][s] = live ? v : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // LayerNorm mode: the products run on the row shifted by its first entry, x - x0 (the shift keeps the products'
  // cancellation against mean * csum at the size of the row's spread); the row's moments are formed beside them
  const float x0 = MODE == 1 && live ? xrow[0] : 0.f;
  load(0, 0);
  // three tiles a workgroup run one workgroup a compute unit (two waves a SIMD): every load of the first chunk is
  // kept ahead of the products, so the wave's whole operand stream is in flight at once
  if constexpr (NC > 1) __builtin_amdgcn_sched_barrier(0);
  float mw = 0.f, m2w = 0.f;  // this wave's mean and sum of squared deviations of the row (LayerNorm mode)
  f32x4 acc[NC];
#pragma unroll
  for (int t = 0; t < NC; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if (c + 1 < C) load(c + 1, (c + 1) & 1);
    const int b = c & 1;
    if constexpr (MODE == 1) {
      // the chunk's 16 S entries of the row (the lane's 4 S and those of lanes l ^ 16, l ^ 32, l ^ 48): their mean
      // and sum of squared deviations, merged into the wave's by the pairwise update (equal counts per chunk)
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) z[b][s][e] -= x0;
      float a = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) a += (z[b][s][0] + z[b][s][1]) + (z[b][s][2] + z[b][s][3]);
      a += __shfl_xor(a, 16);
      a += __shfl_xor(a, 32);
      const float mc = a * (1.f / (16 * S));
      float q = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = z[b][s][e] - mc;
          q += d * d;
        }
      q += __shfl_xor(q, 16);
      q += __shfl_xor(q, 32);
      if (c == 0) {
        mw = mc;
        m2w = q;
      } else {  // merge n = 16 S c entries (mw, m2w) with 16 S new ones (mc, q)
        const float d = mc - mw, f = 1.f / (c + 1);
        mw += d * f;
        m2w += q + d * d * (16.f * S) * c * f;
      }
    } else if constexpr (MODE == 2) {
      // one group of 16 S channels per wave (S = 4 or 8): r = 1 / sqrt(mean of squares + eps) scales the group
      static_assert(S == 4 || S == 8, "the RMS mode runs one 64- or 128-channel group per wave");
      float a = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) a += z[b][s][e] * z[b][s][e];
      a += __shfl_xor(a, 16);
      a += __shfl_xor(a, 32);
      const float r = 1.f / sqrtf(a * (1.f / (16 * S)) + eps);
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) z[b][s][e] *= r;
    }
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int t = 0; t < NC; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(z[b][s][e], wv[b][s][t][e], acc[t], 0, 0, 0);
  }

  // wave partials (and the LayerNorm moments) through LDS; output v = 16 i + c (row i, column c of the block) sits
  // in lane c + 16 (i / 4), entry i % 4
#pragma unroll
  for (int t = 0; t < NC; ++t) *reinterpret_cast<f32x4*>(red + (t * KW + w) * 256 + 4 * l) = acc[t];
  if (MODE == 1 && k4 == 0) stat[w][r16] = float2{mw, m2w};
  __syncthreads();
  for (int v = threadIdx.x; v < 256 * NC; v += blockDim.x) {  // fewer than 4 NC waves take more rounds
    const int tt = v >> 8, ri = (v >> 4) & 15, cc = v & 15;
    const int src = 4 * (cc + 16 * (ri >> 2)) + (ri & 3);
    const float* rt = red + tt * KW * 256;
    float t = 0.f;
    for (int u = 0; u < KW; ++u) t += rt[u * 256 + src];
    const int orow = 16 * zb + ri, col = 16 * (nt0 + tt) + cc;
    if (orow < B && col < N) {
      if constexpr (MODE == 1) {
        // the row's mean (of x - x0) and variance from the waves' pairs in wave order (equal counts); the products
        // of x - x0 minus (mean of x - x0) csum are the products of x - mean
        const float n_w = 16.f * S * C;
        float mean = 0.f;
        for (int u = 0; u < KW; ++u) mean += stat[u][ri].x;
        mean /= KW;
        float m2 = 0.f;
        for (int u = 0; u < KW; ++u) {
          const float2 p = stat[u][ri];
          const float d = p.x - mean;
          m2 += p.y + n_w * d * d;
        }
        t = (t - mean * csum[col]) * (1.f / sqrtf(m2 / K + eps));
      }
      const size_t off = (size_t)orow * N + col;
      if constexpr (ACC) {
        atomicAdd(y + off, (scale ? *scale : 1.f) * t + (bias && ks == 0 ? bias[col] : 0.f));
      } else {
        float r = (scale ? *scale : 1.f) * t + (bias ? bias[col] : 0.f);
        if (act == 1) r = pgn_gelu_erf(r);
        if (resid) r += resid[off];
        y[off] = r;
      }
    }
  }
}

struct Plan {
  int S = 0, C = 0, KW = 0;
};

// The launch shape for (K, mode); false when the kernel does not cover it.
bool make_plan(int64_t K, int mode, Plan& p) {
  if (K <= 0 || K % 16) return false;
  const int64_t KS = K / 16;
  if (mode == 2 || mode == 3) {  // one 64- or 128-channel group per wave
    const int G = mode == 2 ? 64 : 128;
    if (K % G || K / G > MAXW) return false;
    p = Plan{G / 16, 1, (int)(K / G)};
    return true;
  }
  // one chunk a wave when that fits in 16 waves, the chunk as short as that allows (K 768: 16 waves of 3 steps rather
  // than 8 of 6; batch-64 step 0.513 -> 0.487 ms, A/B on one box)
  for (int s : {3, 4, 6})
    if (KS % s == 0 && KS / s <= MAXW) {
      p = Plan{s, 1, (int)(KS / s)};
      return true;
    }
  int S = 1;
  for (int s : {6, 4, 3, 2})
    if (KS % s == 0) {
      S = s;
      break;
    }
  const int64_t R = KS / S;  // chunks to spread over waves: as many waves as allowed, each as few chunks (at 64 rows
                             // and K 3072, 16 waves of 2 chunks took the step 0.608 -> 0.602 ms against 8 of 4)
  for (int c : {1, 2, 4})
    if (R % c == 0 && R / c <= MAXW) {
      p = Plan{S, c, (int)(R / c)};
      return true;
    }
  return false;
}

template <int S, int C, int MODE, int NC, bool ACC = false>
int launch_nc(const Plan& p, const float* x, int B, int K, const float* csum, float eps, const float* Wt, int N,
              const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st,
              int SK = 1) {
  const int NT = (N + 15) / 16, ZB = (B + 15) / 16;
  const int64_t groups = ((NT + NC - 1) / NC + 7) / 8;  // column groups in sets of 8, each set's ZB row blocks together
  hipLaunchKernelGGL((decode_gemm_k<S, C, MODE, NC, ACC>), dim3((unsigned)(groups * 8 * ZB * SK)),
                     dim3((unsigned)(64 * p.KW)), 0, st, x, B, K, csum, eps, Wt, N, NT, ZB, bias, scale, act, resid, y,
                     SK);
  PGN_RETURN_LAUNCH();
}

// Workgroups of three column tiles (each x piece feeds three products: a third fewer operand bytes per CU from L2,
// which is what bounds these layers) when that still leaves this many workgroups; else one tile a workgroup.
constexpr int64_t kWideGroups = 192;

template <int S, int C, int MODE>
int launch(const Plan& p, const float* x, int B, int K, const float* csum, float eps, const float* Wt, int N,
           const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
  if constexpr (C == 1 && MODE < 2) {
    const int64_t NT = (N + 15) / 16, ZB = (B + 15) / 16;
    if (ZB * ((NT + 2) / 3) >= kWideGroups)
      return launch_nc<S, C, MODE, 3>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st);
  }
  return launch_nc<S, C, MODE, 1>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st);
}

template <int C, int MODE>
int dispatch_s(const Plan& p, const float* x, int B, int K, const float* csum, float eps, const float* Wt, int N,
               const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
#define PGN_S(V) return launch<V, C, MODE>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st)
  if constexpr (MODE == 2) {
    if (p.S == 8) PGN_S(8);
    PGN_S(4);
  } else {
    switch (p.S) {
      case 1: PGN_S(1);
      case 2: PGN_S(2);
      case 3: PGN_S(3);
      case 4: PGN_S(4);
      default: PGN_S(6);
    }
  }
#undef PGN_S
}

// The split-K accumulating form: SK splits of Kp = K / SK each; mode 0 with three column tiles a workgroup where that
// still leaves kWideGroups workgroups, the RMS mode (MODE 2, whole channel groups a split) one tile.
template <int S, int C, int MODE>
int launch_acc(const Plan& p, const float* x, int B, int Kp, float eps, const float* Wt, int N, const float* bias,
               const float* scale, float* y, hipStream_t st, int SK) {
  if constexpr (C == 1 && MODE == 0) {
    const int64_t NT = (N + 15) / 16, ZB = (B + 15) / 16;
    if (ZB * ((NT + 2) / 3) * SK >= kWideGroups)
      return launch_nc<S, C, 0, 3, true>(p, x, B, Kp, nullptr, 0.f, Wt, N, bias, scale, 0, nullptr, y, st, SK);
  }
  return launch_nc<S, C, MODE, 1, true>(p, x, B, Kp, nullptr, eps, Wt, N, bias, scale, 0, nullptr, y, st, SK);
}

template <int C>
int acc_s(const Plan& p, const float* x, int B, int Kp, const float* Wt, int N, const float* bias,
          const float* scale, float* y, hipStream_t st, int SK) {
  switch (p.S) {
    case 1: return launch_acc<1, C, 0>(p, x, B, Kp, 0.f, Wt, N, bias, scale, y, st, SK);
    case 2: return launch_acc<2, C, 0>(p, x, B, Kp, 0.f, Wt, N, bias, scale, y, st, SK);
    case 3: return launch_acc<3, C, 0>(p, x, B, Kp, 0.f, Wt, N, bias, scale, y, st, SK);
    case 4: return launch_acc<4, C, 0>(p, x, B, Kp, 0.f, Wt, N, bias, scale, y, st, SK);
    default: return launch_acc<6, C, 0>(p, x, B, Kp, 0.f, Wt, N, bias, scale, y, st, SK);
  }
}

// K split for the accumulating form. Mode 0: four or two splits when each keeps at least 512 of K (whole 16-wide
// steps). RMS modes (groups of G channels): the most splits, of at most four, that keep whole groups and at least
// four of them a split (each group is one wave of the split's workgroup). At 64 rows and 12 heads of 64, batch-64
// step on one box: one split 0.4853 ms, two of six heads 0.4856-0.4860, three of four 0.4815, four of three
// 0.4837-0.4840.
constexpr int64_t kRmsSplitGroups = 4;
int acc_splits(int64_t K, int mode) {
  if (mode >= 2) {
    const int64_t G = mode == 2 ? 64 : 128;
    if (K % G) return 1;
    for (int c : {4, 3, 2})
      if ((K / G) % c == 0 && K / G / c >= kRmsSplitGroups) return c;
    return 1;
  }
  for (int c : {4, 2})
    if (K % (16 * c) == 0 && K / c >= 512) return c;
  return 1;
}

}  // namespace

extern "C" int pragnosia_decode_gemm_waves(int64_t K, int mode) {
  Plan p;
  if (mode < 0 || mode > 3 || !make_plan(K, mode, p)) return -1;
  return p.KW;
}

template <int MODE>
int dispatch_c(const Plan& p, const float* x, int B, int K, const float* csum, float eps, const float* Wt, int N,
               const float* bias, const float* scale, int act, const float* resid, float* y, hipStream_t st) {
  switch (p.C) {
    case 1: return dispatch_s<1, MODE>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st);
    case 2: return dispatch_s<2, MODE>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st);
    default: return dispatch_s<4, MODE>(p, x, B, K, csum, eps, Wt, N, bias, scale, act, resid, y, st);
  }
}

extern "C" int pragnosia_decode_gemm(const float* x, int64_t B, int64_t K, int mode, const float* csum, float eps,
                                     const float* Wt, int64_t N, const float* bias, const float* scale, int act,
                                     const float* resid, float* y, void* stream) {
  PGN_CHECK_ARG(x && Wt && y && B > 0 && K > 0 && N > 0);
  PGN_CHECK_ARG(mode >= 0 && mode <= 3 && (mode != 1 || csum != nullptr));
  PGN_CHECK_ARG(B * N < ((int64_t)1 << 31) && B * K < ((int64_t)1 << 31) &&
                ((N + 15) / 16) * 16 * K < ((int64_t)1 << 31) && ((N + 127) / 128) * 8 * ((B + 15) / 16) < (1 << 30));
  PGN_CHECK_ARG(act == 0 || act == 1);
  PGN_CHECK_ARG(y != x && (resid == nullptr || resid != y));
  PGN_CHECK_ARG(((uintptr_t)x | (uintptr_t)Wt) % 16 == 0);
  Plan p;
  if (!make_plan(K, mode, p)) return PRAGNOSIA_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int b = (int)B, k = (int)K, n = (int)N;
  if (mode == 1) return dispatch_c<1>(p, x, b, k, csum, eps, Wt, n, bias, scale, act, resid, y, st);
  if (mode >= 2) return dispatch_s<1, 2>(p, x, b, k, nullptr, eps, Wt, n, bias, scale, act, resid, y, st);
  return dispatch_c<0>(p, x, b, k, nullptr, eps, Wt, n, bias, scale, act, resid, y, st);
}

extern "C" int pragnosia_decode_gemm_acc(const float* x, int64_t B, int64_t K, int mode, float eps, const float* Wt,
                                         int64_t N, const float* bias, const float* scale, float* y, void* stream) {
  PGN_CHECK_ARG(x && Wt && y && B > 0 && K > 0 && N > 0);
  PGN_CHECK_ARG(mode == 0 || mode == 2 || mode == 3);
  PGN_CHECK_ARG(B * N < ((int64_t)1 << 31) && B * K < ((int64_t)1 << 31) &&
                ((N + 15) / 16) * 16 * K < ((int64_t)1 << 31) && ((N + 127) / 128) * 8 * ((B + 15) / 16) < (1 << 27));
  PGN_CHECK_ARG(((uintptr_t)x | (uintptr_t)Wt) % 16 == 0);
  // the atomics into y run while other workgroups still read x
  const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
  PGN_CHECK_ARG(xa + (uintptr_t)(B * K * 4) <= ya || ya + (uintptr_t)(B * N * 4) <= xa);
  const int SK = acc_splits(K, mode);
  Plan p;
  if (!make_plan(K / SK, mode, p)) return PRAGNOSIA_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int b = (int)B, kp = (int)(K / SK), n = (int)N;
  if (mode >= 2) {  // one G-channel group a wave (S = G / 16)
    if (p.S == 8) return launch_acc<8, 1, 2>(p, x, b, kp, eps, Wt, n, bias, scale, y, st, SK);
    return launch_acc<4, 1, 2>(p, x, b, kp, eps, Wt, n, bias, scale, y, st, SK);
  }
  switch (p.C) {
    case 1: return acc_s<1>(p, x, b, kp, Wt, n, bias, scale, y, st, SK);
    case 2: return acc_s<2>(p, x, b, kp, Wt, n, bias, scale, y, st, SK);
    default: return acc_s<4>(p, x, b, kp, Wt, n, bias, scale, y, st, SK);
  }
}
