// Complex diagonal recurrence h_t = lambda_t h_{t-1} + u_t with per-token lambda_t = exp(logmag_t + i ang_t):
// forward and adjoint backward, parallel over time.
//
// The recurrence composes associatively: a segment of tokens acts on its incoming state as the affine map
// h -> P h + e, P = prod lambda_t (|P| <= 1), e = the segment's own contribution from zero. One workgroup owns
// CH channels of one sequence (a wave = CH channels x 64/CH time segments; with CH = 64 every load instruction
// reads one 256-byte row segment of the D-fastest layout) and walks time in blocks of (64/CH) * NW * SEG tokens:
//   1. each lane takes its segment (SEG tokens of one channel, loaded during the previous block), forms lambda in
//      registers, issues the loads of its segment in the next block, and scans the current one from zero, giving
//      the segment's map (P, e);
//   2. the maps go to LDS; after one barrier every lane folds the maps of the segments before it into the
//      block's carry-in to get its own incoming state (reading the maps four at a time, so the LDS latency is paid
//      once per four segments rather than once per segment);
//   3. the lane re-runs its SEG steps from that state out of registers and writes h.
// The block carry and the map buffers are double-buffered, so each time block costs one barrier. Nothing is
// re-read from HBM: the forward moves 20 B per (b, t, d) element, the backward 32 B.
//
// The backward is the same scan run in reverse on the adjoint a_t = g_t + conj(lambda_{t+1}) a_{t+1} (the
// transpose of multiplication by lambda is multiplication by its conjugate), followed per token by
//   du_t = Re a_t,  dlogmag_t = a_t . (lambda_t h_{t-1}),  dang_t = a_t . (i lambda_t h_{t-1}),
// with (x . y) the real inner product of the complex numbers as 2-vectors. The final-state gradients enter as
// the carry into t = T-1; the carry out of t = 0 is dh0. This restates `src/scan_kernel.py:12-17`.
#include "common.h"

namespace {


struct SegMaps {
  float pr, pi, er, ei;
};

// segment maps folded per batch of LDS reads (swept 1-16 at B16 T512 D768: 4 is fastest, 23.5 -> 21.8 us forward)
constexpr int kFold = 4;

template <int NW, int SEG, int CH>
__global__ __launch_bounds__(NW * 64) void diag_fwd_kernel(
    const float* __restrict__ u, const float* __restrict__ lm, const float* __restrict__ an,
    const float* __restrict__ h0r, const float* __restrict__ h0i, float* __restrict__ hr,
    float* __restrict__ hi, float* __restrict__ hr_last, float* __restrict__ hi_last, int T, int D, int n_ctile) {
  constexpr int SPW = 64 / CH;  // time segments per wave
  constexpr int NSEG = SPW * NW;
  constexpr int TB = NSEG * SEG;
  __shared__ SegMaps maps[2][NSEG][CH];
  __shared__ float2 carry[2][CH];

  const int lane = threadIdx.x & 63;
  const int c = lane % CH;
  const int seg = SPW * (threadIdx.x >> 6) + lane / CH;
  const int b = blockIdx.x / n_ctile;
  const int d = (blockIdx.x - b * n_ctile) * CH + c;
  const bool dok = d < D;
  const size_t base = (size_t)b * T * D + (dok ? d : 0);

  if (threadIdx.x < CH) {
    float2 h = make_float2(0.f, 0.f);
    if (h0r != nullptr && dok) h = make_float2(h0r[(size_t)b * D + d], h0i[(size_t)b * D + d]);
    carry[0][c] = h;
  }

  // raw inputs of the next time block, loaded one block ahead so the loads overlap the current block's compute
  float pu[SEG], pl[SEG], pa[SEG];
  auto fetch = [&](int tb) {
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      const int t = tb + seg * SEG + j;
      const bool ok = dok && t < T;
      const size_t off = base + (size_t)(ok ? t : 0) * D;
      pu[j] = ok ? u[off] : 0.f;
      pl[j] = ok ? lm[off] : 0.f;
      pa[j] = ok ? an[off] : 0.f;
    }
  };
  fetch(0);

  for (int tb = 0, it = 0; tb < T; tb += TB, ++it) {
    const int p = it & 1;
    const int t0 = tb + seg * SEG;
    float xr[SEG], xi[SEG], xu[SEG];
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      xu[j] = pu[j];
      const float m = pgn_exp(pl[j]);
      float s, co;
      pgn_sincos(pa[j], &s, &co);
      xr[j] = m * co;
      xi[j] = m * s;
    }
    if (tb + TB < T) fetch(tb + TB);
    // the segment's map from a zero state
    float er = 0.f, ei = 0.f, pr = 1.f, pi = 0.f;
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      const float nr = xr[j] * er - xi[j] * ei + xu[j];
      const float ni = xi[j] * er + xr[j] * ei;
      er = nr;
      ei = ni;
      const float qr = xr[j] * pr - xi[j] * pi;
      const float qi = xi[j] * pr + xr[j] * pi;
      pr = qr;
      pi = qi;
    }
    maps[p][seg][c] = SegMaps{pr, pi, er, ei};
    __syncthreads();
    // incoming state: the block carry pushed through every earlier segment's map, the maps read kFold at a time
    // (reads issued together, one wait per batch rather than one per segment)
    float2 h = carry[p][c];
#pragma unroll
    for (int s0 = 0; s0 < NSEG - 1; s0 += kFold) {
      if (s0 >= seg) break;  // seg is the wave index (64 channels a wave): a uniform branch
      SegMaps m[kFold];
#pragma unroll
      for (int r = 0; r < kFold; ++r) m[r] = maps[p][min(s0 + r, NSEG - 1)][c];
#pragma unroll
      for (int r = 0; r < kFold; ++r) {
        if (s0 + r < seg) {
          const float nr = m[r].pr * h.x - m[r].pi * h.y + m[r].er;
          const float ni = m[r].pi * h.x + m[r].pr * h.y + m[r].ei;
          h = make_float2(nr, ni);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      const float nr = xr[j] * h.x - xi[j] * h.y + xu[j];
      const float ni = xi[j] * h.x + xr[j] * h.y;
      h = make_float2(nr, ni);
      const int t = t0 + j;
      if (dok && t < T) {
        hr[base + (size_t)t * D] = h.x;
        hi[base + (size_t)t * D] = h.y;
      }
    }
    if (seg == NSEG - 1) carry[p ^ 1][c] = h;
    if (tb + TB >= T && t0 <= T - 1 && T - 1 < t0 + SEG && dok && hr_last != nullptr) {
      hr_last[(size_t)b * D + d] = h.x;  // this lane's segment holds token T-1: the final state
      hi_last[(size_t)b * D + d] = h.y;
    }
  }
}

template <int NW, int SEG, int CH>
__global__ __launch_bounds__(NW * 64) void diag_bwd_kernel(
    const float* __restrict__ g, const float* __restrict__ glr, const float* __restrict__ gli,
    const float* __restrict__ lm, const float* __restrict__ an, const float* __restrict__ hr,
    const float* __restrict__ hi, const float* __restrict__ h0r, const float* __restrict__ h0i,
    float* __restrict__ du, float* __restrict__ dlm, float* __restrict__ dan, float* __restrict__ dh0r,
    float* __restrict__ dh0i, int T, int D, int n_ctile) {
  constexpr int SPW = 64 / CH;
  constexpr int NSEG = SPW * NW;
  constexpr int TB = NSEG * SEG;
  __shared__ SegMaps maps[2][NSEG][CH];
  __shared__ float2 carry[2][CH];

  const int lane = threadIdx.x & 63;
  const int c = lane % CH;
  const int seg = SPW * (threadIdx.x >> 6) + lane / CH;
  const int b = blockIdx.x / n_ctile;
  const int d = (blockIdx.x - b * n_ctile) * CH + c;
  const bool dok = d < D;
  const size_t base = (size_t)b * T * D + (dok ? d : 0);
  const size_t bd = (size_t)b * D + (dok ? d : 0);

  if (threadIdx.x < CH) {
    float2 a = make_float2(0.f, 0.f);
    if (dok) {
      if (glr != nullptr) a.x = glr[bd];
      if (gli != nullptr) a.y = gli[bd];
    }
    carry[0][c] = a;
  }

  const int nblk = (T + TB - 1) / TB;
  // inputs of the next (earlier) time block, loaded one block ahead: g, logmag, ang and h_{t-1}
  float pg[SEG], pl[SEG], pa[SEG], phr[SEG], phi[SEG];
  auto fetch = [&](int blk) {
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      const int t = blk * TB + seg * SEG + j;
      const bool ok = dok && t < T;
      const size_t off = base + (size_t)(ok ? t : 0) * D;
      pg[j] = ok ? g[off] : 0.f;
      pl[j] = ok ? lm[off] : 0.f;
      pa[j] = ok ? an[off] : 0.f;
      float qr = 0.f, qi = 0.f;
      if (ok) {
        if (t > 0) {
          qr = hr[off - D];
          qi = hi[off - D];
        } else if (h0r != nullptr) {
          qr = h0r[bd];
          qi = h0i[bd];
        }
      }
      phr[j] = qr;
      phi[j] = qi;
    }
  };
  fetch(nblk - 1);
  float2 cin = make_float2(0.f, 0.f);
  for (int it = 0; it < nblk; ++it) {
    const int p = it & 1;
    const int t0 = (nblk - 1 - it) * TB + seg * SEG;
    float xr[SEG], xi[SEG], xg[SEG], hpr[SEG], hpi[SEG];  // lambda_t (not conjugated), g_t, h_{t-1}
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      xg[j] = pg[j];
      hpr[j] = phr[j];
      hpi[j] = phi[j];
      const float m = pgn_exp(pl[j]);
      float s, co;
      pgn_sincos(pa[j], &s, &co);
      xr[j] = m * co;
      xi[j] = m * s;
    }
    if (it + 1 < nblk) fetch(nblk - 2 - it);
    // the segment's map on the carry coming from its right: c_out = P c_in + e, where the carry out of a
    // token is conj(lambda_t) a_t and a_t = g_t + (carry in)
    float er = 0.f, ei = 0.f, pr = 1.f, pi = 0.f;
#pragma unroll
    for (int j = SEG - 1; j >= 0; --j) {
      const float ar = xg[j] + er, ai = ei;
      er = xr[j] * ar + xi[j] * ai;
      ei = xr[j] * ai - xi[j] * ar;
      const float qr = xr[j] * pr + xi[j] * pi;
      const float qi = xr[j] * pi - xi[j] * pr;
      pr = qr;
      pi = qi;
    }
    maps[p][seg][c] = SegMaps{pr, pi, er, ei};
    __syncthreads();
    float2 a = carry[p][c];
#pragma unroll
    for (int s0 = NSEG - 1; s0 > 0; s0 -= kFold) {
      if (s0 <= seg) break;
      SegMaps m[kFold];
#pragma unroll
      for (int r = 0; r < kFold; ++r) m[r] = maps[p][max(s0 - r, 0)][c];
#pragma unroll
      for (int r = 0; r < kFold; ++r) {
        if (s0 - r > seg) {
          const float nr = m[r].pr * a.x - m[r].pi * a.y + m[r].er;
          const float ni = m[r].pi * a.x + m[r].pr * a.y + m[r].ei;
          a = make_float2(nr, ni);
        }
      }
    }
#pragma unroll
    for (int j = SEG - 1; j >= 0; --j) {
      const int t = t0 + j;
      const bool ok = dok && t < T;
      const float ar = xg[j] + a.x, ai = a.y;
      const float rr = xr[j] * hpr[j] - xi[j] * hpi[j];  // lambda_t h_{t-1}
      const float ri = xi[j] * hpr[j] + xr[j] * hpi[j];
      if (ok) {
        const size_t off = base + (size_t)t * D;
        du[off] = ar;
        dlm[off] = ar * rr + ai * ri;
        dan[off] = ai * rr - ar * ri;  // i lambda h = (-ri, rr)
      }
      a = make_float2(xr[j] * ar + xi[j] * ai, xr[j] * ai - xi[j] * ar);
    }
    if (seg == 0) carry[p ^ 1][c] = a;
    cin = a;
  }
  if (seg == 0 && dok && dh0r != nullptr) {
    dh0r[bd] = cin.x;
    dh0i[bd] = cin.y;
  }
}

// The empty sequence (T = 0): the final state is the initial one, so the forward writes (x_r, x_i) = h0 (zero when
// h0 is absent) and the backward passes the final state's gradient through to h0's, (x_r, x_i) = (g_last_r,
// g_last_i) (zero when absent). n = B D elements.
__global__ __launch_bounds__(256) void diag_empty_kernel(const float* ar, const float* ai, float* xr, float* xi,
                                                         int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    xr[i] = ar != nullptr ? ar[i] : 0.f;
    xi[i] = ai != nullptr ? ai[i] : 0.f;
  }
}

int launch_empty(const float* ar, const float* ai, float* xr, float* xi, int64_t n, hipStream_t st) {
  if (xr == nullptr) return PRAGNOSIA_OK;
  hipLaunchKernelGGL(diag_empty_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ar, ai, xr, xi, n);
  PGN_RETURN_LAUNCH();
}

template <int NW, int SEG, int CH>
int launch_fwd(const float* u, const float* lm, const float* an, const float* h0r, const float* h0i, float* hr,
               float* hi, float* hrl, float* hil, int B, int T, int D, hipStream_t st) {
  const int nct = (D + CH - 1) / CH;
  hipLaunchKernelGGL((diag_fwd_kernel<NW, SEG, CH>), dim3(B * nct), dim3(NW * 64), 0, st, u, lm, an, h0r, h0i, hr,
                     hi, hrl, hil, T, D, nct);
  PGN_RETURN_LAUNCH();
}

template <int NW, int SEG, int CH>
int launch_bwd(const float* g, const float* glr, const float* gli, const float* lm, const float* an,
               const float* hr, const float* hi, const float* h0r, const float* h0i, float* du, float* dlm,
               float* dan, float* dh0r, float* dh0i, int B, int T, int D, hipStream_t st) {
  const int nct = (D + CH - 1) / CH;
  hipLaunchKernelGGL((diag_bwd_kernel<NW, SEG, CH>), dim3(B * nct), dim3(NW * 64), 0, st, g, glr, gli, lm, an, hr,
                     hi, h0r, h0i, du, dlm, dan, dh0r, dh0i, T, D, nct);
  PGN_RETURN_LAUNCH();
}

bool shape_ok(int64_t B, int64_t T, int64_t D) {
  if (B <= 0 || T < 0 || D <= 0) return false;
  if (B * T * D >= ((int64_t)1 << 40)) return false;
  if (T >= (1 << 30) || D >= (1 << 30)) return false;
  const int64_t blocks = B * ((D + 31) / 32);
  return blocks < ((int64_t)1 << 31);
}

}  // namespace

extern "C" int pragnosia_diag_scan_fwd(const float* u, const float* logmag, const float* ang, const float* h0r,
                                       const float* h0i, float* hr, float* hi, float* hr_last, float* hi_last,
                                       int64_t B, int64_t T, int64_t D, void* stream) {
  PGN_CHECK_ARG(shape_ok(B, T, D));
  PGN_CHECK_ARG((h0r == nullptr) == (h0i == nullptr));
  PGN_CHECK_ARG((hr_last == nullptr) == (hi_last == nullptr));
  hipStream_t st = (hipStream_t)stream;
  if (T == 0) return launch_empty(h0r, h0i, hr_last, hi_last, B * D, st);
  PGN_CHECK_ARG(u && logmag && ang && hr && hi);
  // 16 waves x 64 channels, 4-token segments (64-token time blocks): swept against 4-16 waves, 32/64 channels and
  // 2-16-token segments at B16 T512 D768; short sequences use 4 waves
  if (T >= 64)
    return launch_fwd<16, 4, 64>(u, logmag, ang, h0r, h0i, hr, hi, hr_last, hi_last, (int)B, (int)T, (int)D, st);
  return launch_fwd<4, 4, 64>(u, logmag, ang, h0r, h0i, hr, hi, hr_last, hi_last, (int)B, (int)T, (int)D, st);
}

extern "C" int pragnosia_diag_scan_bwd(const float* g, const float* g_last_r, const float* g_last_i,
                                       const float* logmag, const float* ang, const float* hr, const float* hi,
                                       const float* h0r, const float* h0i, float* du, float* dlogmag, float* dang,
                                       float* dh0r, float* dh0i, int64_t B, int64_t T, int64_t D, void* stream) {
  PGN_CHECK_ARG(shape_ok(B, T, D));
  PGN_CHECK_ARG((h0r == nullptr) == (h0i == nullptr));
  PGN_CHECK_ARG((dh0r == nullptr) == (dh0i == nullptr));
  hipStream_t st = (hipStream_t)stream;
  if (T == 0) return launch_empty(g_last_r, g_last_i, dh0r, dh0i, B * D, st);
  PGN_CHECK_ARG(g && logmag && ang && hr && hi && du && dlogmag && dang);
  if (T >= 64)
    return launch_bwd<16, 4, 64>(g, g_last_r, g_last_i, logmag, ang, hr, hi, h0r, h0i, du, dlogmag, dang, dh0r, dh0i,
                                 (int)B, (int)T, (int)D, st);
  return launch_bwd<4, 4, 64>(g, g_last_r, g_last_i, logmag, ang, hr, hi, h0r, h0i, du, dlogmag, dang, dh0r, dh0i,
                              (int)B, (int)T, (int)D, st);
}
