// The associative carrier's scan with fp32 or fp64 operands (the exact path): plain and delta write rules, forward
// and backward, any head dims Dk <= 384, Dv <= 128.
//
// The reference's `assoc_scan` (src/assoc.py:254-269) computes in fp32, or in fp64 for fp64 inputs, through the
// chunked two-pass forms `_scan_twopass` / `_scan_twopass_delta` (src/assoc.py:118-165, :207-251), whose tests hold
// it to the literal recurrence at 1e-11 in fp64 (tests/test_assoc.py:18-44). The bf16-MFMA kernels of
// aspin_chunk.hip and aspin_delta.hip round every operand to bf16; this file computes the same function with no
// operand rounding, per token, per (batch, head), S (Dk x Dv) with keys on rows:
//     plain:  S_t = a_t S_{t-1} + k_t v_t^T
//     delta:  P_t = a_t S_{t-1},  r_t = v_t - P_t^T k_t,  S_t = P_t + beta_t k_t r_t^T
//     o_t = S_t^T q_t,   a_t = exp(la_t).
// (The chunked form is the same function reassociated; in fp32/fp64 the recurrence itself is the accurate way to
// evaluate it and needs no chunk inverse.)
//
// Layout of the work: one workgroup per (batch, head), ceil(Dv / 16) waves. Lane l of wave w owns value column
// j = 16 w + (l & 15) and the R key rows g R .. g R + R - 1 of that column (g = l >> 4, R = the smallest of 2, 4, 8,
// 16, 32, 48, 96 with 4 R >= Dk), so the state lives in registers (the larger R spill part of it to scratch), the
// update is R fused multiply-adds per lane and a read over the key rows is R products plus a two-step exchange across
// the four row groups of the wave. Inputs are staged through LDS a block of CK = 8 tokens at a time. The backward's
// LDS grows with R times the number of waves, so wide keys take fewer value columns per launch (the entry points
// return PRAGNOSIA_ERR_UNSUPPORTED past 160 KiB; the caller splits the value columns, which are independent).
//
// Forward writes o, the final state, and for a backward the state entering every block of CK tokens (`ckpt`,
// (B, H, ceil(T / CK), Dk, Dv)) and, for the delta rule, the residual r_t ((B, H, T, Dv)), so that re-running the
// recurrence inside a block needs no reduction across lanes: S_t = a_t S_{t-1} + k_t (beta_t r_t)^T.
//
// Backward, blocks in reverse, with X the gradient on S_t from later tokens (dS_final at the end) and G = X + q dO^T:
//     e_j   = sum_i G_ij k_i
//     plain: dv = e,         dk_i = sum_j G_ij v_j,                      dP = G
//     delta: dv = beta e,    du = -beta e,   dk_i = sum_j (beta G_ij r_j + P_ij du_j),   dP = G + k du^T,
//            dbeta = sum_j r_j e_j
//     dq_i = sum_j S_t,ij dO_j,   dla = sum_ij dP_ij P_ij,   X <- a_t dP   (dS0 = X after token 0),
// with S_{t-1} recomputed from the block's checkpoint. Sums over value columns are reduced inside the wave by a
// transpose-reduce over its 16 columns and across waves through LDS, once per block.
#include "common.h"

namespace {

constexpr int CK = PRAGNOSIA_EXACT_CKPT_TOKENS;
constexpr int kMaxDk = 384;  // key rows: R up to 96 a lane (four row groups)
constexpr int kMaxDv = 128;  // value columns: one a lane, up to eight waves

PGN_DEVICE float exp_(float x) { return expf(x); }
PGN_DEVICE double exp_(double x) { return exp(x); }

// Sum over value columns of per-lane vectors x[0..N) for the N key rows of a row group: the 16 lanes of the group
// (lane bits 0..3) exchange halves, so each lane ends with the full sums of N / 16 rows (rows jl N / 16 + n) when
// N >= 16, else of one row (row jl >> (4 - log2 N), the same value on 16 / N lanes).
template <typename real, int N>
PGN_DEVICE void colsum16(real (&x)[N], int jl) {
  int len = N;
#pragma unroll
  for (int s = 8; s >= 1; s >>= 1) {
    if (len > 1) {
      const int half = len / 2;
      const bool hi = (jl & s) != 0;
#pragma unroll
      for (int m = 0; m < half; ++m) {
        const real send = hi ? x[m] : x[m + half];
        const real keep = hi ? x[m + half] : x[m];
        x[m] = keep + __shfl_xor(send, s);
      }
      len = half;
    } else {
      x[0] += __shfl_xor(x[0], s);
    }
  }
}

// Stores the rows colsum16 left in this lane into a row vector `out` (row group g), for rows < Dk.
template <typename real, int N>
PGN_DEVICE void put_colsum(const real (&x)[N], int jl, int g, int Dk, real* out) {
  if constexpr (N >= 16) {
#pragma unroll
    for (int n = 0; n < N / 16; ++n) {
      const int i = g * N + jl * (N / 16) + n;
      if (i < Dk) out[i] = x[n];
    }
  } else {
    constexpr int sh = N == 8 ? 1 : N == 4 ? 2 : 3;
    if ((jl & ((1 << sh) - 1)) == 0) {
      const int i = g * N + (jl >> sh);
      if (i < Dk) out[i] = x[0];
    }
  }
}

template <typename real>
PGN_DEVICE real wave_total(real x) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) x += __shfl_xor(x, s);
  return x;
}

template <typename real, int R, bool DELTA>
__global__ __launch_bounds__(512) void aspin_exact_fwd(const real* __restrict__ q, const real* __restrict__ k,
                                                       const real* __restrict__ v, const real* __restrict__ la,
                                                       const real* __restrict__ beta, const real* __restrict__ S0,
                                                       real* __restrict__ o, real* __restrict__ Sfin,
                                                       real* __restrict__ ckpt, real* __restrict__ resid, int T,
                                                       int Dk, int Dv) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int DKP = 4 * R;
  const int NW = blockDim.x >> 6, DVP = 16 * NW;
  real* qs = reinterpret_cast<real*>(smem_raw);
  real* ks = qs + CK * DKP;
  real* vs = ks + CK * DKP;
  real* las = vs + CK * DVP;
  real* bes = las + CK;
  const int tid = threadIdx.x, l = tid & 63, jl = l & 15, g = l >> 4;
  const int j = 16 * (tid >> 6) + jl;
  const bool jok = j < Dv;
  const size_t bh = blockIdx.x;
  const size_t qoff = bh * T * Dk, voff = bh * T * Dv, soff = bh * Dk * Dv;
  const int NB = (T + CK - 1) / CK;
  real S[R];
#pragma unroll
  for (int m = 0; m < R; ++m) {
    const int i = g * R + m;
    S[m] = (S0 != nullptr && i < Dk && jok) ? S0[soff + (size_t)i * Dv + j] : real(0);
  }
  for (int blk = 0; blk < NB; ++blk) {
    const int t0 = blk * CK, n = min(CK, T - t0);
    if (ckpt != nullptr && jok) {
      real* c = ckpt + (bh * NB + blk) * Dk * Dv;
#pragma unroll
      for (int m = 0; m < R; ++m)
        if (g * R + m < Dk) c[(size_t)(g * R + m) * Dv + j] = S[m];
    }
    for (int e = tid; e < CK * DKP; e += blockDim.x) {
      const int tt = e / DKP, i = e - tt * DKP;
      const bool ok = tt < n && i < Dk;
      const size_t off = qoff + (size_t)(t0 + tt) * Dk + i;
      qs[e] = ok ? q[off] : real(0);
      ks[e] = ok ? k[off] : real(0);
    }
    for (int e = tid; e < CK * DVP; e += blockDim.x) {
      const int tt = e / DVP, jj = e - tt * DVP;
      vs[e] = (tt < n && jj < Dv) ? v[voff + (size_t)(t0 + tt) * Dv + jj] : real(0);
    }
    if (tid < CK) {
      las[tid] = tid < n ? la[bh * T + t0 + tid] : real(0);
      bes[tid] = (DELTA && tid < n) ? beta[bh * T + t0 + tid] : real(0);
    }
    __syncthreads();
    for (int tt = 0; tt < n; ++tt) {
      const real a = exp_(las[tt]);
      const real* kr = ks + tt * DKP + g * R;
      const real* qr = qs + tt * DKP + g * R;
      const real vj = vs[tt * DVP + (j < DVP ? j : 0)];
      real bw = vj;
      if constexpr (DELTA) {
        real up = 0;
#pragma unroll
        for (int m = 0; m < R; ++m) up += S[m] * kr[m];
        up += __shfl_xor(up, 16);
        up += __shfl_xor(up, 32);
        const real rr = vj - a * up;
        if (resid != nullptr && g == 0 && jok) resid[voff + (size_t)(t0 + tt) * Dv + j] = rr;
        bw = bes[tt] * rr;
      }
      real op = 0;
#pragma unroll
      for (int m = 0; m < R; ++m) {
        S[m] = a * S[m] + kr[m] * bw;
        op += S[m] * qr[m];
      }
      op += __shfl_xor(op, 16);
      op += __shfl_xor(op, 32);
      if (g == 0 && jok) o[voff + (size_t)(t0 + tt) * Dv + j] = op;
    }
    __syncthreads();
  }
  if (jok) {
#pragma unroll
    for (int m = 0; m < R; ++m)
      if (g * R + m < Dk) Sfin[soff + (size_t)(g * R + m) * Dv + j] = S[m];
  }
}

template <typename real, int R, bool DELTA>
__global__ __launch_bounds__(512) void aspin_exact_bwd(
    const real* __restrict__ q, const real* __restrict__ k, const real* __restrict__ v, const real* __restrict__ la,
    const real* __restrict__ beta, const real* __restrict__ ckpt, const real* __restrict__ resid,
    const real* __restrict__ dO, const real* __restrict__ dSfin, real* __restrict__ dq, real* __restrict__ dk,
    real* __restrict__ dv, real* __restrict__ dla, real* __restrict__ dbeta, real* __restrict__ dS0, int T, int Dk,
    int Dv) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int DKP = 4 * R;
  const int NW = blockDim.x >> 6, DVP = 16 * NW;
  real* qs = reinterpret_cast<real*>(smem_raw);
  real* ks = qs + CK * DKP;
  real* vs = ks + CK * DKP;
  real* rs = vs + CK * DVP;
  real* dos = rs + CK * DVP;
  real* as_ = dos + CK * DVP;
  real* bes = as_ + CK;
  real* dqp = bes + CK;          // [wave][token][row] partial sums over the wave's columns
  real* dkp = dqp + NW * CK * DKP;
  real* dlp = dkp + NW * CK * DKP;  // [wave][token]
  real* dbp = dlp + NW * CK;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, jl = l & 15, g = l >> 4;
  const int j = 16 * w + jl;
  const bool jok = j < Dv;
  const size_t bh = blockIdx.x;
  const size_t qoff = bh * T * Dk, voff = bh * T * Dv, soff = bh * Dk * Dv;
  const int NB = (T + CK - 1) / CK;
  real X[R];
#pragma unroll
  for (int m = 0; m < R; ++m) {
    const int i = g * R + m;
    X[m] = (dSfin != nullptr && i < Dk && jok) ? dSfin[soff + (size_t)i * Dv + j] : real(0);
  }
  for (int blk = NB - 1; blk >= 0; --blk) {
    const int t0 = blk * CK, n = min(CK, T - t0);
    for (int e = tid; e < CK * DKP; e += blockDim.x) {
      const int tt = e / DKP, i = e - tt * DKP;
      const bool ok = tt < n && i < Dk;
      const size_t off = qoff + (size_t)(t0 + tt) * Dk + i;
      qs[e] = ok ? q[off] : real(0);
      ks[e] = ok ? k[off] : real(0);
    }
    for (int e = tid; e < CK * DVP; e += blockDim.x) {
      const int tt = e / DVP, jj = e - tt * DVP;
      const bool ok = tt < n && jj < Dv;
      const size_t off = voff + (size_t)(t0 + tt) * Dv + jj;
      vs[e] = ok ? v[off] : real(0);
      rs[e] = (DELTA && ok) ? resid[off] : real(0);
      dos[e] = ok ? dO[off] : real(0);
    }
    if (tid < CK) {
      as_[tid] = tid < n ? exp_(la[bh * T + t0 + tid]) : real(1);
      bes[tid] = (DELTA && tid < n) ? beta[bh * T + t0 + tid] : real(0);
    }
    const real* ck = ckpt + (bh * NB + blk) * Dk * Dv;
    __syncthreads();
    const int jc = j < DVP ? j : 0;
    for (int tt = n - 1; tt >= 0; --tt) {
      // S_{t-1}: the block's entering state (re-read from the checkpoint, which stays in cache) carried through its
      // tokens before t
      real Sp[R];
#pragma unroll
      for (int m = 0; m < R; ++m) {
        const int i = g * R + m;
        Sp[m] = (i < Dk && jok) ? ck[(size_t)i * Dv + j] : real(0);
      }
      for (int s = 0; s < tt; ++s) {
        const real as = as_[s];
        const real bw = DELTA ? bes[s] * rs[s * DVP + jc] : vs[s * DVP + jc];
#pragma unroll
        for (int m = 0; m < R; ++m) Sp[m] = as * Sp[m] + ks[s * DKP + g * R + m] * bw;
      }
      const real a = as_[tt], bet = bes[tt];
      const real vj = vs[tt * DVP + jc], doj = dos[tt * DVP + jc];
      const real rr = DELTA ? rs[tt * DVP + jc] : vj;
      const real bw = DELTA ? bet * rr : vj;
      const real* kr = ks + tt * DKP + g * R;
      const real* qr = qs + tt * DKP + g * R;
      real ep = 0;
      {
        real xq[R];
#pragma unroll
        for (int m = 0; m < R; ++m) {
          Sp[m] *= a;                          // P = a S_{t-1}
          xq[m] = (Sp[m] + kr[m] * bw) * doj;  // S_t dO_j
          X[m] += qr[m] * doj;                 // G = X + q dO^T
          ep += X[m] * kr[m];
        }
        colsum16<real, R>(xq, jl);
        put_colsum<real, R>(xq, jl, g, Dk, dqp + (w * CK + tt) * DKP);
      }
      real e = ep + __shfl_xor(ep, 16);
      e += __shfl_xor(e, 32);
      const real du = DELTA ? -bet * e : real(0);
      {
        real xk[R];
#pragma unroll
        for (int m = 0; m < R; ++m) xk[m] = DELTA ? (bet * rr * X[m] + Sp[m] * du) : X[m] * vj;
        colsum16<real, R>(xk, jl);
        put_colsum<real, R>(xk, jl, g, Dk, dkp + (w * CK + tt) * DKP);
      }
      real dl = 0;
#pragma unroll
      for (int m = 0; m < R; ++m) {
        const real dP = DELTA ? X[m] + kr[m] * du : X[m];
        dl += dP * Sp[m];
        X[m] = a * dP;
      }
      if (g == 0 && jok) dv[voff + (size_t)(t0 + tt) * Dv + j] = DELTA ? bet * e : e;
      dl = wave_total(dl);
      const real db = DELTA ? wave_total(rr * ep) : real(0);
      if (l == 0) {
        dlp[w * CK + tt] = dl;
        dbp[w * CK + tt] = db;
      }
    }
    __syncthreads();
    for (int e = tid; e < n * Dk; e += blockDim.x) {
      const int tt = e / Dk, i = e - tt * Dk;
      real sq = 0, sk = 0;
      for (int ww = 0; ww < NW; ++ww) {
        sq += dqp[(ww * CK + tt) * DKP + i];
        sk += dkp[(ww * CK + tt) * DKP + i];
      }
      const size_t off = qoff + (size_t)(t0 + tt) * Dk + i;
      dq[off] = sq;
      dk[off] = sk;
    }
    if (tid < n) {
      real sl = 0, sb = 0;
      for (int ww = 0; ww < NW; ++ww) {
        sl += dlp[ww * CK + tid];
        sb += dbp[ww * CK + tid];
      }
      dla[bh * T + t0 + tid] = sl;
      if (DELTA) dbeta[bh * T + t0 + tid] = sb;
    }
    __syncthreads();
  }
  if (dS0 != nullptr && jok) {
#pragma unroll
    for (int m = 0; m < R; ++m)
      if (g * R + m < Dk) dS0[soff + (size_t)(g * R + m) * Dv + j] = X[m];
  }
}

int rows_per_lane(int64_t Dk) {
  return Dk <= 8 ? 2 : Dk <= 16 ? 4 : Dk <= 32 ? 8 : Dk <= 64 ? 16 : Dk <= 128 ? 32 : Dk <= 192 ? 48 : 96;
}

template <typename real>
size_t fwd_lds(int R, int NW) {
  return (size_t)(2 * CK * 4 * R + CK * 16 * NW + 2 * CK) * sizeof(real);
}

template <typename real>
size_t bwd_lds(int R, int NW) {
  return (size_t)(2 * CK * 4 * R + 3 * CK * 16 * NW + 2 * CK + 2 * NW * CK * 4 * R + 2 * NW * CK) * sizeof(real);
}

constexpr size_t kMaxLds = 160 * 1024;

bool exact_shape_ok(int64_t B, int64_t H, int64_t T, int64_t Dk, int64_t Dv) {
  if (B <= 0 || H <= 0 || T <= 0 || Dk <= 0 || Dv <= 0 || Dk > kMaxDk || Dv > kMaxDv) return false;
  if (B * H >= ((int64_t)1 << 31) || T >= ((int64_t)1 << 28)) return false;
  return B * H * T * kMaxDk < ((int64_t)1 << 46);
}

template <typename real, bool DELTA, int R>
int launch_fwd(const void* q, const void* k, const void* v, const void* la, const void* beta, const void* S0, void* o,
               void* Sfin, void* ckpt, void* resid, int64_t B, int64_t H, int64_t T, int64_t Dk, int64_t Dv,
               hipStream_t st) {
  const int NW = (int)((Dv + 15) / 16);
  const size_t lds = fwd_lds<real>(R, NW);
  if (lds > kMaxLds) return PRAGNOSIA_ERR_UNSUPPORTED;
  const void* fn = (const void*)aspin_exact_fwd<real, R, DELTA>;
  const hipError_t e = pgn_lds_limit(fn, lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((aspin_exact_fwd<real, R, DELTA>), dim3((unsigned)(B * H)), dim3(64 * NW), lds, st,
                     (const real*)q, (const real*)k, (const real*)v, (const real*)la, (const real*)beta,
                     (const real*)S0, (real*)o, (real*)Sfin, (real*)ckpt, (real*)resid, (int)T, (int)Dk, (int)Dv);
  PGN_RETURN_LAUNCH();
}

template <typename real, bool DELTA, int R>
int launch_bwd(const void* q, const void* k, const void* v, const void* la, const void* beta, const void* ckpt,
               const void* resid, const void* dO, const void* dSfin, void* dq, void* dk, void* dv, void* dla,
               void* dbeta, void* dS0, int64_t B, int64_t H, int64_t T, int64_t Dk, int64_t Dv, hipStream_t st) {
  const int NW = (int)((Dv + 15) / 16);
  const size_t lds = bwd_lds<real>(R, NW);
  if (lds > kMaxLds) return PRAGNOSIA_ERR_UNSUPPORTED;
  const void* fn = (const void*)aspin_exact_bwd<real, R, DELTA>;
  const hipError_t e = pgn_lds_limit(fn, lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((aspin_exact_bwd<real, R, DELTA>), dim3((unsigned)(B * H)), dim3(64 * NW), lds, st,
                     (const real*)q, (const real*)k, (const real*)v, (const real*)la, (const real*)beta,
                     (const real*)ckpt, (const real*)resid, (const real*)dO, (const real*)dSfin, (real*)dq,
                     (real*)dk, (real*)dv, (real*)dla, (real*)dbeta, (real*)dS0, (int)T, (int)Dk, (int)Dv);
  PGN_RETURN_LAUNCH();
}

template <typename real, bool DELTA>
int dispatch_fwd(int R, const void* q, const void* k, const void* v, const void* la, const void* beta, const void* S0,
                 void* o, void* Sfin, void* ckpt, void* resid, int64_t B, int64_t H, int64_t T, int64_t Dk,
                 int64_t Dv, hipStream_t st) {
  switch (R) {
    case 2: return launch_fwd<real, DELTA, 2>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    case 4: return launch_fwd<real, DELTA, 4>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    case 8: return launch_fwd<real, DELTA, 8>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    case 16: return launch_fwd<real, DELTA, 16>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    case 32: return launch_fwd<real, DELTA, 32>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    case 48: return launch_fwd<real, DELTA, 48>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
    default: return launch_fwd<real, DELTA, 96>(q, k, v, la, beta, S0, o, Sfin, ckpt, resid, B, H, T, Dk, Dv, st);
  }
}

template <typename real, bool DELTA>
int dispatch_bwd(int R, const void* q, const void* k, const void* v, const void* la, const void* beta,
                 const void* ckpt, const void* resid, const void* dO, const void* dSfin, void* dq, void* dk,
                 void* dv, void* dla, void* dbeta, void* dS0, int64_t B, int64_t H, int64_t T, int64_t Dk,
                 int64_t Dv, hipStream_t st) {
#define PGN_EXACT_BWD(RR)                                                                                          \
  return launch_bwd<real, DELTA, RR>(q, k, v, la, beta, ckpt, resid, dO, dSfin, dq, dk, dv, dla, dbeta, dS0, B, H, \
                                     T, Dk, Dv, st)
  switch (R) {
    case 2: PGN_EXACT_BWD(2);
    case 4: PGN_EXACT_BWD(4);
    case 8: PGN_EXACT_BWD(8);
    case 16: PGN_EXACT_BWD(16);
    case 32: PGN_EXACT_BWD(32);
    case 48: PGN_EXACT_BWD(48);
    default: PGN_EXACT_BWD(96);
  }
#undef PGN_EXACT_BWD
}

}  // namespace

extern "C" int pragnosia_aspin_exact_fwd(const void* q, const void* k, const void* v, const void* la,
                                         const void* beta, const void* S0, void* o, void* S_final, void* ckpt,
                                         void* resid, int64_t B, int64_t H, int64_t T, int64_t Dk, int64_t Dv,
                                         int dtype, void* stream) {
  PGN_CHECK_ARG(exact_shape_ok(B, H, T, Dk, Dv));
  PGN_CHECK_ARG(dtype == PRAGNOSIA_F32 || dtype == PRAGNOSIA_F64);
  PGN_CHECK_ARG(q && k && v && la && o && S_final);
  const bool delta = beta != nullptr;
  if (delta && ckpt != nullptr) PGN_CHECK_ARG(resid != nullptr);
  const int R = rows_per_lane(Dk);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PRAGNOSIA_F32)
    return delta ? dispatch_fwd<float, true>(R, q, k, v, la, beta, S0, o, S_final, ckpt, resid, B, H, T, Dk, Dv, st)
                 : dispatch_fwd<float, false>(R, q, k, v, la, beta, S0, o, S_final, ckpt, resid, B, H, T, Dk, Dv, st);
  return delta ? dispatch_fwd<double, true>(R, q, k, v, la, beta, S0, o, S_final, ckpt, resid, B, H, T, Dk, Dv, st)
               : dispatch_fwd<double, false>(R, q, k, v, la, beta, S0, o, S_final, ckpt, resid, B, H, T, Dk, Dv, st);
}

extern "C" int pragnosia_aspin_exact_bwd(const void* q, const void* k, const void* v, const void* la,
                                         const void* beta, const void* ckpt, const void* resid, const void* dO,
                                         const void* dS_final, void* dq, void* dk, void* dv, void* dla, void* dbeta,
                                         void* dS0, int64_t B, int64_t H, int64_t T, int64_t Dk, int64_t Dv,
                                         int dtype, void* stream) {
  PGN_CHECK_ARG(exact_shape_ok(B, H, T, Dk, Dv));
  PGN_CHECK_ARG(dtype == PRAGNOSIA_F32 || dtype == PRAGNOSIA_F64);
  PGN_CHECK_ARG(q && k && v && la && ckpt && dO && dq && dk && dv && dla);
  const bool delta = beta != nullptr;
  if (delta) PGN_CHECK_ARG(resid != nullptr && dbeta != nullptr);
  const int R = rows_per_lane(Dk);
  const int NW = (int)((Dv + 15) / 16);
  const size_t lds = dtype == PRAGNOSIA_F32 ? bwd_lds<float>(R, NW) : bwd_lds<double>(R, NW);
  if (lds > kMaxLds) return PRAGNOSIA_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PRAGNOSIA_F32)
    return delta ? dispatch_bwd<float, true>(R, q, k, v, la, beta, ckpt, resid, dO, dS_final, dq, dk, dv, dla, dbeta,
                                             dS0, B, H, T, Dk, Dv, st)
                 : dispatch_bwd<float, false>(R, q, k, v, la, beta, ckpt, resid, dO, dS_final, dq, dk, dv, dla,
                                              dbeta, dS0, B, H, T, Dk, Dv, st);
  return delta ? dispatch_bwd<double, true>(R, q, k, v, la, beta, ckpt, resid, dO, dS_final, dq, dk, dv, dla, dbeta,
                                            dS0, B, H, T, Dk, Dv, st)
               : dispatch_bwd<double, false>(R, q, k, v, la, beta, ckpt, resid, dO, dS_final, dq, dk, dv, dla,
                                             dbeta, dS0, B, H, T, Dk, Dv, st);
}
