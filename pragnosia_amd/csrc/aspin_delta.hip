// The associative carrier's chunked scan, delta write rule: forward and hand-written backward.
//
// Per (batch, head), chunk C = 64, head dim D = 64, with L, eL, w, a and dec as in the plain rule and beta_t in (0, 1)
// the write strength, the state S entering a chunk is updated by (the reference's `_scan_twopass_delta`,
// `src/assoc.py:207-251`):
//     N   = diag(beta) strictly_lower((K K^T) o dec),   X = (I + N)^-1
//     U   = K S,   rhs = diag(beta) (V - diag(eL) U),   W = X rhs
//     O   = ((Q K^T) o dec) W + (Q o eL) S,             S' = a S + (K o w)^T W
//
// Four kernels:
//   aspin_delta_inv    four waves per (batch-head, chunk): N from a bf16 MFMA K K^T and fp32 decays, then X in fp32
//                      by 16 x 16 blocks: the diagonal blocks by forward substitution (one column per lane), the
//                      blocks below them by block forward substitution on fp32 MFMA (the reference sums the
//                      diagonal blocks by doubling and substitutes across blocks, `src/assoc.py:168-204`; both are
//                      exact in exact arithmetic). X is stored bf16 for the products; measured against an fp64
//                      inverse it is as close as bf16 rounding of the exact inverse allows, repeated keys included.
//   aspin_delta_fwd    one workgroup of 8 waves per (batch, head) walks the chunks: 4 chain waves and 4 service
//                      waves (decayed scores, staging of the next chunk, its decay scan). The rule is independent
//                      per value column given X, so chain wave w owns value columns 16w..16w+15 for all 64 tokens
//                      and the whole state chain (U -> rhs -> W -> S') stays in that wave's MFMA accumulators: each
//                      product's accumulator is the next product's operand, with no LDS round trip and no barrier
//                      on the chain. Writes o, the residuals W and the entering states (both bf16; each entering
//                      state transposed, (j, d), so a lane's four consecutive key rows are one 8-byte store) for
//                      the backward, and the final fp32 state.
//   aspin_delta_bwd_chain   one workgroup of 8 waves per (batch, head), chunks in reverse: 4 chain waves, chain
//                      wave w owning value columns 16w.. again, and 4 service waves. Carries dS (gradient on the state leaving the chunk) in registers:
//                          dW = A^T dO + w o (K dS),  drhs = X^T dW,  dU = -beta eL o drhs,
//                          dS_prev = a dS + (Q o eL)^T dO + K^T dU,
//                      and writes drhs, the per-chunk dS (bf16, transposed) and the row sums over value columns that the decay
//                      and beta gradients need: sum_j drhs (V - eL U) and -beta sum_j drhs U.
//                      dV = beta o drhs is written by the local kernel from the stored drhs (coalesced, off the
//                      chain).
//   aspin_delta_bwd_local   one workgroup of 8 waves per (batch-head, chunk), fully parallel: everything that is
//                      local to a chunk once drhs and dS are known. With dN = -drhs W^T (the gradient through
//                      W = X rhs, since dX = dW rhs^T and dN = -X^T dX X^T), dKK = diag(beta) dN o dec (strictly
//                      lower), G = dKK + dKK^T, dA = dO W^T, dP = dA o dec:
//                          dQ = dP K + eL o (dO S^T)
//                          dK = dP^T Q + G K + dU S^T + w o (W dS^T)
//                          dbeta_t = sum_j drhs (V - eL U) + sum_{s<t} dN_ts (KK o dec)_ts
//                          dL_t = rowsum(dA o A) - colsum(dA o A) + rowsum(dKK o KK) - colsum(dKK o KK)
//                                 + eL_t (q_t.(S dO_t) - beta_t sum_j drhs U) - w_t k_t.(dS W_t),
//                          dL_{C-1} += sum_t w_t k_t.(dS W_t) + a <S, dS>;  dla = reverse cumsum of dL.
// (the reference's loop kernels `src/assoc_kernel.py:332-458` and inverse `:555-704` compute the same quantities
// with a different split.) Padded tokens of a partial last chunk load as zero with la = 0 and beta = 0: they write
// nothing and receive no gradient.
#include "mfma_tile.h"

using namespace pgn;

PGN_STAMP_UNIT(delta)

namespace {

constexpr int C = 64;
constexpr int DK = 64;
constexpr int TILE = 64 * kPitch;
constexpr int NP = C + 4;  // pitch of the fp32 N^T tile

// Where the delta scan of workgroup index bh finds its rows. KH = 1 (64-wide heads): scan bh is head bh. KH = 2
// (128-wide heads): given X (which depends on the keys, decays and write strengths only) the rule is independent per
// value column, so head hw runs as two scans bh = 2 hw + vh over value columns 64 vh .. 64 vh + 63, each carrying
// the full 128-key state slice (128 x 64). Every (T, .) operand has rows of DKEY elements: q and k are read whole
// (KH 64-wide halves; LDS tiles are 64 wide, so a 128-wide operand is staged as two tiles), v, dO, o, W, drhs and dv
// at columns 64 vh. X is per (head, chunk), shared by both scans. States (S0, S_final, dS_final, dS0; (B, H, DKEY,
// DKEY) fp32, key rows) are read and written at columns 64 vh; the entering states and per-chunk state gradients,
// stored transposed ((value j, key d), (B, H, NC, DKEY, DKEY) bf16), at rows 64 vh. dq, dk, dla and dbeta of a
// 128-wide head sum over its two scans: scan vh writes slot vh (the caller's tensor, or a workspace tensor of the
// same layout), and a last kernel adds the slots.
template <int KH>
struct DeltaRows {
  static constexpr int DKEY = 64 * KH;
  int hw, vh;
  PGN_DEVICE explicit DeltaRows(int bh) : hw(KH == 2 ? bh >> 1 : bh), vh(KH == 2 ? bh & 1 : 0) {}
  PGN_DEVICE size_t rows(int T) const { return (size_t)hw * T * DKEY; }    // q, k, dq, dk
  PGN_DEVICE size_t vals(int T) const { return rows(T) + 64 * vh; }        // v, dO, o, W, drhs, dv
  PGN_DEVICE size_t state() const { return (size_t)hw * DKEY * DKEY + 64 * vh; }
  PGN_DEVICE size_t stateT(int NC, int c) const {
    return ((size_t)hw * NC + c) * DKEY * DKEY + (size_t)64 * vh * DKEY;
  }
  PGN_DEVICE size_t tok(int T) const { return (size_t)hw * T; }            // la, beta, dla, dbeta
  template <class Ptr>
  PGN_DEVICE Ptr slot(Ptr s0, Ptr s1) const {
    return (KH == 2 && vh) ? s1 : s0;
  }
};

// Scan index of workgroup bi in the one-workgroup-per-scan kernels: at KH = 2 a head's two value halves are
// workgroups 8 apart, so they run on one XCD (workgroup i goes to XCD i mod 8) and its q, k and X come from HBM once
// into that L2 (head-dim-128 delta step 0.1775 -> 0.1745 ms on average over five A/B pairs on one box); the grid is
// then padded to whole sets of 16 (scan indices past the last come out >= the scan count, and their workgroups exit).
template <int KH>
PGN_DEVICE int scan_of(int bi) {
  if constexpr (KH == 2) return 2 * ((bi >> 4) * 8 + (bi & 7)) + ((bi >> 3) & 1);
  return bi;
}
template <int KH>
int scan_grid(int64_t heads) {
  if constexpr (KH == 2) return (int)((heads + 7) / 8 * 16);
  return (int)(heads * KH);
}

PGN_DEVICE float incl_scan64(float x, int l) { return wave_prefix_sum(x, l); }

PGN_DEVICE float rev_scan64(float x, int l) { return wave_suffix_sum(x, l); }

// Per-chunk decay statistics into LDS (one wave): L (inclusive cumsum of la), eL = exp(L), w = exp(L_C - L).
PGN_DEVICE void chunk_decays(float la_l, int l, float* Ls, float* eLs, float* ws) {
  const float L = incl_scan64(la_l, l);
  const float LC = lane_value(L, 63);
  Ls[l] = L;
  eLs[l] = __expf(L);
  ws[l] = __expf(fminf(LC - L, 0.f));
}

// ------------------------------------------------------------------------------------------------------------------
// X = (I + N)^-1, one workgroup of four waves per (batch-head, chunk)
// N^T and X are kept as their ten 16 x 16 blocks on and below the diagonal (block (tb, sb), sb <= tb, at index
// tb (tb + 1) / 2 + sb, unpadded rows so the substitution reads four entries at once): 24 KB of LDS per chunk, so
// six chunks (one round of the grid at cfg2, 24 waves) are resident per compute unit. The keys (KH 64-wide tiles) are
// loaded in 16-byte row segments into the N and X block areas (unused until N is formed) and read from there as MFMA
// operands. The waves share the independent work of each phase: the ten N blocks (three, three, two, two), the
// products of each block level (one per wave), the four diagonal blocks' substitutions (one per wave, four lanes per
// column), the staging and the store. Each entry is computed by the same operations in the same order as by one wave,
// so X does not depend on the split.
constexpr int BP = 16;                 // row pitch of a 16 x 16 fp32 block
constexpr int BLK = 16 * BP;
PGN_DEVICE int blk(int tb, int sb) { return (tb * (tb + 1) / 2 + sb) * BLK; }

// x of lane q of each group of four lanes, in all four (q a compile-time constant once the caller's loop unrolls)
PGN_DEVICE float quad_bcast(float x, int q) {
  const int v = __builtin_bit_cast(int, x);
  switch (q) {
    case 0: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x00, 0xf, 0xf, false));
    case 1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x55, 0xf, 0xf, false));
    case 2: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0xAA, 0xf, 0xf, false));
    default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0xFF, 0xf, 0xf, false));
  }
}

// the N blocks (tb, sb) of wave w, -1 past its share
__constant__ const signed char kInvNT[4][3] = {{3, 3, 0}, {3, 1, 1}, {3, 2, -1}, {2, 2, -1}};
__constant__ const signed char kInvNS[4][3] = {{0, 3, 0}, {1, 0, 1}, {2, 0, -1}, {1, 2, -1}};

template <int KH>
__global__ __launch_bounds__(256) void aspin_delta_inv(const __bf16* __restrict__ k, const float* __restrict__ la,
                                                       const float* __restrict__ be, __bf16* __restrict__ X, int T,
                                                       int NC) {
  constexpr int DKEY = 64 * KH;
  __shared__ __align__(16) float NX[20 * BLK];
  float* const NT = NX;             // N^T blocks: NT(tb, sb)[s' * BP + t'] = N[16 tb + t'][16 sb + s']
  float* const Xf = NX + 10 * BLK;  // X blocks: Xf(ib, jb)[r * BP + c] = X[16 ib + r][16 jb + c]
  __shared__ __align__(16) float Tt[3 * BLK];   // per-level sums, one block per product
  __shared__ __align__(16) float Ls[C], bs[C];

  const int bh = blockIdx.x / NC, c = blockIdx.x - bh * NC;  // head (not scan), chunk
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, g = l >> 4, i = l & 15;
  // instrumented build (second buffer): per chunk, wave 0's clocks at the start (entries 0, 1), the end of the key
  // staging (2), of N (3), of the diagonal blocks (4), of the block levels (5), and clocks after the store (6, 7)
  if (w == 0) PGN_STAMP_CLOCKS_AUX(blockIdx.x * 8);
  const int t0 = c * C, nr = min(C, T - t0);
  const __bf16* kc = k + ((size_t)bh * T + t0) * DKEY;
  // the keys in 16-byte row segments (two per thread and tile, rows past T as zeros), staged in the N and X block
  // areas, which nothing uses before N is formed
  __bf16* Kst = reinterpret_cast<__bf16*>(NX);
  static_assert(KH * TILE * sizeof(__bf16) <= sizeof(NX), "the key tiles fit the N and X block areas");
  {
    bf16x8 seg[2 * KH];
#pragma unroll
    for (int n = 0; n < 2 * KH; ++n) seg[n] = load_seg(kc + 64 * (n >> 1), nr, tid + 256 * (n & 1), DKEY);
    // this lane's decay and strength, issued with the keys (range-checked: zero past T, no branch)
    const float lav = load_f32_lane(la + (size_t)bh * T + t0, nr, l);
    const float bev = load_f32_lane(be + (size_t)bh * T + t0, nr, l);
#pragma unroll
    for (int n = 0; n < 2 * KH; ++n) put_seg(Kst + (n >> 1) * TILE, seg[n], tid + 256 * (n & 1));
    if (w == 0) {
      Ls[l] = incl_scan64(lav, l);
      bs[l] = bev;
    }
  }
  __syncthreads();
  if (w == 0) PGN_STAMP_AUX(blockIdx.x * 8 + 2);

  // N^T blocks: accumulator rows s (block sb), lane t (block tb), for sb <= tb; formed in registers, written once
  // every wave has read its key operands (N overwrites the staged keys)
  f32x4 nv[3];
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int tb = kInvNT[w][n], sb = kInvNS[w][n];
    nv[n] = zero4();
    if (tb >= 0) {
      f32x4 acc = zero4();
#pragma unroll
      for (int m = 0; m < 2 * KH; ++m)
        acc = pgn_mfma(frag(Kst + (m >> 1) * TILE, 16 * sb + i, m & 1, g),
                       frag(Kst + (m >> 1) * TILE, 16 * tb + i, m & 1, g), acc);
      const int t = 16 * tb + i;
      const float Lt = Ls[t], bt = bs[t];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = 16 * sb + 4 * g + r;
        nv[n][r] = bt * acc[r] * masked_decay(Lt - Ls[s], s < t);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int tb = kInvNT[w][n], sb = kInvNS[w][n];
    if (tb >= 0) {
      float* nb = NT + blk(tb, sb);
#pragma unroll
      for (int r = 0; r < 4; ++r) nb[(4 * g + r) * BP + i] = nv[n][r];
    }
  }
  __syncthreads();
  if (w == 0) PGN_STAMP_AUX(blockIdx.x * 8 + 3);

  // X by blocks of 16: X_ii = (I + N_ii)^-1 by forward substitution, diagonal block i on wave i; then
  // X_ij = -X_ii sum_{k=j}^{i-1} N_ik X_kj, i > j, level by level (i - j = 1, 2, 3), product j on wave j, on fp32
  // MFMA (v_mfma_f32_16x16x4f32: A[r][k] in lane r + 16k, B[k][c] in lane c + 16k, D[4g + e][c] in lane c + 16g).
  {
    // diagonal block b = w, column cl = l / 4 on four lanes, lane q = l % 4 holding rows t = 4 m + q; row s's value,
    // final after step s - 1, reaches the column's four lanes by a quad broadcast (DPP) before step s
    const int cl = l >> 2, q = l & 3;
    const float* nd = NT + blk(w, w);
    float xr[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xr[m] = (4 * m + q == cl) ? 1.f : 0.f;
    // N[16w + t][16w + s] for the lane's rows and the four steps of a group, read a group ahead and unconditionally
    // (the row condition selects the updated value, not the read, so the reads are not sunk into it)
    float nb[2][4][4];
    auto read_group = [&](int k, float (&dst)[4][4]) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[u][m] = (4 * k + u < 15) ? nd[(4 * k + u) * BP + 4 * m + q] : 0.f;
    };
    read_group(0, nb[0]);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k < 3) read_group(k + 1, nb[(k + 1) & 1]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = 4 * k + u;
        if (s < 15) {
          const float xs = quad_bcast(xr[s >> 2], s & 3);
#pragma unroll
          for (int m = (s + 1) >> 2; m < 4; ++m) {
            const float upd = xr[m] - nb[k & 1][u][m] * xs;
            xr[m] = (4 * m + q > s) ? upd : xr[m];
          }
        }
      }
    }
    float* xb = Xf + blk(w, w);
#pragma unroll
    for (int m = 0; m < 4; ++m) xb[(4 * m + q) * BP + cl] = xr[m];
  }
  __syncthreads();
  if (w == 0) PGN_STAMP_AUX(blockIdx.x * 8 + 4);
  {
    const int r16 = l & 15, k4 = l >> 4;
    // one 16 x 16 x 16 product A B accumulated onto acc: A the block at `Ab`, read transposed when `at`
    // (A[r][k] = Ab[k * BP + r]); B the block at `Bb` (B[k][c] = Bb[k * BP + c])
    auto mm = [&](f32x4 acc, const float* Ab, bool at, const float* Bb) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kx = 4 * kk + k4;
        const float av = at ? Ab[kx * BP + r16] : Ab[r16 * BP + kx];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, Bb[kx * BP + r16], acc, 0, 0, 0);
      }
      return acc;
    };
    const int jb = w;
#pragma unroll
    for (int d = 1; d < 4; ++d) {
      const int ib = jb + d;
      if (ib < 4) {
        f32x4 acc = zero4();
        // N_ik = (N^T block (ib, kb)) transposed, kb = jb .. ib - 1
#pragma unroll
        for (int u = 0; u < d; ++u) acc = mm(acc, NT + blk(ib, jb + u), true, Xf + blk(jb + u, jb));
#pragma unroll
        for (int e = 0; e < 4; ++e) Tt[jb * BLK + (4 * k4 + e) * BP + r16] = acc[e];
      }
      __syncthreads();
      if (ib < 4) {
        const f32x4 xr = mm(zero4(), Xf + blk(ib, ib), false, Tt + jb * BLK);
        float* xo = Xf + blk(ib, jb);
#pragma unroll
        for (int e = 0; e < 4; ++e) xo[(4 * k4 + e) * BP + r16] = -xr[e];
      }
      __syncthreads();
    }
  }
  if (w == 0) PGN_STAMP_AUX(blockIdx.x * 8 + 5);
  // X (bf16, row-major; zero above the diagonal blocks) in 16-byte row segments, two per thread
  __bf16* Xc = X + ((size_t)bh * NC + c) * C * C;
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int e = tid + 256 * n, r = e >> 3, c0 = 8 * (e & 7);
    const int rb = r >> 4, cb = c0 >> 4;
    bf16x8 out;
    if (cb <= rb) {
      const float* xb = Xf + blk(rb, cb) + (r & 15) * BP + (c0 & 15);
#pragma unroll
      for (int u = 0; u < 8; ++u) out[u] = (__bf16)xb[u];
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) out[u] = (__bf16)0.f;
    }
    *reinterpret_cast<bf16x8*>(Xc + r * C + c0) = out;
  }
  if (w == 0) PGN_STAMP_CLOCKS_AUX(blockIdx.x * 8 + 6);
}

// ------------------------------------------------------------------------------------------------------------------
// forward: one workgroup of 8 waves per scan (a 64-wide head, or one value half of a 128-wide one), chunks in order.
// Waves 0-3 carry the chain, wave w owning value columns 16w..16w+15 with its columns of the fp32 state (all key
// rows) in registers (U -> rhs -> W -> S' never leaves them). Waves
// 4-7 serve them: per chunk they compute the decayed scores A (the one operand the chain waves share), then stage the
// next chunk's tiles into the other half of a double-buffered LDS and run its decay scan. Two barriers per chunk: A
// ready (the chain waves form U, rhs and W before it), and the end of the chunk.
// Per chunk: Q and K (KH tiles each), V, X; L, eL, w, beta.
template <int KH>
constexpr int fwd_stage() { return (2 * KH + 2) * TILE; }
constexpr int kFwdVec = 4 * C;         // L, eL, w, beta

template <int KH>
__global__ __launch_bounds__(512) void aspin_delta_fwd(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ be, const __bf16* __restrict__ X,
    const float* __restrict__ S0, __bf16* __restrict__ o, __bf16* __restrict__ Wout, float* __restrict__ Sfin,
    __bf16* __restrict__ sent, int T, int NC, int nscans) {
  constexpr int DKEY = 64 * KH;
  constexpr int kStage = fwd_stage<KH>();
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* stg = reinterpret_cast<__bf16*>(smem);          // two sets of staged tiles, chunk c uses set c & 1
  __bf16* As = stg + 2 * kStage;                           // As[t][s] = A[t][s]
  float* vec = reinterpret_cast<float*>(As + TILE);        // two vector sets, chunk c uses set c & 1
  // instrumented build: per wave, clocks where its role's branch starts (entries 0, 1) and at the kernel's end (2, 3),
  // then the start and end of its phase for chunk c (4 + 2 c, 5 + 2 c)
#define DF_STAMP(k) PGN_STAMP((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * (4 + 2 * NC) + (k))
#define DF_CLOCKS(k) \
  PGN_STAMP_CLOCKS((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * (4 + 2 * NC) + (k))

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  const int bh = scan_of<KH>((int)blockIdx.x);
  if (bh >= nscans) return;  // grid padding (uniform over the workgroup, before any barrier)
  const DeltaRows<KH> R(bh);
  const size_t voff = R.vals(T);

  if (w < 4) {
    // ================= chain waves: value columns j = 16w + i; state rows 16 db + 4g + r
    DF_CLOCKS(0);
    const int j = 16 * w + i;
    f32x4 S[4 * KH];
    {
      // all loads at once (an empty view when there is no entering state: zeros, no branch per element)
      const __amdgpu_buffer_rsrc_t sv = f32_view(S0 ? S0 + R.state() : nullptr, DKEY * DKEY);
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[db][r] = load_f32(sv, (16 * db + 4 * g + r) * DKEY + j);
    }
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
      DF_STAMP(4 + 2 * c);  // the chunk's phase: operand reads, contractions, result stores (across the A barrier)
      const int t0 = c * C, h = c & 1;
      const __bf16* Qs = stg + h * kStage;  // KH tiles: key columns 64 n .. of tile n
      const __bf16* Ks = Qs + KH * TILE;
      const __bf16* Vs = Qs + 2 * KH * TILE;
      const __bf16* Xs = Vs + TILE;
      const float* vs = vec + h * kFwdVec;
      const float* Ls = vs;
      const float* eLs = vs + C;
      const float* ws = vs + 2 * C;
      const float* bs = vs + 3 * C;
      const int out_bytes = min(C, T - t0) * DKEY * (int)sizeof(__bf16);
      // the entering state, bf16, transposed: row j holds key rows d contiguously
      if (sent) {
        __bf16* sc = sent + R.stateT(NC, c) + (size_t)j * DKEY + 4 * g;
#pragma unroll
        for (int db = 0; db < 4 * KH; ++db) *reinterpret_cast<bf16x4*>(sc + 16 * db) = to_bf16x4(S[db]);
      }
      // U = K S (rows t, this wave's columns); rhs = beta (V - eL U)
      bf16x8 sp[2 * KH];  // the state as operands: key rows 32 m .. 32 m + 31
#pragma unroll
      for (int m = 0; m < 2 * KH; ++m) sp[m] = pack(S[2 * m], S[2 * m + 1]);
      f32x4 R4[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 u = zero4();
#pragma unroll
        for (int m = 0; m < 2 * KH; ++m) u = pgn_mfma(frag(Ks + (m >> 1) * TILE, 16 * tb + i, m & 1, g), sp[m], u);
        const f32x4 vv = to_f32x4(ds_read_tr(Vs + (16 * tb + 4 * g + (i >> 2)) * kPitch + 16 * w + 4 * (i & 3)));
        const f32x4 bv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
        const f32x4 ev = *reinterpret_cast<const f32x4*>(eLs + 16 * tb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) R4[tb][r] = bv[r] * (vv[r] - ev[r] * u[r]);
      }
      // W = X rhs (X lower triangular); rows past T fall outside the store's range and are dropped
      const __amdgpu_buffer_rsrc_t w_out =
          __builtin_amdgcn_make_buffer_rsrc(Wout + voff + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
      const bf16x8 r01 = pack(R4[0], R4[1]), r23 = pack(R4[2], R4[3]);
      f32x4 Wt[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        Wt[tb] = pgn_mfma(frag(Xs, 16 * tb + i, 0, g), r01, zero4());
        if (tb >= 2) Wt[tb] = pgn_mfma(frag(Xs, 16 * tb + i, 1, g), r23, Wt[tb]);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, quad_rows(Wt[tb], i)), w_out,
                                              ((16 * tb + 4 * g + (i & 3)) * DKEY + 16 * w + 4 * (i >> 2)) *
                                                  (int)sizeof(__bf16), 0, 0);
      }
      __syncthreads();  // A complete

      // O^T tiles (value rows 16w + 4g + r, token lane 16 tb + i) = W^T A^T + eL_t (S^T Q^T): the decay of the
      // state read is one factor per output column, applied to the accumulator rather than to the Q operand
      const __amdgpu_buffer_rsrc_t o_out =
          __builtin_amdgcn_make_buffer_rsrc(o + voff + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
      const bf16x8 w01 = pack(Wt[0], Wt[1]), w23 = pack(Wt[2], Wt[3]);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int tl = 16 * tb + i;
        f32x4 acc = pgn_mfma(w01, frag(As, tl, 0, g), zero4());
        if (tb >= 2) acc = pgn_mfma(w23, frag(As, tl, 1, g), acc);
        f32x4 qs = zero4();
#pragma unroll
        for (int m = 0; m < 2 * KH; ++m) qs = pgn_mfma(sp[m], frag(Qs + (m >> 1) * TILE, tl, m & 1, g), qs);
        acc += eLs[tl] * qs;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), o_out,
                                              (tl * DKEY + 16 * w + 4 * g) * (int)sizeof(__bf16), 0, 0);
      }
      // S <- a S + K^T (w o W): the per-token weight w_t scales W's fp32 rows before they are rounded, so K enters
      // the product as it is staged
      const float a_c = __expf(Ls[C - 1]);
      bf16x8 ww[2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
        ww[m] = pack(Wt[2 * m] * *reinterpret_cast<const f32x4*>(ws + 32 * m + 4 * g),
                     Wt[2 * m + 1] * *reinterpret_cast<const f32x4*>(ws + 32 * m + 16 + 4 * g));
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db) {
        const __bf16* Kh = Ks + (db >> 2) * TILE;
        S[db] = S[db] * a_c;
        S[db] = pgn_mfma(frag_tr(Kh, 16 * (db & 3), 0, g, i), ww[0], S[db]);
        S[db] = pgn_mfma(frag_tr(Kh, 16 * (db & 3), 1, g, i), ww[1], S[db]);
      }
      DF_STAMP(5 + 2 * c);
      __syncthreads();  // end of the chunk
    }
#pragma unroll
    for (int db = 0; db < 4 * KH; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) Sfin[R.state() + (size_t)(16 * db + 4 * g + r) * DKEY + j] = S[db][r];
  } else {
    // ================= service waves: thread b carries 16-byte row segments b and b + 256 of each staged tile
    DF_CLOCKS(0);
    const int a = w - 4;  // this wave's t block for the scores
    const int b = tid & 255;
    constexpr int NT = 2 * KH + 2;  // tiles per chunk: Q halves, K halves, V, X
    bf16x8 sg[NT][2];
    float pla = 0.f, pbe = 0.f;
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const __bf16* src = u < KH ? q + R.rows(T) + (size_t)n0 * DKEY + 64 * u
                          : u < 2 * KH ? k + R.rows(T) + (size_t)n0 * DKEY + 64 * (u - KH)
                          : u == 2 * KH ? v + voff + (size_t)n0 * DKEY
                                        : X + ((size_t)R.hw * NC + cn) * C * C;
        const int rows = u == NT - 1 ? C : nr, ld = u == NT - 1 ? C : DKEY;
        sg[u][0] = load_seg(src, rows, b, ld);
        sg[u][1] = load_seg(src, rows, b + 256, ld);
      }
      // every service wave loads them (wave 4 uses them): no branch around a load
      pla = load_f32_lane(la + R.tok(T) + n0, nr, x.l);
      pbe = load_f32_lane(be + R.tok(T) + n0, nr, x.l);
    };
    auto stage = [&](int hh) {
      __bf16* base = stg + hh * kStage;
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        put_seg(base + u * TILE, sg[u][0], b);
        put_seg(base + u * TILE, sg[u][1], b + 256);
      }
      if (a == 0) {
        float* vs = vec + hh * kFwdVec;
        chunk_decays(pla, x.l, vs, vs + C, vs + 2 * C);
        vs[3 * C + x.l] = pbe;
      }
    };
    load(0);
    stage(0);
    load(min(1, NC - 1));
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
      const int h = c & 1;
      const __bf16* Qs = stg + h * kStage;
      const __bf16* Ks = Qs + KH * TILE;
      const float* Ls = vec + h * kFwdVec;
      // decayed scores A[t][s] = (q_t . k_s) exp(L_t - L_s), s <= t, into As (row t). The ten nonzero 16 x 16
      // blocks split 2, 3, 3, 2 over the four waves (wave a takes row block a's, and row block 3's first two go to
      // waves 0 and 1), so the last row block's four do not hold up the A barrier the chain waves wait at; each wave
      // zeroes its row block above the diagonal.
      DF_STAMP(4 + 2 * c);
      {
        auto block = [&](int tb, int sb) {
          const int t = 16 * tb + i;
          f32x4 pt = zero4();
#pragma unroll
          for (int m = 0; m < 2 * KH; ++m)
            pt = pgn_mfma(frag(Ks + (m >> 1) * TILE, 16 * sb + i, m & 1, g), frag(Qs + (m >> 1) * TILE, t, m & 1, g),
                          pt);
          const float Lt = Ls[t];
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) pt[r] *= masked_decay(Lt - Lsv[r], 16 * sb + 4 * g + r <= t);
          store_T(As, 16 * tb, 16 * sb, g, i, pt);
        };
#pragma unroll
        for (int sb = 1; sb < 4; ++sb)
          if (sb > a) store_T(As, 16 * a, 16 * sb, g, i, zero4());
        if (a == 0) {
          block(0, 0);
          block(3, 0);
        } else if (a == 1) {
          block(1, 0);
          block(1, 1);
          block(3, 1);
        } else if (a == 2) {
          block(2, 0);
          block(2, 1);
          block(2, 2);
        } else {
          block(3, 2);
          block(3, 3);
        }
      }
      DF_STAMP(5 + 2 * c);
      __syncthreads();  // A complete
      // the next chunk's tiles (loaded a chunk ago), then the loads of the one after (unconditional: the last ones
      // re-read the last chunk, unused)
      if (c + 1 < NC) stage(h ^ 1);
      load(min(c + 2, NC - 1));
      __syncthreads();  // end of the chunk
    }
  }
  DF_CLOCKS(2);
#undef DF_STAMP
#undef DF_CLOCKS
}

// ------------------------------------------------------------------------------------------------------------------
// forward with the chunk inverses formed on chip (64-wide heads): aspin_delta_fwd's chain and service waves plus
// kNIW = 3 inverse waves, one workgroup of 11 waves per (batch, head), so a forward is one launch and X need not pass
// through memory. Inverse wave iw (waves 8..10) forms X for the chunks iw, iw + 3, iw + 6, ..., each over the three
// iterations before the chain reaches it, with the one-wave form of aspin_delta_inv's algorithm (N blocks from a bf16
// MFMA K K^T and fp32 decays, the diagonal blocks by substitution, one column per lane, the blocks below by block
// forward substitution on fp32 MFMA; every entry by the same operations in the same order as aspin_delta_inv, so X is
// bit-identical to its), in six phases, one per barrier interval: keys staged (loaded an iteration earlier), decay
// scan and the ten N blocks; the four diagonal blocks; the three block levels; X into the chunk's X tile (the chain is
// done with the tile's previous chunk by then) and, when asked for, to memory, then the next chunk's loads. The first
// kNIW iterations run before the chain's first chunk (the service waves stage chunk 0 meanwhile). The outputs o, W,
// sent and X are each written only when the caller passes a buffer; without o, the chain waves skip the output
// products and the service waves the scores (the state pass a recomputing backward needs).
constexpr int kNIW = 3;                         // inverse waves; a chunk's inverse spans kNIW iterations
constexpr int kIBS = 16 * 16 + 4;               // floats per 16 x 16 block (16-byte pad: blocks start on other banks)
constexpr int kInvScratch = 23 * kIBS + 2 * C;  // floats per inverse wave: N^T (10 blocks), X (10), level sums (3), L, beta
PGN_DEVICE int iblk(int tb, int sb) { return (tb * (tb + 1) / 2 + sb) * kIBS; }
// dynamic LDS: the staged tiles, the scores and the per-token vectors; the inverse waves' scratch is a static array of
// its own (so the compiler knows their accesses never alias the tiles' and can issue them ahead)
constexpr size_t fwd_inv_smem() { return (2 * 4 * TILE + TILE) * sizeof(__bf16) + 2 * kFwdVec * sizeof(float); }
static_assert(fwd_inv_smem() + kNIW * kInvScratch * sizeof(float) <= 160 * 1024, "the forward's LDS fits a CU");

__global__ __launch_bounds__(64 * (8 + kNIW)) void aspin_delta_fwd_inv(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ be, const float* __restrict__ S0, __bf16* __restrict__ o,
    __bf16* __restrict__ Wout, float* __restrict__ Sfin, __bf16* __restrict__ sent, __bf16* __restrict__ Xout, int T,
    int NC, int maps) {
  constexpr int KH = 1, DKEY = 64;
  constexpr int kStage = 4 * TILE;  // Q, K, V, X
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* stg = reinterpret_cast<__bf16*>(smem);           // two sets of staged tiles, chunk c uses set c & 1
  __bf16* As = stg + 2 * kStage;                            // As[t][s] = A[t][s]
  float* vec = reinterpret_cast<float*>(As + TILE);         // two vector sets, chunk c uses set c & 1
  __shared__ __align__(16) float inv[kNIW * kInvScratch];  // the inverse waves' scratch

  const WaveIdx x = wave_idx();
  const int w = x.w, tid = threadIdx.x;
  // maps > 0 (the state pass of carried windows' affine maps): workgroup maps + n reruns sequence n with zero values
  // from the identity state, so its final state is the sequence's state map, written after the first maps states
  const bool idm = maps > 0 && (int)blockIdx.x >= maps;
  const DeltaRows<KH> R(idm ? (int)blockIdx.x - maps : (int)blockIdx.x);
  const size_t voff = R.vals(T);
  // instrumented build: as aspin_delta_fwd's, for the chain and service waves (first buffer: per wave, clocks where
  // its role's branch starts (entries 0, 1) and at the kernel's end (2, 3), then the start and end of its phase for
  // chunk c (4 + 2 c, 5 + 2 c)); the inverse waves write the second buffer, per (head, chunk) 16 entries: clocks at
  // the inverse's start (0, 1), the start and end of phase p (2 + 2p, 3 + 2p), clocks at its end (14, 15)
#define DF_STAMP(k) PGN_STAMP((blockIdx.x * 8 + w) * (4 + 2 * NC) + (k))
#define DF_CLOCKS(k) PGN_STAMP_CLOCKS((blockIdx.x * 8 + w) * (4 + 2 * NC) + (k))
#define DI_STAMP(cn, k) PGN_STAMP_AUX(((int)blockIdx.x * NC + (cn)) * 16 + (k))
#define DI_CLOCKS(cn, k) PGN_STAMP_CLOCKS_AUX(((int)blockIdx.x * NC + (cn)) * 16 + (k))

  if (w < 4) {
    // ================= chain waves: value columns j = 16w + i; state rows 16 db + 4g + r
    DF_CLOCKS(0);
    f32x4 S[4];
    {
      const int g = x.g, j = 16 * w + x.i;
      const __amdgpu_buffer_rsrc_t sv = f32_view(S0 && !idm ? S0 + R.state() : nullptr, DKEY * DKEY);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * db + 4 * g + r;
          S[db][r] = idm ? (d == j ? 1.f : 0.f) : load_f32(sv, d * DKEY + j);
        }
    }
    for (int it = 0; it < 2 * kNIW; ++it) __syncthreads();  // the kNIW iterations that form X_0
    for (int c = 0; c < NC; ++c) {
      // lane indices recomputed per chunk from an opaque copy of the thread index (loop-invariant LDS addresses
      // hoisted out of the chunk loop would each hold a register)
      const WaveIdx xo = wave_idx_opaque();
      const int g = xo.g, i = xo.i, j = 16 * w + i;
      const int t0 = c * C, h = c & 1;
      const __bf16* Qs = stg + h * kStage;
      const __bf16* Ks = Qs + TILE;
      const __bf16* Vs = Qs + 2 * TILE;
      const __bf16* Xs = Qs + 3 * TILE;
      const float* vs = vec + h * kFwdVec;
      const float* Ls = vs;
      const float* eLs = vs + C;
      const float* ws = vs + 2 * C;
      const float* bs = vs + 3 * C;
      const int out_bytes = min(C, T - t0) * DKEY * (int)sizeof(__bf16);
      DF_STAMP(4 + 2 * c);  // the chunk's phase: operand reads, contractions, result stores (across the A barrier)
      if (sent) {
        __bf16* sc = sent + R.stateT(NC, c) + (size_t)j * DKEY + 4 * g;
#pragma unroll
        for (int db = 0; db < 4; ++db) *reinterpret_cast<bf16x4*>(sc + 16 * db) = to_bf16x4(S[db]);
      }
      // U = K S (rows t, this wave's columns); rhs = beta (V - eL U)
      bf16x8 sp[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) sp[m] = pack(S[2 * m], S[2 * m + 1]);
      f32x4 R4[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 u = zero4();
#pragma unroll
        for (int m = 0; m < 2; ++m) u = pgn_mfma(frag(Ks, 16 * tb + i, m, g), sp[m], u);
        const f32x4 vv = to_f32x4(ds_read_tr(Vs + (16 * tb + 4 * g + (i >> 2)) * kPitch + 16 * w + 4 * (i & 3)));
        const f32x4 bv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
        const f32x4 ev = *reinterpret_cast<const f32x4*>(eLs + 16 * tb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) R4[tb][r] = bv[r] * (vv[r] - ev[r] * u[r]);
      }
      // W = X rhs; stored when asked for (no W buffer: an empty range, the stores dropped)
      const __amdgpu_buffer_rsrc_t w_out = __builtin_amdgcn_make_buffer_rsrc(
          Wout ? Wout + voff + (size_t)t0 * DKEY : nullptr, (short)0, Wout ? out_bytes : 0, 0x00020000);
      const bf16x8 r01 = pack(R4[0], R4[1]), r23 = pack(R4[2], R4[3]);
      f32x4 Wt[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        Wt[tb] = pgn_mfma(frag(Xs, 16 * tb + i, 0, g), r01, zero4());
        if (tb >= 2) Wt[tb] = pgn_mfma(frag(Xs, 16 * tb + i, 1, g), r23, Wt[tb]);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, quad_rows(Wt[tb], i)), w_out,
                                              ((16 * tb + 4 * g + (i & 3)) * DKEY + 16 * w + 4 * (i >> 2)) *
                                                  (int)sizeof(__bf16), 0, 0);
      }
      __syncthreads();  // A complete
      if (o) {
        // O^T tiles (value rows 16w + 4g + r, token lane 16 tb + i) = W^T A^T + eL_t (S^T Q^T)
        const __amdgpu_buffer_rsrc_t o_out =
            __builtin_amdgcn_make_buffer_rsrc(o + voff + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
        const bf16x8 w01 = pack(Wt[0], Wt[1]), w23 = pack(Wt[2], Wt[3]);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const int tl = 16 * tb + i;
          f32x4 acc = pgn_mfma(w01, frag(As, tl, 0, g), zero4());
          if (tb >= 2) acc = pgn_mfma(w23, frag(As, tl, 1, g), acc);
          f32x4 qs = zero4();
#pragma unroll
          for (int m = 0; m < 2; ++m) qs = pgn_mfma(sp[m], frag(Qs, tl, m, g), qs);
          acc += eLs[tl] * qs;
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), o_out,
                                                (tl * DKEY + 16 * w + 4 * g) * (int)sizeof(__bf16), 0, 0);
        }
      }
      // S <- a S + K^T (w o W)
      const float a_c = __expf(Ls[C - 1]);
      bf16x8 ww[2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
        ww[m] = pack(Wt[2 * m] * *reinterpret_cast<const f32x4*>(ws + 32 * m + 4 * g),
                     Wt[2 * m + 1] * *reinterpret_cast<const f32x4*>(ws + 32 * m + 16 + 4 * g));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        S[db] = S[db] * a_c;
        S[db] = pgn_mfma(frag_tr(Ks, 16 * db, 0, g, i), ww[0], S[db]);
        S[db] = pgn_mfma(frag_tr(Ks, 16 * db, 1, g, i), ww[1], S[db]);
      }
      DF_STAMP(5 + 2 * c);
      __syncthreads();  // end of the chunk
    }
    {
      const int g = x.g, j = 16 * w + x.i;
      float* const Sf = Sfin + (idm ? (size_t)maps * DKEY * DKEY : 0) + R.state();
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) Sf[(size_t)(16 * db + 4 * g + r) * DKEY + j] = S[db][r];
    }
  } else if (w < 8) {
    // ================= service waves: thread b carries 16-byte row segments b and b + 256 of Q, K and V
    const int a = w - 4;  // this wave's t block for the scores
    const int b = tid & 255;
    DF_CLOCKS(0);
    bf16x8 sg[3][2];
    float pla = 0.f, pbe = 0.f;
    // without o (the state pass) nothing reads Q: its tile is neither loaded nor staged
    const int u0 = o ? 0 : 1;
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (u < u0) continue;
        const __bf16* src = u == 0 ? q + R.rows(T) + (size_t)n0 * DKEY
                          : u == 1 ? k + R.rows(T) + (size_t)n0 * DKEY
                                   : v + voff + (size_t)n0 * DKEY;
        const int rows = u == 2 && idm ? 0 : nr;  // a state map's values are zero: an empty range reads zero
        sg[u][0] = load_seg(src, rows, b);
        sg[u][1] = load_seg(src, rows, b + 256);
      }
      pla = load_f32_lane(la + R.tok(T) + n0, nr, x.l);
      pbe = load_f32_lane(be + R.tok(T) + n0, nr, x.l);
    };
    auto stage = [&](int hh) {
      __bf16* base = stg + hh * kStage;
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (u < u0) continue;
        put_seg(base + u * TILE, sg[u][0], b);
        put_seg(base + u * TILE, sg[u][1], b + 256);
      }
      if (a == 0) {
        float* vs = vec + hh * kFwdVec;
        chunk_decays(pla, x.l, vs, vs + C, vs + 2 * C);
        vs[3 * C + x.l] = pbe;
      }
    };
    load(0);
    for (int it = 0; it < 2 * kNIW - 2; ++it) __syncthreads();  // the kNIW iterations that form X_0
    stage(0);
    __syncthreads();
    load(min(1, NC - 1));
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
      const WaveIdx xo = wave_idx_opaque();
      const int g = xo.g, i = xo.i;
      const int h = c & 1;
      const __bf16* Qs = stg + h * kStage;
      const __bf16* Ks = Qs + TILE;
      const float* Ls = vec + h * kFwdVec;
      DF_STAMP(4 + 2 * c);
      if (o) {
        // decayed scores A[t][s] = (q_t . k_s) exp(L_t - L_s), s <= t, into As (row t); the ten nonzero blocks split
        // 2, 3, 3, 2 over the four waves, each wave zeroing its row block above the diagonal
        auto block = [&](int tb, int sb) {
          const int t = 16 * tb + i;
          f32x4 pt = zero4();
#pragma unroll
          for (int m = 0; m < 2; ++m) pt = pgn_mfma(frag(Ks, 16 * sb + i, m, g), frag(Qs, t, m, g), pt);
          const float Lt = Ls[t];
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) pt[r] *= masked_decay(Lt - Lsv[r], 16 * sb + 4 * g + r <= t);
          store_T(As, 16 * tb, 16 * sb, g, i, pt);
        };
#pragma unroll
        for (int sb = 1; sb < 4; ++sb)
          if (sb > a) store_T(As, 16 * a, 16 * sb, g, i, zero4());
        if (a == 0) {
          block(0, 0);
          block(3, 0);
        } else if (a == 1) {
          block(1, 0);
          block(1, 1);
          block(3, 1);
        } else if (a == 2) {
          block(2, 0);
          block(2, 1);
          block(2, 2);
        } else {
          block(3, 2);
          block(3, 3);
        }
      }
      DF_STAMP(5 + 2 * c);
      __syncthreads();  // A complete
      if (c + 1 < NC) stage(h ^ 1);
      load(min(c + 2, NC - 1));  // unconditional (the last ones re-read the last chunk, unused)
      __syncthreads();  // end of the chunk
    }
  } else {
    // ================= inverse waves: chunk cn is formed by wave cn % kNIW over iterations cn - kNIW .. cn - 1, in
    // phases 0 .. 2 kNIW - 1 (two per iteration, before and after the A barrier): 0 keys staged, decay scan, N blocks;
    // 1 the diagonal blocks; 2, 3, 4 the three block levels; 5 X into the chunk's X tile (and to memory), then the
    // loads of the wave's next chunk
    static_assert(kNIW == 3, "six phases over three iterations");
    const int iw = w - 8;
    // the inverse waves issue first when their SIMD has a choice: the chain and service waves leave gaps that they
    // fill, and an iteration lasts as long as the slowest phase
    __builtin_amdgcn_s_setprio(2);
    float* NT = inv + iw * kInvScratch;  // N^T blocks: NT(tb, sb)[s' * BP + t'] = N[16 tb + t'][16 sb + s']
    float* Xf = NT + 10 * kIBS;          // X blocks: Xf(ib, jb)[r * BP + c] = X[16 ib + r][16 jb + c]
    float* Tt = Xf + 10 * kIBS;          // per-level sums, one block per product
    float* Li = Tt + 3 * kIBS;
    float* bi = Li + C;
    __bf16* Kst = reinterpret_cast<__bf16*>(Xf);  // the keys, staged in the X block area until N is formed
    static_assert(TILE * sizeof(__bf16) <= 10 * kIBS * sizeof(float), "the key tile fits the X block area");
    bf16x8 seg[8];
    float lav = 0.f, bev = 0.f;
    auto iload = [&](int cn) {  // keys in 16-byte row segments (rows past T as zeros), decays and strengths
      const int t0 = cn * C, nr = min(C, T - t0);
      const __bf16* kc = k + R.rows(T) + (size_t)t0 * DKEY;
#pragma unroll
      for (int n = 0; n < 8; ++n) seg[n] = load_seg(kc, nr, x.l + 64 * n);
      lav = load_f32_lane(la + R.tok(T) + t0, nr, x.l);
      bev = load_f32_lane(be + R.tok(T) + t0, nr, x.l);
    };
    // Each phase reads what it needs into registers before it writes anything: its LDS writes could alias its
    // reads (one scratch array), so the compiler would otherwise issue each read only after the writes before it.
    auto phase_n = [&]() {  // keys staged, decay scan, the N^T blocks
      const WaveIdx xo = wave_idx_opaque();
      const int l = xo.l, g = xo.g, i = xo.i;
#pragma unroll
      for (int n = 0; n < 8; ++n) put_seg(Kst, seg[n], l + 64 * n);
      Li[l] = incl_scan64(lav, l);
      bi[l] = bev;
      bf16x8 kf[4][2];
      float Lt[4], bt[4];
      f32x4 Lsv[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int m = 0; m < 2; ++m) kf[rb][m] = frag(Kst, 16 * rb + i, m, g);
        Lt[rb] = Li[16 * rb + i];
        bt[rb] = bi[16 * rb + i];
        Lsv[rb] = *reinterpret_cast<const f32x4*>(Li + 16 * rb + 4 * g);
      }
      f32x4 nv[10];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int t = 16 * tb + i;
#pragma unroll
        for (int sb = 0; sb <= tb; ++sb) {
          f32x4 acc = zero4();
          acc = pgn_mfma(kf[sb][0], kf[tb][0], acc);
          acc = pgn_mfma(kf[sb][1], kf[tb][1], acc);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = 16 * sb + 4 * g + r;
            nv[tb * (tb + 1) / 2 + sb][r] = bt[tb] * acc[r] * masked_decay(Lt[tb] - Lsv[sb][r], s < t);
          }
        }
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int sb = 0; sb <= tb; ++sb) {
          float* nb = NT + iblk(tb, sb);
#pragma unroll
          for (int r = 0; r < 4; ++r) nb[(4 * g + r) * BP + i] = nv[tb * (tb + 1) / 2 + sb][r];
        }
    };
    // X_ii = (I + N_ii)^-1 by forward substitution, one column of one diagonal block per lane (the keys in the X
    // block area are dead once N is formed)
    auto phase_diag = [&]() {
      const WaveIdx xo = wave_idx_opaque();
      const int bb = xo.l >> 4, cl = xo.l & 15;
      const float* nd = NT + iblk(bb, bb);
      float xd[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) xd[t] = (t == cl) ? 1.f : 0.f;
#pragma unroll
      for (int s = 0; s < 15; ++s) {
        const float xs = xd[s];
#pragma unroll
        for (int t4 = (s + 1) & ~3; t4 < 16; t4 += 4) {
          const f32x4 n = *reinterpret_cast<const f32x4*>(nd + s * BP + t4);  // N[16b + t][16b + s], t = t4..
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (t4 + u > s) xd[t4 + u] -= n[u] * xs;
        }
      }
      float* xb = Xf + iblk(bb, bb);
#pragma unroll
      for (int t = 0; t < 16; ++t) xb[t * BP + cl] = xd[t];
    };
    // level d: X_ij = -X_ii sum_{k=j}^{i-1} N_ik X_kj for i - j = d, on fp32 MFMA (v_mfma_f32_16x16x4f32: A[r][k] in
    // lane r + 16k, B[k][c] in lane c + 16k, D[4g + e][c] in lane c + 16g)
    auto phase_level = [&](int d) {
      const WaveIdx xo = wave_idx_opaque();
      const int r16 = xo.l & 15, k4 = xo.l >> 4;
      // one 16 x 16 x 16 product's operands, A[r][k] and B[k][c] for this lane's k = 4 kk + k4 (A read transposed
      // when `at`: A[r][k] = Ab[k * BP + r]), and the product accumulated onto acc
      struct Ops {
        float a[4], b[4];
      };
      auto rd = [&](const float* Ab, bool at, const float* Bb) {
        Ops o_;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int kx = 4 * kk + k4;
          o_.a[kk] = at ? Ab[kx * BP + r16] : Ab[r16 * BP + kx];
          o_.b[kk] = Bb[kx * BP + r16];
        }
        return o_;
      };
      auto mm = [&](f32x4 acc, const Ops& o_) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o_.a[kk], o_.b[kk], acc, 0, 0, 0);
        return acc;
      };
      // T_j = sum_{k=j}^{i-1} N_ik X_kj (at most three products a level, three terms each: d = 1 has 3 x 1, d = 2
      // 2 x 2, d = 3 1 x 3); all operands read first
      Ops to[3][3];
#pragma unroll
      for (int jb = 0; jb < 3; ++jb)
#pragma unroll
        for (int u = 0; u < 3; ++u)
          if (jb + d < 4 && u < d) to[jb][u] = rd(NT + iblk(jb + d, jb + u), true, Xf + iblk(jb + u, jb));
      f32x4 Tacc[3];
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        if (jb + d < 4) {
          f32x4 acc = zero4();
#pragma unroll
          for (int u = 0; u < 3; ++u)
            if (u < d) acc = mm(acc, to[jb][u]);
          Tacc[jb] = acc;
        }
      }
#pragma unroll
      for (int jb = 0; jb < 3; ++jb)
        if (jb + d < 4)
#pragma unroll
          for (int e = 0; e < 4; ++e) Tt[jb * kIBS + (4 * k4 + e) * BP + r16] = Tacc[jb][e];
      // X_ij = -X_ii T_j
      Ops xo2[3];
#pragma unroll
      for (int jb = 0; jb < 3; ++jb)
        if (jb + d < 4) xo2[jb] = rd(Xf + iblk(jb + d, jb + d), false, Tt + jb * kIBS);
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        if (jb + d < 4) {
          const f32x4 xr = mm(zero4(), xo2[jb]);
          float* xo_ = Xf + iblk(jb + d, jb);
#pragma unroll
          for (int e = 0; e < 4; ++e) xo_[(4 * k4 + e) * BP + r16] = -xr[e];
        }
      }
    };
    // X (bf16, row-major; zero above the diagonal blocks) into chunk cn's X tile and, when asked for, to memory, in
    // 16-byte row segments (every lane reads a block, those above the diagonal selected away: no divergent branch)
    auto phase_store = [&](int cn) {
      const WaveIdx xo = wave_idx_opaque();
      const int l = xo.l;
      __bf16* Xs = stg + (cn & 1) * kStage + 3 * TILE;
      __bf16* Xg = Xout ? Xout + ((size_t)R.hw * NC + cn) * C * C : nullptr;
      f32x4 xv[8][2];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int e = l + 64 * n, r = e >> 3, c0 = 8 * (e & 7);
        const int rb = r >> 4, cb = c0 >> 4;
        const float* xb = Xf + iblk(rb, cb <= rb ? cb : 0) + (r & 15) * BP + (c0 & 15);
        xv[n][0] = *reinterpret_cast<const f32x4*>(xb);
        xv[n][1] = *reinterpret_cast<const f32x4*>(xb + 4);
      }
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int e = l + 64 * n, r = e >> 3, c0 = 8 * (e & 7);
        const bool keep = (c0 >> 4) <= (r >> 4);
        bf16x8 out;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          out[u] = (__bf16)(keep ? xv[n][0][u] : 0.f);
          out[4 + u] = (__bf16)(keep ? xv[n][1][u] : 0.f);
        }
        put_seg(Xs, out, e);
        if (Xg) *reinterpret_cast<bf16x8*>(Xg + r * C + c0) = out;
      }
    };
    auto phase = [&](int ph, int cn) {
      if (ph == 0) DI_CLOCKS(cn, 0);
      DI_STAMP(cn, 2 + 2 * ph);
      if (ph == 0) phase_n();
      else if (ph == 1) phase_diag();
      else if (ph < 5) phase_level(ph - 1);
      else {
        phase_store(cn);
        if (cn + kNIW < NC) iload(cn + kNIW);
      }
      DI_STAMP(cn, 3 + 2 * ph);
      if (ph == 5) DI_CLOCKS(cn, 14);
    };
    if (iw < NC) iload(iw);
    for (int it = -kNIW; it < NC; ++it) {
      const int cn = it + 1 + ((iw - it - 1) % kNIW + kNIW) % kNIW;  // this wave's chunk: cn = iw mod kNIW
      const int ph = 2 * (it - (cn - kNIW));
      const bool mine = cn >= 0 && cn < NC;
      if (mine) phase(ph, cn);
      __syncthreads();  // A complete
      if (mine) phase(ph + 1, cn);
      __syncthreads();  // end of the chunk
    }
  }
  if (w < 8) DF_CLOCKS(2);
#undef DF_STAMP
#undef DF_CLOCKS
#undef DI_STAMP
#undef DI_CLOCKS
}

// ------------------------------------------------------------------------------------------------------------------
// backward, the sequential part: one workgroup of 8 waves per scan (a 64-wide head, or one value half of a 128-wide
// one), chunks in reverse. Waves 0-3 carry the chain, wave w owning value columns 16w..16w+15 with its columns of dS
// (all key rows) in fp32 registers; nothing on the chain is shared between them. Waves 4-7 serve them: per chunk they
// compute the decayed scores A^T (the only operand the four chain waves share), then stage the next chunk's tiles
// (loaded into registers a chunk earlier still), run its decay scan, and reduce the previous chunk's value-column
// partial sums into rsum. Two barriers per chunk: A^T ready (the chain waves do their dS-side and dS-free products
// before it), and the end of the chunk. Operands contracted over a tile's row index use the LDS transpose read.
// LDS per chunk: Q (KH tiles), S_c transposed (KH tiles: value rows j, key columns 64 n .. of tile n) and dO, read
// only before the A^T barrier, in one copy that the service waves restage for the next chunk after that barrier; K
// (KH tiles), V and X, read after it too, double-buffered.
template <int KH>
constexpr int chain_single() { return (2 * KH + 1) * TILE; }
template <int KH>
constexpr int chain_double() { return (KH + 2) * TILE; }
constexpr int kChainVec = 4 * C + 8 * C;  // L, eL, w, beta; per-wave partial sums of drhs V and drhs U

template <int KH>
__global__ __launch_bounds__(512) void aspin_delta_bwd_chain(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ be, const __bf16* __restrict__ X,
    const __bf16* __restrict__ sent, const __bf16* __restrict__ dO, const float* __restrict__ dSfin,
    __bf16* __restrict__ drhs, __bf16* __restrict__ dSc, float* __restrict__ rsum,
    float* __restrict__ dS0, int T, int NC, int nscans) {
  constexpr int DKEY = 64 * KH;
  constexpr int kSingle = chain_single<KH>(), kDouble = chain_double<KH>();
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* sgl = reinterpret_cast<__bf16*>(smem);          // Q, S_c, dO of the current chunk
  __bf16* dbl = sgl + kSingle;                             // two sets of K, V, X: chunk c uses set c & 1
  __bf16* AT = dbl + 2 * kDouble;                          // AT[t][s] = A[s][t]
  float* vec = reinterpret_cast<float*>(AT + TILE);        // two vector sets, chunk c uses set c & 1
  // instrumented build: per wave, clocks where its role's branch starts (entries 0, 1) and at the kernel's end (2, 3),
  // then the start and end of its phase for chunk cc (4 + 2 cc, 5 + 2 cc)
#define DB_STAMP(k) PGN_STAMP((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * (4 + 2 * NC) + (k))
#define DB_CLOCKS(k) \
  PGN_STAMP_CLOCKS((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * (4 + 2 * NC) + (k))

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  const int bh = scan_of<KH>((int)blockIdx.x);
  if (bh >= nscans) return;  // grid padding (uniform over the workgroup, before any barrier)
  const DeltaRows<KH> R(bh);
  const __bf16* Qs = sgl;
  const __bf16* Ss = sgl + KH * TILE;
  const __bf16* Os = sgl + 2 * KH * TILE;

  if (w < 4) {
    // ================= chain waves: value columns j = 16w + i; dS rows 16 db + 4g + r
    DB_CLOCKS(0);
    const int j = 16 * w + i;
    f32x4 dS[4 * KH];
    {
      // all loads at once (an empty view when there is no final-state gradient: zeros, no branch per element)
      const __amdgpu_buffer_rsrc_t dv = f32_view(dSfin ? dSfin + R.state() : nullptr, DKEY * DKEY);
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS[db][r] = load_f32(dv, (16 * db + 4 * g + r) * DKEY + j);
    }
    __syncthreads();
    for (int cc = NC - 1; cc >= 0; --cc) {
      DB_STAMP(4 + 2 * cc);  // the chunk's phase: operand reads, contractions, result stores (across the A^T barrier)
      const int t0 = cc * C, h = cc & 1;
      const __bf16* Ks = dbl + h * kDouble;
      const __bf16* Vs = Ks + KH * TILE;
      const __bf16* Xs = Vs + TILE;
      float* vs = vec + h * kChainVec;
      const float* Ls = vs;
      const float* eLs = vs + C;
      const float* ws = vs + 2 * C;
      const float* bs = vs + 3 * C;
      float* redV = vs + 4 * C;   // [4][C]
      float* redU = vs + 8 * C;   // [4][C]
      // the gradient on the state leaving this chunk, for the chunk-local kernel, transposed ((j, d): a lane's four
      // consecutive key rows are one 8-byte store)
      {
        __bf16* dst = dSc + R.stateT(NC, cc) + (size_t)j * DKEY + 4 * g;
#pragma unroll
        for (int db = 0; db < 4 * KH; ++db) *reinterpret_cast<bf16x4*>(dst + 16 * db) = to_bf16x4(dS[db]);
      }
      // products that do not need A^T: y = K dS, U = K S_c, Yc = (Q o eL)^T dO, on this wave's columns
      bf16x8 dp[2 * KH], scf[2 * KH];
#pragma unroll
      for (int m = 0; m < 2 * KH; ++m) {
        dp[m] = pack(dS[2 * m], dS[2 * m + 1]);
        scf[m] = frag(Ss + (m >> 1) * TILE, 16 * w + i, m & 1, g);  // S_c[d][j], staged (j, d)
      }
      const bf16x8 oc0 = frag_tr(Os, 16 * w, 0, g, i), oc1 = frag_tr(Os, 16 * w, 1, g, i);  // dO[t][j]
      f32x4 y[4], U[4], Yc[4 * KH];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        y[tb] = zero4();
        U[tb] = zero4();
#pragma unroll
        for (int m = 0; m < 2 * KH; ++m) {
          const bf16x8 kk = frag(Ks + (m >> 1) * TILE, 16 * tb + i, m & 1, g);
          y[tb] = pgn_mfma(kk, dp[m], y[tb]);
          U[tb] = pgn_mfma(kk, scf[m], U[tb]);
        }
      }
      // the per-token factor eL_t on the dO operand, shared by the key blocks, rather than on each Q^T block
      const bf16x8 oe0 = scale_frag_k(oc0, *reinterpret_cast<const f32x4*>(eLs + 4 * g),
                                      *reinterpret_cast<const f32x4*>(eLs + 16 + 4 * g));
      const bf16x8 oe1 = scale_frag_k(oc1, *reinterpret_cast<const f32x4*>(eLs + 32 + 4 * g),
                                      *reinterpret_cast<const f32x4*>(eLs + 48 + 4 * g));
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db) {
        const __bf16* Qh = Qs + (db >> 2) * TILE;
        Yc[db] = pgn_mfma(frag_tr(Qh, 16 * (db & 3), 0, g, i), oe0, zero4());
        Yc[db] = pgn_mfma(frag_tr(Qh, 16 * (db & 3), 1, g, i), oe1, Yc[db]);
      }
      __syncthreads();  // A^T complete (and Q, S_c, dO no longer read: the service waves restage them)

      // dW = A^T dO + w o (K dS)
      f32x4 dW[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = zero4();
        if (tb < 2) acc = pgn_mfma(frag(AT, 16 * tb + i, 0, g), oc0, acc);
        acc = pgn_mfma(frag(AT, 16 * tb + i, 1, g), oc1, acc);
        const f32x4 wv = *reinterpret_cast<const f32x4*>(ws + 16 * tb + 4 * g);
        dW[tb] = acc + wv * y[tb];
      }
      // drhs = X^T dW (X^T upper triangular); dU = -beta eL drhs; per-row partial sums (dV = beta drhs is written
      // by the chunk-local kernel from the stored drhs)
      const int out_bytes = min(C, T - t0) * DKEY * (int)sizeof(__bf16);
      const __amdgpu_buffer_rsrc_t dr_out = __builtin_amdgcn_make_buffer_rsrc(
          drhs + R.vals(T) + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
      const bf16x8 w01 = pack(dW[0], dW[1]), w23 = pack(dW[2], dW[3]);
      f32x4 dU[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = zero4();
        if (tb < 2) acc = pgn_mfma(frag_tr(Xs, 16 * tb, 0, g, i), w01, acc);
        acc = pgn_mfma(frag_tr(Xs, 16 * tb, 1, g, i), w23, acc);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
        const f32x4 ev = *reinterpret_cast<const f32x4*>(eLs + 16 * tb + 4 * g);
        const bf16x4 vv4 = ds_read_tr(Vs + (16 * tb + 4 * g + (i >> 2)) * kPitch + 16 * w + 4 * (i & 3));
        const f32x4 vv = to_f32x4(vv4);  // V[16 tb + 4g + r][j]
        float pr[8];  // per token row 4g + r: drhs V and drhs U, summed over this wave's 16 columns below
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tl = 16 * tb + 4 * g + r;
          dU[tb][r] = -bv[r] * ev[r] * acc[r];
          pr[r] = acc[r] * vv[r];
          pr[4 + r] = acc[r] * U[tb][r];
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, (__bf16)acc[r]), dr_out,
                                                (tl * DKEY + j) * (int)sizeof(__bf16), 0, 0);
        }
        // lane i: the total of pr[(i >> 1) & 7], equal in lanes i and i ^ 1 (the last butterfly step adds the same
        // two values in either order), so both write it: no branch splits the chunk's scheduling region
        const float tot = row_totals16x8(pr, i);
        ((i & 8) ? redU : redV)[w * C + 16 * tb + 4 * g + ((i >> 1) & 3)] = tot;
      }
      // dS_prev = a dS + (Q o eL)^T dO + K^T dU
      const float a_c = __expf(Ls[C - 1]);
      const bf16x8 u01 = pack(dU[0], dU[1]), u23 = pack(dU[2], dU[3]);
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db) {
        const __bf16* Kh = Ks + (db >> 2) * TILE;
        f32x4 acc = dS[db] * a_c + Yc[db];
        acc = pgn_mfma(frag_tr(Kh, 16 * (db & 3), 0, g, i), u01, acc);
        acc = pgn_mfma(frag_tr(Kh, 16 * (db & 3), 1, g, i), u23, acc);
        dS[db] = acc;
      }
      DB_STAMP(5 + 2 * cc);
      __syncthreads();  // end of the chunk
    }
    if (dS0) {
#pragma unroll
      for (int db = 0; db < 4 * KH; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS0[R.state() + (size_t)(16 * db + 4 * g + r) * DKEY + j] = dS[db][r];
    }
  } else {
    // ================= service waves: thread b carries 16-byte row segments b and b + 256 of each staged tile:
    // Q halves, S_c halves, dO (the single copy), then K halves, V, X (the double-buffered set)
    DB_CLOCKS(0);
    const int a = w - 4;       // this wave's t block for the scores
    const int b = tid & 255;
    constexpr int NS = 2 * KH + 1, ND = KH + 2;
    bf16x8 sg[NS + ND][2];
    float pla = 0.f, pbe = 0.f;
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
#pragma unroll
      for (int u = 0; u < NS + ND; ++u) {
        const __bf16* src;
        int rows = nr, ld = DKEY;
        if (u < KH) {
          src = q + R.rows(T) + (size_t)n0 * DKEY + 64 * u;
        } else if (u < 2 * KH) {
          src = sent + R.stateT(NC, cn) + 64 * (u - KH);
          rows = DK;
        } else if (u == 2 * KH) {
          src = dO + R.vals(T) + (size_t)n0 * DKEY;
        } else if (u < NS + KH) {
          src = k + R.rows(T) + (size_t)n0 * DKEY + 64 * (u - NS);
        } else if (u == NS + KH) {
          src = v + R.vals(T) + (size_t)n0 * DKEY;
        } else {
          src = X + ((size_t)R.hw * NC + cn) * C * C;
          rows = C;
          ld = C;
        }
        sg[u][0] = load_seg(src, rows, b, ld);
        sg[u][1] = load_seg(src, rows, b + 256, ld);
      }
      // every service wave loads them (wave 4 uses them): no branch around a load
      pla = load_f32_lane(la + R.tok(T) + n0, nr, x.l);
      pbe = load_f32_lane(be + R.tok(T) + n0, nr, x.l);
    };
    auto stage = [&](int hh) {
#pragma unroll
      for (int u = 0; u < NS + ND; ++u) {
        __bf16* dst = u < NS ? sgl + u * TILE : dbl + hh * kDouble + (u - NS) * TILE;
        put_seg(dst, sg[u][0], b);
        put_seg(dst, sg[u][1], b + 256);
      }
      if (a == 0) {
        float* vs = vec + hh * kChainVec;
        chunk_decays(pla, x.l, vs, vs + C, vs + 2 * C);
        vs[3 * C + x.l] = pbe;
      }
    };
    // rsum of a finished chunk from its vector set: sum_j drhs (V - eL U) and -beta sum_j drhs U (per scan)
    auto reduce = [&](int cn) {
      const float* vs = vec + (cn & 1) * kChainVec;
      const int t = x.l, n0 = cn * C;
      const float* redV = vs + 4 * C;
      const float* redU = vs + 8 * C;
      const float pv_ = redV[t] + redV[C + t] + redV[2 * C + t] + redV[3 * C + t];
      const float pu_ = redU[t] + redU[C + t] + redU[2 * C + t] + redU[3 * C + t];
      if (n0 + t < T) {
        rsum[((size_t)bh * T + n0 + t) * 2 + 0] = pv_ - vs[C + t] * pu_;
        rsum[((size_t)bh * T + n0 + t) * 2 + 1] = -vs[3 * C + t] * pu_;
      }
    };
    load(NC - 1);
    stage((NC - 1) & 1);
    load(max(NC - 2, 0));
    __syncthreads();
    for (int cc = NC - 1; cc >= 0; --cc) {
      const int h = cc & 1;
      const __bf16* Ks = dbl + h * kDouble;
      const float* Ls = vec + h * kChainVec;
      // scores, transposed: AT[t][s] = (q_s . k_t) exp(L_s - L_t), s >= t, zero below. Wave a owns token block a's
      // blocks (a, sb >= a) and zeros (a, sb < a); waves 6 and 7 also take (0, 2) and (0, 3), so the ten nonzero
      // blocks split 2, 3, 3, 2 instead of 4, 3, 2, 1 (wave 4 also reduces the previous chunk's sums)
      DB_STAMP(4 + 2 * cc);
      {
        auto score = [&](int ta, int sb, const bf16x8* kf, float Lt) {
          f32x4 sc = zero4();
#pragma unroll
          for (int m = 0; m < 2 * KH; ++m) sc = pgn_mfma(frag(Qs + (m >> 1) * TILE, 16 * sb + i, m & 1, g), kf[m], sc);
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] *= masked_decay(Lsv[r] - Lt, 16 * sb + 4 * g + r >= 16 * ta + i);
          store_T(AT, 16 * ta, 16 * sb, g, i, sc);
        };
        const int t = 16 * a + i;
        bf16x8 kf[2 * KH];
#pragma unroll
        for (int m = 0; m < 2 * KH; ++m) kf[m] = frag(Ks + (m >> 1) * TILE, t, m & 1, g);
        const float Lt = Ls[t];
        const int last = a == 0 ? 1 : 3;
        for (int sb = 0; sb < 4; ++sb) {
          if (sb < a) store_T(AT, 16 * a, 16 * sb, g, i, zero4());
          else if (sb <= last) score(a, sb, kf, Lt);
        }
        if (a >= 2) {
          bf16x8 kf0[2 * KH];
#pragma unroll
          for (int m = 0; m < 2 * KH; ++m) kf0[m] = frag(Ks + (m >> 1) * TILE, i, m & 1, g);
          score(0, a, kf0, Ls[i]);
        }
      }
      DB_STAMP(5 + 2 * cc);
      __syncthreads();  // A^T complete
      if (a == 0 && cc < NC - 1) reduce(cc + 1);  // the later chunk's sums, before its vector set is reused below
      // the next chunk's tiles (loaded a chunk ago), then the loads of the one after (unconditional: the last ones
      // re-read the first chunk, unused)
      if (cc > 0) stage(h ^ 1);
      load(max(cc - 2, 0));
      __syncthreads();  // end of the chunk
    }
    if (a == 0) reduce(0);
  }
  DB_CLOCKS(2);
#undef DB_STAMP
#undef DB_CLOCKS
}

// ------------------------------------------------------------------------------------------------------------------
// backward, the chunk-local part: one workgroup of 8 waves per (scan, chunk). Waves 0-3 own token block
// t = 16w.. (dQ, row sums), waves 4-7 own token block s = 16(w-4).. in the key role (dK, column sums). Staged:
// Q and K (KH tiles each), W, dO, S_c and dS transposed (KH tiles each: value rows j, key columns), drhs.
template <int KH>
constexpr int local_tiles() { return 4 * KH + 3; }

template <int KH>
__global__ __launch_bounds__(512) void aspin_delta_bwd_local(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const float* __restrict__ la,
    const float* __restrict__ be, const __bf16* __restrict__ Win, const __bf16* __restrict__ sent,
    const __bf16* __restrict__ dO, const __bf16* __restrict__ drhs, const __bf16* __restrict__ dSc,
    const float* __restrict__ rsum, __bf16* __restrict__ dq, __bf16* __restrict__ dq1, __bf16* __restrict__ dk,
    __bf16* __restrict__ dk1, __bf16* __restrict__ dv, float* __restrict__ dla, float* __restrict__ dla1,
    float* __restrict__ dbe, float* __restrict__ dbe1, int T, int NC) {
  constexpr int DKEY = 64 * KH;
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* Qs = reinterpret_cast<__bf16*>(smem);
  __bf16* Ks = Qs + KH * TILE;
  __bf16* Ws = Ks + KH * TILE;
  __bf16* Os = Ws + TILE;        // dO
  __bf16* Ss = Os + TILE;        // S_c transposed, (j, d)
  __bf16* dSs = Ss + KH * TILE;  // dS transposed, (j, d)
  __bf16* Rs = dSs + KH * TILE;  // drhs (t, j)
  float* Ls = reinterpret_cast<float*>(Rs + TILE);
  float* eLs = Ls + C;
  float* ws = eLs + C;
  float* bs = ws + C;
  float* rowT = bs + C;     // rowsum(dA o A) + rowsum(dKK o KK) + eL q.(S dO)
  float* dbe2 = rowT + C;   // sum_{s<t} dN M
  float* colS = dbe2 + C;   // colsum(dA o A) + colsum(dKK o KK)
  float* dwv = colS + C;    // k_s . (dS W_s)
  float* sdot = dwv + C;    // per-wave <S, dS>

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  const int sc = blockIdx.x / NC, c = blockIdx.x - sc * NC;
  const DeltaRows<KH> R(sc);
  const int t0 = c * C, nr = min(C, T - t0);
  const size_t roff = R.rows(T) + (size_t)t0 * DKEY;  // the chunk's q, k, dq, dk rows
  const size_t voff = R.vals(T) + (size_t)t0 * DKEY;  // the chunk's W, dO, drhs, dv rows
  const size_t toff = R.stateT(NC, c);                // this scan's rows of the transposed states
  // instrumented build: 40 entries per workgroup, per wave its entry (0-7), tiles in LDS (8-15), past the barrier
  // (16-23) and end (24-31); wave 0's shader and 100 MHz clocks at entry (32, 33) and end (34, 35)
#define DL_STAMP(k) PGN_STAMP_AUX(blockIdx.x * 40 + (k) + w)
  DL_STAMP(0);
  if (w == 0) PGN_STAMP_CLOCKS_AUX(blockIdx.x * 40 + 32);

  // the chunk's per-token vectors, issued right after the tiles and range-checked (zero past the chunk's end, no
  // branch), so no wave waits on a global load after a barrier: this thread's dV row strength, and this lane's decay,
  // strength and rsum pair (the decay scan and the final dla on wave 0)
  float bt_row, lav, bev, r0, r1;
  {
    // every tile staged untransposed, thread tid carrying 16-byte row segment tid of each (operands contracted over
    // a tile's row index use the LDS transpose read)
    constexpr int NT = local_tiles<KH>();
    bf16x8 sg[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      const __bf16* src;
      int rows = nr;
      if (u < KH) src = q + roff + 64 * u;
      else if (u < 2 * KH) src = k + roff + 64 * (u - KH);
      else if (u == 2 * KH) src = Win + voff;
      else if (u == 2 * KH + 1) src = dO + voff;
      else if (u < 3 * KH + 2) { src = sent + toff + 64 * (u - 2 * KH - 2); rows = DK; }
      else if (u < 4 * KH + 2) { src = dSc + toff + 64 * (u - 3 * KH - 2); rows = DK; }
      else src = drhs + voff;
      sg[u] = load_seg(src, rows, tid, DKEY);
    }
    {
      const __amdgpu_buffer_rsrc_t bv = f32_view(be + R.tok(T) + t0, nr);
      const __amdgpu_buffer_rsrc_t rv = f32_view(rsum + ((size_t)sc * T + t0) * 2, 2 * nr);
      bt_row = load_f32(bv, tid >> 3);
      lav = load_f32(f32_view(la + R.tok(T) + t0, nr), x.l);
      bev = load_f32(bv, x.l);
      r0 = load_f32(rv, 2 * x.l);
      r1 = load_f32(rv, 2 * x.l + 1);
    }
#pragma unroll
    for (int u = 0; u < NT; ++u) put_seg(Qs + u * TILE, sg[u], tid);
    DL_STAMP(8);
    {
      // dV = beta drhs, row segment tid (the chain kernel rounds drhs to bf16 once; dV rounds its product again);
      // rows past the end of a partial chunk fall outside the store's range and are dropped
      bf16x8 dvs;
#pragma unroll
      for (int e = 0; e < 8; ++e) dvs[e] = (__bf16)(bt_row * (float)sg[NT - 1][e]);
      const __amdgpu_buffer_rsrc_t dv_out = __builtin_amdgcn_make_buffer_rsrc(
          dv + voff, (short)0, nr * DKEY * (int)sizeof(__bf16), 0x00020000);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, dvs), dv_out,
                                             ((tid >> 3) * DKEY + 8 * (tid & 7)) * (int)sizeof(__bf16), 0, 0);
    }
    if (w == 0) {
      chunk_decays(lav, x.l, Ls, eLs, ws);
      bs[x.l] = bev;
    }
  }
  __syncthreads();
  DL_STAMP(16);
  auto dpart = [&](auto wl_c) {
    constexpr int WL = decltype(wl_c)::value;
    const int me = 16 * WL + i;
      // ---------------- token block WL in the query role: lane t = me
      const float Lt = Ls[me], bt = bs[me];
      bf16x8 qf[2 * KH], kf[2 * KH];
#pragma unroll
      for (int m = 0; m < 2 * KH; ++m) {
        qf[m] = frag(Qs + (m >> 1) * TILE, me, m & 1, g);
        kf[m] = frag(Ks + (m >> 1) * TILE, me, m & 1, g);
      }
      const bf16x8 of0 = frag(Os, me, 0, g), of1 = frag(Os, me, 1, g);
      const bf16x8 rf0 = frag(Rs, me, 0, g), rf1 = frag(Rs, me, 1, g);
      float rowacc = 0.f, db2 = 0.f;
      f32x4 dPT[4];
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        dPT[sb] = zero4();
        if (sb <= WL) {
          // rows s, lane t: P[t][s], dA[t][s], KK[t][s], dN[t][s]
          f32x4 P = zero4(), dA = zero4(), KK = zero4(), dN = zero4();
#pragma unroll
          for (int m = 0; m < 2 * KH; ++m) {
            const bf16x8 ks = frag(Ks + (m >> 1) * TILE, 16 * sb + i, m & 1, g);
            P = pgn_mfma(ks, qf[m], P);
            KK = pgn_mfma(ks, kf[m], KK);
          }
          dA = pgn_mfma(frag(Ws, 16 * sb + i, 0, g), of0, dA);
          dA = pgn_mfma(frag(Ws, 16 * sb + i, 1, g), of1, dA);
          dN = pgn_mfma(frag(Ws, 16 * sb + i, 0, g), rf0, dN);
          dN = pgn_mfma(frag(Ws, 16 * sb + i, 1, g), rf1, dN);
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = 16 * sb + 4 * g + r;
            const float dec = masked_decay(Lt - Lsv[r], s <= me);
            rowacc += dA[r] * P[r] * dec;
            dPT[sb][r] = dA[r] * dec;
            const float dnM = -dN[r] * KK[r] * dec * (s < me ? 1.f : 0.f);  // dN M, strictly lower
            db2 += dnM;
            rowacc += bt * dnM;
          }
        }
      }
      rowacc = sum_groups(rowacc);
      db2 = sum_groups(db2);
      const bf16x8 b0 = pack(dPT[0], dPT[1]), b1 = pack(dPT[2], dPT[3]);
      const float eLt = eLs[me];
      // rows past the end of a partial chunk fall outside the store's range and are dropped
      const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
          R.slot(dq, dq1) + roff, (short)0, nr * DKEY * (int)sizeof(__bf16), 0x00020000);
      float qzt = 0.f;
#pragma unroll
      for (int dt = 0; dt < 4 * KH; ++dt) {
        const int n0 = 16 * (dt & 3);
        const __bf16* Kh = Ks + (dt >> 2) * TILE;
        const __bf16* Sh = Ss + (dt >> 2) * TILE;
        f32x4 acc = zero4(), Z = zero4();
        acc = pgn_mfma(frag_tr(Kh, n0, 0, g, i), b0, acc);
        if (WL >= 2) acc = pgn_mfma(frag_tr(Kh, n0, 1, g, i), b1, acc);
        Z = pgn_mfma(frag_tr(Sh, n0, 0, g, i), of0, Z);
        Z = pgn_mfma(frag_tr(Sh, n0, 1, g, i), of1, Z);
        const f32x4 qq =
            to_f32x4(*reinterpret_cast<const bf16x4*>(Qs + (dt >> 2) * TILE + me * kPitch + n0 + 4 * g));
#pragma unroll
        for (int r = 0; r < 4; ++r) qzt += qq[r] * Z[r];
        acc = acc + Z * eLt;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), out,
                                              (me * DKEY + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
      }
      qzt = sum_groups(qzt);
      if (g == 0) {
        rowT[me] = rowacc + eLt * qzt;
        dbe2[me] = db2;
      }
  };
  auto kpart = [&](auto wl_c) {
    constexpr int WL = decltype(wl_c)::value;
    const int me = 16 * WL + i;
      // ---------------- token block WL in the key role: lane s = me
      const float Lsm = Ls[me], bsm = bs[me], wsm = ws[me], eLsm = eLs[me];
      bf16x8 kf[2 * KH];
#pragma unroll
      for (int m = 0; m < 2 * KH; ++m) kf[m] = frag(Ks + (m >> 1) * TILE, me, m & 1, g);
      const bf16x8 wf0 = frag(Ws, me, 0, g), wf1 = frag(Ws, me, 1, g);
      const bf16x8 rf0 = frag(Rs, me, 0, g), rf1 = frag(Rs, me, 1, g);
      float colacc = 0.f;
      f32x4 dPt[4], Gt[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        dPt[tb] = zero4();
        Gt[tb] = zero4();
        if (tb >= WL) {
          // rows t, lane s: P[t][s], dA[t][s], KK[t][s], dN[t][s]
          f32x4 P = zero4(), dA = zero4(), KK = zero4(), dN = zero4();
#pragma unroll
          for (int m = 0; m < 2 * KH; ++m) {
            P = pgn_mfma(frag(Qs + (m >> 1) * TILE, 16 * tb + i, m & 1, g), kf[m], P);
            KK = pgn_mfma(frag(Ks + (m >> 1) * TILE, 16 * tb + i, m & 1, g), kf[m], KK);
          }
          dA = pgn_mfma(frag(Os, 16 * tb + i, 0, g), wf0, dA);
          dA = pgn_mfma(frag(Os, 16 * tb + i, 1, g), wf1, dA);
          dN = pgn_mfma(frag(Rs, 16 * tb + i, 0, g), wf0, dN);
          dN = pgn_mfma(frag(Rs, 16 * tb + i, 1, g), wf1, dN);
          const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
          const f32x4 btv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * g + r;
            const float dec = masked_decay(Ltv[r] - Lsm, t >= me);
            colacc += dA[r] * P[r] * dec;
            dPt[tb][r] = dA[r] * dec;
            const float dkk = -btv[r] * dN[r] * dec * (t > me ? 1.f : 0.f);  // dKK[t][s], strictly lower
            colacc += dkk * KK[r];
            Gt[tb][r] = dkk;
          }
        }
        if (tb <= WL) {
          // rows t, lane s: dN[s][t] = -sum_j W[t][j] drhs[s][j], for t < s
          f32x4 dN = zero4();
          dN = pgn_mfma(frag(Ws, 16 * tb + i, 0, g), rf0, dN);
          dN = pgn_mfma(frag(Ws, 16 * tb + i, 1, g), rf1, dN);
          const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * g + r;
            Gt[tb][r] += -bsm * dN[r] * masked_decay(Lsm - Ltv[r], t < me);  // dKK[s][t]
          }
        }
      }
      colacc = sum_groups(colacc);
      const bf16x8 p0 = pack(dPt[0], dPt[1]), p1 = pack(dPt[2], dPt[3]);
      const bf16x8 g0 = pack(Gt[0], Gt[1]), g1 = pack(Gt[2], Gt[3]);
      const float us = -bsm * eLsm;  // dU[s] = us * drhs[s]
      const bf16x8 du0 = frag_scaled(Rs, me, 0, g, us), du1 = frag_scaled(Rs, me, 1, g, us);
      // rows past the end of a partial chunk fall outside the store's range and are dropped
      const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
          R.slot(dk, dk1) + roff, (short)0, nr * DKEY * (int)sizeof(__bf16), 0x00020000);
      float dw = 0.f;
#pragma unroll
      for (int dt = 0; dt < 4 * KH; ++dt) {
        const int n0 = 16 * (dt & 3);
        const __bf16* Qh = Qs + (dt >> 2) * TILE;
        const __bf16* Kh = Ks + (dt >> 2) * TILE;
        const __bf16* Sh = Ss + (dt >> 2) * TILE;
        const __bf16* dSh = dSs + (dt >> 2) * TILE;
        f32x4 acc = zero4(), Y = zero4();
        if (WL < 2) acc = pgn_mfma(frag_tr(Qh, n0, 0, g, i), p0, acc);
        acc = pgn_mfma(frag_tr(Qh, n0, 1, g, i), p1, acc);
        acc = pgn_mfma(frag_tr(Kh, n0, 0, g, i), g0, acc);
        acc = pgn_mfma(frag_tr(Kh, n0, 1, g, i), g1, acc);
        acc = pgn_mfma(frag_tr(Sh, n0, 0, g, i), du0, acc);
        acc = pgn_mfma(frag_tr(Sh, n0, 1, g, i), du1, acc);
        Y = pgn_mfma(frag_tr(dSh, n0, 0, g, i), wf0, Y);
        Y = pgn_mfma(frag_tr(dSh, n0, 1, g, i), wf1, Y);
        const f32x4 kk = to_f32x4(*reinterpret_cast<const bf16x4*>(Kh + me * kPitch + n0 + 4 * g));
#pragma unroll
        for (int r = 0; r < 4; ++r) dw += kk[r] * Y[r];
        acc = acc + Y * wsm;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), out,
                                              (me * DKEY + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
      }
      dw = sum_groups(dw);
      if (g == 0) {
        colS[me] = colacc;
        dwv[me] = dw;
      }
      // <S_c, dS> over key rows 16 WL .. of each 64-wide key tile
      float sd = 0.f;
#pragma unroll
      for (int hh = 0; hh < KH; ++hh)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          // S_c and dS at key rows 64 hh + 16 WL + 4g + r, column 16 jt + i: both staged transposed, so a plain read
          // of row 16 jt + i
          const int off = hh * TILE + (16 * jt + i) * kPitch + 16 * WL + 4 * g;
          const f32x4 sv = to_f32x4(*reinterpret_cast<const bf16x4*>(Ss + off));
          const f32x4 dv_ = to_f32x4(*reinterpret_cast<const bf16x4*>(dSs + off));
#pragma unroll
          for (int r = 0; r < 4; ++r) sd += sv[r] * dv_[r];
        }
      sd = wave_sum(sd);
      if (x.l == 0) sdot[WL] = sd;
  };
  // one instantiation per (role, block index): block conditions are compile-time constants
  switch (w) {
    case 0: dpart(std::integral_constant<int, 0>{}); break;
    case 1: dpart(std::integral_constant<int, 1>{}); break;
    case 2: dpart(std::integral_constant<int, 2>{}); break;
    case 3: dpart(std::integral_constant<int, 3>{}); break;
    case 4: kpart(std::integral_constant<int, 0>{}); break;
    case 5: kpart(std::integral_constant<int, 1>{}); break;
    case 6: kpart(std::integral_constant<int, 2>{}); break;
    default: kpart(std::integral_constant<int, 3>{}); break;
  }
  __syncthreads();
  if (w == 0) {
    const int t = x.l;
    const bool ok = t < nr;
    const float wdw = ws[t] * dwv[t];
    float dL = rowT[t] - colS[t] + eLs[t] * r1 - wdw;
    const float tot = wave_sum(wdw);
    const float a_c = __expf(Ls[C - 1]);
    if (t == C - 1) dL += tot + a_c * (sdot[0] + sdot[1] + sdot[2] + sdot[3]);
    dL = rev_scan64(dL, t);
    if (ok) {
      const size_t ti = R.tok(T) + t0 + t;
      R.slot(dla, dla1)[ti] = dL;
      R.slot(dbe, dbe1)[ti] = r0 + dbe2[t];
    }
  }
  DL_STAMP(24);
  if (w == 0) PGN_STAMP_CLOCKS_AUX(blockIdx.x * 40 + 34);
#undef DL_STAMP
}

// ------------------------------------------------------------------------------------------------------------------
// backward in one kernel (64-wide heads): the chain and the chunk-local work of a scan in one workgroup of 16 waves,
// chunks in reverse, so the per-chunk state gradient and drhs pass from the chain to the local work through LDS
// instead of memory, and the staged Q, K, S_c and dO serve both. Waves 0-3 carry dS and waves 4-7 serve them, as in
// aspin_delta_bwd_chain; waves 8-11 and 12-15 do aspin_delta_bwd_local's work for the same chunk, wave 8 + b owning
// token block b in the query role (dQ, row sums, dV) and wave 12 + b in the key role (dK, column sums). Three barriers
// per chunk:
//   B1  A^T complete. Before it: the chain's dS-side products, the service waves' scores, the query role's dA, dP and
//       whole dQ, the key role's dA and dP;
//   B2  drhs ready: the chain's dW and drhs (into LDS) and its row sums; meanwhile the service waves stage the next
//       chunk (Q, K, S_c, V, X, W double-buffered; dO read before B1 only) and the query role forms K K^T;
//   end the chain's dS update (into LDS as the next chunk's dS), the query role's dN terms and dV = beta drhs, the
//       key role's whole dK (its registers would not hold partial sums across the barriers) and its column sums.
// The chunk's dla and dbeta are finished by wave 8 at the start of the next iteration (the last chunk's after the
// loop) from the local waves' per-token sums and the chain's row sums. 16 waves hold at most 128 VGPRs each. LDS: dO,
// A^T, drhs single; Q, S_c, K, V, X, W, dS double-buffered; the chain's and the local waves' per-token vectors, two
// sets each: 156 KB.
constexpr int kFusedTiles = 17;
constexpr int kFusedLVec = 4 * C + 4;  // rowT, dbe2, colS, dwv per token; sdot per token block
constexpr size_t fused_smem() {
  return kFusedTiles * TILE * sizeof(__bf16) + (2 * kChainVec + 2 * kFusedLVec) * sizeof(float);
}

__global__ __launch_bounds__(1024) void aspin_delta_bwd_fused(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ be, const __bf16* __restrict__ X,
    const __bf16* __restrict__ sent, const __bf16* __restrict__ Win, const __bf16* __restrict__ dO,
    const float* __restrict__ dSfin, __bf16* __restrict__ dq, __bf16* __restrict__ dk, __bf16* __restrict__ dv,
    float* __restrict__ dla, float* __restrict__ dbe, float* __restrict__ dS0, int T, int NC) {
  constexpr int DKEY = 64;
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* Os = reinterpret_cast<__bf16*>(smem);  // dO of the current chunk (read before B1 only)
  __bf16* AT = Os + TILE;                          // AT[t][s] = A[s][t]
  __bf16* Rs = AT + TILE;                          // drhs (t, j) of the current chunk
  __bf16* Qb = Rs + TILE;                          // chunk c in set c & 1:
  __bf16* Sb = Qb + 2 * TILE;                      //   S_c transposed (j, d)
  __bf16* Kb = Sb + 2 * TILE;
  __bf16* Vb = Kb + 2 * TILE;
  __bf16* Xb = Vb + 2 * TILE;
  __bf16* Wb = Xb + 2 * TILE;
  __bf16* dSb = Wb + 2 * TILE;                     //   the gradient on the state leaving chunk c, transposed (j, d)
  float* vec = reinterpret_cast<float*>(dSb + 2 * TILE);  // chain vector sets: L, eL, w, beta; row sums
  float* lvec = vec + 2 * kChainVec;                       // local vector sets: rowT, dbe2, colS, dwv, sdot

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  const DeltaRows<1> R(blockIdx.x);
  // instrumented build, as aspin_delta_bwd_chain's (waves 0-7): per wave, clocks where its role's branch starts
  // (entries 0, 1) and at the kernel's end (2, 3), then the start and end of its phase for chunk cc (4 + 2 cc, 5 + 2 cc)
#define DB_STAMP(k) PGN_STAMP((blockIdx.x * 8 + w) * (4 + 2 * NC) + (k))
#define DB_CLOCKS(k) PGN_STAMP_CLOCKS((blockIdx.x * 8 + w) * (4 + 2 * NC) + (k))

  if (w < 4) {
    // ================= chain waves: value columns j = 16w + i; dS rows 16 db + 4g + r
    DB_CLOCKS(0);
    const int j = 16 * w + i;
    f32x4 dS[4];
    {
      const __amdgpu_buffer_rsrc_t dv_ = f32_view(dSfin ? dSfin + R.state() : nullptr, DKEY * DKEY);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS[db][r] = load_f32(dv_, (16 * db + 4 * g + r) * DKEY + j);
    }
    {
      // the last chunk's dS for the local waves
      __bf16* dst = dSb + ((NC - 1) & 1) * TILE + j * kPitch + 4 * g;
#pragma unroll
      for (int db = 0; db < 4; ++db) *reinterpret_cast<bf16x4*>(dst + 16 * db) = to_bf16x4(dS[db]);
    }
    __syncthreads();
    for (int cc = NC - 1; cc >= 0; --cc) {
      DB_STAMP(4 + 2 * cc);  // the chunk's phase: operand reads, contractions, result stores (across B1 and B2)
      const int h = cc & 1;
      const __bf16* Qs = Qb + h * TILE;
      const __bf16* Ss = Sb + h * TILE;
      const __bf16* Ks = Kb + h * TILE;
      const __bf16* Vs = Vb + h * TILE;
      const __bf16* Xs = Xb + h * TILE;
      float* vs = vec + h * kChainVec;
      const float* Ls = vs;
      const float* eLs = vs + C;
      const float* ws = vs + 2 * C;
      const float* bs = vs + 3 * C;
      float* redV = vs + 4 * C;
      float* redU = vs + 8 * C;
      // products that do not need A^T: y = K dS, U = K S_c, Yc = (Q o eL)^T dO, on this wave's columns
      bf16x8 dp[2], scf[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        dp[m] = pack(dS[2 * m], dS[2 * m + 1]);
        scf[m] = frag(Ss, 16 * w + i, m, g);  // S_c[d][j], staged (j, d)
      }
      const bf16x8 oc0 = frag_tr(Os, 16 * w, 0, g, i), oc1 = frag_tr(Os, 16 * w, 1, g, i);  // dO[t][j]
      f32x4 y[4], U[4], Yc[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        y[tb] = zero4();
        U[tb] = zero4();
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const bf16x8 kk = frag(Ks, 16 * tb + i, m, g);
          y[tb] = pgn_mfma(kk, dp[m], y[tb]);
          U[tb] = pgn_mfma(kk, scf[m], U[tb]);
        }
      }
      const bf16x8 oe0 = scale_frag_k(oc0, *reinterpret_cast<const f32x4*>(eLs + 4 * g),
                                      *reinterpret_cast<const f32x4*>(eLs + 16 + 4 * g));
      const bf16x8 oe1 = scale_frag_k(oc1, *reinterpret_cast<const f32x4*>(eLs + 32 + 4 * g),
                                      *reinterpret_cast<const f32x4*>(eLs + 48 + 4 * g));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        Yc[db] = pgn_mfma(frag_tr(Qs, 16 * db, 0, g, i), oe0, zero4());
        Yc[db] = pgn_mfma(frag_tr(Qs, 16 * db, 1, g, i), oe1, Yc[db]);
      }
      __syncthreads();  // B1: A^T complete

      // dW = A^T dO + w o (K dS); drhs = X^T dW into LDS; dU = -beta eL drhs; per-row partial sums
      f32x4 dW[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = zero4();
        if (tb < 2) acc = pgn_mfma(frag(AT, 16 * tb + i, 0, g), oc0, acc);
        acc = pgn_mfma(frag(AT, 16 * tb + i, 1, g), oc1, acc);
        const f32x4 wv = *reinterpret_cast<const f32x4*>(ws + 16 * tb + 4 * g);
        dW[tb] = acc + wv * y[tb];
      }
      const bf16x8 w01 = pack(dW[0], dW[1]), w23 = pack(dW[2], dW[3]);
      f32x4 dU[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = zero4();
        if (tb < 2) acc = pgn_mfma(frag_tr(Xs, 16 * tb, 0, g, i), w01, acc);
        acc = pgn_mfma(frag_tr(Xs, 16 * tb, 1, g, i), w23, acc);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
        const f32x4 ev = *reinterpret_cast<const f32x4*>(eLs + 16 * tb + 4 * g);
        const f32x4 vv = to_f32x4(ds_read_tr(Vs + (16 * tb + 4 * g + (i >> 2)) * kPitch + 16 * w + 4 * (i & 3)));
        float pr[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tl = 16 * tb + 4 * g + r;
          dU[tb][r] = -bv[r] * ev[r] * acc[r];
          pr[r] = acc[r] * vv[r];
          pr[4 + r] = acc[r] * U[tb][r];
          Rs[tl * kPitch + j] = (__bf16)acc[r];
        }
        const float tot = row_totals16x8(pr, i);
        ((i & 8) ? redU : redV)[w * C + 16 * tb + 4 * g + ((i >> 1) & 3)] = tot;
      }
      __syncthreads();  // B2: drhs and the row sums ready

      // dS_prev = a dS + (Q o eL)^T dO + K^T dU, kept in registers and written to LDS as the next chunk's dS
      const float a_c = __expf(Ls[C - 1]);
      const bf16x8 u01 = pack(dU[0], dU[1]), u23 = pack(dU[2], dU[3]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        f32x4 acc = dS[db] * a_c + Yc[db];
        acc = pgn_mfma(frag_tr(Ks, 16 * db, 0, g, i), u01, acc);
        acc = pgn_mfma(frag_tr(Ks, 16 * db, 1, g, i), u23, acc);
        dS[db] = acc;
      }
      {
        __bf16* dst = dSb + (h ^ 1) * TILE + j * kPitch + 4 * g;
#pragma unroll
        for (int db = 0; db < 4; ++db) *reinterpret_cast<bf16x4*>(dst + 16 * db) = to_bf16x4(dS[db]);
      }
      DB_STAMP(5 + 2 * cc);
      __syncthreads();  // end of the chunk
    }
    if (dS0) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS0[R.state() + (size_t)(16 * db + 4 * g + r) * DKEY + j] = dS[db][r];
    }
  } else if (w < 8) {
    // ================= service waves: thread b carries 16-byte row segments b and b + 256 of each staged tile:
    // dO (single), then Q, S_c, K, V, X, W (into the chunk's set)
    DB_CLOCKS(0);
    const int a = w - 4;
    const int b = tid & 255;
    constexpr int NT = 7;
    bf16x8 sg[NT][2];
    float pla = 0.f, pbe = 0.f;
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const __bf16* src;
        int rows = nr;
        if (u == 0) src = dO + R.vals(T) + (size_t)n0 * DKEY;
        else if (u == 1) src = q + R.rows(T) + (size_t)n0 * DKEY;
        else if (u == 2) { src = sent + R.stateT(NC, cn); rows = DK; }
        else if (u == 3) src = k + R.rows(T) + (size_t)n0 * DKEY;
        else if (u == 4) src = v + R.vals(T) + (size_t)n0 * DKEY;
        else if (u == 5) { src = X + ((size_t)R.hw * NC + cn) * C * C; rows = C; }
        else src = Win + R.vals(T) + (size_t)n0 * DKEY;
        sg[u][0] = load_seg(src, rows, b);
        sg[u][1] = load_seg(src, rows, b + 256);
      }
      pla = load_f32_lane(la + R.tok(T) + n0, nr, x.l);
      pbe = load_f32_lane(be + R.tok(T) + n0, nr, x.l);
    };
    auto stage = [&](int hh) {
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        __bf16* dst = u == 0 ? Os : (u == 1 ? Qb : u == 2 ? Sb : u == 3 ? Kb : u == 4 ? Vb : u == 5 ? Xb : Wb) +
                                        hh * TILE;
        put_seg(dst, sg[u][0], b);
        put_seg(dst, sg[u][1], b + 256);
      }
      if (a == 0) {
        float* vs = vec + hh * kChainVec;
        chunk_decays(pla, x.l, vs, vs + C, vs + 2 * C);
        vs[3 * C + x.l] = pbe;
      }
    };
    load(NC - 1);
    stage((NC - 1) & 1);
    load(max(NC - 2, 0));
    __syncthreads();
    for (int cc = NC - 1; cc >= 0; --cc) {
      const int h = cc & 1;
      const __bf16* Qs = Qb + h * TILE;
      const __bf16* Ks = Kb + h * TILE;
      const float* Ls = vec + h * kChainVec;
      // scores, transposed: AT[t][s] = (q_s . k_t) exp(L_s - L_t), s >= t, zero below (split 2, 3, 3, 2)
      DB_STAMP(4 + 2 * cc);
      {
        auto score = [&](int ta, int sb, const bf16x8* kf, float Lt) {
          f32x4 sc = zero4();
#pragma unroll
          for (int m = 0; m < 2; ++m) sc = pgn_mfma(frag(Qs, 16 * sb + i, m, g), kf[m], sc);
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] *= masked_decay(Lsv[r] - Lt, 16 * sb + 4 * g + r >= 16 * ta + i);
          store_T(AT, 16 * ta, 16 * sb, g, i, sc);
        };
        const int t = 16 * a + i;
        bf16x8 kf[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) kf[m] = frag(Ks, t, m, g);
        const float Lt = Ls[t];
        const int last = a == 0 ? 1 : 3;
        for (int sb = 0; sb < 4; ++sb) {
          if (sb < a) store_T(AT, 16 * a, 16 * sb, g, i, zero4());
          else if (sb <= last) score(a, sb, kf, Lt);
        }
        if (a >= 2) {
          bf16x8 kf0[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) kf0[m] = frag(Ks, i, m, g);
          score(0, a, kf0, Ls[i]);
        }
      }
      DB_STAMP(5 + 2 * cc);
      __syncthreads();  // B1
      // the next chunk's tiles (loaded a chunk ago: dO is free after B1, the other sets since the end of the
      // previous chunk), then the loads of the one after (unconditional: the last ones re-read the first chunk)
      if (cc > 0) stage(h ^ 1);
      load(max(cc - 2, 0));
      __syncthreads();  // B2
      __syncthreads();  // end of the chunk
    }
  } else {
    // ================= local waves
    // the finished chunk's dla and dbeta (wave 8), from its vector sets
    auto finish = [&](int cn) {
      const int hh = cn & 1, t = x.l, t0 = cn * C, nr = min(C, T - t0);
      const float* vs = vec + hh * kChainVec;
      const float* lv = lvec + hh * kFusedLVec;
      const float* redV = vs + 4 * C;
      const float* redU = vs + 8 * C;
      const float pv = redV[t] + redV[C + t] + redV[2 * C + t] + redV[3 * C + t];
      const float pu = redU[t] + redU[C + t] + redU[2 * C + t] + redU[3 * C + t];
      const float r0 = pv - vs[C + t] * pu, r1 = -vs[3 * C + t] * pu;
      const float wdw = vs[2 * C + t] * lv[3 * C + t];
      float dL = lv[t] - lv[2 * C + t] + vs[C + t] * r1 - wdw;
      const float tot = wave_sum(wdw);
      const float a_c = __expf(vs[C - 1]);
      if (t == C - 1) dL += tot + a_c * (lv[4 * C] + lv[4 * C + 1] + lv[4 * C + 2] + lv[4 * C + 3]);
      dL = rev_scan64(dL, t);
      if (t < nr) {
        const size_t ti = R.tok(T) + t0 + t;
        dla[ti] = dL;
        dbe[ti] = r0 + lv[C + t];
      }
    };
    // ---------------- query role, token block WL (lane t = me): dQ whole before B1; the row sums; dV
    auto qrole = [&](auto wl_c) {
      constexpr int WL = decltype(wl_c)::value;
      const int me = 16 * WL + i;
      const int lt = tid - 512;  // 0 .. 255
      __syncthreads();
      for (int cc = NC - 1; cc >= 0; --cc) {
        const int h = cc & 1, t0 = cc * C, nr = min(C, T - t0);
        if (WL == 0 && cc < NC - 1) finish(cc + 1);
        const __bf16* Qs = Qb + h * TILE;
        const __bf16* Ss = Sb + h * TILE;
        const __bf16* Ks = Kb + h * TILE;
        const __bf16* Ws = Wb + h * TILE;
        const float* vs = vec + h * kChainVec;
        const float* Ls = vs;
        const float* eLs = vs + C;
        const float* bs = vs + 3 * C;
        float* lv = lvec + h * kFusedLVec;
        const int out_bytes = nr * DKEY * (int)sizeof(__bf16);
        const float Lt = Ls[me], bt = bs[me], eLt = eLs[me];
        bf16x8 qf[2], kf[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          qf[m] = frag(Qs, me, m, g);
          kf[m] = frag(Ks, me, m, g);
        }
        const bf16x8 of0 = frag(Os, me, 0, g), of1 = frag(Os, me, 1, g);
        // rows s, lane t: P[t][s], dA[t][s] for s <= t
        float rowacc = 0.f;
        f32x4 dPT[4];
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
          dPT[sb] = zero4();
          if (sb <= WL) {
            f32x4 P = zero4(), dA = zero4();
#pragma unroll
            for (int m = 0; m < 2; ++m) P = pgn_mfma(frag(Ks, 16 * sb + i, m, g), qf[m], P);
            dA = pgn_mfma(frag(Ws, 16 * sb + i, 0, g), of0, dA);
            dA = pgn_mfma(frag(Ws, 16 * sb + i, 1, g), of1, dA);
            const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float dec = masked_decay(Lt - Lsv[r], 16 * sb + 4 * g + r <= me);
              rowacc += dA[r] * P[r] * dec;
              dPT[sb][r] = dA[r] * dec;
            }
          }
        }
        float qzt = 0.f;
        {
          // dQ = dP K + eL o (dO S^T), whole; rows past the chunk's end dropped
          const bf16x8 b0 = pack(dPT[0], dPT[1]), b1 = pack(dPT[2], dPT[3]);
          const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
              dq + R.rows(T) + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const int n0 = 16 * dt;
            f32x4 acc = zero4(), Z = zero4();
            acc = pgn_mfma(frag_tr(Ks, n0, 0, g, i), b0, acc);
            if (WL >= 2) acc = pgn_mfma(frag_tr(Ks, n0, 1, g, i), b1, acc);
            Z = pgn_mfma(frag_tr(Ss, n0, 0, g, i), of0, Z);
            Z = pgn_mfma(frag_tr(Ss, n0, 1, g, i), of1, Z);
            const f32x4 qq = to_f32x4(*reinterpret_cast<const bf16x4*>(Qs + me * kPitch + n0 + 4 * g));
#pragma unroll
            for (int r = 0; r < 4; ++r) qzt += qq[r] * Z[r];
            acc = acc + Z * eLt;
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), out,
                                                  (me * DKEY + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
          }
        }
        __syncthreads();  // B1
        // K K^T blocks s <= t against this lane's token, while the chain forms drhs
        f32x4 KK[WL + 1];
#pragma unroll
        for (int sb = 0; sb <= WL; ++sb) {
          KK[sb] = zero4();
#pragma unroll
          for (int m = 0; m < 2; ++m) KK[sb] = pgn_mfma(frag(Ks, 16 * sb + i, m, g), kf[m], KK[sb]);
        }
        __syncthreads();  // B2
        // dN[t][s] = -sum_j drhs[t][j] W[s][j], s < t; rows s, lane t
        const bf16x8 rf0 = frag(Rs, me, 0, g), rf1 = frag(Rs, me, 1, g);
        float db2 = 0.f;
#pragma unroll
        for (int sb = 0; sb <= WL; ++sb) {
          f32x4 dN = zero4();
          dN = pgn_mfma(frag(Ws, 16 * sb + i, 0, g), rf0, dN);
          dN = pgn_mfma(frag(Ws, 16 * sb + i, 1, g), rf1, dN);
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s_ = 16 * sb + 4 * g + r;
            const float dec = masked_decay(Lt - Lsv[r], s_ <= me);
            const float dnM = -dN[r] * KK[sb][r] * dec * (s_ < me ? 1.f : 0.f);  // dN M, strictly lower
            db2 += dnM;
            rowacc += bt * dnM;
          }
        }
        rowacc = sum_groups(rowacc);
        db2 = sum_groups(db2);
        qzt = sum_groups(qzt);
        if (g == 0) {
          lv[me] = rowacc + eLt * qzt;  // rowsum(dA o A) + rowsum(dKK o KK) + eL q.(S dO)
          lv[C + me] = db2;             // sum_{s<t} dN M
        }
        {
          // dV = beta drhs, 16-byte row segments lt and lt + 256 of the LDS drhs (rows past the chunk's end dropped)
          const __amdgpu_buffer_rsrc_t dv_out = __builtin_amdgcn_make_buffer_rsrc(
              dv + R.vals(T) + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {
            const int e = lt + 256 * e2, row = e >> 3, c8 = 8 * (e & 7);
            const bf16x4 lo = *reinterpret_cast<const bf16x4*>(Rs + row * kPitch + c8);
            const bf16x4 hi = *reinterpret_cast<const bf16x4*>(Rs + row * kPitch + c8 + 4);
            const float bb = bs[row];
            bf16x8 o8;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              o8[u] = (__bf16)(bb * (float)lo[u]);
              o8[4 + u] = (__bf16)(bb * (float)hi[u]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o8), dv_out,
                                                   (row * DKEY + c8) * (int)sizeof(__bf16), 0, 0);
          }
        }
        __syncthreads();  // end of the chunk
      }
      if (WL == 0) finish(0);
    };
    // ---------------- key role, token block WL (lane s = me): dA and dP before B1, the whole dK after B2
    auto krole = [&](auto wl_c) {
      constexpr int WL = decltype(wl_c)::value;
      const int me = 16 * WL + i;
      __syncthreads();
      for (int cc = NC - 1; cc >= 0; --cc) {
        const int h = cc & 1, t0 = cc * C, nr = min(C, T - t0);
        const __bf16* Qs = Qb + h * TILE;
        const __bf16* Ss = Sb + h * TILE;
        const __bf16* Ks = Kb + h * TILE;
        const __bf16* Ws = Wb + h * TILE;
        const __bf16* dSs = dSb + h * TILE;
        const float* vs = vec + h * kChainVec;
        const float* Ls = vs;
        const float* eLs = vs + C;
        const float* ws = vs + 2 * C;
        const float* bs = vs + 3 * C;
        float* lv = lvec + h * kFusedLVec;
        const int out_bytes = nr * DKEY * (int)sizeof(__bf16);
        const float Lsm = Ls[me];
        // rows t, lane s: P[t][s], dA[t][s] for t >= s
        float colacc = 0.f;
        bf16x8 p0, p1;
        {
          bf16x8 kf[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) kf[m] = frag(Ks, me, m, g);
          const bf16x8 wf0 = frag(Ws, me, 0, g), wf1 = frag(Ws, me, 1, g);
          f32x4 dPt[4];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            dPt[tb] = zero4();
            if (tb >= WL) {
              f32x4 P = zero4(), dA = zero4();
#pragma unroll
              for (int m = 0; m < 2; ++m) P = pgn_mfma(frag(Qs, 16 * tb + i, m, g), kf[m], P);
              dA = pgn_mfma(frag(Os, 16 * tb + i, 0, g), wf0, dA);
              dA = pgn_mfma(frag(Os, 16 * tb + i, 1, g), wf1, dA);
              const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float dec = masked_decay(Ltv[r] - Lsm, 16 * tb + 4 * g + r >= me);
                colacc += dA[r] * P[r] * dec;
                dPt[tb][r] = dA[r] * dec;
              }
            }
          }
          p0 = pack(dPt[0], dPt[1]);
          p1 = pack(dPt[2], dPt[3]);
        }
        __syncthreads();  // B1
        // K K^T blocks t >= s against this lane's token, while the chain forms drhs
        f32x4 KK[4];
        {
          bf16x8 kf[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) kf[m] = frag(Ks, me, m, g);
#pragma unroll
          for (int tb = WL; tb < 4; ++tb) {
            KK[tb] = zero4();
#pragma unroll
            for (int m = 0; m < 2; ++m) KK[tb] = pgn_mfma(frag(Ks, 16 * tb + i, m, g), kf[m], KK[tb]);
          }
        }
        __syncthreads();  // B2
        const float bsm = bs[me], wsm = ws[me], eLsm = eLs[me];
        const bf16x8 wf0 = frag(Ws, me, 0, g), wf1 = frag(Ws, me, 1, g);
        const bf16x8 rf0 = frag(Rs, me, 0, g), rf1 = frag(Rs, me, 1, g);
        f32x4 Gt[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          Gt[tb] = zero4();
          if (tb >= WL) {
            // rows t, lane s: dN[t][s] = -sum_j drhs[t][j] W[s][j]
            f32x4 dN = zero4();
            dN = pgn_mfma(frag(Rs, 16 * tb + i, 0, g), wf0, dN);
            dN = pgn_mfma(frag(Rs, 16 * tb + i, 1, g), wf1, dN);
            const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
            const f32x4 btv = *reinterpret_cast<const f32x4*>(bs + 16 * tb + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = 16 * tb + 4 * g + r;
              const float dec = masked_decay(Ltv[r] - Lsm, t >= me);
              const float dkk = -btv[r] * dN[r] * dec * (t > me ? 1.f : 0.f);  // dKK[t][s], strictly lower
              colacc += dkk * KK[tb][r];
              Gt[tb][r] = dkk;
            }
          }
          if (tb <= WL) {
            // rows t, lane s: dN[s][t] = -sum_j W[t][j] drhs[s][j], for t < s
            f32x4 dN = zero4();
            dN = pgn_mfma(frag(Ws, 16 * tb + i, 0, g), rf0, dN);
            dN = pgn_mfma(frag(Ws, 16 * tb + i, 1, g), rf1, dN);
            const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = 16 * tb + 4 * g + r;
              Gt[tb][r] += -bsm * dN[r] * masked_decay(Lsm - Ltv[r], t < me);  // dKK[s][t]
            }
          }
        }
        colacc = sum_groups(colacc);
        const bf16x8 g0 = pack(Gt[0], Gt[1]), g1 = pack(Gt[2], Gt[3]);
        const float us = -bsm * eLsm;  // dU[s] = us * drhs[s]
        const bf16x8 du0 = frag_scaled(Rs, me, 0, g, us), du1 = frag_scaled(Rs, me, 1, g, us);
        const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
            dk + R.rows(T) + (size_t)t0 * DKEY, (short)0, out_bytes, 0x00020000);
        float dw = 0.f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          // dK = dP^T Q + G K + dU S^T + w o (W dS^T), whole; rows past the chunk's end dropped
          const int n0 = 16 * dt;
          f32x4 acc = zero4(), Y = zero4();
          if (WL < 2) acc = pgn_mfma(frag_tr(Qs, n0, 0, g, i), p0, acc);
          acc = pgn_mfma(frag_tr(Qs, n0, 1, g, i), p1, acc);
          acc = pgn_mfma(frag_tr(Ks, n0, 0, g, i), g0, acc);
          acc = pgn_mfma(frag_tr(Ks, n0, 1, g, i), g1, acc);
          acc = pgn_mfma(frag_tr(Ss, n0, 0, g, i), du0, acc);
          acc = pgn_mfma(frag_tr(Ss, n0, 1, g, i), du1, acc);
          Y = pgn_mfma(frag_tr(dSs, n0, 0, g, i), wf0, Y);
          Y = pgn_mfma(frag_tr(dSs, n0, 1, g, i), wf1, Y);
          const f32x4 kk = to_f32x4(*reinterpret_cast<const bf16x4*>(Ks + me * kPitch + n0 + 4 * g));
#pragma unroll
          for (int r = 0; r < 4; ++r) dw += kk[r] * Y[r];
          acc = acc + Y * wsm;
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), out,
                                                (me * DKEY + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
        }
        dw = sum_groups(dw);
        if (g == 0) {
          lv[2 * C + me] = colacc;  // colsum(dA o A) + colsum(dKK o KK)
          lv[3 * C + me] = dw;      // k_s . (dS W_s)
        }
        {
          // <S_c, dS> over key rows 16 WL .. (both staged transposed: a plain read of row 16 jt + i)
          float sd = 0.f;
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {
            const int off = (16 * jt + i) * kPitch + 16 * WL + 4 * g;
            const f32x4 sv = to_f32x4(*reinterpret_cast<const bf16x4*>(Ss + off));
            const f32x4 dv_ = to_f32x4(*reinterpret_cast<const bf16x4*>(dSs + off));
#pragma unroll
            for (int r = 0; r < 4; ++r) sd += sv[r] * dv_[r];
          }
          sd = wave_sum(sd);
          if (x.l == 0) lv[4 * C + WL] = sd;
        }
        __syncthreads();  // end of the chunk
      }
    };
    switch (w) {
      case 8: qrole(std::integral_constant<int, 0>{}); break;
      case 9: qrole(std::integral_constant<int, 1>{}); break;
      case 10: qrole(std::integral_constant<int, 2>{}); break;
      case 11: qrole(std::integral_constant<int, 3>{}); break;
      case 12: krole(std::integral_constant<int, 0>{}); break;
      case 13: krole(std::integral_constant<int, 1>{}); break;
      case 14: krole(std::integral_constant<int, 2>{}); break;
      default: krole(std::integral_constant<int, 3>{}); break;
    }
  }
  if (w < 8) DB_CLOCKS(2);
#undef DB_STAMP
#undef DB_CLOCKS
}

// The slot sums of the 128-wide backward: x[p][i] <- x[p][i] + y[p][i] for the bf16 pairs (dq, dk; the fp32 sum of
// two bf16 values rounded once, as a bf16 tensor add rounds) over n elements (n % 8 == 0), and f[p][i] <- f[p][i] +
// e[p][i] for the fp32 pairs (dla, dbeta) over m elements (m <= n / 8). Thread u covers elements 8u .. 8u + 7 of
// each bf16 pair and element u of each fp32 pair.
struct DeltaJoin {
  __bf16* x[2];
  const __bf16* y[2];
  float* f[2];
  const float* e[2];
  int64_t n, m;
};

__global__ __launch_bounds__(256) void aspin_delta_join(DeltaJoin a) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (8 * u < a.n) {
    bf16x8 xs[2], ys[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      xs[p] = *reinterpret_cast<const bf16x8*>(a.x[p] + 8 * u);
      ys[p] = *reinterpret_cast<const bf16x8*>(a.y[p] + 8 * u);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xs[p][j] = pgn_bf16(pgn_f32(xs[p][j]) + pgn_f32(ys[p][j]));
      *reinterpret_cast<bf16x8*>(a.x[p] + 8 * u) = xs[p];
    }
  }
  if (u < a.m) {
#pragma unroll
    for (int p = 0; p < 2; ++p) a.f[p][u] += a.e[p][u];
  }
}

template <int KH>
constexpr size_t fwd_smem() {
  return (2 * fwd_stage<KH>() + TILE) * sizeof(__bf16) + 2 * kFwdVec * sizeof(float);
}
template <int KH>
constexpr size_t chain_smem() {
  return (chain_single<KH>() + 2 * chain_double<KH>() + TILE) * sizeof(__bf16) + 2 * kChainVec * sizeof(float);
}
template <int KH>
constexpr size_t local_smem() {
  return local_tiles<KH>() * TILE * sizeof(__bf16) + (9 * C + 4) * sizeof(float);
}

// Head dim D = 64 or 128 (KH = D / 64 key tiles; a 128-wide head runs as two scans).
bool shape_ok(int64_t B, int64_t H, int64_t T, int64_t D, int64_t Cc) {
  if (B <= 0 || H <= 0 || T <= 0) return false;
  if (B * H >= ((int64_t)1 << 23) || T >= ((int64_t)1 << 28)) return false;
  if (2 * B * H * ((T + C - 1) / C) >= ((int64_t)1 << 31)) return false;
  if (B * H * T * D >= ((int64_t)1 << 34)) return false;
  return (D == DK || D == 2 * DK) && Cc == C;
}

// ------------------------------------------------------------------------------------------------------------------
// Carried windows of the delta rule in one pass: the entering state of every window from the windows' affine maps.
// Given X (keys, decays and strengths only) the rule is independent per value column and linear in the state, so a
// window maps its entering state affinely, S_out = M S_in + R, with M (64 x 64) acting on the key rows, the same for
// every value column: R is the window's final state from a zero entering state, M its final state from the identity
// with zero values (both from the forward's state pass, all windows at once). Successive windows restart their
// positions, so the state is rebased between them by -shift theta (key-row pairs rotated, `src/assoc.py:399-402`):
//     S_in[0] = S0,   S_in[w + 1] = Rot(M[w] S_in[w] + R[w]).
// Four workgroups of 256 threads per (batch, head) walk the windows, fp32 throughout, each owning 16 value columns
// (the map acts on the key rows, so the columns' chains are independent). Wave wv forms key rows 16 wv .. 16 wv + 15
// of the 16 columns on fp32 MFMA (v_mfma_f32_16x16x4f32: A[r][k] in lane r + 16 k, B[k][c] in lane c + 16 k,
// D[4 g + e][c] in lane c + 16 g): lane (r, g) holds M[w]'s row 16 wv + r over keys 16 g .. 16 g + 15 in registers,
// the s-th of them the A operand of product s, whose B operand is S_in[w]'s key row 16 g + s from LDS, so 16 products
// over K = 4 cover the 64 keys, and R[w] is added to their sum. Each lane then rotates its two row pairs and writes
// S_in[w + 1] to memory and to the other LDS buffer: one barrier a window, and M never passes through LDS. Every M[w]
// and R[w] is known before the walk, so those of the window after next are loaded while this one is formed, into
// registers read only by the products (no copy of a register still in flight, so no wait on those loads).
// M, R, S_in: (BH, NW, 64, 64) fp32; S0: (BH, 64, 64) fp32 or NULL (zero).
constexpr int kPrefixParts = 4;

__global__ __launch_bounds__(256) void delta_window_prefix(const float* __restrict__ M, const float* __restrict__ R,
                                                           const float* __restrict__ S0,
                                                           const float* __restrict__ theta, float shift,
                                                           float* __restrict__ Sin, int H, int NW) {
  constexpr int P = 68;                       // LDS pitch of a column (floats)
  __shared__ __align__(16) float St[2][16 * P];  // S_in[w] by window parity, column-major: St[c][key]
  const int bh = blockIdx.x / kPrefixParts, part = blockIdx.x % kPrefixParts, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 15, g = lane >> 4;
  const int j = 16 * part + c;      // value column
  const int row0 = 16 * wv + 4 * g;  // output key rows row0 .. row0 + 3 (two rotation pairs)
  float sn[2], cs[2];
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) sincosf(-shift * theta[h * 32 + row0 / 2 + pr], &sn[pr], &cs[pr]);
  const size_t base = (size_t)bh * NW * 4096;
  f32x4 x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = S0 ? S0[(size_t)bh * 4096 + (row0 + e) * 64 + j] : 0.f;
    Sin[base + (row0 + e) * 64 + j] = x[e];
  }
  *reinterpret_cast<f32x4*>(&St[0][c * P + row0]) = x;
  if (NW < 2) return;
  f32x4 ma[4], mb[4], ra, rb;
  auto fetch = [&](f32x4 (&mreg)[4], f32x4& rreg, int w) {  // M[w] row 16 wv + c, keys 16 g ..; R[w] rows row0 ..
    const float* Mw = M + base + (size_t)w * 4096 + (16 * wv + c) * 64 + 16 * g;
    const float* Rw = R + base + (size_t)w * 4096 + row0 * 64 + j;
#pragma unroll
    for (int u = 0; u < 4; ++u) mreg[u] = *reinterpret_cast<const f32x4*>(Mw + 4 * u);
#pragma unroll
    for (int e = 0; e < 4; ++e) rreg[e] = Rw[e * 64];
  };
  auto step = [&](f32x4 (&mreg)[4], f32x4& rreg, int w) {
    __syncthreads();  // S_in[w] in buffer w & 1; every read of the other buffer (window w - 1) done
    const float* Sb = &St[w & 1][c * P + 16 * g];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f32x4 b = *reinterpret_cast<const f32x4*>(Sb + 4 * u);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(mreg[u][t], b[t], acc, 0, 0, 0);
    }
    acc += rreg;  // after the products: R is read once they are done, two windows after its load was issued
    // the set is refilled unconditionally (a spare load at the end) for the window after next
    fetch(mreg, rreg, min(w + 2, NW - 1));
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      const float a0 = acc[2 * pr], a1 = acc[2 * pr + 1];
      x[2 * pr] = a0 * cs[pr] - a1 * sn[pr];
      x[2 * pr + 1] = a0 * sn[pr] + a1 * cs[pr];
    }
    *reinterpret_cast<f32x4*>(&St[(w + 1) & 1][c * P + row0]) = x;
    float* dst = Sin + base + (size_t)(w + 1) * 4096 + row0 * 64 + j;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e * 64] = x[e];
  };
  fetch(ma, ra, 0);
  fetch(mb, rb, min(1, NW - 1));
  int w = 0;
  for (; w + 2 < NW; w += 2) {
    step(ma, ra, w);
    step(mb, rb, w + 1);
  }
  if (w + 1 < NW) step(ma, ra, w);
}

int set_smem(const void* fn, size_t bytes) { return (int)pgn_lds_limit(fn, bytes); }

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// The backward's workspace. At D = 64 the one-kernel backward keeps everything on chip: a token 256 bytes. At D = 128:
// drhs (B, H, T, D) bf16, the per-chunk state gradients (B, H, NC, D, D) bf16 and the per-scan row sums (B H D / 64
// scans, T, 2) fp32, then the second slots of dq and dk ((B, H, T, D) bf16) and of dla and dbeta ((B, H, T) fp32).
struct BwdWorkspace {
  int64_t drhs, dsc, rsum, dq1, dk1, dla1, dbe1, total;
  BwdWorkspace(int64_t B, int64_t H, int64_t T, int64_t D) {
    const int64_t NC = (T + C - 1) / C, KH = D / DK;
    if (KH == 1) {
      drhs = dsc = rsum = dq1 = dk1 = dla1 = dbe1 = -1;
      total = 256;
      return;
    }
    drhs = 0;
    dsc = align256(B * H * T * D * 2);
    rsum = dsc + align256(B * H * NC * D * D * 2);
    const int64_t rs = B * H * KH * T * 2 * 4;
    dq1 = rsum + align256(rs);
    dk1 = dq1 + align256(B * H * T * D * 2);
    dla1 = dk1 + align256(B * H * T * D * 2);
    dbe1 = dla1 + align256(B * H * T * 4);
    total = dbe1 + B * H * T * 4;
  }
};

template <int KH>
int delta_fwd(const void* q, const void* k, const void* v, const float* la, const float* beta, const float* S0,
              void* o, float* S_final, void* sent, void* W, void* X, int64_t B, int64_t H, int64_t T,
              hipStream_t st) {
  const int NC = (int)((T + C - 1) / C);
  const int heads = (int)(B * H);
  if constexpr (KH == 1) {  // one launch: the inverses formed on chip
    const int rc = set_smem((const void*)aspin_delta_fwd_inv, fwd_inv_smem());
    if (rc) return rc;
    hipLaunchKernelGGL(aspin_delta_fwd_inv, dim3((unsigned)heads), dim3(64 * (8 + kNIW)), fwd_inv_smem(), st, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, la, beta, S0, (__bf16*)o, (__bf16*)W, S_final,
                       (__bf16*)sent, (__bf16*)X, (int)T, NC, 0);
    PGN_RETURN_LAUNCH();
  }
  hipLaunchKernelGGL(aspin_delta_inv<KH>, dim3((unsigned)(heads * NC)), dim3(256), 0, st, (const __bf16*)k, la, beta,
                     (__bf16*)X, (int)T, NC);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int rc = set_smem((const void*)aspin_delta_fwd<KH>, fwd_smem<KH>());
  if (rc) return rc;
  hipLaunchKernelGGL(aspin_delta_fwd<KH>, dim3((unsigned)scan_grid<KH>(heads)), dim3(512), fwd_smem<KH>(), st,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, beta, (const __bf16*)X, S0,
                     (__bf16*)o, (__bf16*)W, S_final, (__bf16*)sent, (int)T, NC, (int)(heads * KH));
  PGN_RETURN_LAUNCH();
}

template <int KH>
int delta_bwd(const void* q, const void* k, const void* v, const float* la, const float* beta, const void* sent,
              const void* W, const void* X, const void* dO, const float* dS_final, void* dq, void* dk, void* dv,
              float* dla, float* dbeta, float* dS0, void* workspace, int64_t B, int64_t H, int64_t T,
              hipStream_t st) {
  if constexpr (KH == 1) {  // one kernel: the chain and the chunk-local work share the workgroup, nothing in memory
    const int rc = set_smem((const void*)aspin_delta_bwd_fused, fused_smem());
    if (rc) return rc;
    hipLaunchKernelGGL(aspin_delta_bwd_fused, dim3((unsigned)(B * H)), dim3(1024), fused_smem(), st,
                       (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, beta, (const __bf16*)X,
                       (const __bf16*)sent, (const __bf16*)W, (const __bf16*)dO, dS_final, (__bf16*)dq, (__bf16*)dk,
                       (__bf16*)dv, dla, dbeta, dS0, (int)T, (int)((T + C - 1) / C));
    (void)workspace;
    PGN_RETURN_LAUNCH();
  }
  int rc = set_smem((const void*)aspin_delta_bwd_chain<KH>, chain_smem<KH>());
  if (rc) return rc;
  rc = set_smem((const void*)aspin_delta_bwd_local<KH>, local_smem<KH>());
  if (rc) return rc;
  const int NC = (int)((T + C - 1) / C);
  const int scans = (int)(B * H * KH);
  const BwdWorkspace L(B, H, T, 64 * KH);
  unsigned char* ws = (unsigned char*)workspace;
  __bf16* drhs = (__bf16*)(ws + L.drhs);
  __bf16* dsc = (__bf16*)(ws + L.dsc);
  float* rs = (float*)(ws + L.rsum);
  __bf16* dq1 = KH == 2 ? (__bf16*)(ws + L.dq1) : nullptr;
  __bf16* dk1 = KH == 2 ? (__bf16*)(ws + L.dk1) : nullptr;
  float* dla1 = KH == 2 ? (float*)(ws + L.dla1) : nullptr;
  float* dbe1 = KH == 2 ? (float*)(ws + L.dbe1) : nullptr;
  hipLaunchKernelGGL(aspin_delta_bwd_chain<KH>, dim3((unsigned)scan_grid<KH>(B * H)), dim3(512), chain_smem<KH>(),
                     st, (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, beta, (const __bf16*)X,
                     (const __bf16*)sent, (const __bf16*)dO, dS_final, drhs, dsc, rs, dS0, (int)T, NC, scans);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(aspin_delta_bwd_local<KH>, dim3((unsigned)(scans * NC)), dim3(512), local_smem<KH>(), st,
                     (const __bf16*)q, (const __bf16*)k, la, beta, (const __bf16*)W, (const __bf16*)sent,
                     (const __bf16*)dO, drhs, dsc, rs, (__bf16*)dq, dq1, (__bf16*)dk, dk1, (__bf16*)dv, dla, dla1,
                     dbeta, dbe1, (int)T, NC);
  if (KH == 1) PGN_RETURN_LAUNCH();
  e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  DeltaJoin j = {};
  j.x[0] = (__bf16*)dq;
  j.y[0] = dq1;
  j.x[1] = (__bf16*)dk;
  j.y[1] = dk1;
  j.f[0] = dla;
  j.e[0] = dla1;
  j.f[1] = dbeta;
  j.e[1] = dbe1;
  j.n = B * H * T * 64 * KH;
  j.m = B * H * T;
  hipLaunchKernelGGL(aspin_delta_join, dim3((unsigned)((j.n / 8 + 255) / 256)), dim3(256), 0, st, j);
  PGN_RETURN_LAUNCH();
}

}  // namespace

extern "C" int64_t pragnosia_aspin_delta_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D,
                                                             int64_t chunk) {
  if (!shape_ok(B, H, T, D, chunk)) return -1;
  return BwdWorkspace(B, H, T, D).total;
}

extern "C" int pragnosia_aspin_delta_fwd(const void* q, const void* k, const void* v, const float* la,
                                         const float* beta, const float* S0, void* o, float* S_final, void* sent,
                                         void* W, void* X, int64_t B, int64_t H, int64_t T, int64_t D,
                                         int64_t chunk, void* stream) {
  if ((D != DK && D != 2 * DK) || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && beta && S_final);
  // at D = 128 every output is written (the backward reads W and X); at D = 64 each only when given
  PGN_CHECK_ARG(D == DK || (o && W && X));
  hipStream_t st = (hipStream_t)stream;
  return D == DK ? delta_fwd<1>(q, k, v, la, beta, S0, o, S_final, sent, W, X, B, H, T, st)
                 : delta_fwd<2>(q, k, v, la, beta, S0, o, S_final, sent, W, X, B, H, T, st);
}

extern "C" int pragnosia_aspin_delta_bwd(const void* q, const void* k, const void* v, const float* la,
                                         const float* beta, const void* sent, const void* W, const void* X,
                                         const void* dO, const float* dS_final, void* dq, void* dk, void* dv,
                                         float* dla, float* dbeta, float* dS0, void* workspace,
                                         int64_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                                         int64_t chunk, void* stream) {
  if ((D != DK && D != 2 * DK) || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && beta && sent && W && X && dO && dq && dk && dv && dla && dbeta && workspace);
  PGN_CHECK_ARG(workspace_bytes >= BwdWorkspace(B, H, T, D).total);
  hipStream_t st = (hipStream_t)stream;
  return D == DK ? delta_bwd<1>(q, k, v, la, beta, sent, W, X, dO, dS_final, dq, dk, dv, dla, dbeta, dS0, workspace,
                                B, H, T, st)
                 : delta_bwd<2>(q, k, v, la, beta, sent, W, X, dO, dS_final, dq, dk, dv, dla, dbeta, dS0, workspace,
                                B, H, T, st);
}

extern "C" int pragnosia_aspin_delta_window_maps(const void* q, const void* k, const void* v, const float* la,
                                                 const float* beta, float* RM, int64_t N, int64_t T, void* stream) {
  PGN_CHECK_ARG(shape_ok(2 * N, 1, T, DK, C));
  PGN_CHECK_ARG(q && k && v && la && beta && RM);
  hipStream_t st = (hipStream_t)stream;
  const int rc = set_smem((const void*)aspin_delta_fwd_inv, fwd_inv_smem());
  if (rc) return rc;
  hipLaunchKernelGGL(aspin_delta_fwd_inv, dim3((unsigned)(2 * N)), dim3(64 * (8 + kNIW)), fwd_inv_smem(), st,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, beta, nullptr, nullptr, nullptr, RM,
                     nullptr, nullptr, (int)T, (int)((T + C - 1) / C), (int)N);
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_aspin_delta_window_prefix(const float* M, const float* R, const float* S0, const float* theta,
                                                   float shift, float* S_in, int64_t BH, int64_t H, int64_t NW,
                                                   void* stream) {
  PGN_CHECK_ARG(M && R && theta && S_in && BH > 0 && H > 0 && NW > 0 && BH % H == 0);
  PGN_CHECK_ARG(BH * kPrefixParts < ((int64_t)1 << 31) && BH * NW < ((int64_t)1 << 40));
  PGN_CHECK_ARG(((uintptr_t)M | (uintptr_t)R) % 16 == 0);
  hipLaunchKernelGGL(delta_window_prefix, dim3((unsigned)(BH * kPrefixParts)), dim3(256), 0, (hipStream_t)stream, M,
                     R, S0, theta, shift, S_in, (int)H, (int)NW);
  PGN_RETURN_LAUNCH();
}
