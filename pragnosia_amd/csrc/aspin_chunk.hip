// The associative carrier's chunked scan, plain write rule: forward and hand-written backward on bf16 MFMA.
//
// Per (batch, head), with chunk C = 64 tokens, head dim D = 64, la_t <= 0 the per-token log-decay and, within a
// chunk, L the inclusive cumulative sum of la, dec[t,s] = exp(L_t - L_s) for s <= t (else 0), eL = exp(L),
// w = exp(L_C - L), a = exp(L_C):
//     O   = ((Q K^T) o dec) V + (Q o eL) S_c
//     S_{c+1} = a S_c + (K o w)^T V
// (the reference's `_scan_twopass`, `src/assoc.py:118-165`; its GPU form `src/assoc_kernel.py:47-70,188-202`).
//
// One workgroup (4 waves) owns one (batch, head) and walks its chunks in order with the fp32 state in registers:
// wave w holds rows 16w..16w+15 of S (keys) for all 64 value columns, as four accumulator tiles, and the state
// update is an MFMA accumulating straight onto a*S. Each chunk's Q, K, V tiles are staged in LDS once (K and V also
// transposed) and every contraction reads its operands from there, so HBM sees each input exactly once:
// 8 B per (t, d) element forward (q, k, v read, o written) plus the optional bf16 entering states.
//
// The backward walks the chunks in reverse with dS (the gradient on the state leaving the chunk) in registers and
// the entering states S_c read back from the forward's bf16 copies. Per chunk, with dA = dO V^T, dP = dA o dec,
// A = (Q K^T) o dec:
//     dQ = dP K + eL o (dO S_c^T)            dK = dP^T Q + w o (V dS^T)
//     dV = A^T dO + (K o w) dS               dS_c = a dS + (Q o eL)^T dO
//     dL_t = rowsum(dA o A)_t - colsum(dA o A)_t + eL_t q_t.(S_c dO_t) - w_t k_t.(dS v_t),
//     dL_{C-1} += sum_s w_s k_s.(dS v_s) + a <S_c, dS>,     dla = reverse cumulative sum of dL.
// (equations of `src/assoc_kernel.py:73-116`, `:205-220`, `:279-296`, merged into one pass). Every product that
// has a transposed operand is computed in the orientation whose accumulator is the next product's operand, so
// nothing round-trips through LDS except the two copies of dS.
#include "mfma_tile.h"

using namespace pgn;

namespace {

constexpr int C = 64;
constexpr int DK = 64;
constexpr int TILE = 64 * kPitch;  // one staged 64 x 64 tile

// L, exp(L), exp(L_C - L) of the chunk starting at t0, into LDS (one wave, lane = token).
PGN_DEVICE void chunk_decays(const float* __restrict__ la_bh, int t0, int T, int l, float* Ls, float* eLs,
                             float* ws) {
  float x = (t0 + l < T) ? la_bh[t0 + l] : 0.f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(x, off);
    if (l >= off) x += y;
  }
  const float LC = __shfl(x, 63);
  Ls[l] = x;
  eLs[l] = __expf(x);
  ws[l] = __expf(fminf(LC - x, 0.f));
}

__global__ __launch_bounds__(256) void aspin_plain_fwd(const __bf16* __restrict__ q, const __bf16* __restrict__ k,
                                                       const __bf16* __restrict__ v, const float* __restrict__ la,
                                                       const float* __restrict__ S0, __bf16* __restrict__ o,
                                                       float* __restrict__ Sfin, __bf16* __restrict__ sent, int T,
                                                       int NC) {
  __shared__ __align__(16) __bf16 Qs[TILE], Ks[TILE], KT[TILE], VT[TILE], ST[TILE];
  __shared__ __align__(16) float Ls[C], eLs[C], ws[C];

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i;
  const int bh = blockIdx.x;
  const size_t boff = (size_t)bh * T * DK;
  const size_t soff = (size_t)bh * DK * DK;

  // state rows 16w + 4g + r, column 16 jt + i
  f32x4 S[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) S[jt][r] = S0 ? S0[soff + (16 * w + 4 * g + r) * DK + 16 * jt + i] : 0.f;
    store_T(ST, 16 * jt, 16 * w, g, i, S[jt]);
  }

  const int tq = 16 * w + i;  // this lane's token within the chunk for t-indexed operands
  for (int c = 0; c < NC; ++c) {
    const int t0 = c * C;
    const int nrows = min(C, T - t0);
    stage64(q + boff + (size_t)t0 * DK, DK, nrows, Qs, nullptr);
    stage64(k + boff + (size_t)t0 * DK, DK, nrows, Ks, KT);
    stage64(v + boff + (size_t)t0 * DK, DK, nrows, nullptr, VT);
    if (w == 0) chunk_decays(la + (size_t)bh * T, t0, T, x.l, Ls, eLs, ws);
    __syncthreads();

    // (Q K^T)^T tiles (s block sb, t block w), decayed and masked: lane holds column t = tq, rows s.
    bf16x8 qf[2];
    qf[0] = frag(Qs, tq, 0, g);
    qf[1] = frag(Qs, tq, 1, g);
    const float Lt = Ls[tq];
    f32x4 pt[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      pt[sb] = zero4();
      if (sb <= w) {
        pt[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 0, g), qf[0], pt[sb]);
        pt[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 1, g), qf[1], pt[sb]);
        const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 16 * sb + 4 * g + r;
          pt[sb][r] = (s <= tq) ? pt[sb][r] * __expf(fminf(Lt - Lsv[r], 0.f)) : 0.f;
        }
      }
    }
    const bf16x8 af0 = pack(pt[0], pt[1]);
    const bf16x8 af1 = pack(pt[2], pt[3]);
    const float eLt = eLs[tq];
    const bf16x8 qe0 = frag_scaled(Qs, tq, 0, g, eLt);
    const bf16x8 qe1 = frag_scaled(Qs, tq, 1, g, eLt);

    // O^T tiles (j block jt, t block w) = V^T A^T + S^T (Q o eL)^T; lane holds token tq, values 16jt+4g..+3
    const bool t_ok = t0 + tq < T;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 acc = zero4();
      acc = pgn_mfma(frag(VT, 16 * jt + i, 0, g), af0, acc);
      if (w >= 2) acc = pgn_mfma(frag(VT, 16 * jt + i, 1, g), af1, acc);
      acc = pgn_mfma(frag(ST, 16 * jt + i, 0, g), qe0, acc);
      acc = pgn_mfma(frag(ST, 16 * jt + i, 1, g), qe1, acc);
      if (t_ok) *reinterpret_cast<bf16x4*>(o + boff + (size_t)(t0 + tq) * DK + 16 * jt + 4 * g) = to_bf16x4(acc);
    }

    // the entering state, bf16, (d, j) layout
    if (sent) {
      __bf16* sc = sent + ((size_t)bh * NC + c) * DK * DK;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[(16 * w + 4 * g + r) * DK + 16 * jt + i] = (__bf16)S[jt][r];
    }

    // S <- a S + (K o w)^T V, rows 16w.. of S
    const float a_c = __expf(Ls[C - 1]);
    const bf16x8 kw0 = frag_scaled_k(KT, 16 * w + i, 0, g, ws);
    const bf16x8 kw1 = frag_scaled_k(KT, 16 * w + i, 1, g, ws);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      S[jt] = S[jt] * a_c;
      S[jt] = pgn_mfma(kw0, frag(VT, 16 * jt + i, 0, g), S[jt]);
      S[jt] = pgn_mfma(kw1, frag(VT, 16 * jt + i, 1, g), S[jt]);
    }
    __syncthreads();
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) store_T(ST, 16 * jt, 16 * w, g, i, S[jt]);
  }

#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) Sfin[soff + (16 * w + 4 * g + r) * DK + 16 * jt + i] = S[jt][r];
}

__global__ __launch_bounds__(256) void aspin_plain_bwd(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const __bf16* __restrict__ sent, const __bf16* __restrict__ dO,
    const float* __restrict__ dSfin, __bf16* __restrict__ dq, __bf16* __restrict__ dk, __bf16* __restrict__ dv,
    float* __restrict__ dla, float* __restrict__ dS0, int T, int NC) {
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* Qs = reinterpret_cast<__bf16*>(smem);
  __bf16* QT = Qs + TILE;
  __bf16* Ks = QT + TILE;
  __bf16* KT = Ks + TILE;
  __bf16* Vs = KT + TILE;
  __bf16* VT = Vs + TILE;
  __bf16* Os = VT + TILE;   // dO
  __bf16* OT = Os + TILE;   // dO^T
  __bf16* Ss = OT + TILE;   // S_c, (d, j)
  __bf16* dSs = Ss + TILE;  // dS, (d, j)
  __bf16* dST = dSs + TILE; // dS^T, (j, d)
  float* Ls = reinterpret_cast<float*>(dST + TILE);
  float* eLs = Ls + C;
  float* ws = eLs + C;
  float* rowpart = ws + C;     // [4][C]: row sums of dA o A per s block (wave)
  float* colM = rowpart + 4 * C;  // [C]
  float* qz = colM + C;        // [C]: q_t . (S_c dO_t)
  float* dwv = qz + C;         // [C]: k_s . (dS v_s)
  float* sdot = dwv + C;       // [4]: per-wave <S_c, dS>

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i;
  const int bh = blockIdx.x;
  const size_t boff = (size_t)bh * T * DK;
  const size_t soff = (size_t)bh * DK * DK;

  // dS rows 16w + 4g + r, column 16 jt + i
  f32x4 dS[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) dS[jt][r] = dSfin ? dSfin[soff + (16 * w + 4 * g + r) * DK + 16 * jt + i] : 0.f;
    store_T(dST, 16 * jt, 16 * w, g, i, dS[jt]);
    store_N(dSs, 16 * w, 16 * jt, g, i, dS[jt]);
  }

  const int sw = 16 * w + i;  // this lane's s (column) for s-indexed tiles, and t for t-indexed ones
  for (int cc = NC - 1; cc >= 0; --cc) {
    const int t0 = cc * C;
    const int nrows = min(C, T - t0);
    stage64(q + boff + (size_t)t0 * DK, DK, nrows, Qs, QT);
    stage64(k + boff + (size_t)t0 * DK, DK, nrows, Ks, KT);
    stage64(v + boff + (size_t)t0 * DK, DK, nrows, Vs, VT);
    stage64(dO + boff + (size_t)t0 * DK, DK, nrows, Os, OT);
    stage64(sent + ((size_t)bh * NC + cc) * DK * DK, DK, DK, Ss, nullptr);
    if (w == 0) chunk_decays(la + (size_t)bh * T, t0, T, x.l, Ls, eLs, ws);
    __syncthreads();
    const float a_c = __expf(Ls[C - 1]);

    // (1) A and dP tiles (t block tb >= w, s block w): lane holds column s = sw, rows t = 16tb + 4g + r
    f32x4 At[4], dPt[4];
    const float Ls_s = Ls[sw];
    const bf16x8 kf0 = frag(Ks, sw, 0, g), kf1 = frag(Ks, sw, 1, g);
    const bf16x8 vf0 = frag(Vs, sw, 0, g), vf1 = frag(Vs, sw, 1, g);
    float colsum = 0.f;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      At[tb] = zero4();
      dPt[tb] = zero4();
      float rows[4] = {0.f, 0.f, 0.f, 0.f};
      if (tb >= w) {
        f32x4 P = zero4(), dA = zero4();
        P = pgn_mfma(frag(Qs, 16 * tb + i, 0, g), kf0, P);
        P = pgn_mfma(frag(Qs, 16 * tb + i, 1, g), kf1, P);
        dA = pgn_mfma(frag(Os, 16 * tb + i, 0, g), vf0, dA);
        dA = pgn_mfma(frag(Os, 16 * tb + i, 1, g), vf1, dA);
        const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * g + r;
          const float dec = (t >= sw) ? __expf(fminf(Ltv[r] - Ls_s, 0.f)) : 0.f;
          At[tb][r] = P[r] * dec;
          dPt[tb][r] = dA[r] * dec;
          const float m = dA[r] * At[tb][r];
          colsum += m;
          rows[r] = m;
        }
      }
      // row sums of this s block for rows t = 16tb + 4g + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s16 = sum16(rows[r]);
        if (i == 0) rowpart[w * C + 16 * tb + 4 * g + r] = s16;
      }
    }
    colsum = sum_groups(colsum);
    if (g == 0) colM[sw] = colsum;
    const bf16x8 A0 = pack(At[0], At[1]), A1 = pack(At[2], At[3]);
    const bf16x8 dP0 = pack(dPt[0], dPt[1]), dP1 = pack(dPt[2], dPt[3]);
    const float w_s = ws[sw];

    // (2) dV^T tiles (j block jt, s block w) = dO^T A + w_s dS^T K^T
    const bool s_ok = t0 + sw < T;
    {
      const bf16x8 kw0 = frag_scaled(Ks, sw, 0, g, w_s), kw1 = frag_scaled(Ks, sw, 1, g, w_s);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        f32x4 acc = zero4();
        acc = pgn_mfma(frag(OT, 16 * jt + i, 0, g), A0, acc);
        acc = pgn_mfma(frag(OT, 16 * jt + i, 1, g), A1, acc);
        acc = pgn_mfma(frag(dST, 16 * jt + i, 0, g), kw0, acc);
        acc = pgn_mfma(frag(dST, 16 * jt + i, 1, g), kw1, acc);
        if (s_ok) *reinterpret_cast<bf16x4*>(dv + boff + (size_t)(t0 + sw) * DK + 16 * jt + 4 * g) = to_bf16x4(acc);
      }
    }
    // (3) dK^T tiles (d block dt, s block w) = Q^T dP + w_s (dS V^T); k_s.(dS v_s) on the way
    {
      float dw_s = 0.f;
      const __bf16* krow = Ks + sw * kPitch;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        f32x4 acc = zero4(), Y = zero4();
        acc = pgn_mfma(frag(QT, 16 * dt + i, 0, g), dP0, acc);
        acc = pgn_mfma(frag(QT, 16 * dt + i, 1, g), dP1, acc);
        Y = pgn_mfma(frag(dSs, 16 * dt + i, 0, g), vf0, Y);
        Y = pgn_mfma(frag(dSs, 16 * dt + i, 1, g), vf1, Y);
        const f32x4 kk = to_f32x4(*reinterpret_cast<const bf16x4*>(krow + 16 * dt + 4 * g));
#pragma unroll
        for (int r = 0; r < 4; ++r) dw_s += kk[r] * Y[r];
        acc = acc + Y * w_s;
        if (s_ok) *reinterpret_cast<bf16x4*>(dk + boff + (size_t)(t0 + sw) * DK + 16 * dt + 4 * g) = to_bf16x4(acc);
      }
      dw_s = sum_groups(dw_s);
      if (g == 0) dwv[sw] = dw_s;
    }
    // (4) dP^T tiles (s block sb <= w, t block w): lane holds column t = sw, rows s
    f32x4 dPT[4];
    {
      const float Lt = Ls[sw];
      const bf16x8 of0 = frag(Os, sw, 0, g), of1 = frag(Os, sw, 1, g);
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        dPT[sb] = zero4();
        if (sb <= w) {
          dPT[sb] = pgn_mfma(frag(Vs, 16 * sb + i, 0, g), of0, dPT[sb]);
          dPT[sb] = pgn_mfma(frag(Vs, 16 * sb + i, 1, g), of1, dPT[sb]);
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = 16 * sb + 4 * g + r;
            dPT[sb][r] = (s <= sw) ? dPT[sb][r] * __expf(fminf(Lt - Lsv[r], 0.f)) : 0.f;
          }
        }
      }
    }
    // (5) dQ^T tiles (d block dt, t block w) = K^T dP^T + eL_t (S_c dO^T); q_t.(S_c dO_t) on the way
    {
      const bf16x8 b0 = pack(dPT[0], dPT[1]), b1 = pack(dPT[2], dPT[3]);
      const bf16x8 of0 = frag(Os, sw, 0, g), of1 = frag(Os, sw, 1, g);
      const float eLt = eLs[sw];
      const __bf16* qrow = Qs + sw * kPitch;
      float qzt = 0.f;
      const bool t_ok = t0 + sw < T;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        f32x4 acc = zero4(), Z = zero4();
        acc = pgn_mfma(frag(KT, 16 * dt + i, 0, g), b0, acc);
        acc = pgn_mfma(frag(KT, 16 * dt + i, 1, g), b1, acc);
        Z = pgn_mfma(frag(Ss, 16 * dt + i, 0, g), of0, Z);
        Z = pgn_mfma(frag(Ss, 16 * dt + i, 1, g), of1, Z);
        const f32x4 qq = to_f32x4(*reinterpret_cast<const bf16x4*>(qrow + 16 * dt + 4 * g));
#pragma unroll
        for (int r = 0; r < 4; ++r) qzt += qq[r] * Z[r];
        acc = acc + Z * eLt;
        if (t_ok) *reinterpret_cast<bf16x4*>(dq + boff + (size_t)(t0 + sw) * DK + 16 * dt + 4 * g) = to_bf16x4(acc);
      }
      qzt = sum_groups(qzt);
      if (g == 0) qz[sw] = qzt;
    }
    // (6) <S_c, dS> over this wave's rows of dS
    {
      float sd = 0.f;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sd += (float)Ss[(16 * w + 4 * g + r) * kPitch + 16 * jt + i] * dS[jt][r];
      sd = wave_sum(sd);
      if (x.l == 0) sdot[w] = sd;
    }
    // (7) dS <- a dS + (Q o eL)^T dO, rows 16w.. of dS
    {
      const bf16x8 qe0 = frag_scaled_k(QT, 16 * w + i, 0, g, eLs), qe1 = frag_scaled_k(QT, 16 * w + i, 1, g, eLs);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        dS[jt] = dS[jt] * a_c;
        dS[jt] = pgn_mfma(qe0, frag(OT, 16 * jt + i, 0, g), dS[jt]);
        dS[jt] = pgn_mfma(qe1, frag(OT, 16 * jt + i, 1, g), dS[jt]);
      }
    }
    __syncthreads();
    // (8) dla for this chunk (wave 0), while the others publish the new dS
    if (w == 0) {
      const int t = x.l;
      float dL = rowpart[t] + rowpart[C + t] + rowpart[2 * C + t] + rowpart[3 * C + t] - colM[t] +
                 eLs[t] * qz[t] - ws[t] * dwv[t];
      const float wdw = wave_sum(ws[t] * dwv[t]);
      if (t == C - 1) dL += wdw + a_c * (sdot[0] + sdot[1] + sdot[2] + sdot[3]);
      // reverse inclusive cumulative sum over the chunk
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_down(dL, off);
        if (t + off < 64) dL += y;
      }
      if (t0 + t < T) dla[(size_t)bh * T + t0 + t] = dL;
    }
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      store_T(dST, 16 * jt, 16 * w, g, i, dS[jt]);
      store_N(dSs, 16 * w, 16 * jt, g, i, dS[jt]);
    }
    __syncthreads();
  }
  if (dS0) {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) dS0[soff + (16 * w + 4 * g + r) * DK + 16 * jt + i] = dS[jt][r];
  }
}

constexpr size_t kBwdSmem = 11 * TILE * sizeof(__bf16) + (3 * C + 4 * C + 3 * C + 4) * sizeof(float);

bool shape_ok(int64_t B, int64_t H, int64_t T, int64_t D, int64_t Cc) {
  if (B <= 0 || H <= 0 || T <= 0) return false;
  if (B * H >= ((int64_t)1 << 31) || T >= ((int64_t)1 << 28)) return false;
  return D == DK && Cc == C;
}

}  // namespace

extern "C" int pragnosia_aspin_chunk_fwd(const void* q, const void* k, const void* v, const float* la, const float* S0,
                                         void* o, float* S_final, void* sent, int64_t B, int64_t H, int64_t T,
                                         int64_t D, int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && o && S_final);
  const int NC = (int)((T + C - 1) / C);
  hipLaunchKernelGGL(aspin_plain_fwd, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, S0, (__bf16*)o, S_final,
                     (__bf16*)sent, (int)T, NC);
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_aspin_chunk_bwd(const void* q, const void* k, const void* v, const float* la,
                                         const void* sent, const void* dO, const float* dS_final, void* dq, void* dk,
                                         void* dv, float* dla, float* dS0, int64_t B, int64_t H, int64_t T, int64_t D,
                                         int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && sent && dO && dq && dk && dv && dla);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)aspin_plain_bwd, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kBwdSmem);
    if (e != hipSuccess) return (int)e;
    attr_set = true;
  }
  const int NC = (int)((T + C - 1) / C);
  hipLaunchKernelGGL(aspin_plain_bwd, dim3((unsigned)(B * H)), dim3(256), kBwdSmem, (hipStream_t)stream,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, (const __bf16*)sent,
                     (const __bf16*)dO, dS_final, (__bf16*)dq, (__bf16*)dk, (__bf16*)dv, dla, dS0, (int)T, NC);
  PGN_RETURN_LAUNCH();
}
