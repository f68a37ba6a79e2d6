// The associative carrier's chunked scan, plain write rule: forward and hand-written backward on bf16 MFMA.
//
// Per (batch, head), with chunk C = 64 tokens, head dim D = 64, la_t <= 0 the per-token log-decay and, within a
// chunk, L the inclusive cumulative sum of la, dec[t,s] = exp(L_t - L_s) for s <= t (else 0), eL = exp(L),
// w = exp(L_C - L), a = exp(L_C):
//     O       = ((Q K^T) o dec) V + (Q o eL) S_c
//     S_{c+1} = a S_c + (K o w)^T V
// (the reference's `_scan_twopass`, `src/assoc.py:118-165`; its GPU form `src/assoc_kernel.py:47-70,188-202`).
// Backward, per chunk, with dS_c the gradient on the state LEAVING chunk c, dA = dO V^T, dP = dA o dec,
// A = (Q K^T) o dec:
//     dQ = dP K + eL o (dO S_c^T)            dK = dP^T Q + w o (V dS_c^T)
//     dV = A^T dO + (K o w) dS_c             dS_{c-1} = a dS_c + (Q o eL)^T dO
//     dL_t = rowsum(dA o A)_t - colsum(dA o A)_t + eL_t q_t.(S_c dO_t) - w_t k_t.(dS_c v_t),
//     dL_{C-1} += sum_s w_s k_s.(dS_c v_s) + a <S_c, dS_c>,     dla = reverse cumulative sum of dL
// (equations of `src/assoc_kernel.py:73-116`, `:205-220`, `:279-296`).
//
// The only sequential dependency is the state (forward) or state gradient (backward) carried from chunk to chunk,
// and that recurrence is a scaled add of one 64 x 64 matrix per chunk.
//
// Forward: plain_fwd_sp, one persistent single pass. A work item is one (batch-head, chunk); it computes its
// chunk's state term, publishes it, computes the intra-chunk part of its output, obtains its entering state by
// look-back over its predecessors' publications (lookback.h), and finishes its output. Every input is read once
// and the output, the entering states and the final state are written once.
//
// Backward: two kernels.
//   plain_state<true>  one workgroup of SW waves per (batch, head). Wave w takes chunk w of a group of SW chunks,
//                      stages its X and Y tiles transposed in its own LDS region and computes the chunk's term
//                      (32 bf16 MFMAs), all chunks of the group at once; then the recurrence runs across the waves
//                      through one fp32 LDS buffer (one scaled add per chunk, a barrier between chunks), and every
//                      wave stores the state it read: X = Q, Y = dO, f = eL, gradients dS_c in reverse chunk order
//                      (bf16, a workspace) and dS0.
//   plain_bwd_local    one workgroup of 8 waves per (batch-head, chunk): dQ, dK, dV and dla of one chunk from Q, K,
//                      V, dO, S_c and dS_c. Waves 0-3 own token block wl in the query role (dQ, row sums of
//                      dA o A, q.(S dO)); waves 4-7 own it in the key role (dV, dK, column sums, k.(dS v), <S, dS>).
// Every product that has a transposed operand is computed in the orientation whose accumulator is the next
// product's operand (pgn::pack).
#include <algorithm>

#include "lookback.h"
#include "mfma_tile.h"

using namespace pgn;

namespace {

constexpr int C = 64;
constexpr int DK = 64;
constexpr int TILE = 64 * kPitch;  // one staged 64 x 64 tile
constexpr int SW = 8;              // waves (chunks in flight) of the state pass

PGN_DEVICE float incl_scan64(float x, int l) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(x, off);
    if (l >= off) x += y;
  }
  return x;
}

PGN_DEVICE float rev_scan64(float x, int l) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_down(x, off);
    if (l + off < 64) x += y;
  }
  return x;
}

// Per-chunk decay statistics into LDS (one wave, lane = token): L, eL = exp(L), w = exp(L_C - L).
PGN_DEVICE void chunk_decays(float la_l, int l, float* Ls, float* eLs, float* ws) {
  const float L = incl_scan64(la_l, l);
  const float LC = __shfl(L, 63);
  Ls[l] = L;
  eLs[l] = __expf(L);
  ws[l] = __expf(fminf(LC - L, 0.f));
}

// ------------------------------------------------------------------------------------------------------------------
// state pass. The chunk terms are computed transposed (M^T = Y^T (X o f)), so a lane's accumulator holds four
// consecutive columns of one state row: tile tt = 4 db + jt, lane l, element r is entry
// (16 db + l % 16, 16 jt + 4 (l / 16) + r). The carry buffer holds the state in that order (a wave moves it with
// 16-byte LDS accesses) and every global access of a state is an 8- or 16-byte row segment.
constexpr size_t kStateSmem = (size_t)SW * 2 * TILE * sizeof(__bf16) + 16 * 64 * 4 * sizeof(float) +
                              (size_t)SW * C * sizeof(float) + SW * sizeof(float);

template <bool REV>
__global__ __launch_bounds__(64 * SW) void plain_state(const __bf16* __restrict__ X, const __bf16* __restrict__ Y,
                                                       const float* __restrict__ la, const float* __restrict__ init,
                                                       __bf16* __restrict__ out, float* __restrict__ fin, int T,
                                                       int NC) {
  extern __shared__ __align__(16) unsigned char smem[];
  const WaveIdx x = wave_idx();
  const int w = x.w, l = x.l, g = x.g, i = x.i;
  __bf16* XT = reinterpret_cast<__bf16*>(smem) + (size_t)w * 2 * TILE;  // this wave's X^T (d, t)
  __bf16* YT = XT + TILE;                                                 // this wave's Y^T (j, t)
  f32x4* CB = reinterpret_cast<f32x4*>(smem + (size_t)SW * 2 * TILE * sizeof(__bf16));
  float* fw = reinterpret_cast<float*>(CB + 16 * 64);  // [SW][C] per-token scale of each wave's chunk
  float* aw = fw + SW * C;                             // [SW] chunk decay a_c
  const int bh = blockIdx.x;
  const size_t boff = (size_t)bh * T * DK;
  const size_t soff = (size_t)bh * DK * DK;

  // initial carry: S0 (forward) or dS_final (backward), zero when absent; waves split the 16 tiles
  for (int tt = w; tt < 16; tt += SW) {
    const int db = tt >> 2, jt = tt & 3;
    CB[tt * 64 + l] = init ? *reinterpret_cast<const f32x4*>(init + soff + (size_t)(16 * db + i) * DK + 16 * jt + 4 * g)
                           : zero4();
  }

  const int ngroups = (NC + SW - 1) / SW;
  for (int gi = 0; gi < ngroups; ++gi) {
    const int n = gi * SW + w;  // position of this wave's chunk in processing order
    const bool active = n < NC;
    const int c = REV ? NC - 1 - n : n;
    Blk4 xb[4], yb[4];
    float lav = 0.f;
    if (active) {
      const int t0 = c * C, nr = min(C, T - t0);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        xb[b] = load_blk(X + boff + (size_t)t0 * DK, DK, nr, l + 64 * b);
        yb[b] = load_blk(Y + boff + (size_t)t0 * DK, DK, nr, l + 64 * b);
      }
      lav = l < nr ? la[(size_t)bh * T + t0 + l] : 0.f;
    }
    __syncthreads();  // the previous group is done with the LDS tiles and the scale vectors
    if (active) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int blk = l + 64 * b;
        put_blk_T(XT, xb[b], 4 * (blk >> 4), 4 * (blk & 15));
        put_blk_T(YT, yb[b], 4 * (blk >> 4), 4 * (blk & 15));
      }
      const float L = incl_scan64(lav, l);
      const float LC = __shfl(L, 63);
      fw[w * C + l] = REV ? __expf(L) : __expf(fminf(LC - L, 0.f));
      if (l == 0) aw[w] = __expf(LC);
    }
    __syncthreads();  // staged tiles and scales visible
    f32x4 M[16];
    if (active) {
      // M^T = Y^T (X o f): rows j (block jt), columns d (block db); contracted over the chunk's tokens
      const float* f = fw + w * C;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 b0 = frag_scaled_k(XT, 16 * db + i, 0, g, f), b1 = frag_scaled_k(XT, 16 * db + i, 1, g, f);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          const f32x4 acc = pgn_mfma(frag(YT, 16 * jt + i, 0, g), b0, zero4());
          M[4 * db + jt] = pgn_mfma(frag(YT, 16 * jt + i, 1, g), b1, acc);
        }
      }
    }
    // the recurrence across the group's chunks, in processing order: carry <- a_c carry + M_c
    bf16x4 Sin[16];  // the carry this chunk saw, rounded for the store
#pragma unroll 1
    for (int s = 0; s < SW; ++s) {
      if (w == s && active) {
        const float a = aw[w];
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
          const f32x4 cur = CB[tt * 64 + l];
          Sin[tt] = to_bf16x4(cur);
          CB[tt * 64 + l] = cur * a + M[tt];
        }
      }
      __syncthreads();
    }
    if (active) {  // the state this chunk saw: entering state (forward) or leaving gradient (backward), bf16
      __bf16* dst = out + ((size_t)bh * NC + c) * DK * DK;
#pragma unroll
      for (int tt = 0; tt < 16; ++tt)
        *reinterpret_cast<bf16x4*>(dst + (16 * (tt >> 2) + i) * DK + 16 * (tt & 3) + 4 * g) = Sin[tt];
    }
  }
  // final carry: S_final (forward) or dS0 (backward)
  if (fin) {
    for (int tt = w; tt < 16; tt += SW) {
      *reinterpret_cast<f32x4*>(fin + soff + (size_t)(16 * (tt >> 2) + i) * DK + 16 * (tt & 3) + 4 * g) = CB[tt * 64 + l];
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// Single-pass forward (persistent; look-back scheduling and memory ordering as described in lookback.h). A
// workgroup of 4 waves per item (batch-head, chunk); wave w owns d block w of the chunk's state term and token block
// w of its output. The state term is computed transposed, M^T = V^T (K o w), so a lane holds the four state entries
// (d = 16 w + i, j = 16 jt + 4 g .. + 3) of each value block jt: aggregates and inclusive states are exchanged in
// that order ([item][w][jt][lane] f32x4, 16 KiB) and `sent` is written as 8-byte row segments.
//
// Inputs of the next item are prefetched into registers by waves 1-3 (one tile each: Q, K, V) while the current
// item computes; wave 0 only prefetches the 64 decays, so its polling loads never wait behind tile loads (the
// vector memory counter completes in order).
struct LbPtrs {
  uint64_t* flags;
  float* av;
  f32x4* agg;
  f32x4* incl;
};

PGN_DEVICE LbPtrs lb_ptrs(unsigned char* ws, int64_t n) {
  const LbLayout L = lb_layout(n);
  LbPtrs P;
  P.flags = reinterpret_cast<uint64_t*>(ws + L.flags_off);
  P.av = reinterpret_cast<float*>(ws + L.av_off);
  P.agg = reinterpret_cast<f32x4*>(ws + L.agg_off);
  P.incl = reinterpret_cast<f32x4*>(ws + L.incl_off);
  return P;
}

// Exchange-order offset (bytes) of lane l's value block jt of wave w within one 16 KiB state.
PGN_DEVICE int xoff(int w, int jt, int l) { return ((w * 4 + jt) * 64 + l) * 16; }

// The entering value X of scan position `pos` of head bh, in the exchange order of wave w: wait for the block's
// publications, then run the recurrence from the block's entering value (`init`, fp32 (d, j) row-major or NULL for
// zero, in the first block; the previous block's inclusive value otherwise) through the aggregates of positions
// b .. pos-1, loaded two at a time. Item of position p: p * nbh + bh. s_xcc: LDS, kLbGroup + 1 ints.
PGN_DEVICE void lb_entering(const LbPtrs& P, uint64_t epoch, int pos, int bh, int nbh, int w, int l, int g, int i,
                            int* s_xcc, const float* __restrict__ init, f32x4 (&X)[4]) {
  const int b = pos - pos % kLbGroup;
  const int me = xcc_id();
  if (pos > 0) {
    if (w == 0) {
      int wx = 0;
      const bool ok = lb_wait_block(pos, l, epoch, [&](int p) { return P.flags + (size_t)p * nbh + bh; }, &wx);
      if (l <= pos - b) s_xcc[l] = ok ? wx : -1;
    }
    __syncthreads();
    if (s_xcc[0] < 0) {  // timed out: count it and continue with a zero state (never hang)
      if (threadIdx.x == 0) atomicAdd(&g_lookback_timeouts, 1u);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) X[jt] = zero4();
      return;
    }
  }
  if (b > 0) {
    const bool local = __builtin_amdgcn_readfirstlane(s_xcc[pos - b]) == me;
    const auto r = lb_rsrc(P.incl + ((size_t)(b - 1) * nbh + bh) * 1024, 16384);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) X[jt] = lb_load4(r, xoff(w, jt, l), local);
  } else {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
      X[jt] = init ? *reinterpret_cast<const f32x4*>(init + (size_t)bh * DK * DK + (16 * w + i) * DK + 16 * jt + 4 * g)
                   : zero4();
  }
  for (int j0 = b; j0 < pos; j0 += 2) {
    f32x4 buf[2][4];
    float aj[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = min(j0 + u, pos - 1);
      const size_t it = (size_t)j * nbh + bh;
      const bool local = __builtin_amdgcn_readfirstlane(s_xcc[j - b]) == me;
      const auto r = lb_rsrc(P.agg + it * 1024, 16384);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) buf[u][jt] = lb_load4(r, xoff(w, jt, l), local);
      aj[u] = __hip_atomic_load(P.av + it, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (j0 + u < pos) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) X[jt] = X[jt] * aj[u] + buf[u][jt];
      }
    }
  }
}

constexpr size_t kFwdSmem = 5 * TILE * sizeof(__bf16) + 3 * C * sizeof(float) + 16 * sizeof(int);

__global__ __launch_bounds__(256, 2) void plain_fwd_sp(const __bf16* __restrict__ q, const __bf16* __restrict__ k,
                                                    const __bf16* __restrict__ v, const float* __restrict__ la,
                                                    const float* __restrict__ S0, __bf16* __restrict__ o,
                                                    float* __restrict__ S_final, __bf16* __restrict__ sent,
                                                    unsigned char* ws, uint64_t epoch, int nbh, int T, int NC) {
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* Qs = reinterpret_cast<__bf16*>(smem);
  __bf16* Ks = Qs + TILE;
  __bf16* KT = Ks + TILE;
  __bf16* VT = KT + TILE;
  __bf16* ST = VT + TILE;
  float* Ls = reinterpret_cast<float*>(ST + TILE);
  float* eLs = Ls + C;
  float* wsc = eLs + C;
  int* s_xcc = reinterpret_cast<int*>(wsc + C);
  const WaveIdx x = wave_idx();
  const int w = x.w, l = x.l, g = x.g, i = x.i, tid = threadIdx.x;
  const int n = nbh * NC;
  const LbPtrs P = lb_ptrs(ws, n);
  const int me = xcc_id();

  // prefetch registers: wave 1 the Q tile, wave 2 the K tile, wave 3 the V tile (four 4 x 4 blocks per lane);
  // wave 0 the 64 decays
  Blk4 pre[4];
  float pre_la = 0.f;
  auto prefetch = [&](int it) {
    const int c = it / nbh, bh = it - c * nbh;
    const int t0 = c * C, nr = min(C, T - t0);
    const size_t coff = ((size_t)bh * T + t0) * DK;
    if (w == 0) {
      pre_la = l < nr ? la[(size_t)bh * T + t0 + l] : 0.f;
    } else {
      const __bf16* src = (w == 1 ? q : w == 2 ? k : v) + coff;
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) pre[b4] = load_blk(src, DK, nr, l + 64 * b4);
    }
  };
  int item = blockIdx.x;
  if (item < n) prefetch(item);

  for (; item < n; item += gridDim.x) {
    const int c = item / nbh, bh = item - c * nbh;
    const int t0 = c * C, nr = min(C, T - t0);
    const size_t coff = ((size_t)bh * T + t0) * DK;
    __syncthreads();  // the previous item is done with the LDS tiles and vectors
    if (w == 0) {
      chunk_decays(pre_la, l, Ls, eLs, wsc);
    } else {
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) {
        const int blk = l + 64 * b4, br = 4 * (blk >> 4), bc = 4 * (blk & 15);
        if (w == 1) {
          put_blk(Qs, pre[b4], br, bc);
        } else if (w == 2) {
          put_blk(Ks, pre[b4], br, bc);
          put_blk_T(KT, pre[b4], br, bc);
        } else {
          put_blk_T(VT, pre[b4], br, bc);
        }
      }
    }
    __syncthreads();

    // this chunk's state term, d block w: M^T tiles (j block jt, d block w) = V^T (K o w)
    f32x4 M[4];
    {
      const bf16x8 b0 = frag_scaled_k(KT, 16 * w + i, 0, g, wsc), b1 = frag_scaled_k(KT, 16 * w + i, 1, g, wsc);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        M[jt] = pgn_mfma(frag(VT, 16 * jt + i, 0, g), b0, zero4());
        M[jt] = pgn_mfma(frag(VT, 16 * jt + i, 1, g), b1, M[jt]);
      }
    }
    const float a_c = __expf(Ls[C - 1]);
    const bool last = c == NC - 1;
    const bool block_last = c % kLbGroup == kLbGroup - 1;
    if (!last && !block_last) {  // publish the aggregate for the later chunks of this block
      const auto r = lb_rsrc(P.agg + (size_t)item * 1024, 16384);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) lb_store4(r, xoff(w, jt, l), M[jt]);
      if (tid == 0) __hip_atomic_store(P.av + item, a_c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      lb_publish_flag(P.flags + item, lb_flag_word(epoch, me, kFlagAgg));
    }
    // the next item's inputs, in flight while this one computes
    if (item + (int)gridDim.x < n) prefetch(item + gridDim.x);

    // intra-chunk output, token block w: (Q K^T)^T tiles decayed and masked, then O^T = V^T A^T
    const int t = 16 * w + i;
    f32x4 acc[4];
    {
      const bf16x8 qf0 = frag(Qs, t, 0, g), qf1 = frag(Qs, t, 1, g);
      f32x4 pt[4];
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        pt[sb] = zero4();
        if (sb <= w) {
          pt[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 0, g), qf0, pt[sb]);
          pt[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 1, g), qf1, pt[sb]);
        }
      }
      const float Lt = Ls[t];
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        if (sb <= w) {
          const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) pt[sb][r] *= masked_decay(Lt - Lsv[r], 16 * sb + 4 * g + r <= t);
        }
      }
      const bf16x8 af0 = pack(pt[0], pt[1]), af1 = pack(pt[2], pt[3]);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        acc[jt] = pgn_mfma(frag(VT, 16 * jt + i, 0, g), af0, zero4());
        if (w >= 2) acc[jt] = pgn_mfma(frag(VT, 16 * jt + i, 1, g), af1, acc[jt]);
      }
    }

    // the entering state S_c; the leaving state is published (last chunk of a block) or is the final state
    f32x4 Sx[4];
    lb_entering(P, epoch, c, bh, nbh, w, l, g, i, s_xcc, S0, Sx);
    if (last || block_last) {
      f32x4 Sn[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) Sn[jt] = Sx[jt] * a_c + M[jt];
      if (!last) {
        const auto r = lb_rsrc(P.incl + (size_t)item * 1024, 16384);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) lb_store4(r, xoff(w, jt, l), Sn[jt]);
        lb_publish_flag(P.flags + item, lb_flag_word(epoch, me, kFlagIncl));
      } else {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          *reinterpret_cast<f32x4*>(S_final + (size_t)bh * DK * DK + (16 * w + i) * DK + 16 * jt + 4 * g) = Sn[jt];
      }
    }
    // S_c: to `sent` (bf16 row segments) and, transposed, to LDS for the inter-chunk product
    {
      __bf16* sdst = sent ? sent + ((size_t)bh * NC + c) * DK * DK + (16 * w + i) * DK + 4 * g : nullptr;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const bf16x4 sb4 = to_bf16x4(Sx[jt]);
        if (sdst) *reinterpret_cast<bf16x4*>(sdst + 16 * jt) = sb4;
#pragma unroll
        for (int r = 0; r < 4; ++r) ST[(16 * jt + 4 * g + r) * kPitch + 16 * w + i] = sb4[r];
      }
    }
    __syncthreads();
    // O^T += S^T (Q o eL)^T, then store: lane holds token t, value columns 16 jt + 4 g ..
    const float eLt = eLs[t];
    const bf16x8 qe0 = frag_scaled(Qs, t, 0, g, eLt), qe1 = frag_scaled(Qs, t, 1, g, eLt);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      acc[jt] = pgn_mfma(frag(ST, 16 * jt + i, 0, g), qe0, acc[jt]);
      acc[jt] = pgn_mfma(frag(ST, 16 * jt + i, 1, g), qe1, acc[jt]);
      if (t < nr) *reinterpret_cast<bf16x4*>(o + coff + (size_t)t * DK + 16 * jt + 4 * g) = to_bf16x4(acc[jt]);
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// backward of one chunk: 8 waves
constexpr size_t kLocalSmem = 10 * TILE * sizeof(__bf16) + (7 * C + 4) * sizeof(float);

__global__ __launch_bounds__(512) void plain_bwd_local(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const __bf16* __restrict__ sent, const __bf16* __restrict__ dSc,
    const __bf16* __restrict__ dO, __bf16* __restrict__ dq, __bf16* __restrict__ dk, __bf16* __restrict__ dv,
    float* __restrict__ dla, int T, int NC) {
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* Qs = reinterpret_cast<__bf16*>(smem);
  __bf16* QT = Qs + TILE;
  __bf16* Ks = QT + TILE;
  __bf16* KT = Ks + TILE;
  __bf16* Vs = KT + TILE;
  __bf16* Os = Vs + TILE;    // dO
  __bf16* OT = Os + TILE;    // dO^T
  __bf16* Ss = OT + TILE;    // S_c, (d, j)
  __bf16* dSs = Ss + TILE;   // dS_c, (d, j)
  __bf16* dST = dSs + TILE;  // dS_c^T, (j, d)
  float* Ls = reinterpret_cast<float*>(dST + TILE);
  float* eLs = Ls + C;
  float* ws = eLs + C;
  float* rowM = ws + C;    // row sums of dA o A (query role)
  float* colM = rowM + C;  // column sums of dA o A (key role)
  float* qz = colM + C;    // q_t . (S_c dO_t)
  float* dwv = qz + C;     // k_s . (dS_c v_s)
  float* sdot = dwv + C;   // per-wave <S_c, dS_c>

  const WaveIdx x = wave_idx();
  const int w = x.w, wl = w & 3, g = x.g, i = x.i, tid = threadIdx.x;
  const bool gk = w >= 4;
  const int bh = blockIdx.x / NC, c = blockIdx.x - bh * NC;
  const int t0 = c * C, nr = min(C, T - t0);
  const size_t coff = ((size_t)bh * T + t0) * DK;
  const size_t soff = ((size_t)bh * NC + c) * DK * DK;
  {
    const int b = tid & 255;
    const int br = 4 * (b >> 4), bc = 4 * (b & 15);
    if (tid < 256) {
      const Blk4 pq = load_blk(q + coff, DK, nr, b);
      const Blk4 pv = load_blk(v + coff, DK, nr, b);
      const Blk4 ps = load_blk(sent + soff, DK, DK, b);
      const Blk4 pd = load_blk(dSc + soff, DK, DK, b);
      put_blk(Qs, pq, br, bc);
      put_blk_T(QT, pq, br, bc);
      put_blk(Vs, pv, br, bc);
      put_blk(Ss, ps, br, bc);
      put_blk(dSs, pd, br, bc);
      put_blk_T(dST, pd, br, bc);
    } else {
      const Blk4 pk = load_blk(k + coff, DK, nr, b);
      const Blk4 po = load_blk(dO + coff, DK, nr, b);
      put_blk(Ks, pk, br, bc);
      put_blk_T(KT, pk, br, bc);
      put_blk(Os, po, br, bc);
      put_blk_T(OT, po, br, bc);
    }
    if (w == 0) chunk_decays(x.l < nr ? la[(size_t)bh * T + t0 + x.l] : 0.f, x.l, Ls, eLs, ws);
  }
  __syncthreads();

  const int me = 16 * wl + i;  // query role: this lane's t; key role: this lane's s
  const bool row_ok = me < nr;
  if (!gk) {
    // ---------------- query role: t = me
    const bf16x8 qf0 = frag(Qs, me, 0, g), qf1 = frag(Qs, me, 1, g);
    const bf16x8 of0 = frag(Os, me, 0, g), of1 = frag(Os, me, 1, g);
    f32x4 PT[4], dAT[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {  // rows s, lane t: P[t][s] and dA[t][s]
      PT[sb] = zero4();
      dAT[sb] = zero4();
      if (sb <= wl) {
        PT[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 0, g), qf0, PT[sb]);
        PT[sb] = pgn_mfma(frag(Ks, 16 * sb + i, 1, g), qf1, PT[sb]);
        dAT[sb] = pgn_mfma(frag(Vs, 16 * sb + i, 0, g), of0, dAT[sb]);
        dAT[sb] = pgn_mfma(frag(Vs, 16 * sb + i, 1, g), of1, dAT[sb]);
      }
    }
    const float Lt = Ls[me];
    float rowacc = 0.f;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (sb <= wl) {
        const f32x4 Lsv = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float dec = masked_decay(Lt - Lsv[r], 16 * sb + 4 * g + r <= me);
          rowacc += dAT[sb][r] * (PT[sb][r] * dec);
          dAT[sb][r] *= dec;  // now dP^T
        }
      }
    }
    rowacc = sum_groups(rowacc);
    if (g == 0) rowM[me] = rowacc;
    const bf16x8 b0 = pack(dAT[0], dAT[1]), b1 = pack(dAT[2], dAT[3]);
    const float eLt = eLs[me];
    const __bf16* qrow = Qs + me * kPitch;
    float qzt = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {  // dQ^T tiles (d block dt, t block wl) = K^T dP^T + eL (S dO^T)
      f32x4 acc = pgn_mfma(frag(KT, 16 * dt + i, 0, g), b0, zero4());
      if (wl >= 2) acc = pgn_mfma(frag(KT, 16 * dt + i, 1, g), b1, acc);
      f32x4 Z = pgn_mfma(frag(Ss, 16 * dt + i, 0, g), of0, zero4());
      Z = pgn_mfma(frag(Ss, 16 * dt + i, 1, g), of1, Z);
      const f32x4 qq = to_f32x4(*reinterpret_cast<const bf16x4*>(qrow + 16 * dt + 4 * g));
#pragma unroll
      for (int r = 0; r < 4; ++r) qzt += qq[r] * Z[r];
      acc = acc + Z * eLt;
      if (row_ok) *reinterpret_cast<bf16x4*>(dq + coff + (size_t)me * DK + 16 * dt + 4 * g) = to_bf16x4(acc);
    }
    qzt = sum_groups(qzt);
    if (g == 0) qz[me] = qzt;
  } else {
    // ---------------- key role: s = me
    const bf16x8 kf0 = frag(Ks, me, 0, g), kf1 = frag(Ks, me, 1, g);
    const bf16x8 vf0 = frag(Vs, me, 0, g), vf1 = frag(Vs, me, 1, g);
    f32x4 At[4], dPt[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {  // rows t, lane s: P[t][s] and dA[t][s]
      At[tb] = zero4();
      dPt[tb] = zero4();
      if (tb >= wl) {
        At[tb] = pgn_mfma(frag(Qs, 16 * tb + i, 0, g), kf0, At[tb]);
        At[tb] = pgn_mfma(frag(Qs, 16 * tb + i, 1, g), kf1, At[tb]);
        dPt[tb] = pgn_mfma(frag(Os, 16 * tb + i, 0, g), vf0, dPt[tb]);
        dPt[tb] = pgn_mfma(frag(Os, 16 * tb + i, 1, g), vf1, dPt[tb]);
      }
    }
    const float Ls_s = Ls[me];
    float colacc = 0.f;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      if (tb >= wl) {
        const f32x4 Ltv = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float dec = masked_decay(Ltv[r] - Ls_s, 16 * tb + 4 * g + r >= me);
          At[tb][r] *= dec;
          colacc += dPt[tb][r] * At[tb][r];
          dPt[tb][r] *= dec;
        }
      }
    }
    colacc = sum_groups(colacc);
    if (g == 0) colM[me] = colacc;
    const bf16x8 A0 = pack(At[0], At[1]), A1 = pack(At[2], At[3]);
    const bf16x8 dP0 = pack(dPt[0], dPt[1]), dP1 = pack(dPt[2], dPt[3]);
    const float w_s = ws[me];
    // dV^T tiles (j block jt, s block wl) = dO^T A + dS^T (K o w)^T
    const bf16x8 kw0 = frag_scaled(Ks, me, 0, g, w_s), kw1 = frag_scaled(Ks, me, 1, g, w_s);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 acc = zero4();
      if (wl < 2) acc = pgn_mfma(frag(OT, 16 * jt + i, 0, g), A0, acc);
      acc = pgn_mfma(frag(OT, 16 * jt + i, 1, g), A1, acc);
      acc = pgn_mfma(frag(dST, 16 * jt + i, 0, g), kw0, acc);
      acc = pgn_mfma(frag(dST, 16 * jt + i, 1, g), kw1, acc);
      if (row_ok) *reinterpret_cast<bf16x4*>(dv + coff + (size_t)me * DK + 16 * jt + 4 * g) = to_bf16x4(acc);
    }
    // dK^T tiles (d block dt, s block wl) = Q^T dP + w_s (dS V^T); k_s.(dS v_s) on the way
    const __bf16* krow = Ks + me * kPitch;
    float dw = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 acc = zero4();
      if (wl < 2) acc = pgn_mfma(frag(QT, 16 * dt + i, 0, g), dP0, acc);
      acc = pgn_mfma(frag(QT, 16 * dt + i, 1, g), dP1, acc);
      f32x4 Y = pgn_mfma(frag(dSs, 16 * dt + i, 0, g), vf0, zero4());
      Y = pgn_mfma(frag(dSs, 16 * dt + i, 1, g), vf1, Y);
      const f32x4 kk = to_f32x4(*reinterpret_cast<const bf16x4*>(krow + 16 * dt + 4 * g));
#pragma unroll
      for (int r = 0; r < 4; ++r) dw += kk[r] * Y[r];
      acc = acc + Y * w_s;
      if (row_ok) *reinterpret_cast<bf16x4*>(dk + coff + (size_t)me * DK + 16 * dt + 4 * g) = to_bf16x4(acc);
    }
    dw = sum_groups(dw);
    if (g == 0) dwv[me] = dw;
    // <S_c, dS_c> over key rows 16 wl ..
    float sd = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * wl + 4 * g + r;
        sd += (float)Ss[d * kPitch + 16 * jt + i] * (float)dSs[d * kPitch + 16 * jt + i];
      }
    }
    sd = wave_sum(sd);
    if (x.l == 0) sdot[wl] = sd;
  }
  __syncthreads();
  if (w == 0) {  // dla for this chunk: the reverse cumulative sum of dL
    const int t = x.l;
    const float wdw = ws[t] * dwv[t];
    float dL = rowM[t] - colM[t] + eLs[t] * qz[t] - wdw;
    const float tot = wave_sum(wdw);
    if (t == C - 1) dL += tot + __expf(Ls[C - 1]) * (sdot[0] + sdot[1] + sdot[2] + sdot[3]);
    dL = rev_scan64(dL, t);
    if (t < nr) dla[(size_t)bh * T + t0 + t] = dL;
  }
}

bool shape_ok(int64_t B, int64_t H, int64_t T, int64_t D, int64_t Cc) {
  if (B <= 0 || H <= 0 || T <= 0) return false;
  if (B * H >= ((int64_t)1 << 24) || T >= ((int64_t)1 << 28)) return false;
  if (B * H * ((T + C - 1) / C) >= ((int64_t)1 << 31)) return false;
  return D == DK && Cc == C;
}

int set_smem(const void* fn, size_t bytes, bool& done) {
  if (done) return 0;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) return (int)e;
  done = true;
  return 0;
}

}  // namespace

extern "C" int64_t pragnosia_aspin_chunk_fwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D,
                                                             int64_t chunk) {
  if (!shape_ok(B, H, T, D, chunk)) return -1;
  return lb_layout(B * H * ((T + C - 1) / C)).total;
}

// Resident workgroups of a persistent kernel on the current device (blocks per CU x CUs), cached per kernel.
static int persistent_grid(const void* fn, int threads, size_t smem, int& cached) {
  if (cached > 0) return cached;
  int dev = 0, per_cu = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, smem) != hipSuccess || per_cu < 1)
    return -1;
  cached = per_cu * prop.multiProcessorCount;
  return cached;
}

extern "C" int pragnosia_aspin_chunk_fwd(const void* q, const void* k, const void* v, const float* la, const float* S0,
                                         void* o, float* S_final, void* sent, void* workspace,
                                         int64_t workspace_bytes, uint64_t epoch, int64_t B, int64_t H, int64_t T,
                                         int64_t D, int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && o && S_final && workspace);
  PGN_CHECK_ARG(workspace_bytes >= pragnosia_aspin_chunk_fwd_workspace_bytes(B, H, T, D, chunk));
  PGN_CHECK_ARG(epoch > 0 && epoch < ((uint64_t)1 << 56));
  static bool smem_set = false;
  static int grid_cap = 0;
  int rc = set_smem((const void*)plain_fwd_sp, kFwdSmem, smem_set);
  if (rc) return rc;
  const int cap = persistent_grid((const void*)plain_fwd_sp, 256, kFwdSmem, grid_cap);
  if (cap <= 0) return PRAGNOSIA_ERR_UNSUPPORTED;
  const int NC = (int)((T + C - 1) / C);
  const int nbh = (int)(B * H);
  const int64_t n = (int64_t)nbh * NC;
  const int grid = (int)std::min<int64_t>(n, cap);
  hipLaunchKernelGGL(plain_fwd_sp, dim3((unsigned)grid), dim3(256), kFwdSmem, (hipStream_t)stream,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, S0, (__bf16*)o, S_final,
                     (__bf16*)sent, (unsigned char*)workspace, epoch, nbh, (int)T, NC);
  PGN_RETURN_LAUNCH();
}

extern "C" unsigned int pragnosia_lookback_timeouts(void) { return lb_read_timeouts(); }

extern "C" int64_t pragnosia_aspin_chunk_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D,
                                                             int64_t chunk) {
  if (!shape_ok(B, H, T, D, chunk)) return -1;
  return B * H * ((T + C - 1) / C) * DK * DK * 2;
}

extern "C" int pragnosia_aspin_chunk_bwd(const void* q, const void* k, const void* v, const float* la,
                                         const void* sent, const void* dO, const float* dS_final, void* dq, void* dk,
                                         void* dv, float* dla, float* dS0, void* workspace, int64_t workspace_bytes,
                                         int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && sent && dO && dq && dk && dv && dla && workspace);
  PGN_CHECK_ARG(workspace_bytes >= pragnosia_aspin_chunk_bwd_workspace_bytes(B, H, T, D, chunk));
  static bool state_set = false, local_set = false;
  int rc = set_smem((const void*)plain_state<true>, kStateSmem, state_set);
  if (rc) return rc;
  rc = set_smem((const void*)plain_bwd_local, kLocalSmem, local_set);
  if (rc) return rc;
  const int NC = (int)((T + C - 1) / C);
  const int nbh = (int)(B * H);
  hipStream_t st = (hipStream_t)stream;
  __bf16* dSc = (__bf16*)workspace;
  hipLaunchKernelGGL(plain_state<true>, dim3((unsigned)nbh), dim3(64 * SW), kStateSmem, st, (const __bf16*)q,
                     (const __bf16*)dO, la, dS_final, dSc, dS0, (int)T, NC);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(plain_bwd_local, dim3((unsigned)(nbh * NC)), dim3(512), kLocalSmem, st, (const __bf16*)q,
                     (const __bf16*)k, (const __bf16*)v, la, (const __bf16*)sent, (const __bf16*)dSc,
                     (const __bf16*)dO, (__bf16*)dq, (__bf16*)dk, (__bf16*)dv, dla, (int)T, NC);
  PGN_RETURN_LAUNCH();
}
