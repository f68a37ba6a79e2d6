// The associative carrier's chunked scan, plain write rule: forward and hand-written backward on bf16 MFMA.
//
// Per (batch, head), with chunk C = 64 tokens, head dim D = 64, la_t <= 0 the per-token log-decay and, within a
// chunk, L the inclusive cumulative sum of la, dec[t,s] = exp(L_t - L_s) for s <= t (else 0), eL = exp(L),
// w = exp(L_C - L), a = exp(L_C):
//     O   = ((Q K^T) o dec) V + (Q o eL) S_c
//     S_{c+1} = a S_c + (K o w)^T V
// (the reference's `_scan_twopass`, `src/assoc.py:118-165`; its GPU form `src/assoc_kernel.py:47-70,188-202`).
//
// Forward: one workgroup per (batch, head) walks the chunks in order; eight waves compute (each owns 16 tokens of the
// chunk and 32 value columns, and holds its 16 x 32 block of the fp32 state as accumulator tiles; the state update
// is an MFMA accumulating onto a*S) while four more load and stage the next chunk into the other half of a
// double-buffered LDS. Every contraction reads its operands from LDS, so HBM sees each input once: 8 B per (t, d)
// element forward (q, k, v read, o written) plus the optional bf16 entering states.
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
#include <type_traits>

#include "mfma_tile.h"

using namespace pgn;

PGN_STAMP_UNIT(chunk)

namespace {

constexpr int C = 64;
constexpr int DK = 64;
constexpr int TILE = 64 * kPitch;  // one staged 64 x 64 tile

// Where the scan of workgroup head index bh finds its rows. Narrow heads (64 wide): scan bh is head bh, rows of 64.
// Wide heads (128 wide, plain rule): scan bh = 4 hw + 2 kh + vh runs the 64 x 64 block (key half kh, value half vh)
// of head hw's 128 x 128 state. The plain rule's state rows evolve independently (S_t = a_t S_{t-1} + k_t v_t^T row
// by row) and o_t = S_t^T q_t sums over key rows, so the block's scan is an ordinary 64 x 64 scan of q, k at columns
// 64 kh and v, dO at columns 64 vh of rows of 128, and o (dv) of head hw is the sum of its two key halves' outputs,
// dq and dk the sums over the two value halves. Such a sum has two slots, the caller's tensor (slot 0) and a
// workspace tensor of the same layout (slot 1): o and dv go to slot kh at columns 64 vh, dq and dk to slot vh at
// columns 64 kh. States (S0, S_final, dS_final, dS0) are the caller's (B, H, 128, 128) arrays: block (kh, vh) at rows
// 64 kh, columns 64 vh. The entering states `sent` stay per scan, (B, 4H, NC, 64, 64), at scan index 4 hw + 2 kh + vh.
//
// PASS (wide heads, one workgroup per scan): 0 runs all four scans of a head in one launch, the sums through the
// slots above. 1 and 2 are two launches of two scans per head: launch p = PASS - 1 runs (kh, vh) = (j, j ^ p) at
// workgroup index 2 hw + j, so within a launch no two scans write the same block of o, dq, dk or dv, and the second
// launch adds its outputs to the first's (read, add in fp32, round once), so those sums need no slot and no extra
// pass over the tensors. dla (four terms) keeps two slots there, by kh.
template <bool WIDE, int PASS = 0>
struct HeadRows {
  static_assert(PASS == 0 || WIDE, "two-launch passes are for wide heads");
  static constexpr int ld = WIDE ? 128 : 64;  // row pitch of token-major operands and of states
  static constexpr bool kAccumulate = PASS == 2;
  int hw, kh, vh, scan;
  PGN_DEVICE explicit HeadRows(int bh)
      : hw(!WIDE ? bh : PASS ? bh >> 1 : bh >> 2),
        kh(!WIDE ? 0 : PASS ? bh & 1 : (bh >> 1) & 1),
        vh(!WIDE ? 0 : PASS ? (bh & 1) ^ (PASS - 1) : bh & 1),
        scan(!WIDE ? bh : 4 * hw + 2 * kh + vh) {}
  PGN_DEVICE size_t keys(int T) const { return (size_t)hw * T * ld + 64 * kh; }  // q, k, dq, dk
  PGN_DEVICE size_t vals(int T) const { return (size_t)hw * T * ld + 64 * vh; }  // v, dO, o, dv
  PGN_DEVICE size_t state() const { return (size_t)hw * ld * ld + (size_t)64 * kh * ld + 64 * vh; }
  template <class Ptr>
  PGN_DEVICE Ptr slot(Ptr s0, Ptr s1, int which) const {
    return (WIDE && PASS == 0 && which) ? s1 : s0;
  }
};

// Forward: one workgroup of 16 waves per (batch, head), chunks in order, one barrier per chunk, three roles:
//   output waves (0-7): wave w owns a t block tb and value columns 32 jh .. 32 jh + 31 (jh = w >> 2) and holds its
//       16 x 32 slice of the fp32 state as MFMA accumulators; per chunk c it forms O^T = V^T A^T + S^T (Q o eL)^T for
//       its tokens and columns and the state update S <- a S + (K o w)^T V (an MFMA accumulating onto a S), writing
//       the next chunk's S^T tile into the other half of a double-buffered tile;
//   score waves (8-11): wave a computes the decayed scores A of chunk c + 1 for t block a, one chunk ahead, into the
//       other half of a double-buffered A tile (so the output waves never compute them, and never twice);
//   load waves (12-15): stage chunk c + 2 into a triple-buffered set of Q, K, V tiles (loaded into registers a chunk
//       earlier still), run its decay scan, issue chunk c + 3's loads and copy chunk c's entering state to `sent`.
// The t blocks of the two output-wave halves run in opposite orders, so each SIMD gets one early and one late block.
constexpr int kFwdWaves = 16;
constexpr int kFwdBuf = 3 * TILE * (int)sizeof(__bf16) + 3 * C * (int)sizeof(float);  // Q, K, V, L, eL, w

// S0 is the caller's entering state (head layout, read when there is one segment per head); Sws, when given instead,
// holds each workgroup's entering state (64 x 64 per workgroup, the segmented forward's workspace).
template <bool WIDE, int PASS>
__global__ __launch_bounds__(kFwdWaves * 64) void aspin_plain_fwd(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ S0, const float* __restrict__ Sws,
    __bf16* __restrict__ o, __bf16* __restrict__ o1, float* __restrict__ Sfin, __bf16* __restrict__ sent, int T,
    int NC, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  // input set h (the segment's chunk lc in set lc % 3): Q, K, V tiles and the L (base 2), eL, w vectors; then A
  // (t, s) and S^T (j, d) tiles for two chunks each (chunk lc in lc & 1)
  auto Qb = [&](int h) { return reinterpret_cast<__bf16*>(smem + h * kFwdBuf); };
  auto Kb = [&](int h) { return Qb(h) + TILE; };
  auto Vb = [&](int h) { return Qb(h) + 2 * TILE; };
  auto Vecb = [&](int h) { return reinterpret_cast<float*>(Qb(h) + 3 * TILE); };
  auto ATb = [&](int h) { return reinterpret_cast<__bf16*>(smem + 3 * kFwdBuf) + h * TILE; };
  auto STb = [&](int h) { return reinterpret_cast<__bf16*>(smem + 3 * kFwdBuf) + (2 + h) * TILE; };

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  // instrumented build: per wave, clocks where its role's branch starts (entries 0, 1) and at the kernel's end (2, 3),
  // then the start and end of its phase in barrier interval lc (4 + 2 lc, 5 + 2 lc)
#define FWD_STAMP(k) \
  PGN_STAMP((blockIdx.x * kFwdWaves + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC) + (k))
  // workgroup = (batch-head bh, segment sg): chunks c0 .. c0 + n - 1, entering state S0 of this workgroup
  const int nseg = (NC + P - 1) / P;
  const int bh = blockIdx.x / nseg, sg = blockIdx.x - bh * nseg;
  const int c0 = sg * P, n = min(P, NC - c0);
  using Rows = HeadRows<WIDE, PASS>;
  const Rows R(bh);
  constexpr int ld = Rows::ld;
  const size_t koff = R.keys(T), voff = R.vals(T);

  // decayed scores A[t][s] = (q_t . k_s) exp(L_t - L_s), s <= t, of t block a of chunk `cn` (input set hs) into
  // the A tile `At` (row t), zero above the diagonal block
  auto scores = [&](auto a_c, int hs, __bf16* At, int stamp) {
    constexpr int a = decltype(a_c)::value;
    if (stamp >= 0) FWD_STAMP(stamp);
    const __bf16* Qs = Qb(hs);
    const __bf16* Ks = Kb(hs);
    const float* Ls = Vecb(hs);
    const int tq = 16 * a + i;
    const bf16x8 qf0 = frag(Qs, tq, 0, g), qf1 = frag(Qs, tq, 1, g);
    bf16x8 kf[a + 1][2];
    f32x4 Lsv[a + 1];
#pragma unroll
    for (int sb = 0; sb <= a; ++sb) {
      kf[sb][0] = frag(Ks, 16 * sb + i, 0, g);
      kf[sb][1] = frag(Ks, 16 * sb + i, 1, g);
      Lsv[sb] = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
    }
    const float Lt = Ls[tq];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      f32x4 pt = zero4();
      if (sb <= a) {
        pt = pgn_mfma(kf[sb][0], qf0, pt);
        pt = pgn_mfma(kf[sb][1], qf1, pt);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 16 * sb + 4 * g + r;
          if (sb < a)  // left of the diagonal block every s < t, so the exponent is not positive: no mask
            pt[r] *= exp2_hw(Lt - Lsv[sb][r]);
          else
            pt[r] = (s <= tq) ? pt[r] * exp2_hw(fminf(Lt - Lsv[sb][r], 0.f)) : 0.f;
        }
      }
      store_T(At, 16 * a, 16 * sb, g, i, pt);
    }
    if (stamp >= 0) FWD_STAMP(stamp + 1);
  };

  if (w < 8) {
    // ================= output waves
    PGN_STAMP_CLOCKS((blockIdx.x * kFwdWaves + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC));
    const int tb = w < 4 ? 3 - w : w - 4, j0 = 32 * (w >> 2);
    // state rows 16 tb + 4g + r, columns j0 + 16 jt + i
    f32x4 S[2];
    const float* s0p = Sws ? Sws + (size_t)blockIdx.x * DK * DK : (S0 ? S0 + R.state() : nullptr);
    const int s0ld = Sws ? DK : ld;
    // every load first (an empty view when there is no entering state: zeros, no branch), then the LDS writes
    const __amdgpu_buffer_rsrc_t s0v = f32_view(s0p, DK * s0ld);
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[jt][r] = load_f32(s0v, (16 * tb + 4 * g + r) * s0ld + j0 + 16 * jt + i);
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) store_T(STb(0), j0 + 16 * jt, 16 * tb, g, i, S[jt]);
    __bf16* const obase = R.slot(o, o1, R.kh) + voff;
    // rows past T fall outside the range of a chunk's o rows: stores to them are dropped, loads read zero
    auto o_rows = [&](int c) {
      const int t0 = c * C;
      return __builtin_amdgcn_make_buffer_rsrc(obase + (size_t)t0 * ld, (short)0,
                                               min(C, T - t0) * ld * (int)sizeof(__bf16), 0x00020000);
    };
    __syncthreads();
    __syncthreads();
    auto oloop = [&](auto tb_c) {
      constexpr int TB = decltype(tb_c)::value;
      const int tq = 16 * TB + i;  // this lane's token within the chunk for t-indexed operands
      // accumulating pass: the first launch's o at this lane's outputs, loaded a chunk ahead
      i32x2 opart[2];
      auto load_opart = [&](int c) {
        const __amdgpu_buffer_rsrc_t r = o_rows(c);
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) opart[jt] = load_part4(r, (tq * ld + j0 + 16 * jt + 4 * g) * (int)sizeof(__bf16));
      };
      if constexpr (Rows::kAccumulate) load_opart(c0);
      for (int lc = 0; lc < n; ++lc) {
        const int c = c0 + lc, h3 = lc % 3, h2 = lc & 1, t0 = c * C;
        FWD_STAMP(4 + 2 * lc);  // the chunk's phase: operand reads, contractions, result stores
        const __bf16* Qs = Qb(h3);
        const __bf16* Ks = Kb(h3);
        const __bf16* Vs = Vb(h3);
        const __bf16* At = ATb(h2);
        const __bf16* ST = STb(h2);
        const float* Ls = Vecb(h3);
        const float* eLs = Ls + C;
        const float* ws = Ls + 2 * C;
        // every LDS operand of the chunk first, in the order consumed; V serves both the output (as V^T) and the
        // state update (as V)
        const bf16x8 af0 = frag(At, tq, 0, g);
        const bf16x8 af1 = TB >= 2 ? frag(At, tq, 1, g) : af0;
        const bf16x8 qf0 = frag(Qs, tq, 0, g), qf1 = frag(Qs, tq, 1, g);
        const float eLt = eLs[tq], LC = Ls[C - 1];
        bf16x8 vf[2][2], sf[2][2];
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          vf[jt][0] = frag_tr(Vs, j0 + 16 * jt, 0, g, i);
          vf[jt][1] = frag_tr(Vs, j0 + 16 * jt, 1, g, i);
          sf[jt][0] = frag(ST, j0 + 16 * jt + i, 0, g);
          sf[jt][1] = frag(ST, j0 + 16 * jt + i, 1, g);
        }
        const bf16x8 kt0 = frag_tr(Ks, 16 * TB, 0, g, i), kt1 = frag_tr(Ks, 16 * TB, 1, g, i);
        const f32x4 w00 = *reinterpret_cast<const f32x4*>(ws + 4 * g);
        const f32x4 w01 = *reinterpret_cast<const f32x4*>(ws + 16 + 4 * g);
        const f32x4 w10 = *reinterpret_cast<const f32x4*>(ws + 32 + 4 * g);
        const f32x4 w11 = *reinterpret_cast<const f32x4*>(ws + 48 + 4 * g);
        __builtin_amdgcn_sched_barrier(0);
        // O^T tiles (value block jt, t block TB) = V^T A^T + eL_t (S^T Q^T); lane holds token tq, 4 value columns,
        // so the state read's decay is one factor on the accumulator. Rows past T fall outside the store's range
        // and are dropped.
        const __amdgpu_buffer_rsrc_t o_out = o_rows(c);
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          f32x4 acc = zero4();
          acc = pgn_mfma(vf[jt][0], af0, acc);
          if (TB >= 2) acc = pgn_mfma(vf[jt][1], af1, acc);
          f32x4 qs = pgn_mfma(sf[jt][0], qf0, zero4());
          qs = pgn_mfma(sf[jt][1], qf1, qs);
          acc += eLt * qs;
          if constexpr (Rows::kAccumulate) acc += part4(opart[jt]);  // added last: the load is waited for here
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), o_out,
                                                (tq * ld + j0 + 16 * jt + 4 * g) * (int)sizeof(__bf16), 0, 0);
        }
        if constexpr (Rows::kAccumulate) load_opart(c0 + min(lc + 1, n - 1));  // unconditional: exact counter waits
        // the entering state, bf16 (d, j), from this wave's state slice
        if (sent) {
          __bf16* sc = sent + ((size_t)R.scan * NC + c) * DK * DK;
#pragma unroll
          for (int jt = 0; jt < 2; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[(16 * TB + 4 * g + r) * DK + j0 + 16 * jt + i] = (__bf16)S[jt][r];
        }
        // S <- a S + (K o w)^T V on rows 16 TB.. and this wave's columns; S^T of the next chunk into the other tile
        const float a_c = exp2_hw(LC);
        const bf16x8 kw0 = scale_frag_k(kt0, w00, w01);
        const bf16x8 kw1 = scale_frag_k(kt1, w10, w11);
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          S[jt] = S[jt] * a_c;
          S[jt] = pgn_mfma(kw0, vf[jt][0], S[jt]);
          S[jt] = pgn_mfma(kw1, vf[jt][1], S[jt]);
          store_T(STb(h2 ^ 1), j0 + 16 * jt, 16 * TB, g, i, S[jt]);
        }
        FWD_STAMP(5 + 2 * lc);
        __syncthreads();
      }
    };
    switch (tb) {  // one instantiation per t block: its block conditions are compile-time constants
      case 0: oloop(std::integral_constant<int, 0>{}); break;
      case 1: oloop(std::integral_constant<int, 1>{}); break;
      case 2: oloop(std::integral_constant<int, 2>{}); break;
      default: oloop(std::integral_constant<int, 3>{}); break;
    }
    if (Sfin) {
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) Sfin[R.state() + (16 * tb + 4 * g + r) * ld + j0 + 16 * jt + i] = S[jt][r];
    }
  } else if (w < 12) {
    PGN_STAMP_CLOCKS((blockIdx.x * kFwdWaves + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC));
    // ================= score waves: t block a, one chunk ahead. Wave 8 also runs the decay scans, two chunks ahead
    // (the load waves stage the same chunk's tiles in the same phase): L (base 2), e^L and w = exp(L_C - L).
    const bool scan = w == 8;
    auto la_of = [&](int ln) {  // the segment's chunk ln (zero past the segment or T): a load with no branch
      const int n0 = (c0 + ln) * C;
      return load_f32_lane(la + (size_t)R.hw * T + n0, ln < n ? min(C, T - n0) : 0, x.l);
    };
    auto run_scan = [&](float la_t, int h) {
      const float L = wave_prefix_sum(la_t, x.l);
      const float LC = lane_value(L, 63);
      float* vs = Vecb(h);
      vs[x.l] = L * kLog2e;
      vs[C + x.l] = __expf(L);
      vs[2 * C + x.l] = __expf(fminf(LC - L, 0.f));
    };
    auto sloop = [&](auto a_c) {
      if (scan) {
        run_scan(la_of(0), 0);
        if (n > 1) run_scan(la_of(1), 1);
      }
      __syncthreads();
      scores(a_c, 0, ATb(0), -1);
      __syncthreads();
      for (int c = 0; c < n; ++c) {
        // chunk c + 2's decays, loaded before this phase's scores and used after them: not carried around the
        // loop (a carried load result is copied at the loop's end, which waits for the load)
        const float la_t = la_of(c + 2);
        if (c + 1 < n) scores(a_c, (c + 1) % 3, ATb((c + 1) & 1), 4 + 2 * c);
        if (scan && c + 2 < n) run_scan(la_t, (c + 2) % 3);
        __syncthreads();
      }
    };
    switch (w - 8) {
      case 0: sloop(std::integral_constant<int, 0>{}); break;
      case 1: sloop(std::integral_constant<int, 1>{}); break;
      case 2: sloop(std::integral_constant<int, 2>{}); break;
      default: sloop(std::integral_constant<int, 3>{}); break;
    }
  } else {
    PGN_STAMP_CLOCKS((blockIdx.x * kFwdWaves + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC));
    // ================= load waves: thread b carries 16-byte row segments b and b + 256 of each of Q, K and V.
    // Two register sets alternate, so a chunk's loads are issued two chunks before it is staged.
    const int b = tid & 255;
    struct Regs {
      bf16x8 q0, q1, k0, k1, v0, v1;
    };
    Regs ra, rb;
    auto load = [&](Regs& r, int ln) {  // the segment's chunk ln
      const int n0 = (c0 + ln) * C, nr = min(C, T - n0);
      r.q0 = load_seg(q + koff + (size_t)n0 * ld, nr, b, ld);
      r.q1 = load_seg(q + koff + (size_t)n0 * ld, nr, b + 256, ld);
      r.k0 = load_seg(k + koff + (size_t)n0 * ld, nr, b, ld);
      r.k1 = load_seg(k + koff + (size_t)n0 * ld, nr, b + 256, ld);
      r.v0 = load_seg(v + voff + (size_t)n0 * ld, nr, b, ld);
      r.v1 = load_seg(v + voff + (size_t)n0 * ld, nr, b + 256, ld);
    };
    auto stage = [&](const Regs& r, int h) {
      put_seg(Qb(h), r.q0, b);
      put_seg(Qb(h), r.q1, b + 256);
      put_seg(Kb(h), r.k0, b);
      put_seg(Kb(h), r.k1, b + 256);
      put_seg(Vb(h), r.v0, b);
      put_seg(Vb(h), r.v1, b + 256);
    };
    // Every load is unconditional (chunk indices clamped to the segment's last chunk; the extra loads re-read it,
    // unused), so the compiler counts the loads in flight exactly and the wait before staging a set covers that set
    // only, not the other one issued a chunk later.
    load(ra, 0);
    load(rb, min(1, n - 1));  // both chunks' loads in flight together
    stage(ra, 0);
    stage(rb, 1);  // unconditional (with one chunk, a copy of it into a set nothing reads): the loads stay issued above
    load(ra, min(2, n - 1));
    load(rb, min(3, n - 1));
    __syncthreads();
    __syncthreads();
    // chunk c: stage chunk c + 2 from the set loaded two chunks ago, then reload that set with chunk c + 4
    auto phase = [&](Regs& r, int c) {
      if (c + 2 < n) stage(r, (c + 2) % 3);
      load(r, min(c + 4, n - 1));
      __syncthreads();
    };
    for (int c = 0; c < n; c += 2) {
      phase(ra, c);
      if (c + 1 < n) phase(rb, c + 1);
    }
  }
  PGN_STAMP_CLOCKS((blockIdx.x * kFwdWaves + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC) + 2);
#undef FWD_STAMP
}

// Forward at 128 keys, native: one workgroup of 16 waves per (batch-head hw, value half vh) holds the 128 x 64 state
// S[:, 64 vh ..] (both key halves) and writes its 64 columns of o whole, o = ((Q K^T) o dec) V + (Q o eL) S with
// every contraction over keys running over all 128, so no output is a sum of two scans' outputs (the wide mode's four
// 64 x 64 scans per head read q, k and v twice and o once more to add their halves). Q, K and V of a chunk take 5
// tiles (Q and K as two 64-column halves), so the input sets are double-buffered and each chunk has two barriers:
//   phase 1: output waves 0-7 (t block tb, value columns j0 .. j0 + 31, both key halves' 16 x 32 state slices as
//       accumulators) form eL_t (S^T Q^T) for their tokens from the chunk's S^T tiles, write the entering state to
//       `sent` and update S <- a S + (K o w)^T V in registers; score waves 8-11 form the chunk's decayed scores A (t
//       block a, 128-deep) into the A tile, wave 8 also the next chunk's decay scan; load waves 12-15 stage the next
//       chunk into the other input set and issue the loads of the one after;
//   phase 2 (after the A barrier): output waves add V^T A^T and store o, then write the next chunk's S^T tiles (every
//       read of the current ones was before the barrier).
// `sent` keeps the wide mode's per-scan layout, (B, 4H, NC, 64, 64) at scan 4 hw + 2 kh + vh, so the wide backward
// reads it unchanged. Unsegmented only (one workgroup walks all chunks of its scan).
constexpr int kN128Buf = 5 * TILE * (int)sizeof(__bf16) + 3 * C * (int)sizeof(float);  // Q0, Q1, K0, K1, V, vectors
constexpr size_t kN128Smem = 2 * (size_t)kN128Buf + 3 * TILE * sizeof(__bf16);       // two sets, A, S^T x 2

__global__ __launch_bounds__(kFwdWaves * 64) void aspin_plain_fwd128(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ S0, __bf16* __restrict__ o, float* __restrict__ Sfin,
    __bf16* __restrict__ sent, int T, int NC, int nbh) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int ld = 128;
  auto Qb = [&](int h, int kh) { return reinterpret_cast<__bf16*>(smem + h * kN128Buf) + kh * TILE; };
  auto Kb = [&](int h, int kh) { return Qb(h, 0) + (2 + kh) * TILE; };
  auto Vb = [&](int h) { return Qb(h, 0) + 4 * TILE; };
  auto Vecb = [&](int h) { return reinterpret_cast<float*>(Qb(h, 0) + 5 * TILE); };
  __bf16* const At = reinterpret_cast<__bf16*>(smem + 2 * kN128Buf);
  auto STb = [&](int kh) { return At + (1 + kh) * TILE; };

  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  // the two value halves of a head are workgroups 8 apart, so they run on one XCD (workgroup i goes to XCD i mod 8)
  // and q, k come from HBM once into its L2 (step 0.1104-0.1117 -> 0.1088-0.1092 ms against adjacent indices, A/B
  // on one box); the grid is padded to whole sets of 16
  const int bi = blockIdx.x, hw = (bi >> 4) * 8 + (bi & 7), vh = (bi >> 3) & 1;
  if (hw >= nbh) return;  // padding (uniform over the workgroup, before any barrier)
  const size_t koff = (size_t)hw * T * ld, voff = koff + 64 * vh;
  const size_t soff = (size_t)hw * ld * ld + 64 * vh;  // the (B, H, 128, 128) state's block: rows 64 kh .., columns
                                                       // 64 vh ..

  if (w < 8) {
    // ================= output waves
    const int tb = w < 4 ? 3 - w : w - 4, j0 = 32 * (w >> 2);
    f32x4 S[2][2];  // [key half][value block]: rows 64 kh + 16 tb + 4 g + r, columns j0 + 16 jt + i
    const __amdgpu_buffer_rsrc_t s0v = f32_view(S0 ? S0 + soff : nullptr, ld * ld);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[kh][jt][r] = load_f32(s0v, (64 * kh + 16 * tb + 4 * g + r) * ld + j0 + 16 * jt + i);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) store_T(STb(kh), j0 + 16 * jt, 16 * tb, g, i, S[kh][jt]);
    __bf16* const obase = o + voff;
    auto o_rows = [&](int c) {
      const int t0 = c * C;
      return __builtin_amdgcn_make_buffer_rsrc(obase + (size_t)t0 * ld, (short)0,
                                               min(C, T - t0) * ld * (int)sizeof(__bf16), 0x00020000);
    };
    __syncthreads();
    auto oloop = [&](auto tb_c) {
      constexpr int TB = decltype(tb_c)::value;
      const int tq = 16 * TB + i;
      for (int c = 0; c < NC; ++c) {
        const int h = c & 1;
        const float* Ls = Vecb(h);
        const float* eLs = Ls + C;
        const float* ws = Ls + 2 * C;
        // operands in two groups (all of them at once would not fit the registers of 16 waves): the state read's
        // Q and S^T fragments with V's, then K's and the chunk weights for the update
        bf16x8 qf[2][2], sf[2][2][2], vf[2][2], kt[2][2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            qf[kh][m] = frag(Qb(h, kh), tq, m, g);
#pragma unroll
            for (int jt = 0; jt < 2; ++jt) sf[kh][jt][m] = frag(STb(kh), j0 + 16 * jt + i, m, g);
          }
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
          for (int m = 0; m < 2; ++m) vf[jt][m] = frag_tr(Vb(h), j0 + 16 * jt, m, g, i);
        const float eLt = eLs[tq], LC = Ls[C - 1];
        // the state read eL_t (S^T Q^T) over all 128 keys, before S moves on (no scheduling barrier ahead of it: the
        // compiler interleaving the reads with the products measured 1-2 us faster a step)
        f32x4 acc[2];
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          f32x4 qs = zero4();
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            qs = pgn_mfma(sf[kh][jt][0], qf[kh][0], qs);
            qs = pgn_mfma(sf[kh][jt][1], qf[kh][1], qs);
          }
          acc[jt] = eLt * qs;
        }
        // the entering states, bf16 (d, j) per key half, through range-checked buffers (no buffer: an empty range,
        // the stores dropped), each 16 x 16 block transposed within lane quads so a lane stores 4 columns of one row
        // in 8 bytes (sixteen 2-byte stores a lane took the step 0.1191 -> 0.1100 ms more, A/B on one box)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
              sent ? sent + ((size_t)(4 * hw + 2 * kh + vh) * NC + c) * DK * DK : nullptr, (short)0,
              sent ? DK * DK * (int)sizeof(__bf16) : 0, 0x00020000);
#pragma unroll
          for (int jt = 0; jt < 2; ++jt)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, quad_rows(S[kh][jt], i)), sr,
                                                  ((16 * TB + 4 * g + (i & 3)) * DK + j0 + 16 * jt + 4 * (i >> 2)) *
                                                      (int)sizeof(__bf16), 0, 0);
        }
        // S <- a S + (K o w)^T V, both key halves
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int m = 0; m < 2; ++m) kt[kh][m] = frag_tr(Kb(h, kh), 16 * TB, m, g, i);
        const f32x4 w00 = *reinterpret_cast<const f32x4*>(ws + 4 * g);
        const f32x4 w01 = *reinterpret_cast<const f32x4*>(ws + 16 + 4 * g);
        const f32x4 w10 = *reinterpret_cast<const f32x4*>(ws + 32 + 4 * g);
        const f32x4 w11 = *reinterpret_cast<const f32x4*>(ws + 48 + 4 * g);
        const float a_c = exp2_hw(LC);
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const bf16x8 kw0 = scale_frag_k(kt[kh][0], w00, w01);
          const bf16x8 kw1 = scale_frag_k(kt[kh][1], w10, w11);
#pragma unroll
          for (int jt = 0; jt < 2; ++jt) {
            S[kh][jt] = S[kh][jt] * a_c;
            S[kh][jt] = pgn_mfma(kw0, vf[jt][0], S[kh][jt]);
            S[kh][jt] = pgn_mfma(kw1, vf[jt][1], S[kh][jt]);
          }
        }
        __syncthreads();  // A complete; every read of this chunk's S^T tiles done
        const bf16x8 af0 = frag(At, tq, 0, g);
        const bf16x8 af1 = TB >= 2 ? frag(At, tq, 1, g) : af0;
        const __amdgpu_buffer_rsrc_t o_out = o_rows(c);
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          acc[jt] = pgn_mfma(vf[jt][0], af0, acc[jt]);
          if (TB >= 2) acc[jt] = pgn_mfma(vf[jt][1], af1, acc[jt]);
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc[jt])), o_out,
                                                (tq * ld + j0 + 16 * jt + 4 * g) * (int)sizeof(__bf16), 0, 0);
        }
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int jt = 0; jt < 2; ++jt) store_T(STb(kh), j0 + 16 * jt, 16 * TB, g, i, S[kh][jt]);
        __syncthreads();  // end of the chunk
      }
    };
    switch (tb) {
      case 0: oloop(std::integral_constant<int, 0>{}); break;
      case 1: oloop(std::integral_constant<int, 1>{}); break;
      case 2: oloop(std::integral_constant<int, 2>{}); break;
      default: oloop(std::integral_constant<int, 3>{}); break;
    }
    if (Sfin) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            Sfin[soff + (size_t)(64 * kh + 16 * tb + 4 * g + r) * ld + j0 + 16 * jt + i] = S[kh][jt][r];
    }
  } else if (w < 12) {
    // ================= score waves: t block a of the current chunk; wave 8 also the next chunk's decay scan
    const bool scan = w == 8;
    auto la_of = [&](int c) {  // chunk c's log-decays (zero past T): a load with no branch
      const int n0 = c * C;
      return load_f32_lane(la + (size_t)hw * T + n0, c < NC ? min(C, T - n0) : 0, x.l);
    };
    auto run_scan = [&](float la_t, int h) {
      const float L = wave_prefix_sum(la_t, x.l);
      const float LC = lane_value(L, 63);
      float* vs = Vecb(h);
      vs[x.l] = L * kLog2e;
      vs[C + x.l] = __expf(L);
      vs[2 * C + x.l] = __expf(fminf(LC - L, 0.f));
    };
    auto sloop = [&](auto a_c) {
      constexpr int a = decltype(a_c)::value;
      if (scan) run_scan(la_of(0), 0);
      __syncthreads();
      for (int c = 0; c < NC; ++c) {
        const int h = c & 1;
        const float la_t = la_of(c + 1);
        const float* Ls = Vecb(h);
        const int tq = 16 * a + i;
        bf16x8 qf[2][2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int m = 0; m < 2; ++m) qf[kh][m] = frag(Qb(h, kh), tq, m, g);
        const float Lt = Ls[tq];
        // K fragments of s blocks read two at a time (all four blocks' would not fit the registers)
        bf16x8 kf[2][2][2];
        f32x4 Lsv[2];
        auto read_k = [&](int sb) {
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int m = 0; m < 2; ++m) kf[sb & 1][kh][m] = frag(Kb(h, kh), 16 * sb + i, m, g);
          Lsv[sb & 1] = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
        };
        read_k(0);
        if (a >= 1) read_k(1);
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
          f32x4 pt = zero4();
          if (sb <= a) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
              pt = pgn_mfma(kf[sb & 1][kh][0], qf[kh][0], pt);
              pt = pgn_mfma(kf[sb & 1][kh][1], qf[kh][1], pt);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int s = 16 * sb + 4 * g + r;
              if (sb < a)
                pt[r] *= exp2_hw(Lt - Lsv[sb & 1][r]);
              else
                pt[r] = (s <= tq) ? pt[r] * exp2_hw(fminf(Lt - Lsv[sb & 1][r], 0.f)) : 0.f;
            }
            if (sb + 2 <= a) read_k(sb + 2);  // into the buffers block sb has finished with (K and decays)
          }
          store_T(At, 16 * a, 16 * sb, g, i, pt);
        }
        if (scan && c + 1 < NC) run_scan(la_t, h ^ 1);
        __syncthreads();  // A complete
        __syncthreads();  // end of the chunk
      }
    };
    switch (w - 8) {
      case 0: sloop(std::integral_constant<int, 0>{}); break;
      case 1: sloop(std::integral_constant<int, 1>{}); break;
      case 2: sloop(std::integral_constant<int, 2>{}); break;
      default: sloop(std::integral_constant<int, 3>{}); break;
    }
  } else {
    // ================= load waves: thread b carries 16-byte segments b and b + 256 of each of Q0, Q1, K0, K1, V;
    // two register sets alternate, so a chunk's loads are issued a chunk before it is staged
    const int b = tid & 255;
    struct Regs {
      bf16x8 q[2][2], k[2][2], v[2];
    };
    Regs ra, rb;
    auto load = [&](Regs& r, int c) {
      const int n0 = c * C, nr = min(C, T - n0);
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          r.q[kh][u] = load_seg(q + koff + (size_t)n0 * ld + 64 * kh, nr, b + 256 * u, ld);
          r.k[kh][u] = load_seg(k + koff + (size_t)n0 * ld + 64 * kh, nr, b + 256 * u, ld);
        }
#pragma unroll
      for (int u = 0; u < 2; ++u) r.v[u] = load_seg(v + voff + (size_t)n0 * ld, nr, b + 256 * u, ld);
    };
    auto stage = [&](const Regs& r, int h) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          put_seg(Qb(h, kh), r.q[kh][u], b + 256 * u);
          put_seg(Kb(h, kh), r.k[kh][u], b + 256 * u);
        }
#pragma unroll
      for (int u = 0; u < 2; ++u) put_seg(Vb(h), r.v[u], b + 256 * u);
    };
    // every load unconditional (chunk indices clamped to the last chunk), so the counter waits stay exact
    load(ra, 0);
    load(rb, min(1, NC - 1));
    stage(ra, 0);
    load(ra, min(2, NC - 1));
    __syncthreads();
    // chunk c: stage chunk c + 1 from the set loaded a chunk ago, then reload that set with chunk c + 3
    auto phase = [&](Regs& r, int c) {
      if (c + 1 < NC) stage(r, (c + 1) & 1);
      load(r, min(c + 3, NC - 1));
      __syncthreads();  // A complete
      __syncthreads();  // end of the chunk
    };
    for (int c = 0; c < NC; c += 2) {
      phase(rb, c);
      if (c + 1 < NC) phase(ra, c + 1);
    }
  }
}

// Segment-parallel forward, for few heads over long sequences: the chunks of each head are split into segments of
// P chunks that run as separate workgroups of the forward above, once each segment's entering state is known. The
// state a segment leaves is an affine function of the one it enters, S_out = e^{l} S_in + E, with l the segment's
// total log-decay and E = sum_t exp(L_end - L_t) k_t v_t^T over its tokens (L the cumulative sum of la from the
// segment's start, so the weight is the decay from token t to the segment's end). Windowed carrying (positions
// restarting every `window` tokens, the state rebased between windows as successive forward calls do) adds a
// rotation of the key rows at window boundaries: S_in(next) = R(-window theta) S_out.

// The backward splits the same way in reverse. The gradient on the state leaving the chunk before a segment is
// e^{l} G + F, with G the gradient on the state the segment leaves and F = sum_t exp(L_t) q_t dO_t^T (the decay
// from the segment's start to t, inclusive), so per-segment sums of q and dO, a reverse prefix over segments, and
// the backward kernel per segment started from its G give every chunk's state gradient, hence dq, dk, dv and dla.

// Segment sums: per workgroup (batch-head, segment) sum_t w_t x_t y_t^T and l. TO_END (forward): x = k, y = v and
// w_t = exp(L_end - L_t), the segment's chunks walked from its end so each chunk's decay to the end is a running
// sum. Otherwise (backward): x = q, y = dO and w_t = exp(L_t), walked from the start. Four waves; wave w owns rows
// 16 w.. of the sum as MFMA accumulators; x and y are staged through double-buffered LDS, loaded a chunk ahead.
constexpr int kSumBuf = 2 * TILE * (int)sizeof(__bf16) + C * (int)sizeof(float);  // x, y, w

template <bool TO_END, bool WIDE>
__global__ __launch_bounds__(256) void aspin_plain_segsum(const __bf16* __restrict__ k, const __bf16* __restrict__ v,
                                                          const float* __restrict__ la, float* __restrict__ E,
                                                          float* __restrict__ lseg, int T, int NC, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  auto Kb = [&](int h) { return reinterpret_cast<__bf16*>(smem + h * kSumBuf); };
  auto Vb = [&](int h) { return Kb(h) + TILE; };
  auto Wb = [&](int h) { return reinterpret_cast<float*>(Kb(h) + 2 * TILE); };
  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i;
  const int b = threadIdx.x & 255;
  const int nseg = (NC + P - 1) / P;
  const int bh = blockIdx.x / nseg, sg = blockIdx.x - bh * nseg;
  const int c0 = sg * P, n = min(P, NC - c0);
  // x (k, or q) at the scan's key columns, y (v, or dO) at its value columns
  const HeadRows<WIDE> R(bh);
  constexpr int ld = HeadRows<WIDE>::ld;
  const size_t koff = R.keys(T), voff = R.vals(T);
  bf16x8 k0, k1, v0, v1;
  float lat = 0.f;
  auto load = [&](int ln) {  // the segment's chunk ln; rows past T read as zero
    const int n0 = (c0 + ln) * C, nr = min(C, T - n0);
    k0 = load_seg(k + koff + (size_t)n0 * ld, nr, b, ld);
    k1 = load_seg(k + koff + (size_t)n0 * ld, nr, b + 256, ld);
    v0 = load_seg(v + voff + (size_t)n0 * ld, nr, b, ld);
    v1 = load_seg(v + voff + (size_t)n0 * ld, nr, b + 256, ld);
    lat = load_f32_lane(la + (size_t)R.hw * T + n0, nr, x.l);  // every wave (wave 0 uses it): no branch
  };
  // wave 0: total log-decay of the segment's chunks already staged (after the next one when walking to the end,
  // before it when walking from the start)
  float run = 0.f;
  auto stage = [&](int h) {
    put_seg(Kb(h), k0, b);
    put_seg(Kb(h), k1, b + 256);
    put_seg(Vb(h), v0, b);
    put_seg(Vb(h), v1, b + 256);
    if (w == 0) {
      const float L = wave_prefix_sum(lat, x.l);
      const float tot = lane_value(L, 63);
      Wb(h)[x.l] = TO_END ? __expf(fminf(run + tot - L, 0.f)) : __expf(fminf(run + L, 0.f));
      run += tot;
    }
  };
  // the segment's chunk walked at step it
  auto chunk_at = [&](int it) { return TO_END ? n - 1 - it : it; };
  f32x4 acc[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) acc[jb] = zero4();
  load(chunk_at(0));
  stage(0);
  load(chunk_at(min(1, n - 1)));  // unconditional (clamped; an extra load re-reads a chunk, unused)
  __syncthreads();
  for (int it = 0; it < n; ++it) {
    const int h = it & 1;
    const __bf16* Ks = Kb(h);
    const __bf16* Vs = Vb(h);
    const float* ws = Wb(h);
    const bf16x8 kt0 = frag_tr(Ks, 16 * w, 0, g, i), kt1 = frag_tr(Ks, 16 * w, 1, g, i);
    const f32x4 w00 = *reinterpret_cast<const f32x4*>(ws + 4 * g);
    const f32x4 w01 = *reinterpret_cast<const f32x4*>(ws + 16 + 4 * g);
    const f32x4 w10 = *reinterpret_cast<const f32x4*>(ws + 32 + 4 * g);
    const f32x4 w11 = *reinterpret_cast<const f32x4*>(ws + 48 + 4 * g);
    bf16x8 vf[4][2];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      vf[jb][0] = frag_tr(Vs, 16 * jb, 0, g, i);
      vf[jb][1] = frag_tr(Vs, 16 * jb, 1, g, i);
    }
    const bf16x8 kw0 = scale_frag_k(kt0, w00, w01);
    const bf16x8 kw1 = scale_frag_k(kt1, w10, w11);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      acc[jb] = pgn_mfma(kw0, vf[jb][0], acc[jb]);
      acc[jb] = pgn_mfma(kw1, vf[jb][1], acc[jb]);
    }
    if (it + 1 < n) stage(h ^ 1);
    load(chunk_at(min(it + 2, n - 1)));
    __syncthreads();
  }
  float* e = E + (size_t)blockIdx.x * DK * DK;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int r = 0; r < 4; ++r) e[(16 * w + 4 * g + r) * DK + 16 * jb + i] = acc[jb][r];
  if (w == 0 && x.l == 0) lseg[blockIdx.x] = run;
}

// Segment prefix: the state entering each segment, written over that segment's E, and the final state:
// S_in(0) = S0 (zero if NULL); S_out(g) = e^{l_g} S_in(g) + E_g; S_in(g + 1) = S_out(g), rotated at window boundaries
// (every `wsegs` segments, when theta is given) by -shift theta[h, i] on key rows (2i, 2i + 1); S_final = S_out(last).
// REVERSE (backward): the same recurrence over the segments from the last to the first, S0 the gradient on the final
// state, writing over each F the gradient on the state the segment leaves and, as "final", the gradient on the
// initial state (no rotation). Thread = (value column j, key pair ip): 8 workgroups of 256 per head. Each batch of
// 16 segments is loaded before the recurrence runs over it, so the loads are not serialised behind it. S0 and Sfin
// are in the caller's head layout (HeadRows), E per (scan, segment) 64 x 64. Windows (theta) are for narrow heads.
template <bool REVERSE, bool WIDE>
__global__ __launch_bounds__(256) void aspin_plain_segprefix(const float* __restrict__ S0,
                                                             const float* __restrict__ theta, float shift, int wsegs,
                                                             float* __restrict__ E, const float* __restrict__ lseg,
                                                             float* __restrict__ Sfin, int H, int nseg) {
  const int bh = blockIdx.x >> 3, h = bh % H;
  const int j = threadIdx.x & 63, ip = 4 * (blockIdx.x & 7) + (threadIdx.x >> 6);
  const int e0 = (2 * ip) * DK + j, e1 = e0 + DK;
  const HeadRows<WIDE> R(bh);
  constexpr int ld = HeadRows<WIDE>::ld;
  const size_t u0 = R.state() + (2 * ip) * ld + j, u1 = u0 + ld;
  float s0 = S0 ? S0[u0] : 0.f, s1 = S0 ? S0[u1] : 0.f;
  float sn = 0.f, cs = 1.f;
  if (theta) sincosf(-shift * theta[h * (DK / 2) + ip], &sn, &cs);
  constexpr int kBatch = 16;
  for (int g0 = 0; g0 < nseg; g0 += kBatch) {
    float x0[kBatch], x1[kBatch], a[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (g0 + u < nseg) {
        const int gi = REVERSE ? nseg - 1 - (g0 + u) : g0 + u;
        const size_t off = ((size_t)bh * nseg + gi) * DK * DK;
        x0[u] = E[off + e0];
        x1[u] = E[off + e1];
        a[u] = lseg[(size_t)bh * nseg + gi];
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int gg = g0 + u;
      if (gg < nseg) {
        const size_t off = ((size_t)bh * nseg + (REVERSE ? nseg - 1 - gg : gg)) * DK * DK;
        E[off + e0] = s0;
        E[off + e1] = s1;
        const float dec = __expf(a[u]);
        const float t0 = dec * s0 + x0[u], t1 = dec * s1 + x1[u];
        if (!REVERSE && theta && (gg + 1) % wsegs == 0) {
          s0 = t0 * cs - t1 * sn;
          s1 = t0 * sn + t1 * cs;
        } else {
          s0 = t0;
          s1 = t1;
        }
        if (Sfin && gg == nseg - 1) {
          Sfin[u0] = t0;
          Sfin[u1] = t1;
        }
      }
    }
  }
}

// Backward: 8 waves per (batch, head), chunks in reverse, one barrier per chunk. Waves 4-7 (group K) own s block
// wl = w & 3 and compute dV, dK, the column sums of dA o A and k_s.(dS v_s); they read dS from LDS and do nothing
// else. Waves 0-3 (group D) own t block wl and compute dQ, the row sums of dA o A, q_t.(S_c dO_t), then carry dS:
// wave wl holds rows 16 wl.. of dS in fp32 registers, forms <S_c, dS> and dS <- a dS + (Q o eL)^T dO for them and
// writes the result (bf16, transposed) into the other half of a double-buffered dS^T tile, which group K reads in
// the next chunk. Group D also stages the next chunk's tiles into the other half of double-buffered input tiles
// (loaded a chunk earlier still), and its wave 0 runs the per-chunk scans: L for the next chunk and, from the other
// set of double-buffered per-chunk vectors, the previous (later) chunk's dla. Operands contracted over a tile's row
// index are read with the LDS transpose read, so each input is staged once, untransposed.
// one set of per-chunk vectors: L, eL, w, rowM, colM, qz, dwv (C each) and the per-lane partial sums of <S_c, dS>
// (4 waves x 64 lanes)
constexpr int kVec = 11 * C;

// dla of one chunk from its vector set: dL_t = rowM_t - colM_t + eL_t qz_t - w_t dwv_t, the chunk's last token adds
// sum_s w_s dwv_s + a <S_c, dS>, and dla is the reverse inclusive cumulative sum of dL (plus `part`, lane t's partial
// from an earlier launch, when accumulating). One wave, lane = t.
template <bool ATOMIC = false>
PGN_DEVICE void plain_dla(const float* vs, int lane, __amdgpu_buffer_rsrc_t out, float part = 0.f) {
  const float* Ls = vs;
  const float* eLs = vs + C;
  const float* ws = vs + 2 * C;
  const float* rowM = vs + 3 * C;
  const float* colM = vs + 4 * C;
  const float* qz = vs + 5 * C;
  const float* dwv = vs + 6 * C;
  const float* sdot = vs + 7 * C;
  const int t = lane;
  const float wd = ws[t] * dwv[t];
  float dL = rowM[t] - colM[t] + eLs[t] * qz[t] - wd;
  const float wdw = wave_sum(wd);
  const float sd = wave_sum((sdot[t] + sdot[C + t]) + (sdot[2 * C + t] + sdot[3 * C + t]));
  if (t == C - 1) dL += wdw + exp2_hw(Ls[C - 1]) * sd;
  dL = wave_suffix_sum(dL, t) + part;
  if constexpr (ATOMIC)
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(dL, out, 4 * t, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, dL), out, 4 * t, 0, 0);
}

// L (inclusive cumulative sum of the chunk's la, lane = t, stored in base 2: L log2 e), e^L and w = exp(L_C - L) into a
// vector set. One wave.
PGN_DEVICE void plain_scan(float la_t, int lane, float* vs) {
  const float L = wave_prefix_sum(la_t, lane);
  const float LC = lane_value(L, 63);
  vs[lane] = L * kLog2e;
  vs[C + lane] = __expf(L);
  vs[2 * C + lane] = __expf(fminf(LC - L, 0.f));
}

constexpr int kBwdStage = 5 * TILE;  // Q, K, V, dO, S_c

// dSfin is the caller's gradient on the final state (head layout, read when there is one segment per head); dSws,
// when given instead, holds the gradient on the state each workgroup's segment leaves (64 x 64 per workgroup, the
// segmented backward's workspace). Wide heads: dla of scan 4 hw + s goes to dla (s = 0) or to dla1 slot s - 1.
template <bool WIDE, int PASS>
__global__ __launch_bounds__(512) void aspin_plain_bwd(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ la, const __bf16* __restrict__ sent, const __bf16* __restrict__ dO,
    const float* __restrict__ dSfin, const float* __restrict__ dSws, __bf16* __restrict__ dq,
    __bf16* __restrict__ dq1, __bf16* __restrict__ dk, __bf16* __restrict__ dk1, __bf16* __restrict__ dv,
    __bf16* __restrict__ dv1, float* __restrict__ dla, float* __restrict__ dla1, float* __restrict__ dS0, int T,
    int NC, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* stg = reinterpret_cast<__bf16*>(smem);    // two sets of staged tiles, chunk c uses set c & 1
  __bf16* dSTb = stg + 2 * kBwdStage;                // two dS^T (j, d) tiles: dS leaving chunk c in tile c & 1
  float* vec = reinterpret_cast<float*>(dSTb + 2 * TILE);  // two vector sets, chunk c uses set c & 1

  const WaveIdx x = wave_idx();
  const int w = x.w, wl = w & 3, g = x.g, i = x.i, tid = threadIdx.x;
  // instrumented build: per wave, clocks where its group's branch starts (entries 0, 1) and at the kernel's end (2, 3),
  // then the start and end of its phase for chunk cc (4 + 2 cc, 5 + 2 cc)
#define BWD_STAMP(k) PGN_STAMP((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC) + (k))
  // workgroup = (batch-head bh, segment sg): chunks c0 .. cl, walked from cl down; dSfin indexed per workgroup
  const int nseg = (NC + P - 1) / P;
  const int bh = blockIdx.x / nseg, sg = blockIdx.x - bh * nseg;
  const int c0 = sg * P, cl = min(c0 + P, NC) - 1;
  using Rows = HeadRows<WIDE, PASS>;
  const Rows R(bh);
  constexpr int ld = Rows::ld;
  const size_t koff = R.keys(T), voff = R.vals(T);
  // dla slots: narrow heads one; wide heads in one launch four (slot s = bh & 3: dla, then dla1 s - 1 of nwide heads
  // each); in two launches, the first writes slot kh (dla, dla1) and the second adds its terms into dla with fp32
  // atomics, the key-half-1 scan with the first launch's dla1 (so no pass sums the slots; two adds an element, in
  // arrival order)
  float* dlar = dla + (size_t)R.hw * T;
  const float* dlapr = nullptr;  // where the second launch's partial comes from (none: a zero-size range)
  if constexpr (WIDE && PASS == 0) {
    const int nwide = (int)(gridDim.x / nseg) >> 2;  // wide heads in the launch
    if (bh & 3) dlar = dla1 + ((size_t)((bh & 3) - 1) * nwide + R.hw) * T;
  } else if constexpr (WIDE && PASS == 1) {
    if (R.kh) dlar = dla1 + (size_t)R.hw * T;
  } else if constexpr (WIDE) {
    if (R.kh) dlapr = dla1 + (size_t)R.hw * T;
  }

  // The two groups run separate loops (the branch is on a wave-uniform value) that meet at the same barriers: each
  // loop's registers and memory-counter waits are then its own.
  if (w >= 4) {
    PGN_STAMP_CLOCKS((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC));
    // ================= group K: s = me, d block wl. Waves 6 and 7, whose share of the contractions is the
    // smallest, also stage the Q and K tiles: thread b2 carries 16-byte row segments b2 + 128 n (n = 0..3) of each.
    const bool kstage = wl >= 2;
    const int b2 = tid & 127;
    bf16x8 sq[4], sk[4];
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        sq[n] = load_seg(q + koff + (size_t)n0 * ld, nr, b2 + 128 * n, ld);
        sk[n] = load_seg(k + koff + (size_t)n0 * ld, nr, b2 + 128 * n, ld);
      }
    };
    auto stage = [&](int hh) {
      __bf16* Qs = stg + hh * kBwdStage;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        put_seg(Qs, sq[n], b2 + 128 * n);
        put_seg(Qs + TILE, sk[n], b2 + 128 * n);
      }
    };
    // this chunk's rows of dV and dK: stores to rows past T fall outside the range and are dropped (loads read zero)
    auto out_rows = [&](__bf16* base, int cc) {
      const int t0 = cc * C;
      return __builtin_amdgcn_make_buffer_rsrc(base + (size_t)t0 * ld, (short)0,
                                               min(C, T - t0) * ld * (int)sizeof(__bf16), 0x00020000);
    };
    __bf16* const dv_base = R.slot(dv, dv1, R.kh) + voff;
    __bf16* const dk_base = R.slot(dk, dk1, R.vh) + koff;
    // accumulating pass: the first launch's dV and dK at this lane's outputs (s = 16 wl + i), loaded a chunk ahead.
    // Issued in the order the loop issues them, before the next chunk's staging loads, so that the loop's memory
    // counter waits for them stay exact on its first iteration too.
    const int me_k = 16 * wl + i;
    i32x2 dvp[4], dkp[4];
    auto load_dvp = [&](int cc) {
      const __amdgpu_buffer_rsrc_t r = out_rows(dv_base, cc);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) dvp[jt] = load_part4(r, (me_k * ld + 16 * jt + 4 * g) * (int)sizeof(__bf16));
    };
    auto load_dkp = [&](int cc) {
      const __amdgpu_buffer_rsrc_t r = out_rows(dk_base, cc);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) dkp[dt] = load_part4(r, (me_k * ld + 16 * dt + 4 * g) * (int)sizeof(__bf16));
    };
    if (kstage) {
      load(cl);
      stage(cl & 1);
    }
    if constexpr (Rows::kAccumulate) {
      load_dvp(cl);
      load_dkp(cl);
    }
    __syncthreads();
    auto kloop = [&](auto wl_c) {
      constexpr int WL = decltype(wl_c)::value;
      const int me = 16 * WL + i;
      for (int cc = cl; cc >= c0; --cc) {
        BWD_STAMP(4 + 2 * cc);  // the chunk's phase: operand reads, contractions, result stores
        const int t0 = cc * C, h = cc & 1;
        const __bf16* Qs = stg + h * kBwdStage;
        const __bf16* Ks = Qs + TILE;
        const __bf16* Vs = Qs + 2 * TILE;
        const __bf16* Os = Qs + 3 * TILE;
        const __bf16* dST = dSTb + h * TILE;
        float* vs = vec + h * kVec;
        const float* Ls = vs;
        const float* ws = vs + 2 * C;
        float* colM = vs + 4 * C;  // column sums of dA o A
        float* dwv = vs + 6 * C;   // k_s . (dS v_s)
        const __amdgpu_buffer_rsrc_t dv_out = out_rows(dv_base, cc);
        const __amdgpu_buffer_rsrc_t dk_out = out_rows(dk_base, cc);
        const int cn = max(cc - 1, c0);  // the next chunk walked (unconditional loads: exact counter waits)
        // the next chunk's Q and K, staged after this chunk's phase: loaded and staged within one iteration, so no
        // loaded register is carried around the loop (a carried one is copied at the loop's end, which waits for
        // the load)
        if constexpr (WL >= 2) load(cn);
        const bf16x8 kf0 = frag(Ks, me, 0, g), kf1 = frag(Ks, me, 1, g);
        const bf16x8 vf0 = frag(Vs, me, 0, g), vf1 = frag(Vs, me, 1, g);
        const float Ls_s = Ls[me], w_s = ws[me];
        // The chunk's work as a sequence of steps: the P / dA blocks tb = WL..3, the four dV^T tiles, the four dK^T
        // tiles. Each step's LDS operands are read one step ahead (behind a scheduling barrier), so the reads
        // overlap the MFMAs instead of each MFMA waiting on a read issued just before it.
        constexpr int NA = 4 - WL, NS = NA + 8;
        StepFrags fr[NS];
        auto issue = [&](auto s_c) {
          constexpr int s = decltype(s_c)::value;
          if constexpr (s < NA) {
            constexpr int tb = WL + s;
            fr[s].a = frag(Qs, 16 * tb + i, 0, g);
            fr[s].b = frag(Qs, 16 * tb + i, 1, g);
            fr[s].c = frag(Os, 16 * tb + i, 0, g);
            fr[s].d = frag(Os, 16 * tb + i, 1, g);
            fr[s].L = *reinterpret_cast<const f32x4*>(Ls + 16 * tb + 4 * g);
          } else if constexpr (s < NA + 4) {
            constexpr int jt = s - NA;
            if constexpr (WL < 2) fr[s].a = frag_tr(Os, 16 * jt, 0, g, i);
            fr[s].b = frag_tr(Os, 16 * jt, 1, g, i);
            fr[s].c = frag(dST, 16 * jt + i, 0, g);
            fr[s].d = frag(dST, 16 * jt + i, 1, g);
          } else {
            constexpr int dt = s - NA - 4;
            if constexpr (WL < 2) fr[s].a = frag_tr(Qs, 16 * dt, 0, g, i);
            fr[s].b = frag_tr(Qs, 16 * dt, 1, g, i);
            fr[s].c = frag_tr(dST, 16 * dt, 0, g, i);
            fr[s].d = frag_tr(dST, 16 * dt, 1, g, i);
            fr[s].e = *reinterpret_cast<const bf16x4*>(Ks + me * kPitch + 16 * dt + 4 * g);
          }
        };
        issue(std::integral_constant<int, 0>{});
        float colacc = 0.f, dw = 0.f;
        f32x4 At[4], dPt[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) At[tb] = dPt[tb] = zero4();
        bf16x8 A0, A1, dP0, dP1;
        static_for<0, NS>([&](auto s_c) {
          constexpr int s = decltype(s_c)::value;
          if constexpr (s + 1 < NS) issue(std::integral_constant<int, s + 1>{});
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (s < NA) {
            // (Q K^T) and dA = dO V^T blocks (t block tb, s block WL), decayed: A, dP, column sums of dA o A
            constexpr int tb = WL + s;
            f32x4 P = zero4(), dA = zero4();
            P = pgn_mfma(fr[s].a, kf0, P);
            P = pgn_mfma(fr[s].b, kf1, P);
            dA = pgn_mfma(fr[s].c, vf0, dA);
            dA = pgn_mfma(fr[s].d, vf1, dA);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = 16 * tb + 4 * g + r;
              // below the diagonal block every t > s, so the exponent is not positive: no clamp, no mask
              const float dec = tb > WL ? exp2_hw(fr[s].L[r] - Ls_s)
                                        : (t >= me ? exp2_hw(fminf(fr[s].L[r] - Ls_s, 0.f)) : 0.f);
              At[tb][r] = P[r] * dec;
              dPt[tb][r] = dA[r] * dec;
              colacc += dA[r] * At[tb][r];
            }
            if constexpr (s == NA - 1) {
              colacc = sum_groups(colacc);
              if (g == 0) colM[me] = colacc;
              A0 = pack(At[0], At[1]);
              A1 = pack(At[2], At[3]);
              dP0 = pack(dPt[0], dPt[1]);
              dP1 = pack(dPt[2], dPt[3]);
            }
          } else if constexpr (s < NA + 4) {
            // dV^T tile (j block jt, s block WL) = dO^T A + w_s (dS^T K^T): the w_s scaling after the product
            constexpr int jt = s - NA;
            f32x4 acc = zero4(), acc2 = zero4();
            if constexpr (WL < 2) acc = pgn_mfma(fr[s].a, A0, acc);
            acc = pgn_mfma(fr[s].b, A1, acc);
            acc2 = pgn_mfma(fr[s].c, kf0, acc2);
            acc2 = pgn_mfma(fr[s].d, kf1, acc2);
            acc = acc + acc2 * w_s;
            if constexpr (Rows::kAccumulate) acc += part4(dvp[jt]);  // added last: the load is waited for here
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), dv_out,
                                                  (me * ld + 16 * jt + 4 * g) * (int)sizeof(__bf16), 0, 0);
            if constexpr (Rows::kAccumulate && jt == 3) load_dvp(cn);
          } else {
            // dK^T tile (d block dt, s block WL) = Q^T dP + w_s (dS V^T); k_s.(dS v_s) on the way
            constexpr int dt = s - NA - 4;
            f32x4 acc = zero4(), Y = zero4();
            if constexpr (WL < 2) acc = pgn_mfma(fr[s].a, dP0, acc);
            acc = pgn_mfma(fr[s].b, dP1, acc);
            Y = pgn_mfma(fr[s].c, vf0, Y);
            Y = pgn_mfma(fr[s].d, vf1, Y);
            const f32x4 kk = to_f32x4(fr[s].e);
#pragma unroll
            for (int r = 0; r < 4; ++r) dw += kk[r] * Y[r];
            acc = acc + Y * w_s;
            if constexpr (Rows::kAccumulate) acc += part4(dkp[dt]);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), dk_out,
                                                  (me * ld + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
            if constexpr (s == NS - 1) {
              dw = sum_groups(dw);
              if (g == 0) dwv[me] = dw;
              if constexpr (Rows::kAccumulate) load_dkp(cn);
            }
          }
        });
        BWD_STAMP(5 + 2 * cc);
        if constexpr (WL >= 2) {
          if (cc > c0) stage(h ^ 1);
        }
        __syncthreads();
      }
    };
    switch (wl) {  // one instantiation per block index: its block conditions are compile-time constants
      case 0: kloop(std::integral_constant<int, 0>{}); break;
      case 1: kloop(std::integral_constant<int, 1>{}); break;
      case 2: kloop(std::integral_constant<int, 2>{}); break;
      default: kloop(std::integral_constant<int, 3>{}); break;
    }
  } else {
    PGN_STAMP_CLOCKS((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC));
    // ================= group D: t = me; dS rows 16 wl + 4g + r, column 16 jt + i
    f32x4 dS[4];
    const float* dsp = dSws ? dSws + (size_t)blockIdx.x * DK * DK : (dSfin ? dSfin + R.state() : nullptr);
    const int dsld = dSws ? DK : ld;
    // staging: thread b carries 16-byte row segments b and b + 256 of each of V, dO and S_c (waves 6 and 7 stage
    // Q and K)
    const int b = tid & 255;  // = tid; the mask tells the compiler that every segment row is below 64
    bf16x8 sv0, sv1, so0, so1, ss0, ss1;
    float pla = 0.f;
    auto load = [&](int cn) {
      const int n0 = cn * C, nr = min(C, T - n0);
      sv0 = load_seg(v + voff + (size_t)n0 * ld, nr, b, ld);
      sv1 = load_seg(v + voff + (size_t)n0 * ld, nr, b + 256, ld);
      so0 = load_seg(dO + voff + (size_t)n0 * ld, nr, b, ld);
      so1 = load_seg(dO + voff + (size_t)n0 * ld, nr, b + 256, ld);
      ss0 = load_seg(sent + ((size_t)R.scan * NC + cn) * DK * DK, DK, b);
      ss1 = load_seg(sent + ((size_t)R.scan * NC + cn) * DK * DK, DK, b + 256);
      pla = load_f32_lane(la + (size_t)R.hw * T + n0, nr, x.l);  // every wave (wave 0 uses it): no branch
    };
    auto stage = [&](int h) {
      __bf16* Qs = stg + h * kBwdStage;
      put_seg(Qs + 2 * TILE, sv0, b);
      put_seg(Qs + 2 * TILE, sv1, b + 256);
      put_seg(Qs + 3 * TILE, so0, b);
      put_seg(Qs + 3 * TILE, so1, b + 256);
      put_seg(Qs + 4 * TILE, ss0, b);
      put_seg(Qs + 4 * TILE, ss1, b + 256);
      const float la_t = pin_use(pla);  // (the staging loads have landed by here)
      if (w == 0) plain_scan(la_t, x.l, vec + h * kVec);
    };
    // accumulating pass: the first launch's dQ at this lane's outputs (t = 16 wl + i), loaded a chunk ahead and
    // issued, as in the loop, before the next chunk's staging loads (exact counter waits from the first iteration)
    __bf16* const dq_base = R.slot(dq, dq1, R.vh) + koff;
    auto dq_rows = [&](int cc) {
      const int t0 = cc * C;
      return __builtin_amdgcn_make_buffer_rsrc(dq_base + (size_t)t0 * ld, (short)0,
                                               min(C, T - t0) * ld * (int)sizeof(__bf16), 0x00020000);
    };
    const int me_d = 16 * wl + i;
    i32x2 dqp[4];
    auto load_dqp = [&](int cc) {
      const __amdgpu_buffer_rsrc_t r = dq_rows(cc);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) dqp[dt] = load_part4(r, (me_d * ld + 16 * dt + 4 * g) * (int)sizeof(__bf16));
    };
    load(cl);
    {
      // the gradient on the state the workgroup's chunks leave, 16 values a lane, loaded after the first chunk's
      // staging loads so that the two round trips overlap (an empty view when there is none: zeros, no branch)
      const __amdgpu_buffer_rsrc_t dsv = f32_view(dsp, DK * dsld);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS[jt][r] = load_f32(dsv, (16 * wl + 4 * g + r) * dsld + 16 * jt + i);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) store_T(dSTb + (cl & 1) * TILE, 16 * jt, 16 * wl, g, i, dS[jt]);
    }
    stage(cl & 1);
    if constexpr (Rows::kAccumulate) load_dqp(cl);
    __syncthreads();
    // this chunk's dla: stores to rows past T fall outside the range and are dropped (loads read zero)
    auto dla_rows = [&](int cc) {
      const int t0 = cc * C;
      return __builtin_amdgcn_make_buffer_rsrc(dlar + t0, (short)0, 4 * min(C, T - t0), 0x00020000);
    };
    // accumulating pass, wave 0: the first launch's dla of the chunk whose dla is pending
    float dlap = 0.f;
    auto dloop = [&](auto wl_c) {
      constexpr int WL = decltype(wl_c)::value;
      const int me = 16 * WL + i;
      for (int cc = cl; cc >= c0; --cc) {
        // the next chunk's V, dO and S_c, staged after this chunk's phase: loaded and staged within one iteration,
        // so no loaded register is carried around the loop (a carried one is copied at the loop's end, which waits
        // for the load). Unconditional: the last iteration re-reads this chunk, unused.
        load(max(cc - 1, c0));
        // wave 0: this chunk's dla partial, used when its dla is written after the next chunk's phase
        float dlap_next = 0.f;
        if constexpr (Rows::kAccumulate && WL == 0) {
          const int t0p = cc * C;
          const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
              const_cast<float*>(dlapr ? dlapr + t0p : dla), (short)0, dlapr ? 4 * min(C, T - t0p) : 0, 0x00020000);
          dlap_next = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, 4 * x.l, 0, 0));
        }
        BWD_STAMP(4 + 2 * cc);  // the chunk's phase: operand reads, contractions, result stores
        const int t0 = cc * C, h = cc & 1;
        const __bf16* Qs = stg + h * kBwdStage;
        const __bf16* Ks = Qs + TILE;
        const __bf16* Vs = Qs + 2 * TILE;
        const __bf16* Os = Qs + 3 * TILE;
        const __bf16* Ss = Qs + 4 * TILE;
        float* vs = vec + h * kVec;
        const float* Ls = vs;
        const float* eLs = vs + C;
        float* rowM = vs + 3 * C;  // row sums of dA o A
        float* qz = vs + 5 * C;    // q_t . (S_c dO_t)
        float* sdot = vs + 7 * C;  // per-lane partial sums of <S_c, dS>, summed in the dla
        const __amdgpu_buffer_rsrc_t dq_out = dq_rows(cc);
        const bf16x8 qf0 = frag(Qs, me, 0, g), qf1 = frag(Qs, me, 1, g);
        const bf16x8 of0 = frag(Os, me, 0, g), of1 = frag(Os, me, 1, g);
        const float Lt = Ls[me], eLt = eLs[me], LC = Ls[C - 1];
        // (Q o eL)^T operand of the dS update: read raw with the last dQ step's operands, scaled after that step
        bf16x8 qt0, qt1;
        f32x4 e00, e01, e10, e11;
        // The chunk's work as a sequence of steps: the P^T / dA^T blocks sb = 0..WL, the four dQ^T tiles, the four
        // column blocks of the dS update (with <S_c, dS> on the way). Each step's LDS operands are read one step
        // ahead (behind a scheduling barrier), so the reads overlap the MFMAs.
        constexpr int NA = WL + 1, NS = NA + 8;
        StepFrags fr[NS];
        auto issue = [&](auto s_c) {
          constexpr int s = decltype(s_c)::value;
          if constexpr (s < NA) {
            constexpr int sb = s;
            fr[s].a = frag(Ks, 16 * sb + i, 0, g);
            fr[s].b = frag(Ks, 16 * sb + i, 1, g);
            fr[s].c = frag(Vs, 16 * sb + i, 0, g);
            fr[s].d = frag(Vs, 16 * sb + i, 1, g);
            fr[s].L = *reinterpret_cast<const f32x4*>(Ls + 16 * sb + 4 * g);
          } else if constexpr (s < NA + 4) {
            constexpr int dt = s - NA;
            fr[s].a = frag_tr(Ks, 16 * dt, 0, g, i);
            if constexpr (WL >= 2) fr[s].b = frag_tr(Ks, 16 * dt, 1, g, i);
            fr[s].c = frag(Ss, 16 * dt + i, 0, g);
            fr[s].d = frag(Ss, 16 * dt + i, 1, g);
            fr[s].e = *reinterpret_cast<const bf16x4*>(Qs + me * kPitch + 16 * dt + 4 * g);
            if constexpr (dt == 3) {
              qt0 = frag_tr(Qs, 16 * WL, 0, g, i);
              qt1 = frag_tr(Qs, 16 * WL, 1, g, i);
              e00 = *reinterpret_cast<const f32x4*>(eLs + 4 * g);
              e01 = *reinterpret_cast<const f32x4*>(eLs + 16 + 4 * g);
              e10 = *reinterpret_cast<const f32x4*>(eLs + 32 + 4 * g);
              e11 = *reinterpret_cast<const f32x4*>(eLs + 48 + 4 * g);
            }
          } else {
            constexpr int jt = s - NA - 4;
            fr[s].a = frag_tr(Os, 16 * jt, 0, g, i);
            fr[s].b = frag_tr(Os, 16 * jt, 1, g, i);
            // S_c[16 WL + 4g + r][16 jt + i], r = 0..3: the transpose read of Ss at rows 16 WL.., columns 16 jt..
            fr[s].e = ds_read_tr(Ss + (16 * WL + 4 * g + (i >> 2)) * kPitch + 16 * jt + 4 * (i & 3));
          }
        };
        issue(std::integral_constant<int, 0>{});
        float rowacc = 0.f, qzt = 0.f, sd = 0.f, a_c = 0.f;
        f32x4 dPT[4];
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) dPT[sb] = zero4();
        bf16x8 b0, b1, qe0, qe1;
        __bf16* dSTn = dSTb + (h ^ 1) * TILE;
        static_for<0, NS>([&](auto s_c) {
          constexpr int s = decltype(s_c)::value;
          if constexpr (s + 1 < NS) issue(std::integral_constant<int, s + 1>{});
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (s < NA) {
            // (K Q^T) and dA^T = V dO^T blocks (s block sb, t block WL), decayed: dP^T, row sums of dA o A
            constexpr int sb = s;
            f32x4 PT = zero4(), dAT = zero4();
            PT = pgn_mfma(fr[s].a, qf0, PT);
            PT = pgn_mfma(fr[s].b, qf1, PT);
            dAT = pgn_mfma(fr[s].c, of0, dAT);
            dAT = pgn_mfma(fr[s].d, of1, dAT);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int sr = 16 * sb + 4 * g + r;
              // left of the diagonal block every s < t, so the exponent is not positive: no clamp, no mask
              const float dec = sb < WL ? exp2_hw(Lt - fr[s].L[r])
                                        : (sr <= me ? exp2_hw(fminf(Lt - fr[s].L[r], 0.f)) : 0.f);
              rowacc += dAT[r] * (PT[r] * dec);
              dPT[sb][r] = dAT[r] * dec;
            }
            if constexpr (s == NA - 1) {
              rowacc = sum_groups(rowacc);
              if (g == 0) rowM[me] = rowacc;
              b0 = pack(dPT[0], dPT[1]);
              b1 = pack(dPT[2], dPT[3]);
            }
          } else if constexpr (s < NA + 4) {
            // dQ^T tile (d block dt, t block WL) = K^T dP^T + eL_t (S_c dO_t); q_t.(S_c dO_t) on the way
            constexpr int dt = s - NA;
            f32x4 acc = zero4(), Z = zero4();
            acc = pgn_mfma(fr[s].a, b0, acc);
            if constexpr (WL >= 2) acc = pgn_mfma(fr[s].b, b1, acc);
            Z = pgn_mfma(fr[s].c, of0, Z);
            Z = pgn_mfma(fr[s].d, of1, Z);
            const f32x4 qq = to_f32x4(fr[s].e);
#pragma unroll
            for (int r = 0; r < 4; ++r) qzt += qq[r] * Z[r];
            acc = acc + Z * eLt;
            if constexpr (Rows::kAccumulate) acc += part4(dqp[dt]);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, to_bf16x4(acc)), dq_out,
                                                  (me * ld + 16 * dt + 4 * g) * (int)sizeof(__bf16), 0, 0);
            if constexpr (s == NA + 3) {
              if constexpr (Rows::kAccumulate) load_dqp(max(cc - 1, c0));  // unconditional: exact counter waits
              qzt = sum_groups(qzt);
              if (g == 0) qz[me] = qzt;
              a_c = exp2_hw(LC);
              qe0 = scale_frag_k(qt0, e00, e01);
              qe1 = scale_frag_k(qt1, e10, e11);
            }
          } else {
            // columns 16 jt.. of rows 16 WL.. of dS: <S_c, dS> with the old values, then dS <- a dS + (Q o eL)^T dO
            // into the other dS^T tile
            constexpr int jt = s - NA - 4;
            const f32x4 sv = to_f32x4(fr[s].e);
#pragma unroll
            for (int r = 0; r < 4; ++r) sd += sv[r] * dS[jt][r];
            f32x4 m = pgn_mfma(qe0, fr[s].a, zero4());
            m = pgn_mfma(qe1, fr[s].b, m);
            dS[jt] = dS[jt] * a_c + m;
            store_T(dSTn, 16 * jt, 16 * WL, g, i, dS[jt]);
            if constexpr (s == NS - 1) sdot[WL * 64 + x.l] = sd;
          }
        });
        BWD_STAMP(5 + 2 * cc);
        if (w == 0 && cc < cl)  // the later chunk's dla, from the other vector set (before the scan below)
          plain_dla<Rows::kAccumulate>(vec + (h ^ 1) * kVec, x.l, dla_rows(cc + 1), dlap);
        dlap = dlap_next;
        if (cc > c0) stage(h ^ 1);
        __syncthreads();
      }
    };
    switch (wl) {  // one instantiation per block index: its block conditions are compile-time constants
      case 0: dloop(std::integral_constant<int, 0>{}); break;
      case 1: dloop(std::integral_constant<int, 1>{}); break;
      case 2: dloop(std::integral_constant<int, 2>{}); break;
      default: dloop(std::integral_constant<int, 3>{}); break;
    }
    if (w == 0)  // the first chunk's dla (its vector set)
      plain_dla<Rows::kAccumulate>(vec + (c0 & 1) * kVec, x.l, dla_rows(c0), dlap);
    if (dS0) {
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) dS0[R.state() + (16 * wl + 4 * g + r) * ld + 16 * jt + i] = dS[jt][r];
    }
  }
  PGN_STAMP_CLOCKS((blockIdx.x * 8 + __builtin_amdgcn_readfirstlane(w)) * (4 + 2 * NC) + 2);
#undef BWD_STAMP
}

constexpr size_t kFwdSmem = 3 * (size_t)kFwdBuf + 4 * TILE * sizeof(__bf16);
constexpr size_t kBwdSmem = (2 * kBwdStage + 2 * TILE) * sizeof(__bf16) + 2 * kVec * sizeof(float);

bool shape_ok(int64_t B, int64_t H, int64_t T, int64_t D, int64_t Cc) {
  if (B <= 0 || H <= 0 || T <= 0) return false;
  if (B * H >= ((int64_t)1 << 31) || T >= ((int64_t)1 << 28)) return false;
  return D == DK && Cc == C;
}

// Heads of 128 (four scans each): the scan count and the slot sum's thread count (16 per row of 128) stay in range.
bool wide_shape_ok(int64_t B, int64_t H, int64_t T) {
  if (B <= 0 || H <= 0 || T <= 0) return false;
  if (4 * B * H >= ((int64_t)1 << 31) || T >= ((int64_t)1 << 28)) return false;
  return B * H * T < ((int64_t)1 << 27);
}

int64_t seg_count(int64_t T, int64_t seg_chunks) { return ((T + C - 1) / C + seg_chunks - 1) / seg_chunks; }

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// workspace of the segmented passes over `scans` 64 x 64 scans: E (F in the backward; fp32 64 x 64 per segment,
// later the state entering it) then the segment's total log-decay l
int64_t seg_bytes(int64_t scans, int64_t T, int64_t seg_chunks) {
  const int64_t n = scans * seg_count(T, seg_chunks);
  return n * DK * DK * (int64_t)sizeof(float) + align256(n * (int64_t)sizeof(float));
}

// The plain forward over `scans` scans (B H narrow heads; wide: 4 B H at PASS 0, 2 B H at PASS 1, 2): one workgroup
// per scan when seg_chunks covers the sequence, else (PASS 0) the segmented forward's three launches on `ws`
// (seg_bytes(scans, T, seg_chunks) bytes). theta, window: the carried windows (narrow heads only; H indexes theta).
template <bool WIDE, int PASS = 0>
int launch_fwd(const void* q, const void* k, const void* v, const float* la, const float* S0, const float* theta,
               int64_t window, void* o, void* o1, float* S_final, void* sent, void* ws, int64_t scans, int64_t H,
               int64_t T, int64_t seg_chunks, hipStream_t stream) {
  {
    const hipError_t e = pgn_lds_limit((const void*)aspin_plain_fwd<WIDE, PASS>, kFwdSmem);
    if (e != hipSuccess) return (int)e;
  }
  const int NC = (int)((T + C - 1) / C);
  if (seg_chunks >= NC) {
    hipLaunchKernelGGL((aspin_plain_fwd<WIDE, PASS>), dim3((unsigned)scans), dim3(kFwdWaves * 64), kFwdSmem, stream,
                       (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, S0, nullptr, (__bf16*)o,
                       (__bf16*)o1, S_final, (__bf16*)sent, (int)T, NC, NC);
    PGN_RETURN_LAUNCH();
  }
  if constexpr (PASS != 0) return PRAGNOSIA_ERR_INVALID_ARGUMENT;  // the two-launch passes are unsegmented
  const int64_t nseg = seg_count(T, seg_chunks);
  float* E = (float*)ws;
  float* lseg = E + scans * nseg * DK * DK;
  const unsigned nblk = (unsigned)(scans * nseg);
  hipLaunchKernelGGL((aspin_plain_segsum<true, WIDE>), dim3(nblk), dim3(256), 2 * kSumBuf, stream, (const __bf16*)k,
                     (const __bf16*)v, la, E, lseg, (int)T, NC, (int)seg_chunks);
  hipLaunchKernelGGL((aspin_plain_segprefix<false, WIDE>), dim3((unsigned)(scans * 8)), dim3(256), 0, stream, S0,
                     window > 0 ? theta : nullptr, (float)window, window > 0 ? (int)(window / C / seg_chunks) : 1, E,
                     lseg, S_final, (int)H, (int)nseg);
  hipLaunchKernelGGL((aspin_plain_fwd<WIDE, 0>), dim3(nblk), dim3(kFwdWaves * 64), kFwdSmem, stream, (const __bf16*)q,
                     (const __bf16*)k, (const __bf16*)v, la, nullptr, E, (__bf16*)o, (__bf16*)o1, nullptr,
                     (__bf16*)sent, (int)T, NC, (int)seg_chunks);
  PGN_RETURN_LAUNCH();
}

// The plain backward over `scans` scans, one workgroup per scan or (PASS 0) segmented as the forward.
template <bool WIDE, int PASS = 0>
int launch_bwd(const void* q, const void* k, const void* v, const float* la, const void* sent, const void* dO,
               const float* dS_final, void* dq, void* dq1, void* dk, void* dk1, void* dv, void* dv1, float* dla,
               float* dla1, float* dS0, void* ws, int64_t scans, int64_t T, int64_t seg_chunks, hipStream_t stream) {
  {
    const hipError_t e = pgn_lds_limit((const void*)aspin_plain_bwd<WIDE, PASS>, kBwdSmem);
    if (e != hipSuccess) return (int)e;
  }
  const int NC = (int)((T + C - 1) / C);
  if (seg_chunks >= NC) {
    hipLaunchKernelGGL((aspin_plain_bwd<WIDE, PASS>), dim3((unsigned)scans), dim3(512), kBwdSmem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, la, (const __bf16*)sent, (const __bf16*)dO, dS_final,
                       nullptr, (__bf16*)dq, (__bf16*)dq1, (__bf16*)dk, (__bf16*)dk1, (__bf16*)dv, (__bf16*)dv1, dla,
                       dla1, dS0, (int)T, NC, NC);
    PGN_RETURN_LAUNCH();
  }
  if constexpr (PASS != 0) return PRAGNOSIA_ERR_INVALID_ARGUMENT;  // the two-launch passes are unsegmented
  const int64_t nseg = seg_count(T, seg_chunks);
  float* F = (float*)ws;
  float* lseg = F + scans * nseg * DK * DK;
  const unsigned nblk = (unsigned)(scans * nseg);
  hipLaunchKernelGGL((aspin_plain_segsum<false, WIDE>), dim3(nblk), dim3(256), 2 * kSumBuf, stream, (const __bf16*)q,
                     (const __bf16*)dO, la, F, lseg, (int)T, NC, (int)seg_chunks);
  hipLaunchKernelGGL((aspin_plain_segprefix<true, WIDE>), dim3((unsigned)(scans * 8)), dim3(256), 0, stream, dS_final,
                     nullptr, 0.f, 1, F, lseg, dS0, 1, (int)nseg);
  hipLaunchKernelGGL((aspin_plain_bwd<WIDE, 0>), dim3(nblk), dim3(512), kBwdSmem, stream, (const __bf16*)q,
                     (const __bf16*)k, (const __bf16*)v, la, (const __bf16*)sent, (const __bf16*)dO, nullptr, F,
                     (__bf16*)dq, (__bf16*)dq1, (__bf16*)dk, (__bf16*)dk1, (__bf16*)dv, (__bf16*)dv1, dla, dla1,
                     nullptr, (int)T, NC, (int)seg_chunks);
  PGN_RETURN_LAUNCH();
}

// The slot sums of the wide entry points: for each bf16 pair p with x[p] set, x[p][i] <- x[p][i] + y[p][i] over n
// elements (the fp32 sum of the two bf16 values rounded once to bf16, as a bf16 tensor add rounds), and, when dla is
// set, dla[i] <- (dla[i] + w[i]) + w[m + i] ... over the nw slots of w (m fp32 elements each). Thread u covers
// elements 8u .. 8u + 7 of every pair (n % 8 == 0) and fp32 element u (m <= n / 8).
struct JoinArgs {
  __bf16* x[3];
  const __bf16* y[3];
  float* dla;
  const float* w;
  int64_t n, m;
  int nw;
};

__global__ __launch_bounds__(256) void aspin_wide_join(JoinArgs a) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (8 * u < a.n) {
    bf16x8 xs[3], ys[3];
#pragma unroll
    for (int p = 0; p < 3; ++p)
      if (a.x[p]) {
        xs[p] = *reinterpret_cast<const bf16x8*>(a.x[p] + 8 * u);
        ys[p] = *reinterpret_cast<const bf16x8*>(a.y[p] + 8 * u);
      }
#pragma unroll
    for (int p = 0; p < 3; ++p)
      if (a.x[p]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[p][j] = pgn_bf16(pgn_f32(xs[p][j]) + pgn_f32(ys[p][j]));
        *reinterpret_cast<bf16x8*>(a.x[p] + 8 * u) = xs[p];
      }
  }
  if (a.dla && u < a.m) {
    float d = a.dla[u];
    for (int j = 0; j < a.nw; ++j) d += a.w[j * a.m + u];
    a.dla[u] = d;
  }
}

int launch_join(const JoinArgs& a, hipStream_t stream) {
  const int64_t units = std::max(a.n / 8, a.m);
  hipLaunchKernelGGL(aspin_wide_join, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, stream, a);
  PGN_RETURN_LAUNCH();
}

// workspace of the wide entry points: the slot-1 outputs (o; or dq, dk, dv and three dla slots), then the segmented
// passes' workspace when seg_chunks does not cover the sequence
int64_t wide_slot_bytes(int64_t B, int64_t H, int64_t T) { return align256(B * H * T * 2 * DK * (int64_t)sizeof(__bf16)); }

int64_t wide_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t seg_chunks, bool backward) {
  const int64_t slot = wide_slot_bytes(B, H, T);
  int64_t n = backward ? 3 * slot + align256(3 * B * H * T * (int64_t)sizeof(float)) : slot;
  if (seg_chunks < (T + C - 1) / C) n += seg_bytes(4 * B * H, T, seg_chunks);
  return n;
}

bool wide_args_ok(int64_t B, int64_t H, int64_t T, int64_t seg_chunks) {
  return wide_shape_ok(B, H, T) && seg_chunks >= 1 && seg_chunks < ((int64_t)1 << 28) &&
         4 * B * H * seg_count(T, seg_chunks) < ((int64_t)1 << 31);
}

}  // namespace

extern "C" int pragnosia_aspin_chunk_fwd(const void* q, const void* k, const void* v, const float* la, const float* S0,
                                         void* o, float* S_final, void* sent, int64_t B, int64_t H, int64_t T,
                                         int64_t D, int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && o && S_final);
  return launch_fwd<false>(q, k, v, la, S0, nullptr, 0, o, nullptr, S_final, sent, nullptr, B * H, H, T,
                           (T + C - 1) / C, (hipStream_t)stream);
}

extern "C" int64_t pragnosia_aspin_chunk_seg_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D,
                                                             int64_t chunk, int64_t seg_chunks) {
  if (D != DK || chunk != C || seg_chunks < 1 || !shape_ok(B, H, T, D, chunk)) return -1;
  return seg_bytes(B * H, T, seg_chunks);
}

namespace {

// Host-side checks of the segmented forward's arguments other than its workspace.
bool fwd_seg_args_ok(const void* q, const void* k, const void* v, const float* la, const float* theta,
                     int64_t window, void* o, float* S_final, int64_t B, int64_t H, int64_t T, int64_t D,
                     int64_t chunk, int64_t seg_chunks) {
  if (!shape_ok(B, H, T, D, chunk) || !(q && k && v && la && o && S_final)) return false;
  if (seg_chunks < 1 || seg_chunks >= ((int64_t)1 << 28) || window < 0) return false;
  if (window > 0 && !(theta && window % C == 0 && (window / C) % seg_chunks == 0)) return false;
  return B * H * seg_count(T, seg_chunks) < ((int64_t)1 << 31);
}

// The segmented forward's three launches on a workspace of at least seg_bytes(B H, T, seg_chunks) bytes (seg_chunks
// at least the sequence's chunk count: one workgroup per head, the workspace unused).
int launch_fwd_seg(const void* q, const void* k, const void* v, const float* la, const float* S0, const float* theta,
                   int64_t window, void* o, float* S_final, void* sent, void* workspace, int64_t B, int64_t H,
                   int64_t T, int64_t seg_chunks, void* stream) {
  return launch_fwd<false>(q, k, v, la, S0, theta, window, o, nullptr, S_final, sent, workspace, B * H, H, T,
                           seg_chunks, (hipStream_t)stream);
}

}  // namespace

extern "C" int pragnosia_aspin_chunk_fwd_seg(const void* q, const void* k, const void* v, const float* la,
                                             const float* S0, const float* theta, int64_t window, void* o,
                                             float* S_final, void* sent, void* workspace, int64_t workspace_bytes,
                                             int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk,
                                             int64_t seg_chunks, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(fwd_seg_args_ok(q, k, v, la, theta, window, o, S_final, B, H, T, D, chunk, seg_chunks));
  PGN_CHECK_ARG(workspace && workspace_bytes >= seg_bytes(B * H, T, seg_chunks));
  return launch_fwd_seg(q, k, v, la, S0, theta, window, o, S_final, sent, workspace, B, H, T, seg_chunks, stream);
}

// The allocation-free variant's workspace: one array per GPU, in the library's own device memory, held until the
// process ends. Host code never passes the array's name to a kernel (on the host it is only a stand-in for the
// symbol); the device address comes from hipGetSymbolAddress, once per device with that device current.
static __device__ __align__(256) unsigned char scratch[PRAGNOSIA_SEG_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};  // device address of `scratch` per device ordinal

// The current device's address of `scratch`, looked up on the first call on that device.
hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" int pragnosia_aspin_chunk_fwd_seg_noalloc(const void* q, const void* k, const void* v, const float* la,
                                                     const float* S0, const float* theta, int64_t window, void* o,
                                                     float* S_final, void* sent, int64_t B, int64_t H, int64_t T,
                                                     int64_t D, int64_t chunk, int64_t seg_chunks, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(fwd_seg_args_ok(q, k, v, la, theta, window, o, S_final, B, H, T, D, chunk, seg_chunks));
  if (seg_bytes(B * H, T, seg_chunks) > (int64_t)PRAGNOSIA_SEG_SCRATCH_BYTES) return PRAGNOSIA_ERR_TOO_LARGE;
  void* ws = nullptr;
  const hipError_t e = scratch_address(&ws);
  if (e != hipSuccess) return (int)e;
  // every byte the launches read from the workspace is written by them first (each segment's full sum and decay,
  // then its entering state), so nothing left by an earlier call needs clearing
  return launch_fwd_seg(q, k, v, la, S0, theta, window, o, S_final, sent, ws, B, H, T, seg_chunks, stream);
}

extern "C" int pragnosia_aspin_chunk_bwd(const void* q, const void* k, const void* v, const float* la,
                                         const void* sent, const void* dO, const float* dS_final, void* dq, void* dk,
                                         void* dv, float* dla, float* dS0, int64_t B, int64_t H, int64_t T, int64_t D,
                                         int64_t chunk, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && sent && dO && dq && dk && dv && dla);
  return launch_bwd<false>(q, k, v, la, sent, dO, dS_final, dq, nullptr, dk, nullptr, dv, nullptr, dla, nullptr, dS0,
                           nullptr, B * H, T, (T + C - 1) / C, (hipStream_t)stream);
}

extern "C" int pragnosia_aspin_chunk_bwd_seg(const void* q, const void* k, const void* v, const float* la,
                                             const void* sent, const void* dO, const float* dS_final, void* dq,
                                             void* dk, void* dv, float* dla, float* dS0, void* workspace,
                                             int64_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                                             int64_t chunk, int64_t seg_chunks, void* stream) {
  if (D != DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, H, T, D, chunk));
  PGN_CHECK_ARG(q && k && v && la && sent && dO && dq && dk && dv && dla && workspace);
  PGN_CHECK_ARG(seg_chunks >= 1 && seg_chunks < ((int64_t)1 << 28));
  PGN_CHECK_ARG(workspace_bytes >= seg_bytes(B * H, T, seg_chunks));
  PGN_CHECK_ARG(B * H * seg_count(T, seg_chunks) < ((int64_t)1 << 31));
  return launch_bwd<false>(q, k, v, la, sent, dO, dS_final, dq, nullptr, dk, nullptr, dv, nullptr, dla, nullptr, dS0,
                           workspace, B * H, T, seg_chunks, (hipStream_t)stream);
}

extern "C" int64_t pragnosia_aspin_chunk_wide_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D,
                                                              int64_t chunk, int64_t seg_chunks, int32_t backward) {
  if (D != 2 * DK || chunk != C || !wide_args_ok(B, H, T, seg_chunks)) return -1;
  return wide_workspace_bytes(B, H, T, seg_chunks, backward != 0);
}

extern "C" int pragnosia_aspin_chunk_fwd_wide(const void* q, const void* k, const void* v, const float* la,
                                              const float* S0, void* o, float* S_final, void* sent, void* workspace,
                                              int64_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                                              int64_t chunk, int64_t seg_chunks, void* stream) {
  if (D != 2 * DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(wide_args_ok(B, H, T, seg_chunks));
  PGN_CHECK_ARG(q && k && v && la && o && S_final && workspace);
  PGN_CHECK_ARG(workspace_bytes >= wide_workspace_bytes(B, H, T, seg_chunks, false));
  char* ws = (char*)workspace;
  if (seg_chunks >= (T + C - 1) / C) {
    // one workgroup per (head, value half) over all 128 keys: o written once, no partial sums
    const hipError_t e = pgn_lds_limit((const void*)aspin_plain_fwd128, kN128Smem);
    if (e != hipSuccess) return (int)e;
    const unsigned grid = (unsigned)((B * H + 7) / 8 * 16);
    hipLaunchKernelGGL(aspin_plain_fwd128, dim3(grid), dim3(kFwdWaves * 64), kN128Smem, (hipStream_t)stream,
                       (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, la, S0, (__bf16*)o, S_final,
                       (__bf16*)sent, (int)T, (int)((T + C - 1) / C), (int)(B * H));
    PGN_RETURN_LAUNCH();
  }
  void* o1 = ws;
  const int rc = launch_fwd<true>(q, k, v, la, S0, nullptr, 0, o, o1, S_final, sent, ws + wide_slot_bytes(B, H, T),
                                  4 * B * H, 4 * H, T, seg_chunks, (hipStream_t)stream);
  if (rc != PRAGNOSIA_OK) return rc;
  JoinArgs a = {};
  a.x[0] = (__bf16*)o;
  a.y[0] = (const __bf16*)o1;
  a.n = B * H * T * 2 * DK;
  return launch_join(a, (hipStream_t)stream);
}

extern "C" int pragnosia_aspin_chunk_bwd_wide(const void* q, const void* k, const void* v, const float* la,
                                              const void* sent, const void* dO, const float* dS_final, void* dq,
                                              void* dk, void* dv, float* dla, float* dS0, void* workspace,
                                              int64_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                                              int64_t chunk, int64_t seg_chunks, void* stream) {
  if (D != 2 * DK || chunk != C) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(wide_args_ok(B, H, T, seg_chunks));
  PGN_CHECK_ARG(q && k && v && la && sent && dO && dq && dk && dv && dla && workspace);
  PGN_CHECK_ARG(workspace_bytes >= wide_workspace_bytes(B, H, T, seg_chunks, true));
  char* ws = (char*)workspace;
  const int64_t slot = wide_slot_bytes(B, H, T);
  void *dq1 = ws, *dk1 = ws + slot, *dv1 = ws + 2 * slot;
  float* dla1 = (float*)(ws + 3 * slot);
  if (seg_chunks >= (T + C - 1) / C) {
    // two launches of two scans per head, the second adding its dq, dk, dv to the first's; dla from two slots
    int rc = launch_bwd<true, 1>(q, k, v, la, sent, dO, dS_final, dq, nullptr, dk, nullptr, dv, nullptr, dla, dla1,
                                 dS0, nullptr, 2 * B * H, T, seg_chunks, (hipStream_t)stream);
    if (rc != PRAGNOSIA_OK) return rc;
    return launch_bwd<true, 2>(q, k, v, la, sent, dO, dS_final, dq, nullptr, dk, nullptr, dv, nullptr, dla, dla1,
                               dS0, nullptr, 2 * B * H, T, seg_chunks, (hipStream_t)stream);
  }
  void* segws = ws + 3 * slot + align256(3 * B * H * T * (int64_t)sizeof(float));
  const int rc = launch_bwd<true>(q, k, v, la, sent, dO, dS_final, dq, dq1, dk, dk1, dv, dv1, dla, dla1, dS0, segws,
                                  4 * B * H, T, seg_chunks, (hipStream_t)stream);
  if (rc != PRAGNOSIA_OK) return rc;
  JoinArgs a = {};
  a.x[0] = (__bf16*)dq;
  a.y[0] = (const __bf16*)dq1;
  a.x[1] = (__bf16*)dk;
  a.y[1] = (const __bf16*)dk1;
  a.x[2] = (__bf16*)dv;
  a.y[2] = (const __bf16*)dv1;
  a.dla = dla;
  a.w = dla1;
  a.n = B * H * T * 2 * DK;
  a.m = B * H * T;
  a.nw = 3;
  return launch_join(a, (hipStream_t)stream);
}
