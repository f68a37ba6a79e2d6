// Wave-level 16x16 tile algebra on the gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16), shared by the aspin kernels.
//
// Accumulator (D) layout of a 16x16 fp32 tile, as on every CDNA 16x16 MFMA: lane l = i + 16 g (i = l % 16,
// g = l / 16) holds column i, rows 4g .. 4g + 3 (element r = row 4g + r).
//
// Operands. A (16 x K) and B (K x 16) tiles: lane i + 16 g holds row i of A (column i of B) and 8 values along the
// contracted index. The pairing of (lane group, element) with k is the same for A and B by construction, so any
// bijection gives the exact product. This file fixes one: within a 32-wide k block, lane group g holds
//     k = 4g + {0,1,2,3}  (elements 0..3)   and   k = 16 + 4g + {0,1,2,3}  (elements 4..7).
// With it, an accumulator tile pair (rows 0..15 and 16..31 of a 32-row block) IS an operand whose contracted index
// is the tiles' row index: pack(D_lo, D_hi). Operands read from LDS are two 8-byte loads per lane.
//
// LDS tiles are row-major bf16 with a pitch of kPitch = 68 elements (136 bytes = 34 four-byte banks, 2 mod 32): the
// 16 rows an operand read touches start on the 16 even banks of 32, so each lane group's 8-byte reads cover every
// bank once and a 64-lane read runs at its 2-pass minimum (a pitch of 72 measured slower on every kernel). The
// 16-byte row-segment staging writes spread evenly too (4 passes for 1 KB).
#pragma once
#include <type_traits>

#include "common.h"

namespace pgn {

constexpr int kPitch = 68;

struct WaveIdx {
  int w, l, g, i;
};

// Lane indices recomputed from an opaque copy of the thread index. Persistent kernels call this at the top of
// every work item: addresses derived from the lane are then recomputed per item (a few ALU operations) instead of
// being hoisted out of the item loop and held in registers for the kernel's lifetime.
PGN_DEVICE WaveIdx wave_idx_opaque() {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  return WaveIdx{__builtin_amdgcn_readfirstlane(tid >> 6), tid & 63, (tid & 63) >> 4, tid & 15};
}

// The wave index is made wave-uniform (an SGPR): conditions on it are then scalar branches. That is required, not
// an optimisation: MFMA instructions ignore EXEC, so an MFMA under a condition the compiler believes divergent (a
// lane mask that happens to be empty) would still execute and overwrite its destination.
PGN_DEVICE WaveIdx wave_idx() {
  const int tid = threadIdx.x;
  return WaveIdx{__builtin_amdgcn_readfirstlane(tid >> 6), tid & 63, (tid & 63) >> 4, tid & 15};
}

PGN_DEVICE f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Decay exponents are kept in base 2 (L log2 e), so exp(L_t - L_s) is one hardware exp2 of a difference.
constexpr float kLog2e = 1.4426950408889634f;
PGN_DEVICE float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// f(std::integral_constant<int, S>{}) for S = B .. E - 1 in order: a loop whose index is a compile-time constant in
// the body, for step sequences whose steps differ in kind.
template <int B, int E, class F>
PGN_DEVICE void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Registers for one step's LDS operands in a software-pipelined step sequence (fields used as each step needs).
struct StepFrags {
  bf16x8 a, b, c, d;
  f32x4 L;
  bf16x4 e;
};

PGN_DEVICE bf16x8 cat8(bf16x4 a, bf16x4 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7); }

// Operand fragment of k block m from row `row` of an LDS tile.
PGN_DEVICE bf16x8 frag(const __bf16* tile, int row, int m, int g) {
  const __bf16* p = tile + row * kPitch + 32 * m + 4 * g;
  return cat8(*reinterpret_cast<const bf16x4*>(p), *reinterpret_cast<const bf16x4*>(p + 16));
}

PGN_DEVICE bf16x4 to_bf16x4(f32x4 x) {
  bf16x4 r;
  r[0] = (__bf16)x[0];
  r[1] = (__bf16)x[1];
  r[2] = (__bf16)x[2];
  r[3] = (__bf16)x[3];
  return r;
}

// A 16 x 16 accumulator tile (lane (i, g) holds rows 4g..4g+3 of column i) rounded to bf16 and transposed within
// each quad of lanes (i = 4m..4m+3) by two DPP exchanges (the off-diagonal 2 x 2 blocks between lanes p and p^2,
// then 16-bit halves between lanes p and p^1), so that lane (i, g) ends holding row 4g + (i & 3), columns
// 4 (i >> 2) .. +3 of the tile: one 8-byte row-major store per lane instead of four 2-byte ones. All 64 lanes must
// be active.
PGN_DEVICE bf16x4 quad_rows(f32x4 x, int i) {
  const int p = i & 3;
  const i32x2 v = __builtin_bit_cast(i32x2, to_bf16x4(x));
  unsigned d0 = (unsigned)v[0], d1 = (unsigned)v[1];  // rows (0, 1) and (2, 3) of this lane's column
  const unsigned send = (p & 2) ? d0 : d1;
  const unsigned recv = (unsigned)__builtin_amdgcn_update_dpp(0, (int)send, 0x4E, 0xf, 0xf, false);  // [2,3,0,1]
  if (p & 2) d0 = recv; else d1 = recv;
  const unsigned o0 = (unsigned)__builtin_amdgcn_update_dpp(0, (int)d0, 0xB1, 0xf, 0xf, false);  // [1,0,3,2]
  const unsigned o1 = (unsigned)__builtin_amdgcn_update_dpp(0, (int)d1, 0xB1, 0xf, 0xf, false);
  if (p & 1) {
    d0 = (o0 >> 16) | (d0 & 0xffff0000u);
    d1 = (o1 >> 16) | (d1 & 0xffff0000u);
  } else {
    d0 = (d0 & 0xffffu) | (o0 << 16);
    d1 = (d1 & 0xffffu) | (o1 << 16);
  }
  return __builtin_bit_cast(bf16x4, i32x2{(int)d0, (int)d1});
}

PGN_DEVICE f32x4 to_f32x4(bf16x4 x) { return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]}; }

// Operand from an accumulator tile pair (contracted index = the tiles' row index).
PGN_DEVICE bf16x8 pack(f32x4 lo, f32x4 hi) { return cat8(to_bf16x4(lo), to_bf16x4(hi)); }

// Fragment scaled by one factor (per lane: the operand's row), rounded back to bf16.
PGN_DEVICE bf16x8 frag_scaled(const __bf16* tile, int row, int m, int g, float f) {
  const __bf16* p = tile + row * kPitch + 32 * m + 4 * g;
  f32x4 a = to_f32x4(*reinterpret_cast<const bf16x4*>(p)) * f;
  f32x4 b = to_f32x4(*reinterpret_cast<const bf16x4*>(p + 16)) * f;
  return pack(a, b);
}

// Fragment scaled per contracted index k by s[k] (fp32 LDS vector), rounded back to bf16.
PGN_DEVICE bf16x8 frag_scaled_k(const __bf16* tile, int row, int m, int g, const float* s) {
  const __bf16* p = tile + row * kPitch + 32 * m + 4 * g;
  const f32x4 sa = *reinterpret_cast<const f32x4*>(s + 32 * m + 4 * g);
  const f32x4 sb = *reinterpret_cast<const f32x4*>(s + 32 * m + 16 + 4 * g);
  f32x4 a = to_f32x4(*reinterpret_cast<const bf16x4*>(p)) * sa;
  f32x4 b = to_f32x4(*reinterpret_cast<const bf16x4*>(p + 16)) * sb;
  return pack(a, b);
}

// Transposed operand fragments, on gfx950's LDS transpose read (ds_read_b64_tr_b16). Within each group of 16 lanes
// the instruction hands lane L element L % 4 of the 8 bytes addressed by lanes L / 4, 4 + L / 4, 8 + L / 4 and
// 12 + L / 4 (in that order). So if lane p of group g addresses row (r0 + 4g + p / 4), columns (n0 + 4 (p % 4)) ..
// +3 of a row-major tile X, lane i of group g receives X[r0 + 4g + e][n0 + i] for e = 0..3: column n0 + i of X with
// the contracted index running down X's rows, in this file's k order. frag_tr(X, n0, m, g, i) is therefore the
// operand frag(X^T, n0 + i, m, g) read straight from X, with no transposed copy of X in LDS.
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

PGN_DEVICE bf16x4 ds_read_tr(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

PGN_DEVICE bf16x8 frag_tr(const __bf16* tile, int n0, int m, int g, int i) {
  const __bf16* p = tile + (32 * m + 4 * g + (i >> 2)) * kPitch + n0 + 4 * (i & 3);
  return cat8(ds_read_tr(p), ds_read_tr(p + 16 * kPitch));
}

// frag_tr scaled per contracted index k by s[k] (fp32 LDS vector), rounded back to bf16.
PGN_DEVICE bf16x8 frag_tr_scaled_k(const __bf16* tile, int n0, int m, int g, int i, const float* s) {
  const __bf16* p = tile + (32 * m + 4 * g + (i >> 2)) * kPitch + n0 + 4 * (i & 3);
  const f32x4 sa = *reinterpret_cast<const f32x4*>(s + 32 * m + 4 * g);
  const f32x4 sb = *reinterpret_cast<const f32x4*>(s + 32 * m + 16 + 4 * g);
  f32x4 a = to_f32x4(ds_read_tr(p)) * sa;
  f32x4 b = to_f32x4(ds_read_tr(p + 16 * kPitch)) * sb;
  return pack(a, b);
}

// A fragment already in registers scaled by one factor, or per contracted index k by (sa, sb) (the factors of its
// elements 0..3 and 4..7), rounded back to bf16: frag_scaled and frag_tr_scaled_k without the LDS read, so the read
// can be issued early.
PGN_DEVICE bf16x8 scale_frag(bf16x8 f, float s) {
  return pack(to_f32x4(__builtin_shufflevector(f, f, 0, 1, 2, 3)) * s,
              to_f32x4(__builtin_shufflevector(f, f, 4, 5, 6, 7)) * s);
}

PGN_DEVICE bf16x8 scale_frag_k(bf16x8 f, f32x4 sa, f32x4 sb) {
  return pack(to_f32x4(__builtin_shufflevector(f, f, 0, 1, 2, 3)) * sa,
              to_f32x4(__builtin_shufflevector(f, f, 4, 5, 6, 7)) * sb);
}

// Store an accumulator tile transposed into an LDS tile: rows 4g..4g+3 of column i land contiguously in row
// (col0 + i) of `tile`, columns row0 + 4g .. +3 (one 8-byte write).
PGN_DEVICE void store_T(__bf16* tile, int col0, int row0, int g, int i, f32x4 x) {
  *reinterpret_cast<bf16x4*>(tile + (col0 + i) * kPitch + row0 + 4 * g) = to_bf16x4(x);
}

// Store an accumulator tile untransposed: element r to tile[row0 + 4g + r][col0 + i] (four 2-byte writes).
PGN_DEVICE void store_N(__bf16* tile, int row0, int col0, int g, int i, f32x4 x) {
#pragma unroll
  for (int r = 0; r < 4; ++r) tile[(row0 + 4 * g + r) * kPitch + col0 + i] = (__bf16)x[r];
}

// Staging of 64-row bf16 blocks through registers. A thread owns a 4 x 4 sub-block (rows 4*(b/16).., columns
// 4*(b%16).. for block index b): each of its four 8-byte global loads is part of a 128-byte row segment read by 16
// consecutive lanes, and the transposed copy is a 4 x 4 register transpose followed by four 8-byte LDS writes.
struct Blk4 {
  bf16x4 r[4];
};

PGN_DEVICE bf16x4 zero_bf16x4() {
  bf16x4 z;
  z[0] = z[1] = z[2] = z[3] = (__bf16)0.f;
  return z;
}

// Load block b of a (rows x 64-wide) region starting at src (row stride ld elements); rows >= nrows (>= 1) read as
// zero. Rows past the end load row nrows - 1 and are then replaced by zero, so every load is unconditional (a
// branch per load keeps each load's address and result live across the branch).
PGN_DEVICE Blk4 load_blk(const __bf16* __restrict__ src, int ld, int nrows, int b) {
  const int r0 = 4 * (b >> 4), c0 = 4 * (b & 15);
  Blk4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(src + (size_t)min(r0 + j, nrows - 1) * ld + c0);
    x.r[j] = (r0 + j < nrows) ? v : zero_bf16x4();
  }
  return x;
}

// The same for a region only `ncols` (multiple of 4) wide: block b covers rows 4*(b / (ncols/4)).. . Rows past
// nrows - 1 are outside the blocks any caller passes only when nrows >= 1.
PGN_DEVICE Blk4 load_blk_w(const __bf16* __restrict__ src, int ld, int nrows, int ncols, int b) {
  const int per_row = ncols >> 2;
  const int r0 = 4 * (b / per_row), c0 = 4 * (b % per_row);
  Blk4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(src + (size_t)min(r0 + j, nrows - 1) * ld + c0);
    x.r[j] = (r0 + j < nrows) ? v : zero_bf16x4();
  }
  return x;
}

PGN_DEVICE void put_blk(__bf16* tile, const Blk4& x, int r0, int c0) {
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<bf16x4*>(tile + (r0 + j) * kPitch + c0) = x.r[j];
}

PGN_DEVICE void put_blk_T(__bf16* tile, const Blk4& x, int r0, int c0) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bf16x4 col;
    col[0] = x.r[0][j];
    col[1] = x.r[1][j];
    col[2] = x.r[2][j];
    col[3] = x.r[3][j];
    *reinterpret_cast<bf16x4*>(tile + (c0 + j) * kPitch + r0) = col;
  }
}

// Staging of row-major 64-column bf16 tiles in 16-byte row segments, for tiles that are only ever read untransposed
// or through frag_tr: segment e covers row e / 8, columns 8 (e % 8) .. +7, so one 64-lane load reads eight whole
// 128-byte rows. Rows >= nrows (0 <= nrows <= 64) read as zero: the load goes through a buffer resource whose range
// ends after row nrows - 1, so it needs no branch (with a select on the row instead, the compiler sinks each load
// into a branch, and the memory-counter waits of the loops around it turn conservative). `ld` is the source's row
// pitch in elements (64 for a dense tile; 128 for one half of rows of 128).
PGN_DEVICE bf16x8 load_seg(const __bf16* __restrict__ src, int nrows, int e, int ld = 64) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(src), (short)0,
                                                                     nrows * ld * (int)sizeof(__bf16), 0x00020000);
  return __builtin_bit_cast(
      bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, ((e >> 3) * ld + 8 * (e & 7)) * (int)sizeof(__bf16), 0, 0));
}

// The value, used outside any branch: a load whose only use sits inside a branch is sunk into that branch by the
// compiler (issued there, just before the use, so its latency is exposed); passing it through this where the value
// is needed anyway keeps the load at its place in the code. Emits no instruction.
PGN_DEVICE float pin_use(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// A range-checked view of n fp32 elements at p (an empty one when p is null): a load past the range, or from an empty
// view, reads zero with no branch, so a kernel can issue such loads unconditionally, all before it uses any.
PGN_DEVICE __amdgpu_buffer_rsrc_t f32_view(const float* p, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, p ? n * (int)sizeof(float) : 0,
                                           0x00020000);
}
PGN_DEVICE float load_f32(__amdgpu_buffer_rsrc_t r, int i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, i * (int)sizeof(float), 0, 0));
}

// Element `lane` of an fp32 vector of n elements (0 <= n <= 64; zero at and past n) through a range-checked buffer:
// no select on the lane, so the load is not sunk into a branch.
PGN_DEVICE float load_f32_lane(const float* p, int n, int lane) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, n * (int)sizeof(float), 0x00020000);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane * (int)sizeof(float), 0, 0));
}

// Four bf16 at byte offset `off` of a range-checked buffer (zero past the range), kept packed until used: the partial
// result that an accumulating store adds to (part4 widens it to fp32).
PGN_DEVICE i32x2 load_part4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
PGN_DEVICE f32x4 part4(i32x2 v) { return to_f32x4(__builtin_bit_cast(bf16x4, v)); }

// The segment into an LDS tile (pitch kPitch, so rows are 8-byte aligned: two 8-byte writes).
PGN_DEVICE void put_seg(__bf16* tile, bf16x8 v, int e) {
  __bf16* p = tile + (e >> 3) * kPitch + 8 * (e & 7);
  *reinterpret_cast<bf16x4*>(p) = __builtin_shufflevector(v, v, 0, 1, 2, 3);
  *reinterpret_cast<bf16x4*>(p + 4) = __builtin_shufflevector(v, v, 4, 5, 6, 7);
}

// exp(min(x, 0)) where `keep`, else 0, without a branch: the exponent is never positive, so the unmasked value is
// finite and at most 1 and the mask is a select (a branch per element around the exp serialises the waves).
PGN_DEVICE float masked_decay(float x, bool keep) { return __expf(fminf(x, 0.f)) * (keep ? 1.f : 0.f); }

// Sum over the 16 lanes of a lane group (same g): butterfly over lane bits 0..3.
PGN_DEVICE float sum16(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

// Sum over the 4 lane groups (same i): butterfly over lane bits 4..5.
PGN_DEVICE float sum_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

PGN_DEVICE float wave_sum(float x) { return sum_groups(sum16(x)); }

// x moved by a DPP row operation (CTRL), 0 where the source lane falls outside the lane's row of 16.
template <int CTRL>
PGN_DEVICE float dpp_row0(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

PGN_DEVICE float lane_value(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Sum over the 16 lanes of each row (lane group): an inclusive scan on DPP row shifts, so lane 15 of each row holds
// the row's total (the other lanes hold partial sums).
PGN_DEVICE float row_total16(float x) {
  x += dpp_row0<0x111>(x);
  x += dpp_row0<0x112>(x);
  x += dpp_row0<0x114>(x);
  x += dpp_row0<0x118>(x);
  return x;
}

// Eight sums over the 16 lanes of each row at once: a butterfly that halves the values a lane carries at each step
// (partners at lane distance xor 15, 7, 2, then 1, by DPP row_mirror, row_half_mirror and quad_perm), 15 exchanges
// instead of 8 separate reductions. Lane i of each row ends holding the row's total of a[(i >> 1) & 7].
PGN_DEVICE float row_totals16x8(const float (&a)[8], int i) {
  auto xch = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                                                 0xf, 0xf, false));
  };
  using mirror = std::integral_constant<int, 0x140>;
  using half_mirror = std::integral_constant<int, 0x141>;
  using swap2 = std::integral_constant<int, 0x4E>;
  using swap1 = std::integral_constant<int, 0xB1>;
  const bool b3 = i & 8, b2 = i & 4, b1 = i & 2;
  float s4[4], s2[2];
#pragma unroll
  for (int u = 0; u < 4; ++u)  // keep a[4 b3 + u], add the partner's copy of it
    s4[u] = (b3 ? a[4 + u] : a[u]) + xch(b3 ? a[u] : a[4 + u], mirror{});
#pragma unroll
  for (int u = 0; u < 2; ++u)
    s2[u] = (b2 ? s4[2 + u] : s4[u]) + xch(b2 ? s4[u] : s4[2 + u], half_mirror{});
  const float s1 = (b1 ? s2[1] : s2[0]) + xch(b1 ? s2[0] : s2[1], swap2{});
  return s1 + xch(s1, swap1{});
}

// Inclusive prefix sum over the 64 lanes of a wave (lane `l` = this lane's index): a Hillis-Steele scan inside each
// row of 16 lanes on DPP row shifts (row_shr 1, 2, 4, 8), then each row adds the totals of the rows before it, read
// from lanes 15, 31 and 47. Every step is a VALU or lane read: no LDS round trips.
PGN_DEVICE float wave_prefix_sum(float x, int l) {
  x += dpp_row0<0x111>(x);
  x += dpp_row0<0x112>(x);
  x += dpp_row0<0x114>(x);
  x += dpp_row0<0x118>(x);
  const float r0 = lane_value(x, 15), r1 = lane_value(x, 31), r2 = lane_value(x, 47);
  const int row = l >> 4;
  return x + ((row >= 1 ? r0 : 0.f) + (row >= 2 ? r1 : 0.f) + (row >= 3 ? r2 : 0.f));
}

// Inclusive suffix sum (lane l gets the sum over lanes l..63), the mirror image: row_shl shifts, then the totals of
// the later rows, read from lanes 16, 32 and 48.
PGN_DEVICE float wave_suffix_sum(float x, int l) {
  x += dpp_row0<0x101>(x);
  x += dpp_row0<0x102>(x);
  x += dpp_row0<0x104>(x);
  x += dpp_row0<0x108>(x);
  const float r1 = lane_value(x, 16), r2 = lane_value(x, 32), r3 = lane_value(x, 48);
  const int row = l >> 4;
  return x + ((row <= 2 ? r3 : 0.f) + (row <= 1 ? r2 : 0.f) + (row == 0 ? r1 : 0.f));
}

}  // namespace pgn
