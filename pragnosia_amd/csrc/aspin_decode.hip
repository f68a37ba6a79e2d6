// The associative carrier's single-token recurrent step (decode), fused: rebase, normalise, gate, write, read.
//
// Per (batch, head), from the T = 1 projections qp, kp, vp (64 channels each), the per-head log-decay la, the write
// gate logit (plain rule) or the write strength beta (delta rule), and the carried state S (keys on rows):
//     S' = R_keys(-p0 theta) S                          the rebase of `src/assoc.py:399-402`
//     q, k, v = unit(qp), unit(kp) [* sigmoid(g)], unit(vp)    positions restart at 0, so no rotation of q, k
//     plain:  S_new = a S' + k v^T
//     delta:  S_new = a S' + beta k (v - (a S')^T k)^T
//     o = S_new^T q
// with a = exp(la). This is the reference's T = 1 call of `AssocCarrier.forward`, which runs the two-pass torch form
// with chunk 1 (`src/assoc.py:411`, `:118-165`, `:207-251`); its graphed decode (`src/bench.py:241-317`) replays it.
//
// One workgroup of 256 threads per (batch, head): thread (j, rg) owns value column j and key rows 16rg..16rg+15, so a
// key-row pair is rotated in registers and the 16 KiB state moves HBM -> registers -> HBM once, coalesced (64 threads
// read each 256-byte row). The two reductions over key rows (the delta read and the output) go through LDS. The
// state may be updated in place (S_out == S): every element is read and written by the same thread.
#include "common.h"

namespace {

constexpr int D = 64;

// Where the step reads its inputs: separate (B, H, 64) projections and (B, H) gate / log-decay / strength arrays, or
// (FROM_P) one projection GEMV's output row per sequence, P[b] = [q (H 64) | k | v | decay logits (H) | gate or
// strength logits (H)], with the decay and the gate or strength formed here from their logits and biases as the
// chunked path's prep does: la = -softplus(logit + la_b) exp(A) (floored), gate logit + gate_b, beta =
// max(sigmoid(logit + beta_b), beta_min).
struct StepIn {
  const float* qp;
  const float* kp;
  const float* vp;
  const float* gl;
  const float* la;
  const float* beta;
  // FROM_P
  const float* P;
  int np;                 // row length of P
  int la_col, gate_col, beta_col;  // -1: absent
  const float* la_b;
  const float* A;
  const float* floor;
  const float* gate_b;
  const float* beta_b;
  float beta_min;
};

PGN_DEVICE float softplus_(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// With `on` (the per-head RMSNorm weight), the output is written normalised and token-major, o[b][h 64 + j] =
// (o_j r) on_j with r = 1 / sqrt(mean_j o_j^2 + eps) (nn.RMSNorm(dk), eps=None: fp32 epsilon; `src/assoc.py:505`);
// else o (B, H, 64) as computed. S and Sout may be the same array (the in-place update of the graphed decode), so
// neither is declared __restrict__: every element is read into registers before the thread that owns it stores it.
template <bool FROM_P>
__global__ __launch_bounds__(256) void aspin_decode(const float* S, float* Sout, StepIn in,
                                                    const float* __restrict__ theta, const float* __restrict__ p0d,
                                                    float p0h, const float* __restrict__ on, float on_eps,
                                                    float* __restrict__ o, int H) {
  __shared__ float qs[D], ks[D], vs[D];
  __shared__ float red[4][D];
  const int bh = blockIdx.x, h = bh % H, b = bh / H;
  const int tid = threadIdx.x, j = tid & 63, rg = tid >> 6;
  const size_t voff = (size_t)bh * D;
  const float* prow = FROM_P ? in.P + (size_t)b * in.np : nullptr;
  // the state slice, the rotation frequencies and p0 first: nothing below depends on them until the rotation, so
  // their latency overlaps the projections' loads and the normalisation
  const float* Sbh = S + (size_t)bh * D * D;
  float x[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) x[r] = Sbh[(16 * rg + r) * D + j];
  float thv[8];
#pragma unroll
  for (int pr = 0; pr < 8; ++pr) thv[pr] = theta[h * (D / 2) + 8 * rg + pr];
  const float p0 = p0d ? *p0d : p0h;

  float la_v, gl_v = 0.f, be_v = 0.f;
  bool has_g, has_b;
  if constexpr (FROM_P) {
    la_v = -softplus_(prow[in.la_col + h] + in.la_b[h]) * __expf(in.A[h]);
    if (in.floor) la_v = fmaxf(la_v, in.floor[h]);
    has_g = in.gate_col >= 0;
    has_b = in.beta_col >= 0;
    if (has_g) gl_v = prow[in.gate_col + h] + (in.gate_b ? in.gate_b[h] : 0.f);
    if (has_b) be_v = fmaxf(1.f / (1.f + __expf(-(prow[in.beta_col + h] + (in.beta_b ? in.beta_b[h] : 0.f)))),
                            in.beta_min);
  } else {
    la_v = in.la[bh];
    has_g = in.gl != nullptr;
    has_b = in.beta != nullptr;
    if (has_g) gl_v = in.gl[bh];
    if (has_b) be_v = in.beta[bh];
  }
  if (rg < 3) {
    float x;
    if constexpr (FROM_P)
      x = prow[rg * H * D + h * D + j];
    else
      x = (rg == 0 ? in.qp : (rg == 1 ? in.kp : in.vp))[voff + j];
    float n = x * x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) n += __shfl_xor(n, off);
    float inv = 1.f / fmaxf(sqrtf(n), 1e-12f);
    if (rg == 1 && has_g) inv *= 1.f / (1.f + __expf(-gl_v));
    (rg == 0 ? qs : (rg == 1 ? ks : vs))[j] = x * inv;
  }
  const float a = __expf(la_v);
#pragma unroll
  for (int pr = 0; pr < 8; ++pr) {
    float s, c;
    sincosf(-p0 * thv[pr], &s, &c);
    const float e = x[2 * pr], f = x[2 * pr + 1];
    x[2 * pr] = a * (e * c - f * s);
    x[2 * pr + 1] = a * (e * s + f * c);
  }
  __syncthreads();
  float wv = vs[j];
  if (has_b) {
    float r_ = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) r_ += ks[16 * rg + r] * x[r];
    red[rg][j] = r_;
    __syncthreads();
    const float rd = red[0][j] + red[1][j] + red[2][j] + red[3][j];
    wv = be_v * (wv - rd);
    __syncthreads();
  }
  float y = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    x[r] += ks[16 * rg + r] * wv;
    y += x[r] * qs[16 * rg + r];
  }
  red[rg][j] = y;
  float* Sob = Sout + (size_t)bh * D * D;
#pragma unroll
  for (int r = 0; r < 16; ++r) Sob[(16 * rg + r) * D + j] = x[r];
  __syncthreads();
  if (rg == 0) {
    const float ov = red[0][j] + red[1][j] + red[2][j] + red[3][j];
    if (on) {
      float ss = ov * ov;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
      const float rr = 1.f / sqrtf(ss * (1.f / D) + on_eps);
      o[(size_t)b * H * D + h * D + j] = (ov * rr) * on[j];
    } else {
      o[voff + j] = ov;
    }
  }
}

// The step for D = 64 or 128 with the work of a head split over D / 16 parts of 16 value columns (for latency: a
// one-token step is short, and D / 16 workgroups per head fill the chip at small batches): thread (jj, rg) of part
// `part` owns column 16 part + jj and key rows (D / 16) rg .. (D / 16) rg + D / 16 - 1 (D / 32 rotation pairs), holding
// them in x (loaded by the caller first, so their latency overlaps what follows) and ending with the new state there.
// `nt` is the thread's index within its part (the first 192 of a part's 256 threads normalise q, k and v; `norm`
// selects the part that does), red the part's 16 x 17 LDS block. Returns the thread's share of output column j (the
// sum over its rows of S_new[d][j] q[d]; the part's 16 row groups are added by the caller, red[.][jj] in order).
// Every thread of the workgroup calls this (barriers inside).
template <int DH>
PGN_DEVICE float split_step(float (&x)[DH / 16], const StepIn& in, const float* __restrict__ theta,
                            const float* __restrict__ p0d, float p0h, int H, int b, int h, int part, int nt,
                            bool norm, float* qs, float* ks, float* vs, float (*red)[17]) {
  constexpr int RT = DH / 16;  // key rows per thread
  const int jj = nt & 15, rg = nt >> 4;
  const int j = 16 * part + jj;
  const float* prow = in.P + (size_t)b * in.np;
  float th[RT / 2];
#pragma unroll
  for (int pr = 0; pr < RT / 2; ++pr) th[pr] = theta[h * (DH / 2) + (RT / 2) * rg + pr];
  const float p0 = p0d ? *p0d : p0h;
  const float la_logit = prow[in.la_col + h], la_b = in.la_b[h], Ah = in.A[h];
  const float fl = in.floor ? in.floor[h] : -INFINITY;
  const bool has_g = in.gate_col >= 0, has_b = in.beta_col >= 0;
  const float gl = has_g ? prow[in.gate_col + h] + (in.gate_b ? in.gate_b[h] : 0.f) : 0.f;
  const float bl = has_b ? prow[in.beta_col + h] + (in.beta_b ? in.beta_b[h] : 0.f) : 0.f;
  // q, k, v unit-normalised (k also gated) by waves 0, 1, 2, D / 64 channels a lane
  constexpr int CL = DH / 64;
  float xin[CL];
  if (norm && nt < 3 * 64) {
    const int vec = nt >> 6, l = nt & 63;
#pragma unroll
    for (int e = 0; e < CL; ++e) xin[e] = prow[vec * H * DH + h * DH + 64 * e + l];
    float n = 0.f;
#pragma unroll
    for (int e = 0; e < CL; ++e) n += xin[e] * xin[e];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) n += __shfl_xor(n, off);
    float inv = 1.f / fmaxf(sqrtf(n), 1e-12f);
    if (vec == 1 && has_g) inv *= 1.f / (1.f + __expf(-gl));
    float* dst = vec == 0 ? qs : (vec == 1 ? ks : vs);
#pragma unroll
    for (int e = 0; e < CL; ++e) dst[64 * e + l] = xin[e] * inv;
  }
  const float la_v = fmaxf(-softplus_(la_logit + la_b) * __expf(Ah), fl);
  const float a = __expf(la_v);
  const float be_v = has_b ? fmaxf(1.f / (1.f + __expf(-bl)), in.beta_min) : 0.f;
#pragma unroll
  for (int pr = 0; pr < RT / 2; ++pr) {
    float sn, cs;
    sincosf(-p0 * th[pr], &sn, &cs);
    const float e0 = x[2 * pr], f0 = x[2 * pr + 1];
    x[2 * pr] = a * (e0 * cs - f0 * sn);
    x[2 * pr + 1] = a * (e0 * sn + f0 * cs);
  }
  __syncthreads();
  float wv = vs[j];
  if (has_b) {
    float r_ = 0.f;
#pragma unroll
    for (int r = 0; r < RT; ++r) r_ += ks[RT * rg + r] * x[r];
    red[rg][jj] = r_;
    __syncthreads();
    float rd = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) rd += red[g][jj];
    wv = be_v * (wv - rd);
    __syncthreads();
  }
  float y = 0.f;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    x[r] += ks[RT * rg + r] * wv;
    y += x[r] * qs[RT * rg + r];
  }
  return y;
}

// The split step as D / 16 workgroups of 256 threads per head, raw output token-major o[b][h D + j] (the per-head
// RMSNorm is applied by the consumer, pragnosia_decode_gemv_rms or pragnosia_decode_gemm). Every global load (the
// state slice, the projections, theta, p0, the gate parameters) is issued at the start; the key-row reductions (the
// delta read and the output) go through LDS. A head's parts are numbered 8 apart, so they run on one XCD (workgroup i
// goes to XCD i mod 8) and the 128-byte lines of the state rows they share are fetched into one L2 only.
template <int DH>
__global__ __launch_bounds__(256) void aspin_decode_split(const float* S, float* Sout, StepIn in,
                                                          const float* __restrict__ theta,
                                                          const float* __restrict__ p0d, float p0h,
                                                          float* __restrict__ o, int H, int nbh) {
  constexpr int NP = DH / 16;  // parts per head (workgroups of 16 value columns)
  constexpr int RT = DH / 16;  // key rows per thread
  __shared__ float qs[DH], ks[DH], vs[DH];
  __shared__ float red[16][17];
  const int i = blockIdx.x, part = (i >> 3) % NP, bh = (i / (8 * NP)) * 8 + (i & 7);
  if (bh >= nbh) return;  // padding of the last group of 8 heads
  const int h = bh % H, b = bh / H;
  const int tid = threadIdx.x, jj = tid & 15, rg = tid >> 4;
  const int j = 16 * part + jj;
  const float* Sbh = S + (size_t)bh * DH * DH;
  float x[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) x[r] = Sbh[(RT * rg + r) * DH + j];
  const float y = split_step<DH>(x, in, theta, p0d, p0h, H, b, h, part, tid, true, qs, ks, vs, red);
  red[rg][jj] = y;
  float* Sob = Sout + (size_t)bh * DH * DH;
#pragma unroll
  for (int r = 0; r < RT; ++r) Sob[(RT * rg + r) * DH + j] = x[r];
  __syncthreads();
  if (rg == 0) {
    float ov = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) ov += red[g][jj];
    o[(size_t)b * H * DH + h * DH + j] = ov;
  }
}

// The step, the per-head RMSNorm and this head's share of the gated o-projection in one kernel (64-wide heads, at
// most a few sequences: the small-batch decode, where every launch is a fixed latency). Workgroup (b, h, slice) of
// 1024 threads runs head h's step as the split step's four parts side by side (part = thread / 256, the same
// operations: the new state is the split kernel's), sums each column's row groups, normalises the head's output
// (nn.RMSNorm(dk), `src/assoc.py:505`), then adds scale sum_j Wo[n][64 h + j] o_n[j] to y[b][n] for the kOprojRows
// rows n of its slice (scale: the gate's sigmoid, a device scalar): row n0 + (thread / 16), a 16-byte piece of W_o
// per thread (loaded first, with the state), the row's 16 pieces summed by lane exchange. Every slice reads the old
// state and slice 0 writes the new one to Sout, which must not be S. y holds the residual on entry; the heads'
// contributions are added with atomics in the order they arrive, so y is exact to fp32 rounding in some order of the
// heads, not the same bits from run to run.
constexpr int kOprojRows = 64;

__global__ __launch_bounds__(1024) void aspin_decode_oproj(const float* __restrict__ S, float* __restrict__ Sout,
                                                           StepIn in, const float* __restrict__ theta,
                                                           const float* __restrict__ p0d, float p0h,
                                                           const float* __restrict__ on, float on_eps,
                                                           const float* __restrict__ Wo, int N,
                                                           const float* __restrict__ scale, float* __restrict__ y,
                                                           int H, int NS) {
  constexpr int RT = 4;
  __shared__ float qs[D], ks[D], vs[D];
  __shared__ float red[4][16][17];
  __shared__ float onrm[D];
  const int slice = blockIdx.x % NS, bh = blockIdx.x / NS, h = bh % H, b = bh / H;
  const int tid = threadIdx.x, part = tid >> 8, nt = tid & 255, jj = nt & 15, rg = nt >> 4;
  const int j = 16 * part + jj;
  const float* Sbh = S + (size_t)bh * D * D;
  float x[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) x[r] = Sbh[(RT * rg + r) * D + j];
  // row n0 + tid / 16 of W_o, input columns 64 h + 4 (tid & 15) .. + 3 (rows past N read row N - 1, not added)
  const int n = slice * kOprojRows + (tid >> 4), c4 = tid & 15;
  const f32x4 w4 = *reinterpret_cast<const f32x4*>(Wo + (size_t)min(n, N - 1) * (H * D) + h * D + 4 * c4);
  const float yp = split_step<D>(x, in, theta, p0d, p0h, H, b, h, part, nt, part == 0, qs, ks, vs, red[part]);
  red[part][rg][jj] = yp;
  if (slice == 0) {
    float* Sob = Sout + (size_t)bh * D * D;
#pragma unroll
    for (int r = 0; r < RT; ++r) Sob[(RT * rg + r) * D + j] = x[r];
  }
  __syncthreads();
  if (tid < 64) {  // wave 0: lane j sums column j's row groups, then the head's RMSNorm
    const float(*rp)[17] = red[tid >> 4];
    float ov = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) ov += rp[g][tid & 15];
    float ss = ov * ov;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
    const float rr = 1.f / sqrtf(ss * (1.f / D) + on_eps);
    onrm[tid] = (ov * rr) * on[tid];
  }
  __syncthreads();
  const f32x4 o4 = *reinterpret_cast<const f32x4*>(onrm + 4 * c4);
  float acc = (w4[0] * o4[0] + w4[1] * o4[1]) + (w4[2] * o4[2] + w4[3] * o4[3]);
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off);
  if (c4 == 0 && n < N) atomicAdd(y + (size_t)b * N + n, (scale ? *scale : 1.f) * acc);
}

// The step for many heads (large batches), raw output, D = 64 or 128: one workgroup per (batch, head) and 16-byte
// state accesses. Thread (cq, rg) owns value columns 4 cq .. 4 cq + 3 (CQ = D / 4 quads) and key rows RPT rg .. RPT
// rg + RPT - 1 (RPT = D / (256 / CQ); key-row pairs rotate in registers), so a wave reads and writes whole 256-byte
// rows of the state with one instruction per row; the key-row sums (the delta read and the output) are lane
// exchanges within a wave, then one LDS step over the four waves. At 64 sequences x 12 heads the split form's 3,072
// workgroups of 4-byte accesses took 9.4 us a layer where an elementwise pass over the same state takes 4.2 us.
template <int DH>
__global__ __launch_bounds__(256) void aspin_decode_vec(const float* S, float* Sout, StepIn in,
                                                        const float* __restrict__ theta,
                                                        const float* __restrict__ p0d, float p0h,
                                                        float* __restrict__ o, int H) {
  constexpr int CQ = DH / 4, RG = 256 / CQ, RPT = DH / RG;
  __shared__ float qs[DH], ks[DH], vs[DH];
  __shared__ f32x4 redA[4][CQ], redB[4][CQ];
  const int bh = blockIdx.x, h = bh % H, b = bh / H;
  const int tid = threadIdx.x, cq = tid % CQ, rg = tid / CQ, w = tid >> 6, l = tid & 63;
  const float* prow = in.P + (size_t)b * in.np;
  const float* Sbh = S + (size_t)bh * DH * DH + 4 * cq;
  f32x4 x[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) x[r] = *reinterpret_cast<const f32x4*>(Sbh + (size_t)(RPT * rg + r) * DH);
  float th[RPT / 2];
#pragma unroll
  for (int pr = 0; pr < RPT / 2; ++pr) th[pr] = theta[h * (DH / 2) + (RPT / 2) * rg + pr];
  const float p0 = p0d ? *p0d : p0h;
  const float la_logit = prow[in.la_col + h], la_b = in.la_b[h], Ah = in.A[h];
  const float fl = in.floor ? in.floor[h] : -INFINITY;
  const bool has_g = in.gate_col >= 0, has_b = in.beta_col >= 0;
  const float gl = has_g ? prow[in.gate_col + h] + (in.gate_b ? in.gate_b[h] : 0.f) : 0.f;
  const float bl = has_b ? prow[in.beta_col + h] + (in.beta_b ? in.beta_b[h] : 0.f) : 0.f;
  // q, k, v unit-normalised (k also gated) by waves 0, 1, 2, D / 64 channels a lane
  constexpr int CL = DH / 64;
  if (w < 3) {
    float xin[CL];
#pragma unroll
    for (int e = 0; e < CL; ++e) xin[e] = prow[w * H * DH + h * DH + 64 * e + l];
    float n = 0.f;
#pragma unroll
    for (int e = 0; e < CL; ++e) n += xin[e] * xin[e];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) n += __shfl_xor(n, off);
    float inv = 1.f / fmaxf(sqrtf(n), 1e-12f);
    if (w == 1 && has_g) inv *= 1.f / (1.f + __expf(-gl));
    float* dst = w == 0 ? qs : (w == 1 ? ks : vs);
#pragma unroll
    for (int e = 0; e < CL; ++e) dst[64 * e + l] = xin[e] * inv;
  }
  const float a = __expf(fmaxf(-softplus_(la_logit + la_b) * __expf(Ah), fl));
  const float be_v = has_b ? fmaxf(1.f / (1.f + __expf(-bl)), in.beta_min) : 0.f;
#pragma unroll
  for (int pr = 0; pr < RPT / 2; ++pr) {
    float sn, cs;
    sincosf(-p0 * th[pr], &sn, &cs);
    const f32x4 e0 = x[2 * pr], f0 = x[2 * pr + 1];
    x[2 * pr] = a * (e0 * cs - f0 * sn);
    x[2 * pr + 1] = a * (e0 * sn + f0 * cs);
  }
  __syncthreads();
  // the sum over the wave's row groups (lane bits above the column quad), then over the four waves
  auto wave_rows = [&](f32x4 v) {
#pragma unroll
    for (int off = CQ; off < 64; off <<= 1)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += __shfl_xor(v[e], off);
    return v;
  };
  f32x4 wv = *reinterpret_cast<const f32x4*>(vs + 4 * cq);
  if (has_b) {
    f32x4 r4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; ++r) r4 += ks[RPT * rg + r] * x[r];
    r4 = wave_rows(r4);
    if (l < CQ) redA[w][cq] = r4;
    __syncthreads();
    const f32x4 rd = (redA[0][cq] + redA[1][cq]) + (redA[2][cq] + redA[3][cq]);
    wv = be_v * (wv - rd);
  }
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  float* Sob = Sout + (size_t)bh * DH * DH + 4 * cq;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    x[r] += ks[RPT * rg + r] * wv;
    y += x[r] * qs[RPT * rg + r];
    *reinterpret_cast<f32x4*>(Sob + (size_t)(RPT * rg + r) * DH) = x[r];
  }
  y = wave_rows(y);
  if (l < CQ) redB[w][cq] = y;
  __syncthreads();
  if (tid < CQ) {
    const f32x4 ov = (redB[0][cq] + redB[1][cq]) + (redB[2][cq] + redB[3][cq]);
    *reinterpret_cast<f32x4*>(o + (size_t)b * H * DH + h * DH + 4 * cq) = ov;
  }
}

}  // namespace

extern "C" int pragnosia_aspin_decode_step(const float* S, float* S_out, const float* qp, const float* kp,
                                           const float* vp, const float* gate, const float* la, const float* beta,
                                           const float* theta, const float* p0_dev, float p0, float* o, int64_t B,
                                           int64_t H, int64_t Dh, void* stream) {
  if (Dh != D) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(B > 0 && H > 0 && B * H < ((int64_t)1 << 31));
  PGN_CHECK_ARG(S && S_out && qp && kp && vp && la && theta && o);
  PGN_CHECK_ARG(!(gate && beta));
  StepIn in{};
  in.qp = qp;
  in.kp = kp;
  in.vp = vp;
  in.gl = gate;
  in.la = la;
  in.beta = beta;
  hipLaunchKernelGGL(aspin_decode<false>, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream, S, S_out, in,
                     theta, p0_dev, p0, nullptr, 0.f, o, (int)H);
  PGN_RETURN_LAUNCH();
}

// heads (batch x heads) from which the raw-output step runs one workgroup per head (aspin_decode_vec) rather than
// D / 16 (aspin_decode_split)
constexpr int64_t kVecHeads = 256;

extern "C" int pragnosia_aspin_decode_proj(const float* S, float* S_out, const float* P, int64_t np, int64_t la_col,
                                           int64_t gate_col, int64_t beta_col, const float* la_bias, const float* A,
                                           const float* la_floor, const float* gate_bias, const float* beta_bias,
                                           float beta_min, const float* theta, const float* p0_dev, float p0,
                                           const float* on_weight, float on_eps, float* o, int64_t B, int64_t H,
                                           int64_t Dh, void* stream) {
  // 64-wide heads with or without the fused RMSNorm; 128-wide heads with the raw output only
  if (!(Dh == D || (Dh == 2 * D && on_weight == nullptr))) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(B > 0 && H > 0 && B * H < ((int64_t)1 << 31));
  PGN_CHECK_ARG(S && S_out && P && la_bias && A && theta && o);
  PGN_CHECK_ARG(!(gate_col >= 0 && beta_col >= 0));
  PGN_CHECK_ARG(la_col >= 3 * H * Dh && la_col + H <= np && gate_col + H <= np && beta_col + H <= np);
  StepIn in{};
  in.P = P;
  in.np = (int)np;
  in.la_col = (int)la_col;
  in.gate_col = (int)gate_col;
  in.beta_col = (int)beta_col;
  in.la_b = la_bias;
  in.A = A;
  in.floor = la_floor;
  in.gate_b = gate_bias;
  in.beta_b = beta_bias;
  in.beta_min = beta_min;
  PGN_CHECK_ARG(B * H * 8 < ((int64_t)1 << 31));
  if (on_weight == nullptr && B * H >= kVecHeads) {  // raw output, many heads: one workgroup a head, 16-byte rows
    if (Dh == D)
      hipLaunchKernelGGL(aspin_decode_vec<64>, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream, S, S_out,
                         in, theta, p0_dev, p0, o, (int)H);
    else
      hipLaunchKernelGGL(aspin_decode_vec<128>, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream, S,
                         S_out, in, theta, p0_dev, p0, o, (int)H);
  } else if (on_weight == nullptr) {  // raw output, few heads: Dh / 16 workgroups per head
    if (Dh == D)
      hipLaunchKernelGGL(aspin_decode_split<64>, dim3((unsigned)((B * H + 7) / 8 * 32)), dim3(256), 0,
                         (hipStream_t)stream, S, S_out, in, theta, p0_dev, p0, o, (int)H, (int)(B * H));
    else
      hipLaunchKernelGGL(aspin_decode_split<128>, dim3((unsigned)((B * H + 7) / 8 * 64)), dim3(256), 0,
                         (hipStream_t)stream, S, S_out, in, theta, p0_dev, p0, o, (int)H, (int)(B * H));
  } else
    hipLaunchKernelGGL(aspin_decode<true>, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream, S, S_out, in,
                       theta, p0_dev, p0, on_weight, on_eps, o, (int)H);
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_aspin_decode_oproj(const float* S, float* S_out, const float* P, int64_t np, int64_t la_col,
                                            int64_t gate_col, int64_t beta_col, const float* la_bias, const float* A,
                                            const float* la_floor, const float* gate_bias, const float* beta_bias,
                                            float beta_min, const float* theta, const float* p0_dev, float p0,
                                            const float* on_weight, float on_eps, const float* Wo, int64_t N,
                                            const float* scale, float* y, int64_t B, int64_t H, int64_t Dh,
                                            void* stream) {
  if (Dh != D) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(B > 0 && H > 0 && N > 0);
  PGN_CHECK_ARG(S && S_out && S != S_out && P && la_bias && A && theta && on_weight && Wo && y);
  PGN_CHECK_ARG(!(gate_col >= 0 && beta_col >= 0));
  PGN_CHECK_ARG(la_col >= 3 * H * Dh && la_col + H <= np && gate_col + H <= np && beta_col + H <= np);
  const int64_t NS = (N + kOprojRows - 1) / kOprojRows;
  PGN_CHECK_ARG(B * H * NS < ((int64_t)1 << 31) && N * H * Dh < ((int64_t)1 << 31) && B * N < ((int64_t)1 << 31));
  PGN_CHECK_ARG((uintptr_t)Wo % 16 == 0);
  // every workgroup reads the old state while slice 0 writes the new one, and the atomics into y run while other
  // workgroups still read P: the byte ranges must not overlap
  const auto apart = [](const void* a, int64_t na, const void* b, int64_t nb) {
    const uintptr_t x = (uintptr_t)a, z = (uintptr_t)b;
    return x + (uintptr_t)na <= z || z + (uintptr_t)nb <= x;
  };
  const int64_t sbytes = B * H * Dh * Dh * (int64_t)sizeof(float);
  PGN_CHECK_ARG(apart(S, sbytes, S_out, sbytes));
  PGN_CHECK_ARG(apart(y, B * N * (int64_t)sizeof(float), P, B * np * (int64_t)sizeof(float)));
  PGN_CHECK_ARG(apart(y, B * N * (int64_t)sizeof(float), S, sbytes));
  StepIn in{};
  in.P = P;
  in.np = (int)np;
  in.la_col = (int)la_col;
  in.gate_col = (int)gate_col;
  in.beta_col = (int)beta_col;
  in.la_b = la_bias;
  in.A = A;
  in.floor = la_floor;
  in.gate_b = gate_bias;
  in.beta_b = beta_bias;
  in.beta_min = beta_min;
  hipLaunchKernelGGL(aspin_decode_oproj, dim3((unsigned)(B * H * NS)), dim3(1024), 0, (hipStream_t)stream, S, S_out,
                     in, theta, p0_dev, p0, on_weight, on_eps, Wo, (int)N, scale, y, (int)H, (int)NS);
  PGN_RETURN_LAUNCH();
}
