// The plumbing between the carrier's projections and the scan, and the carried-state rebase.
//
// prep: per (batch, token, head) row of D = 64 or 128 channels: q, k, v are unit-normalised (x / max(|x|, 1e-12)), k is
// scaled by the write gate sigmoid(g) (plain rule; no gate for the delta rule), q and k are rotated by the angle
// pos_t * theta[h, i] on interleaved channel pairs (2i, 2i+1), and the three results are cast to bf16 and written in
// the scan's (B, H, T, D) layout from the projections' (B, T, H, D) layout (the reference's `_prep_fwd`,
// `src/assoc_kernel.py:740-769`; torch form `src/assoc.py:453-460`). The backward recomputes norms, gate and
// angles from the same inputs and uses the closed forms (u = x/|x|, r = R u, g the gradient on r):
//     du = R^T g,   dx = (du - u (u . du)) / |x|,   d(angle) = g2 r1 - g1 r2 per pair,
// writing the projections' gradients in THEIR layout, the gate's per (b, t, h), and theta's as one partial sum per
// (batch, 64-token block) that the caller reduces.
//
// One workgroup of 256 threads per (batch, head, 64-token block): D / 8 threads per row (eight channels, four rotation
// pairs each, one 16-byte access per tensor for bf16), 2048 / D rows per pass; the norms are D / 8-lane butterflies.
// The projections
// (and their gradients) may be column slices of one wider row per token (`in_stride` elements apart), such as one
// GEMM's output holding q, k, v and the gate logits side by side.
//
// rebase: S (B, H, D, D) with keys on dim 2; key rows (2i, 2i+1) are rotated by -p0 * theta[h, i] (the state written
// at positions up to p0 - 1, re-expressed for a window whose positions restart at 0: `src/assoc.py:399-402`).
#include "common.h"

namespace {

constexpr int TB = 64;    // tokens per workgroup

PGN_DEVICE float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

// softplus with torch's default threshold: x above 20 passes through
PGN_DEVICE float softplusf_(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// The decay, write gate and write strength taken from columns of the projections' rows (a single GEMM's output):
// per (b, t, h) the decay logit at acol[row + h], the gate logit at gcol[row + h] and the strength logit at
// bcol[row + h] (row = (b T + t) * S), each plus its bias. la = -softplus(logit + abias[h]) exp(A[h]), floored at
// floor[h] when given (`src/assoc.py:355-359`); the gate is sigmoid(logit + gbias[h]) (`src/assoc.py:458-459`); the
// delta rule's strength is beta = max(sigmoid(logit + bbias[h]), bmin) (`src/assoc.py:468`, bmin = 0.75 with
// write_all, else 0: no floor).
template <typename In>
struct Cols {
  const In* acol;       // decay logits, or NULL (then no la)
  const float* abias;   // (H)
  const float* A;       // (H) log-timescales
  const float* floor;   // (H) or NULL
  const In* gcol;       // gate logits, or NULL (then the separate fp32 gate, if any)
  const float* gbias;   // (H) or NULL
  const In* bcol;       // write-strength logits, or NULL (then no beta)
  const float* bbias;   // (H) or NULL
  float bmin;
};

// 8 consecutive channels of one row: one 16-byte access (bf16) or two (fp32)
template <typename T_>
PGN_DEVICE void ld8(const T_* p, float* x);
template <>
PGN_DEVICE void ld8<float>(const float* p, float* x) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = a[e];
    x[4 + e] = b[e];
  }
}
template <>
PGN_DEVICE void ld8<__bf16>(const __bf16* p, float* x) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)a[e];
}
template <typename T_>
PGN_DEVICE void st8(T_* p, const float* x);
template <>
PGN_DEVICE void st8<float>(float* p, const float* x) {
  *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
}
template <>
PGN_DEVICE void st8<__bf16>(__bf16* p, const float* x) {
  bf16x8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = (__bf16)x[e];
  *reinterpret_cast<bf16x8*>(p) = a;
}

// sum over the L lanes that share a row (lane bits 0 .. log2 L - 1)
template <int L>
PGN_DEVICE float sum_row(float x) {
#pragma unroll
  for (int o = 1; o < L; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

template <int L>
PGN_DEVICE float inv_norm8(const float* x) {
  float n = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) n += x[e] * x[e];
  return 1.f / fmaxf(sqrtf(sum_row<L>(n)), 1e-12f);
}

// Thread = (row slot rs = tid / LANES, channel group j = tid % LANES): channels 8 j .. 8 j + 7 of one row, i.e. the
// interleaved pairs 4 j .. 4 j + 3; LANES = D / 8 threads a row, SLOTS rows per pass.
template <int D>
struct RowSplit {
  static constexpr int LANES = D / 8;
  static constexpr int SLOTS = 256 / LANES;
};

template <typename In, int D>
__global__ __launch_bounds__(256) void prep_fwd(const In* __restrict__ qp, const In* __restrict__ kp,
                                                const In* __restrict__ vp, const float* __restrict__ gl,
                                                const float* __restrict__ theta, const int64_t* __restrict__ pos,
                                                __bf16* __restrict__ q, __bf16* __restrict__ k,
                                                __bf16* __restrict__ v, int T, int H, int ntb, int64_t S,
                                                Cols<In> cols, float* __restrict__ la,
                                                float* __restrict__ beta) {
  constexpr int LANES = RowSplit<D>::LANES, SLOTS = RowSplit<D>::SLOTS;
  const int blk = blockIdx.x;
  const int bh = blk / ntb, tb = blk - bh * ntb;
  const int b = bh / H, h = bh - b * H;
  const int j = threadIdx.x & (LANES - 1), rs = threadIdx.x / LANES;
  float th[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) th[u] = theta[h * (D / 2) + 4 * j + u];
  const float eA = cols.acol ? __expf(cols.A[h]) : 0.f;
#pragma unroll
  for (int p = 0; p < TB / SLOTS; ++p) {
    const int t = tb * TB + p * SLOTS + rs;
    if (t >= T) break;
    const size_t row = ((size_t)b * T + t) * S;
    const size_t in = row + h * D + 8 * j;
    const size_t out = ((size_t)bh * T + t) * D + 8 * j;
    float xq[8], xk[8], xv[8];
    ld8<In>(qp + in, xq);
    ld8<In>(kp + in, xk);
    ld8<In>(vp + in, xv);
    const float iq = inv_norm8<LANES>(xq), iv = inv_norm8<LANES>(xv);
    float ik = inv_norm8<LANES>(xk);
    if (cols.gcol)
      ik *= sigmoidf_((float)cols.gcol[row + h] + (cols.gbias ? cols.gbias[h] : 0.f));
    else if (gl)
      ik *= sigmoidf_(gl[((size_t)b * T + t) * H + h]);
    if (cols.acol && j == 0) {
      float l = -softplusf_((float)cols.acol[row + h] + cols.abias[h]) * eA;
      if (cols.floor) l = fmaxf(l, cols.floor[h]);
      la[(size_t)bh * T + t] = l;
    }
    if (cols.bcol && j == 0)
      beta[(size_t)bh * T + t] =
          fmaxf(sigmoidf_((float)cols.bcol[row + h] + (cols.bbias ? cols.bbias[h] : 0.f)), cols.bmin);
    const float pt = (float)pos[t];
    float oq[8], ok[8], ov[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float sn, cs;
      sincosf(pt * th[u], &sn, &cs);
      const float q1 = xq[2 * u], q2 = xq[2 * u + 1], k1 = xk[2 * u], k2 = xk[2 * u + 1];
      oq[2 * u] = (q1 * cs - q2 * sn) * iq;
      oq[2 * u + 1] = (q1 * sn + q2 * cs) * iq;
      ok[2 * u] = (k1 * cs - k2 * sn) * ik;
      ok[2 * u + 1] = (k1 * sn + k2 * cs) * ik;
      ov[2 * u] = xv[2 * u] * iv;
      ov[2 * u + 1] = xv[2 * u + 1] * iv;
    }
    st8<__bf16>(q + out, oq);
    st8<__bf16>(k + out, ok);
    st8<__bf16>(v + out, ov);
  }
}

// With columns (cols.acol / cols.gcol / cols.bcol), the decay, gate and strength gradients go to the same rows of the
// projections' gradient (dcol = the gradient buffer, same layout and stride): dlogit_a = dla mask (-exp(A))
// sigmoid(logit_a + b) (mask: the floor not active), dlogit_g = dsig sig (1 - sig), dlogit_b = dbeta mask sig (1 -
// sig) (mask: bmin not active); and one partial per workgroup of the three per-head sums (d gbias or d bbias,
// d abias, dA = sum dla mask la) to part, laid out (B, T blocks, H, 3) like the theta partials.
template <typename In, int D>
__global__ __launch_bounds__(256) void prep_bwd(
    const In* __restrict__ qp, const In* __restrict__ kp, const In* __restrict__ vp, const float* __restrict__ gl,
    const float* __restrict__ theta, const int64_t* __restrict__ pos, const __bf16* __restrict__ dq,
    const __bf16* __restrict__ dk, const __bf16* __restrict__ dv, In* __restrict__ dqp, In* __restrict__ dkp,
    In* __restrict__ dvp, float* __restrict__ dgl, float* __restrict__ dth, int T, int H, int ntb, int64_t S,
    Cols<In> cols, const float* __restrict__ dla, const float* __restrict__ dbeta, In* __restrict__ dcol,
    float* __restrict__ part) {
  constexpr int LANES = RowSplit<D>::LANES, SLOTS = RowSplit<D>::SLOTS;
  __shared__ float red[SLOTS][D / 2];
  __shared__ float red3[SLOTS][3];
  const int blk = blockIdx.x;
  const int bh = blk / ntb, tb = blk - bh * ntb;
  const int b = bh / H, h = bh - b * H;
  const int j = threadIdx.x & (LANES - 1), rs = threadIdx.x / LANES;
  float th[4], dth_acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u) th[u] = theta[h * (D / 2) + 4 * j + u];
  const float eA = cols.acol ? __expf(cols.A[h]) : 0.f;
  float dgb = 0.f, dab = 0.f, dA = 0.f;
#pragma unroll
  for (int p = 0; p < TB / SLOTS; ++p) {
    const int t = tb * TB + p * SLOTS + rs;
    if (t >= T) break;
    const size_t row = ((size_t)b * T + t) * S;
    const size_t in = row + h * D + 8 * j;
    if (cols.acol && j == 0) {
      const float x = (float)cols.acol[row + h] + cols.abias[h];
      const float l = -softplusf_(x) * eA;
      const float g = (cols.floor && l < cols.floor[h]) ? 0.f : dla[(size_t)bh * T + t];
      const float dx = -g * eA * sigmoidf_(x);
      dcol[row + (cols.acol - qp) + h] = (In)dx;
      dab += dx;
      dA += g * l;
    }
    if (cols.bcol && j == 0) {
      const float sb = sigmoidf_((float)cols.bcol[row + h] + (cols.bbias ? cols.bbias[h] : 0.f));
      const float db = sb < cols.bmin ? 0.f : dbeta[(size_t)bh * T + t] * sb * (1.f - sb);
      dcol[row + (cols.bcol - qp) + h] = (In)db;
      dgb += db;
    }
    const size_t out = ((size_t)bh * T + t) * D + 8 * j;
    const float pt = (float)pos[t];
    float sn[4], cs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) sincosf(pt * th[u], &sn[u], &cs[u]);
    float dang[4] = {0.f, 0.f, 0.f, 0.f};
    {  // q: normalise, rotate
      float x[8], g[8], du[8], o[8];
      ld8<In>(qp + in, x);
      ld8<__bf16>(dq + out, g);
      const float inv = inv_norm8<LANES>(x);
      float dot = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float u1 = x[2 * u] * inv, u2 = x[2 * u + 1] * inv, g1 = g[2 * u], g2 = g[2 * u + 1];
        dang[u] += g2 * (u1 * cs[u] - u2 * sn[u]) - g1 * (u1 * sn[u] + u2 * cs[u]);
        du[2 * u] = g1 * cs[u] + g2 * sn[u];
        du[2 * u + 1] = g2 * cs[u] - g1 * sn[u];
        dot += u1 * du[2 * u] + u2 * du[2 * u + 1];
      }
      dot = sum_row<LANES>(dot);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (du[e] - x[e] * inv * dot) * inv;
      st8<In>(dqp + in, o);
    }
    {  // k: normalise, gate, rotate
      float x[8], g[8], du[8], o[8], r[8];
      ld8<In>(kp + in, x);
      ld8<__bf16>(dk + out, g);
      const float inv = inv_norm8<LANES>(x);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float u1 = x[2 * u] * inv, u2 = x[2 * u + 1] * inv;
        r[2 * u] = u1 * cs[u] - u2 * sn[u];
        r[2 * u + 1] = u1 * sn[u] + u2 * cs[u];
      }
      if (cols.gcol || gl) {
        const float sg = cols.gcol ? sigmoidf_((float)cols.gcol[row + h] + (cols.gbias ? cols.gbias[h] : 0.f))
                                   : sigmoidf_(gl[((size_t)b * T + t) * H + h]);
        float dsg = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dsg += g[e] * r[e];
        dsg = sum_row<LANES>(dsg);
        if (j == 0) {
          const float dlg = dsg * sg * (1.f - sg);
          if (cols.gcol) {
            dcol[row + (cols.gcol - qp) + h] = (In)dlg;
            dgb += dlg;
          } else {
            dgl[((size_t)b * T + t) * H + h] = dlg;
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] *= sg;
      }
      float dot = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float g1 = g[2 * u], g2 = g[2 * u + 1];
        dang[u] += g2 * r[2 * u] - g1 * r[2 * u + 1];
        du[2 * u] = g1 * cs[u] + g2 * sn[u];
        du[2 * u + 1] = g2 * cs[u] - g1 * sn[u];
        dot += x[2 * u] * inv * du[2 * u] + x[2 * u + 1] * inv * du[2 * u + 1];
      }
      dot = sum_row<LANES>(dot);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (du[e] - x[e] * inv * dot) * inv;
      st8<In>(dkp + in, o);
    }
    {  // v: normalise
      float x[8], g[8], o[8];
      ld8<In>(vp + in, x);
      ld8<__bf16>(dv + out, g);
      const float inv = inv_norm8<LANES>(x);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += x[e] * inv * g[e];
      dot = sum_row<LANES>(dot);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (g[e] - x[e] * inv * dot) * inv;
      st8<In>(dvp + in, o);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) dth_acc[u] += dang[u] * pt;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) red[rs][4 * j + u] = dth_acc[u];
  if (j == 0) {
    red3[rs][0] = dgb;
    red3[rs][1] = dab;
    red3[rs][2] = dA;
  }
  __syncthreads();
  if (threadIdx.x < D / 2) {
    float a = 0.f;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) a += red[r][threadIdx.x];
    dth[(((size_t)b * ntb + tb) * H + h) * (D / 2) + threadIdx.x] = a;
  }
  if (part && threadIdx.x < 3) {
    float a = 0.f;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) a += red3[r][threadIdx.x];
    part[(((size_t)b * ntb + tb) * H + h) * 3 + threadIdx.x] = a;
  }
}

// rebase: one workgroup of 256 threads per (batch, head); thread = (value column j of each 64-column half, group rg
// of D / 4 key rows, i.e. D / 8 rotation pairs)
template <int D>
__global__ __launch_bounds__(256) void rebase_fwd(const float* __restrict__ S, const float* __restrict__ theta,
                                                  const float* __restrict__ p0d, float p0h, float* __restrict__ So,
                                                  int H) {
  constexpr int NP = D / 8;  // rotation pairs per thread
  const int bh = blockIdx.x, h = bh % H;
  const int j = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const float p0 = p0d ? *p0d : p0h;
  const float* src = S + (size_t)bh * D * D;
  float* dst = So + (size_t)bh * D * D;
  float sn[NP], cs[NP];
#pragma unroll
  for (int pr = 0; pr < NP; ++pr) sincosf(-p0 * theta[h * (D / 2) + NP * rg + pr], &sn[pr], &cs[pr]);
#pragma unroll
  for (int ch = 0; ch < D / 64; ++ch) {
    const int col = 64 * ch + j;
    float x[2 * NP];
#pragma unroll
    for (int r = 0; r < 2 * NP; ++r) x[r] = src[(2 * NP * rg + r) * D + col];
#pragma unroll
    for (int pr = 0; pr < NP; ++pr) {
      const int ip = NP * rg + pr;
      const float a = x[2 * pr], bb = x[2 * pr + 1];
      dst[(2 * ip) * D + col] = a * cs[pr] - bb * sn[pr];
      dst[(2 * ip + 1) * D + col] = a * sn[pr] + bb * cs[pr];
    }
  }
}

// backward of rebase: dS = R^T g; d(angle) = g2 r1 - g1 r2 summed over value columns, times -p0 for theta
template <int D>
__global__ __launch_bounds__(256) void rebase_bwd(const float* __restrict__ S, const float* __restrict__ theta,
                                                  const float* __restrict__ p0d, float p0h,
                                                  const float* __restrict__ g, float* __restrict__ dS,
                                                  float* __restrict__ dth, int H) {
  constexpr int NP = D / 8;
  __shared__ float red[4][64][NP + 1];
  const int bh = blockIdx.x, h = bh % H;
  const int j = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const float p0 = p0d ? *p0d : p0h;
  const size_t off = (size_t)bh * D * D;
#pragma unroll
  for (int pr = 0; pr < NP; ++pr) {
    const int ip = NP * rg + pr;
    float s, c;
    sincosf(-p0 * theta[h * (D / 2) + ip], &s, &c);
    float acc = 0.f;
#pragma unroll
    for (int ch = 0; ch < D / 64; ++ch) {
      const int col = 64 * ch + j;
      const float a = S[off + (2 * ip) * D + col], bb = S[off + (2 * ip + 1) * D + col];
      const float g1 = g[off + (2 * ip) * D + col], g2 = g[off + (2 * ip + 1) * D + col];
      const float r1 = a * c - bb * s, r2 = a * s + bb * c;
      if (dS) {
        dS[off + (2 * ip) * D + col] = g1 * c + g2 * s;
        dS[off + (2 * ip + 1) * D + col] = g2 * c - g1 * s;
      }
      acc += g2 * r1 - g1 * r2;
    }
    red[rg][j][pr] = acc * (-p0);
  }
  __syncthreads();
  if (dth && threadIdx.x < D / 2) {
    const int ip = threadIdx.x, rgi = ip / NP, pr = ip % NP;
    float acc = 0.f;
    for (int jj = 0; jj < 64; ++jj) acc += red[rgi][jj][pr];
    dth[(size_t)bh * (D / 2) + ip] = acc;
  }
}

bool shape_ok(int64_t B, int64_t T, int64_t H) {
  return B > 0 && T > 0 && H > 0 && B * H * ((T + TB - 1) / TB) < ((int64_t)1 << 31) && B * T * H < ((int64_t)1 << 40);
}

}  // namespace

namespace {

bool width_ok(int64_t Dh) { return Dh == 64 || Dh == 128; }

// the launches at head width D (64 or 128), input type In
template <typename In, int D>
void launch_prep_fwd(dim3 grid, hipStream_t st, const In* qp, const In* kp, const In* vp, const float* gate,
                     const float* theta, const int64_t* pos, void* q, void* k, void* v, int T, int H, int ntb,
                     int64_t stride, Cols<In> cols, float* la, float* beta) {
  hipLaunchKernelGGL((prep_fwd<In, D>), grid, dim3(256), 0, st, qp, kp, vp, gate, theta, pos, (__bf16*)q, (__bf16*)k,
                     (__bf16*)v, T, H, ntb, stride, cols, la, beta);
}

template <typename In, int D>
void launch_prep_bwd(dim3 grid, hipStream_t st, const In* qp, const In* kp, const In* vp, const float* gate,
                     const float* theta, const int64_t* pos, const void* dq, const void* dk, const void* dv, In* dqp,
                     In* dkp, In* dvp, float* dgate, float* dth, int T, int H, int ntb, int64_t stride, Cols<In> cols,
                     const float* dla, const float* dbeta, In* dcol, float* part) {
  hipLaunchKernelGGL((prep_bwd<In, D>), grid, dim3(256), 0, st, qp, kp, vp, gate, theta, pos, (const __bf16*)dq,
                     (const __bf16*)dk, (const __bf16*)dv, dqp, dkp, dvp, dgate, dth, T, H, ntb, stride, cols, dla,
                     dbeta, dcol, part);
}

template <typename In>
void prep_fwd_any(int64_t Dh, dim3 grid, hipStream_t st, const In* qp, const In* kp, const In* vp, const float* gate,
                  const float* theta, const int64_t* pos, void* q, void* k, void* v, int T, int H, int ntb,
                  int64_t stride, Cols<In> cols, float* la, float* beta) {
  if (Dh == 64)
    launch_prep_fwd<In, 64>(grid, st, qp, kp, vp, gate, theta, pos, q, k, v, T, H, ntb, stride, cols, la, beta);
  else
    launch_prep_fwd<In, 128>(grid, st, qp, kp, vp, gate, theta, pos, q, k, v, T, H, ntb, stride, cols, la, beta);
}

template <typename In>
void prep_bwd_any(int64_t Dh, dim3 grid, hipStream_t st, const In* qp, const In* kp, const In* vp, const float* gate,
                  const float* theta, const int64_t* pos, const void* dq, const void* dk, const void* dv, In* dqp,
                  In* dkp, In* dvp, float* dgate, float* dth, int T, int H, int ntb, int64_t stride, Cols<In> cols,
                  const float* dla, const float* dbeta, In* dcol, float* part) {
  if (Dh == 64)
    launch_prep_bwd<In, 64>(grid, st, qp, kp, vp, gate, theta, pos, dq, dk, dv, dqp, dkp, dvp, dgate, dth, T, H, ntb,
                            stride, cols, dla, dbeta, dcol, part);
  else
    launch_prep_bwd<In, 128>(grid, st, qp, kp, vp, gate, theta, pos, dq, dk, dv, dqp, dkp, dvp, dgate, dth, T, H,
                             ntb, stride, cols, dla, dbeta, dcol, part);
}

}  // namespace

extern "C" int pragnosia_aspin_prep_fwd(const void* qp, const void* kp, const void* vp, const float* gate,
                                        const float* theta, const int64_t* pos, void* q, void* k, void* v,
                                        int64_t B, int64_t T, int64_t H, int64_t Dh, int64_t in_stride, int in_bf16,
                                        void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, T, H));
  PGN_CHECK_ARG(qp && kp && vp && theta && pos && q && k && v && in_stride >= H * Dh);
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  hipStream_t st = (hipStream_t)stream;
  if (in_bf16)
    prep_fwd_any<__bf16>(Dh, grid, st, (const __bf16*)qp, (const __bf16*)kp, (const __bf16*)vp, gate, theta, pos, q, k,
                         v, (int)T, (int)H, ntb, in_stride, Cols<__bf16>{}, nullptr, nullptr);
  else
    prep_fwd_any<float>(Dh, grid, st, (const float*)qp, (const float*)kp, (const float*)vp, gate, theta, pos, q, k, v,
                        (int)T, (int)H, ntb, in_stride, Cols<float>{}, nullptr, nullptr);
  PGN_RETURN_LAUNCH();
}

extern "C" int64_t pragnosia_aspin_prep_theta_partials(int64_t B, int64_t T) { return B * ((T + TB - 1) / TB); }

extern "C" int pragnosia_aspin_prep_bwd(const void* qp, const void* kp, const void* vp, const float* gate,
                                        const float* theta, const int64_t* pos, const void* dq, const void* dk,
                                        const void* dv, void* dqp, void* dkp, void* dvp, float* dgate,
                                        float* dtheta_partial, int64_t B, int64_t T, int64_t H, int64_t Dh,
                                        int64_t in_stride, int in_bf16, void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, T, H));
  PGN_CHECK_ARG(qp && kp && vp && theta && pos && dq && dk && dv && dqp && dkp && dvp && dtheta_partial);
  PGN_CHECK_ARG(in_stride >= H * Dh);
  PGN_CHECK_ARG(gate == nullptr || dgate != nullptr);
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  hipStream_t st = (hipStream_t)stream;
  if (in_bf16)
    prep_bwd_any<__bf16>(Dh, grid, st, (const __bf16*)qp, (const __bf16*)kp, (const __bf16*)vp, gate, theta, pos, dq,
                         dk, dv, (__bf16*)dqp, (__bf16*)dkp, (__bf16*)dvp, dgate, dtheta_partial, (int)T, (int)H, ntb,
                         in_stride, Cols<__bf16>{}, nullptr, nullptr, nullptr, nullptr);
  else
    prep_bwd_any<float>(Dh, grid, st, (const float*)qp, (const float*)kp, (const float*)vp, gate, theta, pos, dq, dk,
                        dv, (float*)dqp, (float*)dkp, (float*)dvp, dgate, dtheta_partial, (int)T, (int)H, ntb,
                        in_stride, Cols<float>{}, nullptr, nullptr, nullptr, nullptr);
  PGN_RETURN_LAUNCH();
}

namespace {

// the H-column groups at la_col (required), gate_col and beta_col (each optional: -1) lie past q, k, v, inside the
// row, and do not overlap; a row has a gate or a strength, not both
bool proj_cols_ok(int64_t H, int64_t Dh, int64_t stride, int64_t la_col, int64_t gate_col, int64_t beta_col) {
  const int64_t hd = H * Dh;
  if (stride < 3 * hd || la_col < 3 * hd || la_col + H > stride) return false;
  if (gate_col >= 0 && beta_col >= 0) return false;
  const int64_t x = gate_col >= 0 ? gate_col : beta_col;
  if (x >= 0 && (x < 3 * hd || x + H > stride || (x < la_col + H && la_col < x + H))) return false;
  return true;
}

template <typename In>
Cols<In> proj_cols(const void* P, int64_t la_col, int64_t gate_col, int64_t beta_col, const float* la_bias,
                   const float* A, const float* la_floor, const float* gate_bias, const float* beta_bias,
                   float beta_min) {
  const In* base = (const In*)P;
  return Cols<In>{base + la_col, la_bias, A, la_floor, gate_col >= 0 ? base + gate_col : nullptr, gate_bias,
                  beta_col >= 0 ? base + beta_col : nullptr, beta_bias, beta_min};
}

}  // namespace

extern "C" int pragnosia_aspin_prep_proj_fwd(const void* P, int64_t stride, int64_t la_col, int64_t gate_col,
                                             int64_t beta_col, const float* la_bias, const float* A,
                                             const float* la_floor, const float* gate_bias, const float* beta_bias,
                                             float beta_min, const float* theta, const int64_t* pos, void* q,
                                             void* k, void* v, float* la, float* beta, int64_t B, int64_t T,
                                             int64_t H, int64_t Dh, int in_bf16, void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, T, H));
  PGN_CHECK_ARG(P && la_bias && A && theta && pos && q && k && v && la && (beta_col < 0 || beta));
  PGN_CHECK_ARG(proj_cols_ok(H, Dh, stride, la_col, gate_col, beta_col));
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  const int64_t hd = H * Dh;
  hipStream_t st = (hipStream_t)stream;
  if (in_bf16) {
    const __bf16* p = (const __bf16*)P;
    prep_fwd_any<__bf16>(Dh, grid, st, p, p + hd, p + 2 * hd, nullptr, theta, pos, q, k, v, (int)T, (int)H, ntb,
                         stride, proj_cols<__bf16>(P, la_col, gate_col, beta_col, la_bias, A, la_floor, gate_bias,
                                                   beta_bias, beta_min),
                         la, beta);
  } else {
    const float* p = (const float*)P;
    prep_fwd_any<float>(Dh, grid, st, p, p + hd, p + 2 * hd, nullptr, theta, pos, q, k, v, (int)T, (int)H, ntb,
                        stride, proj_cols<float>(P, la_col, gate_col, beta_col, la_bias, A, la_floor, gate_bias,
                                                 beta_bias, beta_min),
                        la, beta);
  }
  PGN_RETURN_LAUNCH();
}

extern "C" int64_t pragnosia_aspin_prep_proj_partials(int64_t B, int64_t T, int64_t H) {
  if (!shape_ok(B, T, H)) return -1;
  return B * H * ((T + TB - 1) / TB);
}

extern "C" int pragnosia_aspin_prep_proj_bwd(const void* P, int64_t stride, int64_t la_col, int64_t gate_col,
                                             int64_t beta_col, const float* la_bias, const float* A,
                                             const float* la_floor, const float* gate_bias, const float* beta_bias,
                                             float beta_min, const float* theta, const int64_t* pos,
                                             const void* dq, const void* dk, const void* dv, const float* dla,
                                             const float* dbeta, void* dP, float* dtheta_partial, float* part,
                                             int64_t B, int64_t T, int64_t H, int64_t Dh, int in_bf16,
                                             void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(shape_ok(B, T, H));
  PGN_CHECK_ARG(P && la_bias && A && theta && pos && dq && dk && dv && dla && dP && dtheta_partial && part);
  PGN_CHECK_ARG(beta_col < 0 || dbeta);
  PGN_CHECK_ARG(proj_cols_ok(H, Dh, stride, la_col, gate_col, beta_col) && P != dP);
  const int ntb = (int)((T + TB - 1) / TB);
  const dim3 grid((unsigned)(B * H * ntb));
  const int64_t hd = H * Dh;
  hipStream_t st = (hipStream_t)stream;
  if (in_bf16) {
    const __bf16* p = (const __bf16*)P;
    __bf16* d = (__bf16*)dP;
    prep_bwd_any<__bf16>(Dh, grid, st, p, p + hd, p + 2 * hd, nullptr, theta, pos, dq, dk, dv, d, d + hd, d + 2 * hd,
                         nullptr, dtheta_partial, (int)T, (int)H, ntb, stride,
                         proj_cols<__bf16>(P, la_col, gate_col, beta_col, la_bias, A, la_floor, gate_bias, beta_bias,
                                           beta_min),
                         dla, dbeta, d, part);
  } else {
    const float* p = (const float*)P;
    float* d = (float*)dP;
    prep_bwd_any<float>(Dh, grid, st, p, p + hd, p + 2 * hd, nullptr, theta, pos, dq, dk, dv, d, d + hd, d + 2 * hd,
                        nullptr, dtheta_partial, (int)T, (int)H, ntb, stride,
                        proj_cols<float>(P, la_col, gate_col, beta_col, la_bias, A, la_floor, gate_bias, beta_bias,
                                         beta_min),
                        dla, dbeta, d, part);
  }
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_aspin_rebase_fwd(const float* S, const float* theta, const float* p0_dev, float p0,
                                          float* S_out, int64_t B, int64_t H, int64_t Dh, void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(B > 0 && H > 0 && B * H < ((int64_t)1 << 31));
  PGN_CHECK_ARG(S && theta && S_out && S != S_out);
  hipStream_t st = (hipStream_t)stream;
  if (Dh == 64)
    hipLaunchKernelGGL(rebase_fwd<64>, dim3((unsigned)(B * H)), dim3(256), 0, st, S, theta, p0_dev, p0, S_out, (int)H);
  else
    hipLaunchKernelGGL(rebase_fwd<128>, dim3((unsigned)(B * H)), dim3(256), 0, st, S, theta, p0_dev, p0, S_out,
                       (int)H);
  PGN_RETURN_LAUNCH();
}

extern "C" int pragnosia_aspin_rebase_bwd(const float* S, const float* theta, const float* p0_dev, float p0,
                                          const float* dS_out, float* dS, float* dtheta_partial, int64_t B,
                                          int64_t H, int64_t Dh, void* stream) {
  if (!width_ok(Dh)) return PRAGNOSIA_ERR_UNSUPPORTED;
  PGN_CHECK_ARG(B > 0 && H > 0 && B * H < ((int64_t)1 << 31));
  PGN_CHECK_ARG(S && theta && dS_out);
  hipStream_t st = (hipStream_t)stream;
  if (Dh == 64)
    hipLaunchKernelGGL(rebase_bwd<64>, dim3((unsigned)(B * H)), dim3(256), 0, st, S, theta, p0_dev, p0, dS_out, dS,
                       dtheta_partial, (int)H);
  else
    hipLaunchKernelGGL(rebase_bwd<128>, dim3((unsigned)(B * H)), dim3(256), 0, st, S, theta, p0_dev, p0, dS_out, dS,
                       dtheta_partial, (int)H);
  PGN_RETURN_LAUNCH();
}
