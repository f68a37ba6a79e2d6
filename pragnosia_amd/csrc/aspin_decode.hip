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

__global__ __launch_bounds__(256) void aspin_decode(const float* __restrict__ S, float* __restrict__ Sout,
                                                    const float* __restrict__ qp, const float* __restrict__ kp,
                                                    const float* __restrict__ vp, const float* __restrict__ gl,
                                                    const float* __restrict__ la, const float* __restrict__ beta,
                                                    const float* __restrict__ theta, const float* __restrict__ p0d,
                                                    float p0h, float* __restrict__ o, int H) {
  __shared__ float qs[D], ks[D], vs[D];
  __shared__ float red[4][D];
  const int bh = blockIdx.x, h = bh % H;
  const int tid = threadIdx.x, j = tid & 63, rg = tid >> 6;
  const size_t voff = (size_t)bh * D;

  if (rg < 3) {
    const float* src = rg == 0 ? qp : (rg == 1 ? kp : vp);
    const float x = src[voff + j];
    float n = x * x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) n += __shfl_xor(n, off);
    float inv = 1.f / fmaxf(sqrtf(n), 1e-12f);
    if (rg == 1 && gl) inv *= 1.f / (1.f + __expf(-gl[bh]));
    (rg == 0 ? qs : (rg == 1 ? ks : vs))[j] = x * inv;
  }
  const float p0 = p0d ? *p0d : p0h;
  const float a = __expf(la[bh]);
  const float* Sbh = S + (size_t)bh * D * D;
  float x[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) x[r] = Sbh[(16 * rg + r) * D + j];
#pragma unroll
  for (int pr = 0; pr < 8; ++pr) {
    float s, c;
    sincosf(-p0 * theta[h * (D / 2) + 8 * rg + pr], &s, &c);
    const float e = x[2 * pr], f = x[2 * pr + 1];
    x[2 * pr] = a * (e * c - f * s);
    x[2 * pr + 1] = a * (e * s + f * c);
  }
  __syncthreads();
  float wv = vs[j];
  if (beta) {
    float r_ = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) r_ += ks[16 * rg + r] * x[r];
    red[rg][j] = r_;
    __syncthreads();
    const float rd = red[0][j] + red[1][j] + red[2][j] + red[3][j];
    wv = beta[bh] * (wv - rd);
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
  if (rg == 0) o[voff + j] = red[0][j] + red[1][j] + red[2][j] + red[3][j];
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
  hipLaunchKernelGGL(aspin_decode, dim3((unsigned)(B * H)), dim3(256), 0, (hipStream_t)stream, S, S_out, qp, kp, vp,
                     gate, la, beta, theta, p0_dev, p0, o, (int)H);
  PGN_RETURN_LAUNCH();
}
