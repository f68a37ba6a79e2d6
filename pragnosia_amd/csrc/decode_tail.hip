// The end of one greedy decode step, in one kernel: what the reference's graphed generate does between the head and
// the next step's first layer (`src/bench.py:241-317`: argmax of the logits, the token appended, the position advanced
// modulo the position table, the next input x = tok_emb[tok] + pos_emb[pos]), plus this build's per-step device state
// (the generated-token buffer and its row counter, the carried states' position offsets reset to 1).
//
// One workgroup of 1024 threads per sequence b:
//   tok = argmax_v logits[b][v] (the first index among equal maxima, NaN above every number: torch.argmax's rule),
//   out[c][b] = tok (c = *ctr_in, row c of the generated-token buffer, skipped past its n_rows), tok_out[b] = tok,
//   p = (*pos_in + 1) mod ctx, h[b] = emb[tok] + pemb[p] (fp32, one add per element as torch's),
//   recorded logits (optional): lrec[c][b] = logits[b];
// workgroup 0 also writes *pos_out = p, *ctr_out = c + 1 and p0s[0 .. L - 1] = 1. The counter and the position are
// read from one buffer and written to another (the caller alternates the pair from step to step), so no workgroup
// reads a value another has already advanced, and a captured graph of an even number of steps replays where the last
// replay ended.
#include "common.h"

namespace {

// a better than b under torch.argmax's order: NaN above every number, then the larger value, then the smaller index
PGN_DEVICE bool better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

constexpr int kTailThreads = 1024;
constexpr int kTailLoads = 8;  // logits a thread loads before it compares any: one memory round trip per 8192

__global__ __launch_bounds__(kTailThreads) void decode_tail(const float* __restrict__ logits, int V,
                                                            const float* __restrict__ emb,
                                                            const float* __restrict__ pemb, int d, int ctx,
                                                            const int64_t* __restrict__ ctr_in,
                                                            int64_t* __restrict__ ctr_out,
                                                            const int64_t* __restrict__ pos_in,
                                                            int64_t* __restrict__ pos_out, int64_t* __restrict__ out,
                                                            int64_t n_rows, int64_t* __restrict__ tok_out,
                                                            float* __restrict__ h, float* __restrict__ p0s, int L,
                                                            float* __restrict__ lrec, int B) {
  constexpr int NW = kTailThreads / 64;
  __shared__ float bv_s[NW];
  __shared__ int bi_s[NW];
  __shared__ int tok_s;
  const int b = blockIdx.x, tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  const float* row = logits + (size_t)b * V;
  const int64_t c = *ctr_in;
  const bool rec = lrec && c < n_rows;
  // the next position and its embedding entry do not depend on the argmax: loaded with the logits, so only the token
  // embedding's load follows the reduction
  const int p = (int)((*pos_in + 1) % ctx);
  const float* pr = pemb + (size_t)p * d;
  const float pr0 = tid < d ? pr[tid] : 0.f;
  float bv = 0.f;
  int bi = -1;
  // kTailLoads logits a thread (v = v0 + tid + kTailThreads u), all loaded before any comparison, so a pass over
  // kTailThreads kTailLoads logits costs one memory round trip; each thread keeps the better of its values
  for (int v0 = 0; v0 < V; v0 += kTailThreads * kTailLoads) {
    float xs[kTailLoads];
#pragma unroll
    for (int u = 0; u < kTailLoads; ++u) {
      const int v = v0 + tid + kTailThreads * u;
      xs[u] = v < V ? row[v] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kTailLoads; ++u) {
      const int v = v0 + tid + kTailThreads * u;
      if (v < V) {
        if (bi < 0 || better(xs[u], v, bv, bi)) {
          bv = xs[u];
          bi = v;
        }
        if (rec) lrec[((size_t)c * B + b) * V + v] = xs[u];
      }
    }
  }
  // wave, then workgroup: (value, index) pairs, the better one kept
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || better(ov, oi, bv, bi))) {
      bv = ov;
      bi = oi;
    }
  }
  if (l == 0) {
    bv_s[w] = bv;
    bi_s[w] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int u = 1; u < NW; ++u)
      if (bi_s[u] >= 0 && (bi < 0 || better(bv_s[u], bi_s[u], bv, bi))) {
        bv = bv_s[u];
        bi = bi_s[u];
      }
    tok_s = bi;
    tok_out[b] = bi;
    if (c < n_rows) out[c * B + b] = bi;
  }
  __syncthreads();
  const int t = tok_s;
  const float* er = emb + (size_t)t * d;
  float* hr = h + (size_t)b * d;
  if (tid < d) hr[tid] = er[tid] + pr0;
  for (int k = tid + kTailThreads; k < d; k += kTailThreads) hr[k] = er[k] + pr[k];
  if (b == 0) {
    if (tid == 0) {
      *pos_out = p;
      *ctr_out = c + 1;
    }
    for (int k = tid; k < L; k += kTailThreads) p0s[k] = 1.f;
  }
}

}  // namespace

extern "C" int pragnosia_decode_tail(const float* logits, int64_t B, int64_t V, const float* emb, const float* pemb,
                                     int64_t d, int64_t ctx, const int64_t* ctr_in, int64_t* ctr_out,
                                     const int64_t* pos_in, int64_t* pos_out, int64_t* out, int64_t n_rows,
                                     int64_t* tok, float* h, float* p0s, int64_t L, float* logits_rec, void* stream) {
  PGN_CHECK_ARG(logits && emb && pemb && ctr_in && ctr_out && pos_in && pos_out && out && tok && h);
  PGN_CHECK_ARG(B > 0 && V > 0 && d > 0 && ctx > 0 && n_rows > 0 && L >= 0 && (L == 0 || p0s));
  PGN_CHECK_ARG(B < (1 << 20) && V < ((int64_t)1 << 30) && d < (1 << 30) && ctx < (1 << 30) && L < (1 << 30));
  PGN_CHECK_ARG(B * V < ((int64_t)1 << 40) && n_rows * B * V < ((int64_t)1 << 62));
  PGN_CHECK_ARG(ctr_in != ctr_out && pos_in != pos_out);
  hipLaunchKernelGGL(decode_tail, dim3((unsigned)B), dim3(kTailThreads), 0, (hipStream_t)stream, logits, (int)V, emb,
                     pemb, (int)d, (int)ctx, ctr_in, ctr_out, pos_in, pos_out, out, n_rows, tok, h, p0s, (int)L,
                     logits_rec, (int)B);
  PGN_RETURN_LAUNCH();
}
