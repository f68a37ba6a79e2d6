// Column sums of a row-major fp32 matrix, out[c] = sum_r x[r][c]: the last step of every parameter gradient the
// carrier's backward kernels leave as per-workgroup partial rows (LayerNorm weight and bias, the per-head RMSNorm
// weight, the rotation frequencies, the decay and gate biases). The reference gets these sums from autograd's
// reduction of the broadcast parameter; here one small launch replaces torch's column sum, which zeroes semaphores
// with a memset (a node that a captured HIP graph replays wrongly on this stack), and the ones-vector GEMM, whose fill
// and M = 1 GEMM cost ~10 us per sum.
//
// One workgroup of 16 waves per 64 columns; lane l of wave w sums column 64 blockIdx.x + l over rows w, w + 16, ...
// with eight independent accumulators (eight loads in flight per lane), then the 16 wave partials are added in LDS
// in wave order. The order of the terms is fixed by the shape alone, so the result is deterministic.
#include "common.h"

namespace {

constexpr int kWaves = 16;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(64 * kWaves) void colsum_f32(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                          float* __restrict__ out) {
  __shared__ float red[kWaves][64];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + l;
  float a[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) a[u] = 0.f;
  if (c < cols) {
    int64_t r = w;
    for (; r + (kUnroll - 1) * kWaves < rows; r += kUnroll * kWaves) {
      float v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = x[(r + u * kWaves) * cols + c];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) a[u] += v[u];
    }
    for (; r < rows; r += kWaves) a[0] += x[r * cols + c];
  }
  red[w][l] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  __syncthreads();
  if (w == 0 && c < cols) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) s += red[i][l];
    out[c] = s;
  }
}

}  // namespace

extern "C" int pragnosia_colsum_f32(const float* x, int64_t rows, int64_t cols, float* out, void* stream) {
  PGN_CHECK_ARG(x && out);
  PGN_CHECK_ARG(rows > 0 && cols > 0 && rows < ((int64_t)1 << 31) && cols < ((int64_t)1 << 31));
  PGN_CHECK_ARG(rows * cols < ((int64_t)1 << 40));
  hipLaunchKernelGGL(colsum_f32, dim3((unsigned)((cols + 63) / 64)), dim3(64 * kWaves), 0, (hipStream_t)stream, x,
                     rows, cols, out);
  PGN_RETURN_LAUNCH();
}
