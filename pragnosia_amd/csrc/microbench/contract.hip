// LDS-resident contraction microbenchmark: the MFMA throughput of the operand patterns the aspin kernels use, with
// every operand already on chip (no HBM traffic, no chunk chain). It bounds what the contraction phases of the scan
// kernels could reach if nothing else limited them, and so corroborates their MFMA-utilisation figures.
//
// Each wave runs `iters` iterations of 16 bf16 MFMAs (v_mfma_f32_16x16x32_bf16, 16,384 flop each) into 8
// independent accumulators. Variants:
//   0  both operands in registers: the MFMA pipe alone
//   1  one operand read from an LDS tile per MFMA (the kernels' pattern: 8-byte reads at a 68-element pitch)
//   2  as 1, and half of the MFMAs take their second operand from the packed (bf16) result of an earlier MFMA, the
//      accumulator-to-operand chain the kernels use (scores -> decayed block -> next product)
//   3-5 the same three patterns on v_mfma_f32_32x32x16_bf16 (32,768 flop each, 8 per iteration into 4 accumulators
//      of 16 values): one operand fragment (16 bytes a lane) feeds twice the flop, so an LDS-operand product reads
//      half the LDS bytes per flop of the 16 x 16 x 32 form
// Operand values are a fixed pseudo-random fill; the accumulators' sum is written out so nothing is dropped.
#include "../mfma_tile.h"

using namespace pgn;

namespace {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

PGN_DEVICE f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// the 32 x 32 x 16 forms: lane l holds row l % 32 and k group l / 32 of an operand
template <int VARIANT>
__global__ __launch_bounds__(1024) void contract32(int iters, float* __restrict__ out) {
  __shared__ __align__(16) __bf16 tile[128 * kPitch];
  const WaveIdx x = wave_idx();
  const int l = x.l, r32 = l & 31, kg = l >> 5;
  for (int e = threadIdx.x; e < 128 * kPitch; e += blockDim.x)
    tile[e] = (__bf16)((float)((e * 2654435761u) >> 24) * (1.f / 256.f) - 0.5f);
  __syncthreads();
  bf16x8 a0 = frag(tile, r32, 0, kg), a1 = frag(tile, 32 + r32, 1, kg);
  f32x16 acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[u][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
    const int r0 = (it * 5 + x.w * 3) & 31;
    if constexpr (VARIANT == 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] = mfma32(a0, a1, acc[u]);
        acc[u] = mfma32(a1, a0, acc[u]);
      }
      a0 = __builtin_shufflevector(a0, a0, 1, 2, 3, 4, 5, 6, 7, 0);
    } else if constexpr (VARIANT == 1) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] = mfma32(a0, frag(tile, 32 * (u & 1) + ((r0 + r32) & 31), 0, kg), acc[u]);
        acc[u] = mfma32(a1, frag(tile, 32 * (u & 1) + ((r0 + r32) & 31), 1, kg), acc[u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
        acc[u] = mfma32(a0, frag(tile, 32 * (u >> 1) + ((r0 + r32) & 31), 0, kg), acc[u]);
        acc[u] = mfma32(a1, frag(tile, 32 * (u >> 1) + ((r0 + r32) & 31), 1, kg), acc[u]);
        f32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = acc[u][e] * 0.5f;
          hi[e] = acc[u][4 + e] * 0.25f;
        }
        const bf16x8 p = pack(lo, hi);
        acc[u + 1] = mfma32(frag(tile, 64 + ((r0 + r32) & 31), 0, kg), p, acc[u + 1]);
        acc[u + 1] = mfma32(frag(tile, 64 + ((r0 + r32) & 31), 1, kg), p, acc[u + 1]);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[u][e];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int VARIANT>
__global__ __launch_bounds__(1024) void contract(int iters, float* __restrict__ out) {
  __shared__ __align__(16) __bf16 tile[128 * kPitch];
  const WaveIdx x = wave_idx();
  const int g = x.g, i = x.i;
  for (int e = threadIdx.x; e < 128 * kPitch; e += blockDim.x)
    tile[e] = (__bf16)((float)((e * 2654435761u) >> 24) * (1.f / 256.f) - 0.5f);
  __syncthreads();
  bf16x8 a0 = frag(tile, i, 0, g), a1 = frag(tile, 16 + i, 1, g);
  f32x4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = zero4();
  for (int it = 0; it < iters; ++it) {
    const int r0 = (it * 5 + x.w * 3) & 15;
    if constexpr (VARIANT == 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc[u] = pgn_mfma(a0, a1, acc[u]);
        acc[u] = pgn_mfma(a1, a0, acc[u]);
      }
      a0 = __builtin_shufflevector(a0, a0, 1, 2, 3, 4, 5, 6, 7, 0);
    } else if constexpr (VARIANT == 1) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc[u] = pgn_mfma(a0, frag(tile, 16 * (u & 3) + ((r0 + i) & 15), 0, g), acc[u]);
        acc[u] = pgn_mfma(a1, frag(tile, 16 * (u & 3) + ((r0 + i) & 15), 1, g), acc[u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 8; u += 2) {
        acc[u] = pgn_mfma(a0, frag(tile, 16 * (u & 3) + ((r0 + i) & 15), 0, g), acc[u]);
        acc[u] = pgn_mfma(a1, frag(tile, 16 * (u & 3) + ((r0 + i) & 15), 1, g), acc[u]);
        const bf16x8 p = pack(acc[u] * 0.5f, acc[u] * 0.25f);
        acc[u + 1] = pgn_mfma(frag(tile, 64 + ((r0 + i) & 15), 0, g), p, acc[u + 1]);
        acc[u + 1] = pgn_mfma(frag(tile, 64 + ((r0 + i) & 15), 1, g), p, acc[u + 1]);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) s += acc[u][0] + acc[u][1] + acc[u][2] + acc[u][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

// variant 0..5, waves per workgroup (1..16), iterations, workgroups; out: one float per thread. Every variant runs
// 262,144 flop per wave per iteration. Returns 0, -1 on a bad argument, or a hipError_t.
extern "C" int pragnosia_microbench_contract(int variant, int waves, int iters, int nwg, float* out, void* stream) {
  if (variant < 0 || variant > 5 || waves < 1 || waves > 16 || iters < 1 || nwg < 1 || !out) return -1;
  const dim3 grid((unsigned)nwg), block((unsigned)(64 * waves));
  hipStream_t st = (hipStream_t)stream;
  switch (variant) {
    case 0: hipLaunchKernelGGL(contract<0>, grid, block, 0, st, iters, out); break;
    case 1: hipLaunchKernelGGL(contract<1>, grid, block, 0, st, iters, out); break;
    case 2: hipLaunchKernelGGL(contract<2>, grid, block, 0, st, iters, out); break;
    case 3: hipLaunchKernelGGL(contract32<0>, grid, block, 0, st, iters, out); break;
    case 4: hipLaunchKernelGGL(contract32<1>, grid, block, 0, st, iters, out); break;
    default: hipLaunchKernelGGL(contract32<2>, grid, block, 0, st, iters, out); break;
  }
  return (int)hipGetLastError();
}
