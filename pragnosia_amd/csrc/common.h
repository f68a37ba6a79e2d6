// Shared definitions for the carrier-path HIP kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include <mutex>
#include <set>
#include <utility>

#include "../../include/pragnosia_hip.h"

// Raise a kernel's dynamic LDS limit to `bytes` on the current device, once per (kernel, device). Safe to call from
// several host threads at once (the entry points promise that calls on distinct streams are independent).
inline hipError_t pgn_lds_limit(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({fn, dev})) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) done.insert({fn, dev});
  return e;
}

#define PGN_DEVICE __device__ __forceinline__

// Phase stamps, for the instrumented build only (compiled with -DPRAGNOSIA_PHASE_STAMPS into a separate library; the
// product library has none). A translation unit declares its stamp buffer with PGN_STAMP_UNIT(name), which also
// exports `pragnosia_stamps_set_<name>(void* buffer)` to set it (NULL: no stamps). PGN_STAMP(i) has the wave write
// the low 32 bits of the shader clock (s_memtime) to entry i of the buffer (32-bit entries: differences over a
// kernel's duration do not wrap); PGN_STAMP_CLOCKS(i) writes the shader clock and the constant 100 MHz clock
// (s_memrealtime) to entries i and i + 1, from which the shader clock's rate follows. `i` is wave-uniform: every
// lane stores the same (scalar) value to the same entry, so no branch splits the kernel's scheduled blocks.
#ifdef PRAGNOSIA_PHASE_STAMPS
// The buffer pointer lives in constant memory (one scalar load, hoisted out of the kernels' loops) and points to
// global memory (plain global stores: no wait on the kernel's outstanding loads, stores or LDS traffic).
typedef __attribute__((address_space(1))) unsigned int pgn_stamp_t;
#define PGN_STAMP_UNIT(name)                                                                        \
  static __constant__ pgn_stamp_t* pgn_stamps;                                                      \
  static __constant__ pgn_stamp_t* pgn_stamps_aux;                                                  \
  extern "C" int pragnosia_stamps_set_##name(void* buffer) {                                        \
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(pgn_stamps), &buffer, sizeof(buffer));                 \
  }                                                                                                 \
  extern "C" int pragnosia_stamps_set_##name##_aux(void* buffer) {                                  \
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(pgn_stamps_aux), &buffer, sizeof(buffer));             \
  }
#define PGN_STAMP(i)                                                                                \
  do {                                                                                              \
    pgn_stamp_t* const pgn_b_ = pgn_stamps;                                                         \
    if (pgn_b_ != nullptr) pgn_b_[(i)] = (unsigned int)__builtin_amdgcn_s_memtime();                \
  } while (0)
#define PGN_STAMP_CLOCKS(i)                                                                         \
  do {                                                                                              \
    pgn_stamp_t* const pgn_b_ = pgn_stamps;                                                         \
    if (pgn_b_ != nullptr) {                                                                        \
      pgn_b_[(i)] = (unsigned int)__builtin_amdgcn_s_memtime();                                     \
      pgn_b_[(i) + 1] = (unsigned int)__builtin_amdgcn_s_memrealtime();                             \
    }                                                                                               \
  } while (0)
// The second buffer of a unit (`pragnosia_stamps_set_<name>_aux`), for a kernel launched beside the one stamping the
// first: the shader clock to entry i (PGN_STAMP_AUX), or the shader and 100 MHz clocks to i, i + 1.
#define PGN_STAMP_AUX(i)                                                                            \
  do {                                                                                              \
    pgn_stamp_t* const pgn_b_ = pgn_stamps_aux;                                                     \
    if (pgn_b_ != nullptr) pgn_b_[(i)] = (unsigned int)__builtin_amdgcn_s_memtime();                \
  } while (0)
#define PGN_STAMP_CLOCKS_AUX(i)                                                                     \
  do {                                                                                              \
    pgn_stamp_t* const pgn_b_ = pgn_stamps_aux;                                                     \
    if (pgn_b_ != nullptr) {                                                                        \
      pgn_b_[(i)] = (unsigned int)__builtin_amdgcn_s_memtime();                                     \
      pgn_b_[(i) + 1] = (unsigned int)__builtin_amdgcn_s_memrealtime();                             \
    }                                                                                               \
  } while (0)
#else
#define PGN_STAMP_UNIT(name)
#define PGN_STAMP(i) ((void)0)
#define PGN_STAMP_CLOCKS(i) ((void)0)
#define PGN_STAMP_AUX(i) ((void)0)
#define PGN_STAMP_CLOCKS_AUX(i) ((void)0)
#endif

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

// Launch-time argument failures are reported with negative codes (hipError_t values are non-negative).
#define PGN_CHECK_ARG(cond)                                   \
  do {                                                        \
    if (!(cond)) return PRAGNOSIA_ERR_INVALID_ARGUMENT;       \
  } while (0)

#define PGN_RETURN_LAUNCH()                                   \
  do {                                                        \
    hipError_t e_ = hipGetLastError();                        \
    return e_ == hipSuccess ? PRAGNOSIA_OK : (int)e_;         \
  } while (0)

PGN_DEVICE float pgn_exp(float x) { return __expf(x); }

// GELU, erf form (torch's default F.gelu): 0.5 x (1 + erf(x / sqrt 2)).
PGN_DEVICE float pgn_gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

// Sum over the 64 lanes of a wave of NV values per lane (NV a power of two <= 16): the lanes exchange halves, so the
// sums take 6 + NV - 1 exchanges instead of 6 NV. Lane l ends with the sum of value l >> (6 - log2 NV) in v[0].
template <int NV>
PGN_DEVICE void wave_sum_many(float (&v)[NV], int l) {
  int len = NV;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    if (len > 1) {
      const int half = len / 2;
      const bool hi = (l & s) != 0;
#pragma unroll
      for (int m = 0; m < half; ++m) {
        const float send = hi ? v[m] : v[m + half];
        const float keep = hi ? v[m + half] : v[m];
        v[m] = keep + __shfl_xor(send, s);
      }
      len = half;
    } else {
      v[0] += __shfl_xor(v[0], s);
    }
  }
}

template <int NV>
constexpr int log2_of() { return NV == 1 ? 0 : NV == 2 ? 1 : NV == 4 ? 2 : NV == 8 ? 3 : 4; }

// sin and cos of x. The hardware sine/cosine (through __sincosf) take the argument in revolutions: scaling x to
// revolutions in fp32 costs about |x| * 2^-24 rad of absolute angle error, so they are used for |x| < 64 rad (at
// most ~4e-6 rad; measured 1.3e-6 relative on the diagonal scan's outputs for angles in [-pi, pi]) and the precise
// library routine beyond.
PGN_DEVICE void pgn_sincos(float x, float* s, float* c) {
  if (fabsf(x) < 64.f)
    __sincosf(x, s, c);
  else
    sincosf(x, s, c);
}

// Round-to-nearest-even fp32 -> bf16 (finite inputs).
PGN_DEVICE __bf16 pgn_bf16(float x) { return (__bf16)x; }
PGN_DEVICE float pgn_f32(__bf16 x) { return (float)x; }

// One 16x16x32 bf16 MFMA step: acc += A(16x32) B(32x16).
PGN_DEVICE f32x4 pgn_mfma(bf16x8 a, bf16x8 b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
