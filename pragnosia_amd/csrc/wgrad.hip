// Weight gradient of a linear layer over the token dimension, C (M x N, fp32) = A^T B with A (K x M) and B (K x N)
// bf16, row-major (K = tokens, the rows of both operands): the dW = dY^T X of the carrier's projections and the
// MLP's layers (the reference's autograd forms it for every nn.Linear / F.linear of src/assoc.py:384-512 and
// src/model.py:552-560, as a bf16 GEMM under autocast whose result is then cast to the fp32 parameter's dtype).
// Here the fp32 accumulator is the result: no bf16 rounding, no cast kernel.
//
// The shapes are few outputs over a long reduction (768 x 768 or 2328 x 768 over 8192 tokens): a plain GEMM has
// fewer output tiles than compute units and walks K serially in each. So K is split: workgroup (tile, split) sums its
// K range into an fp32 partial, and a second kernel adds the splits in a fixed order (deterministic, no atomics, no
// memset), optionally onto C. The split count brings the grid to about two workgroups per compute unit.
//
// Tiling: a workgroup of 4 waves computes a 128 x 128 tile of C, wave (wm, wn) its 64 x 64 quarter as 4 x 4 MFMA
// tiles (v_mfma_f32_16x16x32_bf16). K advances 64 rows a step: the step's A and B rows (64 x 128 each, untransposed,
// 16-byte row segments, four per thread per operand) are staged into double-buffered LDS tiles (pitch 68) and read as
// operands contracted over the tile's row index with the LDS transpose read. Global loads run kDepth - 1 steps ahead
// in a ring of kDepth - 1 register sets (the loop unrolled by the ring's size so each set is fixed registers): one
// step's products are far shorter than a load's latency, and with a single step of lead each step waited out a
// whole load (measured ~2 us a step). One barrier per step.
#include <algorithm>

#include "mfma_tile.h"

using namespace pgn;

namespace {

constexpr int TM = 128, TN = 128, KS = 64;
constexpr int TILE = 64 * kPitch;      // one 64 x 64 bf16 LDS tile
constexpr int kSetTiles = 4;           // A halves (m 0..63, 64..127), B halves
constexpr int kTargetGroups = 512;     // two per compute unit
constexpr int kMaxSplits = 16;
constexpr int kXcds = 8;            // XCDs of an MI355X, taking workgroups in turn
constexpr int kDepth = 3;          // pipeline depth: loads issued kDepth - 1 steps ahead of their step

struct Split {
  int S;        // number of K ranges
  int64_t len;  // rows per range, a multiple of KS
};

Split choose_split(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  const int64_t steps = (K + KS - 1) / KS;
  int64_t S = (kTargetGroups + tiles / 2) / tiles;
  S = std::max<int64_t>(1, std::min<int64_t>({S, (int64_t)kMaxSplits, steps}));
  const int64_t len = ((steps + S - 1) / S) * KS;
  return Split{(int)((K + len - 1) / len), len};
}

// A split's rows of an operand as a buffer resource: rows [k_begin, k_end) of pitch ld. Loads past the range return
// zero in hardware (the rows after K, with no branch around the load, so the compiler's wait counts stay exact);
// columns past M or N inside the range read other elements of the same rows and only reach output columns that are
// not stored.
PGN_DEVICE __amdgpu_buffer_rsrc_t rows_rsrc(const __bf16* p, int64_t ld, int64_t k_begin, int64_t k_end) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(p + k_begin * ld), (short)0,
                                           (int)((k_end - k_begin) * ld * (int64_t)sizeof(__bf16)), 0x00020000);
}

PGN_DEVICE bf16x8 load_seg16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

__global__ __launch_bounds__(256) void wgrad_tiles(const __bf16* __restrict__ A, int64_t lda,
                                                   const __bf16* __restrict__ B, int64_t ldb,
                                                   float* __restrict__ out, int64_t ldo, int64_t split_stride,
                                                   int accumulate, int64_t M, int64_t N, int64_t K,
                                                   int64_t len, int nsplit) {
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* lds = reinterpret_cast<__bf16*>(smem);  // two sets of kSetTiles tiles
  const WaveIdx x = wave_idx();
  const int w = x.w, g = x.g, i = x.i, tid = threadIdx.x;
  const int wm = w >> 1, wn = w & 1;
  // work item of this workgroup: consecutive workgroup indices go to the XCDs in turn, so XCD x = blockIdx.x % 8
  // takes the contiguous run x * per .. of the items ordered (split, m tile, n tile), n fastest: its workgroups share
  // their A rows across n tiles and their B rows across m tiles in the XCD's own L2 (ordered by index, the items of
  // one tile row would spread over all eight L2s and each operand be fetched once per XCD that reads it)
  const int64_t tn = (N + TN - 1) / TN, tm = (M + TM - 1) / TM, items = tn * tm * nsplit;
  const int64_t per = (items + kXcds - 1) / kXcds;
  const int64_t item = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (item >= items) return;  // the whole workgroup (the grid is rounded up to a multiple of the XCD count)
  const int64_t split = item / (tn * tm), mn = item - split * tn * tm;
  const int64_t m_base = (mn / tn) * TM, n_base = (mn - (mn / tn) * tn) * TN;
  const int64_t k_begin = split * len, k_end = min(K, k_begin + len);
  const int steps = (int)((k_end - k_begin + KS - 1) / KS);
  float* const dst = out + split * split_stride;

  // A ring of kRing = kDepth - 1 register sets: set j holds the segments of the steps s with s % kRing == j, loaded
  // kRing steps before they are staged, so kRing steps of products cover each load's latency (while step s is
  // contracted, steps s + 1 .. s + kRing are in flight; step s itself was staged before it started).
  constexpr int kRing = kDepth - 1;
  bf16x8 ra[kRing][4], rb[kRing][4];
  const __amdgpu_buffer_rsrc_t a_rows = rows_rsrc(A, lda, k_begin, k_end);
  const __amdgpu_buffer_rsrc_t b_rows = rows_rsrc(B, ldb, k_begin, k_end);
  // Segment u of thread tid: 64-column half u >> 1, row (tid >> 3) + 32 (u & 1) of the step, segment tid & 7 of that
  // half's row. A wave stages eight consecutive rows of one half, eight lanes a row: each 8-lane group fills one
  // 128-byte row (every bank once) and the next group's row starts 2 banks on (pitch 68), so the staging writes
  // run without bank conflicts; in global memory each group reads 128 contiguous bytes.
  auto load = [&](auto j_c, int s) {
    constexpr int j = decltype(j_c)::value;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = s * KS + (tid >> 3) + 32 * (u & 1), c = 64 * (u >> 1) + 8 * (tid & 7);
      ra[j][u] = load_seg16(a_rows, (int)((r * lda + m_base + c) * (int64_t)sizeof(__bf16)));
      rb[j][u] = load_seg16(b_rows, (int)((r * ldb + n_base + c) * (int64_t)sizeof(__bf16)));
    }
  };
  auto stage = [&](auto j_c, int set) {
    constexpr int j = decltype(j_c)::value;
    __bf16* t = lds + set * kSetTiles * TILE;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = 8 * ((tid >> 3) + 32 * (u & 1)) + (tid & 7);
      put_seg(t + (u >> 1) * TILE, ra[j][u], e);
      put_seg(t + (2 + (u >> 1)) * TILE, rb[j][u], e);
    }
  };

  // acc[ib][jb]: rows n = 64 wn + 16 jb + 4 g + r, column m = 64 wm + 16 ib + i of this wave's quarter (C^T tiles,
  // so each lane's four values are consecutive columns of one row of C)
  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  // prologue: steps 0 .. kRing - 1 in flight, step 0 staged. The steps run in whole rounds of kRing (a step past the
  // split's rows loads zeros through the buffer range check and adds nothing), so every step of the loop body is
  // unconditional and the ring's registers are defined on every path.
  const int rounds = (steps + kRing - 1) / kRing;
  static_for<0, kRing>([&](auto j_c) { load(j_c, decltype(j_c)::value); });
  stage(std::integral_constant<int, 0>{}, 0);
  __syncthreads();
  // step s: load step s + kRing into the set step s occupied (staged before step s began), contract step s from LDS
  // set s & 1, stage step s + 1 into the other LDS set (its last reader finished before the previous barrier),
  // barrier
  for (int rd = 0; rd < rounds; ++rd) {
    static_for<0, kRing>([&](auto j_c) {
      constexpr int j = decltype(j_c)::value;
      const int s = rd * kRing + j;
      load(j_c, s + kRing);
      __builtin_amdgcn_sched_barrier(0);  // the loads issue before this step's products, not after them
      const __bf16* t = lds + (s & 1) * kSetTiles * TILE;
      const __bf16* At = t + wm * TILE;
      const __bf16* Bt = t + (2 + wn) * TILE;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        bf16x8 fa[4], fb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          fa[q] = frag_tr(At, 16 * q, kh, g, i);
          fb[q] = frag_tr(Bt, 16 * q, kh, g, i);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a][b] = pgn_mfma(fb[b], fa[a], acc[a][b]);
      }
      stage(std::integral_constant<int, (j + 1) % kRing>{}, (s + 1) & 1);
      __syncthreads();
    });
  }

  if (accumulate) {
    // every earlier value is read before any store, from a clamped (always valid) address with no branch, and
    // dropped outside the matrix (a read-add-write per element, behind a bounds branch, waits for each load in turn)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int64_t m = m_base + 64 * wm + 16 * a + i;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t n = n_base + 64 * wn + 16 * b + 4 * g;
        const float4 o = *reinterpret_cast<const float4*>(dst + std::min(m, M - 1) * ldo + std::min(n, N - 4));
        const float keep = (m < M && n < N) ? 1.f : 0.f;
        acc[a][b] += f32x4{o.x, o.y, o.z, o.w} * keep;
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t m = m_base + 64 * wm + 16 * a + i;
    if (m >= M) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t n = n_base + 64 * wn + 16 * b + 4 * g;
      if (n >= N) continue;
      *reinterpret_cast<float4*>(dst + m * ldo + n) =
          make_float4(acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]);
    }
  }
}

// C (+)= sum over the S splits' partials, each (M, N) with row pitch N, in split order; four columns a thread.
__global__ __launch_bounds__(256) void wgrad_reduce(const float* __restrict__ part, int S, float* __restrict__ C,
                                                    int64_t ldc, int accumulate, int64_t M, int64_t N) {
  const int64_t q = N / 4, total = M * q, plane = M * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / q, n = 4 * (e - m * q);
    const float* p = part + m * N + n;
    float4 s = *reinterpret_cast<const float4*>(p);
    for (int k = 1; k < S; ++k) {
      const float4 t = *reinterpret_cast<const float4*>(p + k * plane);
      s.x += t.x;
      s.y += t.y;
      s.z += t.z;
      s.w += t.w;
    }
    float4* c = reinterpret_cast<float4*>(C + m * ldc + n);
    if (accumulate) {
      const float4 o = *c;
      s.x += o.x;
      s.y += o.y;
      s.z += o.z;
      s.w += o.w;
    }
    *c = s;
  }
}

bool wgrad_shape_ok(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 && M % 8 == 0 && N % 8 == 0 && M < (1 << 24) && N < (1 << 24) &&
         K < ((int64_t)1 << 40);
}

int64_t partial_bytes(int64_t M, int64_t N, int64_t K) {
  const Split sp = choose_split(M, N, K);
  return sp.S > 1 ? (int64_t)sp.S * M * N * (int64_t)sizeof(float) : 0;
}

constexpr int kSmem = 2 * kSetTiles * TILE * (int)sizeof(__bf16);

}  // namespace

extern "C" int64_t pragnosia_wgrad_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (!wgrad_shape_ok(M, N, K)) return -1;
  return partial_bytes(M, N, K);
}

extern "C" int pragnosia_wgrad_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, float* C, int64_t ldc,
                                    int accumulate, void* workspace, int64_t workspace_bytes, int64_t M, int64_t N,
                                    int64_t K, void* stream) {
  PGN_CHECK_ARG(wgrad_shape_ok(M, N, K));
  PGN_CHECK_ARG(A && B && C);
  PGN_CHECK_ARG(lda >= M && ldb >= N && ldc >= N && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0);
  PGN_CHECK_ARG(((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0 && ((uintptr_t)C % 16) == 0);
  const Split sp = choose_split(M, N, K);
  // each split's rows are addressed through a buffer resource with 32-bit byte offsets: the largest offset a load
  // forms is at row len + 3 KS (the ring's look-ahead past the rounded-up last step), columns up to max(M, N) + 128
  PGN_CHECK_ARG(((sp.len + 3 * KS) * std::max(lda, ldb) + std::max(M, N) + 128) * (int64_t)sizeof(uint16_t) <
                ((int64_t)1 << 31));
  const int64_t need = partial_bytes(M, N, K);
  PGN_CHECK_ARG(workspace_bytes >= need && (need == 0 || (workspace && ((uintptr_t)workspace % 16) == 0)));
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = pgn_lds_limit((const void*)wgrad_tiles, kSmem);
  if (e != hipSuccess) return (int)e;
  const int64_t items = ((N + TN - 1) / TN) * ((M + TM - 1) / TM) * sp.S;
  const dim3 grid((unsigned)(((items + kXcds - 1) / kXcds) * kXcds));
  if (sp.S == 1) {
    hipLaunchKernelGGL(wgrad_tiles, grid, dim3(256), kSmem, st, (const __bf16*)A, lda, (const __bf16*)B, ldb, C, ldc,
                       (int64_t)0, accumulate, M, N, K, sp.len, sp.S);
    PGN_RETURN_LAUNCH();
  }
  float* part = (float*)workspace;
  hipLaunchKernelGGL(wgrad_tiles, grid, dim3(256), kSmem, st, (const __bf16*)A, lda, (const __bf16*)B, ldb, part, N,
                     M * N, 0, M, N, K, sp.len, sp.S);
  e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int64_t work = M * (N / 4);
  const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 2048);
  hipLaunchKernelGGL(wgrad_reduce, dim3(blocks), dim3(256), 0, st, part, sp.S, C, ldc, accumulate, M, N);
  PGN_RETURN_LAUNCH();
}
