// Single-pass chunk scans: look-back over per-chunk aggregates of a 64 x 64 affine recurrence, deterministic.
//
// The carried state of a chunked scan obeys X_{p+1} = a_p X_p + M_p over scan positions p (forward: chunks in
// order, X the state entering a chunk; backward: chunks in reverse order, X the state gradient). The work item
// (head, position) computes its chunk's aggregate (a_p, M_p) from the chunk alone and finds its entering value
// X_p from publications of its predecessors. Positions are grouped in blocks of kLbGroup; within the block that
// starts at b, every position p rebuilds X_p by the recurrence itself, in a fixed order,
//     X <- X_b;  for j = b .. p-1:  X <- a_j X + M_j,
// from the block's entering value X_b (the initial state for the first block; otherwise the inclusive value
// P_{b-1} = X_b published by the last position of the previous block) and the aggregates of positions b .. p-1.
// The arithmetic never depends on which workgroup finished first, so results are bit-reproducible. Only the last
// position of a block waits on the previous block's last position; all other waits are on aggregates, which are
// published as soon as a chunk is loaded.
//
// Scheduling. Items are numbered position-major (item = position * heads + head) and a persistent grid walks them
// statically: workgroup g takes items g, g + grid, g + 2 grid, ... in increasing order, prefetching the next
// item's inputs while it computes the current one. An item waits only on items with smaller numbers; with every
// workgroup of the grid resident (the launch sizes the grid to the device's occupancy), the smallest unfinished
// item is always being worked on, so the waits cannot deadlock. No ticket counter is needed: a single hot atomic
// costs about 10 ns per workgroup on this device (one serialised device-scope atomic each). Every wait is also
// bounded (kSpinMax polls): a wait that runs out counts one failure in g_lookback_timeouts and continues with a
// zero state, so the kernel always drains; a timeout means a lost publication (a bug) or a grid that could not
// be made resident, and is reported, never hung on.
//
// Flags and epochs. The workspace persists across calls (zero-filled before its first use); a flag is a 64-bit
// word (epoch << 8 | writer XCD << 4 | state), and a flag counts only when its epoch is the call's: the caller
// passes an epoch larger than any used before with that workspace, so no clearing launch is needed.
//
// Memory ordering. Payloads and flags are written with device-coherent (SC1) stores -- the encoding of agent-scope
// relaxed atomics on this architecture -- which write through the writer's L2, so no L2 writeback or invalidate
// is needed (agent-scope fences would write back or invalidate a whole XCD's L2, once per item). The publisher
// stores its payload, waits until its own stores have completed (vmcnt 0), synchronises the workgroup, and only
// then does one lane store the flag. The reader polls flags with device-coherent loads and, once all are set,
// issues its payload loads: through the L2 (SC0, bypassing only the CU's L1) when the writer ran on the same XCD
// -- whose L2 the write-through updated -- and device-coherent (SC1) otherwise.
#pragma once
#include "common.h"

namespace pgn {

constexpr int kFlagAgg = 1;    // the position's aggregate (a_p, M_p) is published
constexpr int kFlagIncl = 2;   // the position's inclusive value P_p = X_{p+1} is published (last of a block)
constexpr int kLbGroup = 8;    // positions per block
constexpr int kSpinMax = 1 << 18;

// Cache policies (CPol bits, the raw-buffer builtins' `aux` argument): SC1 = device-coherent, SC0 = coherent in
// the XCD's L2 (bypasses the CU's L1).
constexpr int kCohDevice = 16;
constexpr int kCohXcd = 1;

// Failed (timed-out) waits since the library was loaded, per source file that includes this header (each has its
// own copy); the file's host side reads it with lb_read_timeouts().
static __device__ unsigned int g_lookback_timeouts;

inline unsigned int lb_read_timeouts() {
  unsigned int v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_lookback_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess)
    return 0xffffffffu;
  return v;
}

// The XCD (accelerator complex die) this wave runs on: hardware register XCC_ID, bits 3:0.
PGN_DEVICE int xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15; }

// Workspace of one scan with n items: n 64-bit flags, n chunk decays, n aggregates and n inclusive values
// (64 x 64 fp32 each, 16 KiB). Byte offsets.
struct LbLayout {
  int64_t flags_off, av_off, agg_off, incl_off, total;
};

__host__ __device__ inline LbLayout lb_layout(int64_t n) {
  LbLayout L;
  L.flags_off = 0;
  L.av_off = (n * 8 + 255) / 256 * 256;
  L.agg_off = (L.av_off + n * 4 + 255) / 256 * 256;
  L.incl_off = L.agg_off + n * 16384;
  L.total = L.incl_off + n * 16384;
  return L;
}

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

// A raw buffer resource over `bytes` bytes at `base` (a wave-uniform address).
PGN_DEVICE __amdgpu_buffer_rsrc_t lb_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

PGN_DEVICE void lb_store4(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, off, 0, kCohDevice);
}

// Payload load; `local`: the writer ran on this XCD.
PGN_DEVICE f32x4 lb_load4(__amdgpu_buffer_rsrc_t r, int off, bool local) {
  return __builtin_bit_cast(f32x4, local ? __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCohXcd)
                                         : __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCohDevice));
}

PGN_DEVICE uint64_t lb_flag_word(uint64_t epoch, int xcc, int state) {
  return (epoch << 8) | ((uint64_t)xcc << 4) | (uint64_t)state;
}

// Publish: every thread's payload stores complete, then one lane sets the flag.
PGN_DEVICE void lb_publish_flag(uint64_t* flag, uint64_t word) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait, in one wave, until the block predecessors of scan position `pos` have published in this epoch: lane
// l < pos - b watches position b + l for its aggregate, and lane pos - b (if b > 0) watches position b - 1 for its
// inclusive value, where b is the start of pos's block. `flag_of(p)` gives the flag address of position p. On
// success each watching lane leaves its writer's XCD in *xcc (for the payload loads) and the call returns true;
// false if the wait timed out.
template <typename FlagOf>
PGN_DEVICE bool lb_wait_block(int pos, int lane, uint64_t epoch, FlagOf flag_of, int* xcc) {
  const int b = pos - pos % kLbGroup;
  const int nagg = pos - b;
  const bool watch = lane < nagg || (lane == nagg && b > 0);
  const uint64_t want = lane < nagg ? kFlagAgg : kFlagIncl;
  uint64_t* fl = watch ? flag_of(lane < nagg ? b + lane : b - 1) : nullptr;
  for (int it = 0; it < kSpinMax; ++it) {
    const uint64_t f = watch ? __hip_atomic_load(fl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const bool ready = !watch || ((f >> 8) == epoch && (f & 15) >= want);
    if (__ballot(!ready) == 0) {
      *xcc = (int)((f >> 4) & 15);
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

}  // namespace pgn
