// Shared device/host helpers for the gfx950 decode kernels: status reporting for the C ABI,
// packed fp16 types, the XCD-aware workgroup remap and the wave64 cross-lane reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ldk.h"

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------ host side
namespace ldk {

// Records `msg` as this thread's last error and returns `code` (used as `return fail(...)`).
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP launch status to LDK_OK / LDK_ERR_LAUNCH with a message naming `what`.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace ldk

// ---------------------------------------------------------------------------------- device side
namespace ldk {

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on XCD b % 8), and
// each XCD has its own L2. This bijection renumbers workgroups so that logical tiles t and t+1
// (which share cache lines and scale rows) run on the same XCD.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  constexpr int kXcd = 8;
  const int q = n / kXcd, rem = n % kXcd;
  const int x = b % kXcd;
  return x * q + (x < rem ? x : rem) + b / kXcd;
}

__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ half2_t u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// DPP row rotate right: lane i of each 16-lane row receives lane (i - N) mod 16 of that row.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  static_assert(N > 0 && N < 16, "rotation inside a row of 16");
  return u2f(__builtin_amdgcn_update_dpp(0u, f2u(v), 0x120 + N, 0xf, 0xf, false));
}

// v(lane i) + v(lane i ^ 16) with gfx950's permlane16 swap (a VALU op, no LDS traffic). The swap
// exchanges the odd rows of its first operand with the even rows of its second; with v in both,
// each lane ends up holding v(i) in one result and v(i ^ 16) in the other, so their sum is the
// pairwise sum whichever result holds which.
__device__ __forceinline__ float add_xor16(float v) {
  auto p = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
  return u2f(p[0]) + u2f(p[1]);
}
// v(lane i) + v(lane i ^ 32) with gfx950's permlane32 swap (upper half of the first operand
// exchanged with the lower half of the second), by the same argument.
__device__ __forceinline__ float add_xor32(float v) {
  auto p = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
  return u2f(p[0]) + u2f(p[1]);
}

// Sum over the lanes that agree with this lane in their low log2(STRIDE) bits, i.e. over
// lanes {i % STRIDE + STRIDE * j}. STRIDE is a power of two in [1, 64]. Every lane gets the sum
// of its class. Row rotations (DPP) cover strides below 16; permlane swaps cover 16 and 32.
template <int STRIDE>
__device__ __forceinline__ float sum_lanes_strided(float v) {
  if constexpr (STRIDE < 2) v += row_ror<1>(v);
  if constexpr (STRIDE < 4) v += row_ror<2>(v);
  if constexpr (STRIDE < 8) v += row_ror<4>(v);
  if constexpr (STRIDE < 16) v += row_ror<8>(v);
  if constexpr (STRIDE < 32) v = add_xor16(v);
  if constexpr (STRIDE < 64) v = add_xor32(v);
  return v;
}

// Materialises a 32-bit constant in an SGPR / a VGPR behind an opaque asm, so that expressions
// like (a & mask) | magic select one VOP3 v_and_or_b32 (gfx9 VOP3 encodings take no literal
// constants; with visible literals the compiler splits them into v_and_b32 + v_or_b32).
template <uint32_t V>
__device__ __forceinline__ uint32_t sgpr_const() {
  uint32_t r;
  asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(V));
  return r;
}
template <uint32_t V>
__device__ __forceinline__ uint32_t vgpr_const() {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(V));
  return r;
}

// Orders LDS accesses of one wavefront (lanes exchanging data through LDS inside a wave): no
// s_barrier is needed since a wave's LDS operations complete in order, but the compiler must not
// move the reads above the writes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Workgroup barrier that orders LDS only: it does not wait for outstanding global loads, so
// weight loads issued before it stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum of the first n (<= 16) floats at p (16-byte aligned, zero padding not required), in index
// order: the partials of one output from the n waves of a workgroup. Four independent LDS vector
// reads are in flight at once instead of n dependent scalar reads.
__device__ __forceinline__ float sum_partials(const float* p, int n) {
  float4_t v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (4 * i < n) v[i] = reinterpret_cast<const float4_t*>(p)[i];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < n) s += v[i / 4][i % 4];
  return s;
}

// Cross-workgroup split-K finalization. The `splits` workgroups of one output tile each hold a
// partial tile `part(o)` for o < n (fp32, already reduced inside the workgroup). Each writes it to
// its slot of `ws` ([tile][split][n] floats) with agent-scope stores that write through the
// per-XCD L2, waits for them, and increments the tile's counter once; the workgroup that observes
// splits-1 reads the slots back with agent-scope loads (served past the L2), sums them in split
// order (deterministic), calls store(o, value) and resets the counter to 0, so the counters are
// zero again after every launch and never need a clearing launch. No L2 write-back or invalidate
// is issued (an agent-scope fence would flush the whole L2 of every XCD, per workgroup). Must be
// called by every thread of the workgroup (it contains barriers).
template <typename Part, typename Store>
__device__ __forceinline__ void splitk_finalize(int tile, int split, int splits, int n, float* ws,
                                                uint32_t* counters, Part part, Store store) {
  __shared__ int s_last;
  float* mine = ws + ((size_t)tile * splits + split) * n;
  for (int o = threadIdx.x; o < n; o += blockDim.x)
    __hip_atomic_store(mine + o, part(o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();                // ... and every thread's
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(splits - 1);
  __syncthreads();
  if (s_last) {
    const float* all = ws + (size_t)tile * splits * n;
    for (int o = threadIdx.x; o < n; o += blockDim.x) {
      float v = 0.0f;
      for (int sp = 0; sp < splits; ++sp)
        v += __hip_atomic_load(all + (size_t)sp * n + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      store(o, v);
    }
    if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace ldk
