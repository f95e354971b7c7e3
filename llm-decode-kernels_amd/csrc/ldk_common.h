// Shared device/host helpers for the gfx950 decode kernels: status reporting for the C ABI,
// packed fp16 types, buffer-load helpers and the wave64 cross-lane reductions.
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

__host__ __device__ inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace ldk

// ---------------------------------------------------------------------------------- device side
namespace ldk {

// Buffer resource over [p, p + bytes) (gfx9 raw-buffer word 3): a raw buffer load at a byte
// offset outside it returns zero and makes no memory request, so a load that only some lanes
// need is issued unconditionally, with no branch for the compiler to wait at.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0));
}

// SwiGLU's activation of one gate value, shared by the standalone SwiGLU kernel and the fused
// prologues (so their staged values are the same bits): silu in fp32, exp(-f) as 2^(-f log2 e) on
// the hardware exp2 and the division as the hardware reciprocal, rounded to fp16 (the caller
// multiplies by u in fp16). Large |f| saturate as in fp32 arithmetic: 2^(+big) = inf gives -0 for
// very negative gates, 2^(-big) = 0 gives f.
__device__ __forceinline__ half_t silu_f16(half_t g) {
  const float f = (float)g;
  const float e = __builtin_amdgcn_exp2f(f * -1.44269504088896341f);
  float p = f * __builtin_amdgcn_rcpf(1.0f + e);
  // the product is an fp32 value, then rounded to fp16: without this the compiler may form
  // v_fma_mix*_f16 in some kernels, one rounding of the exact product, which differs from the
  // fp32-then-fp16 result in about 1 of 8000 values
  asm volatile("" : "+v"(p));
  return (half_t)p;
}

// RMSNorm's staged value of one element with the steps of the standalone RMSNorm kernel:
// w * fp16(h * rs), the product rounded to fp16 once and the weight applied as an fp16 multiply.
__device__ __forceinline__ half_t rms_f16(half_t h, float rs, half_t w) {
  float v = (float)h * rs;
  asm volatile("" : "+v"(v));  // a -0 * rs must stay -0 (no v_fma_mix with a +0 addend)
  return w * (half_t)v;
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

// Makes a uniform value (a kernel argument) live in SGPRs at this point. Kernel arguments are
// fetched with scalar loads; without a use before the first branch, the compiler sinks some of
// them into the branch and the kernel pays a second scalar round trip before its first vector
// load.
template <typename T>
__device__ __forceinline__ void pin_sgpr(T v) {
  asm volatile("" : : "s"(v));
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

// Sum of p[0], p[stride], ..., p[(n-1)*stride] (n <= 16) in index order: the partials of one
// output from the n waves of a workgroup, stored wave-major. All reads are issued before the
// first add, so their LDS latencies overlap instead of adding up.
__device__ __forceinline__ float sum_waves(const float* p, int stride, int n) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = i < n ? p[i * stride] : 0.0f;
  float s = v[0];
#pragma unroll
  for (int i = 1; i < 16; ++i)
    if (i < n) s += v[i];
  return s;
}

// Cross-workgroup split-K reduction in one memory round trip. The `splits` workgroups of one
// output tile each hold a partial p(o) for o < n (fp32, already reduced inside the workgroup).
// Each adds it to a 64-bit word per output with one agent-scope atomic add:
//   bits [5:0]   arrivals,
//   bits [11:6]  arrivals whose partial took the side path (below),
//   bits [63:12] the sum of round(p * 2^24) in two's complement (fixed point, 2^-24 resolution:
//                the spacing of the smallest fp16 subnormals).
// The add returns the previous word, so the workgroup whose add brings the arrival count to
// `splits` holds the complete sum: it stores the output and writes the word back to zero,
// leaving the workspace zeroed for the next launch (no clearing launch, no barrier, no waiting
// on other workgroups). Integer addition is associative, so the result does not depend on
// arrival order (deterministic).
//
// Side path. A partial with |p| >= 2^21, or a non-finite one, does not fit the fixed-point sum
// (up to 63 partials of |p| < 2^21 keep |sum| < 2^51). Such a partial is stored as fp32 to its
// own slot side[(word - words) * splits + split] (zero-filled, like the words), made visible at
// agent scope by a release fence before the atomic add, and counted in bits [11:6]. The finishing
// workgroup, seeing a non-zero side count, acquires, adds every slot of the word in split order
// to the fixed-point sum in fp32 and zeroes them. So partials that cancel beyond the fixed-point
// range (+3e6 and -3e6 + 10) give the fp32 sum, and inf/NaN partials propagate as in fp32
// arithmetic. The fast path costs one compare.
constexpr float kFixScale = 16777216.0f;  // 2^24
constexpr float kFixRange = 2097152.0f;   // 2^21: partials below this in magnitude stay fixed point
constexpr int kFixMaxSplits = 63;         // arrival count field

struct SplitK {
  uint64_t* words;  // first accumulator word of the launch
  float* side;      // [words][splits] fp32 side slots, zero between launches
  int splits;       // workgroups meeting in each word
  int split;        // this workgroup's index among them
};

// The increment for partial p of `word` (stores p to its side slot when it takes the side path).
__device__ __forceinline__ uint64_t splitk_inc(const SplitK& k, const uint64_t* word, float p) {
  if (__builtin_fabsf(p) < kFixRange) return ((uint64_t)(int64_t)__builtin_rintf(p * kFixScale) << 12) + 1u;
  k.side[(size_t)(word - k.words) * k.splits + k.split] = p;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  return (uint64_t(1) << 6) + 1u;
}
// The two halves of splitk_add, for a caller with several outputs per lane: issue every add first
// (their round trips overlap), then finish each with the word it returned.
__device__ __forceinline__ uint64_t splitk_issue(uint64_t* word, uint64_t inc) {
  return __hip_atomic_fetch_add(word, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool splitk_finish(const SplitK& k, uint64_t* word, uint64_t old, uint64_t inc, float* total) {
  const uint64_t now = old + inc;
  if ((int)(now & 63u) != k.splits) return false;
  float t = (float)((int64_t)now >> 12) * (1.0f / kFixScale);
  if (now & (uint64_t(63) << 6)) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    float* slot = k.side + (size_t)(word - k.words) * k.splits;
    for (int i = 0; i < k.splits; ++i) {
      t += __hip_atomic_load(slot + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      slot[i] = 0.0f;
    }
  }
  __hip_atomic_store(word, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *total = t;
  return true;
}

// Adds partial p of one output to its accumulator word. Returns true in the one contribution that
// completes the count; *total then holds the reduced value and the word is back to zero.
__device__ __forceinline__ bool splitk_add(const SplitK& k, uint64_t* word, float p, float* total) {
  const uint64_t inc = splitk_inc(k, word, p);
  return splitk_finish(k, word, splitk_issue(word, inc), inc, total);
}

template <typename Part, typename Store>
__device__ __forceinline__ void splitk_accumulate(const SplitK& k, uint64_t* acc, int n, Part part, Store store) {
  for (int o = threadIdx.x; o < n; o += blockDim.x) {
    float tot;
    if (splitk_add(k, acc + o, part(o), &tot)) store(o, tot);
  }
}

// Bytes of workspace a launch with `words` accumulator words split `splits` ways needs: the words,
// then (at the next 256-byte boundary) their fp32 side slots.
inline size_t splitk_bytes(int64_t words, int splits) {
  return (((size_t)words * 8 + 255) & ~size_t(255)) + (size_t)words * splits * 4;
}
// The side slots of a launch whose words start at `ws`.
inline float* splitk_side(void* ws, int64_t words) {
  return reinterpret_cast<float*>(static_cast<char*>(ws) + (((size_t)words * 8 + 255) & ~size_t(255)));
}

}  // namespace ldk
