// Greedy decode bookkeeping for the e2e harness: argmax over one row of logits, then
// out[pos] = idx, tok = idx, pos += 1, in one launch.
//
// Replaces the greedy step of the reference's GraphDecoder (kernels/e2e/run.py:69-74:
// `logits.argmax(-1)`, `out.index_copy_(0, pos, nxt)`, `tok.copy_(nxt)`, `pos.add_(1)`). torch's
// argmax over a vocabulary-sized row reduces across workgroups through a semaphore buffer that it
// clears with hipMemsetAsync; a captured memset node is not reliable under repeated graph replay
// on this platform, so the decode graph uses this kernel instead.
//
// Semantics follow torch.argmax: the largest value wins, NaN counts as larger than any number,
// ties go to the smallest index (-0.0 ties with +0.0).
//
// Reduction. Every candidate becomes one 64-bit key whose unsigned order is that ordering: the
// high word is the value's bits mapped to an order-preserving unsigned integer (NaN above +inf),
// the low word is ~index (a lower index is a larger key on ties). A row is split over workgroups
// of 256 threads that each issue all their loads at once; a workgroup reduces its keys with
// wave shuffles and LDS, then adds it to a device-global key with one atomic max and counts
// itself in with one returning atomic add. The workgroup that completes the count reads the
// winning key, writes tok/out/pos and puts the key and the count back to zero, so the state is
// clean for the next launch (also under graph replay; no memset, no second launch). Calls on one
// device share that state and must be stream-ordered.
#include "ldk_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kLoads = 4;  // 16-byte loads per thread, all in flight together

__device__ uint64_t g_best;   // winning key of the launch in progress (0 between launches)
__device__ uint32_t g_count;  // workgroups that have added their key (0 between launches)

template <typename T>
__device__ __forceinline__ float to_f(T v);
template <>
__device__ __forceinline__ float to_f<half_t>(half_t v) { return (float)v; }
template <>
__device__ __forceinline__ float to_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f<uint16_t>(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

// Order-preserving key of (value, index); every real key is > 0.
__device__ __forceinline__ uint64_t key_of(float v, uint32_t i) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if (v == 0.0f) u = 0u;  // -0.0 == +0.0
  uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (v != v) hi = 0xffffffffu;
  return ((uint64_t)hi << 32) | (uint32_t)~i;
}

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <typename T>
__global__ __launch_bounds__(kThreads) void greedy_step_kernel(const T* __restrict__ logits, int64_t V, int64_t nvec,
                                                                int64_t* tok, int64_t* out, int64_t out_len,
                                                                int64_t* pos) {
  constexpr int kVec = 16 / sizeof(T);
  typedef T vec_t __attribute__((ext_vector_type(kVec)));
  __shared__ uint64_t wbest[kThreads / 64];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kThreads * kLoads;  // first vector of this workgroup
  vec_t v[kLoads];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
    const int64_t c = base + tid + (int64_t)u * kThreads;
    v[u] = c < nvec ? *reinterpret_cast<const vec_t*>(logits + c * kVec) : vec_t{};
  }
  uint64_t best = 0;
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
    const int64_t c = base + tid + (int64_t)u * kThreads;
    if (c < nvec) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) best = max64(best, key_of(to_f<T>(v[u][j]), (uint32_t)(c * kVec + j)));
    }
  }
  if (blockIdx.x == gridDim.x - 1)  // the scalar tail after the last whole vector
    for (int64_t i = nvec * kVec + tid; i < V; i += kThreads) best = max64(best, key_of(to_f<T>(logits[i]), (uint32_t)i));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)best, off), hi = __shfl_xor((uint32_t)(best >> 32), off);
    best = max64(best, ((uint64_t)hi << 32) | lo);
  }
  if ((tid & 63) == 0) wbest[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) best = max64(best, wbest[w]);
    __hip_atomic_fetch_max(&g_best, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t done = __hip_atomic_fetch_add(&g_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      const uint64_t k = __hip_atomic_load(&g_best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int64_t idx = (int64_t)(uint32_t)~(uint32_t)k;
      const int64_t p = *pos;
      if (out && p >= 0 && p < out_len) out[p] = idx;
      *tok = idx;
      *pos = p + 1;
      __hip_atomic_store(&g_best, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&g_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <typename T>
int launch(const void* logits, int64_t V, int64_t* tok, int64_t* out, int64_t out_len, int64_t* pos, hipStream_t s) {
  constexpr int kVec = 16 / sizeof(T);
  const int64_t nvec = ldk::aligned(logits, 16) ? V / kVec : 0;  // else one workgroup, scalar loads
  const int64_t per_block = (int64_t)kThreads * kLoads;
  const int64_t blocks = nvec > 0 ? (nvec + per_block - 1) / per_block : 1;
  (void)hipGetLastError();
  greedy_step_kernel<T><<<(unsigned)blocks, kThreads, 0, s>>>((const T*)logits, V, nvec, tok, out, out_len, pos);
  return ldk::check_launch("greedy_step");
}

}  // namespace

extern "C" int ldk_greedy_step(const void* logits, int dtype, int64_t V, int64_t* tok, int64_t* out,
                               int64_t out_len, int64_t* pos, void* stream) {
  if (!logits || !tok || !pos) return ldk::fail(LDK_ERR_INVALID, "greedy_step: null pointer");
  if (V <= 0 || (out && out_len <= 0)) return ldk::fail(LDK_ERR_INVALID, "greedy_step: V=%lld out_len=%lld", (long long)V, (long long)out_len);
  if (V >= ((int64_t)1 << 32) - 1) return ldk::fail(LDK_ERR_UNSUPPORTED, "greedy_step: V=%lld needs 32-bit indices", (long long)V);
  if (!ldk::aligned(tok, 8) || !ldk::aligned(pos, 8) || (out && !ldk::aligned(out, 8)))
    return ldk::fail(LDK_ERR_ALIGN, "greedy_step: tok, pos and out must be 8-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case LDK_F16: return launch<half_t>(logits, V, tok, out, out_len, pos, s);
    case LDK_BF16: return launch<uint16_t>(logits, V, tok, out, out_len, pos, s);
    case LDK_F32: return launch<float>(logits, V, tok, out, out_len, pos, s);
  }
  return ldk::fail(LDK_ERR_INVALID, "greedy_step: unknown dtype %d", dtype);
}
