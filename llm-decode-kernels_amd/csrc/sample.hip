// Greedy decode bookkeeping for the e2e harness: argmax over one row of logits, then
// out[pos] = idx, tok = idx, pos += 1, in one launch.
//
// Replaces the greedy step of the reference's GraphDecoder (kernels/e2e/run.py:69-74:
// `logits.argmax(-1)`, `out.index_copy_(0, pos, nxt)`, `tok.copy_(nxt)`, `pos.add_(1)`). torch's
// argmax over a vocabulary-sized row reduces across workgroups through a semaphore buffer that it
// clears with hipMemsetAsync; a captured memset node is not reliable under repeated graph replay
// on this platform, so the decode graph uses this kernel instead: one workgroup, no memset, no
// cross-workgroup state.
//
// Semantics follow torch.argmax: the largest value wins, NaN counts as larger than any number,
// ties go to the smallest index.
#include "ldk_common.h"

namespace {

constexpr int kThreads = 1024;

struct Best {
  float v;
  int64_t i;
};

// a is preferred over b (torch's ordering, NaN largest, lower index on ties).
__device__ __forceinline__ bool better(float va, int64_t ia, float vb, int64_t ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ void take(Best& b, float v, int64_t i) {
  if (better(v, i, b.v, b.i)) { b.v = v; b.i = i; }
}

template <typename T>
__device__ __forceinline__ float to_f(T v);
template <>
__device__ __forceinline__ float to_f<half_t>(half_t v) { return (float)v; }
template <>
__device__ __forceinline__ float to_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f<uint16_t>(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

template <typename T>
__global__ __launch_bounds__(kThreads) void greedy_step_kernel(const T* __restrict__ logits, int64_t V,
                                                                int64_t* tok, int64_t* out, int64_t out_len,
                                                                int64_t* pos) {
  __shared__ float sv[kThreads / 64];
  __shared__ int64_t si[kThreads / 64];
  const int tid = threadIdx.x;
  Best b{-__builtin_inff(), V};  // index V loses every tie against a real index
  constexpr int kVec = 16 / sizeof(T);
  constexpr int kBatch = 20;  // 16-byte loads per thread in flight at once (a 151936-entry fp16
                              // row is 18992 loads: one batch, one memory round trip)
  const int64_t nvec = ldk::aligned(logits, 16) ? V / kVec : 0;
  typedef T vec_t __attribute__((ext_vector_type(kVec)));
  for (int64_t c0 = 0; c0 < nvec; c0 += (int64_t)kBatch * kThreads) {
    vec_t v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t c = c0 + tid + (int64_t)u * kThreads;
      v[u] = c < nvec ? *reinterpret_cast<const vec_t*>(logits + c * kVec) : vec_t{};
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t c = c0 + tid + (int64_t)u * kThreads;
      if (c < nvec) {
#pragma unroll
        for (int j = 0; j < kVec; ++j) take(b, to_f<T>(v[u][j]), c * kVec + j);
      }
    }
  }
  for (int64_t i = nvec * kVec + tid; i < V; i += kThreads) take(b, to_f<T>(logits[i]), i);
  // wave reduction, then across the waves through LDS
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(b.v, off);
    const int64_t oi = __shfl_xor(b.i, off);
    take(b, ov, oi);
  }
  if ((tid & 63) == 0) { sv[tid >> 6] = b.v; si[tid >> 6] = b.i; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kThreads / 64; ++w) take(b, sv[w], si[w]);
    const int64_t idx = b.i < V ? b.i : 0;
    const int64_t p = *pos;
    if (out && p >= 0 && p < out_len) out[p] = idx;
    *tok = idx;
    *pos = p + 1;
  }
}

}  // namespace

extern "C" int ldk_greedy_step(const void* logits, int dtype, int64_t V, int64_t* tok, int64_t* out,
                               int64_t out_len, int64_t* pos, void* stream) {
  if (!logits || !tok || !pos) return ldk::fail(LDK_ERR_INVALID, "greedy_step: null pointer");
  if (V <= 0 || (out && out_len <= 0)) return ldk::fail(LDK_ERR_INVALID, "greedy_step: V=%lld out_len=%lld", (long long)V, (long long)out_len);
  if (!ldk::aligned(tok, 8) || !ldk::aligned(pos, 8) || (out && !ldk::aligned(out, 8)))
    return ldk::fail(LDK_ERR_ALIGN, "greedy_step: tok, pos and out must be 8-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  switch (dtype) {
    case LDK_F16: greedy_step_kernel<half_t><<<1, kThreads, 0, s>>>((const half_t*)logits, V, tok, out, out_len, pos); break;
    case LDK_BF16: greedy_step_kernel<uint16_t><<<1, kThreads, 0, s>>>((const uint16_t*)logits, V, tok, out, out_len, pos); break;
    case LDK_F32: greedy_step_kernel<float><<<1, kThreads, 0, s>>>((const float*)logits, V, tok, out, out_len, pos); break;
    default: return ldk::fail(LDK_ERR_INVALID, "greedy_step: unknown dtype %d", dtype);
  }
  return ldk::check_launch("greedy_step");
}
