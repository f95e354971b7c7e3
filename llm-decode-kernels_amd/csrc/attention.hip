// Fused decode attention for one new token (T = 1, batch 1): RoPE on q and k, the KV-cache write
// at `pos` and grouped-query softmax attention over positions 0..pos, in one launch per layer.
//
// Replaces the per-layer attention block of the reference's runner (kernels/e2e/model.py:
// 212-243: RoPE with rotate_half, k/v index_copy_ into the static cache, SDPA with a causal
// mask) for decode steps, where that block is ~20 small launches per layer.
//
// Layout: qkv [nq*128 | nkv*128 | nkv*128] fp16 (projection output, bias added, before RoPE);
// the cache keeps K transposed, kt [nkv][128][max_len], and V as v [nkv][max_len][128]; out
// [nq*128] fp16. One workgroup per query head h (kv head h / (nq/nkv)); wave w covers positions
// 64w .. 64w+63 (max_len <= 512, so at most 8 waves).
//
// Numerics: RoPE as the reference's fp16 torch ops (cos/sin of pos * inv_freq in fp32 rounded to
// fp16, q*cos and rotate_half(q)*sin each rounded to fp16, their sum rounded), scores, softmax
// and the weighted sum of V in fp32, the output rounded once to fp16.
#include <algorithm>

#include "ldk_common.h"

namespace {

constexpr int kHD = 128;
constexpr int kMaxWaves = 8;  // max_len <= 512

struct AttnArgs {
  const half_t* qkv;
  const int64_t* pos;
  const float* inv_freq;  // [64]
  half_t* kt;             // [nkv][128][max_len]
  half_t* v;              // [nkv][max_len][128]
  half_t* out;            // [nq*128]
  int nq, nkv, max_len;
  float scale;
};

// fp16 RoPE of element d of a 128-vector x (rotate_half pairs d with d +- 64).
__device__ __forceinline__ half_t rope_elem(const half_t* x, int d, float angle_base) {
  const float ang = angle_base;
  const half_t c = (half_t)cosf(ang), s = (half_t)sinf(ang);
  const half_t xd = x[d];
  const half_t rh = d < 64 ? (half_t)(-(float)x[d + 64]) : x[d - 64];
  const half_t a = (half_t)((float)xd * (float)c);
  const half_t b = (half_t)((float)rh * (float)s);
  return (half_t)((float)a + (float)b);
}

__global__ __launch_bounds__(kMaxWaves * 64) void decode_attention_kernel(AttnArgs a) {
  __shared__ float qs[kHD];              // roped q of this head, fp32
  __shared__ half_t knew[kHD], vnew[kHD];
  __shared__ float ps[kMaxWaves * 64];   // softmax weights by position
  __shared__ float wred[kMaxWaves];
  __shared__ float ored[kMaxWaves][kHD];
  const int h = blockIdx.x;
  const int g = a.nq / a.nkv, kvh = h / g;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int64_t pos = *a.pos;
  const half_t* q = a.qkv + (int64_t)h * kHD;
  const half_t* kx = a.qkv + (int64_t)a.nq * kHD + (int64_t)kvh * kHD;
  const half_t* vx = kx + (int64_t)a.nkv * kHD;
  half_t* kt = a.kt + (int64_t)kvh * kHD * a.max_len;
  half_t* vc = a.v + (int64_t)kvh * a.max_len * kHD;

  // ---- RoPE (q, new k), stage the new k/v, write them to the cache (first head of the group)
  if (tid < kHD) {
    const float ang = (float)pos * a.inv_freq[tid & 63];
    qs[tid] = (float)rope_elem(q, tid, ang);
    const half_t kr = rope_elem(kx, tid, ang);
    knew[tid] = kr;
    vnew[tid] = vx[tid];
    if (h % g == 0 && pos < a.max_len) {
      kt[(int64_t)tid * a.max_len + pos] = kr;
      vc[pos * kHD + tid] = vx[tid];
    }
  }
  __syncthreads();

  // ---- scores: lane = position t; the new token's k comes from LDS
  const int t = wave * 64 + lane;
  const bool live = t <= pos && t < a.max_len;
  float s = -__builtin_inff();
  if (live) {
    float acc = 0.0f;
    if (t == pos) {
#pragma unroll 8
      for (int d = 0; d < kHD; ++d) acc = __builtin_fmaf(qs[d], (float)knew[d], acc);
    } else {
      const half_t* kc = kt + t;
#pragma unroll 16
      for (int d = 0; d < kHD; ++d) acc = __builtin_fmaf(qs[d], (float)kc[(int64_t)d * a.max_len], acc);
    }
    s = acc * a.scale;
  }
  // ---- softmax over live positions
  float m = s;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) wred[wave] = m;
  __syncthreads();
  m = wred[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, wred[i]);
  const float p = live ? __expf(s - m) : 0.0f;
  float l = p;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
  __syncthreads();  // everyone has read wred
  if (lane == 0) wred[wave] = l;
  ps[t] = p;
  __syncthreads();
  l = 0.0f;
  for (int i = 0; i < nw; ++i) l += wred[i];

  // ---- out[d] = sum_t p[t] v[t][d] / l: lane = dims 2*lane, 2*lane+1; wave = its positions
  float o0 = 0.0f, o1 = 0.0f;
  const int t0 = wave * 64;
  const int t1 = (int)min<int64_t>(min(t0 + 64, a.max_len), pos + 1);
  for (int tt = t0; tt < t1; ++tt) {
    const float pw = ps[tt];
    half2_t v2;
    if (tt == pos) v2 = half2_t{vnew[2 * lane], vnew[2 * lane + 1]};
    else v2 = *reinterpret_cast<const half2_t*>(vc + (int64_t)tt * kHD + 2 * lane);
    o0 = __builtin_fmaf(pw, (float)v2[0], o0);
    o1 = __builtin_fmaf(pw, (float)v2[1], o1);
  }
  ored[wave][2 * lane] = o0;
  ored[wave][2 * lane + 1] = o1;
  __syncthreads();
  if (tid < kHD) {
    float o = 0.0f;
    for (int i = 0; i < nw; ++i) o += ored[i][tid];
    a.out[(int64_t)h * kHD + tid] = (half_t)(o / l);
  }
}

}  // namespace

extern "C" int ldk_decode_attention(const void* qkv, const int64_t* pos, const float* inv_freq, void* kt_cache,
                                    void* v_cache, void* out, int nq, int nkv, int head_dim, int64_t max_len,
                                    float scale, void* stream) {
  if (!qkv || !pos || !inv_freq || !kt_cache || !v_cache || !out) return ldk::fail(LDK_ERR_INVALID, "decode_attention: null pointer");
  if (head_dim != kHD) return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: head_dim=%d (only 128)", head_dim);
  if (nq <= 0 || nkv <= 0 || nq % nkv) return ldk::fail(LDK_ERR_INVALID, "decode_attention: nq=%d must be a positive multiple of nkv=%d", nq, nkv);
  if (max_len <= 0 || max_len > kMaxWaves * 64)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: max_len=%lld outside 1..%d", (long long)max_len, kMaxWaves * 64);
  if (!ldk::aligned(v_cache, 4) || !ldk::aligned(pos, 8))
    return ldk::fail(LDK_ERR_ALIGN, "decode_attention: v_cache 4-byte and pos 8-byte aligned");
  const AttnArgs a{(const half_t*)qkv, pos, inv_freq, (half_t*)kt_cache, (half_t*)v_cache, (half_t*)out,
                   nq, nkv, (int)max_len, scale};
  const int nw = (int)std::max<int64_t>(2, (max_len + 63) / 64);  // >= 128 threads: one per dim
  (void)hipGetLastError();
  decode_attention_kernel<<<nq, nw * 64, 0, (hipStream_t)stream>>>(a);
  return ldk::check_launch("decode_attention");
}
