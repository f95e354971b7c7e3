// Fused decode attention for one new token (T = 1, batch 1): RoPE on q and k, the KV-cache write
// at `pos` and grouped-query softmax attention over positions 0..pos, in one launch per layer.
//
// Replaces the per-layer attention block of the reference's runner (kernels/e2e/model.py:
// 212-243: RoPE with rotate_half, k/v index_copy_ into the static cache, SDPA with a causal
// mask) for decode steps, where that block is ~20 small launches per layer.
//
// Layout: qkv [nq*128 | nkv*128 | nkv*128] fp16 (projection output, bias added, before RoPE);
// the cache keeps K transposed, kt [nkv][128][max_len], and V as v [nkv][max_len][128]; out
// [nq*128] fp16. max_len is a multiple of 8 (16-byte rows of 8 positions).
//
// Work split (flash-decoding). The cache positions are cut into `nsplit` ranges of S = 64 * cps
// positions (at most 32 ranges of at least 8 chunks each: one range up to max_len 512), and the
// grid is one workgroup per (query head, range): kv head h / (nq/nkv), up to 8 waves, wave w taking
// the chunks w, w + nw, ... of its range that hold live positions (<= pos). A chunk is 16 KB of K
// and 16 KB of V, and a wave issues all 32 of its 16-byte loads per lane before the first wait,
// so the whole chunk is one memory round trip (a per-position loop would be 64 dependent ones).
// One head's cache thus streams through as many CUs as it has ranges instead of one CU. Ranges
// past pos exit at once. While pos lies in the first range, that workgroup writes the output
// itself; otherwise every live range publishes its partial (running max m, sum l, unnormalised
// output o[128]) to library-owned device memory and counts itself in with one agent-scope atomic,
// and the last to arrive merges the partials, writes the output and re-zeroes the counter.
//  - Scores: lane (pg = lane % 8, dg = lane / 8) loads K^T rows dg + 8i (i < 16), positions
//    8pg .. 8pg+7 of the chunk, and sums q[d] * K[d][p] over its 16 rows for its 8 positions;
//    lanes sharing pg are summed with DPP/permlane (stride 8).
//  - Softmax per chunk (max and sum over a 16-lane row, which holds every pg twice), merged
//    online across a wave's chunks and at the end across the waves through LDS.
//  - Output: lane (dc = lane % 16, pr = lane / 16) loads V rows 16pr + i (i < 16), dims
//    8dc .. 8dc+7, weighted by the chunk's softmax numerators (passed through LDS); lanes sharing
//    dc are summed with permlane swaps (stride 16).
// The cache at `pos` is stale while the range holding pos (first head of the group) writes the new
// k/v, so the score at pos is recomputed from the roped k in LDS and the V row at pos is replaced
// by the new v. Calls on one device must be stream-ordered (the partials and counters are shared).
//
// Numerics: RoPE as the reference's fp16 torch ops (cos/sin of pos * inv_freq in fp32 rounded to
// fp16, q*cos and rotate_half(q)*sin each rounded to fp16, their sum rounded); scores from the
// fp16 q and K with fp32 accumulation (v_dot2_f32_f16); softmax in fp32 with its numerators
// rounded to fp16 before they weight V (the reference's softmax(...).to(fp16) @ v), the V sum
// and the normalisation in fp32, the output rounded once to fp16.
#include <algorithm>

#include "ldk_common.h"

namespace {

constexpr int kHD = 128;
constexpr int kMaxWaves = 8;
constexpr int kChunk = 64;  // positions per wave pass
constexpr int64_t kMaxLen = 1 << 20;
constexpr int kMaxSplits = 32;  // position ranges per head
constexpr int kMaxHeads = 64;   // query heads that can split (more heads run one range each)
// s_waitcnt immediate (gfx9 encoding): vmcnt 0, expcnt and lgkmcnt unconstrained
constexpr int kWaitVmcnt0 = 0x0F70;

constexpr int kMinChunksPerSplit = 8;  // a range keeps >= 8 chunks (512 positions) of work
// Partials of the ranges of a launch in progress: {m, l} per [head][range], o per
// [head][dim][range] (a dim's partials of every range are contiguous for the merge), and per head
// the number of ranges that have published theirs (0 between launches).
__device__ float g_ml[kMaxHeads][kMaxSplits][2];
__device__ __align__(16) float g_o[kMaxHeads][kHD][kMaxSplits];
__device__ uint32_t g_arrive[kMaxHeads];
// buffer-load cache policy: sc1, read at the device coherence point (as agent-scope atomic loads)
constexpr int kCoherent = 16;

struct AttnArgs {
  const half_t* qkv;
  const int64_t* pos;
  const float* inv_freq;  // [64]
  half_t* kt;             // [nkv][128][max_len]
  half_t* v;              // [nkv][max_len][128]
  half_t* out;            // [nq*128]
  int nq, nkv, max_len;
  int cps;                // 64-position chunks per range (gridDim.y ranges)
  int xcd_group;          // 1: gridDim.x = 8 * (nq / nkv); workgroup x takes query head j of kv head
                          // x % 8 (j = x / 8), and exits at once for x % 8 >= nkv
  float scale;
};

// fp16 RoPE of the pair (x[d], x[d + 64]) of a 128-vector, d < 64 (rotate_half pairs d with
// d + 64): returns (x[d] c - x[d+64] s, x[d+64] c + x[d] s) with the reference's fp16 roundings.
__device__ __forceinline__ void rope_pair(const half_t* x, int d, float ang, half_t* lo, half_t* hi) {
  const half_t c = (half_t)cosf(ang), s = (half_t)sinf(ang);
  const half_t x0 = x[d], x1 = x[d + 64];
  const half_t a0 = (half_t)((float)x0 * (float)c), b0 = (half_t)(-(float)x1 * (float)s);
  const half_t a1 = (half_t)((float)x1 * (float)c), b1 = (half_t)((float)x0 * (float)s);
  *lo = (half_t)((float)a0 + (float)b0);
  *hi = (half_t)((float)a1 + (float)b1);
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {  // (lo16(a), lo16(b))
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {  // (hi16(a), hi16(b))
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// Max over the 16 lanes of a DPP row.
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, ldk::row_ror<1>(v));
  v = fmaxf(v, ldk::row_ror<2>(v));
  v = fmaxf(v, ldk::row_ror<4>(v));
  return fmaxf(v, ldk::row_ror<8>(v));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += ldk::row_ror<1>(v);
  v += ldk::row_ror<2>(v);
  v += ldk::row_ror<4>(v);
  return v + ldk::row_ror<8>(v);
}

__global__ __launch_bounds__(kMaxWaves * 64) void decode_attention_kernel(AttnArgs a) {
  __shared__ float qs[kHD];                    // roped q of this head (fp16 values)
  __shared__ half_t knew[kHD], vnew[kHD];      // roped new k, new v
  __shared__ __align__(16) float pw[kMaxWaves][kChunk];  // softmax numerators of a wave's chunk
  __shared__ __align__(16) float ow[kMaxWaves][kHD];     // per-wave unnormalized outputs
  __shared__ float mw[kMaxWaves], lw[kMaxWaves];
  __shared__ int last_flag;
  // The query heads of one kv head read the same K and V: placing them on one XCD (workgroups
  // are dispatched to the 8 XCDs round-robin) lets its L2 serve the group from one fetch
  // (max_len 384: 8.3 -> 8.0 us at pos 300).
  const int gq = a.nq / a.nkv;
  if (a.xcd_group && (int)(blockIdx.x % 8) >= a.nkv) return;
  const int h = a.xcd_group ? (int)(blockIdx.x % 8) * gq + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  const int split = blockIdx.y, nsplit = gridDim.y;
  const int g = a.nq / a.nkv, kvh = h / g;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int L = a.max_len;
  const int64_t pos_in = *a.pos;
  const bool pos_ok = pos_in >= 0 && pos_in < L;  // else: attend over the cache, write nothing
  const int pos = pos_ok ? (int)pos_in : pos_in < 0 ? -1 : L - 1;  // last live position
  const int npos = (int)pos_in;
  // ranges [s0, s0 + S) holding live positions; the first one is live even with none (pos < 0)
  const int S = a.cps * kChunk, s0 = split * S;
  const int nlive = pos < 0 ? 1 : pos / S + 1;
  if (split >= nlive) return;  // uniform over the workgroup
  const int cend = min(s0 + S, pos + 1);  // chunk starts c0 < cend have live positions
  const half_t* q = a.qkv + (int64_t)h * kHD;
  const half_t* kx = a.qkv + (int64_t)a.nq * kHD + (int64_t)kvh * kHD;
  const half_t* vx = kx + (int64_t)a.nkv * kHD;
  half_t* kt = a.kt + (int64_t)kvh * kHD * L;
  half_t* vc = a.v + (int64_t)kvh * L * kHD;

  const int pg = lane & 7, dg = lane >> 3;    // score lanes
  const int dc = lane & 15, pr = lane >> 4;   // output lanes

  // ---- first chunk's loads go out before the RoPE work, so both latencies overlap
  int c0 = s0 + wave * kChunk;
  u32x4 kr[16], vr[16];
  auto issue = [&](int base) {
    const int p8 = min(base + 8 * pg, L - 8);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      kr[i] = *reinterpret_cast<const u32x4*>(kt + (int64_t)(dg + 8 * i) * L + p8);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int p = min(base + 16 * pr + i, L - 1);
      vr[i] = *reinterpret_cast<const u32x4*>(vc + (int64_t)p * kHD + 8 * dc);
    }
  };
  if (c0 < cend) issue(c0);

  // ---- RoPE (q, new k) on dims (d, d + 64), stage the new k/v; the range holding pos writes them
  // to the cache (first head of the group)
  if (tid < 64) {
    const float ang = (float)pos_in * a.inv_freq[tid];
    half_t lo, hi;
    rope_pair(q, tid, ang, &lo, &hi);
    qs[tid] = (float)lo;
    qs[tid + 64] = (float)hi;
    rope_pair(kx, tid, ang, &lo, &hi);
    knew[tid] = lo;
    knew[tid + 64] = hi;
    const half_t v0 = vx[tid], v1 = vx[tid + 64];
    vnew[tid] = v0;
    vnew[tid + 64] = v1;
    if (h % g == 0 && pos_ok && npos >= s0 && npos < s0 + S) {
      kt[(int64_t)tid * L + npos] = lo;
      kt[(int64_t)(tid + 64) * L + npos] = hi;
      vc[(int64_t)npos * kHD + tid] = v0;
      vc[(int64_t)npos * kHD + tid + 64] = v1;
    }
  }
  ldk::lds_barrier();

  // score of the new token at pos (the cache row there is stale): q . knew, over the wave
  float s_new = 0.0f;
  if (pos_ok) {
    s_new = qs[lane] * (float)knew[lane] + qs[lane + 64] * (float)knew[lane + 64];
    s_new = ldk::sum_lanes_strided<1>(s_new) * a.scale;
  }
  half2_t qp[8];  // (q[dg + 16r], q[dg + 16r + 8]): the roped q is exactly fp16
#pragma unroll
  for (int r = 0; r < 8; ++r) qp[r] = half2_t{(half_t)qs[dg + 16 * r], (half_t)qs[dg + 16 * r + 8]};

  float m_run = -__builtin_inff(), l_run = 0.0f;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;

  for (; c0 < cend; c0 += nw * kChunk) {
    // ---- partial scores for positions c0 + 8pg + j over rows dg + 8i: rows 2r and 2r+1 are
    // paired with v_perm_b32 and meet the q pair in one v_dot2_f32_f16
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a0 = kr[2 * r][j], a1 = kr[2 * r + 1][j];
        s[2 * j] = __builtin_amdgcn_fdot2(qp[r], ldk::u2h2(perm_lo(a0, a1)), s[2 * j], false);
        s[2 * j + 1] = __builtin_amdgcn_fdot2(qp[r], ldk::u2h2(perm_hi(a0, a1)), s[2 * j + 1], false);
      }
    }
    float mloc = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int p = c0 + 8 * pg + j;
      float sj = ldk::sum_lanes_strided<8>(s[j]) * a.scale;
      if (pos_ok && p == npos) sj = s_new;
      s[j] = p <= pos ? sj : -__builtin_inff();
      mloc = fmaxf(mloc, s[j]);
    }
    const float mc = row_max16(mloc);  // chunk max (position c0 is live, so finite)
    const float m_new = fmaxf(m_run, mc);
    const float alpha = __expf(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s[j] = __expf(s[j] - m_new);  // 0 for masked positions
      lsum += s[j];
    }
    l_run = l_run * alpha + row_sum16(lsum) * 0.5f;  // the row holds every pg twice
    m_run = m_new;
    if (dg == 0) {
      *reinterpret_cast<float4_t*>(&pw[wave][8 * pg]) = float4_t{s[0], s[1], s[2], s[3]};
      *reinterpret_cast<float4_t*>(&pw[wave][8 * pg + 4]) = float4_t{s[4], s[5], s[6], s[7]};
    }
    ldk::wave_lds_sync();
    // ---- weighted V rows 16pr + i, dims 8dc + e: the weights are rounded to fp16 (the
    // reference's softmax(...).to(fp16)), rows 2r and 2r+1 paired for v_dot2_f32_f16. The new
    // token's row comes from vnew.
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4_t t = *reinterpret_cast<const float4_t*>(&pw[wave][16 * pr + i]);
      pv[i] = t[0];
      pv[i + 1] = t[1];
      pv[i + 2] = t[2];
      pv[i + 3] = t[3];
    }
    float p_new = 0.0f;
    if (pos_ok && npos >= c0 && npos < c0 + kChunk) {
      const int off = npos - c0;
      p_new = (float)(half_t)pw[wave][off];  // uniform
      if ((off >> 4) == pr) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i == (off & 15)) pv[i] = 0.0f;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const half2_t pp = {(half_t)pv[2 * r], (half_t)pv[2 * r + 1]};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a0 = vr[2 * r][j], a1 = vr[2 * r + 1][j];
        o[2 * j] = __builtin_amdgcn_fdot2(pp, ldk::u2h2(perm_lo(a0, a1)), o[2 * j], false);
        o[2 * j + 1] = __builtin_amdgcn_fdot2(pp, ldk::u2h2(perm_hi(a0, a1)), o[2 * j + 1], false);
      }
    }
    if (p_new != 0.0f && pr == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(p_new, (float)vnew[8 * dc + e], o[e]);
    }
    ldk::wave_lds_sync();  // pw is rewritten by the next chunk
    if (c0 + nw * kChunk < cend) issue(c0 + nw * kChunk);
  }
  // ---- lanes sharing dc hold parts of the same 8 outputs: sum over pr
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = ldk::sum_lanes_strided<16>(o[e]);
  if (pr == 0) {
    *reinterpret_cast<float4_t*>(&ow[wave][8 * dc]) = float4_t{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<float4_t*>(&ow[wave][8 * dc + 4]) = float4_t{o[4], o[5], o[6], o[7]};
  }
  if (lane == 0) {
    mw[wave] = m_run;
    lw[wave] = l_run;
  }
  ldk::lds_barrier();
  // ---- merge the waves of this range: threads < 64 take dims d and d + 64
  float M = -__builtin_inff(), l = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
  if (tid < 64) {
    for (int w = 0; w < nw; ++w) M = fmaxf(M, mw[w]);
    for (int w = 0; w < nw; ++w) {
      const float f = mw[w] == -__builtin_inff() ? 0.0f : __expf(mw[w] - M);
      l = __builtin_fmaf(lw[w], f, l);
      acc0 = __builtin_fmaf(ow[w][tid], f, acc0);
      acc1 = __builtin_fmaf(ow[w][tid + 64], f, acc1);
    }
  }
  half_t* out = a.out + (int64_t)h * kHD;
  if (nlive == 1) {  // the only live range: final output
    if (tid < 64) {
      out[tid] = (half_t)(l > 0.0f ? acc0 / l : 0.0f);
      out[tid + 64] = (half_t)(l > 0.0f ? acc1 / l : 0.0f);
    }
    return;
  }
  // ---- publish this range's partial, count in; the last range to arrive merges them all.
  // The partials move only through accesses performed at the device coherence point (sc1:
  // agent-scope atomic stores, buffer loads with sc1). All stores are wave 0's, which waits for
  // their completion (s_waitcnt vmcnt(0)) before its thread 0 bumps the counter, and the reads are
  // issued after the counter's value has returned, so the counter needs no release/acquire of its
  // own: those write back and invalidate the XCD's whole L2 in every workgroup.
  if (tid < 64) {
    __hip_atomic_store(&g_o[h][tid][split], acc0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&g_o[h][tid + 64][split], acc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(&g_ml[h][split][0], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&g_ml[h][split][1], l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this wave's partial stores have completed
      const uint32_t before = __hip_atomic_fetch_add(&g_arrive[h], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = before == (uint32_t)(nlive - 1);
    }
  }
  __syncthreads();
  if (!last_flag || tid >= 64) return;
  // ---- merge (wave 0 of the last range): lane r < nlive holds range r's (m, l); every lane then
  // reads the 32 range partials of its dims d and d + 64 with 16-byte loads, all in flight at once
  const int r = min(lane, nlive - 1);
  const float mr = __hip_atomic_load(&g_ml[h][r][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float lr = __hip_atomic_load(&g_ml[h][r][1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const auto ob = ldk::buffer_rsrc(&g_o[h][0][0], (uint32_t)sizeof(g_o[0]));
  u32x4 ov[2][kMaxSplits / 4];
#pragma unroll
  for (int k = 0; k < kMaxSplits / 4; ++k) {
    ov[0][k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ob, (uint32_t)((tid * kMaxSplits + 4 * k) * 4), 0, kCoherent));
    ov[1][k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ob, (uint32_t)(((tid + 64) * kMaxSplits + 4 * k) * 4), 0, kCoherent));
  }
  float Mg = lane < nlive ? mr : -__builtin_inff();
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) Mg = fmaxf(Mg, __shfl_xor(Mg, off));
  const float fr = lane < nlive ? __expf(mr - Mg) : 0.0f;  // weight of range `lane`
  float lg = lr * fr;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lg += __shfl_xor(lg, off);
  float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxSplits / 4; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = 4 * k + e;
      const float f = __shfl(fr, rr);  // 0 past the live ranges, whose stale words are skipped
      if (rr < nlive) {
        o0 = __builtin_fmaf(ldk::u2f(ov[0][k][e]), f, o0);
        o1 = __builtin_fmaf(ldk::u2f(ov[1][k][e]), f, o1);
      }
    }
  }
  out[tid] = (half_t)(lg > 0.0f ? o0 / lg : 0.0f);
  out[tid + 64] = (half_t)(lg > 0.0f ? o1 / lg : 0.0f);
  if (tid == 0) __hip_atomic_store(&g_arrive[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" int ldk_decode_attention(const void* qkv, const int64_t* pos, const float* inv_freq, void* kt_cache,
                                    void* v_cache, void* out, int nq, int nkv, int head_dim, int64_t max_len,
                                    float scale, void* stream) {
  if (!qkv || !pos || !inv_freq || !kt_cache || !v_cache || !out) return ldk::fail(LDK_ERR_INVALID, "decode_attention: null pointer");
  if (head_dim != kHD) return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: head_dim=%d (only 128)", head_dim);
  if (nq <= 0 || nkv <= 0 || nq % nkv) return ldk::fail(LDK_ERR_INVALID, "decode_attention: nq=%d must be a positive multiple of nkv=%d", nq, nkv);
  if (max_len < 8 || max_len > kMaxLen || max_len % 8)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: max_len=%lld must be a multiple of 8 in 8..%lld",
                     (long long)max_len, (long long)kMaxLen);
  if (!ldk::aligned(kt_cache, 16) || !ldk::aligned(v_cache, 16) || !ldk::aligned(pos, 8))
    return ldk::fail(LDK_ERR_ALIGN, "decode_attention: kt_cache and v_cache 16-byte, pos 8-byte aligned");
  // position ranges: at most kMaxSplits of at least kMinChunksPerSplit whole 64-position chunks
  // (one range per head when the heads exceed the partials' capacity); one wave per chunk of a
  // range, up to 8. A split costs about three memory round trips to merge, so caches of up to
  // 512 positions run one range (measured at max_len 256: 6.3 us one range, 8.3 us four).
  const int64_t nchunks = (max_len + kChunk - 1) / kChunk;
  const int64_t cps = nq <= kMaxHeads ? std::max<int64_t>(kMinChunksPerSplit, (nchunks + kMaxSplits - 1) / kMaxSplits)
                                      : nchunks;
  const int nsplit = (int)((nchunks + cps - 1) / cps);
  const int nw = (int)std::min<int64_t>(kMaxWaves, cps);
  const AttnArgs a{(const half_t*)qkv, pos, inv_freq, (half_t*)kt_cache, (half_t*)v_cache, (half_t*)out,
                   nq, nkv, (int)max_len, (int)cps, nkv <= 8 ? 1 : 0, scale};
  (void)hipGetLastError();
  decode_attention_kernel<<<dim3(nkv <= 8 ? 8 * (nq / nkv) : nq, nsplit), nw * 64, 0, (hipStream_t)stream>>>(a);
  return ldk::check_launch("decode_attention");
}
