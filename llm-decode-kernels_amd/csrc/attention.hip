// Fused decode attention for one new token (T = 1, batch 1): RoPE on q and k, the KV-cache write
// at `pos` and grouped-query softmax attention over positions 0..pos, in one launch per layer.
//
// Replaces the per-layer attention block of the reference's runner (kernels/e2e/model.py:
// 212-243: RoPE with rotate_half, k/v index_copy_ into the static cache, SDPA with a causal
// mask) for decode steps, where that block is ~20 small launches per layer.
//
// Layout: qkv [nq*128 | nkv*128 | nkv*128] fp16 (projection output, bias added, before RoPE);
// out [nq*128] fp16. The cache is kept in the matrix cores' operand order, in 1 KB tiles that are
// each exactly one 16-byte load per lane of a wave (8 whole 128-byte lines per load instruction;
// lane (c16, kb) = (l % 16, l / 16) reads row c16, bytes 16kb .. 16kb + 15):
//  - K, per kv head: [max_len/32 chunks][2 row halves hb][4 dim steps s][16 rows i][32 dims]; row
//    i of half hb of chunk c holds position 32c + 8(i/4) + 4hb + i%4, dims 32s .. 32s + 31;
//  - V^T, per kv head: [max_len/32 steps][8 dim blocks][16 dims][32 positions]; tile (t, b) holds
//    dims 16b .. 16b + 15 at positions 32t .. 32t + 31.
// max_len is a multiple of 32.
//
// Work split. One workgroup of NW waves (8; 4 where a range holds at most 4 chunks) serves up to
// 16 query heads of one kv head (all of them for every GQA shape up to 16 heads per kv head), so
// each K and V byte of a head is read once per launch, and its products run on the matrix cores
// (v_mfma_f32_16x16x32_f16, the 16 heads are the tile's columns). Caches of more than 512 positions are cut into up to 32 position ranges
// of at least 128 positions, with one workgroup per (head tile, range).
//  - Wave w takes the 32-position chunks w, w + NW, ... of its range, two at a time, and loads
//    each chunk's 8 K tiles and 8 V^T tiles (16 KB, all live) before its first use. The RoPE
//    needs no barrier: each lane ropes exactly the q and k dims of its own MFMA operands from
//    loads issued ahead of its first chunk's. The number of chunks in flight is a template
//    parameter, so every wait is a static count.
//  - Scores, S^T = K Q^T: one K tile is the A operand of one MFMA (16 positions x 32 dims), B is
//    the roped q of the 16 heads from LDS. The tile's row order leaves lane (head c16, kb) holding
//    positions 8kb .. 8kb + 7 of the chunk, which is exactly its A operand of P.V: the softmax
//    numerators exp(s - m), rounded to fp16 (the reference's softmax(...).to(fp16)), stay in
//    registers. O = P V: one MFMA per V^T tile (16 dims), fp32 accumulators per wave, online
//    softmax across the wave's chunks, sums in fp32.
//  - The waves' (m, l, O) meet once through LDS at the end.
// The cache at pos is stale while the workgroup holding pos writes the new k/v, so the score at
// pos is taken from q . k_new and the V^T registers at pos are replaced by v_new. The rows past
// pos in the last live chunk may hold any bits (an earlier generation's, or never written): their
// scores are selected to -inf and their V^T entries zeroed in registers, so NaN or inf there
// cannot reach P.V as 0 x NaN.
// With several ranges, every range stores its partial (running max m, sum l, unnormalised output
// o[128] per head) to library-owned device memory, and a second launch on the same stream merges
// them: the kernel boundary orders the stores before the loads, which a last-arriver merge inside
// the range kernel pays for with three device-coherent round trips (partial stores, a counter
// atomic, partial loads). Calls on one device must be stream-ordered (the partials are shared).
// The range entry can give the launch extra workgroups, dispatched after the attention's, that
// read byte ranges (the next projections' weights) into the caches while the attention's few
// workgroups leave the other CUs idle.
//
// Numerics: RoPE as the reference's fp16 torch ops (cos/sin of pos * inv_freq in fp32 rounded to
// fp16, q*cos and rotate_half(q)*sin each rounded to fp16, their sum rounded); scores from the
// fp16 q and K with fp32 accumulation; softmax in fp32 with its numerators rounded to fp16 before
// they weight V, the V sum and the normalisation in fp32, the output rounded once to fp16.
#include <algorithm>
#include <mutex>

#include "attention.h"
#include "ldk_common.h"
#include "warm.h"

namespace {

constexpr int kHD = 128;
constexpr int kTile = 16;    // query heads per workgroup: the MFMA tile's 16 columns
constexpr int kChunk = 32;   // positions per score chunk and per P.V step
constexpr int kBlock = 512;  // positions per softmax block: 16 chunks, two per wave
constexpr int64_t kMaxLen = 1 << 20;
constexpr int kMaxSplits = ldk::kAttnMaxSplits;  // position ranges per head tile
constexpr int kMaxHeads = ldk::kAttnMaxHeads;    // query heads that can split (more run one range per tile)
static_assert(kHD == ldk::kAttnHeadDim, "head_dim of the partials");
constexpr uint32_t kDead = 0x80000000u;  // buffer offset past every resource: the load returns 0
constexpr int kTileHalves = 512;         // halves per 1 KB cache tile

// Cache tile offsets (in halves, from the kv head's base) of K at (position p, dim d) and of V^T
// at (d, p).
__device__ __forceinline__ int k_offset(int p, int d) {
  const int q = p & 31, i = 4 * (q >> 3) + (q & 3), hb = (q >> 2) & 1;
  return (((p >> 5) * 2 + hb) * 4 + (d >> 5)) * kTileHalves + i * 32 + (d & 31);
}
__device__ __forceinline__ int vt_offset(int d, int p) {
  return ((p >> 5) * 8 + (d >> 4)) * kTileHalves + (d & 15) * 32 + (p & 31);
}

// Partials of the ranges of a launch in progress: {m, l} per [head][range] and o per
// [head][range][dim] (a range writes whole lines), written by the range kernel and read by the
// merge launch after it on the same stream.
__device__ float g_ml[kMaxHeads][kMaxSplits][2];
__device__ __align__(16) float g_o[kMaxHeads][kMaxSplits][kHD];

struct AttnArgs {
  const half_t* qkv;
  const int64_t* pos;
  const float* inv_freq;  // [64]
  half_t* k;              // K tiles, [nkv][max_len/32][2][4][16][32]
  half_t* vt;             // V^T tiles, [nkv][max_len/32][8][16][32]
  half_t* out;            // [nq*128]
  int nq, nkv, max_len;
  int ntile;              // workgroups per kv head along x: ceil((nq / nkv) / 16) head tiles
  int rlen;               // positions per range, a multiple of 32
  float scale;
  int partials;           // 1: every range writes its partials, also a lone live range (no output)
  int nattn;              // attention workgroups (nkv * ntile * ranges); the ones after them warm
  ldk::WarmRanges warm;
};

// fp16 RoPE of the pair (x0, x1) = (x[d], x[d + 64]) of a 128-vector (rotate_half pairs d with
// d + 64), c and s the fp16 cos and sin of its angle: (x0 c - x1 s, x1 c + x0 s) with the
// reference's fp16 roundings, in place.
__device__ __forceinline__ void rope_rotate(half_t& x0, half_t& x1, half_t c, half_t s) {
  const half_t a0 = (half_t)((float)x0 * (float)c), b0 = (half_t)(-(float)x1 * (float)s);
  const half_t a1 = (half_t)((float)x1 * (float)c), b1 = (half_t)((float)x0 * (float)s);
  x0 = (half_t)((float)a0 + (float)b0);
  x1 = (half_t)((float)a1 + (float)b1);
}

// max(v(lane i), v(lane i ^ 16)) and max(v(lane i), v(lane i ^ 32)) with gfx950's permlane swaps
// (the argument of ldk::add_xor16 / add_xor32 with max in place of the sum).
__device__ __forceinline__ float max_xor16(float v) {
  auto p = __builtin_amdgcn_permlane16_swap(ldk::f2u(v), ldk::f2u(v), false, false);
  return fmaxf(ldk::u2f(p[0]), ldk::u2f(p[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  auto p = __builtin_amdgcn_permlane32_swap(ldk::f2u(v), ldk::f2u(v), false, false);
  return fmaxf(ldk::u2f(p[0]), ldk::u2f(p[1]));
}

// Maximum over the 64 lanes, in every lane (row rotations, then the permlane swaps).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, ldk::row_ror<1>(v));
  v = fmaxf(v, ldk::row_ror<2>(v));
  v = fmaxf(v, ldk::row_ror<4>(v));
  v = fmaxf(v, ldk::row_ror<8>(v));
  return max_xor32(max_xor16(v));
}

__device__ __forceinline__ float4_t mfma16(u32x4 a, u32x4 b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}

// Clears the V^T operand entries of the positions past the last one attended to. In each of a
// chunk's 8 V^T tiles, lane (c16, kb) holds 8 consecutive positions of one dim, entry e (the
// halves of dword e / 2) at position 8kb + e of the chunk; entries e > last are zeroed. Their
// softmax weights are exactly 0, but those cache rows are not this call's data and may hold any
// bits, and 0 x NaN or 0 x inf in P.V would be NaN. Finite values there give the same sums with
// or without the clearing.
__device__ __forceinline__ void keep_v_through(u32x4 (&v)[8], int last) {
  uint32_t mk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) mk[j] = (2 * j <= last ? 0x0000FFFFu : 0u) | (2 * j + 1 <= last ? 0xFFFF0000u : 0u);
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) v[t][j] &= mk[j];
}

// Warming workgroups (warm.h) of the attention's launch: 128 KB each (16 loads per lane at 8
// waves, 32 at 4), at most one per CU beside the attention's.
constexpr int kWarmLoads = 16;  // per lane at 8 waves
constexpr int kWarmWorkgroups = 248;

// Waves per attention workgroup: 4 where a range holds at most 4 chunks (each wave one chunk; 8
// waves would leave four with no chunk that still rope their operands and join the LDS merge),
// else 8. Graph-timed at a 416-position cache in ranges of 128: the range launch 5.50 / 6.00 /
// 6.35 -> 5.14 / 5.24 / 5.54 us at pos 130 / 250 / 383.
int attn_waves(int64_t rlen) { return rlen <= 4 * kChunk ? 4 : 8; }
constexpr int warm_loads(int nw) { return kWarmLoads * 8 / nw; }

template <int N>
struct IntC {
  static constexpr int value = N;
};

template <int NW>
__global__ __launch_bounds__(NW * 64) void decode_attention_kernel(AttnArgs a) {
  __shared__ __align__(16) half_t vnew[NW][kHD];     // v_new by dim, one copy per wave
  __shared__ __align__(16) half_t knew[kHD];              // the roped k_new, for wave 0's cache write
  __shared__ __align__(16) half_t cs[NW][2][64];      // RoPE cos, sin by dim, per wave
  __shared__ float mw[NW][kTile], lw[NW][kTile];  // per-wave max and sum per head
  __shared__ __align__(16) float ow[NW][kTile][kHD];  // per-wave unnormalised outputs
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches, no waterfalls
  const int c16 = lane & 15, kb = lane >> 4;
  const int gq = a.nq / a.nkv;
  if ((int)blockIdx.x >= a.nattn) {  // uniform: a warming workgroup (dispatched after the attention's)
    ldk::warm_read<NW * 64, warm_loads(NW)>(a.warm, blockIdx.x - a.nattn);
    return;
  }
  // workgroup b = split * (nkv * ntile) + kvh * ntile + tile
  const int xy = a.nkv * a.ntile, bxy = (int)blockIdx.x % xy;
  const int kvh = bxy / a.ntile, tile = bxy % a.ntile;
  const int hbase = kvh * gq + tile * kTile;      // first query head of this workgroup
  const int nh = min(kTile, gq - tile * kTile);   // its heads
  const int split = (int)blockIdx.x / xy;
  const int L = a.max_len;
  const int64_t pos_in = *a.pos;
  const bool pos_ok = pos_in >= 0 && pos_in < L;  // else: attend over the cache, write nothing
  const int pos = pos_ok ? (int)pos_in : pos_in < 0 ? -1 : L - 1;  // last live position
  const int npos = pos_ok ? (int)pos_in : -1;                       // the row replaced this step
  // ranges [s0, s0 + S) holding live positions; the first one is live even with none (pos < 0)
  const int S = a.rlen, s0 = split * S;
  const int nlive = pos < 0 ? 1 : pos / S + 1;
  if (split >= nlive) return;  // uniform over the workgroup
  const int cend = min(s0 + S, pos + 1);  // live positions [s0, cend): empty when pos < 0
  const int ncl = cend > s0 ? (cend - s0 + kChunk - 1) / kChunk : 0;  // live chunks of the range
  const int nk = ncl > wave ? (ncl - wave + NW - 1) / NW : 0; // this wave's chunks
  const auto krs = ldk::buffer_rsrc(a.k + (int64_t)kvh * L * kHD, (uint32_t)L * kHD * 2);
  const auto vrs = ldk::buffer_rsrc(a.vt + (int64_t)kvh * kHD * L, (uint32_t)L * kHD * 2);
  // a tile is 16 rows of 64 bytes; lane (c16, kb) takes row c16, bytes 16kb .. 16kb + 15 (its
  // operand: 8 consecutive dims of one position for K, 8 consecutive positions of one dim for V^T)
  const uint32_t lane_off = (uint32_t)(c16 * 64 + kb * 16);

  // ---- RoPE in registers, no barrier: lane (c16, kb) needs q of head c16 at dims 8kb + 32s .. +7
  // (s < 4, its B operands) and k_new at the same dims (for q . k_new). Those are 16 rotate_half
  // pairs (d, d + 64), d = 8kb + 32s' + e (s' < 2, e < 8): the lane loads them, with v_new at the
  // same dims and inv_freq[lane], ahead of its cache loads; each wave computes the 64 angles'
  // cos and sin once (one per lane) and ropes its own operands, so no wave waits for another
  // before its scores.
  const auto qrs = ldk::buffer_rsrc(a.qkv, (uint32_t)(a.nq + 2 * a.nkv) * kHD * 2);
  const auto frs = ldk::buffer_rsrc(a.inv_freq, 64 * 4);
  u32x4 qx[4], kx[4], vx[4];
  float fr;  // inv_freq[lane]: lane l computes the cos and sin of dim l's angle for its wave
  {
    uint32_t dq = c16 < nh ? 0u : kDead;  // opaque: the select stays a select
    asm volatile("" : "+v"(dq));
    const uint32_t oq = (uint32_t)((hbase + c16) * kHD * 2) | dq;
    const uint32_t ok = (uint32_t)((a.nq + kvh) * kHD * 2), ov = (uint32_t)((a.nq + a.nkv + kvh) * kHD * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t od = (uint32_t)((8 * kb + 32 * s) * 2);
      qx[s] = ldk::buffer_load16(qrs, oq + od);
      kx[s] = ldk::buffer_load16(qrs, ok + od);
      vx[s] = ldk::buffer_load16(qrs, ov + od);
    }
    fr = ldk::u2f(__builtin_amdgcn_raw_buffer_load_b32(frs, (uint32_t)(lane * 4), 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the cache loads (vmcnt retires in order)

  u32x4 qb[4];
  float s_new = 0.0f;
  auto rope = [&]() __attribute__((always_inline)) {
    // the 64 angles' fp16 cos and sin, one per lane, shared through the wave's own LDS row
    {
      const float ang = (float)pos_in * fr;
      cs[wave][0][lane] = (half_t)cosf(ang);
      cs[wave][1][lane] = (half_t)sinf(ang);
    }
    ldk::wave_lds_sync();
    half8_t qh[4], kh[4], ch[2], sh[2];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qh[s] = __builtin_bit_cast(half8_t, qx[s]);
      kh[s] = __builtin_bit_cast(half8_t, kx[s]);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      ch[s] = *reinterpret_cast<const half8_t*>(&cs[wave][0][8 * kb + 32 * s]);
      sh[s] = *reinterpret_cast<const half8_t*>(&cs[wave][1][8 * kb + 32 * s]);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const half_t c = ch[s][e], sn = sh[s][e];
        half_t x0 = qh[s][e], x1 = qh[s + 2][e];
        rope_rotate(x0, x1, c, sn);
        qh[s][e] = x0;
        qh[s + 2][e] = x1;
        x0 = kh[s][e];
        x1 = kh[s + 2][e];
        rope_rotate(x0, x1, c, sn);
        kh[s][e] = x0;
        kh[s + 2][e] = x1;
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qb[s] = __builtin_bit_cast(u32x4, qh[s]);
      const u32x4 kn = __builtin_bit_cast(u32x4, kh[s]);
#pragma unroll
      for (int e = 0; e < 4; ++e) s_new = __builtin_amdgcn_fdot2(ldk::u2h2(qb[s][e]), ldk::u2h2(kn[e]), s_new, false);
    }
    s_new = ldk::add_xor32(ldk::add_xor16(s_new)) * a.scale;
    // v_new by dim for this wave's V patch (wave-local LDS exchange)
    if (c16 == 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) *reinterpret_cast<u32x4*>(&vnew[wave][8 * kb + 32 * s]) = vx[s];
    }
    ldk::wave_lds_sync();
    // the writing wave keeps the roped k_new in LDS too; the cache stores themselves go out after
    // its last chunk (below): issued here, ahead of the remaining chunk loads, the 8 scattered V^T
    // stores held those loads' in-order vmcnt waits (0.2-0.5 us per launch)
    if (wave == 0 && c16 == 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) *reinterpret_cast<half8_t*>(&knew[8 * kb + 32 * s]) = kh[s];
    }
  };

  float m_run = -__builtin_inff(), l_lane = 0.0f;  // head c16's running max; this lane's sum
  float4_t o[8];  // O[heads 4kb .. 4kb+3][dim 16b + c16] per dim block b, unnormalised
#pragma unroll
  for (int b = 0; b < 8; ++b) o[b] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- NC chunks of this wave (its chunks k0, k0 + 1, ...): all their tiles loaded, then each
  // chunk's scores, online softmax and P.V in turn; FIRST runs the RoPE between the two
  auto chunks = [&](auto ncc, auto firstc, int k0) __attribute__((always_inline)) {
    constexpr int NC = decltype(ncc)::value;
    u32x4 kr[NC][8], vr[NC][8];
    auto load = [&](int n) __attribute__((always_inline)) {
      const int c = (s0 >> 5) + wave + NW * (k0 + n);
#pragma unroll
      for (int t = 0; t < 8; ++t) kr[n][t] = ldk::buffer_load16(krs, (uint32_t)((c * 8 + t) * kTileHalves * 2) + lane_off);
#pragma unroll
      for (int t = 0; t < 8; ++t) vr[n][t] = ldk::buffer_load16(vrs, (uint32_t)((c * 8 + t) * kTileHalves * 2) + lane_off);
    };
    // with the RoPE in between, the second chunk's loads go out once the RoPE inputs are dead
    // (their registers and one chunk's do not fit next to two chunks' at 2 waves per SIMD)
    load(0);
    if constexpr (decltype(firstc)::value) rope();
#pragma unroll
    for (int n = 1; n < NC; ++n) load(n);
#pragma unroll
    for (int n = 0; n < NC; ++n) {
      const int cb = s0 + kChunk * (wave + NW * (k0 + n));
      float4_t acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        acc[0] = mfma16(kr[n][s], qb[s], acc[0]);
        acc[1] = mfma16(kr[n][4 + s], qb[s], acc[1]);
      }
      float sv[8];
      float mc = -__builtin_inff();
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = cb + 8 * kb + 4 * hb + r;
          const float v = p == npos ? s_new : acc[hb][r] * a.scale;
          sv[4 * hb + r] = p <= pos ? v : -__builtin_inff();
          mc = fmaxf(mc, sv[4 * hb + r]);
        }
      }
      mc = max_xor32(max_xor16(mc));  // the chunk's max of head c16 (its first position is live)
      const float m_new = fmaxf(m_run, mc);
      const float alpha = __expf(m_run - m_new);
      m_run = m_new;
      half8_t ph;
      float ls = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = __expf(sv[e] - m_new);  // 0 for masked positions
        ls += x;
        ph[e] = (half_t)x;
      }
      l_lane = l_lane * alpha + ls;
      if (npos >= cb && npos < cb + kChunk && kb == ((npos - cb) >> 3)) {  // v_new replaces the
        const int e = npos & 7;                                             // stale V^T at pos
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          half8_t hv = __builtin_bit_cast(half8_t, vr[n][b]);
          hv[e] = vnew[wave][16 * b + c16];
          vr[n][b] = __builtin_bit_cast(u32x4, hv);
        }
      }
      if (cb + kChunk - 1 > pos) keep_v_through(vr[n], pos - cb - 8 * kb);  // uniform per wave
      // rescale O: the heads of this lane's accumulator rows are 4kb .. 4kb+3
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float al = __shfl(alpha, 4 * kb + r);
#pragma unroll
        for (int b = 0; b < 8; ++b) o[b][r] *= al;
      }
      const u32x4 pa = __builtin_bit_cast(u32x4, ph);
#pragma unroll
      for (int b = 0; b < 8; ++b) o[b] = mfma16(pa, vr[n][b], o[b]);
    }
  };
  const int first = min(nk, 2);
  if (first == 2)
    chunks(IntC<2>(), IntC<1>(), 0);
  else if (first == 1)
    chunks(IntC<1>(), IntC<1>(), 0);
  else
    rope();
  for (int k = 2; k < nk; k += 2) {  // longer ranges: further pairs
    if (nk - k >= 2)
      chunks(IntC<2>(), IntC<0>(), k);
    else
      chunks(IntC<1>(), IntC<0>(), k);
  }
  // the cache write at pos by wave 0 of the range holding pos (head tile 0): lanes c16 = 0 store
  // k_new's 8-dim runs (adjacent in a K tile row), lanes kb = 0 store v_new down the V^T tiles'
  // rows. This launch's scores and P.V took both from registers; later launches read them.
  if (wave == 0 && tile == 0 && npos >= s0 && npos < s0 + S) {
    if (c16 == 0) {
      half_t* kw = a.k + (int64_t)kvh * L * kHD;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        *reinterpret_cast<half8_t*>(&kw[k_offset(npos, 8 * kb + 32 * s)]) =
            *reinterpret_cast<const half8_t*>(&knew[8 * kb + 32 * s]);
    }
    if (kb == 0) {
      half_t* vw = a.vt + (int64_t)kvh * kHD * L;
#pragma unroll
      for (int b = 0; b < 8; ++b) vw[vt_offset(16 * b + c16, npos)] = vnew[0][16 * b + c16];
    }
  }

  // ---- the waves meet: per-wave (m, l) per head and O rows of the tile's live heads
  const float l_w = ldk::add_xor32(ldk::add_xor16(l_lane));
  if (kb == 0) {
    mw[wave][c16] = m_run;
    lw[wave][c16] = l_w;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (4 * kb + r < nh) {
#pragma unroll
      for (int b = 0; b < 8; ++b) ow[wave][4 * kb + r][16 * b + c16] = o[b][r];
    }
  ldk::lds_barrier();
  // thread item (head j, dim d): weights exp(m_w - M) of the waves that saw a live position. All
  // 3 x NW LDS reads are issued before the first use and the dead waves get weight 0 (their l
  // and O are 0, so the FMA adds nothing) instead of a branch, which made each wave's reads wait
  // for the previous wave's exp (0.65 us of a 6.4 us launch at 130 live positions)
  const bool single = nlive == 1 && !a.partials;
  for (int e = tid; e < nh * kHD; e += NW * 64) {
    const int j = e >> 7, d = e & (kHD - 1);
    float mv[NW], lv[NW], ov[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mv[w] = mw[w][j];
      lv[w] = lw[w][j];
      ov[w] = ow[w][j][d];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, mv[w]);
    float l = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = mv[w] != -__builtin_inff() ? __expf(mv[w] - M) : 0.0f;
      l = __builtin_fmaf(lv[w], f, l);
      acc = __builtin_fmaf(ov[w], f, acc);
    }
    if (single) {
      a.out[(int64_t)(hbase + j) * kHD + d] = (half_t)(l > 0.0f ? acc / l : 0.0f);
    } else {  // this range's partial, for the merge launch that follows on the stream
      g_o[hbase + j][split][d] = acc;
      if (d == 0) {
        g_ml[hbase + j][split][0] = M;
        g_ml[hbase + j][split][1] = l;
      }
    }
  }
}

// The ranges' partials of one query head (one wave per head, launched after the ranges on the
// same stream, so their stores are visible): lane r < nlive holds range r's (m, l); lane d reads
// dims d and d + 64 of every live range's partial (coalesced dword loads, all in flight at once,
// zero past the live ranges). With a single live range the range kernel has written the output
// and this returns at once.
__global__ __launch_bounds__(64) void attention_merge_kernel(const int64_t* pos_p, half_t* out, int L, int rlen) {
  const int64_t pos_in = *pos_p;
  const bool pos_ok = pos_in >= 0 && pos_in < L;
  const int pos = pos_ok ? (int)pos_in : pos_in < 0 ? -1 : L - 1;
  const int nlive = pos < 0 ? 1 : pos / rlen + 1;
  if (nlive == 1) return;
  const int h = blockIdx.x, lane = threadIdx.x;
  const int r = min(lane, nlive - 1);
  const float mr = g_ml[h][r][0], lr = g_ml[h][r][1];
  const auto ob = ldk::buffer_rsrc(&g_o[h][0][0], (uint32_t)sizeof(g_o[0]));
  float ov0[kMaxSplits], ov1[kMaxSplits];
#pragma unroll
  for (int k = 0; k < kMaxSplits; ++k) {
    const uint32_t off = (uint32_t)((k * kHD + lane) * 4) | (k < nlive ? 0u : kDead);
    ov0[k] = ldk::u2f(__builtin_amdgcn_raw_buffer_load_b32(ob, off, 0, 0));
    ov1[k] = ldk::u2f(__builtin_amdgcn_raw_buffer_load_b32(ob, off + 256, 0, 0));
  }
  const float Mg = wave_max(lane < nlive ? mr : -__builtin_inff());
  const float fr = lane < nlive ? __expf(mr - Mg) : 0.0f;  // weight of range `lane`
  const float lg = ldk::sum_lanes_strided<1>(lr * fr);
  float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxSplits; ++k) {
    // range k's weight, read into a scalar register (0 past the live ranges, whose loads read 0)
    const float f = ldk::u2f(__builtin_amdgcn_readlane(ldk::f2u(fr), k));
    o0 = __builtin_fmaf(ov0[k], f, o0);
    o1 = __builtin_fmaf(ov1[k], f, o1);
  }
  out[(int64_t)h * kHD + lane] = (half_t)(lg > 0.0f ? o0 / lg : 0.0f);
  out[(int64_t)h * kHD + lane + 64] = (half_t)(lg > 0.0f ? o1 / lg : 0.0f);
}

// ------------------------------------------------------------ prompt (many-token) attention
//
// ldk_prefill_attention: T tokens of one sequence at positions pos[T], in two launches.
//  1. prefill_rope_kv_kernel, one workgroup per token: the decode kernel's fp16 RoPE (same cos and
//     sin of pos * inv_freq, same roundings) on the token's q heads, written to q_scratch
//     [T][nq][128], and on its k heads, written with its v heads into the tiled caches at pos[t]
//     (a position outside [0, max_len) writes nothing).
//  2. prefill_attention_kernel, one workgroup per (block of 16 tokens, query head): the decode
//     kernel's score and P.V steps with the MFMA tile's 16 columns the block's tokens instead of
//     a kv head's query heads. Column c16 (token t0 + c16) attends to the cache positions
//     0..pos[t0 + c16] with its own mask, so every token is causal whatever the order of pos.
//     Wave w takes the 32-position chunks w, w + 4, ... up to the block's last position, two
//     chunks' tiles in flight at a time; the waves' (m, l, O) meet through LDS. The V^T entries
//     past the block's last position are zeroed in registers, as in the decode kernel.
// The launch boundary orders the cache writes of launch 1 before the reads of launch 2.
constexpr int kPWaves = 4;

__global__ __launch_bounds__(256) void prefill_rope_kv_kernel(const half_t* qkv, int64_t ldqkv, const int64_t* pos,
                                                              const float* inv_freq, half_t* kc, half_t* vt,
                                                              half_t* qs, int nq, int nkv, int L) {
  // every element a thread ropes has dim pair j = tid % 64 (the loops step by 256), so each thread
  // forms its own cos and sin: no shared table and no barrier, and the row loads need not wait
  // for the position
  const int t = blockIdx.x, tid = threadIdx.x, jt = tid & 63;
  const int64_t p = pos[t];
  const float ang = (float)p * inv_freq[jt];
  const half_t cj = (half_t)cosf(ang), sj = (half_t)sinf(ang);
  const half_t* row = qkv + (int64_t)t * ldqkv;
  half_t* qo = qs + (int64_t)t * nq * kHD;
  for (int e = tid; e < nq * 64; e += 256) {  // (head, dim pair j < 64): dims j and j + 64
    const int h = e >> 6, j = e & 63;
    half_t x0 = row[h * kHD + j], x1 = row[h * kHD + j + 64];
    rope_rotate(x0, x1, cj, sj);
    qo[h * kHD + j] = x0;
    qo[h * kHD + j + 64] = x1;
  }
  if (p < 0 || p >= L) return;  // uniform
  const int pp = (int)p;
  for (int e = tid; e < nkv * 64; e += 256) {
    const int h = e >> 6, j = e & 63;
    half_t x0 = row[(nq + h) * kHD + j], x1 = row[(nq + h) * kHD + j + 64];
    rope_rotate(x0, x1, cj, sj);
    half_t* kw = kc + (int64_t)h * L * kHD;
    kw[k_offset(pp, j)] = x0;
    kw[k_offset(pp, j + 64)] = x1;
  }
  for (int e = tid; e < nkv * kHD; e += 256) {
    const int h = e >> 7, d = e & (kHD - 1);
    vt[(int64_t)h * kHD * L + vt_offset(d, pp)] = row[(nq + nkv + h) * kHD + d];
  }
}

__global__ __launch_bounds__(kPWaves * 64) void prefill_attention_kernel(const half_t* qs, const int64_t* pos, int T,
                                                                        const half_t* kc, const half_t* vt, half_t* out,
                                                                        int64_t ldo, int nq, int nkv, int L,
                                                                        float scale) {
  __shared__ float mw[kPWaves][kTile], lw[kPWaves][kTile];
  __shared__ __align__(16) float ow[kPWaves][kTile][kHD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kb = lane >> 4;
  const int h = (int)blockIdx.y, t0 = (int)blockIdx.x * kTile;
  const int kvh = h / (nq / nkv);
  const int nt = min(kTile, T - t0);  // tokens of this block
  // this lane's column: token t0 + c16 and the last cache position it attends to (-1: none)
  int plim = -1;
  if (c16 < nt) {
    const int64_t pp = pos[t0 + c16];
    plim = pp < 0 ? -1 : pp >= L ? L - 1 : (int)pp;
  }
  const int pmax = (int)wave_max((float)plim);  // the block's last position (exact: < 2^24)
  const int nch = pmax < 0 ? 0 : pmax / kChunk + 1;
  const int nk = nch > wave ? (nch - wave + kPWaves - 1) / kPWaves : 0;  // this wave's chunks
  const auto krs = ldk::buffer_rsrc(kc + (int64_t)kvh * L * kHD, (uint32_t)L * kHD * 2);
  const auto vrs = ldk::buffer_rsrc(vt + (int64_t)kvh * kHD * L, (uint32_t)L * kHD * 2);
  const uint32_t lane_off = (uint32_t)(c16 * 64 + kb * 16);
  // B operands of the scores: lane (c16, kb) holds q of token t0 + c16 at dims 8kb + 32s .. +7
  u32x4 qb[4];
  {
    const auto qrs = ldk::buffer_rsrc(qs, (uint32_t)((int64_t)T * nq * kHD * 2));
    uint32_t dq = c16 < nt ? 0u : kDead;
    asm volatile("" : "+v"(dq));
    const uint32_t oq = (uint32_t)(((int64_t)(t0 + c16) * nq + h) * kHD * 2) | dq;
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = ldk::buffer_load16(qrs, oq + (uint32_t)((8 * kb + 32 * s) * 2));
  }

  float m_run = -__builtin_inff(), l_lane = 0.0f;  // token c16's running max; this lane's sum
  float4_t o[8];  // O[tokens 4kb .. 4kb+3][dim 16b + c16] per dim block b, unnormalised
#pragma unroll
  for (int b = 0; b < 8; ++b) o[b] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto chunks = [&](auto ncc, int k0) __attribute__((always_inline)) {
    constexpr int NC = decltype(ncc)::value;
    u32x4 kr[NC][8], vr[NC][8];
#pragma unroll
    for (int n = 0; n < NC; ++n) {
      const int c = wave + kPWaves * (k0 + n);
#pragma unroll
      for (int t = 0; t < 8; ++t) kr[n][t] = ldk::buffer_load16(krs, (uint32_t)((c * 8 + t) * kTileHalves * 2) + lane_off);
#pragma unroll
      for (int t = 0; t < 8; ++t) vr[n][t] = ldk::buffer_load16(vrs, (uint32_t)((c * 8 + t) * kTileHalves * 2) + lane_off);
    }
#pragma unroll
    for (int n = 0; n < NC; ++n) {
      const int cb = kChunk * (wave + kPWaves * (k0 + n));
      float4_t acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        acc[0] = mfma16(kr[n][s], qb[s], acc[0]);
        acc[1] = mfma16(kr[n][4 + s], qb[s], acc[1]);
      }
      float sv[8];
      float mc = -__builtin_inff();
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = cb + 8 * kb + 4 * hb + r;
          sv[4 * hb + r] = p <= plim ? acc[hb][r] * scale : -__builtin_inff();
          mc = fmaxf(mc, sv[4 * hb + r]);
        }
      }
      mc = max_xor32(max_xor16(mc));  // token c16's max over the chunk (-inf: none live)
      const float m_new = fmaxf(m_run, mc);
      // a token with no live position so far keeps m = -inf; its exponents are taken against 0
      // (every numerator is then exp(-inf) = 0) instead of the NaN of -inf - -inf
      const float m_ref = m_new == -__builtin_inff() ? 0.0f : m_new;
      const float alpha = __expf(m_run - m_ref);
      m_run = m_new;
      half8_t ph;
      float ls = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = __expf(sv[e] - m_ref);  // 0 for masked positions
        ls += x;
        ph[e] = (half_t)x;
      }
      l_lane = l_lane * alpha + ls;
      if (cb + kChunk - 1 > pmax) keep_v_through(vr[n], pmax - cb - 8 * kb);  // uniform per wave
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // the tokens of this lane's accumulator rows are 4kb .. 4kb+3
        const float al = __shfl(alpha, 4 * kb + r);
#pragma unroll
        for (int b = 0; b < 8; ++b) o[b][r] *= al;
      }
      const u32x4 pa = __builtin_bit_cast(u32x4, ph);
#pragma unroll
      for (int b = 0; b < 8; ++b) o[b] = mfma16(pa, vr[n][b], o[b]);
    }
  };
  for (int k = 0; k < nk; k += 2) {
    if (nk - k >= 2)
      chunks(IntC<2>(), k);
    else
      chunks(IntC<1>(), k);
  }

  // ---- the waves meet: per-wave (m, l) per token and O rows of the block's tokens
  const float l_w = ldk::add_xor32(ldk::add_xor16(l_lane));
  if (kb == 0) {
    mw[wave][c16] = m_run;
    lw[wave][c16] = l_w;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (4 * kb + r < nt) {
#pragma unroll
      for (int b = 0; b < 8; ++b) ow[wave][4 * kb + r][16 * b + c16] = o[b][r];
    }
  ldk::lds_barrier();
  for (int e = tid; e < nt * kHD; e += kPWaves * 64) {
    const int j = e >> 7, d = e & (kHD - 1);
    float mv[kPWaves], lv[kPWaves], ov[kPWaves];
#pragma unroll
    for (int w = 0; w < kPWaves; ++w) {
      mv[w] = mw[w][j];
      lv[w] = lw[w][j];
      ov[w] = ow[w][j][d];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kPWaves; ++w) M = fmaxf(M, mv[w]);
    float l = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w = 0; w < kPWaves; ++w) {
      const float f = mv[w] != -__builtin_inff() ? __expf(mv[w] - M) : 0.0f;
      l = __builtin_fmaf(lv[w], f, l);
      acc = __builtin_fmaf(ov[w], f, acc);
    }
    out[(int64_t)(t0 + j) * ldo + (int64_t)h * kHD + d] = (half_t)(l > 0.0f ? acc / l : 0.0f);
  }
}

}  // namespace

namespace ldk {
void note_partials(bool pending, void* stream, const int64_t* pos, int64_t max_len, int64_t rlen, int nq);
}  // namespace ldk

extern "C" int ldk_decode_attention(const void* qkv, const int64_t* pos, const float* inv_freq, void* k_cache,
                                    void* vt_cache, void* out, int nq, int nkv, int head_dim, int64_t max_len,
                                    float scale, const void* const* warm, const int64_t* warm_bytes, int nwarm,
                                    void* stream) {
  if (!qkv || !pos || !inv_freq || !k_cache || !vt_cache || !out) return ldk::fail(LDK_ERR_INVALID, "decode_attention: null pointer");
  if (head_dim != kHD) return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: head_dim=%d (only 128)", head_dim);
  if (nq <= 0 || nkv <= 0 || nq % nkv) return ldk::fail(LDK_ERR_INVALID, "decode_attention: nq=%d must be a positive multiple of nkv=%d", nq, nkv);
  if (max_len < kChunk || max_len > kMaxLen || max_len % kChunk)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention: max_len=%lld must be a multiple of 32 in 32..%lld",
                     (long long)max_len, (long long)kMaxLen);
  if (!ldk::aligned(k_cache, 16) || !ldk::aligned(vt_cache, 16) || !ldk::aligned(pos, 8))
    return ldk::fail(LDK_ERR_ALIGN, "decode_attention: k_cache and vt_cache 16-byte, pos 8-byte aligned");
  // Position ranges: a cache of up to 512 positions runs one range (splitting it costs more in
  // the merge launch than it saves: 384 at pos 300 runs 7.9 us whole, 8.9 us in 128-position
  // ranges); longer ones at most kMaxSplits ranges of at least 128 positions (4096 at pos 4000:
  // 9.5 us, 10.3 with 256-position ranges, 12.5 with 512). Caches with more heads than the
  // partials hold run one range per head tile.
  const int64_t nblocks = (max_len + kBlock - 1) / kBlock;
  const int64_t nchunk = max_len / kChunk;
  int64_t rlen;
  if (nblocks == 1)
    rlen = max_len;
  else if (nq > kMaxHeads)
    rlen = max_len;
  else
    rlen = std::max<int64_t>(128, (nchunk + kMaxSplits - 1) / kMaxSplits * kChunk);
  const int nsplit = (int)((max_len + rlen - 1) / rlen);
  const int gq = nq / nkv, ntile = (gq + kTile - 1) / kTile;
  ldk::WarmRanges w;
  uint32_t nwg = 0;
  const int nw = attn_waves(rlen);
  if (const int st = ldk::make_warm(warm, warm_bytes, nwarm, "decode_attention", nw * 64, warm_loads(nw),
                                    kWarmWorkgroups, w, nwg))
    return st;
  const int nattn = nkv * ntile * nsplit;
  const AttnArgs a{(const half_t*)qkv, pos, inv_freq, (half_t*)k_cache, (half_t*)vt_cache, (half_t*)out,
                   nq, nkv, (int)max_len, ntile, (int)rlen, scale, 0, nattn, w};
  (void)hipGetLastError();
  if (nw == 4)
    decode_attention_kernel<4><<<nattn + nwg, 4 * 64, 0, (hipStream_t)stream>>>(a);
  else
    decode_attention_kernel<8><<<nattn + nwg, 8 * 64, 0, (hipStream_t)stream>>>(a);
  if (nsplit > 1) {
    attention_merge_kernel<<<nq, 64, 0, (hipStream_t)stream>>>(pos, (half_t*)out, (int)max_len, (int)rlen);
    ldk::note_partials(false, stream, nullptr, 0, 0, 0);  // the partials of a pending range call are overwritten
  }
  return ldk::check_launch("decode_attention");
}

// Decode attention that leaves its result as per-range partials for a consumer that merges them
// (the W4A16 o projection's x staging, ldk_w4a16_attn_matmul_residual_stats): the range kernel of
// ldk_decode_attention with `rlen` positions per range, every range (a lone live one too) writing
// {m, l} and its unnormalised output to the library's partials, and no merge launch. Cache write
// and numerics as ldk_decode_attention.
extern "C" int ldk_decode_attention_ranges(const void* qkv, const int64_t* pos, const float* inv_freq, void* k_cache,
                                           void* vt_cache, int nq, int nkv, int head_dim, int64_t max_len,
                                           int64_t rlen, float scale, const void* const* warm,
                                           const int64_t* warm_bytes, int nwarm, void* stream) {
  if (!qkv || !pos || !inv_freq || !k_cache || !vt_cache) return ldk::fail(LDK_ERR_INVALID, "decode_attention_ranges: null pointer");
  if (head_dim != kHD) return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention_ranges: head_dim=%d (only 128)", head_dim);
  if (nq <= 0 || nkv <= 0 || nq % nkv) return ldk::fail(LDK_ERR_INVALID, "decode_attention_ranges: nq=%d must be a positive multiple of nkv=%d", nq, nkv);
  if (nq > kMaxHeads) return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention_ranges: nq=%d above %d heads", nq, kMaxHeads);
  if (max_len < kChunk || max_len > kMaxLen || max_len % kChunk)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention_ranges: max_len=%lld must be a multiple of 32 in 32..%lld",
                     (long long)max_len, (long long)kMaxLen);
  if (rlen < kChunk || rlen % kChunk || rlen > max_len || (max_len + rlen - 1) / rlen > kMaxSplits)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "decode_attention_ranges: rlen=%lld must be a multiple of 32 giving 1..%d ranges of %lld",
                     (long long)rlen, kMaxSplits, (long long)max_len);
  if (!ldk::aligned(k_cache, 16) || !ldk::aligned(vt_cache, 16) || !ldk::aligned(pos, 8))
    return ldk::fail(LDK_ERR_ALIGN, "decode_attention_ranges: k_cache and vt_cache 16-byte, pos 8-byte aligned");
  const int nsplit = (int)((max_len + rlen - 1) / rlen);
  const int gq = nq / nkv, ntile = (gq + kTile - 1) / kTile;
  ldk::WarmRanges w;
  uint32_t nwg = 0;
  const int nw = attn_waves(rlen);
  if (const int st = ldk::make_warm(warm, warm_bytes, nwarm, "decode_attention_ranges", nw * 64, warm_loads(nw),
                                    kWarmWorkgroups, w, nwg))
    return st;
  const int nattn = nkv * ntile * nsplit;
  const AttnArgs a{(const half_t*)qkv, pos, inv_freq, (half_t*)k_cache, (half_t*)vt_cache, nullptr,
                   nq, nkv, (int)max_len, ntile, (int)rlen, scale, 1, nattn, w};
  (void)hipGetLastError();
  if (nw == 4)
    decode_attention_kernel<4><<<nattn + nwg, 4 * 64, 0, (hipStream_t)stream>>>(a);
  else
    decode_attention_kernel<8><<<nattn + nwg, 8 * 64, 0, (hipStream_t)stream>>>(a);
  const int st = ldk::check_launch("decode_attention_ranges");
  ldk::note_partials(st == LDK_OK, stream, pos, max_len, rlen, nq);
  return st;
}

namespace ldk {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_part_mu;
const float* g_part_o[kMaxDevices];  // device addresses of g_o / g_ml per device, set on first use
const float* g_part_ml[kMaxDevices];
struct PartialsNote {  // the last ldk_decode_attention_ranges call per device
  bool pending;
  void* stream;
  const int64_t* pos;  // the position the ranges were written at
  int64_t max_len, rlen;
  int nq;
};
PartialsNote g_part_note[kMaxDevices];
}  // namespace

// Records (pending) or forgets the partials' producer on the current device.
void note_partials(bool pending, void* stream, const int64_t* pos, int64_t max_len, int64_t rlen, int nq) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_part_mu);
  g_part_note[dev] = PartialsNote{pending, stream, pos, max_len, rlen, nq};
}

int attention_partials(const char* what, void* stream, const int64_t* pos, int64_t max_len, int64_t rlen, int nq,
                       const float** o, const float** ml) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(LDK_ERR_LAUNCH, "%s: no current HIP device (or device %d >= %d)", what, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_part_mu);
  const PartialsNote& n = g_part_note[dev];
  if (!n.pending)
    return fail(LDK_ERR_INVALID, "%s: no ldk_decode_attention_ranges partials pending on device %d", what, dev);
  if (n.stream != stream)
    return fail(LDK_ERR_INVALID, "%s: the attention ranges were left on another stream; call it on the same stream", what);
  // the consumer recomputes the live ranges from its own *pos: another position array could name
  // ranges the producer did not write this step
  if (n.pos != pos)
    return fail(LDK_ERR_INVALID, "%s: pos is not the position array the attention ranges were written with", what);
  if (n.max_len != max_len || n.rlen != rlen || n.nq != nq)
    return fail(LDK_ERR_INVALID, "%s: max_len=%lld rlen=%lld nq=%d, the attention ranges were max_len=%lld rlen=%lld nq=%d",
                what, (long long)max_len, (long long)rlen, nq, (long long)n.max_len, (long long)n.rlen, n.nq);
  if (!g_part_o[dev]) {
    void* po = nullptr;
    void* pm = nullptr;
    const hipError_t e1 = hipGetSymbolAddress(&po, HIP_SYMBOL(g_o));
    const hipError_t e2 = hipGetSymbolAddress(&pm, HIP_SYMBOL(g_ml));
    if (e1 != hipSuccess || e2 != hipSuccess || !po || !pm)
      return fail(LDK_ERR_LAUNCH, "%s: hipGetSymbolAddress of the attention partials failed on device %d", what, dev);
    g_part_o[dev] = static_cast<const float*>(po);
    g_part_ml[dev] = static_cast<const float*>(pm);
  }
  *o = g_part_o[dev];
  *ml = g_part_ml[dev];
  return LDK_OK;
}

}  // namespace ldk

// Prompt attention (launches prefill_rope_kv_kernel, then prefill_attention_kernel).
extern "C" int ldk_prefill_attention(const void* qkv, int64_t ldqkv, const int64_t* pos, int64_t T, const float* inv_freq,
                                     void* k_cache, void* vt_cache, void* q_scratch, void* out, int64_t ldo, int nq,
                                     int nkv, int head_dim, int64_t max_len, float scale, void* stream) {
  static const char* fn = "prefill_attention";
  if (!qkv || !pos || !inv_freq || !k_cache || !vt_cache || !q_scratch || !out)
    return ldk::fail(LDK_ERR_INVALID, "%s: null pointer", fn);
  if (head_dim != kHD) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: head_dim=%d (only 128)", fn, head_dim);
  if (nq <= 0 || nkv <= 0 || nq % nkv || nq > 65535)
    return ldk::fail(LDK_ERR_INVALID, "%s: nq=%d must be a positive multiple of nkv=%d (at most 65535)", fn, nq, nkv);
  if (T <= 0 || T > (int64_t(1) << 24)) return ldk::fail(LDK_ERR_INVALID, "%s: T=%lld outside 1..2^24", fn, (long long)T);
  if (max_len < kChunk || max_len > kMaxLen || max_len % kChunk)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: max_len=%lld must be a multiple of 32 in 32..%lld", fn, (long long)max_len,
                     (long long)kMaxLen);
  if (ldqkv < (int64_t)(nq + 2 * nkv) * kHD || ldo < (int64_t)nq * kHD)
    return ldk::fail(LDK_ERR_INVALID, "%s: row strides ldqkv=%lld ldo=%lld below the rows", fn, (long long)ldqkv, (long long)ldo);
  // the q scratch is one buffer resource (32-bit offsets)
  if (T * nq * kHD * 2 > (int64_t)UINT32_MAX) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: T * nq too large", fn);
  if (!ldk::aligned(k_cache, 16) || !ldk::aligned(vt_cache, 16) || !ldk::aligned(q_scratch, 16) ||
      !ldk::aligned(qkv, 2) || !ldk::aligned(out, 2) || !ldk::aligned(pos, 8) || !ldk::aligned(inv_freq, 4))
    return ldk::fail(LDK_ERR_ALIGN, "%s: k_cache, vt_cache and q_scratch 16-byte, pos 8-byte aligned", fn);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  prefill_rope_kv_kernel<<<(unsigned)T, 256, 0, s>>>((const half_t*)qkv, ldqkv, pos, inv_freq, (half_t*)k_cache,
                                                     (half_t*)vt_cache, (half_t*)q_scratch, nq, nkv, (int)max_len);
  int st = ldk::check_launch("prefill_rope_kv");
  if (st) return st;
  const dim3 grid((unsigned)((T + kTile - 1) / kTile), (unsigned)nq);
  prefill_attention_kernel<<<grid, kPWaves * 64, 0, s>>>((const half_t*)q_scratch, pos, (int)T, (const half_t*)k_cache,
                                                         (const half_t*)vt_cache, (half_t*)out, ldo, nq, nkv,
                                                         (int)max_len, scale);
  return ldk::check_launch("prefill_attention");
}
