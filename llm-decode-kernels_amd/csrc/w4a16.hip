// W4A16 matmul for decode (M <= 16): y[M, N] = x[M, K] @ dequant(W)^T (+ bias).
//
// Replaces the reference's Triton GEMV/GEMM launch paths (kernels/w4a16.py:100-160, 214-279) and
// its CUDA decode kernel (kernels/cuda/w4a16_decode.cu:29-121) with one gfx950 design:
//
//  * Work split. A workgroup owns CW = 4*LN output columns and ALL of K. Inside it, LN lanes run
//    along N (each lane owns 4 adjacent columns, so one 128-bit load = one packed row of 4
//    columns = 32 weights) and LK = NW*64/LN lanes run along K ("split-K"), taking packed rows
//    lk, lk+LK, lk+2LK, ... The split is reduced inside the workgroup (DPP row rotations and
//    gfx950 permlane swaps within a wave, then LDS across waves), so there are no global atomics,
//    no zero-fill and no cast launches. The split factor comes from the per-shape table below.
//  * Memory-level parallelism. Every lane issues the loads of its whole batch of UB rows before
//    touching any of them and consumes them in issue order, so s_waitcnt vmcnt(n) releases each
//    row as it lands and the whole weight stream of the launch is in flight at once.
//  * Prologue. Before the weight loads, each thread issues its share of x (16 B) and of the
//    workgroup's scales/zeros (8 B + 8 B); they are turned into LDS tables behind a barrier that
//    waits on LDS only, so the weight loads stay in flight across it.
//  * Dequantization in registers. A nibble q ORed into the mantissa of fp16 1024.0 (0x6400) is
//    exactly the fp16 value 1024 + q, so one v_and_or_b32 per pair turns packed nibbles into fp16
//    pairs (q_i, q_{i+4}); x is staged in LDS as the matching pairs (x_i, x_{i+4}).
//      - EXACT: ((1024+q) - (1024+z)) * s in packed fp16 is exactly the reference's dequantized
//        weight (one RNE rounding, kernels/reference.py:35); v_dot2_f32_f16 then accumulates
//        x*w in fp32. 19 VALU ops per 8 weights at M=1.
//      - FACTORED (M = 1): s * (sum x*q - z * sum x) per packed row, the reference's FACTORED
//        identity (kernels/w4a16.py:116-119). The 1024 offsets are cancelled by starting each
//        dot2 chain at -1024 * (sum of the matching x), and nibbles 1/3/5/7 are masked in place
//        as 16*q (no shift), their sum scaled by 1/16 exactly. 12 VALU ops per 8 weights.
//  * Workgroup-to-XCD remap so that neighbouring column tiles share an L2.
#include <algorithm>
#include <cmath>

#include "ldk_common.h"

namespace {

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

struct W4Args {
  const half_t* x;
  int64_t ldx;
  const uint32_t* qw;
  const half_t* s;
  const half_t* z;
  const half_t* bias;
  half_t* out;
  int64_t ldo;
  int M, N, K, gsh_rows;  // group size = 8 << gsh_rows
};

__device__ __forceinline__ half2_t h2lo(uint32_t a, uint32_t b) {  // (lo16(a), lo16(b))
  return ldk::u2h2(__builtin_amdgcn_perm(b, a, 0x05040100u));
}
__device__ __forceinline__ half2_t h2hi(uint32_t a, uint32_t b) {  // (hi16(a), hi16(b))
  return ldk::u2h2(__builtin_amdgcn_perm(b, a, 0x07060302u));
}

// Writes the LDS row record of one (m, packed row): the x pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7)
// and, for FACTORED, -1024*(x0+x2+x4+x6), -1024*(x1+x3+x5+x7) and the row sum.
template <bool FACT>
__device__ __forceinline__ void store_x_row(unsigned char* dst, u32x4 d) {
  u32x4 p;
  p[0] = ldk::h22u(h2lo(d[0], d[2]));
  p[1] = ldk::h22u(h2hi(d[0], d[2]));
  p[2] = ldk::h22u(h2lo(d[1], d[3]));
  p[3] = ldk::h22u(h2hi(d[1], d[3]));
  *reinterpret_cast<u32x4*>(dst) = p;
  if constexpr (FACT) {
    const half2_t a0 = ldk::u2h2(p[0]), a2 = ldk::u2h2(p[2]);
    const half2_t b1 = ldk::u2h2(p[1]), b3 = ldk::u2h2(p[3]);
    const float xa = ((float)a0[0] + (float)a0[1]) + ((float)a2[0] + (float)a2[1]);
    const float xb = ((float)b1[0] + (float)b1[1]) + ((float)b3[0] + (float)b3[1]);
    float4_t c;
    c[0] = -1024.0f * xa;
    c[1] = -1024.0f * xb;
    c[2] = xa + xb;
    c[3] = 0.0f;
    *reinterpret_cast<float4_t*>(dst + 16) = c;
  }
}

// Writes the LDS record of one (group, 4 columns): FACT -> (s, z) as floats per column;
// EXACT -> (-(1024+z), -(1024+z)) and (s, s) as fp16 pairs per column. 32 bytes either way.
template <bool FACT>
__device__ __forceinline__ void store_sz(unsigned char* dst, u32x2 sv, u32x2 zv) {
  const half4_t s4 = __builtin_bit_cast(half4_t, sv);
  const half4_t z4 = __builtin_bit_cast(half4_t, zv);
  if constexpr (FACT) {
    float4_t a, b;
    a[0] = (float)s4[0]; a[1] = (float)z4[0]; a[2] = (float)s4[1]; a[3] = (float)z4[1];
    b[0] = (float)s4[2]; b[1] = (float)z4[2]; b[2] = (float)s4[3]; b[3] = (float)z4[3];
    *reinterpret_cast<float4_t*>(dst) = a;
    *reinterpret_cast<float4_t*>(dst + 16) = b;
  } else {
    u32x4 a, b;
    half2_t t;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half_t zb = -((half_t)1024.0f + z4[c]);
      t[0] = zb; t[1] = zb;
      const uint32_t zu = ldk::h22u(t);
      t[0] = s4[c]; t[1] = s4[c];
      const uint32_t su = ldk::h22u(t);
      if (c < 2) { a[2 * c] = zu; a[2 * c + 1] = su; } else { b[2 * c - 4] = zu; b[2 * c - 3] = su; }
    }
    *reinterpret_cast<u32x4*>(dst) = a;
    *reinterpret_cast<u32x4*>(dst + 16) = b;
  }
}

template <int MT, int LN, int UB, bool FACT>
__global__ __launch_bounds__(512) void w4a16_skinny_kernel(W4Args a) {
  static_assert(!FACT || MT == 1, "FACTORED is the M = 1 kernel");
  constexpr int CW = 4 * LN;        // output columns per workgroup
  constexpr int LKW = 64 / LN;      // K lanes per wave
  constexpr int ROWB = FACT ? 32 : 16;
  constexpr int PX = (MT * UB + LN - 1) / LN < 4 ? (MT * UB + LN - 1) / LN : 4;
  extern __shared__ __align__(16) unsigned char smem[];

  const int NW = blockDim.x >> 6;
  const int NT = blockDim.x;
  const int LK = NW * LKW;
  const int R = a.K >> 3;
  const int ng = R >> a.gsh_rows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane % LN;
  const int lk = wave * LKW + lane / LN;
  const int n0 = ldk::xcd_remap(blockIdx.x, gridDim.x) * CW;
  const int col = min(n0 + 4 * ln, a.N - 4);  // clamped: tail lanes load valid memory, store nothing

  // LDS: x row records [MT][R] + 1 trash record; scale/zero records [ng][LN] + 1 trash record;
  // the split-K reduction buffer [NW][MT][CW].
  unsigned char* xs = smem;
  unsigned char* szs = smem + ((size_t)MT * R + 1) * ROWB;
  float* red = reinterpret_cast<float*>(szs + ((size_t)ng * LN + 1) * 32);

  // ---- prologue loads, issued before the weights so that waiting for them waits for nothing
  // else. They are unconditional (indices clamped to valid items, duplicates dropped at the LDS
  // store) so that no control flow forces an early s_waitcnt. For a single-batch launch
  // (R <= UB*LK) the x items per thread are at most MT*UB/LN and the scale/zero items at most
  // UB*8/group <= 1 for groups >= 128 rows; anything beyond PX/PS is loaded by the slow loops.
  const int nx = MT * R;      // x items (packed row r, row m) at index r*MT + m
  const int nsz = ng * LN;    // scale/zero items (group g, 4 columns l) at index g*LN + l
  u32x4 xr[PX];
  u32x2 sr, zr;
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    const int it = min(tid + i * NT, nx - 1);
    const int m = min(it & (MT - 1), a.M - 1), r = it / MT;
    xr[i] = *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * r);
  }
  {
    const int it = min(tid, nsz - 1);
    const int g = it / LN, l = it & (LN - 1);
    const int c = min(n0 + 4 * l, a.N - 4);
    sr = *reinterpret_cast<const u32x2*>(a.s + (int64_t)g * a.N + c);
    zr = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + c);
  }

  const uint32_t magic = ldk::vgpr_const<kMagic>();  // v_and_or_b32 operands (see sgpr_const)
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>(), mhi = ldk::sgpr_const<0x00F000F0u>();
  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  u32x4 w[UB];
  auto load_batch = [&](int rb) {
    // ---- weight loads of this batch, all in flight before any is used
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int r = min(rb + lk + u * LK, R - 1);
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw + (int64_t)r * a.N + col));
    }

  };
  auto compute_batch = [&](int rb) {
    // ---- consume rows in issue order
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int r = rb + lk + u * LK;
      if (r < R) {
        const int g = r >> a.gsh_rows;
        const unsigned char* szp = szs + ((size_t)g * LN + ln) * 32;
        if constexpr (FACT) {
          const u32x4 xp = *reinterpret_cast<const u32x4*>(xs + (size_t)r * 32);
          const float4_t kc = *reinterpret_cast<const float4_t*>(xs + (size_t)r * 32 + 16);
          const float4_t sz01 = *reinterpret_cast<const float4_t*>(szp);
          const float4_t sz23 = *reinterpret_cast<const float4_t*>(szp + 16);
          const half2_t p0 = ldk::u2h2(xp[0]), p1 = ldk::u2h2(xp[1]);
          const half2_t p2 = ldk::u2h2(xp[2]), p3 = ldk::u2h2(xp[3]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t wc = w[u][c];
            const uint32_t v = wc >> 8;
            const half2_t u0 = ldk::u2h2(((wc & mlo) | magic));  // 1024 + (q0, q4)
            const half2_t u1 = ldk::u2h2(((wc & mhi) | magic));  // 1024 + 16 (q1, q5)
            const half2_t u2 = ldk::u2h2(((v & mlo) | magic));   // 1024 + (q2, q6)
            const half2_t u3 = ldk::u2h2(((v & mhi) | magic));   // 1024 + 16 (q3, q7)
            const float A = ldk::dot2(p0, u0, ldk::dot2(p2, u2, kc[0]));
            const float B = ldk::dot2(p1, u1, ldk::dot2(p3, u3, kc[1]));
            const float sc = (c < 2) ? sz01[2 * c] : sz23[2 * c - 4];
            const float zc = (c < 2) ? sz01[2 * c + 1] : sz23[2 * c - 3];
            float t = __builtin_fmaf(B, 0.0625f, A);  // sum over the row of x*q
            t = __builtin_fmaf(-zc, kc[2], t);          // - z * sum x
            acc[0][c] = __builtin_fmaf(sc, t, acc[0][c]);
          }
        } else {
          const u32x4 zs01 = *reinterpret_cast<const u32x4*>(szp);
          const u32x4 zs23 = *reinterpret_cast<const u32x4*>(szp + 16);
          u32x4 xp[MT];
#pragma unroll
          for (int m = 0; m < MT; ++m) xp[m] = *reinterpret_cast<const u32x4*>(xs + ((size_t)m * R + r) * 16);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t wc = w[u][c];
            const half2_t zb = ldk::u2h2(c < 2 ? zs01[2 * c] : zs23[2 * c - 4]);
            const half2_t s2 = ldk::u2h2(c < 2 ? zs01[2 * c + 1] : zs23[2 * c - 3]);
            const half2_t d0 = (ldk::u2h2(((wc & mlo) | magic)) + zb) * s2;
            const half2_t d1 = (ldk::u2h2((((wc >> 4) & mlo) | magic)) + zb) * s2;
            const half2_t d2 = (ldk::u2h2((((wc >> 8) & mlo) | magic)) + zb) * s2;
            const half2_t d3 = (ldk::u2h2((((wc >> 12) & mlo) | magic)) + zb) * s2;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              float t = ldk::dot2(ldk::u2h2(xp[m][0]), d0, acc[m][c]);
              t = ldk::dot2(ldk::u2h2(xp[m][1]), d1, t);
              t = ldk::dot2(ldk::u2h2(xp[m][2]), d2, t);
              acc[m][c] = ldk::dot2(ldk::u2h2(xp[m][3]), d3, t);
            }
          }
        }
      }
    }
  };

  // First batch of weight loads, then the LDS tables (their arithmetic sits after the loads in
  // straight-line code, so nothing waits on the weights before the compute), then the batches.
  load_batch(0);
  // ---- prologue: LDS tables, then one LDS-only barrier
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    // Branch-free: out-of-range items go to the trash record, so the load is never sunk into a
    // conditional block behind the weight loads.
    const int it = tid + i * NT;
    const int m = it & (MT - 1), r = it / MT;
    u32x4 d = xr[i];
    if (m >= a.M) d = u32x4{0u, 0u, 0u, 0u};
    const size_t rec = it < nx ? (size_t)m * R + r : (size_t)nx;
    store_x_row<FACT>(xs + rec * ROWB, d);
  }
  for (int it = tid + PX * NT; it < nx; it += NT) {  // only when MT*R > PX*NT
    const int m = it & (MT - 1), r = it / MT;
    u32x4 d = *reinterpret_cast<const u32x4*>(a.x + min(m, a.M - 1) * a.ldx + 8 * r);
    if (m >= a.M) d = u32x4{0u, 0u, 0u, 0u};
    store_x_row<FACT>(xs + ((size_t)m * R + r) * ROWB, d);
  }
  store_sz<FACT>(szs + (size_t)(tid < nsz ? tid : nsz) * 32, sr, zr);
  for (int it = tid + NT; it < nsz; it += NT) {  // only when ng*LN > NT
    const int g = it / LN, l = it & (LN - 1);
    const int c = min(n0 + 4 * l, a.N - 4);
    const u32x2 sv = *reinterpret_cast<const u32x2*>(a.s + (int64_t)g * a.N + c);
    const u32x2 zv = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + c);
    store_sz<FACT>(szs + (size_t)it * 32, sv, zv);
  }
  ldk::lds_barrier();
  for (int rb = 0;;) {
    compute_batch(rb);
    rb += UB * LK;
    if (rb >= R) break;
    load_batch(rb);
  }

  // ---- split-K reduction: lanes of a wave that share `ln`, then the waves through LDS
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = ldk::sum_lanes_strided<LN>(acc[m][c]);
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
      *reinterpret_cast<float4_t*>(red + ((size_t)wave * MT + m) * CW + 4 * lane) =
          float4_t{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
  }
  ldk::lds_barrier();
  for (int o = tid; o < MT * CW; o += NT) {
    const int m = o / CW, c = o - m * CW;
    const int n = n0 + c;
    if (m < a.M && n < a.N) {
      float v = 0.0f;
      for (int wv = 0; wv < NW; ++wv) v += red[((size_t)wv * MT + m) * CW + c];
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)m * a.ldo + n] = (half_t)v;
    }
  }
}

// ------------------------------------------------------------------------------------ dispatch

struct SkinnyCfg {
  int mt, ln, nw, ub;
  bool fact;
};

int round_ub(int rows) {
  static const int kUB[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int u : kUB)
    if (u >= rows) return u;
  return 16;
}

int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

size_t skinny_lds_bytes(const SkinnyCfg& c, int64_t K, int gsh_rows) {
  const int64_t R = K / 8, ng = R >> gsh_rows;
  return ((size_t)c.mt * R + 1) * (c.fact ? 32 : 16) + ((size_t)ng * c.ln + 1) * 32 + (size_t)c.nw * c.mt * 4 * c.ln * 4;
}

// Default choice: 2+ waves per SIMD over the 256 CUs when N allows, at most 12 rows per lane,
// as wide a column tile as that permits (wider tiles read longer contiguous runs per row).
SkinnyCfg choose_skinny(int64_t M, int64_t N, int64_t K, int split_k, int block_n, int flags) {
  SkinnyCfg best{round_mt(M), 1, 4, 1, false};
  best.fact = (best.mt == 1) && !(flags & LDK_EXACT);
  const int64_t R = K / 8;
  double best_score = -1e30;
  for (int ln : {16, 8, 4, 2, 1}) {
    if (block_n && block_n != 4 * ln) continue;
    for (int nw : {4, 8, 2, 1}) {
      const int lk = nw * 64 / ln;
      if (split_k && split_k != lk) continue;
      const int64_t nwg = (N + 4 * ln - 1) / (4 * ln);
      const int64_t rows = (R + lk - 1) / lk;
      const double waves = (double)nwg * nw;
      double score = 0.0;
      score -= std::abs(std::log2(std::max(waves, 1.0) / 2048.0)) * 4.0;  // ~2 waves per SIMD
      score -= rows > 12 ? (rows - 12) * 0.5 : 0.0;
      score -= (double)(R % lk ? 1 : 0) * 0.5;                            // ragged last rows
      score += ln >= 8 ? 1.0 : ln >= 4 ? 0.5 : 0.0;
      score -= nwg < 256 ? (256.0 - nwg) / 64.0 : 0.0;                    // idle CUs
      if (score > best_score) {
        best_score = score;
        best.ln = ln;
        best.nw = nw;
        best.ub = round_ub((int)std::min<int64_t>(rows, 16));
      }
    }
  }
  return best;
}

template <int MT, int LN, int UB, bool FACT>
int launch_skinny_t(const W4Args& a, int nw, hipStream_t stream) {
  const int64_t R = a.K / 8, ng = R >> a.gsh_rows;
  const size_t lds = skinny_lds_bytes(SkinnyCfg{MT, LN, nw, UB, FACT}, a.K, a.gsh_rows);
  auto kern = w4a16_skinny_kernel<MT, LN, UB, FACT>;
  if (lds > 64 * 1024) {
    if (lds > 160 * 1024) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: LDS need %zu B exceeds 160 KiB (M*K too large for the decode kernel)", lds);
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return ldk::fail(LDK_ERR_LAUNCH, "w4a16: cannot raise the LDS limit to %zu B", lds);
  }
  const int grid = (int)((a.N + 4 * LN - 1) / (4 * LN));
  (void)hipGetLastError();
  kern<<<grid, nw * 64, lds, stream>>>(a);
  return ldk::check_launch("w4a16_skinny");
}

template <int MT, int LN, bool FACT>
int launch_skinny_ub(const W4Args& a, const SkinnyCfg& c, hipStream_t s) {
  switch (c.ub) {
    case 1: return launch_skinny_t<MT, LN, 1, FACT>(a, c.nw, s);
    case 2: return launch_skinny_t<MT, LN, 2, FACT>(a, c.nw, s);
    case 3: return launch_skinny_t<MT, LN, 3, FACT>(a, c.nw, s);
    case 4: return launch_skinny_t<MT, LN, 4, FACT>(a, c.nw, s);
    case 6: return launch_skinny_t<MT, LN, 6, FACT>(a, c.nw, s);
    case 8: return launch_skinny_t<MT, LN, 8, FACT>(a, c.nw, s);
    case 12: return launch_skinny_t<MT, LN, 12, FACT>(a, c.nw, s);
    case 16: return launch_skinny_t<MT, LN, 16, FACT>(a, c.nw, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: rows per lane %d not instantiated", c.ub);
}

template <int MT, bool FACT>
int launch_skinny_ln(const W4Args& a, const SkinnyCfg& c, hipStream_t s) {
  switch (c.ln) {
    case 1: return launch_skinny_ub<MT, 1, FACT>(a, c, s);
    case 2: return launch_skinny_ub<MT, 2, FACT>(a, c, s);
    case 4: return launch_skinny_ub<MT, 4, FACT>(a, c, s);
    case 8: return launch_skinny_ub<MT, 8, FACT>(a, c, s);
    case 16: return launch_skinny_ub<MT, 16, FACT>(a, c, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: column tile %d not instantiated", 4 * c.ln);
}

int launch_skinny(const W4Args& a, const SkinnyCfg& c, hipStream_t s) {
  if (c.fact) return launch_skinny_ln<1, true>(a, c, s);
  switch (c.mt) {
    case 1: return launch_skinny_ln<1, false>(a, c, s);
    case 2: return launch_skinny_ln<2, false>(a, c, s);
    case 4: return launch_skinny_ln<4, false>(a, c, s);
    case 8: return launch_skinny_ln<8, false>(a, c, s);
    case 16: return launch_skinny_ln<16, false>(a, c, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: row tile %d not instantiated", c.mt);
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

int validate(const char* fn, const void* x, int64_t ldx, const int32_t* qw, const void* s, const void* z,
             void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int gs, int* gsh_rows) {
  if (!x || !qw || !s || !z || !out) return ldk::fail(LDK_ERR_INVALID, "%s: null pointer", fn);
  if (M <= 0 || N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "%s: M, N, K must be positive (M=%lld N=%lld K=%lld)", fn, (long long)M, (long long)N, (long long)K);
  const int gsh = log2_exact(gs);
  if (gsh < 3 || K % gs) return ldk::fail(LDK_ERR_INVALID, "%s: group_size=%d must be a power of two >= 8 dividing K=%lld", fn, gs, (long long)K);
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N=%lld must be a multiple of 4", fn, (long long)N);
  if (ldx < K || ldo < N) return ldk::fail(LDK_ERR_INVALID, "%s: row strides ldx=%lld ldo=%lld smaller than K/N", fn, (long long)ldx, (long long)ldo);
  if (ldx % 8 || !ldk::aligned(x, 16) || !ldk::aligned(qw, 16) || !ldk::aligned(s, 8) || !ldk::aligned(z, 8))
    return ldk::fail(LDK_ERR_ALIGN, "%s: x and qweight must be 16-byte aligned with ldx %% 8 == 0; scales/zeros 8-byte aligned", fn);
  if (N > INT32_MAX / 8 || K > INT32_MAX / 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N or K too large", fn);
  *gsh_rows = gsh - 3;
  return LDK_OK;
}

}  // namespace

extern "C" int ldk_w4a16_config(int64_t M, int64_t N, int64_t K, int group_size, int* block_n, int* split_k, int* flags) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return ldk::fail(LDK_ERR_INVALID, "w4a16_config: sizes must be positive");
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_config: only the decode path (M <= 16) has a table");
  const SkinnyCfg c = choose_skinny(M, N, K, 0, 0, 0);
  if (block_n) *block_n = 4 * c.ln;
  if (split_k) *split_k = c.nw * 64 / c.ln;
  if (flags) *flags = LDK_PATH_VALU | (c.fact ? LDK_FACTORED : LDK_EXACT);
  return LDK_OK;
}

extern "C" int ldk_w4a16_matmul(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int block_n, int split_k, int flags, void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_matmul", x, ldx, qweight, scales, zeros, out, ldo, M, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: M=%lld > 16 (prefill GEMM not built yet)", (long long)M);
  if ((flags & LDK_FACTORED) && (flags & LDK_EXACT)) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul: FACTORED and EXACT are exclusive");
  if ((flags & LDK_FACTORED) && M > 1) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: FACTORED is the M = 1 kernel");
  if (block_n && (block_n % 4 || block_n > 64 || (block_n & (block_n - 1))))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: block_n=%d must be 4, 8, 16, 32 or 64", block_n);
  SkinnyCfg c = choose_skinny(M, N, K, split_k, block_n, flags);
  if (split_k && c.nw * 64 / c.ln != split_k)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: split_k=%d is not nw*64/(block_n/4) for nw in {1,2,4,8}", split_k);
  if (flags & LDK_FACTORED) c.fact = true;
  const W4Args a{(const half_t*)x, ldx, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K, gsh_rows};
  return launch_skinny(a, c, (hipStream_t)stream);
}

extern "C" int ldk_w4a16_decode(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int split_k, void* stream) {
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_decode: M=%lld > 16 rows", (long long)M);
  return ldk_w4a16_matmul(x, ldx, qweight, scales, zeros, bias, out, ldo, M, N, K, group_size, 0, split_k, 0, stream);
}
