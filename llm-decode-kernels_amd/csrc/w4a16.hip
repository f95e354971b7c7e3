// W4A16 matmul for decode (M <= 16): y[M, N] = x[M, K] @ dequant(W)^T (+ bias).
//
// Replaces the reference's Triton GEMV/GEMM launch paths (kernels/w4a16.py:100-160, 214-279) and
// its CUDA decode kernel (kernels/cuda/w4a16_decode.cu:29-121) with two gfx950 kernels that share
// one work decomposition:
//
//  * Tiles and groups. A workgroup owns CW output columns and a range of quantization groups
//    (all of K, or 1/splits of it). Inside the workgroup each wave takes whole groups, so every
//    lane applies one scale and one zero point per chunk of work and a group's partial sums never
//    leave the lane until the final reduction.
//  * Memory-level parallelism. A lane issues all its loads for a chunk (its x rows, its packed
//    weight rows, one scale and one zero word) before using any of them and consumes them in
//    issue order, so each s_waitcnt vmcnt(n) releases work as data lands and the whole launch's
//    weight stream is in flight at once. Row segments are CW*4 >= 64 bytes long (shorter runs
//    per row were measured to cost 2-7x on MI355X).
//  * No workgroup barrier before the compute: x rows are staged through LDS by the wave that
//    uses them (wave-local exchange), so weight loads never wait on other waves.
//  * Split-K. Partials are reduced inside the workgroup (DPP row rotations and gfx950 permlane
//    swaps within a wave, then LDS across waves). Narrow shapes (few column tiles) also split the
//    groups over `splits` workgroups that meet in a caller-provided workspace; the last one to
//    arrive sums the partials and resets its counter (one launch, no zero-fill, no cast kernel).
//
// Dequantization happens in registers: a nibble q ORed into the mantissa of fp16 1024.0
// (0x6400) is exactly the fp16 value 1024 + q, so one v_and_or_b32 per pair turns packed nibbles
// into fp16 pairs (q_i, q_{i+4}); x is staged as the matching pairs (x_i, x_{i+4}).
//
//  - VALU kernel (M <= 8), wave64 lanes own 4 adjacent columns (one 128-bit load = one packed
//    row of 4 columns = 32 weights):
//      FACTORED (M = 1): s * (sum x*q - z * sum x) per group, the reference's FACTORED identity
//      (kernels/w4a16.py:116-119). Nibbles 1/3/5/7 are masked in place as 16*q and meet x pairs
//      pre-scaled by 1/16; one v_dot2_f32_f16 chain per column runs over all of the lane's rows
//      and starts at -1024*(offset-weighted sum of x) - z*(sum of x). ~9.5 VALU ops per 8 weights.
//      EXACT: ((1024+q) - (1024+z)) * s in packed fp16 is exactly the reference's dequantized
//      weight (one RNE rounding, kernels/reference.py:35), then dot2 with each x row.
//  - MFMA kernel (9 <= M <= 16): an int32 word holds 8 consecutive K of one column, which is
//    exactly one lane's B operand of v_mfma_f32_16x16x32_f16. A lane's 128-bit load feeds four
//    16x16 tiles; B = (q - z) exactly in fp16, A = x rows permuted to the nibble-pair order, the
//    fp32 tile of one group is scaled by s once.
#include <algorithm>
#include <cmath>

#include "ldk_common.h"

namespace {

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves
constexpr size_t kCounterBytes = 4096;    // split-K counters at the start of the workspace

struct W4Args {
  const half_t* x;
  int64_t ldx;
  const uint32_t* qw;
  const half_t* s;
  const half_t* z;
  const half_t* bias;
  half_t* out;
  int64_t ldo;
  int M, N, K, gsh_rows;  // packed rows per group = 1 << gsh_rows
};

struct SplitArgs {
  int splits;          // workgroups per column tile
  int gps;             // groups per split
  float* ws;           // [tiles][splits][MT*CW] partials (splits > 1)
  uint32_t* counters;  // [tiles], zero between launches
};

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {  // (lo16(a), lo16(b))
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {  // (hi16(a), hi16(b))
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// 8 fp16 of x (dwords (x0,x1) (x2,x3) (x4,x5) (x6,x7)) -> pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ u32x4 x_pairs(u32x4 d) {
  return u32x4{perm_lo(d[0], d[2]), perm_hi(d[0], d[2]), perm_lo(d[1], d[3]), perm_hi(d[1], d[3])};
}

// LDS row record of one (packed row, x row): the x pairs; for FACTORED the odd pairs are scaled
// by 1/16 and the record carries c0 = -1024*((x0+x2+x4+x6) + (x1+x3+x5+x7)/16) and x0+...+x7.
template <bool FACT>
__device__ __forceinline__ void store_x_record(unsigned char* dst, u32x4 d) {
  u32x4 p = x_pairs(d);
  if constexpr (FACT) {
    const half2_t a0 = ldk::u2h2(p[0]), a2 = ldk::u2h2(p[2]);
    const half2_t b1 = ldk::u2h2(p[1]), b3 = ldk::u2h2(p[3]);
    const float xa = ((float)a0[0] + (float)a0[1]) + ((float)a2[0] + (float)a2[1]);
    const float xb = ((float)b1[0] + (float)b1[1]) + ((float)b3[0] + (float)b3[1]);
    const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
    p[1] = ldk::h22u(b1 * sixteenth);
    p[3] = ldk::h22u(b3 * sixteenth);
    *reinterpret_cast<float2_t*>(dst + 16) = float2_t{-1024.0f * (xa + 0.0625f * xb), xa + xb};
  }
  *reinterpret_cast<u32x4*>(dst) = p;
}

// ------------------------------------------------------------------------------ VALU kernel
//
// Lane (ln, lkw) of a wave: ln < LN runs along N (columns n0 + 4ln .. +3), lkw < LKW = 64/LN along
// K. LG = rows_per_group / RPL lanes share a group, each taking RPL of its packed rows
// (sub, sub + LG, ...); a wave covers GW = LKW / LG groups per chunk, a workgroup NW * GW.
template <int MT, int LN, int RPL, bool FACT>
__global__ __launch_bounds__(1024) void w4a16_gemv_kernel(W4Args a, SplitArgs sp) {
  static_assert(!FACT || MT == 1, "FACTORED is the M = 1 kernel");
  constexpr int CW = 4 * LN;
  constexpr int LKW = 64 / LN;
  constexpr int ROWB = FACT ? 32 : 16;
  constexpr int PXW = (RPL * MT + LN - 1) / LN;  // x records a lane prepares per chunk
  extern __shared__ __align__(16) unsigned char smem[];

  const int rpg = 1 << a.gsh_rows;
  const int LG = rpg / RPL;
  const int GW = LKW / LG;
  const int NW = blockDim.x >> 6;
  const int R = a.K >> 3;
  const int ng = R >> a.gsh_rows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane % LN, lkw = lane / LN;
  const int gi = lkw / LG, sub = lkw - gi * LG;
  const int tile = blockIdx.x / sp.splits, split = blockIdx.x - tile * sp.splits;
  const int n0 = tile * CW;
  const int col = min(n0 + 4 * ln, a.N - 4);  // clamped: tail lanes load valid memory, store nothing
  const int gb = split * sp.gps, ge = min(ng, gb + sp.gps);
  const int rows_w = GW * rpg;                // packed rows of one wave chunk
  unsigned char* xw = smem + (size_t)wave * rows_w * MT * ROWB;
  float* red = reinterpret_cast<float*>(smem + (size_t)NW * rows_w * MT * ROWB);  // [MT*CW][NWP]

  const uint32_t magic = ldk::vgpr_const<kMagic>();  // v_and_or_b32 operands (see sgpr_const)
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>(), mhi = ldk::sgpr_const<0x00F000F0u>();
  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  for (int gc = gb + wave * GW; gc < ge; gc += NW * GW) {
    // ---- loads, in consumption order: x rows of the chunk, weights, scale, zero
    u32x4 xr[PXW];
#pragma unroll
    for (int i = 0; i < PXW; ++i) {
      const int item = min(lane + 64 * i, rows_w * MT - 1);  // item = rr * MT + m
      const int rr = item / MT, m = min(item % MT, a.M - 1);
      const int row = min(gc * rpg + rr, R - 1);
      xr[i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.ldx + 8 * row);
    }
    const int g = gc + gi;
    const bool gok = g < ge;
    const int gg = gok ? g : ge - 1;
    // FACTORED needs the scale and zero only after its dot chain, EXACT before its first row.
    u32x2 sv, zv;
    if constexpr (!FACT) {
      sv = *reinterpret_cast<const u32x2*>(a.s + (int64_t)gg * a.N + col);
      zv = *reinterpret_cast<const u32x2*>(a.z + (int64_t)gg * a.N + col);
    }
    u32x4 w[RPL];
#pragma unroll
    for (int t = 0; t < RPL; ++t) {
      const int r = gg * rpg + sub + LG * t;
      w[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw + (int64_t)r * a.N + col));
    }
    if constexpr (FACT) {
      sv = *reinterpret_cast<const u32x2*>(a.s + (int64_t)gg * a.N + col);
      zv = *reinterpret_cast<const u32x2*>(a.z + (int64_t)gg * a.N + col);
    }

    // ---- wave-local x staging
#pragma unroll
    for (int i = 0; i < PXW; ++i) {
      const int item = lane + 64 * i;
      if (item < rows_w * MT) {
        u32x4 d = xr[i];
        if (item % MT >= a.M) d = u32x4{0u, 0u, 0u, 0u};
        store_x_record<FACT>(xw + (size_t)item * ROWB, d);
      }
    }
    ldk::wave_lds_sync();
    if (!gok) continue;

    if constexpr (FACT) {
      u32x4 xp[RPL];
      float c0 = 0.0f, xs = 0.0f;
#pragma unroll
      for (int t = 0; t < RPL; ++t) {
        const unsigned char* rec = xw + (size_t)(gi * rpg + sub + LG * t) * ROWB;
        xp[t] = *reinterpret_cast<const u32x4*>(rec);
        const float2_t k = *reinterpret_cast<const float2_t*>(rec + 16);
        c0 += k[0];
        xs += k[1];
      }
      float tt[4] = {c0, c0, c0, c0};
#pragma unroll
      for (int t = 0; t < RPL; ++t) {  // rows in arrival order
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t wc = w[t][c];
          const uint32_t v = wc >> 8;
          tt[c] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[t][3]), ldk::u2h2((v & mhi) | magic), tt[c], false);
          tt[c] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[t][2]), ldk::u2h2((v & mlo) | magic), tt[c], false);
          tt[c] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[t][1]), ldk::u2h2((wc & mhi) | magic), tt[c], false);
          tt[c] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[t][0]), ldk::u2h2((wc & mlo) | magic), tt[c], false);
        }
      }
      const half4_t s4 = __builtin_bit_cast(half4_t, sv);
      const half4_t z4 = __builtin_bit_cast(half4_t, zv);
#pragma unroll
      for (int c = 0; c < 4; ++c)  // s * (sum x*q - z * sum x)
        acc[0][c] = __builtin_fmaf((float)s4[c], __builtin_fmaf(-(float)z4[c], xs, tt[c]), acc[0][c]);
    } else {
      const half4_t s4 = __builtin_bit_cast(half4_t, sv);
      const half4_t z4 = __builtin_bit_cast(half4_t, zv);
#pragma unroll
      for (int t = 0; t < RPL; ++t) {
        u32x4 xp[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
          xp[m] = *reinterpret_cast<const u32x4*>(xw + (size_t)((gi * rpg + sub + LG * t) * MT + m) * ROWB);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t wc = w[t][c];
          const half_t zb1 = -((half_t)1024.0f + z4[c]);
          const half2_t zb = {zb1, zb1};
          const half2_t s2 = {s4[c], s4[c]};
          const half2_t d0 = (ldk::u2h2((wc & mlo) | magic) + zb) * s2;
          const half2_t d1 = (ldk::u2h2(((wc >> 4) & mlo) | magic) + zb) * s2;
          const half2_t d2 = (ldk::u2h2(((wc >> 8) & mlo) | magic) + zb) * s2;
          const half2_t d3 = (ldk::u2h2(((wc >> 12) & mlo) | magic) + zb) * s2;
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            float tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][0]), d0, acc[m][c], false);
            tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][1]), d1, tt, false);
            tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][2]), d2, tt, false);
            acc[m][c] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][3]), d3, tt, false);
          }
        }
      }
    }
  }

  // ---- reduction: lanes of a wave sharing ln, then the waves through LDS
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = ldk::sum_lanes_strided<LN>(acc[m][c]);
  const int NWP = (NW + 3) & ~3;  // partials of one output, wave-minor
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(size_t)(m * CW + 4 * lane + c) * NWP + wave] = acc[m][c];
  }
  __syncthreads();
  auto part = [&](int o) { return ldk::sum_partials(red + (size_t)o * NWP, NW); };
  auto store = [&](int o, float v) {
    const int m = o / CW, n = n0 + (o - m * CW);
    if (m < a.M && n < a.N) {
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)m * a.ldo + n] = (half_t)v;
    }
  };
  if (sp.splits == 1) {
    for (int o = threadIdx.x; o < MT * CW; o += blockDim.x) store(o, part(o));
  } else {
    ldk::splitk_finalize(tile, split, sp.splits, MT * CW, sp.ws, sp.counters, part, store);
  }
}

// ------------------------------------------------------------------------------ MFMA kernel
//
// Lane l of a wave: c16 = l % 16 is the column inside each 16x16 tile and the A row, kb = l / 16
// the 8-wide K block inside a 32-wide K step. The lane's 128-bit load of packed row
// (g*rpg + 4*ks + kb) at columns n0 + 4*c16 .. +3 feeds tiles j = 0..3, whose column c16 is the
// real column n0 + 4*c16 + j. A wave handles whole groups (rpg/4 K steps each).
template <int KS>  // 32-wide K steps per group (group_size / 32)
__global__ __launch_bounds__(1024) void w4a16_mfma16_kernel(W4Args a, SplitArgs sp) {
  constexpr int CW = 64;
  typedef _Float16 half8v __attribute__((ext_vector_type(8)));
  extern __shared__ __align__(16) unsigned char smem[];
  const int rpg = 4 * KS;
  const int NW = blockDim.x >> 6;
  const int R = a.K >> 3;
  const int ng = R >> a.gsh_rows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x / sp.splits, split = blockIdx.x - tile * sp.splits;
  const int n0 = tile * CW;
  const int col = min(n0 + 4 * c16, a.N - 4);
  const int gb = split * sp.gps, ge = min(ng, gb + sp.gps);
  const int xrow = min(c16, a.M - 1);
  const bool xok = c16 < a.M;
  float* red = reinterpret_cast<float*>(smem);  // [16 rows * 64 cols][NWP]

  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>();
  float4_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int g = gb + wave; g < ge; g += NW) {
    // loads in consumption order: zero point, per K step the A fragment and the weight word row,
    // then the scale (used after the group's MFMAs)
    const u32x2 zv = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + col);
    u32x4 ar[KS], w[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int r = g * rpg + 4 * ks + kb;
      ar[ks] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)xrow * a.ldx + 8 * r);
      w[ks] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw + (int64_t)r * a.N + col));
    }
    const u32x2 sv = *reinterpret_cast<const u32x2*>(a.s + (int64_t)g * a.N + col);
    const half4_t z4 = __builtin_bit_cast(half4_t, zv);
    float4_t tmp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) tmp[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      {
        u32x4 ap = x_pairs(ar[ks]);
        if (!xok) ap = u32x4{0u, 0u, 0u, 0u};
        const half8v A = __builtin_bit_cast(half8v, ap);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wc = w[ks][j];
          const half_t zb1 = -((half_t)1024.0f + z4[j]);
          const half2_t zb = {zb1, zb1};
          u32x4 b;
          b[0] = ldk::h22u(ldk::u2h2((wc & mlo) | magic) + zb);          // (q0, q4) - z
          b[1] = ldk::h22u(ldk::u2h2(((wc >> 4) & mlo) | magic) + zb);   // (q1, q5) - z
          b[2] = ldk::h22u(ldk::u2h2(((wc >> 8) & mlo) | magic) + zb);   // (q2, q6) - z
          b[3] = ldk::h22u(ldk::u2h2(((wc >> 12) & mlo) | magic) + zb);  // (q3, q7) - z
          tmp[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(half8v, b), tmp[j], 0, 0, 0);
        }
      }
    }
    const half4_t s4 = __builtin_bit_cast(half4_t, sv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sj = (float)s4[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] = __builtin_fmaf(sj, tmp[j][i], acc[j][i]);
    }
  }

  // tile j, element i of lane l: row 4*kb + i, column 4*c16 + j of the workgroup's 64 columns;
  // partials stored wave-minor ([16*64][NWP])
  const int NWP = (NW + 3) & ~3;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((size_t)(4 * kb + i) * CW + 4 * c16 + j) * NWP + wave] = acc[j][i];
  __syncthreads();
  auto part = [&](int o) { return ldk::sum_partials(red + (size_t)o * NWP, NW); };
  auto store = [&](int o, float v) {
    const int m = o / CW, n = n0 + (o - m * CW);
    if (m < a.M && n < a.N) {
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)m * a.ldo + n] = (half_t)v;
    }
  };
  if (sp.splits == 1) {
    for (int o = threadIdx.x; o < 16 * CW; o += blockDim.x) store(o, part(o));
  } else {
    ldk::splitk_finalize(tile, split, sp.splits, 16 * CW, sp.ws, sp.counters, part, store);
  }
}

// ------------------------------------------------------------------------------------ dispatch

struct Plan {
  bool mfma;
  int mt, ln, rpl;  // VALU kernel shape
  bool fact;
  int nw, splits, gps;
};

int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

size_t plan_lds_bytes(const Plan& p, int gsh_rows) {
  const size_t nwp = (size_t)((p.nw + 3) & ~3);
  if (p.mfma) return nwp * 16 * 64 * 4;
  const int rpg = 1 << gsh_rows;
  const int LG = rpg / p.rpl, GW = (64 / p.ln) / LG;
  return (size_t)p.nw * GW * rpg * p.mt * (p.fact ? 32 : 16) + nwp * p.mt * 4 * p.ln * 4;
}

size_t workspace_need(const Plan& p, int64_t N) {
  if (p.splits <= 1) return 0;
  const int cw = p.mfma ? 64 : 4 * p.ln;
  const int64_t tiles = (N + cw - 1) / cw;
  const int n = p.mfma ? 16 * 64 : p.mt * cw;
  if (tiles > kCounterBytes / 4) return SIZE_MAX;  // one counter per tile
  return kCounterBytes + (size_t)tiles * p.splits * n * 4;
}

// Chooses the kernel, column tile, rows per lane, workgroup size and split count for a shape.
// Measured on MI355X: row runs of >= 64 B per tile, ~8-16 waves per CU across >= 256 CUs and a
// single chunk of loads per lane are what reach the memory-system floor.
Plan make_plan(int64_t M, int64_t N, int64_t K, int gsh_rows, int block_n, int split_k, int flags,
               size_t ws_bytes) {
  Plan p{};
  const int rpg = 1 << gsh_rows;
  const int64_t ng = (K / 8) >> gsh_rows;
  p.mfma = (M > 8 && !(flags & LDK_PATH_VALU)) || (flags & LDK_PATH_MFMA);
  p.mt = p.mfma ? 16 : round_mt(M);
  p.fact = !p.mfma && p.mt == 1 && !(flags & LDK_EXACT);
  if (p.mfma) {
    p.ln = 16;
  } else if (block_n) {
    p.ln = block_n / 4;
  } else {
    p.ln = N >= 8192 ? 16 : N >= 512 ? 8 : 4;
  }
  const int cw = p.mfma ? 64 : 4 * p.ln;
  const int lkw = 64 / p.ln;
  // rows per lane: a group's packed rows over LG lanes with LG | LKW
  p.rpl = rpg;
  for (int rpl : {4, 8, 2, 16, 1, 32}) {
    if (rpl <= rpg && rpg % rpl == 0 && lkw % (rpg / rpl) == 0) { p.rpl = rpl; break; }
  }
  const int gw = p.mfma ? 1 : lkw / (rpg / p.rpl);
  const int64_t tiles = (N + cw - 1) / cw;
  // split count: enough workgroups for the 256 CUs, at most 16 waves per workgroup
  int64_t splits = split_k > 0 ? split_k : 1;
  if (split_k <= 0) {
    while (tiles * splits < 240 && splits * 2 <= ng) splits *= 2;
    while ((ng + splits - 1) / splits > 16 * gw && splits < ng) ++splits;
  }
  splits = std::min<int64_t>(splits, ng);
  p.gps = (int)((ng + splits - 1) / splits);
  p.splits = (int)((ng + p.gps - 1) / p.gps);
  p.nw = (int)std::min<int64_t>(16, (p.gps + gw - 1) / gw);
  if (p.splits > 1 && workspace_need(p, N) > ws_bytes) {  // no room for partials: one split
    p.splits = 1;
    p.gps = (int)ng;
    p.nw = (int)std::min<int64_t>(16, (ng + gw - 1) / gw);
  }
  return p;
}

template <int MT, int LN, int RPL, bool FACT>
int launch_gemv_t(const W4Args& a, const SplitArgs& sp, int nw, size_t lds, hipStream_t stream) {
  auto kern = w4a16_gemv_kernel<MT, LN, RPL, FACT>;
  if (lds > 64 * 1024) {
    if (lds > 160 * 1024) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: LDS need %zu B exceeds 160 KiB", lds);
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return ldk::fail(LDK_ERR_LAUNCH, "w4a16: cannot raise the LDS limit to %zu B", lds);
  }
  const int64_t tiles = (a.N + 4 * LN - 1) / (4 * LN);
  (void)hipGetLastError();
  kern<<<(unsigned)(tiles * sp.splits), nw * 64, lds, stream>>>(a, sp);
  return ldk::check_launch("w4a16_gemv");
}

template <int MT, int LN, bool FACT>
int launch_gemv_rpl(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s) {
  switch (p.rpl) {
    case 1: return launch_gemv_t<MT, LN, 1, FACT>(a, sp, p.nw, lds, s);
    case 2: return launch_gemv_t<MT, LN, 2, FACT>(a, sp, p.nw, lds, s);
    case 4: return launch_gemv_t<MT, LN, 4, FACT>(a, sp, p.nw, lds, s);
    case 8: return launch_gemv_t<MT, LN, 8, FACT>(a, sp, p.nw, lds, s);
    case 16: return launch_gemv_t<MT, LN, 16, FACT>(a, sp, p.nw, lds, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: %d rows per lane not instantiated", p.rpl);
}

template <int MT, bool FACT>
int launch_gemv_ln(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s) {
  switch (p.ln) {
    case 4: return launch_gemv_rpl<MT, 4, FACT>(a, sp, p, lds, s);
    case 8: return launch_gemv_rpl<MT, 8, FACT>(a, sp, p, lds, s);
    case 16: return launch_gemv_rpl<MT, 16, FACT>(a, sp, p, lds, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: block_n=%d not supported (16, 32 or 64)", 4 * p.ln);
}

int launch_plan(const W4Args& a, const Plan& p, void* ws, hipStream_t s) {
  SplitArgs sp{p.splits, p.gps, nullptr, nullptr};
  if (p.splits > 1) {
    sp.counters = reinterpret_cast<uint32_t*>(ws);
    sp.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  }
  const size_t lds = plan_lds_bytes(p, a.gsh_rows);
  if (p.mfma) {
    (void)hipGetLastError();
    const int64_t tiles = (a.N + 63) / 64;
    const unsigned grid = (unsigned)(tiles * p.splits);
    if (lds > 64 * 1024) {
      const void* k[] = {(const void*)w4a16_mfma16_kernel<1>, (const void*)w4a16_mfma16_kernel<2>,
                         (const void*)w4a16_mfma16_kernel<4>, (const void*)w4a16_mfma16_kernel<8>};
      for (const void* f : k)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
          return ldk::fail(LDK_ERR_LAUNCH, "w4a16: cannot raise the LDS limit to %zu B", lds);
    }
    switch (1 << a.gsh_rows) {
      case 4: w4a16_mfma16_kernel<1><<<grid, p.nw * 64, lds, s>>>(a, sp); break;
      case 8: w4a16_mfma16_kernel<2><<<grid, p.nw * 64, lds, s>>>(a, sp); break;
      case 16: w4a16_mfma16_kernel<4><<<grid, p.nw * 64, lds, s>>>(a, sp); break;
      case 32: w4a16_mfma16_kernel<8><<<grid, p.nw * 64, lds, s>>>(a, sp); break;
      default: return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: group size not supported by the MFMA kernel");
    }
    return ldk::check_launch("w4a16_mfma16");
  }
  if (p.fact) return launch_gemv_ln<1, true>(a, sp, p, lds, s);
  switch (p.mt) {
    case 1: return launch_gemv_ln<1, false>(a, sp, p, lds, s);
    case 2: return launch_gemv_ln<2, false>(a, sp, p, lds, s);
    case 4: return launch_gemv_ln<4, false>(a, sp, p, lds, s);
    case 8: return launch_gemv_ln<8, false>(a, sp, p, lds, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: row tile %d not instantiated", p.mt);
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
  if (gs < 32 || gs > 256) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: group_size=%d outside 32..256", fn, gs);
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N=%lld must be a multiple of 4", fn, (long long)N);
  if (ldx < K || ldo < N) return ldk::fail(LDK_ERR_INVALID, "%s: row strides ldx=%lld ldo=%lld smaller than K/N", fn, (long long)ldx, (long long)ldo);
  if (ldx % 8 || !ldk::aligned(x, 16) || !ldk::aligned(qw, 16) || !ldk::aligned(s, 8) || !ldk::aligned(z, 8))
    return ldk::fail(LDK_ERR_ALIGN, "%s: x and qweight must be 16-byte aligned with ldx %% 8 == 0; scales/zeros 8-byte aligned", fn);
  if (N > INT32_MAX / 8 || K > INT32_MAX / 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N or K too large", fn);
  *gsh_rows = gsh - 3;
  return LDK_OK;
}

}  // namespace

extern "C" int64_t ldk_workspace_bytes(void) { return (int64_t)32 << 20; }

extern "C" int ldk_w4a16_config(int64_t M, int64_t N, int64_t K, int group_size, int* block_n, int* split_k, int* flags) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return ldk::fail(LDK_ERR_INVALID, "w4a16_config: sizes must be positive");
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_config: only the decode path (M <= 16) has a table");
  const int gsh = log2_exact(group_size);
  if (gsh < 5 || gsh > 8 || K % group_size) return ldk::fail(LDK_ERR_INVALID, "w4a16_config: bad group_size %d", group_size);
  const Plan p = make_plan(M, N, K, gsh - 3, 0, 0, 0, (size_t)ldk_workspace_bytes());
  if (block_n) *block_n = p.mfma ? 64 : 4 * p.ln;
  if (split_k) *split_k = p.splits;
  if (flags) *flags = (p.mfma ? LDK_PATH_MFMA : LDK_PATH_VALU) | (p.fact ? LDK_FACTORED : LDK_EXACT);
  return LDK_OK;
}

extern "C" int ldk_w4a16_matmul(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int block_n, int split_k, int flags, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_matmul", x, ldx, qweight, scales, zeros, out, ldo, M, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: M=%lld > 16 (prefill GEMM not built yet)", (long long)M);
  if ((flags & LDK_FACTORED) && (flags & LDK_EXACT)) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul: FACTORED and EXACT are exclusive");
  if ((flags & LDK_PATH_VALU) && (flags & LDK_PATH_MFMA)) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul: VALU and MFMA paths are exclusive");
  if ((flags & LDK_FACTORED) && M > 1) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: FACTORED is the M = 1 kernel");
  if ((flags & LDK_PATH_VALU) && M > 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: the VALU kernel takes M <= 8");
  if (block_n && block_n != 16 && block_n != 32 && block_n != 64)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: block_n=%d must be 16, 32 or 64", block_n);
  if (split_k < 0) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul: split_k=%d must be >= 0", split_k);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_matmul: workspace must be a 256-byte aligned pointer");
  const Plan p = make_plan(M, N, K, gsh_rows, block_n, split_k, flags, workspace ? (size_t)workspace_bytes : 0);
  if (p.mfma && block_n && block_n != 64) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul: the MFMA kernel uses block_n=64");
  if (split_k > 1 && p.splits == 1)
    return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul: split_k=%d needs a workspace for the partial sums", split_k);
  const W4Args a{(const half_t*)x, ldx, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K, gsh_rows};
  return launch_plan(a, p, workspace, (hipStream_t)stream);
}

extern "C" int ldk_w4a16_decode(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int split_k, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_decode: M=%lld > 16 rows", (long long)M);
  return ldk_w4a16_matmul(x, ldx, qweight, scales, zeros, bias, out, ldo, M, N, K, group_size, 0, split_k, 0,
                          workspace, workspace_bytes, stream);
}
