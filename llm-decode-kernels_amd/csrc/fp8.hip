// FP8 (OCP e4m3fn) weight-only matmul (W8A16) and its weight format routines for gfx950.
//
// Replaces kernels/fp8.py of the reference: quantize_fp8 (fp8.py:25-30), dequantize_fp8
// (fp8.py:33-35) and the W8A16 GEMV/GEMM (fp8.py:42-127, dispatched by fp8.py:162-223).
//
// Format: wq [K, N] e4m3fn bytes (N contiguous), one scale per output channel n.
// e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities, 0x7F/0xFF = NaN,
// largest finite 448, subnormals m * 2^-9. gfx950's fp8 conversion instructions use this OCP
// encoding (gfx942's were the "fnuz" variant); the GEMV decodes with v_cvt_pk_f32_fp8.
//
// GEMV layout (M <= 16): like the W4A16 skinny kernel, a workgroup owns CW = 16*LN columns and
// all of K; each lane owns 16 adjacent columns, so one 128-bit load = one K row of 16 weights;
// LK = NW*64/LN lanes split K and are reduced in-workgroup (DPP/permlane, then LDS). x is staged
// in LDS as fp16 by the wave that uses it (no workgroup barrier before the FMAs). The
// per-channel scale is applied once after the K reduction (fp8.py:120).
#include <algorithm>

#include "attention.h"
#include "ldk_common.h"
#include "prefill.h"

namespace {

// ------------------------------------------------------------------------------ e4m3 encode

// float (|v| <= 448) -> e4m3fn byte, round to nearest, ties to even, sign of zero kept.
// Written from the format: for |v| in [2^e, 2^(e+1)) with e >= -6 the spacing is 2^(e-3);
// below 2^-6 (subnormal range) the spacing is 2^-9. Scaling by a power of two is exact, so
// rintf on the scaled value performs the RNE rounding to the representable grid.
__device__ __forceinline__ uint8_t e4m3_encode(float v) {
  const uint32_t sign = (__builtin_bit_cast(uint32_t, v) >> 24) & 0x80u;
  const float a = fabsf(v);
  uint32_t code;
  if (a < 0.015625f) {  // 2^-6
    const uint32_t m = (uint32_t)rintf(a * 512.0f);  // 0..8; 8 is the smallest normal 2^-6
    code = m;                                        // m == 8 encodes (e=1, m=0) = 0x08 as well
  } else {
    const int e = (int)((__builtin_bit_cast(uint32_t, a) >> 23) & 0xFF) - 127;  // -6..8
    uint32_t m = (uint32_t)rintf(__builtin_ldexpf(a, 3 - e));                   // 8..16
    int ee = e;
    if (m == 16) { m = 8; ++ee; }
    code = ((uint32_t)(ee + 7) << 3) | (m - 8);
  }
  return (uint8_t)(sign | code);
}

// e4m3fn byte -> float, written from the format (used where bit-exactness is the contract).
__device__ __forceinline__ float e4m3_decode(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;  // m * 2^-9
  else if (e == 15 && m == 7) v = __builtin_nanf("");
  else v = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<half_t>(half_t v) { return (float)v; }
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ half_t from_f32<half_t>(float v) { return (half_t)v; }
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// One thread per output channel n: absmax over its row, then the row is quantized and written
// as column n of wq. Consecutive threads take consecutive n, so each K step writes one
// contiguous run of bytes. Arithmetic as fp8.py:27-29 in float32:
// scale = max(absmax / 448, 1e-12); wq = e4m3(clamp(w / scale, -448, 448)).
template <typename T>
__global__ __launch_bounds__(64) void fp8_quantize_kernel(const T* __restrict__ w, uint8_t* __restrict__ wq,
                                                          T* __restrict__ scale_out, int64_t N, int64_t K) {
  const int64_t n = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (n >= N) return;
  const T* row = w + n * K;
  float amax = 0.0f;
  for (int64_t k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(to_f32<T>(row[k])));
  const float scale = fmaxf(amax / 448.0f, 1e-12f);
  for (int64_t k = 0; k < K; ++k) {
    const float q = fminf(fmaxf(to_f32<T>(row[k]) / scale, -448.0f), 448.0f);
    wq[k * N + n] = e4m3_encode(q);
  }
  scale_out[n] = from_f32<T>(scale);
}

// out [N, K] = (e4m3(wq[k, n]) * scale[n]) rounded once to the scale's dtype (fp8.py:33-35; the
// product of an e4m3 value and an fp16/bf16 scale is exact in fp32).
template <typename T>
__global__ __launch_bounds__(256) void fp8_dequant_kernel(const uint8_t* __restrict__ wq, const T* __restrict__ scale,
                                                          T* __restrict__ out, int64_t N, int64_t K) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N * K) return;
  const int64_t n = i / K, k = i - n * K;
  float p = e4m3_decode(wq[k * N + n]) * to_f32<T>(scale[n]);
  // Keep the f32 product: fused into one v_fma_mix with a +0 addend, the fp16 conversion would
  // turn a -0 product (code 0x80) into +0.
  asm volatile("" : "+v"(p));
  out[i] = from_f32<T>(p);
}

// --------------------------------------------------------------------------------- W8A16 GEMV
//
// out [M, N] = x [M, K] @ (e4m3(wq) * scale)^T (+ bias), wq [K, N] bytes (N contiguous).
//
// Work decomposition (3-D grid: column tile, K split, row block):
//  * Column tiles of CW = 16 * LN columns; a lane owns 16 adjacent columns, so one 128-bit load
//    is one K row of 16 weights, and LN = 8 lanes cover one 128-byte line of a row (the default
//    tile: no line is shared between workgroups).
//  * The LKW = 64 / LN lanes of a wave along K and the NW waves take interleaved K rows; a pass
//    of the workgroup covers RPP = LKW * NW * RPL rows, RPL per lane, all loads of a pass issued
//    before the first wait. A workgroup covers `kps` rows (one or a few passes); workgroups of
//    one tile that split K meet in the fixed-point workspace (ldk::splitk_add, deterministic, one
//    launch).
//  * N % 16 != 0 (TAIL, N % 4 == 0): rows are then only 4-byte aligned, so a lane loads its 16
//    columns of a row as four dwords, each clamped on its own to the row's last dword (a dword
//    past N reads valid memory; its outputs are not stored) instead of one 128-bit load.
//  * Row blocks of MT <= 4 activation rows: a lane keeps 16 * MT fp32 accumulators. More rows
//    run as more row-block workgroups over the same weights (the 256 MB MALL serves the repeats).
//  * x of a pass is staged in LDS transposed, [row][m], so one ds_read gives the MT values of
//    one K row. Weights go from one 128-bit load through v_cvt_pk_f32_fp8 (gfx950's OCP e4m3
//    decode) into fp32 FMAs; the per-channel scale is applied once after the K reduction
//    (fp8.py:120).
struct W8Args {
  const half_t* x;
  int64_t ldx;
  const uint8_t* wq;
  const half_t* scale;
  const half_t* bias;
  half_t* out;
  int64_t ldo;
  int M, N, K;
  // RMSNorm prologue (PRO 2, 3): residual added before the norm, x + residual written by the
  // first workgroup, norm weight [K], eps
  const half_t* res;
  half_t* res_out;
  const half_t* nw;
  float eps;
  // attention-merge prologue (PRO 4): the decode attention's per-range partials (attention.h),
  // its position and range geometry
  const float* att_o = nullptr;
  const float* att_ml = nullptr;
  const int64_t* att_pos = nullptr;
  int att_len = 0, att_rlen = 0;
};

struct W8Split {
  int splits;     // workgroups per column tile along K (gridDim.y)
  int kps;        // K rows per split, a multiple of 8
  uint64_t* acc;  // [tiles][mblocks][MT * CW] fixed-point accumulators (splits > 1)
  float* side;    // their fp32 side slots (ldk::SplitK), zero between launches
};

// Workgroups splitting one column tile (the accumulators count up to ldk::kFixMaxSplits).
constexpr int kW8MaxSplits = 40;
static_assert(kW8MaxSplits <= ldk::kFixMaxSplits, "split count field");

__device__ __forceinline__ ldk::SplitK w8_split_ctx(const W8Split& sp, int split = (int)blockIdx.y) {
  return ldk::SplitK{sp.acc, sp.side, sp.splits, split};
}

// Prologues (one row) that form the activation while it is staged, with the steps of the
// standalone kernels:
//  PRO = 1: the x row is [g | u] of 2K values, activation silu(g) * u (bit-identical to the
//           SwiGLU kernel's output);
//  PRO = 2, 3: RMSNorm of x (PRO 3: of x + residual, written to res_out by the first workgroup)
//           times the norm weight. Each workgroup stages only its K range, so it reduces the
//           row statistic over the whole row itself: its first row vectors are loaded ahead of
//           the pass (one LDS barrier, which waits for those loads only). The statistic's order
//           differs from the RMSNorm kernel's, so a staged value can differ from its output by
//           one fp16 ulp;
//  PRO = 4: x is the decode attention's output, merged from its per-range partials
//           (ldk_decode_attention_ranges) as it is staged: for dim d of head h,
//           x = sum_r f_r o_r / sum_r f_r l_r with f_r = exp(m_r - max m) over the ranges live at
//           pos, rounded once to fp16, the W4A16 o projection's merge (a chain in range order,
//           one reciprocal per value). The partials of all kW8AttnRanges ranges are loaded with
//           the x loads (in bounds: the partials hold kAttnMaxSplits ranges); the ranges past
//           the live ones are left out by selects when x is formed.
constexpr int kW8AttnRanges = 4;  // attention ranges a PRO 4 launch merges (registers)

template <int MT, int LN, int NW, int RPL, int PRO, bool TAIL>
__global__ __launch_bounds__(NW * 64) void w8a16_gemv_kernel(W8Args a, W8Split sp) {
  static_assert(PRO == 0 || MT == 1, "the prologues take one row");
  constexpr bool kRms = PRO == 2 || PRO == 3, kRes = PRO == 3, kAttn = PRO == 4;
  constexpr int CW = 16 * LN;
  constexpr int LKW = 64 / LN;
  constexpr int RPP = LKW * NW * RPL;  // K rows per pass
  constexpr int RPW = LKW * RPL;       // K rows of a pass one wave uses
  constexpr int XPL = (RPW * MT + 63) / 64;  // x values a lane stages per pass
  // x is staged per wave (only the rows the wave uses, so no workgroup barrier): slot lk + j*LKW
  // holds row wave*LKW + lk + j*LKW*NW of the pass
  __shared__ __align__(16) half_t xs[NW][MT][RPW];
  __shared__ __align__(16) float red[NW][MT][CW];
  __shared__ float stat[NW];
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.wq);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane % LN, lk = lane / LN;
  const int tile = blockIdx.x, split = blockIdx.y, mb = blockIdx.z;
  const int n0 = tile * CW;
  // clamped: lanes past N load valid memory and store nothing (TAIL: each dword clamped itself)
  const int col = TAIL ? n0 + 16 * ln : min(n0 + 16 * ln, a.N - 16);
  const int m0 = mb * MT;
  const int rb = split * sp.kps, re = min(a.K, rb + sp.kps);
  const int lrow = wave * LKW + lk;  // this lane's first row inside a pass

  float acc[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = 0.0f;

  // RMSNorm prologue: this thread's first row vector for the statistic, issued ahead of the pass
  // (buffer loads read zeros past the row)
  u32x4 sx0{}, sr0{};
  if constexpr (kRms) {
    sx0 = ldk::buffer_load16(ldk::buffer_rsrc(a.x, (uint32_t)a.K * 2u), 16u * tid);
    if constexpr (kRes) sr0 = ldk::buffer_load16(ldk::buffer_rsrc(a.res, (uint32_t)a.K * 2u), 16u * tid);
  }
  float rs = 0.0f;
  // PRO 4: the ranges live at the attention's position (its clamping of pos)
  int att_live = 1;
  if constexpr (kAttn) {
    const int64_t pin = *a.att_pos;
    const int pos = pin >= 0 && pin < a.att_len ? (int)pin : pin < 0 ? -1 : a.att_len - 1;
    att_live = pos < 0 ? 1 : pos / a.att_rlen + 1;
  }

  for (int p0 = rb; p0 < re; p0 += RPP) {
    // loads in consumption order: this wave's x values, then the weight rows (clamped, branch
    // free; rows past re and x rows past M are zeroed when staged)
    half_t xl[XPL], xu[XPL], xn[XPL];
    float ao[kAttn ? XPL : 1][kW8AttnRanges];  // PRO 4: dim d of head h of each range
    float2_t am[kAttn ? XPL : 1][kW8AttnRanges];  // and its {m, l}
#pragma unroll
    for (int i = 0; i < XPL; ++i) {
      const int e = lane + 64 * i, m = min(e / RPW, MT - 1), rr = e % RPW;
      const int k = p0 + wave * LKW + rr % LKW + (rr / LKW) * LKW * NW;
      const int64_t xo = (int64_t)min(m0 + m, a.M - 1) * a.ldx + min(k, a.K - 1);
      if constexpr (kAttn) {
        const int kk = min(k, a.K - 1), h = kk / ldk::kAttnHeadDim, d = kk % ldk::kAttnHeadDim;
#pragma unroll
        for (int r = 0; r < kW8AttnRanges; ++r) {
          ao[i][r] = a.att_o[(h * ldk::kAttnMaxSplits + r) * ldk::kAttnHeadDim + d];
          const float* ml = a.att_ml + (h * ldk::kAttnMaxSplits + r) * 2;
          am[i][r] = float2_t{ml[0], ml[1]};
        }
      } else {
        xl[i] = a.x[xo];
      }
      if constexpr (PRO == 1) xu[i] = a.x[xo + a.K];
      if constexpr (kRes) xu[i] = a.res[xo];
      if constexpr (kRms) xn[i] = a.nw[xo];
    }
    u32x4 w[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      const int r = min(p0 + lrow + j * LKW * NW, re - 1);  // clamped; such rows meet zero x
      if constexpr (TAIL) {
        const uint8_t* row = a.wq + (int64_t)r * a.N;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          w[j][d] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(row + min(col + 4 * d, a.N - 4)));
      } else {
        w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.wq + (int64_t)r * a.N + col));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the pass is in flight first
    if constexpr (kRms) {
      if (p0 == rb) {  // the row statistic, once (uniform)
        const int nv = a.K >> 3;
        const bool wr = kRes && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
        float ss = 0.0f;
        auto add = [&](u32x4 xv, u32x4 rv, int t) {
          half8_t h = __builtin_bit_cast(half8_t, xv);
          if constexpr (kRes) h = h + __builtin_bit_cast(half8_t, rv);  // fp16 add
          if (wr && t < nv) *reinterpret_cast<half8_t*>(a.res_out + 8 * t) = h;
#pragma unroll
          for (int j = 0; j < 8; ++j) ss = __builtin_fmaf((float)h[j], (float)h[j], ss);
        };
        add(sx0, sr0, tid);
        for (int t = tid + NW * 64; t < nv; t += NW * 64) {  // rows of more than NW*64 vectors
          const u32x4 xv = *reinterpret_cast<const u32x4*>(a.x + 8 * t);
          u32x4 rv{};
          if constexpr (kRes) rv = *reinterpret_cast<const u32x4*>(a.res + 8 * t);
          add(xv, rv, t);
        }
        ss = ldk::sum_lanes_strided<1>(ss);
        if (lane == 0) stat[wave] = ss;
        ldk::lds_barrier();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) tot += stat[w];
        rs = 1.0f / __builtin_sqrtf(tot / (float)a.K + a.eps);
      }
    }
#pragma unroll
    for (int i = 0; i < XPL; ++i) {
      const int e = lane + 64 * i, m = e / RPW, rr = e % RPW;
      const int k = p0 + wave * LKW + rr % LKW + (rr / LKW) * LKW * NW;
      half_t v;
      if constexpr (kAttn) {
        // the ranges past the live ones hold an earlier call's values (any bits): selects, not
        // products with a zero weight, leave them out
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < kW8AttnRanges; ++r) mx = fmaxf(mx, r < att_live ? am[i][r][0] : -__builtin_inff());
        float f[kW8AttnRanges], l = 0.0f;
#pragma unroll
        for (int r = 0; r < kW8AttnRanges; ++r) {
          f[r] = __expf(am[i][r][0] - mx);
          const float lr = __builtin_fmaf(am[i][r][1], f[r], l);
          l = r < att_live ? lr : l;
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < kW8AttnRanges; ++r) {
          const float orr = __builtin_fmaf(ao[i][r], f[r], o);
          o = r < att_live ? orr : o;
        }
        v = (half_t)(l > 0.0f ? o * inv : 0.0f);  // no live position: 0 (o may be NaN)
      } else {
        v = xl[i];
      }
      if constexpr (PRO == 1) v = ldk::silu_f16(xl[i]) * xu[i];  // fp16 multiply
      if constexpr (kRms) v = ldk::rms_f16(kRes ? xl[i] + xu[i] : xl[i], rs, xn[i]);
      if (e < RPW * MT) xs[wave][m][rr] = (m0 + m < a.M && k < re) ? v : (half_t)0.0f;
    }
    ldk::wave_lds_sync();
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      float xv[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) xv[m] = (float)xs[wave][m][lk + j * LKW];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[j][d], false);
        const float2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[j][d], true);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc[m][4 * d + 0] = __builtin_fmaf(xv[m], lo[0], acc[m][4 * d + 0]);
          acc[m][4 * d + 1] = __builtin_fmaf(xv[m], lo[1], acc[m][4 * d + 1]);
          acc[m][4 * d + 2] = __builtin_fmaf(xv[m], hi[0], acc[m][4 * d + 2]);
          acc[m][4 * d + 3] = __builtin_fmaf(xv[m], hi[1], acc[m][4 * d + 3]);
        }
      }
    }
    ldk::wave_lds_sync();  // the next pass rewrites this wave's x slots
  }

  // ---- reduction: the LKW lanes of a wave sharing ln (DPP/permlane), then the NW waves (LDS)
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = ldk::sum_lanes_strided<LN>(acc[m][j]);
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<float4_t*>(&red[wave][m][16 * lane + 4 * d]) =
            float4_t{acc[m][4 * d], acc[m][4 * d + 1], acc[m][4 * d + 2], acc[m][4 * d + 3]};
  }
  ldk::lds_barrier();
  const int nblk = gridDim.z;
  for (int o = tid; o < MT * CW; o += NW * 64) {
    const int m = o / CW, c = o - m * CW;
    const int n = n0 + c;
    if (n >= a.N || (sp.splits == 1 && m0 + m >= a.M)) continue;
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) v += red[wv][m][c];
    v *= (float)a.scale[n];
    if (sp.splits == 1) {
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)(m0 + m) * a.ldo + n] = (half_t)v;
    } else {
      // every (m, n) word of the tile takes part, rows past M too, so each word is re-zeroed
      float tot;
      uint64_t* word = sp.acc + ((size_t)tile * nblk + mb) * (MT * CW) + o;
      if (ldk::splitk_add(w8_split_ctx(sp), word, v, &tot) && m0 + m < a.M) {
        if (a.bias) tot += (float)a.bias[n];
        a.out[(int64_t)(m0 + m) * a.ldo + n] = (half_t)tot;
      }
    }
  }
}

// ------------------------------------------------------------------------ W8A16 MFMA kernel
//
// Rows in blocks of 16 (padded; grid z walks the blocks, which re-read the weights from the
// MALL) on v_mfma_f32_16x16x32_f16, for M >= 2 where the VALU kernel's
// fp32 FMAs (16 x M per 16 weights) bound it. Lane l = (c16 = l % 16, kb = l / 16) of a wave:
//  * B operand: for each 32-row K step it loads rows k0 + 8 kb + i (i < 8) at columns
//    n0 + 8 c16 .. +7, one 8-byte load per row (16 lanes cover a 128-byte line of a row);
//    an in-register 8x8 byte transpose (v_perm_b32, 4x4 blocks) gives each of its 8 columns its
//    8 consecutive K bytes, decoded exactly to fp16 by gfx950's v_cvt_scalef32_pk_f16_fp8 at
//    scale 1 (two bytes per op; every e4m3 value is an fp16 value: against v_cvt_pk_f32_fp8 then
//    v_cvt_pkrtz, half the decode ops). Column j of the lane feeds MFMA tile j (column c16 of tile j
//    is the real column n0 + 8 c16 + j).
//  * A operand: x row m = c16, K block 8 kb, one 16-byte load (zeros past M or past K).
// A workgroup owns 128 columns and a K range; its waves take K steps round-robin, KSW per pass
// with every load of the pass in flight; partial tiles meet in LDS, then the per-channel scale.
// 64-column tiles share each 128-byte line of a K row with their neighbour. A lane's CPL-byte
// loads need rows aligned to CPL bytes: N % 8 == 0 for 128 columns, N % 4 == 0 for 64 (the plan
// takes 64 when N % 8 != 0). Their launch is one
// dimension over (tile, K split) pieces: the two pieces of each line pair (tiles 2q and 2q + 1,
// one split) run as workgroups L and L + 8 of a group of 16, which the dispatcher places on the
// same XCD (workgroup L goes to XCD L % 8) at about the same time, so the line comes into that
// XCD's L2 once. The pairs past the last whole group of 16, then an odd last tile per split, follow
// in plain order.
__device__ __forceinline__ void w8_pair_piece(int b, int tiles, int& tile, int& split) {
  const int q = tiles >> 1;  // line pairs per split
  const int paired = 2 * q * (int)(gridDim.x / tiles);
  const int full = paired & ~15;
  if (b < paired) {
    const int p = b < full ? 8 * (b >> 4) + (b & 7) : (b >> 1);  // pair index
    const int member = b < full ? (b >> 3) & 1 : b & 1;
    split = p / q;
    tile = 2 * (p - split * q) + member;
  } else {
    split = b - paired;
    tile = tiles - 1;
  }
}

template <int NW, int KSW, int CW>
__global__ __launch_bounds__(NW * 64) void w8a16_mfma_kernel(W8Args a, W8Split sp) {
  typedef _Float16 half8v __attribute__((ext_vector_type(8)));
  static_assert(CW == 128 || CW == 64, "128 or 64 columns");
  constexpr int CPL = CW / 16;  // columns per lane: one MFMA tile each
  typedef uint32_t wrow_t __attribute__((ext_vector_type(CPL / 4)));
  extern __shared__ __align__(16) float wred[];  // [NW][16][CW]
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.wq);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, kb = lane >> 4;
  const int ntiles = (a.N + CW - 1) / CW;
  int tile = (int)blockIdx.x, split = (int)blockIdx.y;
  if constexpr (CW == 64) w8_pair_piece((int)blockIdx.x, ntiles, tile, split);
  const int m0 = blockIdx.z * 16;  // row block (rows past 16 re-read the weights from the MALL)
  const int n0 = tile * CW;
  const int col = min(n0 + CPL * c16, a.N - CPL);  // clamped: tail lanes load valid memory, store nothing
  const int rb = split * sp.kps, re = min(a.K, rb + sp.kps);
  const int nks = (re - rb + 31) / 32;  // K steps of this workgroup
  const bool xrow_ok = m0 + c16 < a.M;
  const half_t* xrow = a.x + (int64_t)min(m0 + c16, a.M - 1) * a.ldx;

  float4_t acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) acc[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int s0 = wave; s0 < nks; s0 += NW * KSW) {
    wrow_t w[KSW][8];
    u32x4 xa[KSW];
#pragma unroll
    for (int u = 0; u < KSW; ++u) {
      const int kblk = rb + (s0 + u * NW) * 32 + 8 * kb;  // first of this lane's 8 rows
      const bool kok = s0 + u * NW < nks && kblk < re;
      xa[u] = *reinterpret_cast<const u32x4*>(xrow + min(kblk, a.K - 8));
      if (!kok || !xrow_ok) xa[u] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = min(kblk + i, re - 1);
        w[u][i] = __builtin_nontemporal_load(reinterpret_cast<const wrow_t*>(a.wq + (int64_t)r * a.N + col));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the pass is in flight before the first wait
#pragma unroll
    for (int u = 0; u < KSW; ++u) {
      if (s0 + u * NW >= nks) break;  // uniform
      const half8v A = __builtin_bit_cast(half8v, xa[u]);
      // 8 x CPL byte transpose: t[c][h] = rows 4h..4h+3 of column c
      uint32_t t[CPL][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int q = 0; q < CPL / 4; ++q) {  // columns 4q .. 4q+3
          const uint32_t ra = w[u][4 * h + 0][q], rbb = w[u][4 * h + 1][q];
          const uint32_t rc = w[u][4 * h + 2][q], rd = w[u][4 * h + 3][q];
          const uint32_t ab_lo = __builtin_amdgcn_perm(rbb, ra, 0x05010400u);  // a0 b0 a1 b1
          const uint32_t ab_hi = __builtin_amdgcn_perm(rbb, ra, 0x07030602u);  // a2 b2 a3 b3
          const uint32_t cd_lo = __builtin_amdgcn_perm(rd, rc, 0x05010400u);
          const uint32_t cd_hi = __builtin_amdgcn_perm(rd, rc, 0x07030602u);
          t[4 * q + 0][h] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // a0 b0 c0 d0
          t[4 * q + 1][h] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);  // a1 b1 c1 d1
          t[4 * q + 2][h] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
          t[4 * q + 3][h] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
        }
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        u32x4 b;
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // two e4m3 bytes to two fp16 per op (scale 1: exact)
          b[2 * h + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(t[j][h], 1.0f, false));
          b[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(t[j][h], 1.0f, true));
        }
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(half8v, b), acc[j], 0, 0, 0);
      }
    }
  }

  // tile j, element i of lane l: row 4 kb + i, column CPL c16 + j of the workgroup's CW
  float* red = wred + (size_t)wave * 16 * CW;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* rrow = red + (4 * kb + i) * CW + CPL * c16;
#pragma unroll
    for (int q = 0; q < CPL / 4; ++q)
      *reinterpret_cast<float4_t*>(rrow + 4 * q) = float4_t{acc[4 * q][i], acc[4 * q + 1][i], acc[4 * q + 2][i], acc[4 * q + 3][i]};
  }
  ldk::lds_barrier();
  const int mrows = min(a.M - m0, 16);
  for (int o = tid; o < mrows * CW; o += NW * 64) {
    const int m = o / CW, c = o - m * CW;
    const int n = n0 + c;
    if (n >= a.N) continue;
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) v += wred[((size_t)wv * 16 + m) * CW + c];
    v *= (float)a.scale[n];
    if (sp.splits == 1) {
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)(m0 + m) * a.ldo + n] = (half_t)v;
    } else {
      float tot;
      if (ldk::splitk_add(w8_split_ctx(sp, split), sp.acc + ((size_t)blockIdx.z * ntiles + tile) * 16 * CW + o, v, &tot)) {
        if (a.bias) tot += (float)a.bias[n];
        a.out[(int64_t)(m0 + m) * a.ldo + n] = (half_t)tot;
      }
    }
  }
}

struct W8Plan {
  int mt, ln, nw, rpl;
  int splits, kps, mblocks;
  int64_t words;  // split-K accumulator words (one per output of every tile and row block)
  bool mfma;
  int ksw;  // MFMA kernel: 32-row K steps per wave and pass
};

constexpr int kW8MfmaWaves = 8;
// 64-column tiles at 9-16 rows run 16 waves: each wave then carries half the K steps of a piece
// into the 16-row LDS reduction. Graph-timed on MI355X at M = 16 (8 -> 16 waves): down 9.20 ->
// 8.23 us, q/o 5.82 -> 4.95, k/v 5.02 -> 4.16; at M = 4 and 8 within 1%; 128-column tiles (gate_up)
// lose with 16 (M = 4 / 8 / 16: 8.42 / 9.30 / 10.62 -> 11.00 / 9.93 / 11.03 us).
constexpr int kW8MfmaWavesWide = 16;

// MFMA plan. Shapes of at least 128 tiles of 128 columns (gate_up: 140) keep 128-column tiles
// and, from 5 rows, split K only as far as one pass of at most 6 K steps per wave needs, so
// gate_up runs whole K (a three-way split costs 1-3 us of fixed-point atomics at 8-16 rows;
// up to 4 rows it pays, below; 64-column tiles there measured 12.1 / 12.7 / 15.0 against 8.9 / 9.5 /
// 10.6 us at M = 4 / 8 / 16). Narrower decode shapes take 64-column tiles and pieces of 16 K
// steps (2 per wave), halved down to 4 while the grid has fewer than 128 workgroups. On MI355X
// (graph-timed, M = 4 / 8 / 16), against 128-column tiles in six pieces: down 1536x8960 (18
// pieces of 16 steps, 432 workgroups; 10 pieces of 28 since, below) 9.41 / 10.61 / 12.55 ->
// 7.37 / 7.55 / 9.07 us; q/o
// 1536x1536 (6 pieces of 8, 144 workgroups) 5.02 / 6.03 / 7.80 -> 4.62 / 4.71 / 5.74 (3 pieces:
// 5.04 / 5.17 / 6.26); k/v 256x1536 (12 pieces of 4) 4.44 / 5.44 / 7.11 -> 3.87 / 3.92 / 4.89.
// Half the columns halve each workgroup's 16-row LDS reduction and its share of the epilogue's
// outputs, which is where the 8- and 16-row cases spent their extra time.
// Prefill rows (M > 16) in 16-row blocks. Short K (q/o/qkv) takes 64-column tiles and splits K
// toward 256 workgroups; long K (down) keeps 128-column tiles and the split the decode rows take,
// cut so that the grid stays within 256 workgroups: a CU that runs two finishes last (graph-timed,
// qkv 2048x1536 M = 17 / 32 / 48 / 64: 128-column tiles in 4 splits, 64-512 workgroups, 7.9 / 8.4 /
// 9.4 / 10.4 us -> 5.1 / 5.8 / 6.4 / 6.6 with 16 waves; down 1536x8960 M = 64: 6 splits on 288
// workgroups 23.9 us, 5 on 240 18.5).
bool w8_short_k(int64_t K) { return (K + 31) / 32 <= 64; }
int64_t w8_prefill_splits(int64_t M, int64_t N, int64_t K, int ln, int64_t splits) {
  const int64_t tiles = (N + 16 * ln - 1) / (16 * ln), steps = (K + 31) / 32;
  const int64_t cap = std::max<int64_t>(1, 256 / (tiles * ((M + 15) / 16)));
  return w8_short_k(K) && ln == 4 ? std::min<int64_t>(cap, steps) : std::min<int64_t>(splits, cap);
}

W8Plan make_w8_mfma_plan(int64_t M, int64_t N, int64_t K, int block_n, int split_k, int64_t ws_bytes) {
  W8Plan p{};
  p.mfma = true;
  p.mt = 16;
  p.mblocks = 1;
  const bool narrow = (N + 127) / 128 < 128 && M <= 16;
  // 128-column tiles load 8 bytes of a row per lane: rows must be 8-byte aligned (N % 8 == 0);
  // 64-column tiles load 4 (N % 4 == 0). Prefill rows of short K take 64 columns too.
  p.ln = block_n == 64 || (block_n == 0 && (narrow || N % 8 || (M > 16 && w8_short_k(K)))) ? 4 : 8;
  p.nw = kW8MfmaWaves;
  const int64_t tiles = (N + 16 * p.ln - 1) / (16 * p.ln);
  const int64_t steps = (K + 31) / 32;
  const int64_t one_pass = (steps + 6 * p.nw - 1) / (6 * p.nw);  // fewest splits of one pass each
  int64_t splits;
  if (split_k > 0) {
    splits = split_k;
  } else if (tiles >= 128 && M <= 4) {  // pieces of 16 steps: gate_up M = 2 / 3 / 4 in three,
                                        // 8.76 / 8.83 / 8.73 -> 7.91 / 8.11 / 8.39 us (at 5 rows
                                        // and more the pieces' atomics cost more than they save)
    splits = std::max<int64_t>(one_pass, (steps + 15) / 16);
  } else if (tiles >= 128 || M > 16) {
    splits = std::max<int64_t>(one_pass, std::min<int64_t>(steps / 8, (64 + tiles - 1) / tiles));
    if (M > 16 && block_n == 0) splits = w8_prefill_splits(M, N, K, p.ln, splits);
  } else {
    int64_t piece = 16;
    while (piece > 4 && tiles * ((steps + piece - 1) / piece) < 128) piece /= 2;
    splits = std::max<int64_t>(one_pass, (steps + piece - 1) / piece);
    // at most one workgroup per CU: a CU that runs two pieces finishes last, so a grid just past
    // 256 loses a whole piece's time and one well past it loses to fewer, larger pieces. down
    // 1536x8960 (24 tiles), graph-timed, M = 4 / 8 / 9 / 12 / 16: 18 splits (432 workgroups)
    // 7.35 / 7.37 / 7.38 / 7.59 / 8.22 us, 11 (264) 8.60 / 9.05 / 9.43 / 9.84 / 10.41, 10 (240)
    // 7.13 / 7.30 / 7.27 / 7.47 / 7.72
    if (tiles * splits > 256 && tiles <= 256) splits = std::max<int64_t>(one_pass, 256 / tiles);
  }
  splits = std::max<int64_t>(1, std::min<int64_t>(splits, kW8MaxSplits));
  const int64_t sps = (steps + splits - 1) / splits;  // K steps per split
  p.kps = (int)(sps * 32);
  p.splits = (int)((steps + sps - 1) / sps);
  p.words = ((M + 15) / 16) * tiles * 16 * (16 * p.ln);
  if (p.splits > 1 && (int64_t)ldk::splitk_bytes(p.words, p.splits) > ws_bytes) {
    p.splits = 1;
    p.kps = (int)(steps * 32);
  }
  if (p.ln == 4 && M > 8 && M <= 16) p.nw = kW8MfmaWavesWide;
  // prefill rows of short K in K splits: 16 waves (qkv M = 17 / 64: 5.9 / 7.7 -> 5.1 / 6.6 us);
  // whole K stays on 8 (M = 128: 8.0 against 8.7 us with 16)
  if (p.ln == 4 && M > 16 && p.splits > 1 && w8_short_k(K)) p.nw = kW8MfmaWavesWide;
  const int64_t per_wave = ((p.kps / 32) + p.nw - 1) / p.nw;
  // K steps per wave and pass: 16 waves hold at most 4 each in registers (1024 lanes: 128 VGPRs)
  p.ksw = per_wave <= 1 ? 1 : per_wave <= 2 ? 2 : (per_wave <= 4 || p.nw == kW8MfmaWavesWide) ? 4 : 6;
  return p;
}

template <int NW, int KSW, int CW>
int launch_w8_mfma_t(const W8Args& a, const W8Split& sp, hipStream_t s) {
  const unsigned tiles = (unsigned)((a.N + CW - 1) / CW), blocks = (unsigned)((a.M + 15) / 16);
  // 64-column tiles: one dimension over (tile, split) pieces (w8_pair_piece)
  const dim3 grid = CW == 64 ? dim3(tiles * (unsigned)sp.splits, 1, blocks) : dim3(tiles, (unsigned)sp.splits, blocks);
  const size_t lds = (size_t)NW * 16 * CW * 4;
  static_assert((size_t)NW * 16 * CW * 4 <= 64 * 1024, "the LDS reduction fits the default dynamic LDS limit");
  (void)hipGetLastError();
  w8a16_mfma_kernel<NW, KSW, CW><<<grid, NW * 64, lds, s>>>(a, sp);
  return ldk::check_launch("w8a16_mfma");
}

template <int CW>
int launch_w8_mfma_cw(const W8Args& a, const W8Split& sp, const W8Plan& p, hipStream_t s) {
  if constexpr (CW == 64) {
    if (p.nw == kW8MfmaWavesWide) {
      switch (p.ksw) {
        case 1: return launch_w8_mfma_t<kW8MfmaWavesWide, 1, CW>(a, sp, s);
        case 2: return launch_w8_mfma_t<kW8MfmaWavesWide, 2, CW>(a, sp, s);
        case 4: return launch_w8_mfma_t<kW8MfmaWavesWide, 4, CW>(a, sp, s);
      }
      return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: %d K steps per wave not instantiated for 16 waves", p.ksw);
    }
  }
  if (p.nw != kW8MfmaWaves) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: %d waves not instantiated", p.nw);
  switch (p.ksw) {
    case 1: return launch_w8_mfma_t<kW8MfmaWaves, 1, CW>(a, sp, s);
    case 2: return launch_w8_mfma_t<kW8MfmaWaves, 2, CW>(a, sp, s);
    case 4: return launch_w8_mfma_t<kW8MfmaWaves, 4, CW>(a, sp, s);
    case 6: return launch_w8_mfma_t<kW8MfmaWaves, 6, CW>(a, sp, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: %d K steps per wave not instantiated", p.ksw);
}

int launch_w8_mfma(const W8Args& a, const W8Split& sp, const W8Plan& p, hipStream_t s) {
  return p.ln == 4 ? launch_w8_mfma_cw<64>(a, sp, p, s) : launch_w8_mfma_cw<128>(a, sp, p, s);
}

int w8_round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }

// Chooses the row block, column tile, rows per lane and K split. Column tiles are 128 columns
// (one 128-byte line per K row) unless block_n asks otherwise. Each workgroup runs one pass
// (all its weight loads in flight at once) whenever K fits 40 splits; rows per lane shrink
// (8, 4, 2) until the grid has at least 256 workgroups (one per CU).
W8Plan make_w8_plan(int64_t M, int64_t N, int64_t K, int block_n, int split_k, int64_t ws_bytes) {
  W8Plan p{};
  p.mt = w8_round_mt(M);
  p.mblocks = (int)((M + p.mt - 1) / p.mt);
  p.ln = block_n ? block_n / 16 : 8;
  p.nw = 4;
  const int64_t tiles = (N + 16 * p.ln - 1) / (16 * p.ln);
  const int64_t lanes_k = (int64_t)(64 / p.ln) * p.nw;
  auto passes = [&](int rpl) { return (K + lanes_k * rpl - 1) / (lanes_k * rpl); };
  p.rpl = 2;
  for (int rpl : {8, 4, 2}) {
    if (tiles * p.mblocks * std::min<int64_t>(passes(rpl), kW8MaxSplits) >= 256) { p.rpl = rpl; break; }
  }
  const int64_t rpp = lanes_k * p.rpl;
  int64_t kps;
  if (split_k > 0) {
    kps = (K + split_k - 1) / split_k;
  } else {
    int64_t per = (passes(p.rpl) + kW8MaxSplits - 1) / kW8MaxSplits;  // passes per split
    // two passes per split where that still gives every CU 1.5 workgroups: half the split-K
    // partials (gate_up M = 1: 420 workgroups of two passes 7.60 us, 840 of one 7.92 us; two
    // passes are not overlapped, so the grids below keep one)
    if (per == 1 && tiles * p.mblocks * ((passes(p.rpl) + 1) / 2) >= 384) per = 2;
    kps = per * rpp;
  }
  kps = (kps + 7) / 8 * 8;
  p.kps = (int)kps;
  p.splits = (int)((K + kps - 1) / kps);
  p.words = tiles * p.mblocks * p.mt * 16 * p.ln;
  const int64_t need = p.splits > 1 ? (int64_t)ldk::splitk_bytes(p.words, p.splits) : 0;
  if (need > ws_bytes) {  // no room for the partials: whole K per workgroup
    p.splits = 1;
    p.kps = (int)((K + 7) / 8 * 8);
  }
  return p;
}

template <int MT, int LN, int NW, int RPL, int PRO, bool TAIL>
int launch_w8_t(const W8Args& a, const W8Split& sp, int mblocks, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 16 * LN - 1) / (16 * LN)), (unsigned)sp.splits, (unsigned)mblocks);
  (void)hipGetLastError();
  w8a16_gemv_kernel<MT, LN, NW, RPL, PRO, TAIL><<<grid, NW * 64, 0, s>>>(a, sp);
  return ldk::check_launch("w8a16_gemv");
}

template <int MT, int LN, int PRO, bool TAIL = false>
int launch_w8_rpl(const W8Args& a, const W8Split& sp, const W8Plan& p, hipStream_t s) {
  switch (p.rpl) {
    case 2: return launch_w8_t<MT, LN, 4, 2, PRO, TAIL>(a, sp, p.mblocks, s);
    case 4: return launch_w8_t<MT, LN, 4, 4, PRO, TAIL>(a, sp, p.mblocks, s);
    case 8: return launch_w8_t<MT, LN, 4, 8, PRO, TAIL>(a, sp, p.mblocks, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: %d rows per lane not instantiated", p.rpl);
}

template <int MT, int PRO>
int launch_w8_ln(const W8Args& a, const W8Split& sp, const W8Plan& p, hipStream_t s) {
  if (a.N % 16) {  // rows only 4-byte aligned: the dword-load variant, on 128-column tiles
    if (p.ln != 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: N %% 16 != 0 runs the VALU kernel on block_n 128 only");
    return launch_w8_rpl<MT, 8, PRO, true>(a, sp, p, s);
  }
  switch (p.ln) {
    case 1: return launch_w8_rpl<MT, 1, PRO>(a, sp, p, s);
    case 2: return launch_w8_rpl<MT, 2, PRO>(a, sp, p, s);
    case 4: return launch_w8_rpl<MT, 4, PRO>(a, sp, p, s);
    case 8: return launch_w8_rpl<MT, 8, PRO>(a, sp, p, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: block_n=%d not supported (16, 32, 64 or 128)", 16 * p.ln);
}

int launch_w8(const W8Args& a, const W8Split& sp, const W8Plan& p, hipStream_t s, int pro = 0) {
  if (pro) {
    if (p.mt != 1) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: the prologues take one row");
    switch (pro) {
      case 1: return launch_w8_ln<1, 1>(a, sp, p, s);
      case 2: return launch_w8_ln<1, 2>(a, sp, p, s);
      case 3: return launch_w8_ln<1, 3>(a, sp, p, s);
      case 4: return launch_w8_ln<1, 4>(a, sp, p, s);
    }
    return ldk::fail(LDK_ERR_INVALID, "w8a16: unknown prologue %d", pro);
  }
  switch (p.mt) {
    case 1: return launch_w8_ln<1, 0>(a, sp, p, s);
    case 2: return launch_w8_ln<2, 0>(a, sp, p, s);
    case 4: return launch_w8_ln<4, 0>(a, sp, p, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: row block %d not instantiated", p.mt);
}

inline unsigned blocks_for(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

}  // namespace

extern "C" int ldk_fp8_quantize(const void* w, int dtype, uint8_t* wq, void* scale, int64_t N, int64_t K, void* stream) {
  if (!w || !wq || !scale) return ldk::fail(LDK_ERR_INVALID, "fp8_quantize: null pointer");
  if (N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "fp8_quantize: N=%lld K=%lld must be positive", (long long)N, (long long)K);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  switch (dtype) {
    case LDK_F16: fp8_quantize_kernel<half_t><<<blocks_for(N, 64), 64, 0, s>>>((const half_t*)w, wq, (half_t*)scale, N, K); break;
    case LDK_BF16: fp8_quantize_kernel<uint16_t><<<blocks_for(N, 64), 64, 0, s>>>((const uint16_t*)w, wq, (uint16_t*)scale, N, K); break;
    case LDK_F32: fp8_quantize_kernel<float><<<blocks_for(N, 64), 64, 0, s>>>((const float*)w, wq, (float*)scale, N, K); break;
    default: return ldk::fail(LDK_ERR_INVALID, "fp8_quantize: unknown dtype %d", dtype);
  }
  return ldk::check_launch("fp8_quantize");
}

extern "C" int ldk_fp8_dequant(const uint8_t* wq, const void* scale, int dtype, void* out, int64_t N, int64_t K, void* stream) {
  if (!wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "fp8_dequant: null pointer");
  if (N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "fp8_dequant: N=%lld K=%lld must be positive", (long long)N, (long long)K);
  hipStream_t s = (hipStream_t)stream;
  const unsigned g = blocks_for(N * K, 256);
  (void)hipGetLastError();
  switch (dtype) {
    case LDK_F16: fp8_dequant_kernel<half_t><<<g, 256, 0, s>>>(wq, (const half_t*)scale, (half_t*)out, N, K); break;
    case LDK_BF16: fp8_dequant_kernel<uint16_t><<<g, 256, 0, s>>>(wq, (const uint16_t*)scale, (uint16_t*)out, N, K); break;
    case LDK_F32: fp8_dequant_kernel<float><<<g, 256, 0, s>>>(wq, (const float*)scale, (float*)out, N, K); break;
    default: return ldk::fail(LDK_ERR_INVALID, "fp8_dequant: unknown dtype %d", dtype);
  }
  return ldk::check_launch("fp8_dequant");
}

// Rows from which the prefill GEMM (prefill.hip) replaces the MFMA kernel's 16-row blocks. The
// blocks re-read the e4m3 weights (twice the bytes of int4) once per 16 rows; the GEMM reads them
// once per 64- or 128-row tile.
static constexpr int64_t kW8GemmRows = 64;

static bool w8_gemm_applies(int64_t M, int64_t N, int64_t K, int64_t ldx, const void* out, int64_t ldo) {
  return ldk::gemm_supported(ldk::WFmt::kE4M3, M, N, K, 0, ldx) && ldk::aligned(out, 8) && ldo % 4 == 0;
}

// The library's choice: the GEMM for more than kW8GemmRows rows (on wide shapes more than 16)
// unless the blocks still fit, or a tuning argument names another kernel.
static bool w8_uses_gemm(int64_t M, int64_t N, int64_t K, int64_t ldx, const void* out, int64_t ldo, int block_n,
                         int split_k, int flags) {
  if (flags & LDK_PATH_GEMM) return true;
  // wide shapes (N >= 8192) from 17 rows: the 16-row blocks re-read all of their e4m3 weights per
  // block (gate_up M = 17 / 32 / 64: 16.9 / 20.3 / 29.7 us on the blocks, 10.9 / 11.2 / 15.5 on the
  // GEMM's 32-row tiles)
  if (M <= (N >= 8192 ? 16 : kW8GemmRows) || block_n || split_k || (flags & (LDK_PATH_VALU | LDK_PATH_MFMA))) return false;
  // narrow shapes past 64 rows keep the blocks while they fit in 256 workgroups: short K on
  // 64-column tiles (qkv M = 96 / 128: 8.1 / 8.0 us against 10.2 / 10.1 on the GEMM, o M = 160 8.3
  // against 9.7; qkv M = 160, 320 workgroups, 13.4 against 10.2), long K while they still split K
  // at least twice (down M = 96 / 128 / 160: 19.8 / 23.4 / 23.6 against 26.0 / 26.5 / 24.2; M = 192
  // in whole K 41.0 against 24.6)
  if (N < 8192) {
    const int64_t blocks = (M + 15) / 16;
    if (w8_short_k(K) ? (N + 63) / 64 * blocks <= 256 : (N + 127) / 128 * blocks <= 128) return false;
  }
  return w8_gemm_applies(M, N, K, ldx, out, ldo);
}

namespace {

// What a W8A16 call runs: the prefill GEMM, or a decode-kernel plan.
struct W8Call {
  bool gemm;
  W8Plan p;
};

// A call's shape and tuning arguments checked without its pointers: the errors the call returns
// for them, and what it runs. ldx, ldo and the output's alignment decide whether the prefill GEMM
// takes the call (out may be null for a query: taken as aligned); ws_bytes is the workspace the
// call has.
int w8_plan_call(const char* fn, int64_t M, int64_t N, int64_t K, int64_t ldx, const void* out, int64_t ldo,
                 int block_n, int split_k, int flags, int64_t ws_bytes, W8Call* c) {
  c->gemm = false;
  if (M <= 0 || N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "%s: M, N, K must be positive", fn);
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N=%lld must be a multiple of 4", fn, (long long)N);
  if (K % 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: K=%lld must be a multiple of 8", fn, (long long)K);
  if (ldx < K || ldo < N) return ldk::fail(LDK_ERR_INVALID, "%s: row stride smaller than K/N", fn);
  if (N > INT32_MAX / 16 || K > INT32_MAX / 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N or K too large", fn);
  if (flags & ~(LDK_PATH_VALU | LDK_PATH_MFMA | LDK_PATH_GEMM))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: flags 0x%x not supported", fn, flags);
  if (!!(flags & LDK_PATH_VALU) + !!(flags & LDK_PATH_MFMA) + !!(flags & LDK_PATH_GEMM) > 1)
    return ldk::fail(LDK_ERR_INVALID, "%s: the VALU, MFMA and GEMM paths are exclusive", fn);
  if (split_k < 0 || split_k > kW8MaxSplits) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: split_k=%d outside 0..%d", fn, split_k, kW8MaxSplits);
  if ((flags & LDK_PATH_GEMM) && !w8_gemm_applies(M, N, K, ldx, out, ldo))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the prefill GEMM takes N %% 16 == 0, K %% 64 == 0 and an 8-byte aligned "
                     "output with ldo %% 4 == 0 (M=%lld N=%lld K=%lld)", fn, (long long)M, (long long)N, (long long)K);
  if (w8_uses_gemm(M, N, K, ldx, out, ldo, block_n, split_k, flags)) {
    if (block_n && block_n != 128 && block_n != 256)
      return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d must be 128 or 256 on the GEMM path", fn, block_n);
    c->gemm = true;
    return LDK_OK;
  }
  if (M > 65535LL * 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: M=%lld too large", fn, (long long)M);
  if (M > 16 && (flags & LDK_PATH_VALU)) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the VALU kernel takes M <= 16", fn);
  if (block_n && block_n != 16 && block_n != 32 && block_n != 64 && block_n != 128)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d must be 16, 32, 64 or 128", fn, block_n);
  // MFMA from 2 rows (the VALU kernel's fp32 FMAs grow with M; measured at M = 4: 17.4 us VALU,
  // 9.5 us MFMA at M = 8 on gate_up; at M = 2 gate_up / down / q/o / k/v 8.91 / 6.71 / 4.79 /
  // 4.05 us VALU against 8.62 / 6.66 / 4.19 / 3.51 MFMA); block_n other than 128 keeps the
  // VALU kernel, which has the narrower tiles.
  const bool mfma = M > 16 || (flags & LDK_PATH_MFMA) || (M >= 2 && !(flags & LDK_PATH_VALU) && (block_n == 0 || block_n == 128));
  if (mfma && block_n && block_n != 128 && block_n != 64)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the MFMA kernel takes block_n 64 or 128", fn);
  if (mfma && block_n == 128 && N % 8)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=128 on the MFMA kernel takes N %% 8 == 0 (N=%lld)", fn, (long long)N);
  if (!mfma && N % 16 && block_n && block_n != 128)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N %% 16 != 0 runs the VALU kernel on block_n 128 only", fn);
  c->p = mfma ? make_w8_mfma_plan(M, N, K, block_n, split_k, ws_bytes) : make_w8_plan(M, N, K, block_n, split_k, ws_bytes);
  if (split_k > 1 && c->p.splits == 1)
    return ldk::fail(LDK_ERR_INVALID, "%s: split_k=%d needs a workspace for the partial sums", fn, split_k);
  return LDK_OK;
}

int w8_plan_flags(const W8Plan& p) { return p.mfma ? LDK_PATH_MFMA : LDK_PATH_VALU; }

}  // namespace

extern "C" int ldk_w8a16_matmul(const void* x, int64_t ldx, const uint8_t* wq, const void* scale, const void* bias, void* out,
                                int64_t ldo, int64_t M, int64_t N, int64_t K, int block_n, int split_k, int flags,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  static const char* fn = "w8a16_matmul";
  if (!x || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "%s: null pointer", fn);
  if (!ldk::aligned(x, 2) || !ldk::aligned(wq, 16) || !ldk::aligned(scale, 2))
    return ldk::fail(LDK_ERR_ALIGN, "%s: wq must be 16-byte aligned", fn);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  const int64_t wsb = workspace ? workspace_bytes : 0;
  W8Call c;
  const int st = w8_plan_call(fn, M, N, K, ldx, out, ldo, block_n, split_k, flags, wsb, &c);
  if (st) return st;
  if (c.gemm) {
    const ldk::GemmArgs g{(const half_t*)x, ldx, wq, (const half_t*)scale, nullptr, (const half_t*)bias, (half_t*)out, ldo,
                          (int)M, (int)N, (int)K, 0, workspace, wsb, block_n, split_k};
    return ldk::gemm_launch(ldk::WFmt::kE4M3, g, (hipStream_t)stream);
  }
  const W8Plan& p = c.p;
  const W8Args a{(const half_t*)x, ldx, wq, (const half_t*)scale, (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K};
  const W8Split sp{p.splits, p.kps, p.splits > 1 ? static_cast<uint64_t*>(workspace) : nullptr,
                   p.splits > 1 ? ldk::splitk_side(workspace, p.words) : nullptr};
  return p.mfma ? launch_w8_mfma(a, sp, p, (hipStream_t)stream) : launch_w8(a, sp, p, (hipStream_t)stream);
}

// Prefill rows of gate_up with SwiGLU in the prefill GEMM's epilogue, the e4m3 twin of
// ldk_w4a16_matmul_swiglu: out [M, N/2] = silu(g) * u of the product's halves, bit for bit
// ldk_w8a16_matmul then ldk_swiglu, where the library's plan for the shape is the GEMM on paired
// column groups of at most 4 row tiles with no K split.
static bool w8_swiglu_gemm_applies(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ws_bytes) {
  return N % 8 == 0 && w8_uses_gemm(M, N, K, ldx, nullptr, N, 0, 0, 0) &&
         ldk::gemm_swiglu_applies(ldk::WFmt::kE4M3, M, N, K, 0, ldx, 0, 0, ws_bytes);
}

extern "C" int ldk_w8a16_matmul_swiglu_applies(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 && w8_swiglu_gemm_applies(M, N, K, K, ldk_workspace_bytes()) ? 1 : 0;
}

extern "C" int ldk_w8a16_matmul_swiglu(const void* x, int64_t ldx, const uint8_t* wq, const void* scale, const void* bias,
                                       void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  static const char* fn = "w8a16_matmul_swiglu";
  if (!x || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "%s: null pointer", fn);
  if (!ldk::aligned(x, 2) || !ldk::aligned(wq, 16) || !ldk::aligned(scale, 2))
    return ldk::fail(LDK_ERR_ALIGN, "%s: wq must be 16-byte aligned", fn);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  const int64_t wsb = workspace ? workspace_bytes : 0;
  W8Call c;
  const int st = w8_plan_call(fn, M, N, K, ldx, nullptr, N, 0, 0, 0, wsb, &c);  // out checked below
  if (st) return st;
  if (N % 2 || ldo < N / 2 || ldo % 4 || !ldk::aligned(out, 8))
    return ldk::fail(LDK_ERR_ALIGN, "%s: out [M, N/2] 8-byte aligned with ldo >= N/2 and ldo %% 4 == 0", fn);
  if (!w8_swiglu_gemm_applies(M, N, K, ldx, wsb))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: M=%lld N=%lld K=%lld does not run the prefill GEMM with paired column "
                     "groups (ldk_w8a16_matmul_swiglu_applies)", fn, (long long)M, (long long)N, (long long)K);
  ldk::GemmArgs g{(const half_t*)x, ldx, wq, (const half_t*)scale, nullptr, (const half_t*)bias, (half_t*)out, ldo,
                  (int)M, (int)N, (int)K, 0, workspace, wsb, 0, 0};
  g.swiglu = 1;
  return ldk::gemm_launch(ldk::WFmt::kE4M3, g, (hipStream_t)stream);
}

extern "C" int ldk_w8a16_config(int64_t M, int64_t N, int64_t K, int* block_n, int* split_k, int* flags) {
  static const char* fn = "w8a16_config";
  if (!block_n || !split_k || !flags) return ldk::fail(LDK_ERR_INVALID, "%s: null block_n, split_k or flags", fn);
  W8Call c;
  const int st = w8_plan_call(fn, M, N, K, K, nullptr, N, *block_n, *split_k, *flags, ldk_workspace_bytes(), &c);
  if (st) return st;
  if (c.gemm) {
    ldk::gemm_plan(ldk::WFmt::kE4M3, M, N, K, *block_n, *split_k, ldk_workspace_bytes(), block_n, split_k);
    *flags = LDK_PATH_GEMM;
    return LDK_OK;
  }
  *block_n = 16 * c.p.ln;
  *split_k = c.p.splits;
  *flags = w8_plan_flags(c.p);
  return LDK_OK;
}

// Fused decode entry (one row): the down projection's activation silu(g) * u is formed inside
// the W8A16 GEMV's x staging, one launch fewer per decode layer (the reference's
// OursFP8Backend runs swiglu and the FP8 linear as two, kernels/e2e/model.py:100-118).
extern "C" int ldk_w8a16_swiglu_matmul(const void* gate_up, const uint8_t* wq, const void* scale, const void* bias,
                                       void* out, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  if (!gate_up || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "w8a16_swiglu_matmul: null pointer");
  if (N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "w8a16_swiglu_matmul: N, K must be positive");
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_swiglu_matmul: N=%lld must be a multiple of 4", (long long)N);
  if (K % 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_swiglu_matmul: K=%lld must be a multiple of 8", (long long)K);
  if (!ldk::aligned(gate_up, 2) || !ldk::aligned(wq, 16) || !ldk::aligned(scale, 2))
    return ldk::fail(LDK_ERR_ALIGN, "w8a16_swiglu_matmul: wq must be 16-byte aligned");
  if (N > INT32_MAX / 16 || K > INT32_MAX / 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_swiglu_matmul: N or K too large");
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w8a16_swiglu_matmul: workspace must be a 256-byte aligned pointer");
  const W8Plan p = make_w8_plan(1, N, K, 0, 0, workspace ? workspace_bytes : 0);
  const W8Args a{(const half_t*)gate_up, 2 * K, wq, (const half_t*)scale, (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K};
  const W8Split sp{p.splits, p.kps, p.splits > 1 ? static_cast<uint64_t*>(workspace) : nullptr,
                   p.splits > 1 ? ldk::splitk_side(workspace, p.words) : nullptr};
  return launch_w8(a, sp, p, (hipStream_t)stream, 1);
}

// Fused decode entry (one row): RMSNorm (+ residual) forms the activation inside the W8A16 GEMV's
// x staging, one launch fewer per use (the reference's OursFP8Backend runs rmsnorm and the FP8
// linear as two, kernels/e2e/model.py:79-118).
extern "C" int ldk_w8a16_rmsnorm_matmul(const void* x, const void* residual, void* residual_out, const void* norm_weight,
                                        float eps, const uint8_t* wq, const void* scale, const void* bias, void* out,
                                        int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !norm_weight || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "w8a16_rmsnorm_matmul: null pointer");
  if ((residual == nullptr) != (residual_out == nullptr))
    return ldk::fail(LDK_ERR_INVALID, "w8a16_rmsnorm_matmul: residual and residual_out must both be given or both be null");
  if (residual && (residual == residual_out || x == residual_out))
    return ldk::fail(LDK_ERR_INVALID, "w8a16_rmsnorm_matmul: residual_out must not alias x or residual");
  if (N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "w8a16_rmsnorm_matmul: N, K must be positive");
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_rmsnorm_matmul: N=%lld must be a multiple of 4", (long long)N);
  if (K % 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_rmsnorm_matmul: K=%lld must be a multiple of 8", (long long)K);
  if (!ldk::aligned(x, 16) || !ldk::aligned(norm_weight, 16) || !ldk::aligned(wq, 16) || !ldk::aligned(scale, 2) ||
      (residual && (!ldk::aligned(residual, 16) || !ldk::aligned(residual_out, 16))))
    return ldk::fail(LDK_ERR_ALIGN, "w8a16_rmsnorm_matmul: x, norm_weight, residual, residual_out and wq must be 16-byte aligned");
  if (N > INT32_MAX / 16 || K > INT32_MAX / 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_rmsnorm_matmul: N or K too large");
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w8a16_rmsnorm_matmul: workspace must be a 256-byte aligned pointer");
  const W8Plan p = make_w8_plan(1, N, K, 0, 0, workspace ? workspace_bytes : 0);
  const W8Args a{(const half_t*)x,  K,      wq, (const half_t*)scale, (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K,
                 (const half_t*)residual, (half_t*)residual_out, (const half_t*)norm_weight, eps};
  const W8Split sp{p.splits, p.kps, p.splits > 1 ? static_cast<uint64_t*>(workspace) : nullptr,
                   p.splits > 1 ? ldk::splitk_side(workspace, p.words) : nullptr};
  return launch_w8(a, sp, p, (hipStream_t)stream, residual ? 3 : 2);
}

// Fused decode entry (one row): the o projection with x the decode attention output that
// ldk_decode_attention_ranges left as per-range partials, merged in the W8A16 GEMV's x staging,
// so the attention's merge and the projection are one launch (the reference runs the attention
// block and the FP8 linear as separate ops, kernels/e2e/model.py:100-118,236-243).
extern "C" int ldk_w8a16_attn_matmul(const int64_t* pos, int64_t max_len, int64_t rlen, int nq, const uint8_t* wq,
                                     const void* scale, const void* bias, void* out, int64_t N, int64_t K,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "w8a16_attn_matmul";
  if (!pos || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "%s: null pointer", fn);
  if (N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "%s: N, K must be positive", fn);
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N=%lld must be a multiple of 4", fn, (long long)N);
  if (nq <= 0 || nq > ldk::kAttnMaxHeads || K != (int64_t)nq * ldk::kAttnHeadDim)
    return ldk::fail(LDK_ERR_INVALID, "%s: K=%lld must be nq * 128 with 1 <= nq <= %d", fn, (long long)K, ldk::kAttnMaxHeads);
  if (max_len <= 0 || rlen <= 0 || rlen % 32 || (max_len + rlen - 1) / rlen > kW8AttnRanges || max_len > INT32_MAX)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: max_len=%lld in ranges of rlen=%lld (a multiple of 32) must give 1..%d ranges",
                     fn, (long long)max_len, (long long)rlen, kW8AttnRanges);
  if (!ldk::aligned(pos, 8) || !ldk::aligned(wq, 16) || !ldk::aligned(scale, 2) || !ldk::aligned(out, 2) ||
      (bias && !ldk::aligned(bias, 2)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: pos 8-byte and wq 16-byte aligned", fn);
  if (N > INT32_MAX / 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N too large", fn);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  const float *po = nullptr, *pm = nullptr;
  int st = ldk::attention_partials(fn, stream, pos, max_len, rlen, nq, &po, &pm);
  if (st) return st;
  const W8Plan p = make_w8_plan(1, N, K, 0, 0, workspace ? workspace_bytes : 0);
  W8Args a{nullptr, K, wq, (const half_t*)scale, (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K};
  a.att_o = po;
  a.att_ml = pm;
  a.att_pos = pos;
  a.att_len = (int)max_len;
  a.att_rlen = (int)rlen;
  const W8Split sp{p.splits, p.kps, p.splits > 1 ? static_cast<uint64_t*>(workspace) : nullptr,
                   p.splits > 1 ? ldk::splitk_side(workspace, p.words) : nullptr};
  return launch_w8(a, sp, p, (hipStream_t)stream, 4);
}
