// W4A16 matmul for decode (M <= 16): y[M, N] = x[M, K] @ dequant(W)^T (+ bias).
//
// Replaces the reference's Triton GEMV/GEMM launch paths (kernels/w4a16.py:100-160, 214-279) and
// its CUDA decode kernel (kernels/cuda/w4a16_decode.cu:29-121) with three gfx950 kernels that
// share one work decomposition:
//
//  * Tiles and groups. A workgroup owns CW output columns and a range of quantization groups
//    (all of K, or 1/splits of it). Inside the workgroup each wave takes whole groups, so every
//    lane applies one scale and one zero point per group and a group's partial sums never leave
//    the lane until the final reduction. Column tiles are 128 bytes of packed weight per row (one
//    L2 line) by default: 64-byte tiles put the two halves of a line on different XCDs, which
//    then both fetch it (measured 1.5x slower on MI355X).
//  * Memory-level parallelism. Every load of a pass is issued before the first wait: the x row,
//    the scale and zero words and the packed weight rows, pinned in that order by a scheduling
//    barrier (without it the compiler reuses registers and issues later rows only after the
//    first data has arrived, a second serial memory round trip). Data is consumed in issue order,
//    so each s_waitcnt vmcnt(n) releases work as it lands.
//  * No workgroup barrier before the compute: x rows are staged through LDS by the wave that
//    uses them (wave-local exchange), so weight loads never wait on other waves.
//  * Split-K. Partials are reduced inside the workgroup (DPP row rotations and gfx950 permlane
//    swaps within a wave, then LDS across waves). Narrow shapes (few column tiles) also split the
//    groups over `splits` workgroups that meet in a caller-provided workspace through one 64-bit
//    fixed-point atomic add per output that also counts arrivals; the add that completes the
//    count stores the output and re-zeroes the word (one launch, no zero-fill, no cast kernel,
//    one memory round trip, deterministic).
//
// Dequantization happens in registers: a nibble q ORed into the mantissa of fp16 1024.0
// (0x6400) is exactly the fp16 value 1024 + q, so one v_and_or_b32 per pair turns packed nibbles
// into fp16 pairs (q_i, q_{i+4}); x is staged as the matching pairs (x_i, x_{i+4}).
//
//  - M = 1 kernel (FACTORED, M <= 2): s * (sum x*q - z * sum x) per group, the reference's
//    FACTORED identity (kernels/w4a16.py:116-119). Nibbles 1/3/5/7 are masked in place as 16*q
//    and meet x pairs pre-scaled by 1/16; one v_dot2_f32_f16 chain per column and row runs over
//    the lane's four rows of a group, starting at -1024*(offset-weighted sum of x): 5 + 4M VALU
//    ops per 8 weights (the nibble pairs are decoded once for both rows). All tile parameters are
//    compile-time, so the epilogue is straight-line code.
//  - VALU kernel (M <= 8, EXACT): ((1024+q) - (1024+z)) * s in packed fp16 is exactly the
//    reference's dequantized weight (one RNE rounding, kernels/reference.py:35), then dot2 with
//    each x row. The path when exact dequantization is requested.
//  - MFMA kernel (from 3 rows): an int32 word holds 8 consecutive K of one column, which is exactly
//    one lane's B operand of v_mfma_f32_16x16x32_f16. A lane's 128-bit load feeds four 16x16
//    tiles; B = (q - z) exactly in fp16, A = x rows permuted to the nibble-pair order, the fp32
//    tile of one group is scaled by s once.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "ldk_common.h"
#include "attention.h"
#include "prefill.h"

namespace {

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves
constexpr int kMaxSplits = 32;            // workgroups splitting one column tile (<= ldk::kFixMaxSplits)

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
  int splits;     // workgroups per split column tile
  int gps;        // groups per split
  uint64_t* acc;  // [split tiles][n] fixed-point accumulators (splits > 1), zero between launches
  int full;       // tiles [0, full) run whole (one workgroup, no split); the split workgroups of
                  // tiles [full, tiles) come first in dispatch order
  int nsplit;       // number of those split workgroups
  uint64_t smagic;  // ceil(2^32 / splits): b / splits == (b * smagic) >> 32 for b, splits < 2^16
  float* side;      // fp32 side slots of the accumulators (ldk::SplitK), zero between launches
  int grem;         // 0: every split takes gps groups (the last one the rest); > 0: a split count
                    // the caller asked for, groups dealt evenly: splits s < grem take gps + 1
};

// ceil(2^32 / d) for 1 <= d < 2^16: floor(n / d) == (n * magic) >> 32 for every n < 2^16.
inline uint64_t div_magic(uint32_t d) { return ((uint64_t(1) << 32) + d - 1) / d; }

// Work of one workgroup: a column tile and its range of quantization groups [gb, ge).
struct TileWork {
  int tile, gb, ge;
  int split;   // index among the workgroups splitting the tile's groups
  bool whole;  // all groups of the tile: the result is stored directly, no split-K reduction
};

// The split-K context of a workgroup (ldk::SplitK): the launch's words, their side slots, and its
// index among the tile's splits.
__device__ __forceinline__ ldk::SplitK split_ctx(const SplitArgs& sp, const TileWork& tw) {
  return ldk::SplitK{sp.acc, sp.side, sp.splits, tw.split};
}

// Dispatch order: the split workgroups of tiles [full, tiles) first (splits per tile), then the
// whole tiles [0, full). Requests are served roughly in issue order, so the split workgroups'
// data arrives early and their cross-workgroup round trip overlaps the streaming of the whole
// tiles. Branch-free scalar code with no runtime integer division, so every kernel argument is
// fetched in one scalar round trip before the first vector load.
//
// G > 1 (whole tiles only): workgroups are dispatched to the 8 XCDs round-robin (XCD = id % 8),
// and G adjacent tiles share 128-byte lines of the scales and zeros (and of the weights for
// 16-column tiles). Within each window of 8G workgroups, tile xcd*G + j goes to workgroup
// 8j + xcd, so the G tiles of a line run on one XCD and its L2 fetches the line once, while the
// tiles in flight together stay within an 8G-tile window (DRAM locality). An incomplete last
// window keeps the identity order. Measured on the 16-column tiles of the small projections
// (G = 4, weight lines shared too): q/o M = 1 3.45 -> 3.34 us, qkv 3.50 -> 3.34 us. On gate_up's
// 32-column tiles (G = 2, only the scale and zero lines shared) it measured slower (5.25 -> 5.52 us),
// so those keep the plain order.
template <int G = 1>
__device__ __forceinline__ TileWork map_block(const SplitArgs& sp, int ng) {
  const int bid = blockIdx.x;
  const bool in_split = bid < sp.nsplit;
  const int q = (int)(((uint64_t)(uint32_t)bid * sp.smagic) >> 32);
  TileWork w;
  w.tile = in_split ? sp.full + q : bid - sp.nsplit;
  const int split = in_split ? bid - q * sp.splits : 0;
  w.split = split;
  w.whole = !in_split || sp.splits == 1;
  if constexpr (G > 1) {
    // the whole-tile range: [0, full) after the split workgroups, or every tile without splits
    const int base = in_split ? 0 : sp.nsplit, count = in_split ? sp.nsplit : (int)gridDim.x - sp.nsplit;
    const int l = bid - base, lim = count / (8 * G) * (8 * G);
    if (w.whole && l < lim) w.tile = (in_split ? sp.full : 0) + (l - l % (8 * G)) + (l % 8) * G + (l % (8 * G)) / 8;
  }
  w.gb = w.whole ? 0 : split * sp.gps + min(split, sp.grem);
  w.ge = w.whole ? ng : min(ng, w.gb + sp.gps + (split < sp.grem ? 1 : 0));
  return w;
}

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

// 32-byte LDS record of one packed x row for the FACTORED loop: the x pairs with the odd pairs
// scaled by 1/16 (exact), then c0 = -1024*((x0+x2+x4+x6) + (x1+x3+x5+x7)/16) and x0+...+x7.
__device__ __forceinline__ void store_fact_record(unsigned char* dst, u32x4 d) {
  u32x4 p = x_pairs(d);
  const half2_t a0 = ldk::u2h2(p[0]), a2 = ldk::u2h2(p[2]);
  const half2_t b1 = ldk::u2h2(p[1]), b3 = ldk::u2h2(p[3]);
  const float xa = ((float)a0[0] + (float)a0[1]) + ((float)a2[0] + (float)a2[1]);
  const float xb = ((float)b1[0] + (float)b1[1]) + ((float)b3[0] + (float)b3[1]);
  const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
  p[1] = ldk::h22u(b1 * sixteenth);
  p[3] = ldk::h22u(b3 * sixteenth);
  *reinterpret_cast<u32x4*>(dst) = p;
  *reinterpret_cast<float2_t*>(dst + 16) = float2_t{-1024.0f * (xa + 0.0625f * xb), xa + xb};
}

// Shared epilogue of the multi-row kernels: the workgroup's NW wave partials of n outputs sit
// wave-major in `red`; sum them and store (or hand them to the cross-workgroup split-K
// reduction).
// `words`: the tile's first accumulator word (split tiles only).
template <typename Store>
__device__ __forceinline__ void finish_tile(const float* red, int n, int NW, const TileWork& tw,
                                            const SplitArgs& sp, uint64_t* words, Store store) {
  auto part = [&](int o) { return ldk::sum_waves(red + o, n, NW); };
  if (tw.whole) {
    for (int o = threadIdx.x; o < n; o += blockDim.x) store(o, part(o));
  } else {
    ldk::splitk_accumulate(split_ctx(sp, tw), words, n, part, store);
  }
}

// ---------------------------------------------------------------------------- M = 1 kernel
//
// Lane (ln, lk) of a wave: ln < LN runs along N (columns n0 + 4ln .. +3), lk < LKW = 64/LN along
// K. Each lane owns RPL = 4 packed rows of one group, so LG = rows_per_group / 4 lanes share a
// group (sub = lk % LG takes rows sub, sub + LG, sub + 2LG, sub + 3LG) and a wave covers
// GPW = LKW / LG groups = RPW = 4 * LKW packed rows per pass. Waves take passes over the
// workgroup's groups at a stride of NW * GPW groups.
// RSH > 0 fixes log2(rows per group) at compile time (the common group size 128 has RSH = 4);
// RSH = 0 reads it from the arguments.
//
// PRO selects how the activation row is formed while it is staged (each x row of a pass is read
// by one lane, so an elementwise prologue costs one evaluation per element per workgroup):
//  - kProNone: x as given;
//  - kProRms / kProRmsRes: x = rmsnorm(x (+ residual)) * weight with the rounding steps of the
//    standalone RMSNorm kernel (h = fp16(x + r), fp32 mean of squares, w * fp16(h * rstd)).
//    The row statistic is reduced once per workgroup (wave sums, one LDS barrier). In the
//    EXACT variants (kProRmsX, kProRmsResX: whole tiles and one pass per wave covering the
//    row, which every decode shape is) each wave sums the rows its pass staged anyway, so no
//    load is added and the barrier waits only for the pass's first (x, residual) loads, not for
//    its weight rows. The general variants also load the row (tid, tid + NT, ...) ahead of the
//    pass, as buffer loads that read zero past the row without a branch. Workgroup 0 writes h,
//    the updated residual stream, to res_out;
//  - kProSwiglu: x = fp16(silu(g)) * u from a fused [g | u] row of 2K (the standalone SwiGLU
//    kernel's steps, so the staged values are bit-identical to its output);
//  - kProRmsPre: x = rmsnorm(h) * weight where the row statistic comes from the per-tile partial
//    sums of squares that the kEpiResStat launch producing h wrote: every wave sums them itself
//    (a fixed lane order, so every workgroup gets the same bits), with no barrier and no row
//    loads beyond its own staged rows.
// and one epilogue, for the projection that feeds a residual + RMSNorm:
//  - kEpiResStat (whole tiles, x as given): h = fp16(y + residual) with y the fp16 output (the
//    reference's linear, then the norm's residual add), stored as the output, and the tile's
//    sum of h^2 stored to stats[tile];
//  - kProAttnStat: the kEpiResStat epilogue, with x merged in the staging from the decode
//    attention's per-range partials (ldk_decode_attention_ranges): for the 8 dims of head h a
//    lane stages, x = sum_r f_r o_r / sum_r f_r l_r with f_r = exp(m_r - max m) over the ranges
//    live at pos, rounded once to fp16 (the merge launch's arithmetic, except that its sum of the
//    f_r l_r is a lane reduction, here a chain in range order, and its division per value is one
//    reciprocal per 8 values here: the two can differ in the last fp32 bit).
enum Prologue {
  kProNone = 0, kProRms = 1, kProRmsRes = 2, kProSwiglu = 3, kProRmsX = 4, kProRmsResX = 5,
  kProRmsPre = 6, kEpiResStat = 7, kProAttnStat = 8
};
constexpr int kMaxRowStats = 256;  // per-tile partials a kProRmsPre launch reads
constexpr int kAttnRanges = 4;     // attention ranges a kProAttnStat launch merges (registers)

struct ProArgs {
  const half_t* res;  // kProRmsRes, kEpiResStat: residual added before the norm
  half_t* res_out;    // kProRmsRes: x + residual (written by workgroup 0)
  const half_t* nw;   // kProRms*: norm weight [K]
  float eps;
  float* stats;       // kEpiResStat: per-tile sums of h^2 (written); kProRmsPre: read
  int nstats;
  // kProAttnStat: the attention's partials (attention.h), its position and range geometry
  const float* att_o;
  const float* att_ml;
  const int64_t* att_pos;
  int att_len, att_rlen;
};

// The staged 8 activations of one packed row from the raw loads (x, second operand, norm weight).
template <int PRO>
__device__ __forceinline__ u32x4 pro_stage(u32x4 xr, u32x4 x2, u32x4 x3, float rs) {
  if constexpr (PRO == kProNone || PRO == kEpiResStat) {
    return xr;
  } else if constexpr (PRO == kProSwiglu) {
    const half8_t g = __builtin_bit_cast(half8_t, xr), u = __builtin_bit_cast(half8_t, x2);
    half8_t sv;
#pragma unroll
    for (int j = 0; j < 8; ++j) sv[j] = ldk::silu_f16(g[j]);
    return __builtin_bit_cast(u32x4, sv * u);  // fp16 multiply
  } else {
    half8_t h = __builtin_bit_cast(half8_t, xr);
    if constexpr (PRO == kProRmsRes || PRO == kProRmsResX) h = h + __builtin_bit_cast(half8_t, x2);  // fp16 add
    half8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = (float)h[j] * rs;
      asm volatile("" : "+v"(v));  // a -0 * rs must stay -0 (no v_fma_mix with a +0 addend)
      o[j] = (half_t)v;
    }
    return __builtin_bit_cast(u32x4, __builtin_bit_cast(half8_t, x3) * o);  // fp16 multiply
  }
}

// Static LDS of the M = 1 kernel: x records [NW][MR][RPW] of 32 bytes, wave partials [NW][MR][LN]
// float4 and the statistic slots. Instantiations are limited to 48 KiB so that three workgroups
// fit a CU.
constexpr int m1_lds_bytes(int ln, int nw, int mr) { return nw * mr * (256 / ln) * 32 + nw * mr * ln * 16 + nw * 4; }
constexpr bool m1_lds_ok(int ln, int nw, int mr) { return m1_lds_bytes(ln, nw, mr) <= 48 * 1024; }

// The one-row 32-column kernel is held to 7 waves per SIMD (<= 72 VGPRs): the gate_up grid
// averages 3.1 six-wave workgroups per CU, and at 6 waves per SIMD a CU's fourth workgroup does
// not fit and runs as a tail (measured 5.17 -> 5.80 us at 73 VGPRs).
template <int LN, int NW, int RSH, int PRO, int MR>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(LN == 8 && NW <= 8 && (PRO == kProNone || PRO == kProRmsPre) ? 7 : 1)))
void w4a16_m1_kernel(W4Args a, SplitArgs sp, int out_vec, ProArgs pa) {
  static_assert(MR == 1 || PRO == kProNone, "fused prologues take one row");
  constexpr int LKW = 64 / LN, RPL = 4, RPW = RPL * LKW, CW = 4 * LN;
  // x records of a pass: MR rows x RPW packed rows, XL per lane (record r = lane + 64 i is row
  // r / RPW, packed row r % RPW of the pass)
  constexpr int XREC = MR * RPW, XL = (XREC + 63) / 64;
  constexpr bool kExact = PRO == kProRmsX || PRO == kProRmsResX;
  constexpr bool kRes = PRO == kProRmsRes || PRO == kProRmsResX;
  constexpr bool kRms = kExact || PRO == kProRms || PRO == kProRmsRes;
  constexpr bool kAttn = PRO == kProAttnStat;
  constexpr bool kPre = PRO == kProRmsPre, kEpi = PRO == kEpiResStat || kAttn;
  constexpr int kStatV = 2;  // row vectors per thread loaded ahead of the pass (general variants)
  __shared__ __align__(16) unsigned char xrec[NW][MR][RPW][32];
  __shared__ __align__(16) float4_t red[NW][MR][LN];
  __shared__ float stat[NW];
  const int rsh = RSH ? RSH : a.gsh_rows;  // log2(packed rows per group), >= 2
  const int lgsh = rsh - 2;    // log2(LG)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane % LN, lk = lane / LN;
  const int gi = lk >> lgsh, sub = lk & ((1 << lgsh) - 1);
  const int gpw = LKW >> lgsh;
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.qw);
  const int R = a.K >> 3, ng = R >> rsh;
  const TileWork tw = map_block<(LN == 4 ? 4 : 1)>(sp, ng);  // 16-column tiles: four per line
  const int tile = tw.tile, gb = tw.gb, ge = tw.ge;
  const bool whole = tw.whole;
  const int n0 = tile * CW;
  const int col = min(n0 + 4 * ln, a.N - 4);  // clamped: tail lanes load valid memory, store nothing
  // A split that fits one wave pass is reduced by wave 0 alone, with no LDS round and no barrier
  // (the other waves find no pass in the loop below and leave after it).
  const bool one_wave = !whole && ge - gb <= gpw;

  // ---- loads of one pass, in consumption order: x row(s), scale and zero words, weight rows
  struct Pass {
    u32x4 xr[XL], x2, x3;
    u32x2 sv, zv;
    u32x4 w[RPL];
    u32x4 ao[kAttn ? kAttnRanges : 1][2];  // kProAttnStat: the 8 dims' o of each range
    u32x2 am[kAttn ? kAttnRanges : 1];     // and its {m, l}
  };
  // kProAttnStat: the ranges live at the attention's position (its clamping of pos)
  int att_live = 1;
  if constexpr (kAttn) {
    const int64_t pin = *pa.att_pos;
    const int pos = pin >= 0 && pin < pa.att_len ? (int)pin : pin < 0 ? -1 : pa.att_len - 1;
    att_live = pos < 0 ? 1 : pos / pa.att_rlen + 1;
  }
  auto load_pass = [&](int gp, Pass& P) {
    const int xo = 8 * min((gp << rsh) + lane, R - 1);
    if constexpr (kAttn) {
      // packed row xo / 8 is dims 8 (row % 16) .. + 7 of head row / 16. All kAttnRanges ranges
      // are loaded (in bounds: the partials hold kAttnMaxSplits), so the loads do not wait for
      // pos; the ranges past the live ones are left out by selects when x is formed
      const int hrow = xo >> 3, h = hrow >> 4, d0 = (hrow & 15) * 8;
#pragma unroll
      for (int r = 0; r < kAttnRanges; ++r) {
        const float* o = pa.att_o + (h * ldk::kAttnMaxSplits + r) * ldk::kAttnHeadDim + d0;
        P.ao[r][0] = *reinterpret_cast<const u32x4*>(o);
        P.ao[r][1] = *reinterpret_cast<const u32x4*>(o + 4);
        P.am[r] = *reinterpret_cast<const u32x2*>(pa.att_ml + (h * ldk::kAttnMaxSplits + r) * 2);
      }
    } else if constexpr (MR == 1) {
      P.xr[0] = *reinterpret_cast<const u32x4*>(a.x + xo);
    } else {
#pragma unroll
      for (int i = 0; i < XL; ++i) {  // rows past M repeat the last row; their outputs are not stored
        const int r = lane + 64 * i, m = min(r / RPW, a.M - 1);
        P.xr[i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.ldx + 8 * min((gp << rsh) + r % RPW, R - 1));
      }
    }
    if constexpr (kRes) P.x2 = *reinterpret_cast<const u32x4*>(pa.res + xo);
    if constexpr (PRO == kProSwiglu) P.x2 = *reinterpret_cast<const u32x4*>(a.x + a.K + xo);
    if constexpr (kRms || kPre) P.x3 = *reinterpret_cast<const u32x4*>(pa.nw + xo);
    const int g = min(gp + gi, ge - 1);  // clamped; such lanes are masked out below
    P.sv = *reinterpret_cast<const u32x2*>(a.s + (int64_t)g * a.N + col);
    P.zv = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + col);
#pragma unroll
    for (int t = 0; t < RPL; ++t) {
      const int r = (g << rsh) + sub + (t << lgsh);
      P.w[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw + (int64_t)r * a.N + col));
    }
  };
  // The general RMSNorm variants wait for the row statistic's loads before their barrier. They
  // issue their first pass with buffer loads from every wave, with an out-of-range offset where
  // the wave has no pass (zeros, no request): the load count is then the same on every path, so
  // that wait covers the statistic's loads only.
  auto load_pass_buf = [&](int gp, bool live, Pass& P) {
    constexpr uint32_t kOut = 0x80000000u;  // past every resource below (each < 2 GiB)
    const auto xb = ldk::buffer_rsrc(a.x, (uint32_t)a.K * 2u);
    const auto rb = ldk::buffer_rsrc(pa.res, kRes ? (uint32_t)a.K * 2u : 0u);
    const auto nb = ldk::buffer_rsrc(pa.nw, (uint32_t)a.K * 2u);
    const auto sb = ldk::buffer_rsrc(a.s, (uint32_t)ng * (uint32_t)a.N * 2u);
    const auto zb = ldk::buffer_rsrc(a.z, (uint32_t)ng * (uint32_t)a.N * 2u);
    const auto wb = ldk::buffer_rsrc(a.qw, (uint32_t)R * (uint32_t)a.N * 4u);
    // a dead wave ORs kOut into every offset (a VALU op; a select on the uniform flag would
    // become a branch around the loads)
    const uint32_t dead = ldk::vgpr_const<0>() | (live ? 0u : kOut);
    const uint32_t xo = (16u * (uint32_t)min((gp << rsh) + lane, R - 1)) | dead;
    P.xr[0] = ldk::buffer_load16(xb, xo);
    if constexpr (kRes) P.x2 = ldk::buffer_load16(rb, xo);
    P.x3 = ldk::buffer_load16(nb, xo);
    const int g = min(gp + gi, ge - 1);
    const uint32_t so = (2u * (uint32_t)(g * a.N + col)) | dead;
    P.sv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sb, so, 0, 0));
    P.zv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(zb, so, 0, 0));
#pragma unroll
    for (int t = 0; t < RPL; ++t) {
      const int r = (g << rsh) + sub + (t << lgsh);
      const uint32_t wo = (4u * (uint32_t)(r * a.N + col)) | dead;
      P.w[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wb, wo, 0, 2));  // nt
    }
  };

  // ---- general RMSNorm variants: row vectors tid, tid + NT, ... for the statistic, first
  u32x4 sx[kStatV], sr[kStatV];
  if constexpr (kRms && !kExact) {
    const auto xb = ldk::buffer_rsrc(a.x, (uint32_t)a.K * 2u);
    const auto rb = ldk::buffer_rsrc(pa.res, kRes ? (uint32_t)a.K * 2u : 0u);
#pragma unroll
    for (int i = 0; i < kStatV; ++i) {
      const uint32_t off = 16u * (threadIdx.x + i * NW * 64);
      sx[i] = ldk::buffer_load16(xb, off);
      if constexpr (kRes) sr[i] = ldk::buffer_load16(rb, off);
    }
  }
  // ---- kProRmsPre: the per-tile partial sums of squares, ahead of the pass (zeros past nstats)
  float pst[kMaxRowStats / 64];
  if constexpr (kPre) {
    const auto sb = ldk::buffer_rsrc(pa.stats, (uint32_t)pa.nstats * 4u);
#pragma unroll
    for (int i = 0; i < kMaxRowStats / 64; ++i)
      pst[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sb, 4u * (uint32_t)(lane + 64 * i), 0, 0));
  }
  int gp = gb + wave * gpw;
  Pass P;
  if constexpr (kExact) {
    load_pass(gp, P);  // every wave has exactly one pass
  } else if constexpr (kRms || kPre) {  // branch free: the statistic's wait covers its loads only
    load_pass_buf(gp, gp < ge, P);
  } else {
    if (gp < ge) load_pass(gp, P);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load of the pass is in flight before the first wait

  float rs = 0.0f;
  if constexpr (kPre) {  // same lanes, same order in every wave and workgroup
    float ss = pst[0];
#pragma unroll
    for (int i = 1; i < kMaxRowStats / 64; ++i) ss += pst[i];
    ss = ldk::sum_lanes_strided<1>(ss);
    rs = 1.0f / __builtin_sqrtf(ss / (float)a.K + pa.eps);
  }
  if constexpr (kRms) {
    float ss = 0.0f;
    const bool wr = kRes && blockIdx.x == 0;
    if constexpr (kExact) {  // this wave's pass rows, lanes < RPW
      if (lane < RPW) {
        half8_t h = __builtin_bit_cast(half8_t, P.xr[0]);
        if constexpr (kRes) h = h + __builtin_bit_cast(half8_t, P.x2);
        if (wr) *reinterpret_cast<half8_t*>(pa.res_out + 8 * ((gp << rsh) + lane)) = h;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __builtin_fmaf((float)h[j], (float)h[j], ss);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kStatV; ++i) {  // lanes past the row hold zeros
        half8_t h = __builtin_bit_cast(half8_t, sx[i]);
        if constexpr (kRes) h = h + __builtin_bit_cast(half8_t, sr[i]);
        const int t = threadIdx.x + i * NW * 64;
        if (wr && t < R) *reinterpret_cast<half8_t*>(pa.res_out + 8 * t) = h;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __builtin_fmaf((float)h[j], (float)h[j], ss);
      }
      for (int t = threadIdx.x + kStatV * NW * 64; t < R; t += NW * 64) {  // rows beyond kStatV per thread
        half8_t h = *reinterpret_cast<const half8_t*>(a.x + 8 * t);
        if constexpr (kRes) h = h + *reinterpret_cast<const half8_t*>(pa.res + 8 * t);
        if (wr) *reinterpret_cast<half8_t*>(pa.res_out + 8 * t) = h;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __builtin_fmaf((float)h[j], (float)h[j], ss);
      }
    }
    ss = ldk::sum_lanes_strided<1>(ss);
    if (lane == 0) stat[wave] = ss;
    ldk::lds_barrier();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += stat[w];
    rs = 1.0f / __builtin_sqrtf(tot / (float)a.K + pa.eps);
  }

  const uint32_t magic = ldk::vgpr_const<kMagic>();  // v_and_or_b32 operands (see sgpr_const)
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>(), mhi = ldk::sgpr_const<0x00F000F0u>();
  float acc[MR][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[m][q] = 0.0f;
  for (bool first = true; gp < ge; gp += NW * gpw, first = false) {
    if (!first) {
      if constexpr ((kRms && !kExact) || kPre) load_pass_buf(gp, true, P);
      else load_pass(gp, P);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MR == 1) {
      if constexpr (kAttn) {
        if (lane < RPW) {
          float M = -__builtin_inff();
#pragma unroll
          for (int r = 0; r < kAttnRanges; ++r) M = fmaxf(M, r < att_live ? ldk::u2f(P.am[r][0]) : -__builtin_inff());
          // the ranges past the live ones hold an earlier call's values (any bits): selects, not
          // products with a zero weight, leave them out
          float f[kAttnRanges], l = 0.0f;
#pragma unroll
          for (int r = 0; r < kAttnRanges; ++r) {
            f[r] = __expf(ldk::u2f(P.am[r][0]) - M);
            const float lr = __builtin_fmaf(ldk::u2f(P.am[r][1]), f[r], l);
            l = r < att_live ? lr : l;
          }
          // one division for the 8 dims (o * (1 / l) can differ from o / l in the last fp32 bit)
          const float inv = l > 0.0f ? 1.0f / l : 0.0f;
          half8_t xh;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float o = 0.0f;
#pragma unroll
            for (int r = 0; r < kAttnRanges; ++r) {
              const float orr = __builtin_fmaf(ldk::u2f(P.ao[r][j >> 2][j & 3]), f[r], o);
              o = r < att_live ? orr : o;
            }
            xh[j] = (half_t)(l > 0.0f ? o * inv : 0.0f);  // no live position: 0 (o may be NaN)
          }
          store_fact_record(&xrec[wave][0][lane][0], __builtin_bit_cast(u32x4, xh));
        }
      } else {
        if (lane < RPW) store_fact_record(&xrec[wave][0][lane][0], pro_stage<PRO>(P.xr[0], P.x2, P.x3, rs));
      }
    } else {
#pragma unroll
      for (int i = 0; i < XL; ++i) {
        const int r = lane + 64 * i;
        if (r < XREC) store_fact_record(&xrec[wave][r / RPW][r % RPW][0], P.xr[i]);
      }
    }
    ldk::wave_lds_sync();
    // one row: every record read up front; more rows: a packed row's records when it is used
    // (registers: the kernel is held to 72 VGPRs)
    u32x4 xp[MR][RPL];
    float c0[MR], xs[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      c0[m] = 0.0f;
      xs[m] = 0.0f;
#pragma unroll
      for (int t = 0; t < RPL; ++t) {
        const int rr = (gi << rsh) + sub + (t << lgsh);
        if constexpr (MR == 1) xp[m][t] = *reinterpret_cast<const u32x4*>(&xrec[wave][m][rr][0]);
        const float2_t k = *reinterpret_cast<const float2_t*>(&xrec[wave][m][rr][16]);
        c0[m] += k[0];
        xs[m] += k[1];
      }
    }
    float tt[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) tt[m][q] = c0[m];
#pragma unroll
    for (int t = 0; t < RPL; ++t) {  // rows in arrival order
      if constexpr (MR > 1) {
        const int rr = (gi << rsh) + sub + (t << lgsh);
#pragma unroll
        for (int m = 0; m < MR; ++m) xp[m][t] = *reinterpret_cast<const u32x4*>(&xrec[wave][m][rr][0]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // the decoded nibble pairs are common to all rows
        const uint32_t wc = P.w[t][q], v = wc >> 8;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          tt[m][q] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][t][3]), ldk::u2h2((v & mhi) | magic), tt[m][q], false);
          tt[m][q] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][t][2]), ldk::u2h2((v & mlo) | magic), tt[m][q], false);
          tt[m][q] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][t][1]), ldk::u2h2((wc & mhi) | magic), tt[m][q], false);
          tt[m][q] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][t][0]), ldk::u2h2((wc & mlo) | magic), tt[m][q], false);
        }
      }
    }
    const bool gok = gp + gi < ge;
    const half4_t s4 = __builtin_bit_cast(half4_t, P.sv), z4 = __builtin_bit_cast(half4_t, P.zv);
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // s * (sum x*q - z * sum x)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float v = (float)s4[q] * __builtin_fmaf(-(float)z4[q], xs[m], tt[m][q]);
        acc[m][q] += gok ? v : 0.0f;
      }
    }
    ldk::wave_lds_sync();  // the next pass rewrites this wave's records
  }

  // ---- reduction: lanes sharing ln within the wave, then the NW waves through LDS
  if constexpr (MR == 1) {
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[0][q] = ldk::sum_lanes_strided<LN>(acc[0][q]);
    if (one_wave) {
      if (wave != 0) return;
      // lane l < CW owns output n0 + l: element l % 4 of the lanes holding columns 4(l/4)..
      const int src = (lane >> 2) % LN, e = lane & 3;
      const float e0 = __shfl(acc[0][0], src), e1 = __shfl(acc[0][1], src);
      const float e2 = __shfl(acc[0][2], src), e3 = __shfl(acc[0][3], src);
      const float v = e == 0 ? e0 : e == 1 ? e1 : e == 2 ? e2 : e3;
      const int c = n0 + lane;
      float tot;
      if (lane < CW && c < a.N && ldk::splitk_add(split_ctx(sp, tw), sp.acc + (size_t)(tile - sp.full) * CW + lane, v, &tot)) {
        if (a.bias) tot += (float)a.bias[c];
        a.out[c] = (half_t)tot;
      }
      return;
    }
    if (lane < LN) red[wave][0][lane] = float4_t{acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
    __syncthreads();
    if (wave != 0) return;
    if (whole || sp.splits == 1) {
      const int c = n0 + 4 * lane;
      if constexpr (kEpi) {  // h = fp16(y + residual) stored, the tile's sum of h^2 published
        float ps = 0.0f;
        if (lane < LN && c < a.N) {
          float4_t v = red[0][0][lane];
#pragma unroll
          for (int i = 1; i < NW; ++i) v += red[i][0][lane];
          if (a.bias) v += float4_t{(float)a.bias[c], (float)a.bias[c + 1], (float)a.bias[c + 2], (float)a.bias[c + 3]};
          const half4_t y{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
          const half4_t h = y + *reinterpret_cast<const half4_t*>(pa.res + c);  // fp16 add
          *reinterpret_cast<half4_t*>(a.out + c) = h;
#pragma unroll
          for (int q = 0; q < 4; ++q) ps = __builtin_fmaf((float)h[q], (float)h[q], ps);
        }
        ps = ldk::sum_lanes_strided<1>(ps);
        if (lane == 0) pa.stats[tile] = ps;
        return;
      }
      if (lane >= LN || c >= a.N) return;
      float4_t v = red[0][0][lane];
#pragma unroll
      for (int i = 1; i < NW; ++i) v += red[i][0][lane];
      if (a.bias) v += float4_t{(float)a.bias[c], (float)a.bias[c + 1], (float)a.bias[c + 2], (float)a.bias[c + 3]};
      const half4_t o{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      if (out_vec) {
        *reinterpret_cast<half4_t*>(a.out + c) = o;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) a.out[c + q] = o[q];
      }
    } else {
      // one output per lane, so the CW returning atomics of the tile are in flight together
      const int c = n0 + lane;
      if (lane >= CW || c >= a.N) return;
      const float* rf = reinterpret_cast<const float*>(&red[0][0][0]);
      float v = rf[lane];
#pragma unroll
      for (int i = 1; i < NW; ++i) v += rf[i * CW + lane];
      float tot;
      if (ldk::splitk_add(split_ctx(sp, tw), sp.acc + (size_t)(tile - sp.full) * CW + lane, v, &tot)) {
        if (a.bias) tot += (float)a.bias[c];
        a.out[c] = (half_t)tot;
      }
    }
    return;
  }
  // ---- several rows: the split-K words of a split tile are [MR][CW] (row m, column n0 + l)
  const int mrows = min(MR, a.M);
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[m][q] = ldk::sum_lanes_strided<LN>(acc[m][q]);
  uint64_t* const words = whole ? nullptr : sp.acc + (size_t)(tile - sp.full) * MR * CW;
  if (one_wave) {
    if (wave != 0) return;
    // lane l < CW owns output n0 + l: element l % 4 of the lanes holding columns 4(l/4)..
    const int src = (lane >> 2) % LN, e = lane & 3;
    const int c = n0 + lane;
    uint64_t inc[MR], old[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float e0 = __shfl(acc[m][0], src), e1 = __shfl(acc[m][1], src);
      const float e2 = __shfl(acc[m][2], src), e3 = __shfl(acc[m][3], src);
      inc[m] = 0;
      if (lane < CW && c < a.N && m < mrows)
        inc[m] = ldk::splitk_inc(split_ctx(sp, tw), words + m * CW + lane, e == 0 ? e0 : e == 1 ? e1 : e == 2 ? e2 : e3);
    }
    if (lane >= CW || c >= a.N) return;
#pragma unroll
    for (int m = 0; m < MR; ++m)  // every add in flight before the first result is used
      if (m < mrows) old[m] = ldk::splitk_issue(words + m * CW + lane, inc[m]);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float tot;
      if (m < mrows && ldk::splitk_finish(split_ctx(sp, tw), words + m * CW + lane, old[m], inc[m], &tot)) {
        if (a.bias) tot += (float)a.bias[c];
        a.out[(int64_t)m * a.ldo + c] = (half_t)tot;
      }
    }
    return;
  }
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave][m][lane] = float4_t{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
  }
  __syncthreads();
  if (wave != 0) return;
  if (whole || sp.splits == 1) {
    // lane l: row l / LN, columns n0 + 4 (l % LN) .. +3
#pragma unroll
    for (int l0 = 0; l0 < MR * LN; l0 += 64) {
      const int l = l0 + lane, m = l / LN, j = l % LN;
      const int c = n0 + 4 * j;
      if (l >= MR * LN || m >= mrows || c >= a.N) continue;
      float4_t v = red[0][m][j];
#pragma unroll
      for (int i = 1; i < NW; ++i) v += red[i][m][j];
      if (a.bias) v += float4_t{(float)a.bias[c], (float)a.bias[c + 1], (float)a.bias[c + 2], (float)a.bias[c + 3]};
      const half4_t o{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      half_t* dst = a.out + (int64_t)m * a.ldo + c;
      if (out_vec) {
        *reinterpret_cast<half4_t*>(dst) = o;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[q] = o[q];
      }
    }
  } else {
    // one output per lane and row, so the CW returning atomics of a row are in flight together
    const int c = n0 + lane;
    if (lane >= CW || c >= a.N) return;
    uint64_t inc[MR], old[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = reinterpret_cast<const float*>(&red[0][m][0])[lane];
#pragma unroll
      for (int i = 1; i < NW; ++i) v += reinterpret_cast<const float*>(&red[i][m][0])[lane];
      inc[m] = m < mrows ? ldk::splitk_inc(split_ctx(sp, tw), words + m * CW + lane, v) : 0;
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < mrows) old[m] = ldk::splitk_issue(words + m * CW + lane, inc[m]);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float tot;
      if (m < mrows && ldk::splitk_finish(split_ctx(sp, tw), words + m * CW + lane, old[m], inc[m], &tot)) {
        if (a.bias) tot += (float)a.bias[c];
        a.out[(int64_t)m * a.ldo + c] = (half_t)tot;
      }
    }
  }
}

// --------------------------------------------------------------------- VALU kernel (EXACT)
//
// Lane (ln, lkw) of a wave: ln < LN runs along N (columns n0 + 4ln .. +3), lkw < LKW = 64/LN along
// K. LG = rows_per_group / RPL lanes share a group, each taking RPL of its packed rows
// (sub, sub + LG, ...); a chunk is GW = LKW / LG groups (LKW*RPL packed rows). Chunk k of the
// workgroup's range covers groups gb + k*GW ..; wave w takes chunks w, w + NW, ... in rounds of
// CPW chunks.
template <int MT, int LN, int RPL, int CPW>
__global__ __launch_bounds__(1024) void w4a16_gemv_kernel(W4Args a, SplitArgs sp) {
  constexpr int CW = 4 * LN;
  constexpr int LKW = 64 / LN;
  constexpr int ROWB = 16;
  constexpr int RPC = LKW * RPL;                // packed rows per chunk
  constexpr int ITEMS = CPW * RPC * MT;         // x records a wave stages per round
  constexpr int PXW = (ITEMS + 63) / 64;        // ... per lane
  constexpr int SLOTS = 64 * PXW;
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
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.qw);
  const TileWork tw = map_block(sp, ng);
  const int n0 = tw.tile * CW;
  const int col = min(n0 + 4 * ln, a.N - 4);  // clamped: tail lanes load valid memory, store nothing
  const int gb = tw.gb, ge = tw.ge;
  const int rb = gb << a.gsh_rows, re = ge << a.gsh_rows;  // packed rows of this workgroup
  const int nchunks = (ge - gb + GW - 1) / GW;
  unsigned char* xw = smem + (size_t)wave * SLOTS * ROWB;
  float* red = reinterpret_cast<float*>(smem + (size_t)NW * SLOTS * ROWB);  // [NW][MT*CW]

  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>();
  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  for (int k0 = wave; k0 < nchunks; k0 += NW * CPW) {
    // ---- loads, in consumption order: x rows of the round's chunks, then per chunk the scale
    // and zero words and the weight rows
    u32x4 xr[PXW];
#pragma unroll
    for (int i = 0; i < PXW; ++i) {
      const int item = min(lane + 64 * i, ITEMS - 1);  // item = (c * RPC + rr) * MT + m
      const int m = min(item % MT, a.M - 1), rc = item / MT;
      const int c = rc / RPC, rr = rc - c * RPC;
      const int row = min(rb + (k0 + NW * c) * GW * rpg + rr, R - 1);
      xr[i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.ldx + 8 * row);
    }
    u32x4 w[CPW][RPL];
    u32x2 sv[CPW], zv[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int gg = min(gb + (k0 + NW * c) * GW + gi, ge - 1);  // clamped; such lanes meet zero x
      sv[c] = *reinterpret_cast<const u32x2*>(a.s + (int64_t)gg * a.N + col);
      zv[c] = *reinterpret_cast<const u32x2*>(a.z + (int64_t)gg * a.N + col);
#pragma unroll
      for (int t = 0; t < RPL; ++t) {
        const int r = gg * rpg + sub + LG * t;
        w[c][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.qw + (int64_t)r * a.N + col));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the round is in flight before the first wait

    // ---- wave-local x staging: every lane writes its own slots (no branches, no conflicts).
    // Rows outside the workgroup's groups and x rows >= M are staged as zeros.
#pragma unroll
    for (int i = 0; i < PXW; ++i) {
      const int item = lane + 64 * i;
      const int m = item % MT, rc = item / MT;
      const int c = rc / RPC, rr = rc - c * RPC;
      const int row = rb + (k0 + NW * c) * GW * rpg + rr;
      const bool ok = item < ITEMS && m < a.M && row < re;
      *reinterpret_cast<u32x4*>(xw + (size_t)item * ROWB) = x_pairs(ok ? xr[i] : u32x4{0u, 0u, 0u, 0u});
    }
    ldk::wave_lds_sync();

#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      if (k0 + NW * c >= nchunks) break;  // uniform: the rest of the round is past the range
      const unsigned char* xc = xw + (size_t)(c * RPC + gi * rpg + sub) * MT * ROWB;
      const half4_t s4 = __builtin_bit_cast(half4_t, sv[c]);
      const half4_t z4 = __builtin_bit_cast(half4_t, zv[c]);
#pragma unroll
      for (int t = 0; t < RPL; ++t) {
        u32x4 xp[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
          xp[m] = *reinterpret_cast<const u32x4*>(xc + (size_t)(LG * t * MT + m) * ROWB);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t wc = w[c][t][q];
          const half_t zb1 = -((half_t)1024.0f + z4[q]);
          const half2_t zb = {zb1, zb1};
          const half2_t s2 = {s4[q], s4[q]};
          const half2_t d0 = (ldk::u2h2((wc & mlo) | magic) + zb) * s2;
          const half2_t d1 = (ldk::u2h2(((wc >> 4) & mlo) | magic) + zb) * s2;
          const half2_t d2 = (ldk::u2h2(((wc >> 8) & mlo) | magic) + zb) * s2;
          const half2_t d3 = (ldk::u2h2(((wc >> 12) & mlo) | magic) + zb) * s2;
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            float tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][0]), d0, acc[m][q], false);
            tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][1]), d1, tt, false);
            tt = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][2]), d2, tt, false);
            acc[m][q] = __builtin_amdgcn_fdot2(ldk::u2h2(xp[m][3]), d3, tt, false);
          }
        }
      }
    }
    ldk::wave_lds_sync();  // the next round rewrites this wave's records
  }

  // ---- reduction: lanes of a wave sharing ln, then the waves through LDS
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[m][q] = ldk::sum_lanes_strided<LN>(acc[m][q]);
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
      *reinterpret_cast<float4_t*>(red + (size_t)(wave * MT + m) * CW + 4 * lane) =
          float4_t{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
  }
  __syncthreads();
  finish_tile(red, MT * CW, NW, tw, sp, sp.acc + (size_t)(tw.tile - sp.full) * MT * CW, [&](int o, float v) {
    const int m = o / CW, n = n0 + (o - m * CW);
    if (m < a.M && n < a.N) {
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)m * a.ldo + n] = (half_t)v;
    }
  });
}

// ------------------------------------------------------------------------------ MFMA kernel
//
// Rows in blocks of 16 * MT on v_mfma_f32_16x16x32_f16, one block per grid row: MT = 1 for decode
// (padded to 16) and for prefill rows whose 16-row blocks fit in 256 workgroups (up to 16 waves
// each); MT = 2 otherwise, the decoded weights of a K step serving both 16-row tiles. The other
// blocks re-read the weights from the MALL. A workgroup owns CW = 64 * NH output
// columns (NH 128-byte line halves of the packed rows: 128 columns on wide shapes, 140 workgroups
// for gate_up, one per CU, instead of 280 that put two 64-column tiles on 24 CUs) and a range of
// quantization groups; its waves (up to 16 at 64 columns, 8 at 128) take groups round-robin, CPW
// groups per pass with every load of the pass in flight.
//
// Lane l = (c16 = l % 16, kb = l / 16). For 32-row K step ks of group g it loads packed row
// g*rpg + 4*ks + kb at columns n0 + 64h + 4*c16 .. +3 (one 16-byte load per half h): each of the 4
// words is exactly one lane's B operand (8 consecutive K of one column), so word j feeds MFMA
// tile (h, j), whose column c16 is the real column n0 + 64h + 4*c16 + j. The A operand is x row
// c16 in the matching nibble-pair order (x_pairs), zeros past M.
//
// FACTORED on the matrix cores: B is the magic-decoded 1024 + q (one v_and_or_b32 per pair, no
// subtraction), and one more MFMA per K step against an all-ones B gives sum(x) of each output
// row in the same fragment layout. A group then adds s * (sum x*(1024+q) - (1024+z) * sum x) =
// s * sum x*(q - z) to the fp32 accumulator: 4 VALU ops per 8 weights plus a per-group epilogue,
// against 12 for dequantizing every weight to fp16 first.
// NWD: packed words per lane and load, 4 (16-byte loads, 64-column halves) or 2 (8-byte loads,
// 32-column tiles: the M = 1 kernel's 128-byte tile, whose grid fills every CU on wide shapes).
template <int NH, int KS, int CPW, int MT, int NWD>  // KS: 32-wide K steps per group; MT: 16-row tiles
__global__ __launch_bounds__(NH == 1 && MT == 1 ? 1024 : 512) void w4a16_mfma_kernel(W4Args a, SplitArgs sp) {
  static_assert(NWD == 2 || NWD == 4, "4 or 2 words per lane");
  constexpr int HW = 16 * NWD;                 // columns of one load across the 16 column lanes
  constexpr int CW = HW * NH, NT = NWD * NH;   // columns, 16-column MFMA tiles
  typedef _Float16 half8v __attribute__((ext_vector_type(8)));
  extern __shared__ __align__(16) unsigned char smem[];
  const int rpg = 4 * KS;
  const int NW = blockDim.x >> 6;
  const int R = a.K >> 3;
  const int ng = R >> a.gsh_rows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, kb = lane >> 4;
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.qw);
  const TileWork tw = map_block(sp, ng);
  const int n0 = tw.tile * CW;
  const int m0 = blockIdx.y * 16 * MT;  // first row of this workgroup's row block
  int col[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) col[h] = min(n0 + HW * h + NWD * c16, a.N - NWD);  // clamped: tail lanes store nothing
  const int gb = tw.gb, ge = tw.ge;
  int xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    xrow[t] = min(m0 + 16 * t + c16, a.M - 1);
    xok[t] = m0 + 16 * t + c16 < a.M;
  }
  const int mrows = min(a.M - m0, 16 * MT);
  float* red = reinterpret_cast<float*>(smem);  // [NW][mrows][CW]
  // A rows past M are buffer loads past the end of the resource: zeros, and no memory request,
  // so a decode block of M < 16 rows moves only its M rows of x
  // (the resource spans this block's rows; the launcher keeps it below 2 GiB)
  const auto xb = ldk::buffer_rsrc(a.x + (int64_t)m0 * a.ldx, (uint32_t)((int64_t)(mrows - 1) * a.ldx * 2 + a.K * 2));
  uint32_t xoff[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xoff[t] = xok[t] ? (uint32_t)((int64_t)(xrow[t] - m0) * a.ldx * 2) : 0x80000000u;

  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>();
  const half8v ones = {(half_t)1.0f, (half_t)1.0f, (half_t)1.0f, (half_t)1.0f,
                       (half_t)1.0f, (half_t)1.0f, (half_t)1.0f, (half_t)1.0f};
  float4_t acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[t][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int g0 = gb + wave; g0 < ge; g0 += NW * CPW) {
    // loads in consumption order, group by group: per K step the A fragments and the weight
    // words of each half, then the zero points and scales (used after the group's MFMAs)
    u32x2 zv[CPW][NH], sv[CPW][NH];
    u32x4 ar[CPW][KS][MT], w[CPW][KS][NH];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int g = min(g0 + NW * c, ge - 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int r = g * rpg + 4 * ks + kb;
#pragma unroll
        for (int t = 0; t < MT; ++t) ar[c][ks][t] = ldk::buffer_load16(xb, xoff[t] + 16u * (uint32_t)r);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const uint32_t* wp = a.qw + (int64_t)r * a.N + col[h];
          if constexpr (NWD == 4) {
            w[c][ks][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp));
          } else {
            const u32x2 w2 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wp));
            w[c][ks][h] = u32x4{w2[0], w2[1], 0u, 0u};
          }
        }
      }
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        if constexpr (NWD == 4) {
          zv[c][h] = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + col[h]);
          sv[c][h] = *reinterpret_cast<const u32x2*>(a.s + (int64_t)g * a.N + col[h]);
        } else {
          zv[c][h] = u32x2{*reinterpret_cast<const uint32_t*>(a.z + (int64_t)g * a.N + col[h]), 0u};
          sv[c][h] = u32x2{*reinterpret_cast<const uint32_t*>(a.s + (int64_t)g * a.N + col[h]), 0u};
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the pass is in flight before the first wait
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      if (g0 + NW * c >= ge) break;  // uniform
      float4_t tmp[MT][NT], sx[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        sx[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < NT; ++j) tmp[t][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u32x4 bq[NT];  // decoded once, used by every row tile
#pragma unroll
        for (int h = 0; h < NH; ++h) {
#pragma unroll
          for (int j = 0; j < NWD; ++j) {
            const uint32_t wc = w[c][ks][h][j];
            bq[NWD * h + j][0] = (wc & mlo) | magic;          // 1024 + (q0, q4)
            bq[NWD * h + j][1] = ((wc >> 4) & mlo) | magic;   // 1024 + (q1, q5)
            bq[NWD * h + j][2] = ((wc >> 8) & mlo) | magic;   // 1024 + (q2, q6)
            bq[NWD * h + j][3] = ((wc >> 12) & mlo) | magic;  // 1024 + (q3, q7)
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const u32x4 ap = x_pairs(ar[c][ks][t]);  // zeros past M
          const half8v A = __builtin_bit_cast(half8v, ap);
#pragma unroll
          for (int j = 0; j < NT; ++j)
            tmp[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(half8v, bq[j]), tmp[t][j], 0, 0, 0);
          sx[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, ones, sx[t], 0, 0, 0);
        }
      }
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const half4_t z4 = __builtin_bit_cast(half4_t, zv[c][h]), s4 = __builtin_bit_cast(half4_t, sv[c][h]);
#pragma unroll
        for (int j = 0; j < NWD; ++j) {
          const float zz = 1024.0f + (float)z4[j], sj = (float)s4[j];
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[t][NWD * h + j][i] =
                  __builtin_fmaf(sj, __builtin_fmaf(-zz, sx[t][i], tmp[t][NWD * h + j][i]), acc[t][NWD * h + j][i]);
        }
      }
    }
  }

  // tile (t, h, j), element i of lane l: row 16t + 4*kb + i of the block, column HW*h + NWD*c16 + j
  // of the workgroup's CW. Rows past M are all zero and not stored; each lane writes NWD
  // consecutive columns per half.
  const int n = mrows * CW;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * t + 4 * kb + i;
      if (row < mrows) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          float* dst = red + (size_t)wave * n + row * CW + HW * h + NWD * c16;
          if constexpr (NWD == 4)
            *reinterpret_cast<float4_t*>(dst) =
                float4_t{acc[t][4 * h][i], acc[t][4 * h + 1][i], acc[t][4 * h + 2][i], acc[t][4 * h + 3][i]};
          else
            *reinterpret_cast<float2_t*>(dst) = float2_t{acc[t][2 * h][i], acc[t][2 * h + 1][i]};
        }
      }
    }
  }
  __syncthreads();
  // split words: [row block][split tile][outputs of the block], the block's stride its full rows
  // (M rows when a single block of M <= 16 rows)
  const int wstride = a.M <= 16 ? n : 16 * MT * CW;
  const int stiles = (a.N + CW - 1) / CW - sp.full;
  uint64_t* const words = sp.acc + ((size_t)blockIdx.y * stiles + (tw.tile - sp.full)) * wstride;
  finish_tile(red, n, NW, tw, sp, words, [&](int o, float v) {
    const int m = o / CW, nn = n0 + (o - m * CW);
    if (nn < a.N) {
      if (a.bias) v += (float)a.bias[nn];
      a.out[(int64_t)(m0 + m) * a.ldo + nn] = (half_t)v;
    }
  });
}

// ----------------------------------------------- MFMA kernel with x staged in LDS (decode rows)
//
// Decode rows (3 .. 16) with group size 128 and K <= 1536 (12 groups): one workgroup per 32-column
// tile over all of K (gate_up: 560 workgroups, the M = 1 kernel's grid; k/v: 8), NW waves of GPW
// groups each, no split-K and no atomics. Longer K (down: 70 groups) stays on the wide-tile kernel:
// split over workgroups into ranges of 12 groups this kernel measured slower there (M = 4 / 8 / 16:
// 5.5 / 6.1 / 7.1 against 5.2 / 5.5 / 6.9 us).
//
// The x operand is what limits the wide-tile MFMA kernel at these rows: its A fragments (16 rows x
// 64 bytes per load) are re-read by every workgroup straight from L2. Here each wave first loads
// the x rows of its own groups with coalesced 16-byte loads (16 lanes = 256 contiguous bytes of one
// row), issued before its weight loads, turns them into A records in LDS and reads its A fragments
// back with ds_read_b128 (no workgroup barrier: a wave only reads the records it wrote):
//  - record of (packed row r, row m) = the A fragment of lane (c16 = m, kb = r % 4): pairs
//    (x0,x4) (x1/16,x5/16) (x2,x6) (x3/16,x7/16), stored at [r][m ^ (r % MP)] so that the 16
//    lanes writing one row's 16 packed rows and the 16 lanes reading one packed row's 16 rows hit
//    distinct LDS banks;
//  - per (group, row) the offset c = 1024 * sum(A) (the magic 1024 of every decoded weight times
//    the staged x) and sum(x), for the epilogue s * (sum x*(1024+q) - c - z * sum x) =
//    s * sum x*(q - z), come from one more MFMA per K step against a constant B whose columns
//    0-7 pick the even pairs and 8-15 the odd (x/16) pairs: E = sum of the even x, O = sum of the
//    odd x / 16, c = 1024 (E + O), sum x = E + 16 O (a DPP rotation by 8 lanes brings the two
//    halves together). Summing them in the staging lanes instead (DPP row reductions of two
//    values per record) cost 0.35 us at 16 rows on gate_up.
// B is one v_and_or_b32 per pair (odd nibbles in place as 16q, met by x/16): 5 VALU ops per 8
// weights and no all-ones MFMA for sum(x). A lane loads CPL = 2 words (two columns) per packed
// row, the M = 1 kernel's 128-byte tile, or 4 (64-column tiles, two lines per packed row, for the
// wide shapes at 5-16 rows, where the x rows every workgroup stages cost more than the weights);
// X5 adds a fifth 16-column tile to the four-word lanes (one more word per packed row, column
// 64 + c16: 80-column tiles, for shapes whose 64-column tiles would need more than 256
// workgroups); the waves' partial tiles meet in LDS at the end.
// Measured on MI355X (graph replays, rotating sets), wide-tile kernel against this one: gate_up
// M = 4 / 8 / 16 7.50 / 8.07 / 9.37 -> 5.91 / 6.68 / 7.48 us, q/o 4.26 / 4.40 / 5.12 -> 3.48 /
// 3.69 / 3.99, k/v (8 tiles) 4.12 / 4.29 / 5.00 -> 3.33 / 3.49 / 3.85.
template <int MP, int NW, int GPW, int CPL, bool X5>
__global__ __launch_bounds__(NW * 64) void w4a16_mfma_x_kernel(W4Args a) {
  static_assert(MP == 4 || MP == 8 || MP == 16, "row tile");
  static_assert(CPL == 2 || CPL == 4, "two or four columns per lane");
  static_assert(!X5 || CPL == 4, "the fifth 16-column tile follows four columns per lane");
  constexpr int NG = NW * GPW, WUNITS = GPW * MP * 16, WUPT = WUNITS / 64;
  constexpr int CWT = 16 * CPL + (X5 ? 16 : 0);  // columns of the tile
  static_assert(WUNITS % 64 == 0, "whole staging units per lane");
  constexpr int NREC = NG * 16 * MP, NRED = (NW * MP * CWT + 3) / 4;  // records, partial tiles (u32x4)
  typedef _Float16 half8v __attribute__((ext_vector_type(8)));
  typedef uint32_t wrow_t __attribute__((ext_vector_type(CPL)));      // CPL packed words of a row
  typedef uint32_t sz_t __attribute__((ext_vector_type(CPL / 2)));    // CPL fp16 scales or zeros
  __shared__ __align__(16) u32x4 xs[NREC > NRED ? NREC : NRED];  // A records; the waves' partial tiles at the end
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, kb = lane >> 4;
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.qw);
  const int ng = (a.K >> 3) >> 4;  // groups of 16 packed rows, <= NG
  // X5: an 80-column tile is 2.5 lines of each packed row, so tiles 2q and 2q + 1 share a line.
  // They run as workgroups L and L + 8 of a group of 16, which the dispatcher places on the same
  // XCD (workgroup L goes to XCD L % 8) at about the same time: the shared line comes into that
  // XCD's L2 once. Workgroups past the last whole group of 16 take their tiles in plain order.
  int tile = blockIdx.x;
  if constexpr (X5) {
    if (tile < (int)(gridDim.x & ~15u)) tile = (tile & ~15) + 2 * (tile & 7) + ((tile >> 3) & 1);
  }
  const int n0 = tile * CWT;
  const int col = min(n0 + CPL * c16, a.N - CPL);  // clamped: tail lanes load valid memory, store nothing
  const int col5 = min(n0 + 16 * CPL + c16, a.N - 1);  // X5: the fifth tile's column of the lane
  const int M = a.M;
  // ---- this wave's x rows first (unit u = lane + 64 i: packed row rr of group wave * GPW + u / (16 MP),
  //      row m)
  u32x4 xr[WUPT];
#pragma unroll
  for (int i = 0; i < WUPT; ++i) {
    const int u = lane + 64 * i, rr = u & 15, m = (u >> 4) % MP;
    const int g = min(wave * GPW + u / (16 * MP), ng - 1);
    xr[i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)min(m, M - 1) * a.ldx + 8 * (16 * g + rr));
  }
  // ---- then its weights: K step ks of group g is packed row 16 g + 4 ks + kb, columns col ..
  //      col + CPL - 1
  wrow_t w[GPW][4];
  sz_t sv[GPW], zv[GPW];
  uint32_t w5[X5 ? GPW : 1][4];  // X5: one word of the fifth tile per K step
  half_t s5[X5 ? GPW : 1], z5[X5 ? GPW : 1];
#pragma unroll
  for (int gi = 0; gi < GPW; ++gi) {
    const int g = min(wave * GPW + gi, ng - 1);  // clamped: surplus waves load valid memory, use nothing
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      w[gi][ks] = __builtin_nontemporal_load(
          reinterpret_cast<const wrow_t*>(a.qw + (int64_t)(16 * g + 4 * ks + kb) * a.N + col));
      if constexpr (X5) w5[gi][ks] = __builtin_nontemporal_load(a.qw + (int64_t)(16 * g + 4 * ks + kb) * a.N + col5);
    }
    sv[gi] = *reinterpret_cast<const sz_t*>(a.s + (int64_t)g * a.N + col);
    zv[gi] = *reinterpret_cast<const sz_t*>(a.z + (int64_t)g * a.N + col);
    if constexpr (X5) {
      s5[gi] = a.s[(int64_t)g * a.N + col5];
      z5[gi] = a.z[(int64_t)g * a.N + col5];
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first wait
  // ---- A records
  const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
#pragma unroll
  for (int i = 0; i < WUPT; ++i) {
    const int u = lane + 64 * i, rr = u & 15, m = (u >> 4) % MP, g = wave * GPW + u / (16 * MP);
    const u32x4 d = m < M ? xr[i] : u32x4{0u, 0u, 0u, 0u};  // rows past M stage zeros
    const half2_t b1 = ldk::u2h2(perm_hi(d[0], d[2])) * sixteenth, b3 = ldk::u2h2(perm_hi(d[1], d[3])) * sixteenth;
    if (g < ng)
      xs[(16 * g + rr) * MP + (m ^ (rr & (MP - 1)))] =
          u32x4{perm_lo(d[0], d[2]), ldk::h22u(b1), perm_lo(d[1], d[3]), ldk::h22u(b3)};
  }
  ldk::wave_lds_sync();
  // the stats MFMA's B: column c16 < 8 ones at the even pairs (1, 1, 0, 0, 1, 1, 0, 0), c16 >= 8
  // at the odd ones
  const uint32_t one2 = 0x3C003C00u, ev = c16 < 8 ? one2 : 0u, od = c16 < 8 ? 0u : one2;
  const half8v bstat = __builtin_bit_cast(half8v, u32x4{ev, od, ev, od});
  // ---- MFMA over the wave's groups: tile t holds columns n0 + CPL c16 + t
  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>(), mhi = ldk::sgpr_const<0x00F000F0u>();
  float4_t acc[CPL], acc5 = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < CPL; ++t) acc[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int gi = 0; gi < GPW; ++gi) {
    const int g = wave * GPW + gi;
    if (g >= ng) break;  // uniform
    float4_t tmp[CPL], tmp5 = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < CPL; ++t) tmp[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float4_t sacc = float4_t{0.0f, 0.0f, 0.0f, 0.0f};  // E (c16 < 8) or O (c16 >= 8) per row
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int r = 16 * g + 4 * ks + kb;  // packed row (r % MP = (4 ks + kb) % MP)
      u32x4 ar = u32x4{0u, 0u, 0u, 0u};
      if (c16 < MP) ar = xs[r * MP + (c16 ^ (r & (MP - 1)))];
      const half8v A = __builtin_bit_cast(half8v, ar);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bstat, sacc, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < CPL; ++t) {
        const uint32_t wc = w[gi][ks][t], v = wc >> 8;
        const u32x4 b{(wc & mlo) | magic, (wc & mhi) | magic, (v & mlo) | magic, (v & mhi) | magic};
        tmp[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(half8v, b), tmp[t], 0, 0, 0);
      }
      if constexpr (X5) {
        const uint32_t wc = w5[gi][ks], v = wc >> 8;
        const u32x4 b{(wc & mlo) | magic, (wc & mhi) | magic, (v & mlo) | magic, (v & mhi) | magic};
        tmp5 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(half8v, b), tmp5, 0, 0, 0);
      }
    }
    typedef _Float16 halfc_t __attribute__((ext_vector_type(CPL)));
    const halfc_t s2 = __builtin_bit_cast(halfc_t, sv[gi]), z2 = __builtin_bit_cast(halfc_t, zv[gi]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // element i of lane (c16, kb): row 4 kb + i
      const float mine = sacc[i], other = ldk::row_ror<8>(mine);  // lane c16 ^ 8 of the same row
      const float e = c16 < 8 ? mine : other, o = c16 < 8 ? other : mine;
      const float c = 1024.0f * (e + o), sx = __builtin_fmaf(16.0f, o, e);
#pragma unroll
      for (int t = 0; t < CPL; ++t)
        acc[t][i] = __builtin_fmaf((float)s2[t], tmp[t][i] - __builtin_fmaf((float)z2[t], sx, c), acc[t][i]);
      if constexpr (X5)
        acc5[i] = __builtin_fmaf((float)s5[gi], tmp5[i] - __builtin_fmaf((float)z5[gi], sx, c), acc5[i]);
    }
  }
  // ---- the NW partial tiles meet in LDS (over the records, once every wave is done with them)
  ldk::lds_barrier();
  float* red = reinterpret_cast<float*>(xs);  // [NW][MP][CWT]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (4 * kb + i < M) {
#pragma unroll
      for (int t = 0; t < CPL; ++t) red[(wave * MP + 4 * kb + i) * CWT + CPL * c16 + t] = acc[t][i];
      if constexpr (X5) red[(wave * MP + 4 * kb + i) * CWT + 16 * CPL + c16] = acc5[i];
    }
  }
  ldk::lds_barrier();
  const int n = M * CWT;  // outputs o = row * CWT + column of the tile
  auto store = [&](int o, float v) {
    const int nn = n0 + o % CWT;
    if (nn < a.N) {
      if (a.bias) v += (float)a.bias[nn];
      a.out[(int64_t)(o / CWT) * a.ldo + nn] = (half_t)v;
    }
  };
  for (int o = threadIdx.x; o < n; o += NW * 64) store(o, ldk::sum_waves(red + o, MP * CWT, NW));
}

// ------------------------------------------------------------------------------------ dispatch

enum Kern { kM1 = 0, kValu = 1, kMfma = 2, kMfmaX = 3 };

struct Plan {
  Kern kern;
  int mt, ln, rpl, cpw;  // row tile, lanes along N (MFMA: 16 * 64-column halves), rows per lane,
                         // chunks (MFMA: groups) per wave and pass
  int nw, splits, gps;  // gps: groups of the largest split
  bool even;  // splits asked for by the caller: the groups are dealt evenly over exactly `splits`
  int full;   // M = 1 kernel: leading tiles run whole while the rest split (0: all tiles alike)
  int mtile;  // MFMA kernel: 16-row tiles per workgroup (1, or 2 when M > 16)
};

int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

// Instantiated (MT, LN, RPL, CPW) shapes of the EXACT VALU kernel: those that fit the register
// budget of 1024-thread workgroups (128 VGPRs) without spilling. RPL = 8 is only needed for
// LN = 16 with 32-row groups (the plan takes RPL = 4 otherwise).
constexpr bool gemv_shape_ok(int mt, int ln, int rpl, int cpw) {
  if (ln != 4 && ln != 8 && ln != 16) return false;
  if (rpl == 8) return ln == 16 && cpw == 1;
  if (rpl != 4) return false;
  if (mt <= 2) return cpw == 1 || cpw == 2;
  if (mt == 4) return cpw == 1 || (cpw == 2 && ln >= 8);
  return mt == 8 && cpw == 1 && ln >= 8;
}

// Wave counts the M = 1 kernel is instantiated for (a plan rounds up; surplus waves idle).
constexpr int kM1Waves[] = {1, 2, 3, 4, 6, 8, 12, 16};

int m1_round_nw(int64_t want) {
  for (int w : kM1Waves)
    if (w >= want) return w;
  return 16;
}

// Most waves per workgroup the M = 1 kernel is instantiated for at this tile width and row count.
int m1_max_waves(int ln, int mr) {
  for (int i = (int)(sizeof(kM1Waves) / sizeof(kM1Waves[0])) - 1; i > 0; --i)
    if (m1_lds_ok(ln, kM1Waves[i], mr)) return kM1Waves[i];
  return 1;
}

int gemv_pxw(const Plan& p) { return (p.cpw * p.rpl * p.mt + p.ln - 1) / p.ln; }

size_t plan_lds_bytes(const Plan& p, int64_t M) {
  if (p.kern == kM1 || p.kern == kMfmaX) return 0;  // static LDS
  if (p.kern == kMfma) return (size_t)p.nw * std::min<int64_t>(M, 16 * p.mtile) * (4 * p.ln) * 4;
  return (size_t)p.nw * 64 * gemv_pxw(p) * 16 + (size_t)p.nw * p.mt * 4 * p.ln * 4;
}

int plan_cw(const Plan& p) { return 4 * p.ln; }

// Accumulator words of a split launch: one per output of every split tile (the MFMA kernel's row
// blocks of more than 16 rows: each block's full 16 * mtile rows).
int64_t split_words(const Plan& p, int64_t M, int64_t N) {
  const int cw = plan_cw(p);
  const int64_t tiles = (N + cw - 1) / cw - p.full;
  if (p.kern == kMfma && M > 16) return tiles * ((M + 16 * p.mtile - 1) / (16 * p.mtile)) * 16 * p.mtile * cw;
  const int64_t n = p.kern == kMfma ? std::min<int64_t>(M, 16) * cw : (int64_t)p.mt * cw;
  return tiles * n;
}

size_t workspace_need(const Plan& p, int64_t M, int64_t N) {
  return p.splits <= 1 ? 0 : ldk::splitk_bytes(split_words(p, M, N), p.splits);
}

int cpw_from_flags(int flags) {
  const int v = (flags & LDK_CPW_MASK) >> 4;
  return v ? 1 << (v - 1) : 0;
}

// The MFMA kernel with x staged in LDS takes decode rows 3-16 with group size 128 and K of at
// most 12 groups; a tuning argument that names another variant (block_n, split_k, EXACT, VALU,
// chunks per wave) keeps the wide-tile kernel or the VALU kernel.
bool mfma_x_applies(int64_t M, int64_t K, int gsh_rows, int block_n, int split_k, int flags) {
  return M >= 3 && M <= 16 && gsh_rows == 4 && (K >> 7) <= 12 && block_n == 0 && split_k <= 1 &&
         !(flags & (LDK_EXACT | LDK_PATH_VALU | LDK_CPW_MASK));
}

template <int MP, int NW, int GPW, int CPL, bool X5>
int launch_mfma_x_t(const W4Args& a, hipStream_t s) {
  constexpr int CWT = 16 * CPL + (X5 ? 16 : 0);
  (void)hipGetLastError();
  w4a16_mfma_x_kernel<MP, NW, GPW, CPL, X5><<<(unsigned)((a.N + CWT - 1) / CWT), NW * 64, 0, s>>>(a);
  return ldk::check_launch("w4a16_mfma_x");
}

template <int MP, int CPL, bool X5 = false>
int launch_mfma_x_mp(const W4Args& a, int nw, int gpw, hipStream_t s) {
  if (nw == 12 && gpw == 1) return launch_mfma_x_t<MP, 12, 1, CPL, X5>(a, s);
  if (nw == 6 && gpw == 2) return launch_mfma_x_t<MP, 6, 2, CPL, X5>(a, s);
  if (nw == 6 && gpw == 1) return launch_mfma_x_t<MP, 6, 1, CPL, X5>(a, s);
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: x-staged MFMA kernel with %d waves of %d groups not instantiated", nw, gpw);
}

int launch_mfma_x(const W4Args& a, const Plan& p, hipStream_t s) {
  // the kernel's LDS holds nw * cpw groups (all of K) and MP = mt rows; 64- and 80-column tiles
  // (ln 16, 20) take N a multiple of 4 (whole 16-byte loads of the clamped last lane)
  if (a.gsh_rows != 4 || a.M > p.mt || ((a.K >> 3) >> 4) > p.nw * p.cpw || (a.N + 31) / 32 > INT32_MAX ||
      (p.ln != 8 && p.ln != 16 && p.ln != 20) || (p.ln != 8 && a.N % 4))
    return ldk::fail(LDK_ERR_INVALID, "w4a16: x-staged MFMA plan does not fit M=%d N=%d K=%d", a.M, a.N, a.K);
  if (p.ln == 20) {
    switch (p.mt) {
      case 4: return launch_mfma_x_mp<4, 4, true>(a, p.nw, p.cpw, s);
      case 8: return launch_mfma_x_mp<8, 4, true>(a, p.nw, p.cpw, s);
      case 16: return launch_mfma_x_mp<16, 4, true>(a, p.nw, p.cpw, s);
    }
  } else if (p.ln == 16) {
    switch (p.mt) {
      case 4: return launch_mfma_x_mp<4, 4>(a, p.nw, p.cpw, s);
      case 8: return launch_mfma_x_mp<8, 4>(a, p.nw, p.cpw, s);
      case 16: return launch_mfma_x_mp<16, 4>(a, p.nw, p.cpw, s);
    }
  } else {
    switch (p.mt) {
      case 4: return launch_mfma_x_mp<4, 2>(a, p.nw, p.cpw, s);
      case 8: return launch_mfma_x_mp<8, 2>(a, p.nw, p.cpw, s);
      case 16: return launch_mfma_x_mp<16, 2>(a, p.nw, p.cpw, s);
    }
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: x-staged MFMA row tile %d", p.mt);
}

// Chooses the kernel, column tile, rows per lane, chunks per wave, workgroup size and split
// count for a shape. Measured on MI355X (decode shapes of Qwen2.5-1.5B, graph-timed sweeps over
// block_n, split_k and waves per workgroup): 128-byte row runs per tile read best (one L2 line);
// fewer than ~150 workgroups leave bandwidth unused once a shape moves more than a couple of MB
// (M = 1 down projection: 4.5 us at 240 workgroups against 7.7 us at 48), while a split costs one
// dependent atomic round trip (~0.3 us), so only large, narrow shapes split. For M = 1 six waves of
// two groups each (four rows per lane) beat deeper waves (three of four groups: +4%) and shallower
// ones (twelve of one: +12%) on the gate_up shape; shapes of <= 2 MB run 16-column tiles (o
// projection 3.2 us against 3.45 us at 32 columns).
Plan make_plan(int64_t M, int64_t N, int64_t K, int gsh_rows, int block_n, int split_k, int flags,
               size_t ws_bytes) {
  Plan p{};
  const int rpg = 1 << gsh_rows;
  const int64_t ng = (K / 8) >> gsh_rows;
  const int64_t wbytes = N * K / 2;
  // M = 1 and 2 run the factored VALU kernel (5 + 4M VALU ops per 8 weights, issued once the
  // pass's loads land: with 4 rows that compute alone outlasts the loads), from 3 rows the MFMA
  // kernel (4 VALU ops per 8 weights for all 16 rows of its B operand). A block_n only the VALU
  // kernels take (16 or 32) keeps M <= 8 on the VALU path. EXACT keeps M <= 8 on the VALU
  // kernels, which dequantize every weight as dequantize_ref does.
  // Two rows on a narrow shape of more than 2 MB (down) also take the MFMA kernel, split K ten
  // ways: 4.9 against 5.4 us for the two-row VALU kernel (wide shapes keep it: gate_up 5.7 us).
  const bool narrow_long = N < 128 * 128 && wbytes > (2 << 20);
  const bool mfma_auto = M > 8 || (!(flags & LDK_EXACT) && (M > 2 || (M == 2 && narrow_long && block_n == 0)) &&
                                   (block_n == 0 || block_n >= 64));
  const bool mfma = (flags & LDK_PATH_MFMA) || (mfma_auto && !(flags & LDK_PATH_VALU));
  const bool m1 = !mfma && !(flags & LDK_EXACT) && M <= 2;  // the factored VALU kernel
  p.kern = mfma ? kMfma : m1 ? kM1 : kValu;
  if (mfma && mfma_x_applies(M, K, gsh_rows, block_n, split_k, flags)) {
    // x staged in LDS, whole 32-column tiles: twelve waves of one group, or six of two for up to
    // four rows on grids of at least one tile per CU (gate_up M = 4: 6.3 against 6.4 us; q/o M = 4
    // on 48 tiles: 3.9 against 3.7 us with twelve), six of one for K <= 768
    const int ngx = (int)((K / 8) >> gsh_rows);
    p.kern = kMfmaX;
    p.mt = M <= 4 ? 4 : M <= 8 ? 8 : 16;
    // 64-column tiles from 5 rows on shapes of at least 256 of them: every workgroup stages its
    // x rows once for twice the columns, halving the x traffic through L2, which at 16 rows is
    // twice the weight bytes (gate_up M = 8 / 16: 6.48 / 7.36 -> 6.23 / 6.96 us; at 4 rows, and
    // on the narrow shapes with their half as many workgroups, 32 columns stay faster: gate_up
    // M = 4 5.88 against 6.67 us, q/o M = 16 3.98 against 4.54)
    p.ln = (M > 4 && N % 64 == 0 && N / 64 >= 256) ? 16 : 8;
    // a grid past 256 workgroups runs a second round on the CUs that take two tiles: where 64
    // columns give more than 256 tiles and 80 give at most 256, 80-column tiles
    if (M > 4 && N % 4 == 0 && (N + 63) / 64 > 256 && (N + 79) / 80 <= 256) p.ln = 20;
    p.rpl = 4;
    p.nw = ngx <= 6 ? 6 : (M <= 4 && N / 32 >= 256) ? 6 : 12;
    p.cpw = (ngx + p.nw - 1) / p.nw;
    p.splits = 1;
    p.gps = ngx;
    p.full = 0;
    p.mtile = 1;
    return p;
  }
  p.mt = mfma ? 16 : round_mt(M);
  p.mtile = mfma && M > 16 ? 2 : 1;
  if (mfma) {  // 128 columns on shapes wide enough to fill the CUs with them, else 64 (and 64 for
              // 32-row blocks of group-256 weights, whose 128-column variant runs out of registers);
              // decode rows on shapes of <= 2 MB take 32 columns (q/o/k/v at M = 8: 4.7 -> 4.4 us),
              // and so do 13-16 rows of the narrow long shapes (down), where half the K splits
              // halve the split-K words (below)
    p.ln = block_n == 32    ? 8
           : block_n == 64  ? 16
           : block_n == 128 ? 32
           : (M <= 16 && wbytes <= (2 << 20)) ? 8
           : (M > 12 && M <= 16 && N < 128 * 128 && split_k <= 0) ? 8
           : (N >= 128 * 128 && !(M > 16 && rpg > 16) ? 32 : 16);
  } else if (block_n) {
    p.ln = block_n / 4;
  } else if (m1) {  // small shapes are latency-bound: more, narrower workgroups
    p.ln = (wbytes <= (2 << 20) && N <= 4096) ? 4 : 8;
  } else if (p.mt == 8) {
    p.ln = N >= 1024 ? 16 : 8;
  } else {
    p.ln = N >= 512 ? 8 : 4;
  }
  const int cw = plan_cw(p);
  const int lkw = 64 / p.ln;
  if (m1) {
    p.rpl = 4;
  } else {
    p.rpl = (lkw % (rpg / std::min(rpg, 4)) == 0) ? std::min(rpg, 4) : 8;  // LG = rpg/rpl divides LKW
  }
  // groups a wave covers per pass / chunk
  const int gw = mfma ? 1 : lkw / (rpg / p.rpl);
  const int64_t tiles = (N + cw - 1) / cw;
  int64_t splits = split_k > 0 ? split_k : 1;
  // narrow shapes that move more than a couple of MB split K across workgroups (M = 1: about one
  // workgroup per CU). Multi-row splits carry M outputs per column through returning atomics,
  // so small shapes keep whole tiles and split K over the waves of a workgroup instead (q/o at
  // M = 16: 5.9 us whole, 25 us split twelve ways).
  // (MFMA: about 240 workgroups, with one returning atomic per thread below: down M = 2 / 4 /
  // 8 / 16 in 10 splits 4.9 / 5.0 / 5.45 / 6.70 us, in 8 splits 5.2 / 5.2 / 5.6 / 6.73)
  if (split_k <= 0 && tiles < 128 && wbytes > (2 << 20) && M <= 16)
    splits = m1 ? std::max<int64_t>(2, 256 / tiles) : (240 + tiles - 1) / tiles;
  // Prefill rows in row blocks of 32 (mtile 2, at most 8 waves) or 16 (mtile 1, up to 16 waves).
  // A long-K shape whose tiles and blocks leave most CUs idle splits K toward 256 workgroups, at
  // most 8 ways and never past 256 (a CU with two finishes last: down 1536x8960 M = 128 in 32-row
  // blocks, 2 splits 17.5 us, 3 splits on 288 workgroups 25.4); the short-K shapes (q/o/qkv, 12
  // groups) lose with any split (o M = 128 8.5 -> 10.9 us at 2). 16-row blocks, twice the
  // workgroups with twice the waves each, win wherever they fit in 256 workgroups on short K
  // (qkv M = 17 / 32 / 128: 6.6 / 8.1 / 8.4 -> 5.3 / 5.5 / 5.7 us; at 144 rows, 288 workgroups,
  // 9.8 against 8.4) and on long K where they split K at least twice over 192 or more workgroups,
  // or fill more of the grid than the 32-row blocks (down M = 17 / 32 / 48 / 64 / 80: 9.0 / 10.8 /
  // 12.1 / 12.8 / 14.4 -> 7.1 / 7.7 / 10.4 / 11.5 / 11.8 us in 5 / 5 / 3 / 2 / 2 splits). Whole
  // K over all of it in 16-row blocks reads the weights twice as often and stays level with the
  // 32-row blocks at the same grid (M = 128: 17.8 against 17.5; M = 96: 144 workgroups, 17.8,
  // against 14.7 for 32-row blocks in 3 splits on 216).
  if (M > 16 && split_k <= 0) {
    const bool long_k = mfma && ng >= 24;
    auto fill = [&](int64_t base) {  // splits toward 256 workgroups, at most 8, none past 256
      return long_k && base < 160 ? std::max<int64_t>(1, std::min<int64_t>(256 / base, 8)) : int64_t(1);
    };
    const int64_t b32 = tiles * ((M + 31) / 32), b16 = tiles * ((M + 15) / 16);
    const int64_t s32 = fill(b32), s16 = long_k ? std::max<int64_t>(1, std::min<int64_t>(256 / b16, 8)) : 1;
    splits = s32;
    if (mfma && b16 <= 256 && (!long_k || (s16 >= 2 && b16 * s16 >= 192) || b16 * s16 > b32 * s32)) {
      p.mtile = 1;
      splits = s16;
    } else if (long_k && block_n == 0 && p.ln == 16 && rpg <= 16) {
      // 128-column tiles where their K split fills a grid half again as large (down M = 192:
      // 64-column blocks over all of K on 144 workgroups 25.5 us, 128-column in 3 splits on 216
      // 22.4; M = 128 / 160 give 192 / 240 workgroups either way, and 64 columns stay faster,
      // 17.9 / 18.4 against 20.5 / 20.3)
      const int64_t b2 = (N + 127) / 128 * ((M + 31) / 32), s2 = fill(b2);
      if (2 * b2 * s2 >= 3 * b32 * s32) {
        p.ln = 32;
        splits = s2;
      }
    }
  }
  splits = std::min<int64_t>(std::min<int64_t>(splits, ng), kMaxSplits);
  p.gps = (int)((ng + splits - 1) / splits);
  p.splits = (int)((ng + p.gps - 1) / p.gps);
  // a split count the caller names is run as asked (the reference's SPLIT_K programs, each a K
  // range): its groups are dealt evenly, so e.g. 4 groups in 3 splits run as 2 + 1 + 1
  if (split_k > 0 && M <= 16) {
    p.splits = (int)splits;
    p.even = p.splits > 1 && ng % p.splits != 0;
  }
  if (p.splits > 1 && workspace_need(p, M, N) > ws_bytes) {  // no room for partials: one split
    p.splits = 1;
    p.gps = (int)ng;
    p.even = false;
  }
  // M = 1 with more than one round of 256 tiles: whole tiles give every CU the same whole-tile
  // count, and the remainder tiles split into one-wave-pass pieces that spread over all CUs
  // (gate_up: 512 whole tiles + 48 tiles x 6 splits of 2 groups; 560 whole tiles leave 48 CUs
  // with a third tile, measured 5.40 -> 5.06 us). The multi-row kernels keep whole tiles: their
  // split pieces carry M times the outputs through the workspace (MFMA gate_up M=16 measured
  // 10.15 -> 12.49 us with the same split).
  if (m1 && split_k <= 0 && tiles > 256 && tiles % 256) {
    const int64_t rem = tiles % 256;
    // groups per split: whole wave passes, chosen so that rem * splits lands nearest 256
    int64_t gps_r = ng, best = INT64_MAX;
    for (int64_t g = gw; g < ng; g += gw) {
      const int64_t s = (ng + g - 1) / g;
      const int64_t d = std::abs(rem * s - 256);
      if (s <= kMaxSplits && d < best) { best = d; gps_r = g; }
    }
    Plan q = p;
    q.gps = (int)gps_r;
    q.splits = (int)((ng + gps_r - 1) / gps_r);
    q.full = (int)(tiles - rem);
    if (q.splits > 1 && workspace_need(q, M, N) <= ws_bytes) p = q;
  }
  const int64_t chunks = ((p.full ? ng : p.gps) + gw - 1) / gw;  // wave passes of the largest workgroup
  if (m1) {
    p.cpw = 1;
    p.nw = m1_round_nw(std::min<int64_t>(m1_max_waves(p.ln, p.mt), chunks));
    return p;
  }
  // chunks per wave and round: the smallest that fits all chunks in one round of <= 16 waves
  int cpw = cpw_from_flags(flags);
  if (!cpw) {
    cpw = 4;
    for (int c : {1, 2, 4})
      if (chunks <= 16 * c) { cpw = c; break; }
  }
  if (mfma) {  // groups per wave and pass: all in one pass where registers allow (<= 16 waves at
              // 64 columns, <= 8 at 128)
    // up to 16 waves on 64-column tiles, and on 32-column tiles from 9 rows: down M = 16 on 32
    // columns in 5 splits (14 waves of one group) 6.41-6.42 us against 6.60 on 8 waves of two and
    // 6.70-6.71 for 64 columns in 10 splits; at 12 rows and fewer the 64-column plan stays
    // (M = 12 / 9 / 8 / 4: 5.94 / 5.67 / 5.56 / 5.33 against 5.84 / 5.61 / 5.50 / 5.06 us)
    const int wmax = (p.ln == 16 || (p.ln == 8 && M > 8)) && p.mtile == 1 ? 16 : 8;
    if (!cpw_from_flags(flags)) cpw = chunks > wmax ? 2 : 1;
    cpw = std::min(cpw, rpg <= 16 && p.mtile == 1 ? 2 : 1);
    p.cpw = cpw;
    p.nw = (int)std::min<int64_t>(wmax, (chunks + cpw - 1) / cpw);
    // a split tile's outputs leave through one returning atomic each, a thread's in turn: with
    // more outputs than lanes, the workgroup takes extra waves (no groups of their own) so that
    // every thread carries one (down M = 16 in 10 splits: 7.60 -> 6.70 us; M = 8: 5.99 -> 5.45)
    if (p.splits > 1 && M > 4)
      p.nw = std::max<int>(p.nw, std::min<int>(wmax, (int)((std::min<int64_t>(M, 16) * plan_cw(p) + 63) / 64)));
    return p;
  }
  while (cpw > 1 && !gemv_shape_ok(p.mt, p.ln, p.rpl, cpw)) cpw >>= 1;
  p.cpw = cpw;
  p.nw = (int)std::min<int64_t>(16, (chunks + cpw - 1) / cpw);
  return p;
}

template <int LN, int NW, int MR>
int launch_m1_rows(const W4Args& a, const SplitArgs& sp, int out_vec, hipStream_t stream) {
  if constexpr (m1_lds_ok(LN, NW, MR)) {
    const unsigned grid = (unsigned)(sp.full + sp.nsplit);
    ProArgs pa{};
    (void)hipGetLastError();
    if (a.gsh_rows == 4)
      w4a16_m1_kernel<LN, NW, 4, kProNone, MR><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa);
    else
      w4a16_m1_kernel<LN, NW, 0, kProNone, MR><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa);
    return ldk::check_launch("w4a16_m1");
  } else {
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: %d rows on %d waves of block_n %d exceed the LDS budget", MR, NW,
                     4 * LN);
  }
}

template <int LN, int NW>
int launch_m1_t(const W4Args& a, const SplitArgs& sp, int mr, int pro, const ProArgs& pa, hipStream_t stream) {
  const int out_vec = ldk::aligned(a.out, 8) && (a.M == 1 || a.ldo % 4 == 0) ? 1 : 0;
  const unsigned grid = (unsigned)(sp.full + sp.nsplit);
  if (pro != kProNone) {
    // fused prologues are built for the decode tile widths and group size 128
    if constexpr (LN == 4 || LN == 8) {
      if (a.gsh_rows != 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: fused prologues need group_size 128");
      (void)hipGetLastError();
      // exact: whole tiles, and one wave pass per wave covers the row
      const int gpw = (64 / LN) >> (a.gsh_rows - 2);
      const bool exact = sp.splits == 1 && sp.full == 0 && ((a.K >> 3) >> a.gsh_rows) == NW * gpw;
      if (exact && pro == kProRms) pro = kProRmsX;
      if (exact && pro == kProRmsRes) pro = kProRmsResX;
      switch (pro) {
        case kProRms: w4a16_m1_kernel<LN, NW, 4, kProRms, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProRmsRes: w4a16_m1_kernel<LN, NW, 4, kProRmsRes, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProRmsX: w4a16_m1_kernel<LN, NW, 4, kProRmsX, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProRmsResX: w4a16_m1_kernel<LN, NW, 4, kProRmsResX, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProSwiglu: w4a16_m1_kernel<LN, NW, 4, kProSwiglu, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProRmsPre: w4a16_m1_kernel<LN, NW, 4, kProRmsPre, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kEpiResStat: w4a16_m1_kernel<LN, NW, 4, kEpiResStat, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        case kProAttnStat: w4a16_m1_kernel<LN, NW, 4, kProAttnStat, 1><<<grid, NW * 64, 0, stream>>>(a, sp, out_vec, pa); break;
        default: return ldk::fail(LDK_ERR_INVALID, "w4a16: unknown prologue %d", pro);
      }
      return ldk::check_launch("w4a16_m1");
    } else {
      return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: fused prologues take block_n 16 or 32");
    }
  }
  switch (mr) {
    case 1: return launch_m1_rows<LN, NW, 1>(a, sp, out_vec, stream);
    case 2: return launch_m1_rows<LN, NW, 2>(a, sp, out_vec, stream);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: row tile %d not instantiated for the factored VALU kernel", mr);
}

template <int LN>
int launch_m1_ln(const W4Args& a, const SplitArgs& sp, int nw, int mr, int pro, const ProArgs& pa, hipStream_t s) {
  switch (nw) {
    case 1: return launch_m1_t<LN, 1>(a, sp, mr, pro, pa, s);
    case 2: return launch_m1_t<LN, 2>(a, sp, mr, pro, pa, s);
    case 3: return launch_m1_t<LN, 3>(a, sp, mr, pro, pa, s);
    case 4: return launch_m1_t<LN, 4>(a, sp, mr, pro, pa, s);
    case 6: return launch_m1_t<LN, 6>(a, sp, mr, pro, pa, s);
    case 8: return launch_m1_t<LN, 8>(a, sp, mr, pro, pa, s);
    case 12: return launch_m1_t<LN, 12>(a, sp, mr, pro, pa, s);
    case 16: return launch_m1_t<LN, 16>(a, sp, mr, pro, pa, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: %d waves per workgroup not instantiated", nw);
}

template <int MT, int LN, int RPL, int CPW>
int launch_gemv_t(const W4Args& a, const SplitArgs& sp, int nw, size_t lds, hipStream_t stream) {
  auto kern = w4a16_gemv_kernel<MT, LN, RPL, CPW>;
  if (lds > 64 * 1024) {
    if (lds > 160 * 1024) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: LDS need %zu B exceeds 160 KiB", lds);
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return ldk::fail(LDK_ERR_LAUNCH, "w4a16: cannot raise the LDS limit to %zu B", lds);
  }
  (void)hipGetLastError();
  kern<<<(unsigned)(sp.full + sp.nsplit), nw * 64, lds, stream>>>(a, sp);
  return ldk::check_launch("w4a16_gemv");
}

template <int MT, int LN, int RPL, int CPW>
int try_gemv(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s, bool* done) {
  if constexpr (gemv_shape_ok(MT, LN, RPL, CPW)) {
    if (p.rpl == RPL && p.cpw == CPW) {
      *done = true;
      return launch_gemv_t<MT, LN, RPL, CPW>(a, sp, p.nw, lds, s);
    }
  }
  return LDK_OK;
}

template <int MT, int LN>
int launch_gemv_shape(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s) {
  bool done = false;
  int st = try_gemv<MT, LN, 4, 1>(a, sp, p, lds, s, &done);
  if (!done) st = try_gemv<MT, LN, 4, 2>(a, sp, p, lds, s, &done);
  if (!done) st = try_gemv<MT, LN, 8, 1>(a, sp, p, lds, s, &done);
  if (!done)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: VALU shape mt=%d block_n=%d rpl=%d cpw=%d not instantiated", MT,
                     4 * LN, p.rpl, p.cpw);
  return st;
}

template <int MT>
int launch_gemv_ln(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s) {
  switch (p.ln) {
    case 4: return launch_gemv_shape<MT, 4>(a, sp, p, lds, s);
    case 8: return launch_gemv_shape<MT, 8>(a, sp, p, lds, s);
    case 16: return launch_gemv_shape<MT, 16>(a, sp, p, lds, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: block_n=%d not supported (16, 32 or 64)", 4 * p.ln);
}

template <int NH, int KS, int CPW, int MT, int NWD>
int launch_mfma_t(const W4Args& a, const SplitArgs& sp, int nw, size_t lds, hipStream_t s) {
  auto kern = w4a16_mfma_kernel<NH, KS, CPW, MT, NWD>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return ldk::fail(LDK_ERR_LAUNCH, "w4a16: cannot raise the LDS limit to %zu B", lds);
  const int64_t mblocks = (a.M + 16 * MT - 1) / (16 * MT);
  if (mblocks > 65535) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: M=%d needs more than 65535 row blocks", a.M);
  if ((int64_t)(16 * MT - 1) * a.ldx * 2 + (int64_t)a.K * 2 >= (int64_t(1) << 31))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: a row block of x spans 2 GiB or more (ldx=%lld)", (long long)a.ldx);
  (void)hipGetLastError();
  kern<<<dim3((unsigned)(sp.full + sp.nsplit), (unsigned)mblocks), nw * 64, lds, s>>>(a, sp);
  return ldk::check_launch("w4a16_mfma");
}

template <int NH, int NWD>
int launch_mfma_nh(const W4Args& a, const SplitArgs& sp, const Plan& p, size_t lds, hipStream_t s) {
  const bool two = p.cpw == 2;
  if (p.mtile == 2) {
    switch (1 << a.gsh_rows) {
      case 4: return launch_mfma_t<NH, 1, 1, 2, NWD>(a, sp, p.nw, lds, s);
      case 8: return launch_mfma_t<NH, 2, 1, 2, NWD>(a, sp, p.nw, lds, s);
      case 16: return launch_mfma_t<NH, 4, 1, 2, NWD>(a, sp, p.nw, lds, s);
      case 32:
        if constexpr (NH == 1) return launch_mfma_t<NH, 8, 1, 2, NWD>(a, sp, p.nw, lds, s);
        return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: group_size 256 with M > 16 takes block_n=64");
    }
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: group size not supported by the MFMA kernel");
  }
  switch (1 << a.gsh_rows) {
    case 4: return two ? launch_mfma_t<NH, 1, 2, 1, NWD>(a, sp, p.nw, lds, s) : launch_mfma_t<NH, 1, 1, 1, NWD>(a, sp, p.nw, lds, s);
    case 8: return two ? launch_mfma_t<NH, 2, 2, 1, NWD>(a, sp, p.nw, lds, s) : launch_mfma_t<NH, 2, 1, 1, NWD>(a, sp, p.nw, lds, s);
    case 16: return two ? launch_mfma_t<NH, 4, 2, 1, NWD>(a, sp, p.nw, lds, s) : launch_mfma_t<NH, 4, 1, 1, NWD>(a, sp, p.nw, lds, s);
    case 32: return launch_mfma_t<NH, 8, 1, 1, NWD>(a, sp, p.nw, lds, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: group size not supported by the MFMA kernel");
}

int launch_plan(const W4Args& a, const Plan& p, void* ws, hipStream_t s, int pro = kProNone,
                const ProArgs& pa = ProArgs{}) {
  const int64_t tiles = (a.N + plan_cw(p) - 1) / plan_cw(p);
  const bool split = p.splits > 1;
  const int ng = (a.K >> 3) >> a.gsh_rows;
  const SplitArgs sp{p.splits, p.even ? ng / p.splits : p.gps, split ? static_cast<uint64_t*>(ws) : nullptr, p.full,
                     (int)((tiles - p.full) * p.splits), div_magic(p.splits),
                     split ? ldk::splitk_side(ws, split_words(p, a.M, a.N)) : nullptr, p.even ? ng % p.splits : 0};
  if (sp.full + (int64_t)sp.nsplit >= 65536)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: %lld workgroups exceed the grid mapping limit", (long long)(sp.full + (int64_t)sp.nsplit));
  const size_t lds = plan_lds_bytes(p, a.M);
  if (lds > 160 * 1024) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: LDS need %zu B exceeds 160 KiB", lds);
  if (p.kern == kM1) {
    // LG = rows_per_group / 4 lanes per group must divide the 64 / LN lanes along K
    if ((1 << a.gsh_rows) > 4 * (64 / p.ln))
      return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: block_n=%d too wide for group_size %d on the M = 1 kernel",
                       4 * p.ln, 8 << a.gsh_rows);
    switch (p.ln) {
      case 4: return launch_m1_ln<4>(a, sp, p.nw, p.mt, pro, pa, s);
      case 8: return launch_m1_ln<8>(a, sp, p.nw, p.mt, pro, pa, s);
      case 16: return launch_m1_ln<16>(a, sp, p.nw, p.mt, pro, pa, s);
    }
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: block_n=%d not supported (16, 32 or 64)", 4 * p.ln);
  }
  if (pro != kProNone) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16: fused prologues run on the M = 1 kernel");
  if (p.kern == kMfmaX) return launch_mfma_x(a, p, s);
  if (p.kern == kMfma) {
    if (p.ln == 8) return launch_mfma_nh<1, 2>(a, sp, p, lds, s);  // 32-column tiles
    return p.ln == 16 ? launch_mfma_nh<1, 4>(a, sp, p, lds, s) : launch_mfma_nh<2, 4>(a, sp, p, lds, s);
  }
  switch (p.mt) {
    case 1: return launch_gemv_ln<1>(a, sp, p, lds, s);
    case 2: return launch_gemv_ln<2>(a, sp, p, lds, s);
    case 4: return launch_gemv_ln<4>(a, sp, p, lds, s);
    case 8: return launch_gemv_ln<8>(a, sp, p, lds, s);
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

int plan_flags(const Plan& p) {
  const int cpw_code = p.kern == kValu ? (p.cpw == 1 ? 1 : p.cpw == 2 ? 2 : 3) : 0;
  return (p.kern == kMfma || p.kern == kMfmaX ? LDK_PATH_MFMA : LDK_PATH_VALU) | (p.kern == kValu ? LDK_EXACT : LDK_FACTORED) |
         (cpw_code << 4);
}

}  // namespace

extern "C" int64_t ldk_workspace_bytes(void) { return (int64_t)64 << 20; }

// Rows from which the prefill GEMM (prefill.hip) may replace the MFMA kernel's 32-row blocks.
static constexpr int64_t kGemmRows = 64;
static constexpr int64_t kGemmWideRows = 32;  // from this many rows on shapes of N >= 8192

static bool gemm_applies(int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx, const void* out, int64_t ldo, bool forced) {
  return (forced || M > 16) && ldk::gemm_supported(ldk::WFmt::kInt4, M, N, K, group_size, ldx) && (!out || ldk::aligned(out, 8)) &&
         ldo % 4 == 0;
}

// The library's choice for prefill rows, from graph-timed sweeps on MI355X over the Qwen2.5-1.5B
// shapes (M = 65 .. 2048): the row blocks re-read the packed weights per block but split K over
// the waves of a workgroup, which wins while the weights dominate and the tiles are few (qkv/o at
// M <= 128: 5.3-5.7 us on 16-row blocks, at M <= 256: 8.5 us on 32-row blocks, against 10.3-12.4
// us; down at M = 256: 25.7 against 31.1 us); the GEMM reads
// them once per 64/128-row tile and wins on wide shapes at every row count (gate_up M = 65: 18.4
// against 22.2 us; M = 2048: 116 against 364 us) and on narrow shapes whose 32-row blocks would need more than 256
// workgroups, or that have 512 rows or more (qkv M = 512: 12.6 against 15.1 us; down M = 512: 34.8
// against 47.5 us). A tuning argument that names another
// kernel keeps it.
static bool uses_gemm(int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx, const void* out, int64_t ldo, int block_n,
               int split_k, int flags) {
  if (flags & LDK_PATH_GEMM) return true;
  if (block_n || split_k || (flags & (LDK_PATH_VALU | LDK_PATH_MFMA | LDK_EXACT | LDK_FACTORED))) return false;
  // wide shapes from 32 rows: the 32-row blocks re-read all the weights per block (gate_up M = 32 /
  // 64: 12.0 / 22.6 us on the blocks, 10.5 / 15.3 on the GEMM's 32-row tiles; M = 17: 9.5 against
  // 10.3)
  if (M < (N >= 8192 ? kGemmWideRows : kGemmRows + 1)) return false;
  // narrow shapes from 257 rows where the blocks need more than 256 workgroups, and from 512 rows:
  // past 256 workgroups the blocks lose a round (qkv M = 288 / 384 on 9 / 12 x 32 blocks: 14.9 /
  // 15.0 us against 10.3 on the GEMM; down M = 384 / 448: 47.7 / 47.4 against 28.8 / 29.7), below
  // it they keep the lead (down M = 288 on 9 x 24 blocks: 25.8 against 33.0; M = 256: 25.6 against
  // 28.4; qkv M = 256 on 8 x 32: 8.5 against 10.3)
  const int64_t blocks = (N + 63) / 64 * ((M + 31) / 32);
  if (!(N >= 8192 || M >= 512 || (M > 256 && blocks > 256))) return false;
  return gemm_applies(M, N, K, group_size, ldx, out, ldo, false);
}

// Name of the kernel instantiation launch_plan runs for a plan, as the profiler lists it.
static int plan_kernel_name(const Plan& p, int gsh_rows, char* buf, size_t len) {
  const int rpg = 1 << gsh_rows;
  int n = 0;
  if (p.kern == kM1) {
    n = snprintf(buf, len, "w4a16_m1_kernel<%d, %d, %d, 0, %d>", p.ln, p.nw, gsh_rows == 4 ? 4 : 0, p.mt);
  } else if (p.kern == kMfmaX) {
    n = snprintf(buf, len, "w4a16_mfma_x_kernel<%d, %d, %d, %d, %s>", p.mt, p.nw, p.cpw, p.ln == 8 ? 2 : 4,
                 p.ln == 20 ? "true" : "false");
  } else if (p.kern == kValu) {
    n = snprintf(buf, len, "w4a16_gemv_kernel<%d, %d, %d, %d>", p.mt, p.ln, p.rpl, p.cpw);
  } else {
    const int nh = p.ln == 32 ? 2 : 1, nwd = p.ln == 8 ? 2 : 4, ks = rpg / 4;
    const int cpw = p.mtile == 2 ? 1 : (p.cpw == 2 && rpg <= 16 ? 2 : 1);
    n = snprintf(buf, len, "w4a16_mfma_kernel<%d, %d, %d, %d, %d>", nh, ks, cpw, p.mtile, nwd);
  }
  return n < 0 || (size_t)n >= len ? ldk::fail(LDK_ERR_INVALID, "w4a16_kernel_name: buffer of %zu bytes too small", len) : LDK_OK;
}

extern "C" int ldk_w4a16_kernel_name(int64_t M, int64_t N, int64_t K, int group_size, char* buf, int64_t buf_len) {
  if (M <= 0 || N <= 0 || K <= 0 || !buf || buf_len <= 0) return ldk::fail(LDK_ERR_INVALID, "w4a16_kernel_name: bad arguments");
  const int gsh = log2_exact(group_size);
  if (gsh < 5 || gsh > 8 || K % group_size) return ldk::fail(LDK_ERR_INVALID, "w4a16_kernel_name: bad group_size %d", group_size);
  if (uses_gemm(M, N, K, group_size, K, nullptr, N % 4 == 0 ? N : 1, 0, 0, 0)) {
    const int n = snprintf(buf, (size_t)buf_len, "%s", ldk::gemm_kernel_name(ldk::WFmt::kInt4, M, N, K, 0));
    return n < 0 || n >= buf_len ? ldk::fail(LDK_ERR_INVALID, "w4a16_kernel_name: buffer too small") : LDK_OK;
  }
  const Plan p = make_plan(M, N, K, gsh - 3, 0, 0, 0, (size_t)ldk_workspace_bytes());
  return plan_kernel_name(p, gsh - 3, buf, (size_t)buf_len);
}

// The launch limits of a plan (instantiated shapes, LDS, grid), checked before anything is
// launched, so that a plan query reports what the call would do (launch_plan and its launchers
// keep their own checks). ldx: the row stride of x the call passes (K for a query).
static int plan_check(const char* fn, const Plan& p, int64_t M, int64_t N, int64_t K, int gsh_rows, int64_t ldx) {
  const int64_t tiles = (N + plan_cw(p) - 1) / plan_cw(p);
  if (p.full + (tiles - p.full) * p.splits >= 65536)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: %lld workgroups exceed the grid mapping limit", fn,
                     (long long)(p.full + (tiles - p.full) * p.splits));
  if (plan_lds_bytes(p, M) > 160 * 1024)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: LDS need %zu B exceeds 160 KiB", fn, plan_lds_bytes(p, M));
  const int rpg = 1 << gsh_rows;
  switch (p.kern) {
    case kM1:
      if (p.ln != 4 && p.ln != 8 && p.ln != 16)
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d not supported (16, 32 or 64)", fn, 4 * p.ln);
      if (rpg > 4 * (64 / p.ln))
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d too wide for group_size %d on the M = 1 kernel", fn,
                         4 * p.ln, 8 * rpg);
      if (p.mt > 2 || !m1_lds_ok(p.ln, p.nw, p.mt))
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: %d rows on %d waves of block_n %d not instantiated", fn, p.mt, p.nw,
                         4 * p.ln);
      return LDK_OK;
    case kValu:
      if (!gemv_shape_ok(p.mt, p.ln, p.rpl, p.cpw))
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: VALU shape mt=%d block_n=%d rpl=%d cpw=%d not instantiated", fn,
                         p.mt, 4 * p.ln, p.rpl, p.cpw);
      return LDK_OK;
    case kMfmaX:
      if (gsh_rows != 4 || M > p.mt || ((K >> 3) >> 4) > p.nw * p.cpw || (p.ln != 8 && p.ln != 16 && p.ln != 20) ||
          (p.ln != 8 && N % 4))
        return ldk::fail(LDK_ERR_INVALID, "%s: x-staged MFMA plan does not fit M=%lld N=%lld K=%lld", fn, (long long)M,
                         (long long)N, (long long)K);
      return LDK_OK;
    case kMfma:
      if (p.mtile == 2 && rpg == 32 && p.ln == 32)
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: group_size 256 with M > 16 takes block_n=64", fn);
      if ((M + 16 * p.mtile - 1) / (16 * p.mtile) > 65535)
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: M=%lld needs more than 65535 row blocks", fn, (long long)M);
      if ((int64_t)(16 * p.mtile - 1) * ldx * 2 + K * 2 >= (int64_t(1) << 31))
        return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: a row block of x spans 2 GiB or more (ldx=%lld)", fn, (long long)ldx);
      return LDK_OK;
  }
  return ldk::fail(LDK_ERR_INVALID, "%s: unknown kernel %d", fn, (int)p.kern);
}

// What a call runs: the prefill GEMM, or a decode-kernel plan.
struct Call {
  bool gemm;
  Plan p;
};

// A call's shape and tuning arguments checked without its pointers: the errors the call returns
// for them, and what it runs. ldx, ldo and the output's alignment decide whether the prefill GEMM
// takes the call (out may be null for a query: taken as aligned); ws_bytes is the workspace the
// call has.
static int plan_call(const char* fn, int64_t M, int64_t N, int64_t K, int group_size, int gsh_rows, int64_t ldx,
                     const void* out, int64_t ldo, int block_n, int split_k, int flags, size_t ws_bytes, Call* c) {
  c->gemm = false;
  if (M > 65535LL * 32) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: M=%lld too large", fn, (long long)M);
  if (flags & ~(LDK_FACTORED | LDK_EXACT | LDK_PATH_VALU | LDK_PATH_MFMA | LDK_PATH_GEMM | LDK_CPW_MASK))
    return ldk::fail(LDK_ERR_INVALID, "%s: unknown flags 0x%x", fn, flags);
  if (flags & LDK_PATH_GEMM) {
    if (flags & (LDK_PATH_VALU | LDK_PATH_MFMA | LDK_FACTORED))
      return ldk::fail(LDK_ERR_INVALID, "%s: the GEMM path excludes the VALU/MFMA paths and FACTORED", fn);
    if (!gemm_applies(M, N, K, group_size, ldx, out, ldo, true))
      return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the prefill GEMM takes group_size >= 64, N %% 8 == 0, K %% 64 == 0 "
                       "and an 8-byte aligned output with ldo %% 4 == 0 (M=%lld N=%lld K=%lld group_size=%d)", fn,
                       (long long)M, (long long)N, (long long)K, group_size);
  }
  if (uses_gemm(M, N, K, group_size, ldx, out, ldo, block_n, split_k, flags)) {
    if (block_n && block_n != 128 && block_n != 256)
      return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d must be 128 or 256 on the GEMM path", fn, block_n);
    if (split_k < 0) return ldk::fail(LDK_ERR_INVALID, "%s: split_k=%d must be >= 0", fn, split_k);
    c->gemm = true;
    return LDK_OK;
  }
  if ((flags & LDK_FACTORED) && (flags & LDK_EXACT)) return ldk::fail(LDK_ERR_INVALID, "%s: FACTORED and EXACT are exclusive", fn);
  if ((flags & LDK_PATH_VALU) && (flags & LDK_PATH_MFMA)) return ldk::fail(LDK_ERR_INVALID, "%s: VALU and MFMA paths are exclusive", fn);
  if ((flags & LDK_FACTORED) && (flags & LDK_PATH_VALU) && M > 2)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: FACTORED on the VALU kernel takes M <= 2; more rows run it on the MFMA kernel", fn);
  if ((flags & LDK_EXACT) && (flags & LDK_PATH_MFMA))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the MFMA kernel computes the factored form; EXACT runs on the VALU kernels (M <= 8)", fn);
  if ((flags & LDK_PATH_VALU) && M > 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the VALU kernel takes M <= 8", fn);
  if (block_n && block_n != 16 && block_n != 32 && block_n != 64 && block_n != 128)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d must be 16, 32, 64 or 128 (MFMA; 128 or 256 on the GEMM path)", fn,
                     block_n);
  if (block_n == 128 && !(flags & LDK_PATH_MFMA) && M <= 8 && (M <= 2 || (flags & (LDK_EXACT | LDK_PATH_VALU))))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: block_n=128 is the MFMA kernel's tile (M > 2 or the MFMA flag)", fn);
  if (split_k < 0) return ldk::fail(LDK_ERR_INVALID, "%s: split_k=%d must be >= 0", fn, split_k);
  if (split_k > kMaxSplits) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: split_k=%d above %d", fn, split_k, kMaxSplits);
  c->p = make_plan(M, N, K, gsh_rows, block_n, split_k, flags, ws_bytes);
  if (c->p.kern == kMfma && block_n && block_n != 32 && block_n != 64 && block_n != 128)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: the MFMA kernel uses block_n 32, 64 or 128", fn);
  if (split_k > 1 && c->p.splits == 1 && (K / group_size) > 1 && M <= 16) {
    const Plan want = make_plan(M, N, K, gsh_rows, block_n, split_k, flags, SIZE_MAX);
    return ldk::fail(LDK_ERR_INVALID, "%s: split_k=%d needs %zu bytes of workspace for its partial sums, %zu available",
                     fn, split_k, workspace_need(want, M, N), ws_bytes);
  }
  return plan_check(fn, c->p, M, N, K, gsh_rows, ldx);
}

static int w4a16_matmul_impl(const char* fn, const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                             const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                             int group_size, int block_n, int split_k, int flags, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  int gsh_rows = 0;
  int st = validate(fn, x, ldx, qweight, scales, zeros, out, ldo, M, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  Call c;
  st = plan_call(fn, M, N, K, group_size, gsh_rows, ldx, out, ldo, block_n, split_k, flags,
                 workspace ? (size_t)workspace_bytes : 0, &c);
  if (st) return st;
  if (c.gemm) {
    const ldk::GemmArgs g{(const half_t*)x, ldx, qweight, (const half_t*)scales, (const half_t*)zeros,
                          (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K, group_size,
                          workspace, workspace ? workspace_bytes : 0, block_n, split_k};
    return ldk::gemm_launch(ldk::WFmt::kInt4, g, (hipStream_t)stream);
  }
  const W4Args a{(const half_t*)x, ldx, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K, gsh_rows};
  return launch_plan(a, c.p, workspace, (hipStream_t)stream);
}

// Prefill rows of the gate_up projection with SwiGLU in the GEMM's epilogue: out [M, N/2] =
// swiglu_fused(x @ dequant(W)^T (+ bias)) with the standalone SwiGLU's steps on the fp16 products,
// where the library's plan for [M, N, K] is the prefill GEMM with two or more column groups and no
// K split (ldk_w4a16_matmul_swiglu_applies); the fused SwiGLU launch and the [M, N] round trip
// through memory go away.
static bool swiglu_gemm_applies(int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx, int64_t ws_bytes) {
  return N % 8 == 0 && uses_gemm(M, N, K, group_size, ldx, nullptr, N, 0, 0, 0) &&
         ldk::gemm_swiglu_applies(ldk::WFmt::kInt4, M, N, K, group_size, ldx, 0, 0, ws_bytes);
}

extern "C" int ldk_w4a16_matmul_swiglu_applies(int64_t M, int64_t N, int64_t K, int group_size) {
  return M > 0 && N > 0 && K > 0 && group_size > 0 && swiglu_gemm_applies(M, N, K, group_size, K, ldk_workspace_bytes()) ? 1 : 0;
}

extern "C" int ldk_w4a16_matmul_swiglu(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                                       const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M, int64_t N,
                                       int64_t K, int group_size, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "w4a16_matmul_swiglu";
  int gsh_rows = 0;
  int st = validate(fn, x, ldx, qweight, scales, zeros, out, N, M, N, K, group_size, &gsh_rows);  // out checked below
  if (st) return st;
  if (N % 2 || ldo < N / 2 || ldo % 4 || !ldk::aligned(out, 8))
    return ldk::fail(LDK_ERR_ALIGN, "%s: out [M, N/2] 8-byte aligned with ldo >= N/2 and ldo %% 4 == 0", fn);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  if (!swiglu_gemm_applies(M, N, K, group_size, ldx, workspace ? workspace_bytes : 0))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: M=%lld N=%lld K=%lld does not run the prefill GEMM with paired column "
                     "groups (ldk_w4a16_matmul_swiglu_applies)", fn, (long long)M, (long long)N, (long long)K);
  ldk::GemmArgs g{(const half_t*)x, ldx, qweight, (const half_t*)scales, (const half_t*)zeros, (const half_t*)bias,
                  (half_t*)out, ldo, (int)M, (int)N, (int)K, group_size, workspace, workspace ? workspace_bytes : 0, 0, 0};
  g.swiglu = 1;
  return ldk::gemm_launch(ldk::WFmt::kInt4, g, (hipStream_t)stream);
}

extern "C" int ldk_w4a16_config(int64_t M, int64_t N, int64_t K, int group_size, int* block_n, int* split_k, int* flags) {
  static const char* fn = "w4a16_config";
  if (!block_n || !split_k || !flags) return ldk::fail(LDK_ERR_INVALID, "%s: null block_n, split_k or flags", fn);
  if (M <= 0 || N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "%s: M, N, K must be positive", fn);
  const int gsh = log2_exact(group_size);
  if (gsh < 3 || K % group_size) return ldk::fail(LDK_ERR_INVALID, "%s: group_size=%d must be a power of two >= 8 dividing K=%lld", fn, group_size, (long long)K);
  if (group_size < 32 || group_size > 256) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: group_size=%d outside 32..256", fn, group_size);
  if (N % 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N=%lld must be a multiple of 4", fn, (long long)N);
  if (N > INT32_MAX / 8 || K > INT32_MAX / 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: N or K too large", fn);
  Call c;
  const int st = plan_call(fn, M, N, K, group_size, gsh - 3, K, nullptr, N, *block_n, *split_k, *flags,
                           (size_t)ldk_workspace_bytes(), &c);
  if (st) return st;
  if (c.gemm) {
    ldk::gemm_plan(ldk::WFmt::kInt4, M, N, K, *block_n, *split_k, ldk_workspace_bytes(), block_n, split_k);
    *flags = LDK_PATH_GEMM;
    return LDK_OK;
  }
  *block_n = plan_cw(c.p);
  *split_k = c.p.splits;
  *flags = plan_flags(c.p);
  return LDK_OK;
}

extern "C" int ldk_w4a16_matmul(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int block_n, int split_k, int flags, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  return w4a16_matmul_impl("w4a16_matmul", x, ldx, qweight, scales, zeros, bias, out, ldo, M, N, K, group_size, block_n,
                           split_k, flags, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------- allocation-free entry point
//
// ldk_w4a16_matmul_noalloc is ldk_w4a16_matmul with the split-K workspace taken from `scratch`, a
// file-scope device array of LDK_NOALLOC_SCRATCH_BYTES per GPU, instead of a caller-provided
// buffer: for callers that cannot allocate (code under graph capture that has no workspace yet,
// tight serving loops, harnesses that forbid hipMalloc). Host code never passes the array's name
// to a kernel (on the host it is only a stand-in for the symbol): the first call on each device
// looks up the device address with hipGetSymbolAddress, with that device current, clears the
// array once with a fill kernel, and keeps the address per device. The kernels leave every
// accumulator word and side slot they use zero again, so later calls need no clearing. Calls on
// one GPU share its array: calls that overlap on one GPU (different streams, no ordering) race.
namespace {
constexpr size_t kScratchBytes = LDK_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, set on first use

__global__ void zero_fill_kernel(u32x4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

// The current device's scratch address, looked up (and the array cleared on `stream`) on the
// first call on that device.
int current_scratch(const char* fn, hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return ldk::fail(LDK_ERR_LAUNCH, "%s: no current HIP device (or device %d >= %d)", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return ldk::fail(LDK_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                       hipGetErrorString(e));
    if (!ldk::aligned(ptr, 256)) return ldk::fail(LDK_ERR_ALIGN, "%s: scratch is not 256-byte aligned", fn);
    (void)hipGetLastError();
    zero_fill_kernel<<<256, 256, 0, stream>>>(static_cast<u32x4*>(ptr), kScratchBytes / 16);
    const int st = ldk::check_launch("w4a16_matmul_noalloc scratch clear");
    if (st) return st;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return LDK_OK;
}
}  // namespace

extern "C" int ldk_w4a16_matmul_noalloc(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                                        const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M,
                                        int64_t N, int64_t K, int group_size, int block_n, int split_k, int flags,
                                        void* stream) {
  static const char* fn = "w4a16_matmul_noalloc";
  void* ws = nullptr;
  const int st = current_scratch(fn, (hipStream_t)stream, &ws);
  if (st) return st;
  return w4a16_matmul_impl(fn, x, ldx, qweight, scales, zeros, bias, out, ldo, M, N, K, group_size, block_n, split_k,
                           flags, ws, (int64_t)kScratchBytes, stream);
}

extern "C" int ldk_w4a16_decode(const void* x, int64_t ldx, const int32_t* qweight, const void* scales, const void* zeros,
                                const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                                int split_k, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_decode: M=%lld > 16 rows", (long long)M);
  return ldk_w4a16_matmul(x, ldx, qweight, scales, zeros, bias, out, ldo, M, N, K, group_size, 0, split_k, 0,
                          workspace, workspace_bytes, stream);
}

// Fused decode entries (M = 1): the activation row is formed inside the W4A16 kernel's x staging,
// which removes one launch each from a decode layer (the reference runs rmsnorm and swiglu as
// kernels of their own, kernels/e2e/model.py:79-97).

extern "C" int ldk_w4a16_rmsnorm_matmul(const void* x, const void* residual, void* residual_out, const void* norm_weight,
                                        float eps, const int32_t* qweight, const void* scales, const void* zeros,
                                        const void* bias, void* out, int64_t N, int64_t K, int group_size,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_rmsnorm_matmul", x, K, qweight, scales, zeros, out, N, 1, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (!norm_weight) return ldk::fail(LDK_ERR_INVALID, "w4a16_rmsnorm_matmul: null norm_weight");
  if ((residual == nullptr) != (residual_out == nullptr))
    return ldk::fail(LDK_ERR_INVALID, "w4a16_rmsnorm_matmul: residual and residual_out must both be given or both be null");
  if (residual && (residual == residual_out || x == residual_out))
    return ldk::fail(LDK_ERR_INVALID, "w4a16_rmsnorm_matmul: residual_out must not alias x or residual");
  if (!ldk::aligned(norm_weight, 16) || (residual && (!ldk::aligned(residual, 16) || !ldk::aligned(residual_out, 16))))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_rmsnorm_matmul: norm_weight, residual and residual_out must be 16-byte aligned");
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_rmsnorm_matmul: workspace must be a 256-byte aligned pointer");
  Plan p = make_plan(1, N, K, gsh_rows, 0, 0, 0, workspace ? (size_t)workspace_bytes : 0);
  if (p.full) {  // whole tiles: every workgroup then reads the whole row, which its statistic needs
    p.full = 0;
    p.splits = 1;
    p.gps = (int)((K / 8) >> gsh_rows);
  }
  const W4Args a{(const half_t*)x, K, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K, gsh_rows};
  const ProArgs pa{(const half_t*)residual, (half_t*)residual_out, (const half_t*)norm_weight, eps};
  return launch_plan(a, p, workspace, (hipStream_t)stream, residual ? kProRmsRes : kProRms, pa);
}

extern "C" int ldk_w4a16_swiglu_matmul(const void* gate_up, const int32_t* qweight, const void* scales, const void* zeros,
                                       const void* bias, void* out, int64_t N, int64_t K, int group_size,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_swiglu_matmul", gate_up, 2 * K, qweight, scales, zeros, out, N, 1, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_swiglu_matmul: workspace must be a 256-byte aligned pointer");
  const Plan p = make_plan(1, N, K, gsh_rows, 0, 0, 0, workspace ? (size_t)workspace_bytes : 0);
  const W4Args a{(const half_t*)gate_up, 2 * K, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K, gsh_rows};
  return launch_plan(a, p, workspace, (hipStream_t)stream, kProSwiglu, ProArgs{});
}

// Residual + RMSNorm split across the two projections around it (decode, one row). The first
// launch (the o projection of a layer) computes h = fp16(y + residual), the new residual stream,
// for its columns and publishes one partial sum of h^2 per column tile; the second (gate_up)
// forms rmsnorm(h) * weight while it stages h, summing those partials instead of reducing the
// row itself (no barrier, no extra row loads, and its balanced grid). The pair replaces
// linear + rmsnorm(x, residual) + linear of the reference's layer (kernels/e2e/model.py:79-97,
// 226-233). The first launch runs whole column tiles (each tile's columns end in one workgroup).

namespace {
Plan residual_stats_plan(int64_t N, int64_t K, int gsh_rows, size_t ws) {
  Plan p = make_plan(1, N, K, gsh_rows, 0, 0, 0, ws);
  p.full = 0;
  p.splits = 1;
  p.gps = (int)((K / 8) >> gsh_rows);
  const int gw = (64 / p.ln) >> (gsh_rows - 2);
  p.nw = m1_round_nw(std::min<int64_t>(m1_max_waves(p.ln, 1), (p.gps + gw - 1) / gw));
  return p;
}
}  // namespace

extern "C" int64_t ldk_w4a16_row_stats_count(int64_t N, int64_t K, int group_size) {
  const int gsh = log2_exact(group_size);
  if (N <= 0 || K <= 0 || gsh < 5 || gsh > 8 || K % group_size)
    return -(int64_t)ldk::fail(LDK_ERR_INVALID, "w4a16_row_stats_count: bad shape N=%lld K=%lld group_size=%d",
                               (long long)N, (long long)K, group_size);
  const Plan p = residual_stats_plan(N, K, gsh - 3, (size_t)ldk_workspace_bytes());
  return (N + plan_cw(p) - 1) / plan_cw(p);
}

extern "C" int ldk_w4a16_matmul_residual_stats(const void* x, const void* residual, void* h_out, float* row_stats,
                                               const int32_t* qweight, const void* scales, const void* zeros,
                                               const void* bias, int64_t N, int64_t K, int group_size, void* workspace,
                                               int64_t workspace_bytes, void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_matmul_residual_stats", x, K, qweight, scales, zeros, h_out, N, 1, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (!residual || !row_stats) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul_residual_stats: null residual or row_stats");
  if (h_out == x) return ldk::fail(LDK_ERR_INVALID, "w4a16_matmul_residual_stats: h_out must not alias x");
  if (!ldk::aligned(residual, 8) || !ldk::aligned(h_out, 8) || !ldk::aligned(row_stats, 4))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_matmul_residual_stats: residual and h_out 8-byte, row_stats 4-byte aligned");
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_matmul_residual_stats: workspace must be a 256-byte aligned pointer");
  const Plan p = residual_stats_plan(N, K, gsh_rows, workspace ? (size_t)workspace_bytes : 0);
  const int64_t tiles = (N + plan_cw(p) - 1) / plan_cw(p);
  if (tiles > kMaxRowStats)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_matmul_residual_stats: %lld column tiles exceed %d partials",
                     (long long)tiles, kMaxRowStats);
  const W4Args a{(const half_t*)x, K, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)h_out, N, 1, (int)N, (int)K, gsh_rows};
  const ProArgs pa{(const half_t*)residual, nullptr, nullptr, 0.0f, row_stats, (int)tiles};
  return launch_plan(a, p, workspace, (hipStream_t)stream, kEpiResStat, pa);
}

// The o projection of a decode layer straight from the decode attention's per-range partials
// (left by ldk_decode_attention_ranges for nq heads over a cache of max_len positions in ranges of
// rlen, at the position *pos): x is merged in the x staging (kProAttnStat), then as
// ldk_w4a16_matmul_residual_stats: h_out = fp16(x W^T (+ bias) + residual) and the per-tile sums
// of h^2 in row_stats for ldk_w4a16_rmsnorm_stats_matmul. One launch where the attention's merge
// launch and the projection were two. K = nq * 128, at most 4 ranges, group size 128.
extern "C" int ldk_w4a16_attn_matmul_residual_stats(const int64_t* pos, int64_t max_len, int64_t rlen, int nq,
                                                    const void* residual, void* h_out, float* row_stats,
                                                    const int32_t* qweight, const void* scales, const void* zeros,
                                                    const void* bias, int64_t N, int64_t K, int group_size,
                                                    void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "w4a16_attn_matmul_residual_stats";
  if (!pos || !residual || !row_stats) return ldk::fail(LDK_ERR_INVALID, "%s: null pos, residual or row_stats", fn);
  int gsh_rows = 0;
  int st = validate(fn, residual, K, qweight, scales, zeros, h_out, N, 1, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (nq <= 0 || nq > ldk::kAttnMaxHeads || K != (int64_t)nq * ldk::kAttnHeadDim)
    return ldk::fail(LDK_ERR_INVALID, "%s: K=%lld must be nq * 128 with 1 <= nq <= %d", fn, (long long)K, ldk::kAttnMaxHeads);
  if (gsh_rows != 4) return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: group_size %d (the fused prologues take 128)", fn, group_size);
  if (max_len <= 0 || rlen <= 0 || rlen % 32 || (max_len + rlen - 1) / rlen > kAttnRanges || max_len > INT32_MAX)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: max_len=%lld in ranges of rlen=%lld (a multiple of 32) must give 1..%d ranges",
                     fn, (long long)max_len, (long long)rlen, kAttnRanges);
  if (!ldk::aligned(pos, 8) || !ldk::aligned(h_out, 8) || !ldk::aligned(row_stats, 4))
    return ldk::fail(LDK_ERR_ALIGN, "%s: pos and h_out 8-byte, row_stats 4-byte aligned", fn);
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "%s: workspace must be a 256-byte aligned pointer", fn);
  const float *po = nullptr, *pm = nullptr;
  st = ldk::attention_partials(fn, stream, pos, max_len, rlen, nq, &po, &pm);
  if (st) return st;
  const Plan p = residual_stats_plan(N, K, gsh_rows, workspace ? (size_t)workspace_bytes : 0);
  const int64_t tiles = (N + plan_cw(p) - 1) / plan_cw(p);
  if (tiles > kMaxRowStats)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "%s: %lld column tiles exceed %d partials", fn, (long long)tiles, kMaxRowStats);
  const W4Args a{(const half_t*)residual, K, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)h_out, N, 1, (int)N, (int)K, gsh_rows};
  const ProArgs pa{(const half_t*)residual, nullptr, nullptr, 0.0f, row_stats, (int)tiles, po, pm, pos, (int)max_len,
                   (int)rlen};
  return launch_plan(a, p, workspace, (hipStream_t)stream, kProAttnStat, pa);
}

extern "C" int ldk_w4a16_rmsnorm_stats_matmul(const void* h, const float* row_stats, int nstats, const void* norm_weight,
                                              float eps, const int32_t* qweight, const void* scales, const void* zeros,
                                              const void* bias, void* out, int64_t N, int64_t K, int group_size,
                                              void* workspace, int64_t workspace_bytes, void* stream) {
  int gsh_rows = 0;
  int st = validate("w4a16_rmsnorm_stats_matmul", h, K, qweight, scales, zeros, out, N, 1, N, K, group_size, &gsh_rows);
  if (st) return st;
  if (!row_stats || !norm_weight) return ldk::fail(LDK_ERR_INVALID, "w4a16_rmsnorm_stats_matmul: null row_stats or norm_weight");
  if (nstats <= 0 || nstats > kMaxRowStats)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w4a16_rmsnorm_stats_matmul: nstats=%d outside 1..%d", nstats, kMaxRowStats);
  if (!ldk::aligned(norm_weight, 16) || !ldk::aligned(row_stats, 4))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_rmsnorm_stats_matmul: norm_weight 16-byte, row_stats 4-byte aligned");
  if (workspace_bytes && (!workspace || !ldk::aligned(workspace, 256)))
    return ldk::fail(LDK_ERR_ALIGN, "w4a16_rmsnorm_stats_matmul: workspace must be a 256-byte aligned pointer");
  const Plan p = make_plan(1, N, K, gsh_rows, 0, 0, 0, workspace ? (size_t)workspace_bytes : 0);
  const W4Args a{(const half_t*)h, K, (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros,
                 (const half_t*)bias, (half_t*)out, N, 1, (int)N, (int)K, gsh_rows};
  const ProArgs pa{nullptr, nullptr, (const half_t*)norm_weight, eps, const_cast<float*>(row_stats), nstats};
  return launch_plan(a, p, workspace, (hipStream_t)stream, kProRmsPre, pa);
}
