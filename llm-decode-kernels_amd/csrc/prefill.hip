// Prefill weight-only GEMMs: y[M, N] = x[M, K] @ W^T (+ bias) for many rows, on the matrix cores
// of gfx950 (v_mfma_f32_16x16x32_f16), for two weight formats:
//  * int4 (W4A16): the reference's counterpart is its Triton tensor-core GEMM for prefill rows
//    (kernels/w4a16.py:31-97, routed at w4a16.py:264-268,328-329), which dequantizes each weight
//    tile to fp16 and runs tl.dot with fp32 accumulation. Same numerics here: every weight is
//    dequantized exactly as dequantize_ref does it (kernels/reference.py:27-36, one fp16 rounding
//    of (q - z) * s), products accumulate in fp32, the output is rounded once.
//  * e4m3 (W8A16): the reference's _w8a16_kernel (kernels/fp8.py:42-91, run for prefill rows at
//    fp8.py:221-222) converts the fp8 tile to fp16 (exact: every e4m3fn value is an fp16 value),
//    accumulates tl.dot in fp32 and multiplies by the column scale after the K loop, then adds the
//    bias. Same order here.
//
// Work decomposition (one workgroup per BM x BN output tile, all of K or one split of it):
//  * BN = 64 * WAVES columns. Wave w owns 64 of them for all BM rows, so each wave loads and
//    decodes only its own weights (no decode is repeated across waves), and x is the operand the
//    waves share, through LDS.
//  * MFMA B operand: lane l = (c16 = l % 16, kb = l / 16) supplies 8 consecutive K of four columns
//    n0 + 4 * c16 + j (j < 4); column j feeds 16-column tile j, whose column c16 is that column.
//  * int4 weights: 16 bytes of packed row 4 * sub + kb at those 4 columns are the lane's 4 words,
//    each 8 consecutive K of one column. Nibbles are decoded with the fp16 magic-number trick
//    ((w & 0x000F000F) | 0x6400 -> 1024 + q per half, pairs (q0, q4) .. (q3, q7)); then
//    (1024 + q) - (1024 + z) is exact, one packed fp16 multiply by s rounds once, and four
//    v_perm_b32 put the eight halves in K order (q0, q1) .. (q6, q7).
//  * e4m3 weights ([K, N], N contiguous): the wave's stage tile is 64 K rows x 64 bytes. The lane
//    reads one dword (its 4 columns) from each of its 8 K rows, a 4 x 4 byte transpose (8
//    v_perm_b32 per 4 rows) gives each column its K-ordered bytes, and
//    v_cvt_scalef32_pk_f16_fp8 (scale 1.0) turns two bytes into two exact fp16 halves. K row r is
//    stored at tile row r ^ ((r / 8) % 4): the four lane groups kb read rows 8 kb + i, which then
//    sit in four different 16-bank quarters of LDS instead of all in the same one.
//  * Pipeline: an S-stage ring of K-steps of 64, each stage a distinct LDS array holding the
//    x tile (BM rows x 128 bytes) and every wave's weight bytes (and, for int4, the scales and
//    zeros of the step's group). All of it is loaded with gfx950's 16-byte loads to LDS
//    (buffer_load ... lds: lane i writes base + 16 i), so S - 1 stages are in flight without
//    holding registers. x chunks are stored XOR-swizzled (chunk c of row r at slot c ^ (r % 8)),
//    so the 8 rows an MFMA A operand reads per LDS phase fall in distinct banks; rows past M are
//    buffer loads past the resource, which write zeros. Each step waits (explicit vmcnt) for its
//    own stage only, then one barrier, then issues stage ks + S - 1 into the slot all waves
//    finished reading before that barrier. The loop is unrolled by S so every slot is a fixed
//    array: the compiler then needs no conservative waits on the LDS reads.
#include <algorithm>
#include <cstdint>
#include <cstdio>

#include "prefill.h"

namespace {

using ldk::WFmt;

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

constexpr int kStep = 64;                 // K per pipeline stage (two MFMA K-substeps of 32)
constexpr int kXRow = kStep * 2;          // bytes of one x row of a stage
constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// s_waitcnt vmcnt(N): at most N vector-memory loads of this wave still outstanding. Loads complete
// in issue order for this count, so it waits for every load issued before the last N. The builtin
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left open) is what the
// compiler's own wait insertion reads, so it knows the older stages are complete and adds no wait
// of its own before their LDS reads; the empty asm with a memory clobber on each side keeps the
// compiler from moving any load or LDS access across it, which the count relies on.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" : : : "memory");
}

// The e4m3 epilogue's scaled accumulators are fp32 values, then the bias is added in fp32, then
// the sum is rounded to fp16 (the split-K reduction's steps). Without this the compiler may
// contract the three into one v_fma_mixlo_f16, a single rounding, in some kernels and not others.
__device__ __forceinline__ void pin_f32(float4_t& v) { asm volatile("" : "+v"(v)); }

// Workgroup barrier that is also a compiler memory barrier, without the vmcnt(0) a C++ fence adds
// (the ring keeps later stages' loads in flight across it).
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" : : : "memory");
}

// 16-byte buffer loads to LDS (lane i writes lds_base + 16 i), issued as inline asm: the
// compiler's wait insertion then does not track them, so it adds no conservative vmcnt wait before
// the LDS reads of other stages (it would after the loop's back edge, where it no longer knows
// which LDS array each pending load writes); the ring's own vmcnt waits order them. M0 holds the
// LDS base for the load; the asm restores M0's previous value itself (M0 is reserved to the
// compiler, which does not save a clobbered M0). An LDS DMA that reads M0 right after an SALU
// write of it needs one wait state on gfx9-family chips (gfx950 included); the compiler's hazard
// recognizer inserts it for its own M0 writes but cannot see inside this asm string, so the string
// carries its own s_nop 0. The address is base + voffset + soffset; only
// voffset is checked against the
// resource's size, so every load that relies on the check (x rows past M, scales past N) keeps
// its whole offset in voffset, and soffset carries only the uniform K-step offset of loads that
// stay inside their arrays.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma_buffer16(u32x4 rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds_base) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %4 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voffset), "s"(rsrc), "s"(lds_base), "s"(soffset)
               : "memory");
}
// Raw buffer descriptor over [p, p + bytes): a load at an offset past it returns zeros (and, to
// LDS, writes zeros).
__device__ __forceinline__ u32x4 raw_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// Two fp16 halves from bytes (0, 1) (HI = false) or (2, 3) of an e4m3fn word, exact.
template <bool HI>
__device__ __forceinline__ uint32_t e4m3_pair(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

// Byte transpose of four words r0..r3 (byte j of r_i = column j at K row i) into col[j] = the K
// rows 0..3 of column j, in K order.
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t* col) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0[0] r1[0] r0[1] r1[1]
  const uint32_t ab_hi = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0[2] r1[2] r0[3] r1[3]
  const uint32_t cd_lo = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
  const uint32_t cd_hi = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
  col[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // r0[0] r1[0] r2[0] r3[0]
  col[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
  col[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  col[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

template <WFmt F>
struct Fmt;
template <>
struct Fmt<WFmt::kInt4> {
  static constexpr int WBYTES = 2048;  // per wave and stage: 8 packed rows x 64 columns x 4 bytes
  static constexpr int WI = 2;         // weight load instructions per wave and stage
  static constexpr int SZBYTES = 256;  // scales (128 bytes) and zeros of the wave's 64 columns
  static constexpr int SZI = 2;
};
template <>
struct Fmt<WFmt::kE4M3> {
  static constexpr int WBYTES = 4096;  // 64 K rows x 64 columns x 1 byte
  static constexpr int WI = 4;
  static constexpr int SZBYTES = 0;    // column scales are applied after the K loop
  static constexpr int SZI = 0;
};

template <WFmt F, int WAVES, int MT, int S>
struct GemmCfg {
  using T = Fmt<F>;
  static constexpr int BM = 16 * MT, NT = 4, NTHR = WAVES * 64;
  static constexpr int XI = BM / 8 / WAVES;  // x load instructions per wave and stage (8 rows each)
  static constexpr int XBYTES = BM * kXRow;
  static constexpr int WOFF = XBYTES;                          // weights, T::WBYTES per wave
  static constexpr int SZOFF = WOFF + WAVES * T::WBYTES;       // int4 scales and zeros per wave
  static constexpr int STAGE = SZOFF + WAVES * T::SZBYTES;
  static constexpr int LOADS = XI + T::WI + T::SZI;            // per wave and stage
  static_assert(XI * WAVES * 8 == BM, "whole x load instructions");
  static_assert(S * STAGE <= 160 * 1024, "LDS");
};

// KG wave groups per workgroup split the workgroup's K range in two halves (KG = 2): each group of
// WAVES waves walks its half through its own ring (the second half of every stage array), and the
// groups' accumulators meet in LDS at the end. That doubles the waves on a tile without the fp32
// partials in memory that a split over workgroups costs.
template <WFmt F, int WAVES, int MT, int S, int KG, bool SW>
__device__ __forceinline__ void gemm_body(const ldk::GemmArgs& a, int kps, float* partial, int mfast) {
  using C = GemmCfg<F, WAVES, MT, S>;
  using T = Fmt<F>;
  constexpr bool kInt4 = F == WFmt::kInt4;
  constexpr int BM = C::BM, NT = C::NT;
  static_assert(S >= 2 && S <= 4, "ring of 2 to 4 stages");
  static_assert(KG == 1 || KG == 2, "one or two K groups");
  static_assert(KG * S * C::STAGE <= 160 * 1024, "LDS");
  // the K groups' accumulators meet in st0 (tiles t < MH) and st1 (the rest)
  constexpr int MH = MT > 1 ? MT / 2 : 1;
  static_assert(KG == 1 || WAVES * MH * NT * 64 * 16 <= KG * C::STAGE, "reduction fits two stage slots");
  constexpr int SLOT = KG * C::STAGE;
  __shared__ __align__(16) unsigned char st0[SLOT], st1[SLOT], st2[S >= 3 ? SLOT : 16], st3[S == 4 ? SLOT : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases go to M0
  const int wave = KG == 1 ? wid : wid % WAVES;               // column group
  const int kg = KG == 1 ? 0 : wid / WAVES;                   // K group
  const int gofs = kg * C::STAGE;                             // the K group's part of a stage slot
  const int c16 = lane & 15, kb = lane >> 4;
  // mfast: the grid's x dimension walks the row tiles, so consecutive workgroups (which the
  // dispatcher deals round-robin to the 8 XCDs) share a column tile, and each XCD keeps a fixed
  // subset of the row tiles: its slice of x stays in its L2 and each weight tile it reads serves
  // all of its row tiles. Otherwise x walks the column tiles.
  const int bn = mfast ? blockIdx.y : blockIdx.x, bm = mfast ? blockIdx.x : blockIdx.y;
  // SwiGLU fused (SW, a.swiglu): column groups [0, WAVES/2) take g columns, the others the
  // matching u columns N/2 further on
  static_assert(!SW || (WAVES >= 2 && WAVES % 2 == 0), "SwiGLU pairs column groups");
  constexpr int HW = WAVES / 2;
  const bool up = SW && wave >= HW;
  const int n0 = !SW ? bn * (64 * WAVES) + 64 * wave
                     : (up ? a.N / 2 : 0) + bn * (64 * HW) + 64 * (up ? wave - HW : wave);
  const int m0 = bm * BM;
  const int mrows = min(a.M - m0, BM);
  // K-steps [kbeg, kbeg + nks) of split blockIdx.z; K group g takes [kbeg + g h, + gn) of them
  const int kbeg0 = blockIdx.z * kps;
  const int nks = min(a.K / kStep - kbeg0, kps);
  const int h = (nks + KG - 1) / KG;  // steps every wave walks (the ring's barriers are workgroup-wide)
  const int kbeg = kbeg0 + kg * h;
  const int gn = max(0, min(h, nks - kg * h));
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.w);

  // x: instruction i of this wave covers rows r0 = 8 (XI * wave + i) .. + 7; lane l takes row
  // r0 + l / 8, slot l % 8, which holds chunk (l % 8) ^ (row % 8) of that row
  const u32x4 xb = raw_rsrc(a.x + (int64_t)m0 * a.ldx, (uint32_t)((int64_t)(mrows - 1) * a.ldx * 2 + (int64_t)a.K * 2));
  uint32_t xoff[C::XI];
#pragma unroll
  for (int i = 0; i < C::XI; ++i) {
    const int row = 8 * (C::XI * wave + i) + (lane >> 3), chunk = (lane & 7) ^ (row & 7);
    xoff[i] = row < mrows ? (uint32_t)((int64_t)row * a.ldx * 2 + chunk * 16) : 0x80000000u;
  }

  // weights: per-lane offsets of the first K-step, plus wstep bytes per K-step (in soffset).
  // Columns are clamped so lanes past N read valid memory; their outputs are not stored.
  const u32x4 wb = raw_rsrc(a.w, (uint32_t)(kInt4 ? (int64_t)a.K / 2 * a.N : (int64_t)a.K * a.N));
  uint32_t woff[T::WI];
  uint32_t wstep;
  if constexpr (kInt4) {
    // instruction sub: lane (c16, kb) takes packed row 4 sub + kb at columns n0 + 4 c16 .. + 3
    const int col = min(n0 + 4 * c16, a.N - 4);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) woff[sub] = 4u * (uint32_t)((int64_t)(4 * sub + kb) * a.N + col);
    wstep = 32u * (uint32_t)a.N;  // 8 packed rows
  } else {
    // instruction i fills tile rows 16 i .. + 15: lane l writes tile row 16 i + l / 4, 16-byte
    // chunk l % 4, from K row (tile row) ^ ((tile row / 8) % 4) of the step
    const int wcol = min(n0 + 16 * (lane & 3), a.N - 16);
#pragma unroll
    for (int i = 0; i < T::WI; ++i) {
      const int tr = 16 * i + (lane >> 2), r = tr ^ ((tr >> 3) & 3);
      woff[i] = (uint32_t)r * (uint32_t)a.N + (uint32_t)wcol;
    }
    wstep = 64u * (uint32_t)a.N;
  }

  // int4 scales and zeros of a stage: lanes 0-7 each take 16 bytes (8 columns) of the wave's 64;
  // past N (and past the arrays) zeros
  const int gsh = kInt4 ? __builtin_ctz(a.group_size) - 6 : 0;  // log2(K-steps per group)
  const uint32_t szb = kInt4 ? (uint32_t)(a.K / a.group_size) * (uint32_t)a.N * 2u : 0u;
  const u32x4 sb = raw_rsrc(a.s, szb), zb = raw_rsrc(a.z, szb);
  const uint32_t szoff = 2u * (uint32_t)(n0 + 8 * (lane & 7));

  auto issue = [&](unsigned char* stage, int kstep) {
    const int ks = kbeg + kstep;
#pragma unroll
    for (int i = 0; i < C::XI; ++i)
      dma_buffer16(xb, xoff[i], (uint32_t)(ks * kXRow), lds_addr(stage + 8 * (C::XI * wave + i) * kXRow));
#pragma unroll
    for (int i = 0; i < T::WI; ++i)
      dma_buffer16(wb, woff[i], (uint32_t)ks * wstep, lds_addr(stage + C::WOFF + T::WBYTES * wave + 1024 * i));
    if constexpr (kInt4) {
      const uint32_t g = 2u * (uint32_t)(ks >> gsh) * (uint32_t)a.N;
      if (lane < 8) {  // one instruction each; lanes 8-63 idle (every wave has lanes 0-7 active)
        dma_buffer16(sb, g + szoff, 0u, lds_addr(stage + C::SZOFF + 256 * wave));
        dma_buffer16(zb, g + szoff, 0u, lds_addr(stage + C::SZOFF + 256 * wave + 128));
      }
    }
  };

  float4_t acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[t][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>();
  // e4m3: byte offset of K row 8 kb + i (i < 4; rows i + 4 are 256 bytes further) of the lane's
  // group in a K-substep's 32 rows, at the lane's 4 columns
  uint32_t roff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) roff[i] = (uint32_t)(512 * kb + 64 * (i ^ kb) + 4 * c16);

  auto compute = [&](const unsigned char* stage) {
    half4_t s4, z4;
    if constexpr (kInt4) {
      s4 = *reinterpret_cast<const half4_t*>(stage + C::SZOFF + 256 * wave + 8 * c16);
      z4 = *reinterpret_cast<const half4_t*>(stage + C::SZOFF + 256 * wave + 128 + 8 * c16);
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      half8v B[NT];
      if constexpr (kInt4) {
        const u32x4 wq = *reinterpret_cast<const u32x4*>(stage + C::WOFF + 2048 * wave + 1024 * sub + 16 * lane);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const half_t zz = -((half_t)1024.0f + z4[j]);
          const half2_t zh = {zz, zz}, s2 = {s4[j], s4[j]};
          const uint32_t wc = wq[j];
          const uint32_t d0 = ldk::h22u((ldk::u2h2((wc & mlo) | magic) + zh) * s2);          // (q0, q4)
          const uint32_t d1 = ldk::h22u((ldk::u2h2(((wc >> 4) & mlo) | magic) + zh) * s2);   // (q1, q5)
          const uint32_t d2 = ldk::h22u((ldk::u2h2(((wc >> 8) & mlo) | magic) + zh) * s2);   // (q2, q6)
          const uint32_t d3 = ldk::h22u((ldk::u2h2(((wc >> 12) & mlo) | magic) + zh) * s2);  // (q3, q7)
          B[j] = __builtin_bit_cast(half8v, u32x4{perm_lo(d0, d1), perm_lo(d2, d3), perm_hi(d0, d1), perm_hi(d2, d3)});
        }
      } else {
        const unsigned char* wt = stage + C::WOFF + 4096 * wave + 2048 * sub;
        uint32_t r[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          r[i] = *reinterpret_cast<const uint32_t*>(wt + roff[i]);
          r[i + 4] = *reinterpret_cast<const uint32_t*>(wt + roff[i] + 256);
        }
        uint32_t lo[4], hi[4];  // column j: K rows 0-3 and 4-7 of the lane's 8
        transpose4x4(r[0], r[1], r[2], r[3], lo);
        transpose4x4(r[4], r[5], r[6], r[7], hi);
#pragma unroll
        for (int j = 0; j < NT; ++j)
          B[j] = __builtin_bit_cast(half8v, u32x4{e4m3_pair<false>(lo[j]), e4m3_pair<true>(lo[j]),
                                                  e4m3_pair<false>(hi[j]), e4m3_pair<true>(hi[j])});
      }
      const int slot = (4 * sub + kb) ^ (c16 & 7);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const half8v A = *reinterpret_cast<const half8v*>(stage + (16 * t + c16) * kXRow + 16 * slot);
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[j], acc[t][j], 0, 0, 0);
      }
    }
  };

  unsigned char* const stages[4] = {st0, st1, st2, st3};
#pragma unroll
  for (int i = 0; i < S - 1; ++i)
    if (i < gn) issue(stages[i] + gofs, i);

  // step ks reads slot I = ks % S and refills slot (I + S - 1) % S with stage ks + S - 1. A K
  // group with fewer steps than h (the second half of an odd count) still takes the barriers.
  auto step = [&](auto I_, int ks) {
    constexpr int I = decltype(I_)::value, J = (I + S - 1) % S;
    const int pend = min(S - 2, gn - 1 - ks);  // stages issued after ks that may stay in flight
    if (pend >= S - 2) wait_vm<C::LOADS * (S - 2)>();
    else if (S == 4 && pend == 1) wait_vm<C::LOADS * (S == 4 ? 1 : 0)>();
    else wait_vm<0>();
    ring_barrier();
    if (ks + S - 1 < gn) issue(stages[J] + gofs, ks + S - 1);
    if (KG == 1 || ks < gn) compute(stages[I] + gofs);
  };
  for (int ks = 0; ks < h; ks += S) {
    step(std::integral_constant<int, 0>{}, ks);
    if (ks + 1 < h) step(std::integral_constant<int, 1>{}, ks + 1);
    if constexpr (S >= 3)
      if (ks + 2 < h) step(std::integral_constant<int, 2>{}, ks + 2);
    if constexpr (S == 4)
      if (ks + 3 < h) step(std::integral_constant<int, 3>{}, ks + 3);
  }

  if constexpr (KG == 2) {
    // every wave is done with the rings (each group's last step waited for all of its loads):
    // group 1 leaves its accumulators in st0 / st1, lane-major, and group 0 adds them
    ring_barrier();
    float4_t* red0 = reinterpret_cast<float4_t*>(st0);
    float4_t* red1 = reinterpret_cast<float4_t*>(st1);
    if (kg == 1) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          (t < MH ? red0 : red1)[((wave * MH + t % MH) * NT + j) * 64 + lane] = acc[t][j];
    }
    ring_barrier();
    if (kg == 1) return;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[t][j] += (t < MH ? red0 : red1)[((wave * MH + t % MH) * NT + j) * 64 + lane];
  }

  if constexpr (SW) {
    {
      // every wave rounds its tile as the plain epilogue does (column scale, bias, fp16); the u
      // waves hand theirs to the g waves through LDS, lane for lane (the same rows and columns
      // of the pair), and the g waves store fp16(silu(g)) * u
      static_assert(MT * 4 * 64 * 8 <= SLOT, "a wave's fp16 tile fits one stage slot");
      const int c = n0 + 4 * c16;
      if constexpr (!kInt4) {  // the plain epilogue's steps: column scale, then bias, then fp16
        const float cs[4] = {(float)a.s[c], (float)a.s[c + 1], (float)a.s[c + 2], (float)a.s[c + 3]};
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            acc[t][j] *= cs[j];
            pin_f32(acc[t][j]);
          }
      }
      float4_t b4 = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      if (a.bias) b4 = float4_t{(float)a.bias[c], (float)a.bias[c + 1], (float)a.bias[c + 2], (float)a.bias[c + 3]};
      half4_t o[MT][4];
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[t][i] = half4_t{(half_t)(acc[t][0][i] + b4[0]), (half_t)(acc[t][1][i] + b4[1]), (half_t)(acc[t][2][i] + b4[2]),
                            (half_t)(acc[t][3][i] + b4[3])};
      ring_barrier();  // every wave is past its last read of the stage slots
      static_assert(HW <= 2, "the pairs' exchange slots are st0 and st1");
      static_assert(MT % 2 == 0, "the pair splits the row tiles");
      // the g wave finishes row tiles [0, MT/2) and the u wave [MT/2, MT): each hands the other
      // the half of its tile that the other finishes, so both waves evaluate silu and store
      constexpr int MH2 = MT / 2;
      half4_t* const xs = reinterpret_cast<half4_t*>((up ? wave - HW : wave) == 0 ? st0 : st1);
      half4_t* const to_u = xs;                 // g of tiles [MH2, MT)
      half4_t* const to_g = xs + MH2 * 4 * 64;  // u of tiles [0, MH2)
#pragma unroll
      for (int t = 0; t < MH2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (up)
            to_g[(t * 4 + i) * 64 + lane] = o[t][i];
          else
            to_u[(t * 4 + i) * 64 + lane] = o[MH2 + t][i];
        }
      ring_barrier();
      auto finish = [&](auto tb_) {
        constexpr int TB = decltype(tb_)::value;  // the first row tile this wave finishes
        const int co = TB ? c - a.N / 2 : c;      // the g column of the pair
        const half4_t* from = TB ? to_u : to_g;
#pragma unroll
        for (int t = 0; t < MH2; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * (TB + t) + 4 * kb + i;
            const half4_t mine = o[TB + t][i], other = from[(t * 4 + i) * 64 + lane];
            const half4_t g = TB ? other : mine, u = TB ? mine : other;
            half4_t v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = ldk::silu_f16(g[j]);
            if (r < mrows) *reinterpret_cast<half4_t*>(a.out + (int64_t)(m0 + r) * a.ldo + co) = v * u;  // fp16 multiply
          }
        }
      };
      if (up)
        finish(std::integral_constant<int, MH2>{});
      else
        finish(std::integral_constant<int, 0>{});
      return;
    }
  }

  // acc[t][j][i] is row 16t + 4kb + i of the tile, column n0 + 4 * c16 + j
  const int c = n0 + 4 * c16;
  if (c >= a.N) return;
  if (partial) {  // one split of K: fp32 partial tile [split][M][N], summed by gemm_reduce_kernel
    float* dst = partial + (int64_t)blockIdx.z * a.M * a.N;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * t + 4 * kb + i;
        if (r < mrows)
          *reinterpret_cast<float4_t*>(dst + (int64_t)(m0 + r) * a.N + c) =
              float4_t{acc[t][0][i], acc[t][1][i], acc[t][2][i], acc[t][3][i]};
      }
    return;
  }
  if constexpr (!kInt4) {  // column scales after the K reduction (fp8.py:80-81)
    const float cs[4] = {(float)a.s[c], (float)a.s[c + 1], (float)a.s[c + 2], (float)a.s[c + 3]};
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        acc[t][j] *= cs[j];
        pin_f32(acc[t][j]);
      }
  }
  float4_t b4 = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (a.bias) b4 = float4_t{(float)a.bias[c], (float)a.bias[c + 1], (float)a.bias[c + 2], (float)a.bias[c + 3]};
#pragma unroll
  for (int t = 0; t < MT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * t + 4 * kb + i;
      if (r < mrows) {
        const half4_t o{(half_t)(acc[t][0][i] + b4[0]), (half_t)(acc[t][1][i] + b4[1]), (half_t)(acc[t][2][i] + b4[2]),
                        (half_t)(acc[t][3][i] + b4[3])};
        *reinterpret_cast<half4_t*>(a.out + (int64_t)(m0 + r) * a.ldo + c) = o;
      }
    }
  }
}

template <int WAVES, int MT, int S, int KG>
__global__ __launch_bounds__(WAVES * KG * 64) __attribute__((amdgpu_waves_per_eu(2))) void w4a16_gemm_kernel(
    ldk::GemmArgs a, int kps, float* partial, int mfast) {
  gemm_body<WFmt::kInt4, WAVES, MT, S, KG, false>(a, kps, partial, mfast);
}

template <int WAVES, int MT, int S, int KG>
__global__ __launch_bounds__(WAVES * KG * 64) __attribute__((amdgpu_waves_per_eu(2))) void w8a16_gemm_kernel(
    ldk::GemmArgs a, int kps, float* partial, int mfast) {
  gemm_body<WFmt::kE4M3, WAVES, MT, S, KG, false>(a, kps, partial, mfast);
}

// The same GEMMs with SwiGLU in the epilogue (GemmArgs::swiglu; no K split).
template <int WAVES, int MT, int S, int KG>
__global__ __launch_bounds__(WAVES * KG * 64) __attribute__((amdgpu_waves_per_eu(2))) void w4a16_gemm_swiglu_kernel(
    ldk::GemmArgs a, int kps, int mfast) {
  gemm_body<WFmt::kInt4, WAVES, MT, S, KG, true>(a, kps, nullptr, mfast);
}

template <int WAVES, int MT, int S, int KG>
__global__ __launch_bounds__(WAVES * KG * 64) __attribute__((amdgpu_waves_per_eu(2))) void w8a16_gemm_swiglu_kernel(
    ldk::GemmArgs a, int kps, int mfast) {
  gemm_body<WFmt::kE4M3, WAVES, MT, S, KG, true>(a, kps, nullptr, mfast);
}

// Tiles that take the SwiGLU epilogue: paired column groups, and at most 4 row tiles (the 8-row-tile
// accumulators leave no registers for the rounded pair)
constexpr bool swiglu_tile(int waves, int mt) { return waves >= 2 && waves % 2 == 0 && mt <= 4; }

// y[m, n] = fp16(sum over splits of partial[split][m][n] (x colscale[n]) (+ bias[n])), the splits
// added in index order (the result does not depend on which split finished first). 4 columns per
// thread. Every partial read is written back to zero: the workspace is zero between calls, which
// the decode kernels' split-K accumulators rely on.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(float* partial, int splits, const half_t* colscale,
                                                          const half_t* bias, half_t* out, int64_t ldo, int M, int N) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // quad of columns
  const int nq = N / 4;
  if (q >= (int64_t)M * nq) return;
  const int m = (int)(q / nq), n = 4 * (int)(q - (int64_t)m * nq);
  const int64_t plane = (int64_t)M * N;
  float4_t* p0 = reinterpret_cast<float4_t*>(partial + (int64_t)m * N + n);
  float4_t v = *p0;
  *p0 = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int z = 1; z < splits; ++z) {
    float4_t* pz = reinterpret_cast<float4_t*>(partial + z * plane + (int64_t)m * N + n);
    v += *pz;
    *pz = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  if (colscale) v *= float4_t{(float)colscale[n], (float)colscale[n + 1], (float)colscale[n + 2], (float)colscale[n + 3]};
  if (bias) v += float4_t{(float)bias[n], (float)bias[n + 1], (float)bias[n + 2], (float)bias[n + 3]};
  *reinterpret_cast<half4_t*>(out + (int64_t)m * ldo + n) = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Tile shape, K groups and K split per problem. From graph-timed sweeps on MI355X over the
// Qwen2.5-1.5B shapes (M = 512 / 1024 / 2048, int4 and e4m3):
//  * Long K: the largest tile whose split grid still gives most CUs a workgroup, with the split
//    count that balances the CUs (below): down M = 2048 on 128 x 256 tiles split 5 ways (int4
//    75 us, e4m3 74 us, against 90 / 81 us on 64-row tiles).
//  * Short K: 128 x 256 tiles when they give at least 384 workgroups (gate_up M = 2048: int4
//    117 us, e4m3 114 us); otherwise 64-row tiles on the widest workgroup (4, 2 or 1 column groups)
//    that still gives most CUs one and, with two K groups, leaves LDS for two per CU (qkv M = 2048
//    on 4 x 64 columns and two K groups: int4 20 us, against 29 us on one K group and 28 us for
//    dequantize + hipBLASLt); where that leaves one column group, 32-row tiles on two.
//  * Two K groups when a short-K shape leaves fewer than two waves per SIMD (e4m3: one); long K
//    splits over workgroups instead (the partials of few rows are cheap).
struct GemmShape {
  int waves, mt, kg, splits;
  int mfast;  // grid x walks the row tiles (see gemm_body)
};

constexpr int kLongK = 48;  // K-steps of 64 from which a shape counts as long

// Ring depth per format and shape, from the same sweeps: a third stage on the 2 x 8 tiles costs the
// registers of a second workgroup per CU (occupancy 1) and loses; one column group with two K
// groups gains from a third stage, which its small LDS footprint leaves room for.
constexpr int stages_of(WFmt f, int waves, int mt, int kg) {
  return waves == 4 && mt == 8 ? (f == WFmt::kInt4 ? 3 : 2) : (waves == 1 && kg == 2) || mt <= 2 ? 3 : 2;
}

// LDS of a workgroup: KG rings of S stages (x tile, weights, int4 scales and zeros).
constexpr int lds_of(WFmt f, int waves, int mt, int kg) {
  return kg * stages_of(f, waves, mt, kg) *
         (16 * mt * kXRow + waves * (f == WFmt::kInt4 ? Fmt<WFmt::kInt4>::WBYTES + Fmt<WFmt::kInt4>::SZBYTES
                                                        : Fmt<WFmt::kE4M3>::WBYTES));
}

GemmShape pick_shape(WFmt f, int64_t M, int64_t N, int64_t K, int block_n, int split_k, int64_t ws_bytes) {
  const int64_t steps = K / kStep;
  const bool long_k = steps >= kLongK;
  auto tiles = [&](int waves, int mt) { return ((N + 64 * waves - 1) / (64 * waves)) * ((M + 16 * mt - 1) / (16 * mt)); };
  // K split (long K, or split_k), as far as the workspace holds the fp32 partials: the count that
  // minimises the busiest CU's share of the work, ceil(t s / 256) / s for t tiles (one or two
  // workgroups per CU run at once), at most 6 ways and 8 K-steps per split. down M = 1024 on
  // 48 tiles: 5 splits (240 workgroups, one per CU) 47.6 us, 6 splits (288: 32 CUs with two)
  // 51.0 us (int4).
  auto splits = [&](int64_t t) {
    const int64_t room = std::max<int64_t>(1, std::min<int64_t>(64, ws_bytes / (M * N * 4)));
    if (split_k > 0) return (int)std::min<int64_t>(std::min<int64_t>(split_k, steps), room);
    if (!long_k) return 1;
    const int64_t most = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(6, steps / 8), room));
    int64_t best = 1;
    for (int64_t sp = 2; sp <= most; ++sp)  // ceil(t sp / 256) / sp < ceil(t best / 256) / best
      if (((t * sp + 255) / 256) * best < ((t * best + 255) / 256) * sp) best = sp;
    return (int)best;
  };
  // long K with at least 16 row tiles: row tiles on the grid's fast axis (down M = 1024 / 2048:
  // int4 53.6 -> 51.6 / 80.0 -> 76.7 us, e4m3 50.7 -> 49.8 / 78.2 -> 75.2 us; on the short-K
  // shapes it helped or hurt by a few percent either way, and at 8 row tiles it lost 13%)
  auto mfast = [&](int mt) { return long_k && (M + 16 * mt - 1) / (16 * mt) >= 16 ? 1 : 0; };
  if (block_n == 256) return {4, 8, 1, splits(tiles(4, 8)), 0};
  if (block_n == 128) {
    const int mt = tiles(2, 8) >= 512 ? 8 : 4;
    return {2, mt, 1, splits(tiles(2, mt)), 0};
  }
  if (long_k) {  // the largest tile whose split grid still gives most CUs a workgroup
    for (int w : {4, 2, 1})
      for (int mt : {8, 4}) {
        if (w != 4 && mt == 8) continue;
        const int64_t t = tiles(w, mt);
        const int sp = splits(t);
        if (t * sp >= 192 || (w == 1 && mt == 4)) return {w, mt, 1, sp, mfast(mt)};
      }
  }
  if (tiles(4, 8) >= 384) return {4, 8, 1, 1, 0};
  for (int w : {4, 2, 1}) {
    const int64_t t = tiles(w, 4);
    // e4m3 takes two K groups only below half as many waves: its 4-wave two-group tiles do not
    // fit the LDS, and the 2-wave ones lost to one group from 256 rows (gate_up M = 256 / 384:
    // 28.7 / 34.9 us on 2 x 64 columns in two groups, 24.9 / 28.3 on 4 x 64 in one)
    const int kg = split_k <= 0 && t * w < (f == WFmt::kE4M3 ? 1025 : 2048) && steps >= 16 ? 2 : 1;
    if (w > 1 && !(t >= 192 && lds_of(f, w, 4, kg) <= 80 * 1024)) continue;
    // 4-wave two-group tiles (two workgroups per CU) on 257-383 tiles leave some CUs a second
    // workgroup after the others are done; 2-wave tiles spread twice the workgroups evenly
    // (int4 gate_up M = 256 / 320: 30.1 / 31.0 -> 26.5 / 27.9 us; M = 192 (210 tiles) and
    // 384 (420) keep the 4-wave tiles: 19.2 against 20.7, 32.7 against 35.2)
    if (w == 4 && kg == 2 && t > 256 && t < 384) continue;
    // one column group of 64-row tiles: 32-row tiles on two column groups instead (qkv M = 512:
    // 10.5 against 12.7 us int4, 10.4 against 12.1 us e4m3; e4m3 qkv / o at M = 65-256, 48-128
    // tiles: 9.3-10.1 against 11.8-12.2 us; gate_up at M = 17-64 from the 32-row blocks: e4m3
    // 16.9 / 20.3 / 29.7 -> 10.9 / 11.2 / 15.5 us at M = 17 / 32 / 64, int4 12.0 -> 10.5 at 32)
    if (w == 1 && kg == 2) return {2, 2, 2, 1, 0};
    return {w, 4, kg, splits(t), 0};
  }
  return {1, 4, 1, 1, 0};  // not reached
}

template <WFmt F, int WAVES, int MT, int KG, int S = stages_of(F, WAVES, MT, KG)>
int launch(const ldk::GemmArgs& a, int splits, int mfast, hipStream_t s) {
  const int64_t tn = (a.N + 64 * WAVES - 1) / (64 * WAVES), tm = (a.M + 16 * MT - 1) / (16 * MT);
  const int steps = a.K / kStep, kps = (steps + splits - 1) / splits;
  const int nz = (steps + kps - 1) / kps;  // splits actually used (none empty)
  float* partial = nz > 1 ? static_cast<float*>(a.workspace) : nullptr;
  if (tn > 65535) mfast = 0;  // the column tiles then stay in the grid's x dimension
  const dim3 grid = mfast ? dim3((unsigned)tm, (unsigned)tn, (unsigned)nz) : dim3((unsigned)tn, (unsigned)tm, (unsigned)nz);
  (void)hipGetLastError();
  if constexpr (swiglu_tile(WAVES, MT)) {
    if (a.swiglu) {  // gemm_launch has checked the plan: no K split
      if constexpr (F == WFmt::kInt4)
        w4a16_gemm_swiglu_kernel<WAVES, MT, S, KG><<<grid, WAVES * KG * 64, 0, s>>>(a, kps, mfast);
      else
        w8a16_gemm_swiglu_kernel<WAVES, MT, S, KG><<<grid, WAVES * KG * 64, 0, s>>>(a, kps, mfast);
      return ldk::check_launch(F == WFmt::kInt4 ? "w4a16_gemm_swiglu" : "w8a16_gemm_swiglu");
    }
  }
  if (a.swiglu) return ldk::fail(LDK_ERR_UNSUPPORTED, "gemm: SwiGLU epilogue not built for %d x %d tiles", WAVES, MT);
  if constexpr (F == WFmt::kInt4)
    w4a16_gemm_kernel<WAVES, MT, S, KG><<<grid, WAVES * KG * 64, 0, s>>>(a, kps, partial, mfast);
  else
    w8a16_gemm_kernel<WAVES, MT, S, KG><<<grid, WAVES * KG * 64, 0, s>>>(a, kps, partial, mfast);
  int st = ldk::check_launch(F == WFmt::kInt4 ? "w4a16_gemm" : "w8a16_gemm");
  if (st || nz == 1) return st;
  const int64_t quads = (int64_t)a.M * (a.N / 4);
  const half_t* colscale = F == WFmt::kE4M3 ? a.s : nullptr;
  gemm_reduce_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>(partial, nz, colscale, a.bias, a.out, a.ldo, a.M, a.N);
  return ldk::check_launch("gemm_reduce");
}

GemmShape shape_for(WFmt f, const ldk::GemmArgs& a) {
  return pick_shape(f, a.M, a.N, a.K, a.block_n, a.split_k, a.workspace ? a.workspace_bytes : 0);
}

template <WFmt F>
int launch_fmt(const ldk::GemmArgs& a, hipStream_t s) {
  const GemmShape sh = shape_for(F, a);
  switch (sh.waves * 100 + sh.mt * 10 + sh.kg) {
    case 481: return launch<F, 4, 8, 1>(a, sh.splits, sh.mfast, s);
    case 281: return launch<F, 2, 8, 1>(a, sh.splits, sh.mfast, s);
    case 441: return launch<F, 4, 4, 1>(a, sh.splits, sh.mfast, s);
    case 442: return launch<F, 4, 4, 2>(a, sh.splits, sh.mfast, s);
    case 241: return launch<F, 2, 4, 1>(a, sh.splits, sh.mfast, s);
    case 242: return launch<F, 2, 4, 2>(a, sh.splits, sh.mfast, s);
    case 141: return launch<F, 1, 4, 1>(a, sh.splits, sh.mfast, s);
    case 142: return launch<F, 1, 4, 2>(a, sh.splits, sh.mfast, s);
    case 222: return launch<F, 2, 2, 2>(a, sh.splits, sh.mfast, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "gemm: shape %d x %d with %d K groups not instantiated", sh.waves, sh.mt, sh.kg);
}

}  // namespace

namespace ldk {

bool gemm_supported(WFmt f, int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx) {
  if (M <= 0 || N <= 0 || K <= 0 || K % kStep) return false;
  if (f == WFmt::kInt4) {
    if (group_size < kStep || (group_size & (group_size - 1)) || K % group_size || N % 8) return false;
    // scales and zeros are read through 32-bit buffer offsets
    if ((K / group_size) * N * 2 >= (int64_t(1) << 31)) return false;
  } else if (N % 16) {
    return false;
  }
  if ((M + 63) / 64 > 65535 || (M * (N / 4) + 255) / 256 > INT32_MAX) return false;
  // the x resource of one row tile spans less than 2 GiB
  if ((int64_t)127 * ldx * 2 + K * 2 >= (int64_t(1) << 31)) return false;
  // the weights are one buffer resource (32-bit size and offsets)
  const int64_t wbytes = f == WFmt::kInt4 ? K / 2 * N : K * N;
  return wbytes <= (int64_t)UINT32_MAX && N <= INT32_MAX / 64;
}

int gemm_launch(WFmt f, const GemmArgs& a, hipStream_t s) {
  const char* fn = f == WFmt::kInt4 ? "w4a16_gemm" : "w8a16_gemm";
  if (!gemm_supported(f, a.M, a.N, a.K, a.group_size, a.ldx))
    return fail(LDK_ERR_UNSUPPORTED, "%s: shape M=%d N=%d K=%d group_size=%d not supported", fn, a.M, a.N, a.K,
                a.group_size);
  if (a.swiglu && !gemm_swiglu_applies(f, a.M, a.N, a.K, a.group_size, a.ldx, a.block_n, a.split_k,
                                       a.workspace ? a.workspace_bytes : 0))
    return fail(LDK_ERR_UNSUPPORTED, "%s: SwiGLU in the epilogue needs a plan of two or more column groups with no K "
                "split (M=%d N=%d K=%d)", fn, a.M, a.N, a.K);
  if (a.block_n && a.block_n != 128 && a.block_n != 256)
    return fail(LDK_ERR_UNSUPPORTED, "%s: block_n=%d must be 128 or 256", fn, a.block_n);
  return f == WFmt::kInt4 ? launch_fmt<WFmt::kInt4>(a, s) : launch_fmt<WFmt::kE4M3>(a, s);
}

bool gemm_swiglu_applies(WFmt f, int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx, int block_n,
                         int split_k, int64_t ws_bytes) {
  if (N % 2 || !gemm_supported(f, M, N, K, group_size, ldx)) return false;
  const GemmShape sh = pick_shape(f, M, N, K, block_n, split_k, ws_bytes);
  const int steps = (int)(K / kStep), kps = (steps + sh.splits - 1) / sh.splits;
  // e4m3 on 2-wave tiles: a wave's 64 columns are 64 bytes per K row, so the g (or u) wave of a
  // workgroup reads half of each 128-byte line and the next workgroup (on another XCD) the other
  // half; gate_up M = 32 / 128 measured 13.50 / 20.25 us composed against 14.63 / 24.51 fused.
  // From 4 waves (M = 256 / 512: 28.20 / 42.02 -> 26.38 / 39.26 us) the pair's g waves cover
  // whole lines. int4 rows are 256 bytes per wave.
  if (f == WFmt::kE4M3 && sh.waves < 4) return false;
  return swiglu_tile(sh.waves, sh.mt) && (steps + kps - 1) / kps == 1 && (N / 2) % (64 * (sh.waves / 2)) == 0;
}

void gemm_plan(WFmt f, int64_t M, int64_t N, int64_t K, int block_n, int split_k, int64_t ws_bytes, int* tile_n,
               int* splits) {
  const GemmShape sh = pick_shape(f, M, N, K, block_n, split_k, ws_bytes);
  const int steps = (int)(K / kStep), kps = (steps + sh.splits - 1) / sh.splits;
  *tile_n = 64 * sh.waves;
  *splits = (steps + kps - 1) / kps;  // as launch(): no empty split
}

const char* gemm_kernel_name(WFmt f, int64_t M, int64_t N, int64_t K, int block_n) {
  // the library's workspace (64 MiB) bounds the split, as in a call through ldk_*_matmul
  const GemmShape sh = pick_shape(f, M, N, K, block_n, 0, int64_t(64) << 20);
  static thread_local char buf[64];
  snprintf(buf, sizeof(buf), "%s_gemm_kernel<%d, %d, %d, %d>", f == WFmt::kInt4 ? "w4a16" : "w8a16", sh.waves, sh.mt,
           stages_of(f, sh.waves, sh.mt, sh.kg), sh.kg);
  return buf;
}

}  // namespace ldk
