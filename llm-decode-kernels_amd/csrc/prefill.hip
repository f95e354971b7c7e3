// Prefill W4A16 GEMM: y[M, N] = x[M, K] @ dequant(W)^T (+ bias) for many rows, on the matrix
// cores of gfx950 (v_mfma_f32_16x16x32_f16). The reference's counterpart is its Triton tensor-core
// GEMM for prefill rows (kernels/w4a16.py:31-97, routed at w4a16.py:264-268,328-329), which
// dequantizes each weight tile to fp16 and runs tl.dot with fp32 accumulation. Same numerics
// here: every weight is dequantized exactly as dequantize_ref does it (kernels/reference.py:27-36,
// one fp16 rounding of (q - z) * s), products accumulate in fp32, the output is rounded once.
//
// Work decomposition (one workgroup per BM x BN output tile, all of K):
//  * BN = 64 * WAVES columns. Wave w owns 64 of them for all BM rows, so each wave loads and
//    decodes only its own weights (no decode is repeated across waves), and x is the operand the
//    waves share, through LDS.
//  * Weights: lane l = (c16 = l % 16, kb = l / 16) takes 16 bytes of packed row 4 * sub + kb at
//    columns n0 + 4 * c16 .. + 3. Each of the 4 words holds 8 consecutive K of one column, which
//    is exactly one lane's B operand of the MFMA: word j feeds 16-column tile j, whose column c16
//    is the real column n0 + 4 * c16 + j. Nibbles are decoded with the fp16 magic-number trick
//    ((w & 0x000F000F) | 0x6400 -> 1024 + q per half, pairs (q0, q4) .. (q3, q7)); then
//    (1024 + q) - (1024 + z) is exact, one packed fp16 multiply by s rounds once, and four
//    v_perm_b32 put the eight halves in K order (q0, q1) .. (q6, q7).
//  * Pipeline: an S-stage ring of K-steps of 64, each stage a distinct LDS array holding the
//    x tile (BM rows x 128 bytes) and every wave's packed weight words (2 KB per wave). Both are
//    loaded with gfx950's 16-byte loads to LDS (buffer_load/global_load ... lds: lane i writes
//    base + 16 i), so S - 1 stages are in flight without holding registers. x chunks are stored
//    XOR-swizzled (chunk c of row r at slot c ^ (r % 8)), so the 8 rows an MFMA A operand reads
//    per LDS phase fall in distinct banks; rows past M are buffer loads past the resource, which
//    write zeros. Each stage also holds the scales and zeros of its group. Each step waits
//    (explicit vmcnt) for its own stage only, then one barrier, then issues stage ks + S - 1 into
//    the slot all waves finished reading before that barrier. The loop is unrolled by S so every
//    slot is a fixed array: the compiler then needs no conservative waits on the LDS reads.
#include <algorithm>
#include <cstdint>

#include "prefill.h"

namespace {

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

// Workgroup barrier that is also a compiler memory barrier, without the vmcnt(0) a C++ fence adds
// (the ring keeps later stages' loads in flight across it).
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" : : : "memory");
}

// 16-byte loads to LDS (lane i writes lds_base + 16 i), issued as inline asm: the compiler's wait
// insertion then does not track them, so it adds no conservative vmcnt wait before the LDS reads
// of other stages (it would after the loop's back edge, where it no longer knows which LDS array
// each pending load writes); the ring's own vmcnt waits order them. M0 holds the LDS base.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma_buffer16(u32x4 rsrc, uint32_t voffset, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voffset), "s"(rsrc), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_global16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(lds_base) : "memory", "m0");
}
// Raw buffer descriptor over [p, p + bytes): a load at an offset past it returns zeros (and, to
// LDS, writes zeros).
__device__ __forceinline__ u32x4 raw_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

template <int WAVES, int MT, int S>
struct GemmCfg {
  static constexpr int BM = 16 * MT, NT = 4, NTHR = WAVES * 64;
  static constexpr int XI = BM / 8 / WAVES;         // x load instructions per wave and stage (8 rows each)
  static constexpr int XBYTES = BM * kXRow;
  static constexpr int SZ = XBYTES + WAVES * 2048;    // then 256 bytes of scales and zeros per wave
  static constexpr int STAGE = SZ + WAVES * 256;     // x tile, 2 KB of weight words per wave, s and z
  static constexpr int LOADS = XI + 2 + 2;           // per wave and stage: x, weights (2), scales, zeros
  static_assert(XI * WAVES * 8 == BM, "whole x load instructions");
};

template <int WAVES, int MT, int S>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(MT == 8 ? 2 : 1))) void w4a16_gemm_kernel(ldk::W4GemmArgs a, int kps, float* partial) {
  using C = GemmCfg<WAVES, MT, S>;
  constexpr int BM = C::BM, NT = C::NT;
  static_assert(S == 3 || S == 4, "ring of 3 or 4 stages");
  __shared__ __align__(16) unsigned char st0[C::STAGE], st1[C::STAGE], st2[C::STAGE], st3[S == 4 ? C::STAGE : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases go to M0
  const int c16 = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * (64 * WAVES) + 64 * wave;
  const int m0 = blockIdx.y * BM;
  const int mrows = min(a.M - m0, BM);
  const int col = min(n0 + 4 * c16, a.N - 4);  // clamped: lanes past N load valid memory, store nothing
  // K-steps [kbeg, kbeg + nks) of split blockIdx.z
  const int kbeg = blockIdx.z * kps;
  const int nks = min(a.K / kStep - kbeg, kps);
  const int gsh = __builtin_ctz(a.group_size) - 6;  // log2(K-steps per group)
  ldk::pin_sgpr(a.x);
  ldk::pin_sgpr(a.qw);

  // x: instruction i of this wave covers rows r0 = 8 (XI * wave + i) .. + 7; lane l takes row
  // r0 + l / 8, slot l % 8, which holds chunk (l % 8) ^ (row % 8) of that row
  const u32x4 xb = raw_rsrc(a.x + (int64_t)m0 * a.ldx, (uint32_t)((int64_t)(mrows - 1) * a.ldx * 2 + (int64_t)a.K * 2));
  // scales and zeros of a stage: lanes 0-7 each take 16 bytes (8 columns) of the wave's 64, past N
  // (and past the arrays) zeros
  const uint32_t szb = (uint32_t)(a.K / a.group_size) * (uint32_t)a.N * 2u;
  const u32x4 sb = raw_rsrc(a.s, szb), zb = raw_rsrc(a.z, szb);
  const uint32_t szoff = 2u * (uint32_t)(n0 + 8 * (lane & 7));
  uint32_t xoff[C::XI];
#pragma unroll
  for (int i = 0; i < C::XI; ++i) {
    const int row = 8 * (C::XI * wave + i) + (lane >> 3), chunk = (lane & 7) ^ (row & 7);
    xoff[i] = row < mrows ? (uint32_t)((int64_t)row * a.ldx * 2 + chunk * 16) : 0x80000000u;
  }
  const uint32_t* wp = a.qw + (int64_t)kb * a.N + col;

  auto issue = [&](unsigned char* stage, int kstep) {
    const int ks = kbeg + kstep;
#pragma unroll
    for (int i = 0; i < C::XI; ++i)
      dma_buffer16(xb, xoff[i] + (uint32_t)(ks * kXRow), lds_addr(stage + 8 * (C::XI * wave + i) * kXRow));
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
      dma_global16(wp + (int64_t)(8 * ks + 4 * sub) * a.N, lds_addr(stage + C::XBYTES + 2048 * wave + 1024 * sub));
    const uint32_t g = 2u * (uint32_t)(ks >> gsh) * (uint32_t)a.N;
    if (lane < 8) {  // one instruction each; lanes 8-63 idle (every wave has lanes 0-7 active)
      dma_buffer16(sb, g + szoff, lds_addr(stage + C::SZ + 256 * wave));
      dma_buffer16(zb, g + szoff, lds_addr(stage + C::SZ + 256 * wave + 128));
    }
  };

  float4_t acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[t][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t magic = ldk::vgpr_const<kMagic>();
  const uint32_t mlo = ldk::sgpr_const<0x000F000Fu>();

  auto compute = [&](const unsigned char* stage) {
    const half4_t s4 = *reinterpret_cast<const half4_t*>(stage + C::SZ + 256 * wave + 8 * c16);
    const half4_t z4 = *reinterpret_cast<const half4_t*>(stage + C::SZ + 256 * wave + 128 + 8 * c16);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const u32x4 wq = *reinterpret_cast<const u32x4*>(stage + C::XBYTES + 2048 * wave + 1024 * sub + 16 * lane);
      half8v B[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const half_t zz = -((half_t)1024.0f + z4[j]);
        const half2_t zb = {zz, zz}, s2 = {s4[j], s4[j]};
        const uint32_t wc = wq[j];
        const uint32_t d0 = ldk::h22u((ldk::u2h2((wc & mlo) | magic) + zb) * s2);          // (q0, q4)
        const uint32_t d1 = ldk::h22u((ldk::u2h2(((wc >> 4) & mlo) | magic) + zb) * s2);   // (q1, q5)
        const uint32_t d2 = ldk::h22u((ldk::u2h2(((wc >> 8) & mlo) | magic) + zb) * s2);   // (q2, q6)
        const uint32_t d3 = ldk::h22u((ldk::u2h2(((wc >> 12) & mlo) | magic) + zb) * s2);  // (q3, q7)
        B[j] = __builtin_bit_cast(half8v, u32x4{perm_lo(d0, d1), perm_lo(d2, d3), perm_hi(d0, d1), perm_hi(d2, d3)});
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
    if (i < nks) issue(stages[i], i);

  // step ks reads slot I = ks % S and refills slot (I + S - 1) % S with stage ks + S - 1
  auto step = [&](auto I_, int ks) {
    constexpr int I = decltype(I_)::value, J = (I + S - 1) % S;
    const int pend = min(S - 2, nks - 1 - ks);  // stages issued after ks that may stay in flight
    if (pend >= S - 2) wait_vm<C::LOADS * (S - 2)>();
    else if (S == 4 && pend == 1) wait_vm<C::LOADS * (S == 4 ? 1 : 0)>();
    else wait_vm<0>();
    ring_barrier();
    if (ks + S - 1 < nks) issue(stages[J], ks + S - 1);
    compute(stages[I]);
  };
  for (int ks = 0; ks < nks; ks += S) {
    step(std::integral_constant<int, 0>{}, ks);
    if (ks + 1 < nks) step(std::integral_constant<int, 1>{}, ks + 1);
    if (ks + 2 < nks) step(std::integral_constant<int, 2>{}, ks + 2);
    if constexpr (S == 4)
      if (ks + 3 < nks) step(std::integral_constant<int, 3>{}, ks + 3);
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

// y[m, n] = fp16(sum over splits of partial[split][m][n] (+ bias[n])), the splits added in index
// order (the result does not depend on which split finished first). 4 columns per thread. Every
// partial read is written back to zero: the workspace is zero between calls, which the decode
// kernels' split-K accumulators rely on.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(float* partial, int splits, const half_t* bias, half_t* out,
                                                          int64_t ldo, int M, int N) {
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
  if (bias) v += float4_t{(float)bias[n], (float)bias[n + 1], (float)bias[n + 2], (float)bias[n + 3]};
  *reinterpret_cast<half4_t*>(out + (int64_t)m * ldo + n) = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Tile shape and K split per problem, from graph-timed sweeps on MI355X (Qwen2.5-1.5B shapes,
// M = 1024 / 2048). Long K (at least 48 K-steps) takes 128 x 256 tiles split over up to 6
// workgroups (down: 52 / 81 us, against 62 / 94 us for 64 x 128 tiles split 2-3 ways): each
// workgroup's K walk is serial, so a long walk is the thing to cut. Short K takes no split (qkv
// M = 1024: 20.6 us unsplit, 25.8 us split 2 ways: the partials' extra traffic outweighs the
// extra workgroups) and the largest tile that still gives 512 workgroups.
struct GemmShape {
  int waves, mt;
};

constexpr int kLongK = 48;  // K-steps of 64 from which a shape counts as long

GemmShape pick_shape(int64_t M, int64_t N, int64_t K, int block_n) {
  auto wgs = [&](int waves, int mt) { return ((N + 64 * waves - 1) / (64 * waves)) * ((M + 16 * mt - 1) / (16 * mt)); };
  if (block_n == 256) return {4, 8};
  if (block_n == 128) return wgs(2, 8) >= 512 ? GemmShape{2, 8} : GemmShape{2, 4};
  if (K / kStep >= kLongK) return {4, 8};
  if (wgs(4, 8) >= 512) return {4, 8};
  if (wgs(2, 8) >= 512) return {2, 8};
  return {2, 4};
}

// K split (long K only, unless split_k asks): toward 512 workgroups (two per CU), at most 6 ways and
// at least 8 K-steps per split, as far as the workspace holds the fp32 partials.
int pick_splits(const ldk::W4GemmArgs& a, int64_t tiles) {
  const int64_t steps = a.K / kStep;
  int64_t splits = a.split_k > 0        ? std::min<int64_t>(a.split_k, steps)
                   : steps >= kLongK ? std::min<int64_t>(std::min<int64_t>((512 + tiles - 1) / tiles, 6), steps / 8)
                                       : 1;
  const int64_t plane = (int64_t)a.M * a.N * 4;
  if (a.workspace) splits = std::min<int64_t>(splits, a.workspace_bytes / plane);
  else splits = 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>(splits, 64));
}

template <int WAVES, int MT, int S>
int launch(const ldk::W4GemmArgs& a, hipStream_t s) {
  const int64_t tn = (a.N + 64 * WAVES - 1) / (64 * WAVES), tm = (a.M + 16 * MT - 1) / (16 * MT);
  const int splits = pick_splits(a, tn * tm);
  const int steps = a.K / kStep, kps = (steps + splits - 1) / splits;
  const int nz = (steps + kps - 1) / kps;  // splits actually used (none empty)
  float* partial = nz > 1 ? static_cast<float*>(a.workspace) : nullptr;
  (void)hipGetLastError();
  w4a16_gemm_kernel<WAVES, MT, S><<<dim3((unsigned)tn, (unsigned)tm, (unsigned)nz), WAVES * 64, 0, s>>>(a, kps, partial);
  int st = ldk::check_launch("w4a16_gemm");
  if (st || nz == 1) return st;
  const int64_t quads = (int64_t)a.M * (a.N / 4);
  gemm_reduce_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>(partial, nz, a.bias, a.out, a.ldo, a.M, a.N);
  return ldk::check_launch("w4a16_gemm_reduce");
}

}  // namespace

namespace ldk {

bool w4a16_gemm_supported(int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx) {
  if (group_size < kStep || (group_size & (group_size - 1)) || K % group_size || N % 8) return false;
  if (M <= 0 || N <= 0 || K <= 0) return false;
  if ((M + 63) / 64 > 65535 || (M * (N / 4) + 255) / 256 > INT32_MAX) return false;
  // the x resource of one row tile spans less than 2 GiB; packed-row offsets fit 32 bits per lane
  if ((int64_t)127 * ldx * 2 + K * 2 >= (int64_t(1) << 31)) return false;
  // scales and zeros are read through 32-bit buffer offsets
  return (K / 8) * N < (int64_t(1) << 31) && (K / group_size) * N * 2 < (int64_t(1) << 31) && N <= INT32_MAX / 8;
}

int w4a16_gemm_launch(const W4GemmArgs& a, hipStream_t s) {
  if (!w4a16_gemm_supported(a.M, a.N, a.K, a.group_size, a.ldx))
    return fail(LDK_ERR_UNSUPPORTED, "w4a16_gemm: shape M=%d N=%d K=%d group_size=%d not supported", a.M, a.N, a.K, a.group_size);
  if (a.block_n && a.block_n != 128 && a.block_n != 256)
    return fail(LDK_ERR_UNSUPPORTED, "w4a16_gemm: block_n=%d must be 128 or 256", a.block_n);
  const GemmShape sh = pick_shape(a.M, a.N, a.K, a.block_n);
  if (sh.waves == 4) return launch<4, 8, 3>(a, s);
  if (sh.mt == 8) return launch<2, 8, 3>(a, s);
  return launch<2, 4, 4>(a, s);
}

const char* w4a16_gemm_kernel_name(int64_t M, int64_t N, int64_t K, int block_n) {
  const GemmShape sh = pick_shape(M, N, K, block_n);
  return sh.waves == 4 ? "w4a16_gemm_kernel<4, 8, 3>" : sh.mt == 8 ? "w4a16_gemm_kernel<2, 8, 3>" : "w4a16_gemm_kernel<2, 4, 4>";
}

}  // namespace ldk
