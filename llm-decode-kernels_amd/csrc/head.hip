// One-row fp16 GEMV, y = W x, for the tied fp16 lm_head of the e2e decode step.
//
// Replaces `F.linear(h, self.lm_head)` of the reference's runner (kernels/e2e/model.py:253) at
// one decode row: W is the fp16 embedding table [N, K] (151936 x 1536, 466.7 MB), x one fp16 row
// of K, y fp16 [N]. The library GEMM (hipBLASLt's 32x16 macro tile) streams that table at about
// 2.9 TB/s on MI355X; the read is the largest single one of the decode step.
//
// Layout and work split. Each wave owns RPW consecutive rows. A row of K halves is KC = K / 8
// 16-byte chunks; lane l loads chunks l, l + 64, ... (KJ of them), so one load instruction reads
// 1 KB of one row, eight whole 128-byte lines, and every lane reuses the same KJ chunks of x from
// registers for all its rows. A wave issues all RPW x KJ weight loads (non-temporal: each byte is
// read once) before its first product, the rows' dot products run on v_dot2_f32_f16 with fp32
// accumulation, and each row's 64 lane partials meet by DPP row rotations and two lane swaps.
// Lane r of the wave stores row r's fp16 result (round to nearest even).
//
// No LDS, no barrier, no atomics: workgroups are independent, 4 waves each, one launch.
#include "ldk_common.h"

namespace {

constexpr int kWaves = 4;

// Optional prologue (NORM): x = rmsnorm(h (+ residual)) * norm_weight, the reference's final
// `self.norm(h, residual)` before the head (kernels/e2e/model.py:250-253) with the standalone
// RMSNorm kernel's rounding steps. A wave's KJ chunks per lane cover the whole row, so every wave
// forms the row statistic from its own loads (DPP + permlane reduction, no LDS, no barrier) and
// stages its x in registers; the h + residual sum is not written back (the head is its last use).
struct NormArgs {
  const half_t* res;  // residual row or null
  const half_t* nw;   // norm weight [K]
  float eps;
};

template <int KJ, int RPW, bool FULL, bool NORM>
__global__ __launch_bounds__(kWaves * 64) void f16_gemv_kernel(const half_t* __restrict__ x,
                                                               const half_t* __restrict__ w, int64_t ldw,
                                                               half_t* __restrict__ y, int64_t N, int KC,
                                                               NormArgs na) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * RPW;
  if (row0 >= N) return;  // uniform per wave
  u32x4 xv[KJ], rv[KJ], nv[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    const int c = lane + 64 * j;
    const bool in = FULL || c < KC;
    xv[j] = in ? *reinterpret_cast<const u32x4*>(x + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    if constexpr (NORM) {
      rv[j] = in && na.res ? *reinterpret_cast<const u32x4*>(na.res + 8 * c) : u32x4{0u, 0u, 0u, 0u};
      nv[j] = in ? *reinterpret_cast<const u32x4*>(na.nw + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  u32x4 wv[RPW][KJ];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = min(row0 + r, N - 1);  // rows past N repeat the last one; not stored
    const half_t* wr = w + row * ldw;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int c = lane + 64 * j;
      wv[r][j] = (FULL || c < KC) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + 8 * c))
                                  : u32x4{0u, 0u, 0u, 0u};
    }
  }
  if constexpr (NORM) {
    half8_t hv[KJ];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {  // chunks past K are zeros and add nothing
      hv[j] = __builtin_bit_cast(half8_t, xv[j]);
      if (na.res) hv[j] = hv[j] + __builtin_bit_cast(half8_t, rv[j]);  // fp16 add
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf((float)hv[j][e], (float)hv[j][e], ss);
    }
    ss = ldk::sum_lanes_strided<1>(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)(8 * KC) + na.eps);
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const half8_t wn = __builtin_bit_cast(half8_t, nv[j]);
      half8_t o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = ldk::rms_f16(hv[j][e], rs, wn[e]);
      xv[j] = __builtin_bit_cast(u32x4, o);
    }
  }
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      // elements pass by value: __builtin_bit_cast of a vector-element lvalue (v[p]) compiles
      // to a read of element 0 for every p here
#pragma unroll
      for (int p = 0; p < 4; ++p) a = __builtin_amdgcn_fdot2(ldk::u2h2(wv[r][j][p]), ldk::u2h2(xv[j][p]), a, false);
    }
    acc[r] = ldk::sum_lanes_strided<1>(a);  // every lane holds the row's sum
  }
  float mine = acc[0];
#pragma unroll
  for (int r = 1; r < RPW; ++r) mine = lane == r ? acc[r] : mine;
  if (lane < RPW && row0 + lane < N) y[row0 + lane] = (half_t)mine;
}

template <int KJ, int RPW, bool NORM>
int launch_rpw(const half_t* x, const half_t* w, int64_t ldw, half_t* y, int64_t N, int KC, const NormArgs& na,
               hipStream_t s) {
  const int64_t waves = (N + RPW - 1) / RPW;
  const int64_t blocks = (waves + kWaves - 1) / kWaves;
  (void)hipGetLastError();
  if (KC == 64 * KJ)
    f16_gemv_kernel<KJ, RPW, true, NORM><<<(unsigned)blocks, kWaves * 64, 0, s>>>(x, w, ldw, y, N, KC, na);
  else
    f16_gemv_kernel<KJ, RPW, false, NORM><<<(unsigned)blocks, kWaves * 64, 0, s>>>(x, w, ldw, y, N, KC, na);
  return ldk::check_launch("f16_gemv");
}

template <int KJ, bool NORM>
int launch_kj(const half_t* x, const half_t* w, int64_t ldw, half_t* y, int64_t N, int KC, int rpw, const NormArgs& na,
              hipStream_t s) {
  return rpw == 4 ? launch_rpw<KJ, 4, NORM>(x, w, ldw, y, N, KC, na, s) : launch_rpw<KJ, 8, NORM>(x, w, ldw, y, N, KC, na, s);
}

// Shared argument checks and dispatch of both entry points.
int f16_gemv(const void* x, const NormArgs* na, const void* w, int64_t ldw, void* y, int64_t N, int64_t K,
             int rows_per_wave, void* stream) {
  if (!x || !w || !y || (na && !na->nw)) return ldk::fail(LDK_ERR_INVALID, "f16_gemv: null pointer");
  if (N <= 0 || K <= 0 || ldw < K) return ldk::fail(LDK_ERR_INVALID, "f16_gemv: N=%lld K=%lld ldw=%lld", (long long)N, (long long)K, (long long)ldw);
  if (rows_per_wave != 0 && rows_per_wave != 4 && rows_per_wave != 8)
    return ldk::fail(LDK_ERR_INVALID, "f16_gemv: rows_per_wave=%d (0, 4 or 8)", rows_per_wave);
  if (K % 8 != 0 || ldw % 8 != 0 || !ldk::aligned(x, 16) || !ldk::aligned(w, 16) ||
      (na && (!ldk::aligned(na->nw, 16) || (na->res && !ldk::aligned(na->res, 16)))))
    return ldk::fail(LDK_ERR_ALIGN, "f16_gemv: K and ldw must be multiples of 8; x, residual, norm weight and w 16-byte aligned");
  if (!ldk::aligned(y, 2)) return ldk::fail(LDK_ERR_ALIGN, "f16_gemv: y must be 2-byte aligned");
  if (K > 2048) return ldk::fail(LDK_ERR_UNSUPPORTED, "f16_gemv: K=%lld > 2048", (long long)K);
  if ((N + 7) / 8 > (int64_t)kWaves * 0x7fffffff) return ldk::fail(LDK_ERR_UNSUPPORTED, "f16_gemv: N=%lld", (long long)N);
  const int KC = (int)(K / 8), KJ = (KC + 63) / 64;
  const int rpw = rows_per_wave ? rows_per_wave : 4;  // 151936x1536: 66.1 us at 4, 67.6 at 8
  const half_t *xp = (const half_t*)x, *wp = (const half_t*)w;
  half_t* yp = (half_t*)y;
  hipStream_t s = (hipStream_t)stream;
  const NormArgs a = na ? *na : NormArgs{nullptr, nullptr, 0.0f};
  if (na) {
    switch (KJ) {
      case 1: return launch_kj<1, true>(xp, wp, ldw, yp, N, KC, rpw, a, s);
      case 2: return launch_kj<2, true>(xp, wp, ldw, yp, N, KC, rpw, a, s);
      case 3: return launch_kj<3, true>(xp, wp, ldw, yp, N, KC, rpw, a, s);
      default: return launch_kj<4, true>(xp, wp, ldw, yp, N, KC, rpw, a, s);
    }
  }
  switch (KJ) {
    case 1: return launch_kj<1, false>(xp, wp, ldw, yp, N, KC, rpw, a, s);
    case 2: return launch_kj<2, false>(xp, wp, ldw, yp, N, KC, rpw, a, s);
    case 3: return launch_kj<3, false>(xp, wp, ldw, yp, N, KC, rpw, a, s);
    default: return launch_kj<4, false>(xp, wp, ldw, yp, N, KC, rpw, a, s);
  }
}

}  // namespace

extern "C" int ldk_f16_gemv(const void* x, const void* w, int64_t ldw, void* y, int64_t N, int64_t K,
                            int rows_per_wave, void* stream) {
  return f16_gemv(x, nullptr, w, ldw, y, N, K, rows_per_wave, stream);
}

extern "C" int ldk_f16_rmsnorm_gemv(const void* h, const void* residual, const void* norm_weight, float eps,
                                    const void* w, int64_t ldw, void* y, int64_t N, int64_t K, int rows_per_wave,
                                    void* stream) {
  const NormArgs na{(const half_t*)residual, (const half_t*)norm_weight, eps};
  return f16_gemv(h, &na, w, ldw, y, N, K, rows_per_wave, stream);
}
