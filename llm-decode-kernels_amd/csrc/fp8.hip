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
// in LDS as fp16. The per-channel scale is applied once after the K reduction (fp8.py:120).
#include <algorithm>

#include "ldk_common.h"

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

struct W8Args {
  const half_t* x;
  int64_t ldx;
  const uint8_t* wq;
  const half_t* scale;
  const half_t* bias;
  half_t* out;
  int64_t ldo;
  int M, N, K;
};

// x is staged in LDS one K chunk of KC columns at a time (KC = K when the whole row fits), so the
// LDS need stays bounded for any K: [MT][KC] fp16 + one trash chunk, then the reduction buffer.
template <int MT, int LN, int UB>
__global__ __launch_bounds__(512) void w8a16_skinny_kernel(W8Args a, int KC) {
  constexpr int CW = 16 * LN;
  constexpr int LKW = 64 / LN;
  constexpr int PXr = (MT * UB + 8 * LN - 1) / (8 * LN);
  constexpr int PX = PXr < 4 ? PXr : 4;
  extern __shared__ __align__(16) unsigned char smem[];
  const int NW = blockDim.x >> 6, NT = blockDim.x;
  const int LK = NW * LKW;
  const int K = a.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane % LN;
  const int lk = wave * LKW + lane / LN;
  const int n0 = ldk::xcd_remap(blockIdx.x, gridDim.x) * CW;
  const int col = min(n0 + 16 * ln, a.N - 16);

  // LDS: x [MT][KC] fp16 + one trash chunk, then the reduction buffer [NW][MT][CW] floats.
  half_t* xs = reinterpret_cast<half_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + (((size_t)MT * KC + 8) * 2 + 15) / 16 * 16);
  int kc0 = 0;                    // first K column of the staged chunk
  int kcn = min(KC, K);           // its width
  int nx = MT * kcn / 8;          // 16-byte x items of the chunk, item = c*MT + m

  u32x4 xr[PX];
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    const int it = min(tid + i * NT, nx - 1);
    const int m = min(it % MT, a.M - 1), c = it / MT;
    xr[i] = *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c);
  }

  float acc[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = 0.0f;

  u32x4 w[UB];
  auto load_batch = [&](int kb) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int k = min(kb + lk + u * LK, K - 1);
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.wq + (int64_t)k * a.N + col));
    }
  };
  auto compute_batch = [&](int kb) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int k = kb + lk + u * LK;
      if (k < K) {
        float xv[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) xv[m] = (float)xs[(size_t)m * KC + (k - kc0)];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[u][d], false);
          const float2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[u][d], true);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            acc[m][4 * d + 0] = __builtin_fmaf(xv[m], lo[0], acc[m][4 * d + 0]);
            acc[m][4 * d + 1] = __builtin_fmaf(xv[m], lo[1], acc[m][4 * d + 1]);
            acc[m][4 * d + 2] = __builtin_fmaf(xv[m], hi[0], acc[m][4 * d + 2]);
            acc[m][4 * d + 3] = __builtin_fmaf(xv[m], hi[1], acc[m][4 * d + 3]);
          }
        }
      }
    }
  };

  load_batch(0);
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    const int it = tid + i * NT;
    const int m = it % MT, c = it / MT;
    u32x4 d = xr[i];
    if (m >= a.M) d = u32x4{0u, 0u, 0u, 0u};
    const size_t off = it < nx ? (size_t)m * KC + 8 * c : (size_t)MT * KC;  // trash chunk
    *reinterpret_cast<u32x4*>(xs + off) = d;
  }
  for (int it = tid + PX * NT; it < nx; it += NT) {
    const int m = it % MT, c = it / MT;
    u32x4 d = *reinterpret_cast<const u32x4*>(a.x + min(m, a.M - 1) * a.ldx + 8 * c);
    if (m >= a.M) d = u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(xs + (size_t)m * KC + 8 * c) = d;
  }
  ldk::lds_barrier();
  // KC is a multiple of the batch step UB * LK, so no batch straddles two chunks. The next batch's
  // weight loads are issued before a chunk switch's barriers and stay in flight across them.
  for (int kb = 0;;) {
    compute_batch(kb);
    kb += UB * LK;
    if (kb >= K) break;
    load_batch(kb);
    if (kb >= kc0 + kcn) {  // uniform: restage x for the next chunk
      kc0 = kb;
      kcn = min(KC, K - kc0);
      nx = MT * kcn / 8;
      ldk::lds_barrier();  // every wave is done reading the previous chunk
      for (int it = tid; it < nx; it += NT) {
        const int m = it % MT, c = it / MT;
        u32x4 d = *reinterpret_cast<const u32x4*>(a.x + min(m, a.M - 1) * a.ldx + kc0 + 8 * c);
        if (m >= a.M) d = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(xs + (size_t)m * KC + 8 * c) = d;
      }
      ldk::lds_barrier();
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = ldk::sum_lanes_strided<LN>(acc[m][j]);
  if (lane < LN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<float4_t*>(red + ((size_t)wave * MT + m) * CW + 16 * lane + 4 * d) =
            float4_t{acc[m][4 * d], acc[m][4 * d + 1], acc[m][4 * d + 2], acc[m][4 * d + 3]};
  }
  ldk::lds_barrier();
  for (int o = tid; o < MT * CW; o += NT) {
    const int m = o / CW, c = o - m * CW;
    const int n = n0 + c;
    if (m < a.M && n < a.N) {
      float v = 0.0f;
      for (int wv = 0; wv < NW; ++wv) v += red[((size_t)wv * MT + m) * CW + c];
      v *= (float)a.scale[n];
      if (a.bias) v += (float)a.bias[n];
      a.out[(int64_t)m * a.ldo + n] = (half_t)v;
    }
  }
}

struct W8Cfg {
  int mt, ln, nw, ub;
};

constexpr int64_t kW8MaxLds = 160 * 1024;  // LDS per workgroup on gfx950

// LDS a configuration needs with x staged in chunks of at least one batch step.
int64_t w8_min_lds(int mt, int ln, int nw, int ub, int64_t K) {
  const int64_t step = (int64_t)ub * nw * (64 / ln);
  return (int64_t)mt * std::min<int64_t>(K, step) * 2 + 48 + (int64_t)nw * mt * 16 * ln * 4;
}

int round_ub8(int rows) {
  static const int kUB[] = {2, 4, 6, 8, 12, 16};
  for (int u : kUB)
    if (u >= rows) return u;
  return 16;
}

W8Cfg choose_w8(int64_t M, int64_t N, int64_t K, int block_n, int split_k) {
  W8Cfg best{M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16, 1, 4, 2};
  double best_score = -1e30;
  for (int ln : {4, 2, 1, 8}) {
    if (block_n && block_n != 16 * ln) continue;
    for (int nw : {4, 8, 2, 1}) {
      const int lk = nw * 64 / ln;
      if (split_k && split_k != lk) continue;
      const int64_t nwg = (N + 16 * ln - 1) / (16 * ln);
      const int64_t rows = (K + lk - 1) / lk;
      if (w8_min_lds(best.mt, ln, nw, round_ub8((int)std::min<int64_t>(rows, 16)), K) > kW8MaxLds) continue;
      const double waves = (double)nwg * nw;
      double score = -std::abs(std::log2(std::max(waves, 1.0) / 2048.0)) * 4.0;
      score -= rows > 16 ? (rows - 16) * 0.5 : 0.0;
      score -= nwg < 256 ? (256.0 - nwg) / 64.0 : 0.0;
      if (score > best_score) {
        best_score = score;
        best.ln = ln;
        best.nw = nw;
        best.ub = round_ub8((int)std::min<int64_t>(rows, 16));
      }
    }
  }
  return best;
}

template <int MT, int LN, int UB>
int launch_w8_t(const W8Args& a, int nw, hipStream_t s) {
  // x chunk width: all of K when [MT][K] fp16 fits 64 KiB, else the largest multiple of the
  // batch step (UB rows for each of the nw*64/LN lanes along K) that does.
  const int64_t step = (int64_t)UB * nw * (64 / LN);
  const int64_t red_bytes = (int64_t)nw * MT * 16 * LN * 4;
  int64_t kc = a.K;
  const int64_t max_kc = ((kW8MaxLds - red_bytes - 32) / (2 * MT)) / 8 * 8;
  if (kc > max_kc) {
    kc = max_kc / step * step;
    if (kc < step) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: x chunk smaller than one batch (M=%d)", a.M);
  }
  const size_t lds = (((size_t)MT * kc + 8) * 2 + 15) / 16 * 16 + (size_t)red_bytes;
  auto kern = w8a16_skinny_kernel<MT, LN, UB>;
  if (lds > 64 * 1024) {
    if (lds > 160 * 1024) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: LDS need %zu B exceeds 160 KiB (M*K too large for the decode kernel)", lds);
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return ldk::fail(LDK_ERR_LAUNCH, "w8a16: cannot raise the LDS limit to %zu B", lds);
  }
  const int grid = (int)((a.N + 16 * LN - 1) / (16 * LN));
  (void)hipGetLastError();
  kern<<<grid, nw * 64, lds, s>>>(a, (int)kc);
  return ldk::check_launch("w8a16_skinny");
}

template <int MT, int LN>
int launch_w8_ub(const W8Args& a, const W8Cfg& c, hipStream_t s) {
  switch (c.ub) {
    case 2: return launch_w8_t<MT, LN, 2>(a, c.nw, s);
    case 4: return launch_w8_t<MT, LN, 4>(a, c.nw, s);
    case 6: return launch_w8_t<MT, LN, 6>(a, c.nw, s);
    case 8: return launch_w8_t<MT, LN, 8>(a, c.nw, s);
    case 12: return launch_w8_t<MT, LN, 12>(a, c.nw, s);
    case 16: return launch_w8_t<MT, LN, 16>(a, c.nw, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: rows per lane %d not instantiated", c.ub);
}

template <int MT>
int launch_w8_ln(const W8Args& a, const W8Cfg& c, hipStream_t s) {
  switch (c.ln) {
    case 1: return launch_w8_ub<MT, 1>(a, c, s);
    case 2: return launch_w8_ub<MT, 2>(a, c, s);
    case 4: return launch_w8_ub<MT, 4>(a, c, s);
    case 8: return launch_w8_ub<MT, 8>(a, c, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: column tile %d not instantiated", 16 * c.ln);
}

int launch_w8(const W8Args& a, const W8Cfg& c, hipStream_t s) {
  switch (c.mt) {
    case 1: return launch_w8_ln<1>(a, c, s);
    case 2: return launch_w8_ln<2>(a, c, s);
    case 4: return launch_w8_ln<4>(a, c, s);
    case 8: return launch_w8_ln<8>(a, c, s);
    case 16: return launch_w8_ln<16>(a, c, s);
  }
  return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16: row tile %d not instantiated", c.mt);
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

extern "C" int ldk_w8a16_matmul(const void* x, int64_t ldx, const uint8_t* wq, const void* scale, const void* bias, void* out,
                                int64_t ldo, int64_t M, int64_t N, int64_t K, int block_n, int split_k, int flags,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (!x || !wq || !scale || !out) return ldk::fail(LDK_ERR_INVALID, "w8a16_matmul: null pointer");
  if (M <= 0 || N <= 0 || K <= 0) return ldk::fail(LDK_ERR_INVALID, "w8a16_matmul: M, N, K must be positive");
  if (M > 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: M=%lld > 16 (prefill GEMM not built yet)", (long long)M);
  if (N % 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: N=%lld must be a multiple of 16", (long long)N);
  if (K % 8) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: K=%lld must be a multiple of 8", (long long)K);
  if (ldx < K || ldo < N) return ldk::fail(LDK_ERR_INVALID, "w8a16_matmul: row stride smaller than K/N");
  if (ldx % 8 || !ldk::aligned(x, 16) || !ldk::aligned(wq, 16))
    return ldk::fail(LDK_ERR_ALIGN, "w8a16_matmul: x and wq must be 16-byte aligned with ldx %% 8 == 0");
  if (N > INT32_MAX / 16 || K > INT32_MAX / 16) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: N or K too large");
  if (flags & ~(LDK_PATH_VALU)) return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: flags 0x%x not supported", flags);
  if (block_n && (block_n % 16 || block_n > 128 || (block_n & (block_n - 1))))
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: block_n=%d must be 16, 32, 64 or 128", block_n);
  const W8Cfg c = choose_w8(M, N, K, block_n, split_k);
  if (split_k && c.nw * 64 / c.ln != split_k)
    return ldk::fail(LDK_ERR_UNSUPPORTED, "w8a16_matmul: split_k=%d is not nw*64/(block_n/16) for nw in {1,2,4,8}", split_k);
  const W8Args a{(const half_t*)x, ldx, wq, (const half_t*)scale, (const half_t*)bias, (half_t*)out, ldo, (int)M, (int)N, (int)K};
  return launch_w8(a, c, (hipStream_t)stream);
}
