// int4 weight format on the GPU: pack, unpack, RTN quantize and the bit-exact dequantizer.
//
// Format (kernels/quant.py:3-10 of the reference): qweight int32 [K/8, N]; nibble i (bits
// 4i..4i+3) of word [r, n] is q[8r+i, n]; scales/zeros [K/G, N]; w = (q - z) * s.
#include "ldk_common.h"

namespace {

// ------------------------------------------------------------------------------ pack / unpack

// One thread per packed word [r, n]; consecutive threads take consecutive n (coalesced).
// The sum of q << 4i is taken modulo 2^32 and reinterpreted as int32, which is what
// quant.py:24-28 computes in int64 for any integer input (for 0..15 it is a plain OR).
__global__ void int4_pack_kernel(const int32_t* __restrict__ q, uint32_t* __restrict__ packed,
                                 int64_t R, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * N) return;
  const int64_t r = i / N, n = i - r * N;
  const int32_t* src = q + (8 * r) * N + n;
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc += (uint32_t)src[k * N] << (4 * k);
  packed[i] = acc;
}

// q[8r+k, n] = (packed[r, n] >> 4k) & 0xF (quant.py:31-35).
__global__ void int4_unpack_kernel(const uint32_t* __restrict__ packed, int32_t* __restrict__ q,
                                   int64_t R, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * N) return;
  const int64_t r = i / N, n = i - r * N;
  const uint32_t w = packed[i];
  int32_t* dst = q + (8 * r) * N + n;
#pragma unroll
  for (int k = 0; k < 8; ++k) dst[k * N] = (int32_t)((w >> (4 * k)) & 0xFu);
}

// ------------------------------------------------------------------------------ RTN quantizer

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<half_t>(const half_t* p) { return (float)*p; }
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p) {  // bf16 bits
  return __builtin_bit_cast(float, (uint32_t)*p << 16);
}

// float32 -> storage type with round-to-nearest-even (the `.to(dtype)` of quant.py:49).
template <typename T>
__device__ __forceinline__ T store_cast(float v);
template <>
__device__ __forceinline__ half_t store_cast<half_t>(float v) { return (half_t)v; }
template <>
__device__ __forceinline__ float store_cast<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t store_cast<uint16_t>(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// One thread per (group g, column n), consecutive threads on consecutive n so that the packed
// words, scales and zeros are written coalesced. Each thread reads its group's G contiguous
// weights of row n twice (min/max pass, then quantize pass; the second pass hits in cache).
//
// The arithmetic is the float32 sequence of quant.py:42-47, each step one IEEE operation:
// scale = max((wmax - wmin) / 15, 1e-6); zero = clamp(rint(-wmin / scale), 0, 15);
// q = clamp(rint(w / scale + zero), 0, 15). Division is correctly rounded (the library is built
// with -fhip-fp32-correctly-rounded-divide-sqrt) and rint rounds half to even like torch.round.
template <typename T>
__global__ void quantize_rtn_kernel(const T* __restrict__ w, uint32_t* __restrict__ qweight,
                                    T* __restrict__ scales, T* __restrict__ zeros, int64_t N,
                                    int64_t K, int G) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t ng = K / G;
  if (i >= ng * N) return;
  const int64_t g = i / N, n = i - g * N;
  const T* src = w + n * K + g * G;
  float wmin = load_f32(src), wmax = wmin;
  for (int k = 1; k < G; ++k) {
    const float v = load_f32(src + k);
    wmin = fminf(wmin, v);
    wmax = fmaxf(wmax, v);
  }
  const float scale = fmaxf((wmax - wmin) / 15.0f, 1e-6f);
  // Compare-select clamp keeps a -0.0 from rint, as torch's CPU clamp and numpy's clip do.
  float zero = rintf(-wmin / scale);
  zero = zero < 0.0f ? 0.0f : zero;
  zero = zero > 15.0f ? 15.0f : zero;
  uint32_t* dst = qweight + (g * (G / 8)) * N + n;
  for (int r = 0; r < G / 8; ++r) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = load_f32(src + 8 * r + k);
      const float q = fminf(fmaxf(rintf(v / scale + zero), 0.0f), 15.0f);
      word |= (uint32_t)q << (4 * k);
    }
    dst[(int64_t)r * N] = word;
  }
  scales[i] = store_cast<T>(scale);
  zeros[i] = store_cast<T>(zero);
}

// ---------------------------------------------------------------------------------- dequant

// out [N, K] fp16 = (q - z) * s, one fp16 rounding (reference.py:27-36). Lane mapping favours
// the 4x larger output: 8 consecutive lanes take 8 consecutive packed rows of one column and
// write 8 x 16 B = 128 contiguous bytes of output row n.
__global__ __launch_bounds__(256) void w4a16_dequant_kernel(const uint32_t* __restrict__ qw,
                                                            const half_t* __restrict__ sc,
                                                            const half_t* __restrict__ zr,
                                                            half_t* __restrict__ out, int64_t N,
                                                            int64_t K, int gshift_rows) {
  const int64_t R = K / 8;
  const int64_t rt = (R + 7) / 8;  // row tiles of 8 packed rows
  const int64_t t = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);  // (column, row-tile) pair
  const int64_t n = t / rt;
  const int64_t r = (t - n * rt) * 8 + (threadIdx.x & 7);
  if (n >= N || r >= R) return;
  const uint32_t word = qw[r * N + n];
  const int64_t g = r >> gshift_rows;
  const half_t s = sc[g * N + n], z = zr[g * N + n];
  half8_t v;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const half_t q = (half_t)(float)((word >> (4 * k)) & 0xFu);
    v[k] = (half_t)(q - z) * s;
  }
  *reinterpret_cast<half8_t*>(out + n * K + 8 * r) = v;
}

inline int blocks_for(int64_t n, int threads) { return (int)((n + threads - 1) / threads); }

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

}  // namespace

extern "C" int ldk_int4_pack(const int32_t* q, int32_t* packed, int64_t K, int64_t N, void* stream) {
  if (!q || !packed) return ldk::fail(LDK_ERR_INVALID, "int4_pack: null pointer");
  if (K <= 0 || N <= 0 || K % 8) return ldk::fail(LDK_ERR_INVALID, "int4_pack: K=%lld must be a positive multiple of 8, N=%lld > 0", (long long)K, (long long)N);
  const int64_t R = K / 8;
  if (R * N > (int64_t)INT32_MAX * 256) return ldk::fail(LDK_ERR_UNSUPPORTED, "int4_pack: too large");
  (void)hipGetLastError();
  int4_pack_kernel<<<blocks_for(R * N, 256), 256, 0, (hipStream_t)stream>>>(q, (uint32_t*)packed, R, N);
  return ldk::check_launch("int4_pack");
}

extern "C" int ldk_int4_unpack(const int32_t* packed, int32_t* q, int64_t K, int64_t N, void* stream) {
  if (!q || !packed) return ldk::fail(LDK_ERR_INVALID, "int4_unpack: null pointer");
  if (K <= 0 || N <= 0 || K % 8) return ldk::fail(LDK_ERR_INVALID, "int4_unpack: K=%lld must be a positive multiple of 8, N=%lld > 0", (long long)K, (long long)N);
  const int64_t R = K / 8;
  (void)hipGetLastError();
  int4_unpack_kernel<<<blocks_for(R * N, 256), 256, 0, (hipStream_t)stream>>>((const uint32_t*)packed, q, R, N);
  return ldk::check_launch("int4_unpack");
}

extern "C" int ldk_quantize_rtn(const void* w, int dtype, int32_t* qweight, void* scales, void* zeros,
                                int64_t N, int64_t K, int group_size, void* stream) {
  if (!w || !qweight || !scales || !zeros) return ldk::fail(LDK_ERR_INVALID, "quantize_rtn: null pointer");
  if (N <= 0 || K <= 0 || group_size <= 0 || group_size % 8 || K % group_size)
    return ldk::fail(LDK_ERR_INVALID, "quantize_rtn: K=%lld must be a multiple of group_size=%d, which must be a multiple of 8", (long long)K, group_size);
  const int64_t n = (K / group_size) * N;
  const int blocks = blocks_for(n, 256);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  switch (dtype) {
    case LDK_F16:
      quantize_rtn_kernel<half_t><<<blocks, 256, 0, s>>>((const half_t*)w, (uint32_t*)qweight, (half_t*)scales, (half_t*)zeros, N, K, group_size);
      break;
    case LDK_BF16:
      quantize_rtn_kernel<uint16_t><<<blocks, 256, 0, s>>>((const uint16_t*)w, (uint32_t*)qweight, (uint16_t*)scales, (uint16_t*)zeros, N, K, group_size);
      break;
    case LDK_F32:
      quantize_rtn_kernel<float><<<blocks, 256, 0, s>>>((const float*)w, (uint32_t*)qweight, (float*)scales, (float*)zeros, N, K, group_size);
      break;
    default:
      return ldk::fail(LDK_ERR_INVALID, "quantize_rtn: unknown dtype %d", dtype);
  }
  return ldk::check_launch("quantize_rtn");
}

extern "C" int ldk_w4a16_dequant(const int32_t* qweight, const void* scales, const void* zeros, void* out,
                                 int64_t N, int64_t K, int group_size, void* stream) {
  if (!qweight || !scales || !zeros || !out) return ldk::fail(LDK_ERR_INVALID, "w4a16_dequant: null pointer");
  const int gsh = log2_exact(group_size);
  if (N <= 0 || K <= 0 || K % 8 || gsh < 3 || K % group_size)
    return ldk::fail(LDK_ERR_INVALID, "w4a16_dequant: need K %% 8 == 0, group_size a power of two >= 8 dividing K (K=%lld, group_size=%d)", (long long)K, group_size);
  if (!ldk::aligned(out, 16)) return ldk::fail(LDK_ERR_ALIGN, "w4a16_dequant: out must be 16-byte aligned");
  const int64_t pairs = N * ((K / 8 + 7) / 8);
  (void)hipGetLastError();
  w4a16_dequant_kernel<<<blocks_for(pairs, 32), 256, 0, (hipStream_t)stream>>>(
      (const uint32_t*)qweight, (const half_t*)scales, (const half_t*)zeros, (half_t*)out, N, K, gsh - 3);
  return ldk::check_launch("w4a16_dequant");
}
