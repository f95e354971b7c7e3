// Calibration kernels for the roofline of the W4A16 M = 1 GEMV (measurement infrastructure,
// built into kernels/bench/libldk_probe.so, not part of libldk_amd.so's C ABI).
//
// What a kernel that moves 13.76 MB on this GPU cannot go below, measured with the same profiler
// and timing as the product kernels:
//  - probe_empty:  a kernel that does nothing, on one workgroup or on a given grid (the launch,
//                  dispatch and end-of-kernel cost on its own);
//  - probe_stream: a contiguous read of `bytes`, one 16-byte non-temporal load per lane and
//                  `loads` per lane, XOR-folded so no load is dead (the floor for the bytes);
//  - probe_tile:   the packed [R, N] int32 weight read in the M = 1 kernel's pattern, loads only:
//                  one workgroup per 32-column tile (128 bytes of each packed row), 6 waves of
//                  lanes (8 along N x 8 along K), each lane 4 rows of 16 bytes (the floor for the
//                  kernel's access pattern).
// Each writes one word per workgroup to `sink` only if its fold equals a value the inputs never
// produce, so the compiler keeps every load and the kernels write nothing in practice.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

__global__ void probe_empty_kernel() {}

template <int LOADS>
__global__ __launch_bounds__(256) void probe_stream_kernel(const u32x4* src, int64_t n16, uint32_t* sink) {
  u32x4 v[LOADS];
  const int64_t base = (int64_t)blockIdx.x * LOADS * blockDim.x + threadIdx.x;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int64_t idx = base + (int64_t)i * blockDim.x;
    v[i] = idx < n16 ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

// One workgroup per 32-column tile of a packed [R, N] int32 matrix, 6 waves x 64 lanes; lane
// (ln = lane % 8, lk = lane / 8) of wave w reads rows w * RPW + lk + 8t (t < 4) at columns
// 32 * tile + 4 * ln .. + 3, RPW = R / 6 rows per wave (R = 192 for K = 1536).
__global__ __launch_bounds__(384) void probe_tile_kernel(const uint32_t* qw, int R, int N, uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 7, lk = lane >> 3;
  const int rpw = R / 6;
  const int col = blockIdx.x * 32 + 4 * ln;
  uint32_t acc = 0;
  for (int r0 = wave * rpw; r0 < (wave + 1) * rpw; r0 += 32) {
    u32x4 v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = r0 + lk + 8 * t;
      v[t] = r < R ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(qw + (int64_t)r * N + col))
                   : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) acc ^= v[t][0] ^ v[t][1] ^ v[t][2] ^ v[t][3];
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x * 384 + threadIdx.x] = acc;
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : 4; }

}  // namespace

extern "C" int ldk_probe_empty(int workgroups, int threads, void* stream) {
  if (workgroups <= 0 || threads <= 0 || threads > 1024) return 1;
  (void)hipGetLastError();
  probe_empty_kernel<<<workgroups, threads, 0, (hipStream_t)stream>>>();
  return launched();
}

// Reads `bytes` (a multiple of 16) from src with `loads` (1, 4 or 16) 16-byte loads per lane of
// 256-lane workgroups; sink holds one word per workgroup.
extern "C" int ldk_probe_stream(const void* src, int64_t bytes, int loads, void* sink, void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16) return 1;
  const int64_t n16 = bytes / 16;
  const int64_t grid = (n16 + 256 * loads - 1) / (256 * loads);
  if (grid > INT32_MAX) return 3;
  (void)hipGetLastError();
  auto s = (hipStream_t)stream;
  auto src16 = static_cast<const u32x4*>(src);
  auto out = static_cast<uint32_t*>(sink);
  switch (loads) {
    case 1: probe_stream_kernel<1><<<(unsigned)grid, 256, 0, s>>>(src16, n16, out); break;
    case 4: probe_stream_kernel<4><<<(unsigned)grid, 256, 0, s>>>(src16, n16, out); break;
    case 16: probe_stream_kernel<16><<<(unsigned)grid, 256, 0, s>>>(src16, n16, out); break;
    default: return 3;
  }
  return launched();
}

// Reads a packed [R, N] int32 matrix (R a multiple of 192, N of 32, 16-byte aligned) in the M = 1
// kernel's tile pattern: N / 32 workgroups of 384 lanes; sink holds 384 words per workgroup.
extern "C" int ldk_probe_tile(const void* qweight, int R, int N, void* sink, void* stream) {
  if (!qweight || !sink || R <= 0 || R % 192 || N <= 0 || N % 32) return 1;
  (void)hipGetLastError();
  probe_tile_kernel<<<N / 32, 384, 0, (hipStream_t)stream>>>(static_cast<const uint32_t*>(qweight), R, N,
                                                            static_cast<uint32_t*>(sink));
  return launched();
}
