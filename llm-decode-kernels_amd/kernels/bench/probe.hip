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
//                  kernel's access pattern);
//  - probe_piece:  the same bytes cut into K pieces per workgroup, and what each way of meeting the
//                  pieces' partials costs at the end of the kernel (plain store, returning
//                  fixed-point atomic, non-returning fp32 atomic).
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

// Piece patterns and cross-workgroup reductions: the packed [R, N] matrix read by workgroups of W
// waves that each own CW columns x RW rows (lane: column quad lane % (CW/4), row lane / (CW/4),
// 16-byte non-temporal loads), workgroup b taking column tile b % (N/CW) and row piece b / (N/CW).
// Each workgroup folds its loads into one fp32 partial per column (a stand-in for the dot
// products), sums them over its lanes and waves, and ends with RED:
//   0 nothing stored (the loads and the fold alone),
//   1 a plain fp32 store of the partial per column,
//   2 one returning 64-bit fixed-point atomic add per column whose low 6 bits count arrivals;
//     the add that completes the R / RW pieces stores the fp16 sum and re-zeroes the word (the
//     product's split-K reduction, ldk_common.h),
//   3 one non-returning fp32 atomic add per column (no completion: the floor for atomics).
template <int CW, int RW, int W, int RED>
__global__ __launch_bounds__(W * 64) void probe_piece_kernel(const uint32_t* qw, int R, int N, uint64_t* words,
                                                            float* part, _Float16* out) {
  constexpr int LN = CW / 4, LK = 64 / LN, RPW = RW / W, LPL = RPW / LK;
  static_assert(LPL * LK * W == RW && CW <= 256, "piece shape");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tiles_n = N / CW, splits = R / RW;
  const int tn = blockIdx.x % tiles_n, tk = blockIdx.x / tiles_n;
  const int col = tn * CW + 4 * (lane % LN), lk = lane / LN;
  u32x4 v[LPL];
#pragma unroll
  for (int t = 0; t < LPL; ++t)
    v[t] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(qw + (int64_t)(tk * RW + wave * RPW + t * LK + lk) * N + col));
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < LPL; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] += (float)(v[t][q] & 0xFFu) * (1.0f / 256.0f);
#pragma unroll
  for (int off = LN; off < 64; off <<= 1)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] += __shfl_xor(acc[q], off);
  __shared__ float red[W][CW];
  if (lk == 0)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[wave][4 * (lane % LN) + q] = acc[q];
  __syncthreads();
  if (wave) return;
  for (int j = lane; j < CW; j += 64) {
    float p = red[0][j];
#pragma unroll
    for (int w = 1; w < W; ++w) p += red[w][j];
    const int c = tn * CW + j;
    if constexpr (RED == 0) {
      if (p == -1.0f) out[c] = (_Float16)p;  // never: the fold is non-negative
    } else if constexpr (RED == 1) {
      part[(size_t)tk * N + c] = p;
    } else if constexpr (RED == 2) {
      const uint64_t inc = ((uint64_t)(int64_t)__builtin_rintf(p * 16777216.0f) << 12) + 1u;
      const uint64_t now = __hip_atomic_fetch_add(words + c, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
      if ((int)(now & 63u) == splits) {
        out[c] = (_Float16)((float)((int64_t)now >> 12) * (1.0f / 16777216.0f));
        __hip_atomic_store(words + c, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      __hip_atomic_fetch_add(part + c, p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : 4; }

template <int CW, int RW, int W, int RED>
int launch_piece(const void* qw, int R, int N, void* ws, void* out, hipStream_t s) {
  if (R % RW || N % CW || R / RW > 63) return 1;
  auto words = static_cast<uint64_t*>(ws);                                        // [N]
  auto part = reinterpret_cast<float*>(static_cast<char*>(ws) + (size_t)N * 8);  // [R / RW][N]
  probe_piece_kernel<CW, RW, W, RED><<<(N / CW) * (R / RW), W * 64, 0, s>>>(static_cast<const uint32_t*>(qw), R, N,
                                                                          words, part, static_cast<_Float16*>(out));
  return launched();
}

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

// Piece pattern `shape` with reduction `red` (probe_piece_kernel): shape 0 = whole 32-column
// tiles of all R rows, 6 waves (the M = 1 kernel's tile); 1 = 64 x 64 pieces, one wave;
// 2 = 256 x 16 pieces, one wave; 3 = 256 x 4 pieces, one wave. `ws` holds N 64-bit words (zero on
// entry, left zero by red 2) and (R / RW) x N floats; `out` N fp16.
extern "C" int ldk_probe_piece(int shape, int red, const void* qweight, int R, int N, void* ws, void* out,
                               void* stream) {
  if (!qweight || !ws || !out || R <= 0 || N <= 0 || red < 0 || red > 3) return 1;
  (void)hipGetLastError();
  auto s = (hipStream_t)stream;
#define LDK_PIECE(CW, RW, W)                                       \
  switch (red) {                                                   \
    case 0: return launch_piece<CW, RW, W, 0>(qweight, R, N, ws, out, s); \
    case 1: return launch_piece<CW, RW, W, 1>(qweight, R, N, ws, out, s); \
    case 2: return launch_piece<CW, RW, W, 2>(qweight, R, N, ws, out, s); \
    default: return launch_piece<CW, RW, W, 3>(qweight, R, N, ws, out, s); \
  }
  switch (shape) {
    case 0: LDK_PIECE(32, 192, 6)
    case 1: LDK_PIECE(64, 64, 1)
    case 2: LDK_PIECE(256, 16, 1)
    case 3: LDK_PIECE(256, 4, 1)
  }
#undef LDK_PIECE
  return 1;
}
