// Internal interface of the prefill (many-row) weight-only GEMMs in prefill.hip, called by the
// ldk_w4a16_matmul dispatch in w4a16.hip and the ldk_w8a16_matmul dispatch in fp8.hip. Not part
// of the C ABI.
#pragma once

#include <stdint.h>

#include "ldk_common.h"

namespace ldk {

// Weight formats of the prefill GEMM.
enum class WFmt {
  kInt4,  // packed int4 [K/8, N] int32 words, asymmetric: fp16 scales and zeros [K/group, N]
  kE4M3,  // OCP float8 e4m3fn [K, N] bytes, one fp16 scale per output column [N]
};

struct GemmArgs {
  const half_t* x;  // [M, K] fp16, row stride ldx
  int64_t ldx;
  const void* w;       // weights in the format's layout
  const half_t* s;     // kInt4: scales [K/group, N]; kE4M3: column scales [N]
  const half_t* z;     // kInt4: zeros [K/group, N]; kE4M3: unused
  const half_t* bias;  // [N] or null
  half_t* out;         // [M, N] fp16, row stride ldo
  int64_t ldo;
  int M, N, K;
  int group_size;    // kInt4: a power of two >= 64 dividing K
  void* workspace;   // fp32 partial tiles of a K split (may be null: no split)
  int64_t workspace_bytes;
  int block_n;       // output-tile width 128 or 256 (0: the library's choice)
  int split_k;       // workgroups splitting K per tile (0: the library's choice)
  // 1: SwiGLU fused into the epilogue. The product's columns [0, N/2) are g and [N/2, N) are u
  // (the reference's swiglu_fused halves); out [M, N/2] (row stride ldo) receives
  // fp16(silu(g)) * u of the fp16-rounded products, the standalone SwiGLU's steps. Only where
  // gemm_swiglu_applies.
  int swiglu = 0;
};

// Whether the prefill GEMM takes this shape (K a multiple of 64; kInt4: group_size >= 64, N a
// multiple of 8; kE4M3: N a multiple of 16; sizes within its 32-bit buffer offsets), and launches
// it (with a K split over workgroups when the shape's K is long and the workspace holds the
// partials; a second launch then sums them in split order). Both leave the last-error message on
// failure.
bool gemm_supported(WFmt f, int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx);
int gemm_launch(WFmt f, const GemmArgs& a, hipStream_t stream);

// The output-tile width (columns per workgroup) and the number of K splits gemm_launch uses for a
// shape with these tuning arguments and a workspace of ws_bytes (for plan queries).
void gemm_plan(WFmt f, int64_t M, int64_t N, int64_t K, int block_n, int split_k, int64_t ws_bytes, int* tile_n,
               int* splits);

// Whether gemm_launch takes GemmArgs::swiglu for this shape: a plan of at least two column groups
// per workgroup (half of them compute g, the other half the matching u columns), no K split, and
// N / 2 a multiple of the workgroup's g columns.
bool gemm_swiglu_applies(WFmt f, int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx, int block_n,
                         int split_k, int64_t ws_bytes);

// Name of the kernel instantiation gemm_launch runs for a shape (for reports).
const char* gemm_kernel_name(WFmt f, int64_t M, int64_t N, int64_t K, int block_n);

}  // namespace ldk
