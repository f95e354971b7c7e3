// Internal interface of the prefill (many-row) W4A16 GEMM in prefill.hip, called by the
// ldk_w4a16_matmul dispatch in w4a16.hip. Not part of the C ABI.
#pragma once

#include <stdint.h>

#include "ldk_common.h"

namespace ldk {

struct W4GemmArgs {
  const half_t* x;  // [M, K] fp16, row stride ldx
  int64_t ldx;
  const uint32_t* qw;  // packed int4 [K/8, N]
  const half_t* s;     // scales [K/group, N]
  const half_t* z;     // zeros [K/group, N]
  const half_t* bias;  // [N] or null
  half_t* out;         // [M, N] fp16, row stride ldo
  int64_t ldo;
  int M, N, K;
  int group_size;    // a power of two >= 64 dividing K
  void* workspace;   // fp32 partial tiles of a K split (may be null: no split)
  int64_t workspace_bytes;
  int block_n;       // output-tile width 128 or 256 (0: the library's choice)
  int split_k;       // workgroups splitting K per tile (0: the library's choice)
};

// Whether the prefill GEMM takes this shape (group_size >= 64, K a multiple of 64, N a multiple
// of 8, sizes within its indexing), and launches it (with a K split over workgroups when the
// shape gives too few tiles and the workspace holds the partials; a second launch then sums them
// in split order). Both leave the last-error message on failure.
bool w4a16_gemm_supported(int64_t M, int64_t N, int64_t K, int group_size, int64_t ldx);
int w4a16_gemm_launch(const W4GemmArgs& a, hipStream_t stream);

// Name of the kernel instantiation w4a16_gemm_launch runs for a shape (for reports).
const char* w4a16_gemm_kernel_name(int64_t M, int64_t N, int64_t K, int block_n);

}  // namespace ldk
