// Internal interface between the decode attention (attention.hip) and the W4A16 o projection that
// merges its position ranges in its x staging (w4a16.hip). Not part of the C ABI.
#pragma once

#include <stdint.h>

#include "ldk_common.h"

namespace ldk {

constexpr int kAttnHeadDim = 128;  // head_dim of the decode attention
constexpr int kAttnMaxSplits = 32;  // position ranges per head the partials hold
constexpr int kAttnMaxHeads = 128;  // query heads the partials hold

// Device addresses, on the current device, of the decode attention's per-range partials: `ml` is
// float [kAttnMaxHeads][kAttnMaxSplits][2] = {running max, sum} and `o` float
// [kAttnMaxHeads][kAttnMaxSplits][kAttnHeadDim], the unnormalised outputs. Written by the range
// kernel of ldk_decode_attention_ranges, read by the launches after it on the same stream. The
// host records the stream, position array and geometry of the last ldk_decode_attention_ranges
// call per device (and forgets them when ldk_decode_attention's own range launch overwrites the
// partials): a consumer on another stream, with another position array or geometry, or with no
// ranges pending is refused (LDK_ERR_INVALID, naming `what`).
int attention_partials(const char* what, void* stream, const int64_t* pos, int64_t max_len, int64_t rlen, int nq,
                       const float** o, const float** ml);

}  // namespace ldk
