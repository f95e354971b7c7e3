// Cache warming by spare workgroups of a launch: byte ranges that later launches will read (the
// next projections' weights) are read, with nothing written, by extra workgroups dispatched after
// a launch's own, so that they come from the MALL (and the reading XCD's L2) instead of HBM when
// their consumer runs. Used by the decode attention (attention.hip), whose few workgroups leave
// most CUs idle. Not part of the C ABI.
#pragma once

#include <stdint.h>

#include <algorithm>

#include "ldk_common.h"

namespace ldk {

// Range k is p[k] [0, end[k] - end[k - 1]) in 16-byte units and is read by the warming
// workgroups [wg_end[k - 1], wg_end[k]); both cumulative, entries past the used ones repeat the
// last values (empty ranges with no workgroups).
constexpr int kWarmMax = 8;
struct WarmRanges {
  const u32x4* p[kWarmMax];
  uint32_t end[kWarmMax];
  uint32_t wg_end[kWarmMax];
};

// Warming workgroup wg of LANES lanes: its range found from the cumulative workgroup counts
// (scalar selects, no indexing), then LOADS 16-byte loads per lane in flight over its share of the
// range, each value consumed by an empty asm so that the loads are kept and completed. Indices
// past the range's end re-read its last 16 bytes (in bounds). Every range is read at the same time.
template <int LANES, int LOADS>
__device__ __forceinline__ void warm_read(const WarmRanges& w, uint32_t wg) {
  const u32x4* p = w.p[0];
  uint32_t beg = 0, n = w.end[0], wbeg = 0, nw = w.wg_end[0];
#pragma unroll
  for (int k = 1; k < kWarmMax; ++k) {
    const bool in = wg >= w.wg_end[k - 1];
    p = in ? w.p[k] : p;
    beg = in ? w.end[k - 1] : beg;
    n = in ? w.end[k] : n;
    wbeg = in ? w.wg_end[k - 1] : wbeg;
    nw = in ? w.wg_end[k] : nw;
  }
  n -= beg;
  const uint32_t step = (nw - wbeg) * LANES;
  for (uint32_t i0 = (wg - wbeg) * LANES + threadIdx.x; i0 < n; i0 += LOADS * step) {
    u32x4 v[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) v[u] = p[min(i0 + u * step, n - 1)];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) asm volatile("" ::"v"(v[u]));
  }
}

// The warm ranges of a launch from the caller's arrays (nwarm of them, 0..kWarmMax; each pointer
// non-null and 16-byte aligned, each size a multiple of 16, under 32 GiB in all), and the number
// of warming workgroups to add to its grid: enough for LOADS loads per lane where they all fit in
// max_wg, else in proportion to each range's bytes (at least one per non-empty range).
inline int make_warm(const void* const* warm, const int64_t* warm_bytes, int nwarm, const char* what, int lanes,
                     int loads, int max_wg, WarmRanges& w, uint32_t& nwg) {
  w = WarmRanges{};
  nwg = 0;
  if (nwarm < 0 || nwarm > kWarmMax || (nwarm > 0 && (!warm || !warm_bytes)))
    return fail(LDK_ERR_INVALID, "%s: nwarm=%d must be 0..%d with both arrays", what, nwarm, kWarmMax);
  const uint64_t per_wg = (uint64_t)lanes * loads;  // 16-byte units one workgroup pass reads
  uint64_t end = 0, need = 0;
  for (int k = 0; k < nwarm; ++k) {
    if (!warm[k] || warm_bytes[k] < 0 || warm_bytes[k] % 16 || !aligned(warm[k], 16))
      return fail(LDK_ERR_ALIGN, "%s: warm range %d must be non-null, 16-byte aligned, a multiple of 16 bytes (%lld)",
                  what, k, (long long)warm_bytes[k]);
    end += (uint64_t)warm_bytes[k] / 16;
    if (end >= (1ull << 31)) return fail(LDK_ERR_UNSUPPORTED, "%s: warm ranges above 32 GiB", what);
    w.p[k] = static_cast<const u32x4*>(warm[k]);
    w.end[k] = (uint32_t)end;
    need += ((uint64_t)warm_bytes[k] / 16 + per_wg - 1) / per_wg;
  }
  uint32_t wge = 0;
  for (int k = 0; k < nwarm; ++k) {
    const uint64_t units = w.end[k] - (k ? w.end[k - 1] : 0);
    uint64_t c = (units + per_wg - 1) / per_wg;
    if (need > (uint64_t)max_wg && units) c = std::max<uint64_t>(1, units * (uint64_t)(max_wg - kWarmMax) / end);
    wge += (uint32_t)c;
    w.wg_end[k] = wge;
  }
  for (int k = nwarm; k < kWarmMax; ++k) {  // empty ranges
    w.p[k] = nwarm ? w.p[nwarm - 1] : nullptr;
    w.end[k] = (uint32_t)end;
    w.wg_end[k] = wge;
  }
  nwg = wge;
  return LDK_OK;
}

}  // namespace ldk
