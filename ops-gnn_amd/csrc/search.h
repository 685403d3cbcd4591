// Wavefront-cooperative searches over sorted pointer arrays.
#pragma once

#include "ogn_device.h"

namespace ogn {

// Upper bound of `key` in ptr[0 .. n) for two keys at once: lanes 0-31 search
// key_lo, lanes 32-63 key_hi.  Each round probes 32 evenly spaced entries
// and keeps the bracket between the last probe <= key and the first > key,
// so 10^6 rows take 4 rounds of one load each (instead of 20 dependent
// loads of a per-thread binary search).  Called by the whole wavefront.
template <typename IDX>
__device__ __forceinline__ int64_t wave_upper_bound2(const IDX* __restrict__ ptr, int64_t n, int64_t key_lo,
                                                     int64_t key_hi) {
  const int lane = lane_id();
  const int half = lane >> 5, j = lane & 31;
  const int64_t key = half ? key_hi : key_lo;
  int64_t lo = 0, hi = n;
  while (true) {
    const bool done = lo >= hi;
    if (__all(done)) break;
    const int64_t step = done ? 1 : (hi - lo + 31) / 32;
    const int64_t q = lo + (int64_t)j * step;
    const bool valid = !done && q < hi;
    const bool le = valid && (int64_t)ptr[q] <= key;
    const uint64_t m = __ballot(le);
    const uint64_t mv = __ballot(valid);
    const uint32_t mh = (uint32_t)(half ? (m >> 32) : m);
    const uint32_t vh = (uint32_t)(half ? (mv >> 32) : mv);
    const int c = __popc(mh);  // probes <= key form a prefix of the valid ones
    const int nv = __popc(vh);
    if (!done) {
      const int64_t nlo = c > 0 ? lo + (int64_t)(c - 1) * step + 1 : lo;
      const int64_t nhi = c < nv ? lo + (int64_t)c * step : hi;
      lo = nlo;
      hi = c > 0 ? nhi : lo;
    }
  }
  return lo;
}

}  // namespace ogn
