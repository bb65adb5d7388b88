// Tagged carry slots of the look-back walks (scan_lookback.hip,
// scan_chain.hip), kept in a caller-provided workspace.
#ifndef ASC_LOOKBACK_SLOTS_H
#define ASC_LOOKBACK_SLOTS_H

#include "asc_common.h"

namespace asc {

typedef unsigned long long u64;
// One carry slot per tile, two tagged words: x holds (status << 32 | value)
// with status kLbAgg (the tile's aggregate X) or kLbIncl (its inclusive
// value, the state after the tile); a holds (kLbAgg << 32 | A).  Each word is
// read and written whole, so a reader never sees a value without its tag.
struct LbSlot {
  u64 x, a;
};
enum : uint32_t { kLbNone = 0, kLbAgg = 1, kLbIncl = 2 };

__device__ inline void lb_put(u64* p, uint32_t st, float v) {
  const u64 w = (static_cast<u64>(st) << 32) | __float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline u64 lb_get(u64* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t lb_status(u64 w) { return static_cast<uint32_t>(w >> 32); }
__device__ inline float lb_value(u64 w) {
  return __uint_as_float(static_cast<uint32_t>(w));
}
// Both words of a slot in one round trip; returns the slot's kind.
__device__ inline int lb_read(LbSlot* s, float& a, float& x) {
  const u64 wx = lb_get(&s->x);
  const u64 wa = lb_get(&s->a);
  x = lb_value(wx);
  a = lb_value(wa);
  const uint32_t sx = lb_status(wx);
  if (sx == kLbIncl) return kLbIncl;
  return (sx == kLbAgg && lb_status(wa) == kLbAgg) ? kLbAgg : kLbNone;
}

}  // namespace asc

#endif  // ASC_LOOKBACK_SLOTS_H
