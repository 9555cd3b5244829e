// Index bounds shared by the device code and the host checks of the tests
// (plain C++: no HIP types, so g++ builds it too).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define KVV_HD __host__ __device__
#else
#define KVV_HD
#endif

namespace kvv {

// The keys of one select round's cell that the final read-off reads: the
// round's table gives the cell's start (t_lo) and the next cell's start (t_hi).
// Both are clamped to the round's own sample count (`chunk` samples per round,
// fewer in a group's last round), so lo + len never passes the round's span of
// the sample array, whatever the table words hold.
struct CellSpan {
  uint32_t lo, len;
};

KVV_HD inline CellSpan cell_span(uint32_t t_lo, uint32_t t_hi, int64_t count, int64_t round, int64_t chunk) {
  const int64_t left = count - round * chunk;
  const uint32_t rsz = left <= 0 ? 0u : (left < chunk ? (uint32_t)left : (uint32_t)chunk);
  uint32_t lo = t_lo < rsz ? t_lo : rsz;
  uint32_t len = t_hi - t_lo;  // wraps when the words are out of order: the clamp below bounds it
  len = len <= rsz - lo ? len : rsz - lo;
  return CellSpan{lo, len};
}

}  // namespace kvv
