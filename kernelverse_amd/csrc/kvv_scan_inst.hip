// Instantiates the scan, near-zero and input-select kernels of one element type.  The build
// compiles this file once per dtype code (-DKVV_DT=<kvv_dtype>) so the fifteen
// dtypes compile in parallel; kvv.hip reaches the kernels through the
// kvv_scan_fn_<n> / kvv_near_fn_<n> / kvv_isel_fn_<n> accessors defined here.
#include <hip/hip_runtime.h>

#include "kvv.h"
#include "kvv_kernels.h"
#include "kvv_launch.h"

#ifndef KVV_DT
#error "compile with -DKVV_DT=<kvv_dtype code>"
#endif

namespace kvv {

namespace {
constexpr int kDt = KVV_DT;
constexpr int kNative = Elem<kDt>::is_float ? KVV_MODE_ISCLOSE : KVV_MODE_MAX_ABS_DIFF;
constexpr int kCross = kNative == KVV_MODE_ISCLOSE ? KVV_MODE_MAX_ABS_DIFF : KVV_MODE_ISCLOSE;

template <int MODE, int KIND>
ScanFn pick(bool batch) {
  return batch ? (ScanFn)scan_kernel<kDt, MODE, KIND, true> : (ScanFn)scan_kernel<kDt, MODE, KIND, false>;
}

// single fp16/bf16 pairs whose near-zero diagnostics are taken as entries
constexpr bool kNearEntries = kDt == KVV_F16 || kDt == KVV_BF16;
template <int KIND>
ScanFn pick_nz() {
  if constexpr (kNearEntries) return (ScanFn)scan_kernel<kDt, KVV_MODE_ISCLOSE, KIND, false, true>;
  else return nullptr;
}
}  // namespace

// The dtype's natural test (isclose for floats, max_abs_diff for integers) gets
// the vector kinds; the other test, which only unusual tolerance configs ask
// for, always takes the scalar kind.
ScanFn KVV_SCAN_FN(KVV_DT)(int mode, int kind, bool batch, bool nz) {
  if (nz) {
    if (batch || mode != KVV_MODE_ISCLOSE) return nullptr;
    if (kind == K_CONTIG) return pick_nz<K_CONTIG>();
    if (kind == K_ROWS) return pick_nz<K_ROWS>();
    return nullptr;
  }
  if (mode == kNative) {
    if (kind == K_CONTIG) return pick<kNative, K_CONTIG>(batch);
    if (kind == K_ROWS) return pick<kNative, K_ROWS>(batch);
    return pick<kNative, K_SCALAR>(batch);
  }
  return pick<kCross, K_SCALAR>(batch);
}

NearFn KVV_NEAR_FN(KVV_DT)(int mode) {
  return mode == KVV_MODE_ISCLOSE ? (NearFn)near_kernel<kDt, KVV_MODE_ISCLOSE>
                                  : (NearFn)near_kernel<kDt, KVV_MODE_MAX_ABS_DIFF>;
}

// Input-select kernels that read the inputs (which: 0 fallback, 2 capture
// pivot, 3 capture pass of strided samples): contiguous segments only, so the
// dtype's natural test.
IselFn KVV_ISEL_FN(KVV_DT)(int which) {
  if (which == 2) return (IselFn)isel_pivot_kernel<kDt, kNative>;
  if (which == 3) return (IselFn)isel_capture_kernel<kDt, kNative>;
  return which == 0 ? (IselFn)isel_fallback_kernel<kDt, kNative> : nullptr;
}

}  // namespace kvv
