// Kernel accessors shared between the per-dtype instantiation units and kvv.hip.
#pragma once

#include "kvv_kernels.h"

namespace kvv {

using ScanFn = void (*)(ScanArgs);
using NearFn = void (*)(NearArgs);
using IselFn = void (*)(IselArgs);

#define KVV_CAT_(a, b) a##b
#define KVV_CAT(a, b) KVV_CAT_(a, b)
#define KVV_SCAN_FN(dt) KVV_CAT(kvv_scan_fn_, dt)
#define KVV_NEAR_FN(dt) KVV_CAT(kvv_near_fn_, dt)
#define KVV_ISEL_FN(dt) KVV_CAT(kvv_isel_fn_, dt)

#define KVV_DECLARE(dt)                          \
  ScanFn KVV_SCAN_FN(dt)(int mode, int kind, bool batch, bool nz); \
  NearFn KVV_NEAR_FN(dt)(int mode);                      \
  IselFn KVV_ISEL_FN(dt)(int which);

KVV_DECLARE(0)
KVV_DECLARE(1)
KVV_DECLARE(2)
KVV_DECLARE(3)
KVV_DECLARE(4)
KVV_DECLARE(5)
KVV_DECLARE(6)
KVV_DECLARE(7)
KVV_DECLARE(8)
KVV_DECLARE(9)
KVV_DECLARE(10)
KVV_DECLARE(11)
KVV_DECLARE(12)
KVV_DECLARE(13)
KVV_DECLARE(14)

}  // namespace kvv
