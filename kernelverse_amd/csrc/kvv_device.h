// Device-side element decoding, ordering keys and wave/block reductions for
// the verdict kernels.  Compiled for gfx950 only (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <limits>
#include <type_traits>

#include "kvv.h"
#include "kvv_bounds.h"

namespace kvv {

constexpr int kBlock = 256;           // threads per block (4 waves of 64)
constexpr int kWaves = kBlock / 64;
constexpr int kBuckets = KVV_HIST_BUCKETS;
constexpr uint64_t kNone = ~0ull;     // "no index yet"
constexpr uint32_t kNone32 = ~0u;     // the same for 32-bit offsets

// Per-thread LDS counters (one column per thread, so increments never collide).
enum LdsCounter {
  LC_VIOL = 0, LC_NAN_G, LC_NAN_R, LC_PINF_G, LC_PINF_R, LC_NINF_G, LC_NINF_R, LC_NANPAIR,
  LC_NEAR, LC_FARMM, LC_NEARBAD,
  LC_HIST0,  // + bucket
  LC_COUNT = LC_HIST0 + kBuckets
};

// ---------------------------------------------------------------- float keys
// Monotone map float -> uint32 (NaN is above +inf): ascending key == ascending value.
__device__ __forceinline__ uint32_t fkey(float x) {
  uint32_t b = __float_as_uint(x);
  if (__builtin_isnan(x)) return 0xFFFFFFFFu;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__host__ __device__ inline float fkey_value(uint32_t k) {
  if (k == 0xFFFFFFFFu) return __builtin_nanf("");
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  float f;
  __builtin_memcpy(&f, &b, 4);
  return f;
}
// Monotone map int32 -> uint32.
__device__ __forceinline__ uint32_t ikey(int32_t x) { return (uint32_t)x ^ 0x80000000u; }
__host__ __device__ inline int32_t ikey_value(uint32_t k) { return (int32_t)(k ^ 0x80000000u); }

// x86 semantics of float -> int32 truncation (cvttss2si / cvttsd2si): NaN and
// out-of-range values give INT32_MIN.  torch-CPU's Tensor.to(torch.int32) runs that.
__device__ __forceinline__ int32_t x86_trunc_i32(double x) {
  if (!(x > -2147483649.0 && x < 2147483648.0)) return INT32_MIN;
  return (int32_t)x;
}

// Bucket of a ULP / integer distance: 0 for 0, else min(bit_length(d), 15).
__device__ __forceinline__ int ulp_bucket(uint64_t d) {
  if (d == 0) return 0;
  int bl = 64 - __clzll(d);
  return bl < kBuckets - 1 ? bl : kBuckets - 1;
}

// ------------------------------------------------------------ element traits
// T is the raw storage type; decoding never rounds except where torch rounds
// too (float64 -> float32, int64 -> float32).
template <int DT> struct Elem;

struct FloatElemBase { static constexpr bool is_float = true; };
struct IntElemBase { static constexpr bool is_float = false; };

template <> struct Elem<KVV_F32> : FloatElemBase {
  using T = uint32_t;
  static constexpr int width = 32;
  __device__ static float f32(T c) { return __uint_as_float(c); }
  __device__ static double f64(T c) { return (double)__uint_as_float(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32((double)__uint_as_float(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7FFFFFFFu) > 0x7F800000u; }
  __device__ static bool isinf(T c) { return (c & 0x7FFFFFFFu) == 0x7F800000u; }
  __device__ static bool finite(T c) { return (c & 0x7F800000u) != 0x7F800000u; }
  __device__ static bool sign(T c) { return c >> 31; }
  __device__ static uint64_t mag(T c) { return c & 0x7FFFFFFFu; }
};

template <> struct Elem<KVV_BF16> : FloatElemBase {
  using T = uint16_t;
  static constexpr int width = 16;
  __device__ static float f32(T c) { return __uint_as_float((uint32_t)c << 16); }
  __device__ static double f64(T c) { return (double)f32(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32((double)f32(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7FFFu) > 0x7F80u; }
  __device__ static bool isinf(T c) { return (c & 0x7FFFu) == 0x7F80u; }
  __device__ static bool finite(T c) { return (c & 0x7F80u) != 0x7F80u; }
  __device__ static bool sign(T c) { return c >> 15; }
  __device__ static uint64_t mag(T c) { return c & 0x7FFFu; }
};

template <> struct Elem<KVV_F16> : FloatElemBase {
  using T = uint16_t;
  static constexpr int width = 16;
  __device__ static float f32(T c) { return (float)__builtin_bit_cast(_Float16, c); }
  __device__ static double f64(T c) { return (double)f32(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32((double)f32(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7FFFu) > 0x7C00u; }
  __device__ static bool isinf(T c) { return (c & 0x7FFFu) == 0x7C00u; }
  __device__ static bool finite(T c) { return (c & 0x7C00u) != 0x7C00u; }
  __device__ static bool sign(T c) { return c >> 15; }
  __device__ static uint64_t mag(T c) { return c & 0x7FFFu; }
};

template <> struct Elem<KVV_F64> : FloatElemBase {
  using T = uint64_t;
  static constexpr int width = 64;
  __device__ static double f64(T c) { return __longlong_as_double((long long)c); }
  __device__ static float f32(T c) { return (float)f64(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32(f64(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7FFFFFFFFFFFFFFFull) > 0x7FF0000000000000ull; }
  __device__ static bool isinf(T c) { return (c & 0x7FFFFFFFFFFFFFFFull) == 0x7FF0000000000000ull; }
  __device__ static bool finite(T c) { return (c & 0x7FF0000000000000ull) != 0x7FF0000000000000ull; }
  __device__ static bool sign(T c) { return c >> 63; }
  __device__ static uint64_t mag(T c) { return c & 0x7FFFFFFFFFFFFFFFull; }
};

// OCP float8 e4m3fn: bias 7, no infinities, S.1111.111 is NaN, max 448.
template <> struct Elem<KVV_F8E4M3FN> : FloatElemBase {
  using T = uint8_t;
  static constexpr int width = 8;
  // gfx950's v_cvt_f32_fp8 decodes OCP e4m3fn exactly: every one of the 256
  // codes (NaN, subnormals and both zeros included) matched a decode from the
  // format's definition on the device.
  __device__ static float f32(T c) { return __builtin_amdgcn_cvt_f32_fp8((int)c, 0); }
  __device__ static double f64(T c) { return (double)f32(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32((double)f32(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7Fu) == 0x7Fu; }
  __device__ static bool isinf(T) { return false; }
  __device__ static bool finite(T c) { return (c & 0x7Fu) != 0x7Fu; }
  __device__ static bool sign(T c) { return c >> 7; }
  __device__ static uint64_t mag(T c) { return c & 0x7Fu; }
};

// float8 e5m2 is the high byte of an IEEE half.
template <> struct Elem<KVV_F8E5M2> : FloatElemBase {
  using T = uint8_t;
  static constexpr int width = 8;
  // (v_cvt_f32_bf8 decodes OCP e5m2 exactly, as checked over all 256 codes)
  __device__ static float f32(T c) { return __builtin_amdgcn_cvt_f32_bf8((int)c, 0); }
  __device__ static double f64(T c) { return (double)f32(c); }
  __device__ static int32_t i32(T c) { return x86_trunc_i32((double)f32(c)); }
  __device__ static bool isnan(T c) { return (c & 0x7Fu) > 0x7Cu; }
  __device__ static bool isinf(T c) { return (c & 0x7Fu) == 0x7Cu; }
  __device__ static bool finite(T c) { return (c & 0x7Cu) != 0x7Cu; }
  __device__ static bool sign(T c) { return c >> 7; }
  __device__ static uint64_t mag(T c) { return c & 0x7Fu; }
};

template <typename Raw, typename Signed>
struct IntElem : IntElemBase {
  using T = Raw;
  static constexpr int width = 8 * sizeof(Raw);
  __device__ static int64_t v(T c) { return (int64_t)(Signed)c; }
  __device__ static float f32(T c) { return (float)v(c); }     // RNE, as torch's int -> float32
  __device__ static double f64(T c) { return (double)v(c); }
  __device__ static int32_t i32(T c) { return (int32_t)(uint32_t)(uint64_t)v(c); }  // wraps like .to(int32)
  __device__ static bool isnan(T) { return false; }
  __device__ static bool isinf(T) { return false; }
  __device__ static bool finite(T) { return true; }
};
template <> struct Elem<KVV_I8> : IntElem<uint8_t, int8_t> {};
template <> struct Elem<KVV_U8> : IntElem<uint8_t, uint8_t> {};
template <> struct Elem<KVV_I16> : IntElem<uint16_t, int16_t> {};
template <> struct Elem<KVV_I32> : IntElem<uint32_t, int32_t> {};
template <> struct Elem<KVV_I64> : IntElem<uint64_t, int64_t> {};
template <> struct Elem<KVV_U16> : IntElem<uint16_t, uint16_t> {};
template <> struct Elem<KVV_U32> : IntElem<uint32_t, uint32_t> {};
// uint64: the float conversions take the unsigned value (torch's uint64 ->
// float32/float64); v(), which only the integer ULP distance reads, is the
// int64 reinterpretation of the code.
template <> struct Elem<KVV_U64> : IntElem<uint64_t, int64_t> {
  __device__ static float f32(T c) { return (float)c; }
  __device__ static double f64(T c) { return (double)c; }
};
template <> struct Elem<KVV_BOOL> : IntElemBase {
  using T = uint8_t;
  static constexpr int width = 8;
  __device__ static int64_t v(T c) { return c != 0; }
  __device__ static float f32(T c) { return c != 0 ? 1.0f : 0.0f; }
  __device__ static double f64(T c) { return c != 0 ? 1.0 : 0.0; }
  __device__ static int32_t i32(T c) { return c != 0; }
  __device__ static bool isnan(T) { return false; }
  __device__ static bool isinf(T) { return false; }
  __device__ static bool finite(T) { return true; }
};

// Bucket of a ULP / integer distance (width <= 32 bits).
__device__ __forceinline__ int ulp_bucket32(uint32_t d) {
  const int bl = 32 - __clz(d);  // 0 for d == 0
  return bl < kBuckets - 1 ? bl : kBuckets - 1;
}

// ULP / integer distance bucket of a pair (never called for NaN pairs).  Float
// codes compare as sign-magnitude (through zero for opposite signs, so +0 and
// -0 coincide); integers by value.  Types of at most 32 bits stay in 32-bit math.
template <int DT>
__device__ __forceinline__ int pair_bucket(typename Elem<DT>::T g, typename Elem<DT>::T r) {
  using E = Elem<DT>;
  if constexpr (E::width <= 32) {
    if constexpr (E::is_float) {
      const uint32_t mg = (uint32_t)E::mag(g), mr = (uint32_t)E::mag(r);
      const uint32_t d = (E::sign(g) == E::sign(r)) ? (mg > mr ? mg - mr : mr - mg) : mg + mr;
      return ulp_bucket32(d);
    } else {
      const int64_t a = E::v(g), b = E::v(r);
      return ulp_bucket32((uint32_t)(a > b ? a - b : b - a));
    }
  } else {
    uint64_t d;
    if constexpr (E::is_float) {
      const uint64_t mg = E::mag(g), mr = E::mag(r);
      d = (E::sign(g) == E::sign(r)) ? (mg > mr ? mg - mr : mr - mg) : mg + mr;
    } else {
      const int64_t a = E::v(g), b = E::v(r);
      d = a > b ? (uint64_t)a - (uint64_t)b : (uint64_t)b - (uint64_t)a;
    }
    return ulp_bucket(d);
  }
}

// ----------------------------------------------------------------- reductions
// Wave reductions through DPP: row shifts by 1, 2, 4 and 8, then the row
// broadcasts of lanes 15 and 31, leave lane 63 with the result of the whole
// wave, which readlane hands to every lane.  No LDS round trips (a shuffle is
// a ds_bpermute each), and the tree is fixed, so fp64 sums are reproducible.
// `ident` fills lanes whose DPP source lies outside the row.
template <int CTRL, int RM, typename T>
__device__ __forceinline__ T dpp_move(T v, T ident) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ident), __builtin_bit_cast(int, v),
                                                             CTRL, RM, 0xf, false));
  } else {
    static_assert(sizeof(T) == 8, "32- or 64-bit lanes");
    const uint64_t b = __builtin_bit_cast(uint64_t, v), o = __builtin_bit_cast(uint64_t, ident);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)o, (int)(uint32_t)b, CTRL, RM, 0xf, false);
    const uint32_t hi =
        (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(o >> 32), (int)(uint32_t)(b >> 32), CTRL, RM, 0xf, false);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}
template <typename T>
__device__ __forceinline__ T lane63(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, T ident, Op op) {
  v = op(v, dpp_move<0x111, 0xf>(v, ident));  // row_shr:1
  v = op(v, dpp_move<0x112, 0xf>(v, ident));  // row_shr:2
  v = op(v, dpp_move<0x114, 0xf>(v, ident));  // row_shr:4
  v = op(v, dpp_move<0x118, 0xf>(v, ident));  // row_shr:8
  v = op(v, dpp_move<0x142, 0xa>(v, ident));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_move<0x143, 0xc>(v, ident));  // row_bcast:31 into rows 2 and 3
  return lane63(v);
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return wave_reduce(v, (T)0, [](T x, T y) { return x + y; });
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  return wave_reduce(v, std::numeric_limits<T>::lowest(), [](T x, T y) { return y > x ? y : x; });
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
  return wave_reduce(v, std::numeric_limits<T>::max(), [](T x, T y) { return y < x ? y : x; });
}
// (key, index) argmax: larger key wins, equal keys -> smaller index.
template <typename I>
__device__ __forceinline__ void wave_argmax_t(uint32_t& key, I& idx) {
  auto step = [&](uint32_t k, I i) {
    if (k > key || (k == key && i < idx)) {
      key = k;
      idx = i;
    }
  };
  const I none = std::numeric_limits<I>::max();
  step(dpp_move<0x111, 0xf>(key, 0u), dpp_move<0x111, 0xf>(idx, none));
  step(dpp_move<0x112, 0xf>(key, 0u), dpp_move<0x112, 0xf>(idx, none));
  step(dpp_move<0x114, 0xf>(key, 0u), dpp_move<0x114, 0xf>(idx, none));
  step(dpp_move<0x118, 0xf>(key, 0u), dpp_move<0x118, 0xf>(idx, none));
  step(dpp_move<0x142, 0xa>(key, 0u), dpp_move<0x142, 0xa>(idx, none));
  step(dpp_move<0x143, 0xc>(key, 0u), dpp_move<0x143, 0xc>(idx, none));
  key = lane63(key);
  idx = lane63(idx);
}
__device__ __forceinline__ void wave_argmax(uint32_t& key, uint64_t& idx) { wave_argmax_t(key, idx); }
__device__ __forceinline__ void wave_argmax32(uint32_t& key, uint32_t& idx) { wave_argmax_t(key, idx); }
__device__ __forceinline__ bool better(uint32_t k, uint64_t i, uint32_t bk, uint64_t bi) {
  return k > bk || (k == bk && i < bi);
}
__device__ __forceinline__ bool better32(uint32_t k, uint32_t i, uint32_t bk, uint32_t bi) {
  return k > bk || (k == bk && i < bi);
}

}  // namespace kvv
