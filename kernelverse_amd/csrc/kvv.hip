// libkvv: MI355X verdict library -- C ABI entry points (include/kvv.h),
// planning (dimension coalescing, layout and access choice, workspace
// layout) and the launch sequence of the verdict kernels.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "kvv.h"
#define KVV_COMMON_KERNELS 1  // reduce/select live in this unit only
#include "kvv_kernels.h"
#include "kvv_launch.h"

namespace kvv {
namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define KVV_HIP(call)                                                                                \
  do {                                                                                               \
    hipError_t e_ = (call);                                                                          \
    if (e_ != hipSuccess) return fail(KVV_E_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

constexpr int64_t kMaxNumel = int64_t(1) << 40;
constexpr int64_t kMaxSamplesCap = int64_t(1) << 24;

int elem_size(int dt) {
  switch (dt) {
    case KVV_F32: case KVV_I32: case KVV_U32: return 4;
    case KVV_F16: case KVV_BF16: case KVV_I16: case KVV_U16: return 2;
    case KVV_F64: case KVV_I64: case KVV_U64: return 8;
    case KVV_F8E4M3FN: case KVV_F8E5M2: case KVV_I8: case KVV_U8: case KVV_BOOL: return 1;
    default: return 0;
  }
}

bool is_float_dtype(int dt) {
  return dt == KVV_F32 || dt == KVV_F16 || dt == KVV_BF16 || dt == KVV_F64 || dt == KVV_F8E4M3FN || dt == KVV_F8E5M2;
}

// One item is one wave's unit of work: 64 lanes x kUnroll 16-byte vectors of each tensor.
int item_elems_for(int dt) { return 64 * (16 / elem_size(dt)) * kUnroll; }

int device_cus() {
  static thread_local int cached_dev = -1, cached_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

// Persistent-style grid: exactly as many blocks as the device keeps resident for
// this kernel (one round, no straggler round), each streaming a contiguous
// range of items.
int64_t blocks_target(ScanFn fn) {
  // resident blocks per CU of each kernel seen on this thread (a few dozen at most)
  struct Occ {
    ScanFn fn;
    int dev, nb;
  };
  static thread_local Occ cache[64];
  static thread_local int used = 0;
  int dev = 0;
  (void)hipGetDevice(&dev);
  int nb = 0;
  for (int i = 0; i < used; ++i)
    if (cache[i].fn == fn && cache[i].dev == dev) nb = cache[i].nb;
  if (nb == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(fn), kBlock, 0) != hipSuccess ||
        nb <= 0)
      nb = 2;
    cache[used < 64 ? used++ : 63] = Occ{fn, dev, nb};
  }
  const int64_t b = (int64_t)device_cus() * nb;
  return b < 4096 ? b : 4096;
}

// Which scan kernel a segment takes: the vector kinds need the dtype's natural
// test and 16-byte aligned contiguous rows; everything else is scalar.
int scan_kind(const SegDesc& d) {
  const int native = is_float_dtype(d.dtype) ? KVV_MODE_ISCLOSE : KVV_MODE_MAX_ABS_DIFF;
  if (d.mode != native || !d.vec) return K_SCALAR;
  return d.layout == L_CONTIG ? K_CONTIG : K_ROWS;
}

ScanFn scan_fn(int dt, int mode, int kind, bool batch, bool nz = false) {
  switch (dt) {
#define KVV_CASE(X) case X: return KVV_SCAN_FN(X)(mode, kind, batch, nz);
    KVV_CASE(0) KVV_CASE(1) KVV_CASE(2) KVV_CASE(3) KVV_CASE(4) KVV_CASE(5)
    KVV_CASE(6) KVV_CASE(7) KVV_CASE(8) KVV_CASE(9) KVV_CASE(10) KVV_CASE(11)
    KVV_CASE(12) KVV_CASE(13) KVV_CASE(14)
#undef KVV_CASE
    default: return nullptr;
  }
}

IselFn isel_fn(int dt, int which) {
  switch (dt) {
#define KVV_CASE(X) case X: return KVV_ISEL_FN(X)(which);
    KVV_CASE(0) KVV_CASE(1) KVV_CASE(2) KVV_CASE(3) KVV_CASE(4) KVV_CASE(5)
    KVV_CASE(6) KVV_CASE(7) KVV_CASE(8) KVV_CASE(9) KVV_CASE(10) KVV_CASE(11)
    KVV_CASE(12) KVV_CASE(13) KVV_CASE(14)
#undef KVV_CASE
    default: return nullptr;
  }
}

NearFn near_fn(int dt, int mode) {
  switch (dt) {
#define KVV_CASE(X) case X: return KVV_NEAR_FN(X)(mode);
    KVV_CASE(0) KVV_CASE(1) KVV_CASE(2) KVV_CASE(3) KVV_CASE(4) KVV_CASE(5)
    KVV_CASE(6) KVV_CASE(7) KVV_CASE(8) KVV_CASE(9) KVV_CASE(10) KVV_CASE(11)
    KVV_CASE(12) KVV_CASE(13) KVV_CASE(14)
#undef KVV_CASE
    default: return nullptr;
  }
}

// Largest magnitude code of a 16-bit float type whose value is at most t, or -1
// when even +0 is above t (t negative or NaN): |ref| <= t <=> (code & 0x7FFF) <= it.
float half_value(int dt, uint32_t mag) {
  if (dt == KVV_BF16) {
    const uint32_t b = mag << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
  }
  const uint32_t e = (mag >> 10) & 31u, m = mag & 1023u;
  if (e == 31) return m ? __builtin_nanf("") : __builtin_inff();
  return e == 0 ? std::ldexp((float)m, -24) : std::ldexp((float)(m | 1024u), (int)e - 25);
}

int32_t near_code(int dt, float t) {
  if (dt != KVV_F16 && dt != KVV_BF16) return -1;
  if (!(half_value(dt, 0) <= t)) return -1;
  uint32_t lo = 0, hi = dt == KVV_BF16 ? 0x7F80u : 0x7C00u;  // magnitudes up to the infinity code ascend
  if (half_value(dt, hi) <= t) return (int32_t)hi;
  while (hi - lo > 1) {  // value(lo) <= t < value(hi)
    const uint32_t mid = (lo + hi) / 2;
    if (half_value(dt, mid) <= t) lo = mid; else hi = mid;
  }
  return (int32_t)lo;
}

// Coalesces the joint (size, gen stride, ref stride) dims and picks the layout.
// Select blocks per array of a group of m samples: one for a small group, one
// per `rounds` x kSelChunk samples otherwise.
int64_t select_chunks(int64_t m, int rounds) {
  if (m == 0) return 0;
  if (m <= kSmall) return 1;
  const int64_t per = (int64_t)rounds * kSelChunk;
  return (m + per - 1) / per;
}

int plan_segment(const kvv_tensor* g, const kvv_tensor* r, const kvv_policy* p, SegDesc& d) {
  if (!g || !r || !p) return fail(KVV_E_INVALID, "null tensor or policy");
  if (g->dtype != r->dtype) return fail(KVV_E_INVALID, "generated and reference dtypes differ");
  const int es = elem_size(r->dtype);
  if (es == 0) return fail(KVV_E_INVALID, "unknown dtype code " + std::to_string(r->dtype));
  if (g->ndim != r->ndim || r->ndim < 0 || r->ndim > KVV_MAX_DIMS)
    return fail(KVV_E_INVALID, "ndim mismatch or out of range");
  int64_t n = 1;
  for (int i = 0; i < r->ndim; ++i) {
    if (g->sizes[i] != r->sizes[i]) return fail(KVV_E_INVALID, "shapes differ");
    if (r->sizes[i] < 0) return fail(KVV_E_INVALID, "negative size");
    if (r->sizes[i] > 0 && n > kMaxNumel / r->sizes[i]) return fail(KVV_E_UNSUPPORTED, "more than 2^40 elements");
    n *= r->sizes[i];
  }
  if (n > kMaxNumel) return fail(KVV_E_UNSUPPORTED, "more than 2^40 elements");
  if (p->mode != KVV_MODE_ISCLOSE && p->mode != KVV_MODE_MAX_ABS_DIFF) return fail(KVV_E_INVALID, "bad mode");
  if (p->mode == KVV_MODE_MAX_ABS_DIFF && (p->max_abs_diff < INT32_MIN || p->max_abs_diff > INT32_MAX))
    return fail(KVV_E_INVALID, "max_abs_diff does not fit int32");
  if (p->max_samples < 2 || p->max_samples > kMaxSamplesCap)
    return fail(KVV_E_INVALID, "max_samples must be in [2, 2^24]");
  if (n > 0 && (!g->data || !r->data)) return fail(KVV_E_INVALID, "null data pointer");

  std::memset(&d, 0, sizeof(d));
  d.g = g->data;
  d.r = r->data;
  d.n = n;
  d.max_samples = p->max_samples;
  d.m = n < p->max_samples ? n : p->max_samples;
  d.mode = p->mode;
  // the reference takes near-zero diagnostics for fp16/bf16 references only (GCR:491-492)
  d.flags = (r->dtype == KVV_F16 || r->dtype == KVV_BF16) ? (p->flags & KVV_FLAG_NEAR_ZERO) : 0u;
  d.rtol = (float)p->rtol;
  d.atol = (float)p->atol;
  d.zero_tol = (p->rtol == 0.0 && p->atol == 0.0) ? 1 : 0;
  d.max_abs_diff = (int32_t)p->max_abs_diff;
  d.nz_abs = (float)p->near_zero_abs;
  d.nz_bad = (float)p->near_zero_bad_abs;
  // A bit-identical finite pair is a non-mismatch with abs_diff 0 -- unless the integer
  // threshold is negative (0 > t) or a negative near-zero "bad" threshold counts 0 as bad.
  d.fast = !(p->mode == KVV_MODE_MAX_ABS_DIFF && p->max_abs_diff < 0) &&
           !((d.flags & KVV_FLAG_NEAR_ZERO) && d.nz_bad < 0.0f);
  d.nz_code = near_code(r->dtype, d.nz_abs);
  d.dtype = r->dtype;
  d.item_elems = item_elems_for(r->dtype);
  d.row_items = 0;

  // joint coalescing: drop size-1 dims, merge i into i+1 when both strides chain
  int64_t sz[KVV_MAX_DIMS], gs[KVV_MAX_DIMS], rs[KVV_MAX_DIMS];
  int nd = 0;
  for (int i = 0; i < r->ndim; ++i) {
    if (r->sizes[i] == 1) continue;
    if (nd > 0 && gs[nd - 1] == g->strides[i] * r->sizes[i] && rs[nd - 1] == r->strides[i] * r->sizes[i]) {
      sz[nd - 1] *= r->sizes[i];
      gs[nd - 1] = g->strides[i];
      rs[nd - 1] = r->strides[i];
    } else {
      sz[nd] = r->sizes[i];
      gs[nd] = g->strides[i];
      rs[nd] = r->strides[i];
      ++nd;
    }
  }
  const int V = 16 / es;
  const bool aligned =
      (reinterpret_cast<uintptr_t>(g->data) % 16 == 0) && (reinterpret_cast<uintptr_t>(r->data) % 16 == 0);
  if (n == 0 || nd == 0 || (nd == 1 && gs[0] == 1 && rs[0] == 1)) {
    d.layout = L_CONTIG;
    d.vec = aligned;
  } else if (gs[nd - 1] == 1 && rs[nd - 1] == 1) {
    d.layout = L_ROWS;
    d.row_len = sz[nd - 1];
    d.dims.ndim = nd - 1;
    bool ok = aligned && (d.row_len % V == 0);
    for (int i = 0; i < nd - 1; ++i) {
      d.dims.sizes[i] = sz[i];
      d.dims.gstr[i] = gs[i];
      d.dims.rstr[i] = rs[i];
      ok = ok && ((gs[i] * es) % 16 == 0) && ((rs[i] * es) % 16 == 0);
    }
    d.vec = ok;
    // one outer dim and rows of whole items: each item lies in one row
    if (ok && nd == 2 && d.row_len % d.item_elems == 0 && d.row_len / d.item_elems < (1ll << 31))
      d.row_items = (int32_t)(d.row_len / d.item_elems);
  } else {
    d.layout = L_GENERIC;
    d.dims.ndim = nd;
    for (int i = 0; i < nd; ++i) {
      d.dims.sizes[i] = sz[i];
      d.dims.gstr[i] = gs[i];
      d.dims.rstr[i] = rs[i];
    }
    d.vec = 0;
  }
  d.item_count = (n + d.item_elems - 1) / d.item_elems;
  d.sel_rounds = 1;
  d.chunk_count = select_chunks(d.m, 1);
  d.lslot = -1;
  d.isel_slot = -1;
  d.s_div = 1;  // n <= max_samples: every element is a sample (stride 1)
  d.s_mod = 0;
  d.s_magic = 0;
  d.s_shift = 0;
  if (n > p->max_samples) {
    const uint64_t num = (uint64_t)n - 1, den = (uint64_t)d.m - 1;
    d.s_div = num / den;
    d.s_mod = num % den;
    // floor(t / den) = mulhi(t, s_magic) >> s_shift for every t < 64 * den (the
    // cursor's dividends): with l = ceil(log2 den) and N = max(6 + l, 32 - l),
    // magic = ceil(2^(N+l) / den) < 2^32 and the rounding error stays below 1/den.
    d.s_magic = 0;
    d.s_shift = 0;
    if (den > 1) {
      int l = 0;
      while ((1ull << l) < den) ++l;
      const int N = 6 + l > 32 - l ? 6 + l : 32 - l;
      const int k = N + l;
      d.s_magic = (uint32_t)(((1ull << k) + den - 1) / den);
      d.s_shift = (uint32_t)(k - 32);
    }
  }
  return KVV_OK;
}

// ------------------------------------------------------------ workspace
struct WsLayout {
  int64_t run_stride;
  size_t runs_u32, runs_u64, sample_abs, sample_rel, slots, slot_bytes, item_near, item_near_off, item_near_sum, near_sample,
      near_cm, ent, near_wave, ent_fill, wave_range, near_psum, table, chunk_seg, isel_state, isel_seg,
      isel_sums, fb_segs, fb_counts, cap_runs, cap_chunks, subtab,
      submm, starts, upload_end, total;
};

// Work-list counts: the input-select passes' chunk lists (one per scan group),
// their segment list, then the capture pass's chunk lists (one per scan group).
constexpr int kMaxGroups = 15 * 2 * 3;
// wave ranges kept per batch group (a grid of at most 4096 blocks, and one end)
constexpr int64_t kGroupStarts = 4096 * kWaves + 1;

// Near-zero entries of a single fp16/bf16 pair (kFlagNearEntries), 8 bytes each,
// split evenly over the main pass's waves.  A wave's share is an eighth of its
// element range when the workspace holds that (the size kvv_workspace_size
// asks for), else kEntPool entries in all (the least workspace such a verdict
// runs with); never more than the wave's elements.  A wave whose entries do
// not fit is read again by the first tail launch.  Up to kScatterMax blocks of
// that launch place the entries, each for an equal run of consecutive waves.
constexpr int64_t kEntPool = int64_t(1) << 21;
constexpr int64_t kEntFrac = 8;
constexpr int kScatterMax = 2048;

// How a single pair's near-zero diagnostics are taken: none, entries recorded
// in the main pass, or the near-zero pass over the inputs after it.
struct NearMode {
  bool any() const { return exact || entries; }
  bool exact = false, entries = false;
  int64_t waves = 0, ent_total = 0;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Run slots a segment may need: one per wave range it meets, at most one per
// item and at most one per wave of a launch (the grid is capped at 4096 blocks).
int64_t run_slot_bound(int64_t item_count) {
  const int64_t units = 4096 * kWaves;
  const int64_t b = item_count < units ? item_count : units;
  return (b + 3) & ~int64_t(3);
}

WsLayout workspace_layout(int64_t run_slots, int64_t samples, int64_t nseg, int64_t nslots, int64_t chunks,
                          int64_t items, const NearMode& near, bool batch, int64_t nisel = 0, int64_t isel_chunks = 0,
                          int rounds = 1, int64_t ngroups = 0) {
  WsLayout L{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off += align256(bytes);
    return at;
  };
  L.run_stride = run_slots;
  L.runs_u32 = take((size_t)run_slots * kColU32 * 4);
  L.runs_u64 = take((size_t)run_slots * kColU64 * 8);
  L.sample_abs = take((size_t)samples * 4);
  L.sample_rel = take((size_t)samples * 4);
  // the select slots and the input-select states: one region, cleared by the first main-pass launch
  const size_t slot_part = (size_t)nslots * kArrays * kSlotWords * 4;
  L.slot_bytes = slot_part + (size_t)nisel * kIselStateWords * 4;
  L.slots = take(L.slot_bytes);
  L.isel_state = L.slots + slot_part;
  if (near.exact) {
    L.item_near = take((size_t)items * 4);
    L.item_near_off = take((size_t)items * 8);
    L.item_near_sum = take((size_t)items * 8);
  }
  if (near.any()) {
    L.near_sample = take((size_t)samples * 4);
    L.near_cm = take((size_t)nseg * 16);
  }
  if (near.entries) {
    L.ent = take((size_t)near.ent_total * 8);
    L.near_wave = take((size_t)near.waves * 4);
    L.ent_fill = take((size_t)near.waves * 4);
    L.wave_range = take((size_t)near.waves * 8);
    L.near_psum = take((size_t)kScatterMax * 8);
  }
  if (nslots > 0) {
    // level-1 candidate tables: kSubTab u16 per select round, per array
    L.subtab = take((size_t)kArrays * chunks * rounds * kSubTab * 2);
    L.submm = take((size_t)kArrays * chunks * rounds * kSubMM * 4);
  }
  if (batch) {
    // what the host writes, in one block [table, upload_end): one copy per call
    L.table = take((size_t)nseg * sizeof(SegDesc));
    L.starts = take((size_t)ngroups * kGroupStarts * 8);  // the main-pass launches' wave ranges
    L.chunk_seg = take((size_t)chunks * 8);
    L.isel_seg = take((size_t)nisel * 4);
    L.cap_chunks = take((size_t)isel_chunks * 8);  // the capture pass's chunk work lists
    L.fb_segs = take((size_t)nisel * 4);           // the fallback's segment work list
    L.fb_counts = take((size_t)(2 * kMaxGroups + 1) * 4);
    L.upload_end = off;
    L.isel_sums = take((size_t)isel_chunks * 3 * 8);
    L.cap_runs = take((size_t)run_slots * 16);
  }
  L.total = off + 256;
  return L;
}

template <typename T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

RunCols run_cols(const WsLayout& L, void* ws) {
  return RunCols{at<uint32_t>(ws, L.runs_u32), at<uint64_t>(ws, L.runs_u64), L.run_stride};
}

int check_ws(const WsLayout& L, void* ws, size_t ws_bytes, kvv_result* out) {
  if (!ws) return fail(KVV_E_WORKSPACE, "workspace is null");
  if (ws_bytes < L.total) return fail(KVV_E_WORKSPACE, "workspace too small: need " + std::to_string(L.total));
  if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(KVV_E_WORKSPACE, "workspace must be 256-byte aligned");
  if (!out) return fail(KVV_E_INVALID, "null result pointer");
  return KVV_OK;
}

// One near_kernel launch per scan group (the kernel is templated on dtype/mode).
struct NearLaunch {
  NearFn fn;
  int seg_lo;
  int nseg;
  int64_t item_lo, items;
};

// The launches after the main pass, shared by the single and batch paths:
// run-record fold + first select level (+ small groups) of the abs/rel samples
// in one launch; with near-zero diagnostics the near-zero sample and its first
// level; then select level 1 and the final read-off of every array.
int launch_tail(const SegDesc* seg0, const SegDesc* dtable, const int64_t* dchunk, int nseg, int64_t total_chunks,
                int64_t nslots, const NearMode& nm, const WsLayout& L, void* ws, kvv_result* out, hipStream_t st,
                const std::vector<NearLaunch>& nears, bool stream_groups = false, int rounds = 1,
                int64_t max_runs = -1, bool stream_ar = true) {
  const bool near = nm.any();
  TailArgs t{};
  if (seg0) t.seg0 = *seg0;
  t.table = dtable;
  t.chunk_seg = dchunk;
  t.nseg = nseg;
  t.total_chunks = total_chunks > 0 ? total_chunks : 1;
  t.res = out;
  t.runs = run_cols(L, ws);
  t.reduce_roles = nm.exact ? 6 : 5;
  // a batch whose segments have at most 64 runs each: a wave folds each segment
  const bool wave_fold = dtable != nullptr && !nm.any() && max_runs >= 0 && max_runs <= 64;
  if (wave_fold) t.reduce_roles = 0;
  t.arr[0] = at<float>(ws, L.sample_abs);
  t.arr[1] = at<float>(ws, L.sample_rel);
  t.arr[2] = near ? at<float>(ws, L.near_sample) : nullptr;
  t.slots = at<uint32_t>(ws, L.slots);
  if (nslots > 0) {
    t.subtab = at<uint16_t>(ws, L.subtab);
    t.submm = at<uint32_t>(ws, L.submm);
    t.total_sub = (total_chunks > 0 ? total_chunks : 1) * rounds;
  }
  t.item_near = nm.exact ? at<uint32_t>(ws, L.item_near) : nullptr;
  t.item_near_off = nm.exact ? at<uint64_t>(ws, L.item_near_off) : nullptr;
  t.item_near_sum = nm.exact ? at<double>(ws, L.item_near_sum) : nullptr;
  int scatter = 0;
  if (nm.entries) {
    t.ent = at<uint2>(ws, L.ent);
    t.near_wave = at<uint32_t>(ws, L.near_wave);
    t.ent_fill = at<uint32_t>(ws, L.ent_fill);
    t.wave_range = at<uint2>(ws, L.wave_range);
    t.nwaves = (int32_t)nm.waves;
    t.ent_quota = (uint32_t)(nm.ent_total / nm.waves);
    scatter = nm.waves < kScatterMax ? (int)nm.waves : kScatterMax;
    t.scatter_blocks = scatter;
    t.near_psum = at<double>(ws, L.near_psum);
  }
  t.isel_sums = at<double>(ws, L.isel_sums);
  t.near_cm = near ? at<uint64_t>(ws, L.near_cm) : nullptr;
  const bool batch = dtable != nullptr;
  auto launch = [&](int reduce_blocks, int level, int arr_lo, int narr) -> int {
    TailArgs x = t;
    x.reduce_blocks = reduce_blocks;
    x.level = level;
    x.arr_lo = arr_lo;
    x.narr = narr;
    int64_t chunks = total_chunks;
    if (!batch && level == 2 && chunks > 0) {
      // a single pair's final read-off runs on each array's first chunk only: one
      // block per array instead of a grid of blocks that return at once
      chunks = 1;
      x.total_chunks = 1;
    }
    const int64_t grid = reduce_blocks + (chunks > 0 ? (int64_t)narr * chunks : 0);
    if (grid == 0) return KVV_OK;
    void (*fn)(TailArgs) = nullptr;
    switch (level) {
      case 0: fn = batch ? tail_kernel<0, true> : tail_kernel<0, false>; break;
      case 1: fn = batch ? tail_kernel<1, true> : tail_kernel<1, false>; break;
      case 2: fn = batch ? tail_kernel<2, true> : tail_kernel<2, false>; break;
      case 3: fn = tail_kernel<3, false>; break;  // single pairs only
      default: fn = tail_kernel<4, true>; break;  // many-group launches are batches
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(kBlock), 0, st, x);
    KVV_HIP(hipGetLastError());
    return KVV_OK;
  };
  // near-zero entries: their own launch builds the near-zero sample and its level-0
  // histogram, so the first tail launch selects it like abs and rel
  if (scatter > 0) {
    hipLaunchKernelGGL(near_scatter_kernel, dim3((unsigned)scatter), dim3(kBlock), 0, st, t);
    KVV_HIP(hipGetLastError());
  }
  // a single pair whose main pass did select level 0 of abs/rel starts at level 1 there
  const bool main_hist = seg0 && (seg0->flags & kFlagMainHist);
  int rc = launch(wave_fold ? (nseg + kWaves - 1) / kWaves : nseg * t.reduce_roles, main_hist ? 3 : 0, 0,
                  nm.entries ? 3 : 2);
  if (rc) return rc;
  if (stream_groups && stream_ar) {
    rc = launch(0, 4, 0, 2);
    if (rc) return rc;
  }
  if (nm.exact) {
    for (const auto& nl : nears) {
      if (nl.items == 0) continue;
      NearArgs na{};
      if (seg0) na.seg0 = *seg0;
      na.table = dtable ? dtable + nl.seg_lo : nullptr;
      na.nseg = nl.nseg;
      na.seg_lo = nl.seg_lo;
      na.near_cm = at<uint64_t>(ws, L.near_cm);
      na.item_lo = nl.item_lo;
      na.items = nl.items;
      na.res = out;
      na.item_near_off = at<uint64_t>(ws, L.item_near_off);
      na.item_near = at<uint32_t>(ws, L.item_near);
      na.near_sample = at<float>(ws, L.near_sample);
      na.item_near_sum = at<double>(ws, L.item_near_sum);
      hipLaunchKernelGGL(nl.fn, dim3((unsigned)nl.items), dim3(kBlock), 0, st, na);
      KVV_HIP(hipGetLastError());
    }
    rc = launch(0, 0, 2, 1);
    if (rc) return rc;
    if (stream_groups) {
      rc = launch(0, 4, 2, 1);
      if (rc) return rc;
    }
  }
  if (nslots > 0) {
    const int narr = near ? 3 : 2;
    if (!main_hist) rc = launch(0, 1, 0, narr);
    else if (nm.exact) rc = launch(0, 1, 2, 1);  // abs/rel (and an entries-built near-zero sample) took level 1 first
    if (rc) return rc;
    rc = launch(0, 2, 0, narr);
    if (rc) return rc;
  }
  return KVV_OK;
}

// ------------------------------------------------------------ one verdict
// A single pair too small to give every wave of the grid two full items takes
// smaller items (down to one 16-byte vector per lane): more waves then share
// its work, which for all-slow data is latency, not bandwidth.  The kernels
// treat the vectors past an item's end as absent.
int plan_single(const kvv_tensor* g, const kvv_tensor* r, const kvv_policy* p, SegDesc& d) {
  int rc = plan_segment(g, r, p, d);
  if (rc) return rc;
  // a vector-kind fp16/bf16 pair takes its near-zero diagnostics as entries in
  // the main pass, unless the caller asks for the pass over the inputs
  if ((d.flags & KVV_FLAG_NEAR_ZERO) && !(p->flags & KVV_FLAG_NEAR_EXACT) && d.mode == KVV_MODE_ISCLOSE &&
      scan_kind(d) != K_SCALAR)
    d.flags = (d.flags & ~KVV_FLAG_NEAR_ZERO) | kFlagNearEntries;
  if (scan_kind(d) == K_CONTIG) {
    const int64_t min_elems = d.item_elems / kUnroll;
    const int64_t want = 2 * 12 * (int64_t)device_cus();  // two items per wave of a full grid
    while (d.item_elems > min_elems && d.item_count < want) {
      d.item_elems /= 2;
      d.item_count = (d.n + d.item_elems - 1) / d.item_elems;
    }
  }
  return KVV_OK;
}

// Relative item rates of the three dispatch rounds of a scan grid that holds
// three blocks per CU (oldest round first).  The grid is dispatched one block
// per CU at a time and the waves of earlier rounds are served faster: with
// equal shares on MI355X the bf16 main pass's first-round blocks finished in
// 143 us, the second round's in 164 us and the third round's in 191 us (the
// kernel ends with the slowest).  Shares in proportion to the rates, refined
// once from the per-round end times they gave, let the rounds finish together.
constexpr double kRoundRate3[3] = {1.18, 1.0, 0.79};
// The same for batch launches, whose items are mostly bound by instruction
// issue (e.g. fp32 pairs that differ everywhere): the scan's oldest waves are
// issued first.  Measured with equal shares on the C4 batch (per-wave clocks):
// the rounds' waves ended at 575 / 641 / 764 us (fp32) and 179 / 196 / 219 us
// (bf16) on average; refined from the ends the cost-weighted shares then gave
// (fp32 676 / 690 / 701 us at 1.14 / 1.0 / 0.80, bf16 205 / 209 / 213 us at
// 1.10 / 1.0 / 0.86).
constexpr double kBatchRoundRate3[3] = {1.12, 1.0, 0.84};
constexpr double kBatchRoundRateF32[3] = {1.16, 1.0, 0.78};

// Relative cost of a batch item by what its segment asks of the main pass, in
// items of a capture segment (least squares over per-wave clocks of the C4
// batch: per item and per segment, fp32 / bf16): a strided-sample segment's
// items (no capture: 0.74 / 0.68), a small segment's (its samples written:
// 1.05 / 1.55), and each segment's start and end (its first load and run
// record, the partial last vector: 2.3 / 2.6).
struct ItemCost {
  double strided, small, segment;
};
constexpr ItemCost kItemCostF32{0.74, 1.05, 2.3};
constexpr ItemCost kItemCost16{0.68, 1.55, 2.6};

// Splits a grid's a.items items over its dispatch rounds at the given rates
// (a.rounds = 1: one share for every wave).
void plan_rounds(ScanArgs& a, ScanFn scan, int64_t grid, const double* rate = kRoundRate3) {
  a.rounds = 1;
  const int64_t cus = device_cus();
  if (cus <= 0 || blocks_target(scan) != 3 * cus || grid <= 2 * cus) return;
  const int64_t nb[3] = {cus, cus, grid - 2 * cus};
  double wsum = 0.0;
  for (int r = 0; r < 3; ++r) wsum += rate[r] * (double)nb[r];
  int64_t first = 0;
  for (int r = 0; r < 3; ++r) {
    const int64_t n = r < 2 ? (int64_t)((double)a.items * rate[r] * (double)nb[r] / wsum) : a.items - first;
    const int64_t waves = nb[r] * kWaves;
    a.round_first[r] = first;
    a.round_ipw[r] = n > 0 ? (n + waves - 1) / waves : 0;
    first += n;
  }
  a.round_first[3] = a.items;
  a.rounds = 3;
  a.round_blocks = (int32_t)cus;
}

// The wave ranges of a batch group's main-pass launch (grid blocks over items
// [item_lo, item_lo + items) of segments [seg_lo, seg_hi)): each wave's share
// of the group's cost (ItemCost) in proportion to its dispatch round's rate;
// every range holds at least one item while items remain (the ranges after
// the last item are empty).  Fills st[0 .. grid * kWaves] (relative to
// item_lo) and each segment's run count and first range starting inside it.
void plan_wave_ranges(std::vector<SegDesc>& table, int seg_lo, int seg_hi, int64_t item_lo, int64_t items,
                      int64_t grid, ScanFn scan, const ItemCost& ic, const double* rates, int64_t* st) {
  const int64_t nw = grid * kWaves;
  auto cost_of = [&](const SegDesc& d) {
    if (d.m <= kSmall) return ic.small;
    if ((d.flags & kFlagInputSelect) && !(d.flags & kFlagCaptureElems)) return ic.strided;
    return 1.0;
  };
  double total = 0.0;
  for (int s = seg_lo; s < seg_hi; ++s)
    if (table[s].item_count > 0) total += ic.segment + cost_of(table[s]) * (double)table[s].item_count;
  // wave weights: dispatch rounds of one block per CU (equal weights when the
  // grid does not fill three rounds)
  const int64_t cus = device_cus();
  const bool rounds = cus > 0 && blocks_target(scan) == 3 * cus && grid > 2 * cus;
  auto weight = [&](int64_t k) {
    if (!rounds) return 1.0;
    const int64_t r = k / (cus * kWaves);
    return rates[r < 2 ? r : 2];
  };
  double wsum = 0.0;
  for (int64_t k = 0; k < nw; ++k) wsum += weight(k);
  st[0] = 0;
  int s = seg_lo;
  int64_t seg_first = 0;  // the first item of segment s (relative)
  double before = 0.0;    // the cost of the segments before s
  double wcum = 0.0;
  for (int64_t k = 1; k < nw; ++k) {
    wcum += weight(k - 1);
    const double t = total * wcum / wsum;
    while (s < seg_hi) {
      const SegDesc& d = table[s];
      const double whole = d.item_count > 0 ? ic.segment + cost_of(d) * (double)d.item_count : 0.0;
      if (before + whole > t) break;
      before += whole;
      seg_first += d.item_count;
      ++s;
    }
    int64_t i = items;
    if (s < seg_hi) {
      const SegDesc& d = table[s];
      const double rem = t - before - ic.segment;
      int64_t j = rem <= 0.0 ? 0 : (int64_t)std::ceil(rem / cost_of(d));
      if (j > d.item_count) j = d.item_count;
      i = seg_first + j;
    }
    if (i <= st[k - 1]) i = st[k - 1] + 1;
    if (i > items) i = items;
    st[k] = i;
  }
  st[nw] = items;
  // runs: the segment's first item and each range start strictly inside it
  for (int q = seg_lo; q < seg_hi; ++q) {
    SegDesc& d = table[q];
    const int64_t b = d.item_begin - item_lo, e = b + d.item_count;
    const int64_t k0 = std::upper_bound(st, st + nw + 1, b) - st;
    const int64_t k1 = std::lower_bound(st, st + nw + 1, e) - st;
    d.run_k0 = k0;
    d.run_n = d.item_count > 0 ? 1 + (k1 > k0 ? k1 - k0 : 0) : 0;
  }
}

// The main-pass launch of a single pair: kernel, items per wave, grid, the
// dispatch-round shares, and the near-zero mode with its entry quota.
struct SingleGeom {
  ScanFn scan = nullptr;
  int64_t ipw = 1, grid = 0;
  ScanArgs rounds{};  // the round fields
  NearMode near;
  uint32_t ent_quota = 0;
};

// full: the entry share of the size kvv_workspace_size asks for; else the least.
int single_geom(const SegDesc& d, SingleGeom& g, bool full = true) {
  const bool nz = (d.flags & kFlagNearEntries) != 0;
  g.scan = scan_fn(d.dtype, d.mode, scan_kind(d), false, nz);
  if (!g.scan) return fail(KVV_E_INVALID, "no kernel for dtype");
  const int64_t target = blocks_target(g.scan) * kWaves;  // waves of the grid
  g.ipw = d.item_count > 0 ? (d.item_count + target - 1) / target : 1;  // items per wave
  const int64_t per_block = g.ipw * kWaves;
  g.grid = d.item_count > 0 ? (d.item_count + per_block - 1) / per_block : 0;
  g.rounds.items = d.item_count;
  plan_rounds(g.rounds, g.scan, g.grid);
  int64_t max_ipw = g.ipw;
  if (g.rounds.rounds > 1)
    for (int r = 0; r < g.rounds.rounds; ++r) max_ipw = g.rounds.round_ipw[r] > max_ipw ? g.rounds.round_ipw[r] : max_ipw;
  if ((uint64_t)max_ipw * kWaves * (uint64_t)d.item_elems >= (1ull << 32))
    return fail(KVV_E_UNSUPPORTED, "tensor too large for 32-bit per-block counts");
  g.near.exact = (d.flags & KVV_FLAG_NEAR_ZERO) != 0;
  g.near.entries = nz;
  if (nz) {
    // an even share of the pool, but never more than a wave's elements
    g.near.waves = g.grid * kWaves > 0 ? g.grid * kWaves : kWaves;
    const int64_t range = max_ipw * (int64_t)d.item_elems;
    int64_t share = kEntPool / g.near.waves;
    if (full && range / kEntFrac > share) share = range / kEntFrac;
    g.ent_quota = (uint32_t)(share < range ? share : range);
    g.near.ent_total = (int64_t)g.ent_quota * g.near.waves;
  }
  return KVV_OK;
}

WsLayout single_layout(const SegDesc& d, const SingleGeom& g) {
  return workspace_layout(run_slot_bound(d.item_count), d.m, 1, d.m > kSmall ? 1 : 0, d.chunk_count, d.item_count,
                          g.near, false);
}

// ------------------------------------------------------------ kept workspaces
// Byte ranges of caller workspaces whose select slots a single-pair verdict left
// clear (its final read-off zeroes them), per device.  KVV_FLAG_WS_KEPT lets the
// next verdict on the same workspace skip its clearing launch when its slots lie
// inside that range.  Any call on a workspace first drops its record: whatever
// the call writes voids it.
struct KeptRange {
  int dev;
  const void* ws;
  size_t off, len;
};
std::mutex g_kept_mu;
std::vector<KeptRange> g_kept;
constexpr size_t kKeptMax = 64;

// Drops the record of ws on the current device; returns whether [off, off + len)
// lay inside it (only asked when the caller set KVV_FLAG_WS_KEPT).
bool take_kept(const void* ws, size_t off, size_t len) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(g_kept_mu);
  for (size_t i = 0; i < g_kept.size(); ++i) {
    const KeptRange k = g_kept[i];
    if (k.dev == dev && k.ws == ws) {
      g_kept.erase(g_kept.begin() + (std::ptrdiff_t)i);
      return len > 0 && off >= k.off && off + len <= k.off + k.len;
    }
  }
  return false;
}

void put_kept(const void* ws, size_t off, size_t len) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  std::lock_guard<std::mutex> lock(g_kept_mu);
  for (size_t i = 0; i < g_kept.size(); ++i)
    if (g_kept[i].dev == dev && g_kept[i].ws == ws) {
      g_kept.erase(g_kept.begin() + (std::ptrdiff_t)i);
      break;
    }
  if (g_kept.size() >= kKeptMax) g_kept.erase(g_kept.begin());
  g_kept.push_back(KeptRange{dev, ws, off, len});
}

// Whether the launches on `st` are being recorded into a graph instead of run.
// Host-side decisions taken now (skipping the clearing launch) would then be
// frozen into a graph that replays later, on a workspace other calls may have
// written in between.  The legacy default stream cannot be captured; a failed
// query counts as capturing (the safe side: the clearing launch is kept).
bool stream_capturing(hipStream_t st) {
  if (st == nullptr) return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

int run_single(const SegDesc& d0, kvv_result* out, void* ws, size_t ws_bytes, hipStream_t st, bool kept,
               hipEvent_t ev_begin = nullptr, hipEvent_t ev_end = nullptr) {
  // under capture the slots are always cleared, and the record of this
  // workspace is dropped (take_kept below) and not renewed: a replay runs later
  const bool capturing = stream_capturing(st);
  if (capturing) kept = false;
  SegDesc d = d0;
  d.item_begin = 0;
  d.sample_off = 0;
  d.chunk_begin = 0;
  d.out_index = 0;
  d.lslot = d.m > kSmall ? 0 : -1;
  const int64_t nslots = d.lslot >= 0 ? 1 : 0;
  d.run_slot0 = 0;
  SingleGeom g;
  int rc = single_geom(d, g);
  if (rc) return rc;
  WsLayout L = single_layout(d, g);
  if (g.near.entries && ws_bytes < L.total) {
    // a smaller workspace: the least entry pool (waves whose entries overflow it are read again)
    rc = single_geom(d, g, false);
    if (rc) return rc;
    L = single_layout(d, g);
  }
  rc = check_ws(L, ws, ws_bytes, out);
  if (rc) return rc;
  // A large group of a vector layout: the main pass's blocks histogram select
  // level 0 of abs/rel (two 16-bit LDS counts per word: a block's samples must
  // stay below 2^16), so the tail starts at level 1 for them.
  if (nslots > 0 && scan_kind(d) != K_SCALAR) {
    int64_t max_ipw = g.ipw;
    if (g.rounds.rounds > 1)
      for (int r = 0; r < g.rounds.rounds; ++r) max_ipw = g.rounds.round_ipw[r] > max_ipw ? g.rounds.round_ipw[r] : max_ipw;
    const int64_t elems = max_ipw * kWaves * (int64_t)d.item_elems;
    const int64_t per_block = d.m == d.n ? elems : elems * d.m / d.n + 2;
    if (per_block < 65536) d.flags |= kFlagMainHist;
  }
  const bool main_hist = (d.flags & kFlagMainHist) != 0;
  // slots left clear by the previous call on this workspace need no clearing launch
  const bool slots_clear = take_kept(ws, L.slots, L.slot_bytes) && kept && main_hist;
  // one run record per block: its waves fold theirs (a single-segment launch)
  d.run_n = g.grid;
  d.run_k0 = 0;
  if (d.item_count > 0) {
    ScanArgs a = g.rounds;
    a.seg0 = d;
    a.table = nullptr;
    a.nseg = 1;
    a.item_lo = 0;
    a.items = d.item_count;
    a.items_per_wave = g.ipw;
    a.runs = run_cols(L, ws);
    a.sample_abs = at<float>(ws, L.sample_abs);
    a.sample_rel = at<float>(ws, L.sample_rel);
    a.item_near = g.near.exact ? at<uint32_t>(ws, L.item_near) : nullptr;
    a.zero_ptr = at<uint4>(ws, L.slots);
    a.zero_n4 = (int64_t)(L.slot_bytes / 16);
    a.slots = nullptr;
    if (main_hist) {
      // the main pass adds into the slots: they are cleared by a launch before it,
      // unless the previous call on this workspace left them clear
      if (!slots_clear) {
        const int64_t n4 = a.zero_n4;
        const int64_t blocks = (n4 + kBlock * 4 - 1) / (kBlock * 4);
        hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)(blocks > 0 ? blocks : 1)), dim3(kBlock), 0, st,
                           a.zero_ptr, n4);
        KVV_HIP(hipGetLastError());
      }
      a.zero_n4 = 0;
      a.slots = at<uint32_t>(ws, L.slots);
    }
    if (g.near.entries) {
      a.ent = at<uint2>(ws, L.ent);
      a.near_wave = at<uint32_t>(ws, L.near_wave);
      a.ent_fill = at<uint32_t>(ws, L.ent_fill);
      a.wave_range = at<uint2>(ws, L.wave_range);
      a.ent_quota = g.ent_quota;
      // the near-zero sample starts at zero: entries fill in its nonzero values
      a.zero2_ptr = at<uint4>(ws, L.near_sample);
      a.zero2_n4 = (int64_t)((align256((size_t)d.m * 4)) / 16);
    }
    if (ev_begin || ev_end) {
      // the events take the kernel's own start and end from its dispatch
      // (no marker packets between the launches of the verdict)
      void* args[] = {&a};
      KVV_HIP(hipExtLaunchKernel(reinterpret_cast<const void*>(g.scan), dim3((unsigned)g.grid), dim3(kBlock), args,
                                 0, st, ev_begin, ev_end, 0));
    } else {
      hipLaunchKernelGGL(g.scan, dim3((unsigned)g.grid), dim3(kBlock), 0, st, a);
      KVV_HIP(hipGetLastError());
    }
  }
  std::vector<NearLaunch> nears{{near_fn(d.dtype, d.mode), 0, 1, 0, d.item_count}};
  rc = launch_tail(&d, nullptr, nullptr, 1, d.chunk_count, nslots, g.near, L, ws, out, st, nears);
  // the final read-off zeroes every slot it read: the next call may skip the clearing
  if (rc == KVV_OK && main_hist && d.item_count > 0 && !capturing) put_kept(ws, L.slots, L.slot_bytes);
  return rc;
}

// full: the workspace with the full entry share (what kvv_workspace_size reports);
// else the least one a verdict runs with.
int single_workspace_bytes(const SegDesc& d, size_t* bytes, bool full = true) {
  SingleGeom g;
  const int rc = single_geom(d, g, full);
  if (rc) return rc;
  *bytes = single_layout(d, g).total;
  return KVV_OK;
}

// ------------------------------------------------------------ no-alloc entry
// kvv_verdict_noalloc's workspace: a fixed device array in the code object, so
// the call needs no allocation.  Each GPU holds its own copy from the library's
// first use until the process ends.  In host code `scratch` only names the
// symbol: its device address, per device, comes from hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxScratchDevices] = {};
// a no-alloc verdict was captured into a graph on this device: its replays
// write the scratch array at times the library does not see
bool g_scratch_graphed[kMaxScratchDevices] = {};

// The current device's scratch address, looked up once per device.  `kept`:
// whether only the library's own eager calls can have written the array since
// the previous one (no no-alloc verdict on this device was ever captured;
// `capturing` says this one is).
int scratch_address(void** p, bool capturing, bool* kept) {
  int dev = 0;
  KVV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(KVV_E_UNSUPPORTED, "device ordinal " + std::to_string(dev) + " beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* q = nullptr;
    KVV_HIP(hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)));
    if (!q) return fail(KVV_E_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch[dev] = q;
  }
  if (capturing) g_scratch_graphed[dev] = true;
  *p = g_scratch[dev];
  *kept = !g_scratch_graphed[dev];
  return KVV_OK;
}

// ------------------------------------------------------------ batch
struct BatchPlan {
  std::vector<SegDesc> table;   // sorted by (dtype, mode, kind) group, then input order
  std::vector<int64_t> chunk_seg;
  struct Group {
    int dt, mode, kind;
    int seg_lo, seg_hi;
    int64_t item_lo, items, ipb;
    int64_t grid;  // the main-pass launch: blocks, and its wave ranges at starts[g * kGroupStarts]
    int64_t ick_lo, ick_n;  // this group's input-select chunks in isel_chunk
    int64_t isel_lo, isel_n;  // this group's input-select segments in isel_seg
  };
  std::vector<int32_t> isel_seg;      // input-select segments
  std::vector<int32_t> isel_chunk;    // (segment, chunk of the segment) pairs, grouped like the scans
  std::vector<Group> groups;
  std::vector<int64_t> starts;  // kGroupStarts per group: wave k of its launch owns [starts[k], starts[k + 1])
  bool stream_groups = false;  // large groups selected one block each (tail level 4)
  int rounds = 1;              // select rounds per chunk block (every segment of the batch)
  int64_t items = 0, samples = 0, chunks = 0, nslots = 0, run_slots = 0;
  bool near = false;
  // run-time work lists of the fallback and capture passes (host copies, filled by run_batch)
  std::vector<int32_t> work_segs, cap_work;
  std::vector<uint32_t> work_counts;
  // the planner's own per-pair scratch
  std::vector<SegDesc> segs;
  std::vector<int> order, kinds;
  // Empties the plan for the next call; the vectors keep their memory, so a
  // thread's repeated batches of one size allocate (and first-touch) nothing.
  void reset() {
    table.clear();
    chunk_seg.clear();
    isel_seg.clear();
    isel_chunk.clear();
    groups.clear();
    starts.clear();
    stream_groups = false;
    rounds = 1;
    items = samples = chunks = nslots = run_slots = 0;
    near = false;
    work_segs.clear();
    cap_work.clear();
    work_counts.clear();
    segs.clear();
    order.clear();
    kinds.clear();
  }
};

// The calling thread's plan, reused call after call.
BatchPlan& thread_plan() {
  static thread_local BatchPlan bp;
  bp.reset();
  return bp;
}

int plan_batch(int32_t count, const kvv_tensor* gens, const kvv_tensor* refs, const kvv_policy* pols, BatchPlan& bp) {
  if (count < 0) return fail(KVV_E_INVALID, "negative count");
  if (count > 0 && (!gens || !refs || !pols)) return fail(KVV_E_INVALID, "null batch arrays");
  std::vector<SegDesc>& segs = bp.segs;
  std::vector<int>& order = bp.order;
  std::vector<int>& kinds = bp.kinds;
  segs.assign((size_t)count, SegDesc{});
  order.assign((size_t)count, 0);
  kinds.assign((size_t)count, 0);
  bp.table.reserve((size_t)count);
  for (int i = 0; i < count; ++i) {
    int rc = plan_segment(&gens[i], &refs[i], &pols[i], segs[i]);
    if (rc) return fail(rc, "pair " + std::to_string(i) + ": " + g_err);
    segs[i].out_index = i;
    kinds[i] = scan_kind(segs[i]);
    order[i] = i;
  }
  // many samples in one launch: fewer, fuller select blocks (each block's fixed
  // work -- its group's state, its histogram's clear and flush -- is paid once
  // per kMaxSelRounds rounds)
  int64_t chunks1 = 0, large = 0, max_m = 0;
  for (const SegDesc& d : segs) {
    chunks1 += d.chunk_count;
    if (d.m > kSmall) {
      ++large;
      max_m = d.m > max_m ? d.m : max_m;
    }
  }
  // enough large groups to fill the device by themselves: each is selected by
  // one block in the first tail launch (no global histograms, no level launches)
  const bool group_mode = large >= (int64_t)device_cus() && max_m <= kGroupStreamMax;
  bp.stream_groups = group_mode;
  const int rounds = chunks1 >= 4 * 8192 ? 4 : (chunks1 >= 2 * 8192 ? 2 : 1);
  static_assert(kMaxSelRounds >= 4, "select rounds");
  bp.rounds = group_mode ? 1 : rounds;
  for (int i = 0; i < count; ++i) {
    SegDesc& d = segs[i];
    d.sel_rounds = group_mode ? 1 : rounds;
    d.chunk_count = group_mode ? (d.m > 0 ? 1 : 0) : select_chunks(d.m, rounds);
    // a large contiguous group: the p99 of abs/rel is selected from the inputs:
    // the main pass captures its sampled values above pivot thresholds (and the
    // input-select passes select it if that misses)
    if (group_mode && d.m > kSmall && kinds[i] == K_CONTIG) {
      d.flags |= kFlagInputSelect | kFlagCapture;
      if (d.m == d.n) d.flags |= kFlagCaptureElems;
    }
  }
  auto key = [&](int i) { return (segs[i].dtype * 2 + segs[i].mode) * 3 + kinds[i]; };
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return key(a) < key(b); });
  bp.table.clear();
  int64_t item = 0, sample = 0, chunk = 0;
  for (int i : order) {
    SegDesc d = segs[i];
    d.item_begin = item;
    d.sample_off = sample;
    d.chunk_begin = chunk;
    d.lslot = !group_mode && d.m > kSmall ? (int32_t)bp.nslots++ : -1;
    d.run_slot0 = bp.run_slots;
    bp.run_slots += run_slot_bound(d.item_count);
    const int s = (int)bp.table.size();
    for (int64_t c = 0; c < d.chunk_count; ++c) bp.chunk_seg.push_back((int64_t)s);
    item += d.item_count;
    sample += (d.m + 63) & ~int64_t(63);  // each segment's samples start on a 256-byte line
    chunk += d.chunk_count;
    bp.near = bp.near || (d.flags & KVV_FLAG_NEAR_ZERO);
    if (bp.groups.empty() || bp.groups.back().dt != d.dtype || bp.groups.back().mode != d.mode ||
        bp.groups.back().kind != kinds[i]) {
      bp.groups.push_back({d.dtype, d.mode, kinds[i], s, s + 1, d.item_begin, d.item_count, 1, 0, 0, 0,
                           (int64_t)bp.isel_seg.size(), 0});
    } else {
      bp.groups.back().seg_hi = s + 1;
      bp.groups.back().items += d.item_count;
    }
    if (d.flags & kFlagInputSelect) {
      d.isel_slot = (int32_t)bp.isel_seg.size();
      d.isel_group = (int32_t)bp.groups.size() - 1;
      bp.isel_seg.push_back(s);
      ++bp.groups.back().isel_n;
    }
    bp.table.push_back(d);
  }
  bp.starts.assign(bp.groups.size() * (size_t)kGroupStarts, 0);
  for (size_t g = 0; g < bp.groups.size(); ++g) {
    auto& gr = bp.groups[g];
    const ScanFn scan = scan_fn(gr.dt, gr.mode, gr.kind, true);
    const int64_t target = blocks_target(scan) * kWaves;  // waves
    gr.ipb = gr.items > 0 ? (gr.items + target - 1) / target : 1;  // items per wave, equal shares
    gr.grid = gr.items > 0 ? (gr.items + gr.ipb * kWaves - 1) / (gr.ipb * kWaves) : 0;
    if (gr.grid * kWaves + 1 > kGroupStarts) return fail(KVV_E_UNSUPPORTED, "batch group grid too large");
    int64_t* st = bp.starts.data() + g * kGroupStarts;
    plan_wave_ranges(bp.table, gr.seg_lo, gr.seg_hi, gr.item_lo, gr.items, gr.grid, scan,
                     gr.dt == KVV_F32 ? kItemCostF32 : kItemCost16,
                     gr.dt == KVV_F32 && gr.mode == KVV_MODE_ISCLOSE ? kBatchRoundRateF32 : kBatchRoundRate3, st);
    int64_t max_ipw = 0;
    for (int64_t k = 0; k < gr.grid * kWaves; ++k) max_ipw = st[k + 1] - st[k] > max_ipw ? st[k + 1] - st[k] : max_ipw;
    if ((uint64_t)max_ipw * (uint64_t)item_elems_for(gr.dt) >= (1ull << 32))
      return fail(KVV_E_UNSUPPORTED, "batch group too large for 32-bit per-wave counts");
  }
  bp.items = item;
  bp.samples = sample;
  bp.chunks = chunk;
  // the input-select chunk launches follow the scan groups (one kernel per
  // dtype); strided-sample chunks (element loads, slower) are dispatched first
  if (bp.groups.size() > (size_t)kMaxGroups) return fail(KVV_E_INVALID, "too many scan groups");
  for (auto& gr : bp.groups) {
    gr.ick_lo = (int64_t)bp.isel_chunk.size() / 2;
    for (int pass = 0; pass < 2; ++pass) {
      for (int s = gr.seg_lo; s < gr.seg_hi; ++s) {
        const SegDesc& d = bp.table[s];
        if (!(d.flags & kFlagInputSelect) || (d.m == d.n) != (pass == 1)) continue;
        bp.table[s].isel_chunk0 = (int32_t)(bp.isel_chunk.size() / 2);
        for (int64_t c = 0; c * isel_chunk_len(d) < d.m; ++c) {
          bp.isel_chunk.push_back(s);
          bp.isel_chunk.push_back((int32_t)c);
        }
      }
    }
    gr.ick_n = (int64_t)bp.isel_chunk.size() / 2 - gr.ick_lo;
  }
  if (bp.stream_groups) {
    // one select block per group: the largest groups first, so the longest
    // blocks start early and the small ones fill in behind them
    std::vector<int> by_size;
    for (int s = 0; s < (int)bp.table.size(); ++s)
      if (bp.table[s].chunk_count > 0) by_size.push_back(s);
    std::stable_sort(by_size.begin(), by_size.end(), [&](int x, int y) { return bp.table[x].m > bp.table[y].m; });
    for (size_t k = 0; k < by_size.size(); ++k) {
      bp.table[by_size[k]].chunk_begin = (int64_t)k;
      bp.chunk_seg[k] = by_size[k];
    }
  }
  return KVV_OK;
}

// ------------------------------------------------------------ batch uploads
// What a batch call writes from the host (its table, wave ranges and work
// lists) lies in one block of the workspace.  It goes over in one copy from a
// pinned staging buffer per device, which the next call refills only after the
// copy that read it has finished (its event): one DMA per call instead of one
// per part from pageable memory (C4: five copies, 68 us of the call).  The
// buffer is kept until the process ends.  (A batch is never captured into a
// graph: kvv_verdict_batch refuses a capturing stream.)
struct UploadPart {
  size_t at;  // workspace offset
  const void* src;
  size_t bytes;
};
constexpr int kStageDevices = 64;
struct Staging {
  void* buf = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};
std::mutex g_stage_mu;
Staging g_stage[kStageDevices];

int upload_parts(const std::vector<UploadPart>& parts, size_t lo, size_t hi, void* ws, hipStream_t st) {
  int dev = -1;
  KVV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kStageDevices) {
    for (const auto& u : parts)
      if (u.bytes) KVV_HIP(hipMemcpyAsync((char*)ws + u.at, u.src, u.bytes, hipMemcpyHostToDevice, st));
    return KVV_OK;
  }
  std::lock_guard<std::mutex> lock(g_stage_mu);
  Staging& S = g_stage[dev];
  if (S.pending) {
    KVV_HIP(hipEventSynchronize(S.done));
    S.pending = false;
  }
  const size_t need = hi - lo;
  if (S.cap < need) {
    if (S.buf) KVV_HIP(hipHostFree(S.buf));
    S.buf = nullptr;
    S.cap = 0;
    const size_t c = need + need / 4 + 65536;
    KVV_HIP(hipHostMalloc(&S.buf, c, hipHostMallocDefault));
    S.cap = c;
  }
  if (!S.done) KVV_HIP(hipEventCreateWithFlags(&S.done, hipEventDisableTiming));
  for (const auto& u : parts)
    if (u.bytes) std::memcpy((char*)S.buf + (u.at - lo), u.src, u.bytes);
  KVV_HIP(hipMemcpyAsync((char*)ws + lo, S.buf, need, hipMemcpyHostToDevice, st));
  KVV_HIP(hipEventRecord(S.done, st));
  S.pending = true;
  return KVV_OK;
}

// ------------------------------------------------------------ side stream
// A batch whose input-select segments fall in two or more dtype groups runs
// the groups' pivot and capture launches on two streams: they touch disjoint
// segments, and each launch is latency-bound, so one group's blocks use the
// device time the other's leave idle.  One side stream per device (default
// priority), forked from the caller's stream and joined back into it with
// events before the main passes.
struct Side {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
Side g_side[kStageDevices];

int run_batch(BatchPlan& bp, kvv_result* out, void* ws, size_t ws_bytes, hipStream_t st) {
  const int nseg = (int)bp.table.size();
  if (nseg == 0) return KVV_OK;
  const int64_t nisel = (int64_t)bp.isel_seg.size(), isel_chunks = (int64_t)bp.isel_chunk.size() / 2;
  NearMode near;
  near.exact = bp.near;
  const WsLayout L = workspace_layout(bp.run_slots, bp.samples, nseg, bp.nslots, bp.chunks, bp.items, near, true,
                                      nisel, isel_chunks, bp.rounds, (int64_t)bp.groups.size());
  int rc = check_ws(L, ws, ws_bytes, out);
  if (rc) return rc;
  SegDesc* dtable = at<SegDesc>(ws, L.table);
  int64_t* dchunk = at<int64_t>(ws, L.chunk_seg);
  uint32_t* istate = at<uint32_t>(ws, L.isel_state);
  for (SegDesc& d : bp.table) {
    if (!(d.flags & kFlagCapture)) continue;
    // the capture buffers are the segment's sample region; the thresholds come from the pivot launch
    d.cap_buf[0] = at<float>(ws, L.sample_abs) + d.sample_off;
    d.cap_buf[1] = at<float>(ws, L.sample_rel) + d.sample_off;
    d.cap_state = istate + (size_t)d.isel_slot * kIselStateWords;
  }
  std::vector<UploadPart> parts;
  parts.push_back({L.table, bp.table.data(), nseg * sizeof(SegDesc)});
  int64_t* dstarts = at<int64_t>(ws, L.starts);
  parts.push_back({L.starts, bp.starts.data(), bp.starts.size() * 8});
  parts.push_back({L.chunk_seg, bp.chunk_seg.data(), (size_t)bp.chunks * 8});
  int32_t* disel = at<int32_t>(ws, L.isel_seg);
  int32_t* dfbseg = at<int32_t>(ws, L.fb_segs);
  uint32_t* dcounts = at<uint32_t>(ws, L.fb_counts);
  int2* dcapchunk = at<int2>(ws, L.cap_chunks);
  const int ngroups = (int)bp.groups.size();
  if (nisel) {
    // work lists: the fallback's starts with the segments that do not capture
    // (none at present), to which the capture final adds those that miss; the
    // capture pass's hold the chunks of the capture segments with strided
    // samples
    bp.cap_work.assign((size_t)isel_chunks * 2, 0);
    bp.work_segs.clear();
    bp.work_counts.assign((size_t)2 * ngroups + 1, 0u);
    for (int g = 0; g < ngroups; ++g) {
      const auto& gr = bp.groups[g];
      for (int64_t k = gr.ick_lo; k < gr.ick_lo + gr.ick_n; ++k) {
        const int32_t s = bp.isel_chunk[2 * k];
        const uint32_t f = bp.table[s].flags;
        if (!(f & kFlagCapture) || (f & kFlagCaptureElems)) continue;  // not captured, or by the main pass
        uint32_t& cnt = bp.work_counts[ngroups + 1 + g];
        const int64_t at_k = gr.ick_lo + cnt++;
        bp.cap_work[2 * at_k] = s;
        bp.cap_work[2 * at_k + 1] = bp.isel_chunk[2 * k + 1];
      }
    }
    for (int32_t s : bp.isel_seg)
      if (!(bp.table[s].flags & kFlagCapture)) bp.work_segs.push_back(s);
    bp.work_counts[ngroups] = (uint32_t)bp.work_segs.size();
    parts.push_back({L.isel_seg, bp.isel_seg.data(), (size_t)nisel * 4});
    parts.push_back({L.cap_chunks, bp.cap_work.data(), (size_t)isel_chunks * 8});
    parts.push_back({L.fb_segs, bp.work_segs.data(), bp.work_segs.size() * 4});
    parts.push_back({L.fb_counts, bp.work_counts.data(), (size_t)(2 * ngroups + 1) * 4});
  }
  rc = upload_parts(parts, L.table, L.upload_end, ws, st);
  if (rc) return rc;
  IselArgs ia{};
  ia.table = dtable;
  ia.segs = disel;
  ia.state = istate;
  ia.sums = at<double>(ws, L.isel_sums);
  ia.buf[0] = at<float>(ws, L.sample_abs);
  ia.buf[1] = at<float>(ws, L.sample_rel);
  ia.res = out;
  ia.cap_runs = at<uint4>(ws, L.cap_runs);
  ia.fb_segs = dfbseg;
  ia.fb_scount = dcounts + ngroups;
  // input-select segments: their state is cleared, and the capture thresholds
  // estimated, before the main pass (one block per segment, per dtype); every
  // other group's launches go to the side stream
  int isel_groups = 0;
  for (const auto& gr : bp.groups) isel_groups += gr.isel_n > 0 ? 1 : 0;
  std::unique_lock<std::mutex> side_lock;
  Side* side = nullptr;
  if (isel_groups >= 2) {
    int dev = -1;
    KVV_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < kStageDevices) {
      side_lock = std::unique_lock<std::mutex>(g_side_mu);
      side = &g_side[dev];
      if (!side->s) {
        KVV_HIP(hipStreamCreateWithFlags(&side->s, hipStreamNonBlocking));
        KVV_HIP(hipEventCreateWithFlags(&side->fork, hipEventDisableTiming));
        KVV_HIP(hipEventCreateWithFlags(&side->join, hipEventDisableTiming));
      }
      KVV_HIP(hipEventRecord(side->fork, st));
      KVV_HIP(hipStreamWaitEvent(side->s, side->fork, 0));
    }
  }
  int isel_k = 0;
  for (int g = 0; g < ngroups; ++g) {
    const auto& gr = bp.groups[g];
    if (gr.isel_n == 0) continue;
    const hipStream_t sg = side && (isel_k++ & 1) ? side->s : st;
    IselFn fn = isel_fn(gr.dt, 2);
    if (!fn) return fail(KVV_E_INVALID, "no input-select kernel for dtype");
    IselArgs x = ia;
    x.segs = disel + gr.isel_lo;
    hipLaunchKernelGGL(fn, dim3((unsigned)gr.isel_n), dim3(kBlock), 0, sg, x);
    KVV_HIP(hipGetLastError());
    // then the capture pass over the strided samples of the group's capture segments
    const int64_t ncap = bp.work_counts[ngroups + 1 + g];
    if (ncap > 0) {
      IselFn cf = isel_fn(gr.dt, 3);
      IselArgs c = ia;
      c.chunks = dcapchunk + gr.ick_lo;
      c.nchunks = dcounts + ngroups + 1 + g;
      hipLaunchKernelGGL(cf, dim3((unsigned)(ncap < kIselWorkBlocks ? ncap : kIselWorkBlocks)), dim3(kBlock), 0, sg, c);
      KVV_HIP(hipGetLastError());
    }
  }
  if (side) {
    KVV_HIP(hipEventRecord(side->join, side->s));
    KVV_HIP(hipStreamWaitEvent(st, side->join, 0));
    side_lock.unlock();
  }
  std::vector<NearLaunch> nears;
  bool zeroed = false;
  for (const auto& gr : bp.groups) {
    nears.push_back({near_fn(gr.dt, gr.mode), gr.seg_lo, gr.seg_hi - gr.seg_lo, gr.item_lo, gr.items});
    if (gr.items == 0) continue;
    ScanFn scan = scan_fn(gr.dt, gr.mode, gr.kind, true);
    if (!scan) return fail(KVV_E_INVALID, "no kernel for dtype");
    ScanArgs a{};
    a.starts = dstarts + (&gr - bp.groups.data()) * kGroupStarts;
    a.table = dtable + gr.seg_lo;
    a.nseg = gr.seg_hi - gr.seg_lo;
    a.item_lo = gr.item_lo;
    a.items = gr.items;
    a.items_per_wave = gr.ipb;
    a.runs = run_cols(L, ws);
    a.sample_abs = at<float>(ws, L.sample_abs);
    a.sample_rel = at<float>(ws, L.sample_rel);
    a.item_near = bp.near ? at<uint32_t>(ws, L.item_near) : nullptr;
    a.cap_runs = at<uint4>(ws, L.cap_runs);
    if (!zeroed) {
      // the first main-pass launch clears the select slots of the whole batch
      // (the input-select states after them were cleared by the pivot launch)
      a.zero_ptr = at<uint4>(ws, L.slots);
      a.zero_n4 = (int64_t)((L.isel_state - L.slots) / 16);
      zeroed = true;
    }
    // (the grid keeps the equal shares' size: three blocks per CU)
    hipLaunchKernelGGL(scan, dim3((unsigned)gr.grid), dim3(kBlock), 0, st, a);
    KVV_HIP(hipGetLastError());
  }
  int64_t max_runs = 0;
  // abs/rel groups that the one-block stream select takes (large, with sample
  // arrays, not selected from the inputs): none, and its launch is left out
  bool stream_ar = false;
  for (const auto& d : bp.table) {
    max_runs = d.run_n > max_runs ? d.run_n : max_runs;
    stream_ar = stream_ar || (d.chunk_count > 0 && d.m > kSmall && !(d.flags & kFlagInputSelect));
  }
  auto tail = [&](hipStream_t ts) {
    return launch_tail(nullptr, dtable, dchunk, nseg, bp.chunks, bp.nslots, near, L, ws, out, ts, nears,
                       bp.stream_groups, bp.rounds, max_runs, stream_ar);
  };
  if (!nisel) return tail(st);
  // The tail launches (the run fold, the small groups' selects) need nothing of
  // the capture final's or the fallback's when every input-select segment
  // captures (the fallback then writes no chunk sums): they go to the side
  // stream, beside those launches, and are joined back before the call ends.
  std::unique_lock<std::mutex> tail_lock;
  Side* tside = nullptr;
  if (bp.work_segs.empty()) {
    int dev = -1;
    KVV_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < kStageDevices) {
      tail_lock = std::unique_lock<std::mutex>(g_side_mu);
      tside = &g_side[dev];
      if (!tside->s) {
        KVV_HIP(hipStreamCreateWithFlags(&tside->s, hipStreamNonBlocking));
        KVV_HIP(hipEventCreateWithFlags(&tside->fork, hipEventDisableTiming));
        KVV_HIP(hipEventCreateWithFlags(&tside->join, hipEventDisableTiming));
      }
      KVV_HIP(hipEventRecord(tside->fork, st));
      KVV_HIP(hipStreamWaitEvent(tside->s, tside->fork, 0));
      rc = tail(tside->s);
      if (rc) return rc;
      KVV_HIP(hipEventRecord(tside->join, tside->s));
    }
  }
  // p99 of the input-select segments: the capture segments' selection among
  // their captured values; then the fallback, one launch per group, for the
  // other input-select segments and the capture segments that missed (its
  // blocks loop over the list, which is empty unless a capture missed)
  hipLaunchKernelGGL(isel_cap_final_kernel, dim3((unsigned)(2 * nisel)), dim3(kBlock), 0, st, ia);
  KVV_HIP(hipGetLastError());
  IselArgs wl = ia;
  wl.segs = dfbseg;
  wl.nsegs = dcounts + ngroups;
  const int64_t fgrid = nisel < kIselWorkBlocks ? nisel : kIselWorkBlocks;
  for (int g = 0; g < ngroups; ++g) {
    const auto& gr = bp.groups[g];
    if (gr.isel_n == 0) continue;
    IselFn fn = isel_fn(gr.dt, 0);
    if (!fn) return fail(KVV_E_INVALID, "no input-select kernel for dtype");
    IselArgs x = wl;
    x.group = g;
    hipLaunchKernelGGL(fn, dim3((unsigned)fgrid), dim3(kBlock), 0, st, x);
    KVV_HIP(hipGetLastError());
  }
  if (!tside) return tail(st);
  KVV_HIP(hipStreamWaitEvent(st, tside->join, 0));
  return KVV_OK;
}

}  // namespace
}  // namespace kvv

// ================================================================ C ABI
extern "C" {

int kvv_abi_version(void) { return KVV_ABI_VERSION; }

const char* kvv_last_error(void) { return kvv::g_err.c_str(); }

int kvv_workspace_size(const kvv_tensor* gen, const kvv_tensor* ref, const kvv_policy* policy, size_t* bytes) {
  if (!bytes) return kvv::fail(KVV_E_INVALID, "null bytes pointer");
  kvv::SegDesc d;
  int rc = kvv::plan_single(gen, ref, policy, d);
  if (rc) return rc;
  return kvv::single_workspace_bytes(d, bytes);
}

int kvv_verdict(const kvv_tensor* gen, const kvv_tensor* ref, const kvv_policy* policy, kvv_result* out,
                void* workspace, size_t workspace_bytes, void* stream) {
  kvv::SegDesc d;
  int rc = kvv::plan_single(gen, ref, policy, d);
  if (rc) return rc;
  return kvv::run_single(d, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                         (policy->flags & KVV_FLAG_WS_KEPT) != 0);
}

int kvv_verdict_timed(const kvv_tensor* gen, const kvv_tensor* ref, const kvv_policy* policy, kvv_result* out,
                      void* workspace, size_t workspace_bytes, void* stream, void* main_begin, void* main_end) {
  kvv::SegDesc d;
  int rc = kvv::plan_single(gen, ref, policy, d);
  if (rc) return rc;
  return kvv::run_single(d, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                         (policy->flags & KVV_FLAG_WS_KEPT) != 0, static_cast<hipEvent_t>(main_begin),
                         static_cast<hipEvent_t>(main_end));
}

int kvv_verdict_noalloc(const kvv_tensor* gen, const kvv_tensor* ref, const kvv_policy* policy, kvv_result* out,
                        void* stream) {
  kvv::SegDesc d;
  int rc = kvv::plan_single(gen, ref, policy, d);
  if (rc) return rc;
  size_t need = 0;
  rc = kvv::single_workspace_bytes(d, &need, false);
  if (rc) return rc;
  if (need > kvv::kScratchBytes)
    return kvv::fail(KVV_E_WORKSPACE, "this verdict needs " + std::to_string(need) +
                                          " bytes of workspace; the no-alloc entry point holds " +
                                          std::to_string(kvv::kScratchBytes) +
                                          " (lower max_samples, or call kvv_verdict with a workspace)");
  void* ws = nullptr;
  bool kept = false;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  rc = kvv::scratch_address(&ws, kvv::stream_capturing(st), &kept);
  if (rc) return rc;
  // the scratch array is the library's own: only its calls write it, eagerly,
  // until a graph holding one of them exists on the device
  return kvv::run_single(d, out, ws, kvv::kScratchBytes, st, kept);
}

int kvv_batch_workspace_size(int32_t count, const kvv_tensor* gens, const kvv_tensor* refs,
                             const kvv_policy* policies, size_t* bytes) {
  if (!bytes) return kvv::fail(KVV_E_INVALID, "null bytes pointer");
  kvv::BatchPlan& bp = kvv::thread_plan();
  int rc = kvv::plan_batch(count, gens, refs, policies, bp);
  if (rc) return rc;
  kvv::NearMode near;
  near.exact = bp.near;
  *bytes = kvv::workspace_layout(bp.run_slots, bp.samples, (int64_t)bp.table.size(), bp.nslots, bp.chunks, bp.items,
                                 near, true, (int64_t)bp.isel_seg.size(), (int64_t)bp.isel_chunk.size() / 2, bp.rounds,
                                 (int64_t)bp.groups.size())
               .total;
  return KVV_OK;
}

int kvv_verdict_batch(int32_t count, const kvv_tensor* gens, const kvv_tensor* refs, const kvv_policy* policies,
                      kvv_result* out, void* workspace, size_t workspace_bytes, void* stream) {
  // the call uploads its host-written table (and plans on the host): a graph
  // would replay a stale upload
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) != hipSuccess)
    return kvv::fail(KVV_E_HIP, "hipStreamIsCapturing failed");
  if (cs != hipStreamCaptureStatusNone)
    return kvv::fail(KVV_E_UNSUPPORTED, "kvv_verdict_batch cannot be captured into a graph");
  kvv::BatchPlan& bp = kvv::thread_plan();
  int rc = kvv::plan_batch(count, gens, refs, policies, bp);
  if (rc) return rc;
  kvv::take_kept(workspace, 0, 0);  // a batch writes the workspace its own way
  return kvv::run_batch(bp, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
