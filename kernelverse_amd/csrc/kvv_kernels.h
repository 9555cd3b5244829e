// Verdict kernels for gfx950 (wave64).
//
//   scan_kernel   one HBM pass over both tensors.  Every wave owns a
//                 contiguous range of "items" (64 lanes x kUnroll 16-byte
//                 vectors of each tensor) and streams it with no block
//                 barrier; the next item's loads are in flight while the
//                 current one, staged in the wave's LDS region, is processed:
//                   phase A  bit-identical finite pairs settled with packed
//                            dot products (their squares feed the fp64 sums);
//                            an exact per-element form re-runs an item whose
//                            dot sums leave the range where they are exact;
//                   phase B  the other pairs, compacted into a per-wave LDS
//                            queue, get the full per-element treatment;
//                   samples  the strided sample of p99 / cosine / norm ratio,
//                            gathered from the stage into a per-wave LDS
//                            buffer that is written out at the end.
//                 A single-pair launch folds its four wave records into one
//                 block record (last wave of the block); a batch launch
//                 writes one record per wave and segment run.
//   near_kernel   tolerant-policy near-zero diagnostics: the rank-strided
//                 sample of the compacted near-zero abs_diff array.
//   tail_kernel   (kvv_tail.h) the fold of the run records into kvv_result
//                 and the radix selection of the p99 order statistics.
#pragma once

#include "kvv_device.h"

namespace kvv {

constexpr int kUnroll = 4;            // 16-byte vectors per thread per item
constexpr int kSelChunk = 8192;       // sample values per select round of a large group
constexpr int kStreamChunk = 8192;    // values per round when one block streams a whole group
constexpr int kMaxSelRounds = 4;      // rounds per select block (many samples in a launch: fewer, fuller blocks)
constexpr int kMaxRounds = 4;         // dispatch rounds of a single-segment scan grid (blocks per CU)
constexpr int kSmall = 8192;          // groups of at most this many samples are selected by one block
constexpr int64_t kGroupStreamMax = 1 << 22;  // largest group one block streams in a many-group launch
constexpr int kArrays = 3;            // abs, rel, near-zero abs
constexpr uint32_t kFlagInputSelect = 0x80000000u;  // SegDesc.flags: abs/rel p99 selected from the inputs
// SegDesc.flags: the near-zero diagnostics of a single fp16/bf16 pair, taken in the main pass as "entries"
// (near-zero elements with a nonzero abs_diff: their rank among the wave's near-zero elements and value);
// the other near-zero elements are the zeros of the compacted array (GCR:525-529)
constexpr uint32_t kFlagNearEntries = 0x40000000u;
constexpr uint32_t kFlagNearAny = KVV_FLAG_NEAR_ZERO | kFlagNearEntries;
// SegDesc.flags: a single pair whose main pass also histograms the top 8 key bits of its abs/rel
// samples (select level 0) into the select slots, which a launch before it cleared
constexpr uint32_t kFlagMainHist = 0x20000000u;
// SegDesc.flags: an input-select segment whose sampled abs/rel values at or above the thresholds a
// pivot launch estimated (cap_key) are captured and the nonzero ones below them counted; the p99
// order statistics are then selected among the captured values.  With kFlagCaptureElems every
// element is a sample (m == n) and the main pass captures; otherwise a capture pass over the
// strided samples does.
constexpr uint32_t kFlagCapture = 0x10000000u;
constexpr uint32_t kFlagCaptureElems = 0x08000000u;
// Per-segment input-select state (u32 words), cleared by the pivot launch
// (IS_HIST .. IS_BASE: the input-select passes; the rest: the capture path).
enum IselWord {
  IS_HIST = 0,                 // [2][2048] top-digit histograms of abs_diff, rel_diff (zeros aside)
  IS_ZEROS = 2 * 2048,         // exact zeros (abs_diff == rel_diff == +0)
  IS_FILL,                     // [2] values captured (the capture pass), per array
  IS_NAN = IS_FILL + 2,        // [2] the array holds a NaN
  IS_PFX = IS_NAN + 2,         // [2][2] bin of each order statistic
  IS_BASE = IS_PFX + 4,        // [2][2] values below each of those bins
  IS_BELOW = IS_BASE + 4,      // [2] kFlagCapture: nonzero values below the capture thresholds
  IS_CNAN = IS_BELOW + 2,      // [2] kFlagCapture: a captured value is NaN
  IS_CNEG = IS_CNAN + 2,       // kFlagCapture: a negative abs_diff (an int32 difference of INT_MIN) sits
                               // below the zeros, which the counts do not place: the segment falls back
  IS_FALLBACK,                 // kFlagCapture: an order statistic lies below the thresholds, so the
                               // input-select passes select this segment instead
  IS_GFILL,                    // [2] values appended by the input-select gather, per array
  kIselStateWords = 4160       // 16,640 bytes: a multiple of 256
};
static_assert(IS_GFILL + 1 < kIselStateWords && (kIselStateWords * 4) % 256 == 0, "input-select state");
constexpr int64_t kIselChunk = 1 << 17;        // elements per input-select chunk (every element a sample)
constexpr int64_t kIselChunkSampled = 1 << 14;  // samples per chunk at strided positions (element loads)
// Per (large segment, array) slot: level-0 histogram (256), its kH0Copies
// copies that the main pass's blocks add into (block b into copy b mod
// kH0Copies: the bins every block touches, e.g. the zeros, would otherwise
// serialise 768 device-scope atomics on one address), level-1 histograms
// (2 ranks x 4096) and the NaN count.
constexpr int kH0Copies = 16;
constexpr int kH0 = 0, kH0R = 256, kH1 = 256 + kH0Copies * 256, kMisc = kH1 + 8192;
constexpr int kSlotWords = kMisc + 64;
// Level-1 candidates of a select round (kSelChunk samples): its values under the
// ranks' level-0 prefixes, grouped by (rank, level-1 digit), with the start of
// every cell of 8 of those 8192 groups (and the total) in a table of kSubTab
// u16, and the smallest and largest candidate of every cell (kSubMM words).
// Cells this narrow usually hold one value when the values are discrete (e.g.
// ULP steps of 8-bit significands lie 8 or more groups apart): the final
// read-off then takes the key from the cell bounds and reads no candidate.
constexpr int kCellShift = 3;
constexpr int kCells = 8192 >> kCellShift;
constexpr int kSubTab = kCells + 2;
constexpr int kSubMM = 2 * kCells;
// fkey(+0.0f), the abs and rel diffs of identical pairs.  Select level 1
// leaves these exact zeros out of its histograms and candidates.
constexpr uint32_t kZeroKey = 0x80000000u;

enum Layout { L_CONTIG = 0, L_ROWS = 1, L_GENERIC = 2 };
enum ScanKind { K_CONTIG = 0, K_ROWS = 1, K_SCALAR = 2 };

// Wave-level counters kept in LDS (one row per wave): the LdsCounter set.
// The wave's LDS counters: the run columns' counts, then (kFlagCapture) the
// run's nonzero abs / rel values below the capture thresholds (added to the
// segment's input-select state at the end of the run), its captured abs / rel
// values so far, and the run's first element (where its captures go).
constexpr int WC_BELOW = LC_COUNT, WC_CFILL = LC_COUNT + 2, WC_CBASE = LC_COUNT + 4;
constexpr int WC_COUNT = LC_COUNT + 5;

struct Dims {
  int32_t ndim;
  int32_t pad;
  int64_t sizes[KVV_MAX_DIMS];
  int64_t gstr[KVV_MAX_DIMS];
  int64_t rstr[KVV_MAX_DIMS];
};

// One tensor pair ("segment") as the kernels see it.
struct SegDesc {
  const void* g;
  const void* r;
  int64_t n;              // numel
  int64_t m;              // sample count: min(n, max_samples)
  int64_t max_samples;
  int64_t item_begin;     // first global item of this segment
  int64_t item_count;
  int64_t sample_off;     // offset into the sample arrays
  int64_t chunk_begin;    // first select chunk of this segment (per array)
  int64_t chunk_count;    // select chunks per array (sized for m)
  // The runs of this segment (a run: the part of one wave's item range, in a
  // batch, or of one block's, for a single pair, inside the segment): how
  // many, and the first wave range that starts inside it (batch).
  int64_t run_n;
  int64_t run_k0;
  uint64_t s_div, s_mod;  // (n-1) = s_div*(m-1) + s_mod: sample i sits at i*s_div + floor(i*s_mod/(m-1))
  uint32_t s_magic;       // floor(t/(m-1)) = mulhi(t, s_magic) >> s_shift for t < 64*(m-1)
  uint32_t s_shift;
  int32_t layout;         // enum Layout
  int32_t vec;            // 16-byte vector access allowed
  int32_t mode;           // enum kvv_mode
  uint32_t flags;
  int32_t zero_tol;       // rtol == atol == 0: isclose is plain equality
  int32_t fast;           // bit-identical finite pairs may take the short path
  int32_t max_abs_diff;
  float rtol, atol, nz_abs, nz_bad;
  int32_t dtype;
  int32_t item_elems;
  int32_t out_index;      // position of this pair's kvv_result in the caller's array
  int32_t lslot;          // large-group select slot (m > kSmall), else -1
  int32_t sel_rounds;     // kSelChunk sub-chunks per select block of a large group (1..kMaxSelRounds)
  int32_t isel_slot;      // input-select state of the segment (kFlagInputSelect), else -1
  int32_t isel_chunk0;    // its first input-select chunk (batch-wide numbering)
  int32_t nz_code;        // kFlagNearEntries: largest magnitude code with |value| <= nz_abs, -1 for none
  int32_t row_items;      // L_ROWS with one outer dim and rows of whole items: items per row, else 0
  int64_t run_slot0;      // first run slot of this segment (a multiple of 4)
  int64_t row_len;        // L_ROWS: contiguous inner length
  Dims dims;              // L_ROWS: outer dims; L_GENERIC: all dims
  // kFlagCapture (the thresholds are written by the pivot launch, on the device):
  float* cap_buf[2];      // where the captured abs / rel values go (the segment's sample region)
  uint32_t* cap_state;    // the segment's input-select state words
  uint32_t cap_key[2];    // capture the nonzero values whose key is at least these (abs, rel)
  float cap_rel_lo;       // rel_diff can reach cap_key[1] only where abs_diff >= cap_rel_lo * den
  float cap_rel_hi;       // rel_diff reaches cap_key[1] where abs_diff >= fma(cap_rel_hi, |ref|, cap_rel_hic)
  float cap_rel_hic;
  int32_t isel_group;     // input-select: the segment's dtype group (which fallback launch takes it)
  int32_t isel_pad[2];
};

// Samples per input-select chunk of segment d.
__host__ __device__ inline int64_t isel_chunk_len(const SegDesc& d) {
  return d.m == d.n ? kIselChunk : kIselChunkSampled;
}

// Partial verdict of a contiguous run of items handled by one block, stored
// field-major ("columns") at a dense run slot: column c of slot k is at
// u32[c * stride + k] or u64[c * stride + k].  Counts of one run fit 32 bits
// (the host keeps a block's element range below 2^32).
enum RunColU32 { CU_MISM = LC_COUNT, CU_MMABS, CU_MMREL, CU_GABSK, CU_GRELK, kColU32 };
enum RunColU64 { CL_FIRSTMM = 0, CL_FIRSTVIOL, CL_GABSI, CL_GRELI, CL_S0, kColU64 = CL_S0 + 7 };
struct RunCols {
  uint32_t* u32;
  uint64_t* u64;
  int64_t stride;  // slots per column (a multiple of 4)
};

struct ScanArgs {
  SegDesc seg0;            // the segment when table == nullptr
  const SegDesc* table;    // batch: segments of this launch, ascending item_begin
  int32_t nseg;
  int32_t pad;
  int64_t item_lo;         // items of this launch: [item_lo, item_lo + items)
  int64_t items;
  int64_t items_per_wave;  // each wave of the grid owns this many consecutive items
  const int64_t* starts;   // batch: wave k owns items [starts[k], starts[k + 1]) (from item_lo)
  // single-segment launches filling the device in `rounds` dispatch rounds of
  // `round_blocks` blocks (rounds > 1): round r's waves own round_ipw[r] items
  // each, from round_first[r] on (round_first[rounds] == items)
  int32_t rounds;
  int32_t round_blocks;
  int64_t round_first[kMaxRounds + 1];
  int64_t round_ipw[kMaxRounds];
  RunCols runs;            // one slot per run (see run_slot)
  float* sample_abs;
  float* sample_rel;
  uint32_t* item_near;     // near-zero count per item (KVV_FLAG_NEAR_ZERO)
  uint4* zero_ptr;         // select slots cleared by this launch (split over its blocks)
  int64_t zero_n4;         // their size in 16-byte words (0: none)
  uint4* zero2_ptr;        // a second region cleared likewise (the near-zero sample built from entries)
  int64_t zero2_n4;
  // kFlagNearEntries: wave q owns entries [q * ent_quota, (q + 1) * ent_quota) and writes, when done,
  // its near-zero count and its entry count (kNone32 when its entries did not fit)
  uint2* ent;              // (rank among the wave's near-zero elements, abs_diff bits)
  uint32_t* near_wave;
  uint32_t* ent_fill;
  uint2* wave_range;       // the wave's items [x, y), relative to the segment's first item (a wave whose
                           // entries did not fit is re-read from them by the first tail launch)
  uint32_t ent_quota;
  uint32_t pad_ent;
  uint32_t* slots;         // kFlagMainHist: the select slots (abs, rel) the blocks' level-0 histograms join
  uint4* cap_runs;         // batch, kFlagCapture: per run slot (first element, captured abs, captured rel, 0)
};

// Per-lane accumulators.  Counts live in the per-wave LDS counters instead.
struct Acc {
  uint32_t mm_abs, mm_rel;
  uint32_t gabs_k, grel_k;
  uint32_t nfast;          // bit-identical finite pairs (ULP bucket 0, never a mismatch)
  uint32_t nmm;            // mismatches
  uint32_t nnear_fast;     // ... of which near zero
  float rel_thr;           // rel-max filter: only rel >= ~rel_thr can still win
  // element indices are offsets from the run's first element (a run spans
  // fewer than 2^32 - 1 elements), kNone32 for none
  uint32_t first_mm, first_viol;
  uint32_t gabs_i, grel_i;
  uint32_t first_fast;     // lowest index of such a pair (an abs/rel argmax candidate of value 0)
  double e_sq;             // sum of g*g over those pairs (there g == r: it feeds gg, rr and gr)
  double s[7];             // other pairs: gg rr gr dd | sampled gg rr gr
  __device__ void init() {
    mm_abs = mm_rel = 0;
    gabs_k = grel_k = 0;
    nfast = nnear_fast = nmm = 0;
    rel_thr = -__builtin_inff();
    first_mm = first_viol = kNone32;
    gabs_i = grel_i = kNone32;
    first_fast = kNone32;
    e_sq = 0.0;
#pragma unroll
    for (int i = 0; i < 7; ++i) s[i] = 0.0;
  }
};

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// Wave-uniform values, stated as such so that they live in scalar registers.
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ uint64_t uniform(uint64_t v) {
  return (uint64_t)uniform((uint32_t)v) | ((uint64_t)uniform((uint32_t)(v >> 32)) << 32);
}

// Adds the number of lanes where `pred` holds to a per-wave LDS counter
// (one ds_add by one lane, whatever the number of lanes).
__device__ __forceinline__ void wave_add(uint32_t* wc, int c, bool pred) {
  const uint64_t b = __ballot(pred);
  if (b && lane_id() == __ffsll((long long)b) - 1) atomicAdd(&wc[c], (uint32_t)__popcll(b));
}

// ------------------------------------------------------------ addressing
__device__ __forceinline__ void outer_offsets(const Dims& dm, int64_t row, int64_t& og, int64_t& orr) {
  og = 0;
  orr = 0;
  for (int k = dm.ndim - 1; k >= 0; --k) {
    const int64_t sz = dm.sizes[k];
    const int64_t q = (k > 0) ? row / sz : 0;
    const int64_t c = (k > 0) ? row - q * sz : row;
    og += c * dm.gstr[k];
    orr += c * dm.rstr[k];
    row = q;
  }
}

__device__ __forceinline__ void elem_offsets(const SegDesc& d, int64_t idx, int64_t& og, int64_t& orr) {
  if (d.layout == L_CONTIG) {
    og = orr = idx;
  } else if (d.layout == L_ROWS) {
    const int64_t row = idx / d.row_len;
    const int64_t col = idx - row * d.row_len;
    outer_offsets(d.dims, row, og, orr);
    og += col;
    orr += col;
  } else {
    outer_offsets(d.dims, idx, og, orr);
  }
}

template <int DT>
__device__ __forceinline__ typename Elem<DT>::T load_elem(const void* base, int64_t off) {
  return reinterpret_cast<const typename Elem<DT>::T*>(base)[off];
}

// ------------------------------------------------------------ per element
// The reference's arithmetic, in float32 with every operation rounded on its
// own (the library is built with -ffp-contract=off):
//   float branch (GCR:722-727)  abs_diff = |g - r|,
//       mismatch = !( r == g || (isfinite(abs_diff) && abs_diff <= atol + |rtol * g|) )
//   integer branch (GCR:716-719) abs_diff = |int32(g) - int32(r)| (wrapping),
//       mismatch = abs_diff > max_abs_diff
//   rel_diff = float(abs_diff) / (|float(r)| + 1e-12f)        (GCR:730)
template <int DT, int MODE>
__device__ __forceinline__ void elem_test(typename Elem<DT>::T gc, typename Elem<DT>::T rc, const SegDesc& d,
                                          float& adf, uint32_t& abs_key, bool& mm, float& rf) {
  using E = Elem<DT>;
  const float gf = E::f32(gc);
  rf = E::f32(rc);
  if constexpr (MODE == KVV_MODE_ISCLOSE) {
    const float ad = fabsf(gf - rf);
    const bool eq = (rf == gf);
    bool close;
    if (d.zero_tol) {
      close = eq;
    } else {
      const float allowed = d.atol + fabsf(d.rtol * gf);
      close = eq || (__builtin_isfinite(ad) && ad <= allowed);
    }
    mm = !close;
    adf = ad;
    abs_key = fkey(ad);
  } else {
    const uint32_t diff = (uint32_t)E::i32(gc) - (uint32_t)E::i32(rc);
    const int32_t sd = (int32_t)diff;
    const int32_t ad = sd < 0 ? (int32_t)(0u - diff) : sd;
    mm = ad > d.max_abs_diff;
    adf = (float)ad;
    abs_key = ikey(ad);
  }
}

// Lower bound below which a rel_diff can no longer beat `best` (conservative:
// the caller skips an element only when abs_diff < thr * (|r| + 1e-12)).  A
// best of +inf keeps a finite bound: a finite abs_diff over a small enough
// denominator also divides to +inf, and such a tie at a lower index must be
// seen.  NaN (the largest key) admits only NaN and +-inf abs_diff, for which
// the comparison fails.
__device__ __forceinline__ float rel_threshold(float best) {
  if (best != best) return __builtin_inff();
  if (best == __builtin_inff()) return 3.4028234e38f * 0.99999f;
  if (best > 0.0f) return best * 0.99999f;
  if (best < 0.0f) return best * 1.00001f;
  return 0.0f;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

// ------------------------------------------------------------ capture (kFlagCapture)
// A run of items (one wave's, within one segment) writes its captured values
// compacted into its own elements' part of the segment's sample region: from
// the run's first element (WC_CBASE) on, WC_CFILL values per array.  A run
// never captures more values than it has elements, so no space is reserved
// and no atomic is taken; the run's counts go to a run record at its end.

// Whether this lane is the lowest active lane of the wave (the one that
// updates a wave-uniform LDS word).
__device__ __forceinline__ bool first_active() {
  return lane_id() == __ffsll((long long)__ballot(true)) - 1;
}

// Appends v for the lanes with p to the run's captures of array x.  Every
// active lane of the wave calls it.
__device__ __forceinline__ void cap_put(const SegDesc& d, uint32_t* wc, int x, bool p, float v) {
  const uint64_t b = __ballot(p);
  if (!b) return;
  const uint32_t fill = wc[WC_CFILL + x], base = wc[WC_CBASE];
  const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
  if (p) d.cap_buf[x][base + fill + below] = v;
  if (first_active()) wc[WC_CFILL + x] = fill + (uint32_t)__popcll(b);
}

// Marks a capture array as holding a NaN when a lane with p captured one.
__device__ __forceinline__ void cap_nan(const SegDesc& d, int x, bool p) {
  const uint64_t b = __ballot(p);
  if (b && lane_id() == __ffsll((long long)b) - 1) d.cap_state[IS_CNAN + x] = 1u;
}

// A capture segment's abs/rel values of the lanes with nz (nonzero abs_diff),
// captured as ca / cr say, the others counted below the thresholds.
__device__ __forceinline__ void capture_put(const SegDesc& d, uint32_t* wc, bool nz, bool ca, bool cr, float adf,
                                            float rel) {
  wave_add(wc, WC_BELOW, nz && !ca);
  wave_add(wc, WC_BELOW + 1, nz && !cr);
  if (__ballot(ca || cr)) {
    cap_put(d, wc, 0, ca, adf);
    cap_put(d, wc, 1, cr, rel);
    cap_nan(d, 0, ca && adf != adf);
    cap_nan(d, 1, cr && rel != rel);
  }
}

// One element of a capture segment whose elements are all samples, for the
// lanes with `act` (every active lane calls it).  A nonzero abs_diff (NaN
// included) is captured when its key reaches cap_key[0], else counted below
// the threshold; rel_diff likewise, divided out only where abs_diff can reach
// its threshold.  Zeros are neither: they are what the counts leave of the
// segment's m values.  A negative abs_diff (max_abs_diff mode: an int32
// difference of INT_MIN) would sit below the zeros: it is flagged, and the
// segment falls back.
__device__ __forceinline__ void capture_elem(const SegDesc& d, float adf, float den, bool act, uint32_t* wc) {
  const bool nz = act && !(adf == 0.0f);
  if (__ballot(act && adf < 0.0f) && first_active()) d.cap_state[IS_CNEG] = 1u;
  const bool ca = nz && fkey(adf) >= d.cap_key[0];
  float rel = 0.0f;
  bool cr = false;
  if (nz && !(adf < d.cap_rel_lo * den)) {
    rel = adf / den;
    cr = fkey(rel) >= d.cap_key[1];
  }
  capture_put(d, wc, nz, ca, cr, adf, rel);
}

// Full treatment of one element for the lanes with `act` set.  Every lane of
// the wave calls it (it uses ballots); counts go to the wave's LDS row `wc`.
template <int DT, int MODE>
__device__ __forceinline__ void slow_elem(typename Elem<DT>::T gc, typename Elem<DT>::T rc, bool act, uint32_t idx,
                                          const SegDesc& d, Acc& acc, uint32_t* wc) {
  using E = Elem<DT>;
  float adf, rf;
  uint32_t abs_key;
  bool mm;
  elem_test<DT, MODE>(gc, rc, d, adf, abs_key, mm, rf);
  const float den = fabsf(rf) + 1e-12f;
  if (d.flags & kFlagCaptureElems) capture_elem(d, adf, den, act, wc);
  mm = mm && act;
  acc.nmm += mm ? 1u : 0u;
  if (mm) {
    const float rel = adf / den;
    const uint32_t rk = fkey(rel);
    if (idx < acc.first_mm) acc.first_mm = idx;
    acc.mm_abs = abs_key > acc.mm_abs ? abs_key : acc.mm_abs;
    acc.mm_rel = rk > acc.mm_rel ? rk : acc.mm_rel;
  }
  if (act && better32(abs_key, idx, acc.gabs_k, acc.gabs_i)) {
    acc.gabs_k = abs_key;
    acc.gabs_i = idx;
  }
  // rel argmax: an element below the wave's best so far cannot be the argmax,
  // so the bound is shared by the wave's lanes (the division is then rare)
  bool raised = false;
  if (act && !(adf < acc.rel_thr * den)) {
    const float rel = adf / den;
    const uint32_t rk = fkey(rel);
    if (better32(rk, idx, acc.grel_k, acc.grel_i)) {
      acc.grel_k = rk;
      acc.grel_i = idx;
      const float t = rel_threshold(rel);
      raised = !(t <= acc.rel_thr);
      acc.rel_thr = raised ? t : acc.rel_thr;
    }
  }
  if (__ballot(raised)) acc.rel_thr = wave_max_f32(acc.rel_thr);
  bool nan_pair = false;
  if constexpr (E::is_float) {
    const bool nf = act && !(E::finite(gc) && E::finite(rc));
    if (__ballot(nf)) {
      // finite-pattern rule of GCR:414-437 at a non-finite position
      const bool ng = E::isnan(gc), nr = E::isnan(rc);
      const bool ig = E::isinf(gc), ir = E::isinf(rc);
      const bool ok = (ng && nr) || (ig && ir && E::sign(gc) == E::sign(rc));
      const bool viol = nf && !ok;
      wave_add(wc, LC_VIOL, viol);
      if (viol && idx < acc.first_viol) acc.first_viol = idx;
      wave_add(wc, LC_NAN_G, nf && ng);
      wave_add(wc, LC_NAN_R, nf && nr);
      wave_add(wc, LC_PINF_G, nf && ig && !E::sign(gc));
      wave_add(wc, LC_NINF_G, nf && ig && E::sign(gc));
      wave_add(wc, LC_PINF_R, nf && ir && !E::sign(rc));
      wave_add(wc, LC_NINF_R, nf && ir && E::sign(rc));
      nan_pair = ng || nr;
      wave_add(wc, LC_NANPAIR, act && nan_pair);
    }
  }
  // ULP histogram: one aggregated add when the wave's elements share a bucket
  // (e.g. 1-ULP steps), else every lane adds its own in one LDS atomic
  // instruction (a loop over the distinct buckets would serialise the wave)
  const bool hv = act && !nan_pair;
  const int bk = pair_bucket<DT>(gc, rc);
  const uint64_t hb = __ballot(hv);
  if (hb) {
    const int l0 = __ffsll((long long)hb) - 1;
    const int kb = __builtin_amdgcn_readlane(bk, l0);  // l0 is wave-uniform: a register read, no LDS trip
    const uint64_t same = __ballot(hv && bk == kb);
    if (same == hb) {
      if (lane_id() == l0) atomicAdd(&wc[LC_HIST0 + kb], (uint32_t)__popcll(same));
    } else if (hv) {
      atomicAdd(&wc[LC_HIST0 + bk], 1u);
    }
  }
  if (act) {
    const double g64 = E::f64(gc), r64 = E::f64(rc);
    const double d64 = g64 - r64;
    acc.s[0] = fma(g64, g64, acc.s[0]);
    acc.s[1] = fma(r64, r64, acc.s[1]);
    acc.s[2] = fma(g64, r64, acc.s[2]);
    acc.s[3] = fma(d64, d64, acc.s[3]);
  }
  if (d.flags & kFlagNearAny) {
    const bool near = fabsf(rf) <= d.nz_abs;
    // (with near-zero entries, every element's near-zero count comes from the item's masks)
    if (d.flags & KVV_FLAG_NEAR_ZERO) wave_add(wc, LC_NEAR, act && near);
    wave_add(wc, LC_NEARBAD, act && near && adf > d.nz_bad);
    wave_add(wc, LC_FARMM, mm && !near);
  }
}

// One sampled element: its abs/rel go to the sample arrays at sample index i,
// its values into the sampled fp64 sums (cosine and norm ratio, GCR:351-393).
template <int DT, int MODE>
__device__ __forceinline__ void sample_one(const SegDesc& d, int64_t idx, int64_t i, Acc& acc, float* sabs,
                                           float* srel) {
  using E = Elem<DT>;
  int64_t og, orr;
  elem_offsets(d, idx, og, orr);
  const auto gc = load_elem<DT>(d.g, og);
  const auto rc = load_elem<DT>(d.r, orr);
  float adf, rf;
  uint32_t k;
  bool mm;
  elem_test<DT, MODE>(gc, rc, d, adf, k, mm, rf);
  sabs[d.sample_off + i] = adf;
  srel[d.sample_off + i] = adf / (fabsf(rf) + 1e-12f);
  const double g64 = E::f64(gc), r64 = E::f64(rc);
  acc.s[4] = fma(g64, g64, acc.s[4]);
  acc.s[5] = fma(r64, r64, acc.s[5]);
  acc.s[6] = fma(g64, r64, acc.s[6]);
}

// Sample indices of the logical range [L0, L1): idx_i = i*(n-1)//(m-1) (GCR:346-347),
// or every index when n <= max_samples.  The elements were just streamed by this
// block, so these loads are served by the caches.
template <int DT, int MODE>
__device__ __forceinline__ void sample_range(const SegDesc& d, int64_t L0, int64_t L1, Acc& acc, float* sabs,
                                             float* srel) {
  if (d.n <= d.max_samples) {
    for (int64_t idx = L0 + lane_id(); idx < L1; idx += 64) sample_one<DT, MODE>(d, idx, idx, acc, sabs, srel);
    return;
  }
  const uint64_t num = (uint64_t)d.n - 1, den = (uint64_t)d.m - 1;
  uint64_t i = ((uint64_t)L0 * den + num - 1) / num + (uint64_t)lane_id();
  for (; i < (uint64_t)d.m; i += 64) {
    const uint64_t idx = i * num / den;
    if (idx >= (uint64_t)L1) break;
    sample_one<DT, MODE>(d, (int64_t)idx, (int64_t)i, acc, sabs, srel);
  }
}

// ------------------------------------------------------------ vector item
template <int DT>
struct VecIO {
  using T = typename Elem<DT>::T;
  static constexpr int V = 16 / sizeof(T);
  static constexpr int NE = V * kUnroll;
  union Vec {
    uint4 u;
    T e[V];
  };
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 nt_load16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The item's LDS stage, addressed as LDS explicitly: reads of it must stay
// ds_read instructions.  Through a generic pointer the compiler may merge an
// LDS read and a global read of the same value into one flat load, whose wait
// also waits for the next item's loads in flight.
#define KVV_LDS __attribute__((address_space(3)))
typedef const KVV_LDS uint4* StageP;

template <typename T>
__device__ __forceinline__ T stage_elem(StageP stage, int slot, int e) {
  return ((const KVV_LDS T*)(stage + slot))[e];
}

__device__ __forceinline__ uint4 stage_vec(StageP stage, int slot) {
  const u32x4 v = *(const KVV_LDS u32x4*)(stage + slot);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Issues the 16-byte loads of one item (kUnroll vectors per thread per tensor).
// The (row, item of the row) of the next item a wave loads, for rows made of
// whole items (d.row_items > 0): the item's offsets are then one wave-uniform
// base plus the lane's position, with no per-lane division.
struct RowCursor {
  int64_t row;
  int32_t col_item;
};

__device__ __forceinline__ RowCursor row_cursor_at(const SegDesc& d, int64_t item) {
  RowCursor c{0, 0};
  if (d.row_items > 0) {
    c.row = item / d.row_items;
    c.col_item = (int32_t)(item - c.row * d.row_items);
  }
  return c;
}

template <int DT, int KIND>
__device__ __forceinline__ uint32_t load_item(const SegDesc& d, int64_t L0, int64_t L1, uint4* gv, uint4* rv,
                                              RowCursor* rc = nullptr) {
  using IO = VecIO<DT>;
  using T = typename IO::T;
  constexpr int V = IO::V;
  uint32_t full = 0;
  if constexpr (KIND == K_ROWS) {
    if (rc && d.row_items > 0) {
      // every vector of the item lies in row rc->row (no partial vectors: n is whole items)
      const int64_t col0 = (int64_t)rc->col_item * d.item_elems;
      const int64_t og0 = rc->row * d.dims.gstr[0] + col0, or0 = rc->row * d.dims.rstr[0] + col0;
      if (++rc->col_item == d.row_items) {
        rc->col_item = 0;
        ++rc->row;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t off = (int64_t)(u * 64 + lane_id()) * V;
        gv[u] = nt_load16(reinterpret_cast<const T*>(d.g) + og0 + off);
        rv[u] = nt_load16(reinterpret_cast<const T*>(d.r) + or0 + off);
      }
      return (1u << kUnroll) - 1;
    }
  }
  // rows: one division per lane and item; a lane's later vectors step the
  // (row, column) pair, rows being at least one step (64 vectors) long
  int64_t row = 0, col = 0;
  const bool step_rows = KIND != K_CONTIG && d.row_len >= 64 * V;
  if constexpr (KIND != K_CONTIG) {
    if (step_rows) {
      const int64_t v0 = L0 + (int64_t)lane_id() * V;
      row = ((v0 | d.row_len) >> 32) == 0 ? (int64_t)((uint32_t)v0 / (uint32_t)d.row_len) : v0 / d.row_len;
      col = v0 - row * d.row_len;
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = L0 + (int64_t)(u * 64 + lane_id()) * V;
    if constexpr (KIND != K_CONTIG) {
      if (u > 0 && step_rows) {
        col += 64 * V;
        if (col >= d.row_len) {
          col -= d.row_len;
          ++row;
        }
      }
    }
    if (v + V <= L1) {
      full |= 1u << u;
      int64_t og, orr;
      if constexpr (KIND == K_CONTIG) {
        og = orr = v;
      } else {
        int64_t r = row, c = col;
        if (!step_rows) {
          r = v / d.row_len;
          c = v - r * d.row_len;
        }
        outer_offsets(d.dims, r, og, orr);
        og += c;
        orr += c;
      }
      // streamed once: non-temporal loads keep them from displacing reusable lines
      gv[u] = nt_load16(reinterpret_cast<const T*>(d.g) + og);
      rv[u] = nt_load16(reinterpret_cast<const T*>(d.r) + orr);
    } else {
      gv[u] = make_uint4(0, 0, 0, 0);  // a partial last vector: patch_partial fills it
      rv[u] = make_uint4(0, 0, 0, 0);
    }
  }
  return full;
}

// Puts the elements of a lane's partial last vector (numel not a multiple of
// the vector width; load_item left it zero) into its registers before the
// stage write, so that every element of the item is in the stage and the
// item's later steps read LDS only.  It runs before the next item's loads are
// issued: a global load among the later steps would make the compiler wait
// (vmcnt counts in issue order) for those loads as well.
template <int DT, int KIND>
__device__ __forceinline__ void patch_partial(const SegDesc& d, int64_t L0, int64_t L1, uint32_t full, uint4* gv,
                                              uint4* rv) {
  using T = typename Elem<DT>::T;
  constexpr int V = VecIO<DT>::V;
  constexpr int W = 8 * (int)sizeof(T);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = L0 + (int64_t)(u * 64 + lane_id()) * V;
    const int ne = ((full >> u) & 1u) || v >= L1 ? 0 : (int)(L1 - v);  // < V
    if (ne == 0) continue;
    uint64_t g0 = 0, g1 = 0, r0 = 0, r1 = 0;
#pragma unroll 1
    for (int e = 0; e < ne; ++e) {
      int64_t og, orr;
      if constexpr (KIND == K_CONTIG) {
        og = orr = v + e;
      } else {
        elem_offsets(d, v + e, og, orr);
      }
      const uint64_t gx = (uint64_t)load_elem<DT>(d.g, og), rx = (uint64_t)load_elem<DT>(d.r, orr);
      const int b = e * W;
      if (b < 64) {
        g0 |= gx << b;
        r0 |= rx << b;
      } else {
        g1 |= gx << (b - 64);
        r1 |= rx << (b - 64);
      }
    }
    gv[u] = make_uint4((uint32_t)g0, (uint32_t)(g0 >> 32), (uint32_t)g1, (uint32_t)(g1 >> 32));
    rv[u] = make_uint4((uint32_t)r0, (uint32_t)(r0 >> 32), (uint32_t)r1, (uint32_t)(r1 >> 32));
  }
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves only (no LDS):
// shifts 1, 2, 4, 8 inside each 16-lane row, then row 15 -> next row and lane 31
// -> upper half.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false); // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false); // row_bcast:31
  return v;
}

// ------------------------------------------------------------ phase A (SWAR)
// Phase A classifies every element of a lane's full vectors as "fast" (the
// pair is bit-identical and finite: abs_diff = rel_diff = 0, ULP bucket 0,
// never a mismatch) or "slow" (everything else, finished in phase B).  The
// test runs on whole dwords with packed integer arithmetic, so it costs a few
// instructions per dword instead of compares and lane masks per element.
//
// Slow-mask layout (one bit per element of the lane's kUnroll vectors, dword
// d = u * 4 + j of the item, element s inside the dword):
//   8-bit  elements: bit (d >> 3) * 32 + s * 8 + (d & 7)
//   16-bit elements: bit s * 16 + d
//   32-bit elements: bit d
//   64-bit elements: bit u * 2 + s   (s = element of the vector)
// slot_of() maps a bit back to (vector u, element e of that vector).
static_assert(kUnroll == 4, "the slow-mask layout assumes 16 dwords per lane and item");

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

template <int W>
__device__ __forceinline__ void slot_of(int p, int& u, int& e) {
  if constexpr (W == 8) {
    const int dd = ((p >> 5) << 3) | (p & 7);
    u = dd >> 2;
    e = ((dd & 3) << 2) | ((p >> 3) & 3);
  } else if constexpr (W == 16) {
    const int dd = p & 15;
    u = dd >> 2;
    e = ((dd & 3) << 1) | (p >> 4);
  } else if constexpr (W == 32) {
    u = p >> 2;
    e = p & 3;
  } else {
    u = p >> 1;
    e = p & 1;
  }
}

// Packed per-half minimum with 1: 0 where the 16-bit half is 0, else 1.
__device__ __forceinline__ uint32_t pk_nonzero16(uint32_t v) {
  uint32_t o;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(o) : "v"(v), "s"(0x00010001u));
  return o;
}

// Per-element slow flags of one dword (32-bit codes): 1 at bit s * W of
// element s when the pair differs bitwise or the generated value is not finite.
template <int DT>
__device__ __forceinline__ uint32_t dword_flags(uint32_t g, uint32_t r) {
  using E = Elem<DT>;
  constexpr int W = E::width;
  if constexpr (W == 8) {
    const uint32_t x = g ^ r;
    uint32_t t = ((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x;  // bit 7 of a byte: byte != 0
    if constexpr (DT == KVV_F8E4M3FN) {
      t |= (g & 0x7F7F7F7Fu) + 0x01010101u;              // bit 7: magnitude 0x7F (NaN)
    } else if constexpr (DT == KVV_F8E5M2) {
      t |= (g & 0x7C7C7C7Cu) + 0x04040404u;              // bit 7: exponent all ones
    }
    return (t >> 7) & 0x01010101u;
  } else if constexpr (W == 16) {
    uint32_t v = g ^ r;
    if constexpr (DT == KVV_BF16 || DT == KVV_F16) {
      constexpr uint32_t em = DT == KVV_BF16 ? 0x7F80u : 0x7C00u;
      const u16x2 ge = __builtin_bit_cast(u16x2, g & (em | (em << 16)));
      const u16x2 nf = __builtin_elementwise_sub_sat(ge, (u16x2){(uint16_t)(em - 1), (uint16_t)(em - 1)});
      v |= __builtin_bit_cast(uint32_t, nf);
    }
    return pk_nonzero16(v);
  } else {  // 32-bit lanes (64-bit elements are combined by the caller)
    uint32_t v = g ^ r;
    if constexpr (DT == KVV_F32) v |= __builtin_elementwise_sub_sat(g & 0x7F800000u, 0x7F7FFFFFu);
    return v < 1u ? v : 1u;
  }
}

// Zero mask of a dword from its flags: all ones over each flagged element.
template <int W>
__device__ __forceinline__ uint32_t flag_mask(uint32_t f) {
  // 8-bit: 0x80 | 0x7F per flagged byte, from full-rate ops ((f << 8) - f would
  // become a quarter-rate 32-bit multiply by 255)
  if constexpr (W == 8) {
    uint32_t h = f << 7;
    asm("" : "+v"(h));  // keeps the compiler from folding h | (h - f) back into f * 255
    return h | (h - f);
  }
  else if constexpr (W == 16) return __umul24(f, 0xFFFFu);
  else return 0u - f;
}

// Sum of squares (fp64) and near-zero count of the elements of one dword whose
// code was zeroed where slow (a zeroed element adds 0 and counts as near).
template <int DT, bool NEAR>
__device__ __forceinline__ void dword_fast_sums(uint32_t gz, float nz_abs, double& s0, double& s1, uint32_t& nnear) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int W = E::width;
  constexpr int EPD = 32 / W;
#pragma unroll
  for (int k = 0; k < EPD; ++k) {
    const T c = (T)(gz >> (k * W));
    if constexpr (NEAR) {
      const float f = E::f32(c);
      nnear += fabsf(f) <= nz_abs ? 1u : 0u;
      const double v = (double)f;
      if (k & 1) s1 = fma(v, v, s1); else s0 = fma(v, v, s0);
    } else {
      const double v = E::f64(c);
      if (k & 1) s1 = fma(v, v, s1); else s0 = fma(v, v, s0);
    }
  }
}

// What phase A settled for one lane and item: the slow mask, the number of
// fast (bit-identical finite) pairs, the sum of their squares and, with the
// tolerant policy, how many of them are near zero.  The caller adds them to
// the accumulators once (updates of the accumulators inside the variants were
// merged by the compiler through an address select, which kept them in scratch).
struct PhaseA {
  uint64_t slow;
  uint32_t nfast, nnear;
  double esq;
};

// Lowest logical index of a fast element of the item (vectors in order, then
// elements): an abs/rel argmax candidate of value 0 until a positive one exists.
template <int DT>
__device__ __forceinline__ void track_first_fast(uint32_t R0, uint32_t full, uint64_t slow, Acc& acc) {
  constexpr int V = VecIO<DT>::V;
  uint32_t ff = acc.first_fast;
  for (int p = 0; p < V * kUnroll; ++p) {
    int u, e;
    slot_of<Elem<DT>::width>(p, u, e);
    if (!((full >> u) & 1u) || ((slow >> p) & 1u)) continue;
    const uint32_t idx = R0 + (uint32_t)((u * 64 + lane_id()) * V + e);
    if (idx < ff) ff = idx;
  }
  acc.first_fast = ff;
}

// Phase A over the stage copy of one item: bit-identical finite pairs are
// finished here (count; g*g into e_sq, which feeds gg, rr and gr since g == r);
// returns the lane's slow mask in the layout above.
template <int DT, bool NEAR>
__device__ __forceinline__ PhaseA phase_a(const SegDesc& d, StageP stage, uint32_t full) {
  using E = Elem<DT>;
  using IO = VecIO<DT>;
  constexpr int V = IO::V;
  constexpr int W = E::width;
  const int lane = lane_id();
  uint32_t m0 = 0, m1 = 0;  // slow mask, low and high 32 bits
  double s0 = 0.0, s1 = 0.0;
  uint32_t nnear = 0, nvec = 0;
  const float nz_abs = d.nz_abs;
#pragma unroll 1
  for (int u = 0; u < kUnroll; ++u) {
    if (!((full >> u) & 1u)) continue;
    ++nvec;
    const uint4 gq = stage_vec(stage, (2 * u) * 64 + lane);
    const uint4 rq = stage_vec(stage, (2 * u + 1) * 64 + lane);
    const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
    const uint32_t rw[4] = {rq.x, rq.y, rq.z, rq.w};
    if constexpr (W == 64) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t glo = gw[2 * e], ghi = gw[2 * e + 1];
        uint32_t v = (glo ^ rw[2 * e]) | (ghi ^ rw[2 * e + 1]);
        if constexpr (DT == KVV_F64) v |= __builtin_elementwise_sub_sat(ghi & 0x7FF00000u, 0x7FEFFFFFu);
        const uint32_t f = v < 1u ? v : 1u;
        m0 |= f << (u * 2 + e);
        const uint32_t z = ~(0u - f);
        const uint64_t c = ((uint64_t)(ghi & z) << 32) | (glo & z);
        const double x = E::f64(c);
        if (e) s1 = fma(x, x, s1); else s0 = fma(x, x, s0);
      }
    } else if constexpr (W == 32 && !NEAR) {
      // one element per dword: the squares only where the wave has a fast pair
      uint32_t f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[j] = dword_flags<DT>(gw[j], rw[j]);
        m0 |= f[j] << (u * 4 + j);
      }
      if (__ballot((f[0] & f[1] & f[2] & f[3]) == 0u)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dword_fast_sums<DT, false>(gw[j] & ~flag_mask<W>(f[j]), nz_abs, s0, s1, nnear);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int dd = u * 4 + j;
        const uint32_t f = dword_flags<DT>(gw[j], rw[j]);
        if constexpr (W == 8) {
          if (dd < 8) m0 |= f << dd; else m1 |= f << (dd - 8);
        } else {
          m0 |= f << dd;
        }
        const uint32_t gz = gw[j] & ~flag_mask<W>(f);
        dword_fast_sums<DT, NEAR>(gz, nz_abs, s0, s1, nnear);
      }
    }
  }
  PhaseA o;
  o.slow = ((uint64_t)m1 << 32) | m0;
  const uint32_t nslow = (uint32_t)__popcll(o.slow);
  o.esq = s0 + s1;
  o.nfast = nvec * V - nslow;
  // zeroed slow elements were counted as near when 0 <= nz_abs
  o.nnear = NEAR ? nnear - (0.0f <= nz_abs ? nslow : 0u) : 0u;
  return o;
}

// ------------------------------------------------------------ phase A, dot form
// For 8- and 16-bit codes the squares of the bit-identical pairs are summed
// with the packed dot instructions (two bf16/f16 squares, or four int8 squares,
// per instruction) instead of one fp64 multiply-add per element.
//
// * bf16 / f16 (v_dot2_f32_bf16 / v_dot2_f32_f16): products of two 8- or
//   11-bit significands are exact in fp32; each instruction then rounds the
//   (non-negative) sum downward by at most 1.5 ulp (measured over 2^20 cases per
//   format).  Every accumulator takes kUnroll instructions, so a lane's partial
//   sum is low by at most 4 * 1.5 * 2^-23 < 7.2e-7 relative before it joins the
//   fp64 accumulator.
// * f8 codes become f16 halves: e5m2 is the high byte of an f16; e4m3fn's
//   magnitude bits placed at bits 7..13 of an f16 read as value * 2^-8 (the
//   sum is scaled back by 2^16, exactly).  Signs do not matter for squares.
// * int8 / uint8 (v_dot4_i32_i8 / v_dot4_u32_u8): exact integer sums.
//
// Bit-identical is the only test of the quick form: a lane whose partial sum is
// not finite (an identical NaN or Inf pair, or a bf16 square beyond fp32's
// range), or is below 2^-60 while its values are not all zero (a bf16 square
// below fp32's normal range), re-runs the item with the exact per-element
// classification and fp64 squares (phase_a).  The careful form (CAREFUL) also
// tests finiteness per element, as phase_a does, so only bf16's range can
// still send a lane to phase_a; a wave uses it for a few items after a re-run
// (data with scattered NaN/Inf).  e4m3fn has no infinity and its NaN code is
// part of the identity test, so it never re-runs.
template <int DT>
struct DotForm {
  static constexpr bool on = DT == KVV_BF16 || DT == KVV_F16 || DT == KVV_F8E4M3FN || DT == KVV_F8E5M2 ||
                             DT == KVV_I8 || DT == KVV_U8;
  static constexpr bool is_int = DT == KVV_I8 || DT == KVV_U8;
  static constexpr int NA = Elem<DT>::width == 8 && !is_int ? 8 : 4;  // accumulators per lane
  using A = typename std::conditional<is_int, int32_t, float>::type;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_sq_f16(uint32_t h, float a) {
  const f16x2_t v = __builtin_bit_cast(f16x2_t, h);
  return __builtin_amdgcn_fdot2(v, v, a, false);
}

// Adds the squares of the (zeroed-where-slow) codes of dword j into the accumulators.
template <int DT>
__device__ __forceinline__ void dot_sq(uint32_t z, typename DotForm<DT>::A* a, int j) {
  if constexpr (DT == KVV_BF16) {
    const bf16x2_t v = __builtin_bit_cast(bf16x2_t, z);
    a[j] = __builtin_amdgcn_fdot2_f32_bf16(v, v, a[j], false);
  } else if constexpr (DT == KVV_F16) {
    a[j] = dot2_sq_f16(z, a[j]);
  } else if constexpr (DT == KVV_F8E5M2) {
    a[j] = dot2_sq_f16((z << 8) & 0xFF00FF00u, a[j]);     // bytes 0 and 2
    a[j + 4] = dot2_sq_f16(z & 0xFF00FF00u, a[j + 4]);    // bytes 1 and 3
  } else if constexpr (DT == KVV_F8E4M3FN) {
    a[j] = dot2_sq_f16((z << 7) & 0x3F803F80u, a[j]);     // bytes 0 and 2, value * 2^-8
    a[j + 4] = dot2_sq_f16((z >> 1) & 0x3F803F80u, a[j + 4]);  // bytes 1 and 3
  } else if constexpr (DT == KVV_I8) {
    a[j] = __builtin_amdgcn_sdot4((int)z, (int)z, a[j], false);
  } else {
    a[j] = (int32_t)__builtin_amdgcn_udot4(z, z, (uint32_t)a[j], false);
  }
}

// Per-element slow flags (layout of dword_flags) from bitwise identity alone;
// for e4m3fn also the NaN code, which the f16 mapping above would not expose.
template <int DT>
__device__ __forceinline__ uint32_t ident_flags(uint32_t g, uint32_t r) {
  if constexpr (Elem<DT>::width == 8) {
    const uint32_t x = g ^ r;
    uint32_t t = ((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x;
    if constexpr (DT == KVV_F8E4M3FN) t |= (g & 0x7F7F7F7Fu) + 0x01010101u;
    return (t >> 7) & 0x01010101u;
  } else {
    return pk_nonzero16(g ^ r);
  }
}

template <int DT, bool CAREFUL>
__device__ __forceinline__ PhaseA phase_a_dot(const SegDesc& d, StageP stage, uint32_t full, bool& redone) {
  using DF = DotForm<DT>;
  using A = typename DF::A;
  constexpr int V = VecIO<DT>::V;
  constexpr int W = Elem<DT>::width;
  const int lane = lane_id();
  uint32_t m0 = 0, m1 = 0, orz = 0;
  A a[DF::NA];
#pragma unroll
  for (int k = 0; k < DF::NA; ++k) a[k] = 0;
  // every vector of the item is a full load here (phase_a_any); one vector per
  // iteration keeps the LDS reads in flight (and their registers) few
#pragma unroll 1
  for (int u = 0; u < kUnroll; ++u) {
    const uint4 gq = stage_vec(stage, (2 * u) * 64 + lane);
    const uint4 rq = stage_vec(stage, (2 * u + 1) * 64 + lane);
    const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
    const uint32_t rw[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int dd = u * 4 + j;
      if constexpr (W == 16 && !CAREFUL) {
        // per half: same = sat(1 - (g ^ r)) is 1 for an identical pair, else 0;
        // g * same keeps the identical codes; m0 collects the identical flags
        // (inverted into slow flags below)
        const u16x2 same = __builtin_elementwise_sub_sat(u16x2{1, 1}, __builtin_bit_cast(u16x2, gw[j] ^ rw[j]));
        const uint32_t z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, gw[j]) * same);
        m0 |= __builtin_bit_cast(uint32_t, same) << dd;
        if constexpr (DT == KVV_BF16) orz |= z;
        dot_sq<DT>(z, a, j);
      } else {
        const uint32_t f = CAREFUL ? dword_flags<DT>(gw[j], rw[j]) : ident_flags<DT>(gw[j], rw[j]);
        if constexpr (W == 8) {
          if (dd < 8) m0 |= f << dd; else m1 |= f << (dd - 8);
        } else {
          m0 |= f << dd;
        }
        const uint32_t z = gw[j] & ~flag_mask<W>(f);
        if constexpr (DT == KVV_BF16) orz |= z;
        dot_sq<DT>(z, a, j);
      }
    }
  }
  if constexpr (W == 16 && !CAREFUL) m0 = ~m0;  // identical flags -> slow flags (every vector is full)
  bool redo = false;
  if constexpr (!DF::is_int && DT != KVV_F8E4M3FN) {
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < DF::NA; ++k) t += a[k];
    redo = !(t <= 3.4028234e38f);
    if constexpr (DT == KVV_BF16) redo = redo || (t < 0x1p-60f && (orz & 0x7FFF7FFFu) != 0u);
  }
  redone = __ballot(redo) != 0;
  if (redone && redo) return phase_a<DT, false>(d, stage, full);
  PhaseA o;
  o.slow = ((uint64_t)m1 << 32) | m0;
  double e = 0.0;
#pragma unroll
  for (int k = 0; k < DF::NA; ++k) e += (double)a[k];
  if constexpr (DT == KVV_F8E4M3FN) e *= 65536.0;
  o.esq = e;
  o.nfast = (uint32_t)(kUnroll * V) - (uint32_t)__popcll(o.slow);
  o.nnear = 0;
  return o;
}

// The wave's queue holds 64 * slots entries (entry = (lane << 6) | slot, in
// lane order): kQSlots for 8- and 16-bit elements; 32- and 64-bit elements
// (16 or 8 per lane and item) keep half of it, and the other half holds their
// replicated ULP-bucket counters (QueueGeom).  queue_all appends every slow
// element of the lanes when they fit and returns their number, else returns it
// without writing anything; queue_part then appends the slots [p0, p0 + slots)
// of every lane.
constexpr int kQSlots = 16;
constexpr int kRep = 16;  // copies of each ULP bucket counter of the dense path
template <int DT>
struct QueueGeom {
  static constexpr bool wide = VecIO<DT>::NE <= 16;
  static constexpr int slots = wide ? kQSlots / 2 : kQSlots;
  static constexpr int rep_words = wide ? kBuckets * kRep : 1;
  static_assert(!wide || 64 * slots * 2 >= kBuckets * kRep * 4, "the counters take the queue's other half");
};

template <int SLOTS>
__device__ __forceinline__ uint32_t queue_all(uint64_t slow, uint16_t* queue) {
  const int lane = lane_id();
  const uint32_t cnt = (uint32_t)__popcll(slow);
  const uint32_t incl = wave_incl_scan(cnt);
  const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  if (total > 64u * SLOTS) return total;
  uint32_t at = incl - cnt;
  while (slow) {
    queue[at++] = (uint16_t)((lane << 6) | __builtin_ctzll(slow));
    slow &= slow - 1;
  }
  return total;
}

template <int SLOTS>
__device__ __forceinline__ uint32_t queue_part(uint32_t part, int p0, uint16_t* queue) {
  const int lane = lane_id();
  part &= (1u << SLOTS) - 1;
  const uint32_t cnt = (uint32_t)__popc(part);
  const uint32_t incl = wave_incl_scan(cnt);
  const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  uint32_t at = incl - cnt;
  while (part) {
    queue[at++] = (uint16_t)((lane << 6) | (p0 + __builtin_ctz(part)));
    part &= part - 1;
  }
  return total;
}

// Phase B: the wave's queued elements, 64 at a time, from the LDS stage.
template <int DT, int MODE>
__device__ __forceinline__ void phase_b(const SegDesc& d, uint32_t R0, uint32_t total, StageP stage,
                                        const uint16_t* queue, Acc& acc, uint32_t* wc) {
  using IO = VecIO<DT>;
  using T = typename IO::T;
  constexpr int V = IO::V;
  const int lane = lane_id();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (uint32_t j = 0; j < total; j += 64) {
    const uint32_t qi = j + lane;
    const bool act = qi < total;
    const uint32_t ent = act ? queue[qi] : 0u;
    const int src = (int)(ent >> 6);
    int u, e;
    slot_of<Elem<DT>::width>((int)(ent & 63), u, e);
    const T gc = stage_elem<T>(stage, (2 * u) * 64 + src, e);
    const T rc = stage_elem<T>(stage, (2 * u + 1) * 64 + src, e);
    const uint32_t idx = R0 + (uint32_t)((u * 64 + src) * V + e);
    slow_elem<DT, MODE>(gc, rc, act, idx, d, acc, wc);
  }
}

// Phase B in place, for an item of 32- or 64-bit elements whose pairs are
// mostly slow (e.g. every pair perturbed by noise): each lane finishes its own
// slot p of the stage, p = 0 .. NE-1, one slow_elem call per slot, with no
// queue (its writes, reads and the stage reads that depend on them).  Taken
// when every lane has at least 3/4 of its slots slow, where the queue would
// need nearly as many calls.  Returns whether it ran.  (Narrower elements keep
// the queue: mostly-slow items are rare there, and the extra path in their
// item loop cost more than it saved.)
template <int DT, int MODE>
__device__ __forceinline__ bool phase_b_dense(const SegDesc& d, uint32_t R0, uint64_t slow, StageP stage, Acc& acc,
                                              uint32_t* wc) {
  using IO = VecIO<DT>;
  using T = typename IO::T;
  constexpr int V = IO::V;
  if constexpr (IO::NE > 16) {
    return false;
  } else {
    if (__ballot((uint32_t)__popcll(slow) * 4u < 3u * (uint32_t)IO::NE)) return false;
    const int lane = lane_id();
#pragma unroll 1
    for (int p = 0; p < IO::NE; ++p) {
      int u, e;
      slot_of<Elem<DT>::width>(p, u, e);
      const T gc = stage_elem<T>(stage, (2 * u) * 64 + lane, e);
      const T rc = stage_elem<T>(stage, (2 * u + 1) * 64 + lane, e);
      slow_elem<DT, MODE>(gc, rc, ((slow >> p) & 1u) != 0, R0 + (uint32_t)((u * 64 + lane) * V + e), d, acc, wc);
    }
    return true;
  }
}

// Phase B in place for an fp32 item of mostly slow pairs under the isclose test
// without near-zero diagnostics (e.g. every pair perturbed by noise): each lane
// walks its own slots once and finishes every slow pair whose values have one
// sign, other bits (a nonzero difference) and a finite abs_diff.  Such a "lean"
// pair has no finite-pattern or NaN outputs; its ULP distance is the distance
// of its codes.  Its ULP bucket goes to copy lane % kRep of the wave's
// replicated counters `rep` (no ballots, and at most four increments of one
// element step meet at an address); its abs key, fp64 sums and captures are
// taken in registers.
//
// Two conservative single-compare tests keep the division off the common path:
// * tolerance: abs_diff <= fma(|gen|, rtol_lo, atol_lo) with both tolerances
//   lowered by 2^-21 (lean_tol), which never exceeds the exact allowed bound
//   fl(atol + fl(rtol * |gen|)): such a pair is close;
// * rel bound: abs_diff < fl(thr * |ref|), never above fl(thr * den): such a
//   pair cannot be the rel argmax.
// A pair that fails either takes slow_elem's exact tests in place (the
// mismatch counters, the rel argmax).  The capture of rel_diff is settled by
// fl(cap_rel_lo * |ref|) below and fma(cap_rel_hi, |ref|, cap_rel_hic) above
// (set_thresholds); the division is left to the thin band between.
//
// The other slow pairs (opposite signs, +0 against -0, non-finite values) are
// returned as a mask for the queue and slow_elem.  The lean pairs of a lane
// come in ascending index order and precede the item's queued pairs, so a
// strict key comparison keeps the lowest index of a tie.  The bound only
// rises, so a pair below it now stays below it.  Only the slots of fully loaded
// vectors are walked (vec_tail takes a partial one's elements; a bit-identical
// pair, which phase A finished, has a zero difference and is never lean).
// Taken when every lane has at least 3/4 of those slots slow.  Otherwise
// `slow` comes back unchanged.
struct LeanTol {
  float rtol, atol;
};

// Tolerances for the lean form of the isclose test: fma(|g|, rtol_lo, atol_lo)
// with x_lo = fl(x * (1 - 2^-21)) <= x * (1 - 2^-22) is at most (X + A) * (1 -
// 2^-22) before its one rounding, where X = rtol * |g| and A = atol; the exact
// bound fl(A + fl(X)) is at least (X + A) * (1 - 2^-24) - 2^-150.  For A >=
// 2^-127 the first is the smaller, and for A = 0 rounding's monotonicity
// orders them.  Tolerances outside [2^-100, 2^100] (zero aside) or a zero
// tolerance (plain equality) give bounds below zero: no lean pair.
__device__ __forceinline__ LeanTol lean_tol(const SegDesc& d) {
  auto ok = [](float t) { return t == 0.0f || (t >= 0x1p-100f && t <= 0x1p100f); };
  if (d.zero_tol || !ok(d.rtol) || !ok(d.atol)) return LeanTol{-1.0f, -1.0f};
  return LeanTol{d.rtol * (1.0f - 0x1p-21f), d.atol * (1.0f - 0x1p-21f)};
}

// Absolute difference of two codes (one instruction).
__device__ __forceinline__ uint32_t abs_diff_u32(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_sad_u32 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

template <int DT, int MODE>
__device__ __forceinline__ uint64_t phase_b_lean(const SegDesc& d, uint32_t R0, uint64_t slow, uint32_t full,
                                                 StageP stage, Acc& acc, KVV_LDS uint32_t* rep, uint32_t* wc) {
  constexpr int V = VecIO<DT>::V;
  if constexpr (DT != KVV_F32 || MODE != KVV_MODE_ISCLOSE) {
    return slow;
  } else {
    // (a lane's slots: those of its fully loaded vectors; the others are vec_tail's)
    if (__ballot((uint32_t)__popcll(slow) * 4u < 3u * (uint32_t)V * (uint32_t)__popc(full))) return slow;
    const int lane = lane_id();
    float thr = acc.rel_thr;
    if (__ballot(!(thr > -__builtin_inff()))) {
      // no bound yet (the run's first pairs): the largest finite rel_diff of the
      // wave's slot-0 pairs gives one.  The pairs that reach it are queued, so
      // every pair skipped below it has a strictly smaller rel_diff than a
      // pair slow_elem will see.
      const float g = stage_elem<float>(stage, lane, 0), r = stage_elem<float>(stage, 64 + lane, 0);
      const float rel = fabsf(g - r) / (fabsf(r) + 1e-12f);
      const float m = wave_max_f32((slow & 1u) && __builtin_isfinite(rel) ? rel : -__builtin_inff());
      if (m > -__builtin_inff()) {
        const float t = rel_threshold(m);
        thr = t > thr ? t : thr;
      }
    }
    const LeanTol lt = lean_tol(d);
    const bool zt = d.zero_tol != 0;
    // the ULP counters by leading zeros of the distance: row j - 17 for bucket
    // 32 - j, bucket 15 (distances of 2^14 and more) in row 0
    KVV_LDS uint32_t* const mine = rep + (lane & (kRep - 1)) - 17 * kRep;
    // the lane's largest lean abs_diff (its bits; abs_diff >= 0) and its slot
    uint32_t best = acc.gabs_k > kZeroKey ? acc.gabs_k & 0x7FFFFFFFu : 0u;
    int bslot = -1;
    uint32_t leanm = 0;
    const bool capseg = (d.flags & kFlagCaptureElems) != 0;
    uint32_t cm[2] = {0u, 0u};  // capture segment: the lean slots whose abs / rel value is captured
    // (the thresholds in registers: loads of them inside the loop would wait on its LDS atomics)
    const uint32_t ca0 = uniform(d.cap_key[0]) & 0x7FFFFFFFu, ck1 = uniform(d.cap_key[1]);
    const float crlo = __uint_as_float(uniform(__float_as_uint(d.cap_rel_lo)));
    const float crhi = __uint_as_float(uniform(__float_as_uint(d.cap_rel_hi)));
    const float crhc = __uint_as_float(uniform(__float_as_uint(d.cap_rel_hic)));
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (__ballot(((slow >> (u * V)) & 0xFu) != 0) == 0) continue;
      const uint4 gq = stage_vec(stage, (2 * u) * 64 + lane);
      const uint4 rq = stage_vec(stage, (2 * u + 1) * 64 + lane);
      const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
      const uint32_t rw[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = u * 4 + e;
        const float g = __uint_as_float(gw[e]), r = __uint_as_float(rw[e]);
        const float ad = fabsf(g - r);
        const uint32_t ab = __float_as_uint(ad);
        // (a loaded vector; one sign and other bits: a nonzero difference)
        const bool lean = ((full >> u) & 1u) && (int32_t)(gw[e] ^ rw[e]) > 0 && ad < __builtin_inff();
        leanm |= (lean ? 1u : 0u) << p;
        if (lean) {
          const bool tol = ad <= fmaf(fabsf(g), lt.rtol, lt.atol);
          const bool below = ad < thr * fabsf(r);
          if (!(tol && below)) {
            // a mismatch or a rel-argmax candidate (slow_elem's tests, exactly)
            const float rel = ad / (fabsf(r) + 1e-12f);
            const uint32_t rk = fkey(rel);
            const uint32_t idx = R0 + (uint32_t)((u * 64 + lane) * V + e);
            if (!tol && (zt || !(ad <= d.atol + fabsf(d.rtol * g)))) {
              ++acc.nmm;
              acc.first_mm = idx < acc.first_mm ? idx : acc.first_mm;
              acc.mm_abs = fkey(ad) > acc.mm_abs ? fkey(ad) : acc.mm_abs;
              acc.mm_rel = rk > acc.mm_rel ? rk : acc.mm_rel;
            }
            if (!below && better32(rk, idx, acc.grel_k, acc.grel_i)) {
              acc.grel_k = rk;
              acc.grel_i = idx;
              const float t = rel_threshold(rel);
              thr = t > thr ? t : thr;
            }
          }
          if (ab > best) {
            best = ab;
            bslot = p;
          }
          // one sign: the ULP distance is the distance of the codes (nonzero here)
          const uint32_t lz = (uint32_t)__builtin_clz(abs_diff_u32(gw[e], rw[e]));
          atomicAdd((uint32_t*)(mine + (lz > 17u ? lz : 17u) * kRep), 1u);
          const double g64 = (double)g, r64 = (double)r;
          const double d64 = g64 - r64;
          acc.s[0] = fma(g64, g64, acc.s[0]);
          acc.s[1] = fma(r64, r64, acc.s[1]);
          acc.s[2] = fma(g64, r64, acc.s[2]);
          acc.s[3] = fma(d64, d64, acc.s[3]);
          if (capseg) {
            const bool hi = ad >= fmaf(crhi, fabsf(r), crhc);
            cm[0] |= (ab >= ca0 ? 1u : 0u) << p;
            cm[1] |= (hi ? 1u : 0u) << p;
            if (!hi && !(ad < crlo * fabsf(r)) && fkey(ad / (fabsf(r) + 1e-12f)) >= ck1) cm[1] |= 1u << p;
          }
        }
      }
    }
    acc.rel_thr = thr;
    if (bslot >= 0) {
      acc.gabs_k = best | kZeroKey;
      acc.gabs_i = R0 + (uint32_t)((((bslot >> 2) * 64 + lane) * V) + (bslot & 3));
    }
    const uint64_t rare = slow & ~(uint64_t)leanm;
    if (capseg) {
      // the captured values of the lean pairs, lane by lane in slot order, from
      // the stage, after the run's captures so far; the lean pairs not captured
      // are nonzero values below the threshold
      const uint32_t nl = (uint32_t)__popc(leanm);
      const uint32_t c0 = (uint32_t)__popc(cm[0]), c1 = (uint32_t)__popc(cm[1]);
      const uint32_t pk = c0 | (c1 << 16);  // (a wave adds at most 1024 to each half)
      const uint32_t incl = wave_incl_scan(pk);
      const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
      const uint32_t nb = wave_sum((nl - c0) | ((nl - c1) << 16));
      if (tot | nb) {
        const uint32_t base = wc[WC_CBASE], f0 = wc[WC_CFILL], f1 = wc[WC_CFILL + 1];
        const uint32_t ex = incl - pk;
        float* pa = d.cap_buf[0] + base + f0 + (ex & 0xFFFFu);
        float* pr = d.cap_buf[1] + base + f1 + (ex >> 16);
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          for (uint32_t mk = cm[x]; mk; mk &= mk - 1) {
            const int p = __builtin_ctz(mk), u = p >> 2, e = p & 3;
            const float g = stage_elem<float>(stage, (2 * u) * 64 + lane, e);
            const float r = stage_elem<float>(stage, (2 * u + 1) * 64 + lane, e);
            const float ad = fabsf(g - r);
            if (x == 0) *pa++ = ad; else *pr++ = ad / (fabsf(r) + 1e-12f);
          }
        }
        if (lane == 0) {
          wc[WC_CFILL] = f0 + (tot & 0xFFFFu);
          wc[WC_CFILL + 1] = f1 + (tot >> 16);
          wc[WC_BELOW] += nb & 0xFFFFu;
          wc[WC_BELOW + 1] += nb >> 16;
        }
      }
    }
    return rare;
  }
}

// Adds the wave's replicated ULP-bucket counters into its LDS counters and
// clears them (before the wave's counters are read for a record).
__device__ __forceinline__ void fold_rep(KVV_LDS uint32_t* rep, uint32_t* wc) {
  const int lane = lane_id();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // row i counts bucket 15 - i (phase_b_lean)
  if (lane < kBuckets - 1) {
    uint32_t t = 0;
#pragma unroll
    for (int c = 0; c < kRep; ++c) {
      t += rep[lane * kRep + c];
      rep[lane * kRep + c] = 0;
    }
    wc[LC_HIST0 + (kBuckets - 1) - lane] += t;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------ near-zero entries
// The near-zero elements (|ref| <= near_zero_abs) of a lane's vectors of 16-bit
// codes, found on the codes, as a mask in the slow-mask layout: bit dd of the
// low half and bit 16 + dd of the high half of dword dd = u * 4 + j, i.e.
// elements 2j and 2j + 1 of vector u.  pre[u] counts the near-zero elements of
// the item before vector u of this lane in row-major order (vectors u, then
// lanes, then elements); preA holds u = 0, 1 and preB u = 2, 3 as 16-bit
// halves.  total is the item's count (wave-uniform).
struct NearItem {
  uint32_t mask, preA, preB, total;
};

template <int DT>
__device__ __forceinline__ NearItem near_item(const SegDesc& d, StageP stage, int64_t L0, int64_t L1, uint32_t full) {
  static_assert(VecIO<DT>::V == 8 && kUnroll == 4, "16-bit codes, four vectors per lane");
  const int lane = lane_id();
  // per half: |code| <= nz_code exactly when bit 15 of (code - (nz_code + 1)) differs
  // from the sign bit (the 16-bit difference of two values below 0x8000 borrows
  // exactly when the magnitude is below t1; a set sign bit flips bit 15)
  const uint32_t t1 = (uint32_t)(d.nz_code + 1) & 0xFFFFu;
  const u16x2 t = {(uint16_t)t1, (uint16_t)t1};
  uint32_t mask = 0;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint4 rq = stage_vec(stage, (2 * u + 1) * 64 + lane);
    const uint32_t rw[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u16x2 diff = __builtin_bit_cast(u16x2, rw[j]) - t;
      // the flags at bits 0 and 16, then at bits u*4+j and 16+u*4+j
      const u16x2 f = (diff ^ __builtin_bit_cast(u16x2, rw[j])) >> (u16x2){15, 15};
      mask |= __builtin_bit_cast(uint32_t, f) << (u * 4 + j);
    }
  }
  // only the elements inside the item: a lane's full vectors are inside it; a
  // partial or absent vector keeps the elements before L1.  None when no
  // magnitude is near zero (nz_code < 0).
  uint32_t valid = 0xFFFFFFFFu;
  if (full != (1u << kUnroll) - 1) {
    valid = 0;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t left = L1 - (L0 + (int64_t)(u * 64 + lane) * 8);  // elements of vector u inside the item
      const uint32_t lo = left >= 7 ? 0xFu : (left > 0 ? (1u << ((left + 1) >> 1)) - 1u : 0u);  // elements 2j < left
      const uint32_t hi = left >= 8 ? 0xFu : (left > 1 ? (1u << (left >> 1)) - 1u : 0u);        // elements 2j + 1 < left
      valid |= ((full >> u) & 1u) ? 0x000F000Fu << (u * 4) : (lo << (u * 4)) | (hi << (16 + u * 4));
    }
  }
  mask &= d.nz_code < 0 ? 0u : valid;
  NearItem o;
  o.mask = mask;
  // counts per vector, two to a word, then one packed scan per word (each
  // 16-bit field stays below 64 * 8)
  const uint32_t c0 = __popc(mask & 0x000F000Fu), c1 = __popc(mask & 0x00F000F0u);
  const uint32_t c2 = __popc(mask & 0x0F000F00u), c3 = __popc(mask & 0xF000F000u);
  const uint32_t x = c0 | (c1 << 16), y = c2 | (c3 << 16);
  const uint32_t ix = wave_incl_scan(x), iy = wave_incl_scan(y);
  const uint32_t tx = (uint32_t)__builtin_amdgcn_readlane((int)ix, 63), ty = (uint32_t)__builtin_amdgcn_readlane((int)iy, 63);
  const uint32_t ex = ix - x, ey = iy - y;
  const uint32_t t0 = tx & 0xFFFFu, t1c = tx >> 16, t2 = ty & 0xFFFFu;
  const uint32_t p0 = ex & 0xFFFFu, p1 = t0 + (ex >> 16);
  const uint32_t p2 = t0 + t1c + (ey & 0xFFFFu), p3 = t0 + t1c + t2 + (ey >> 16);
  o.preA = p0 | (p1 << 16);
  o.preB = p2 | (p3 << 16);
  o.total = uniform(t0 + t1c + t2 + (ty >> 16));
  return o;
}

// Where a wave's near-zero entries go: its own stretch of `quota` entries.
// run_near counts the near-zero elements of the wave's run before the current
// item (an entry's rank is that plus its rank inside the item).
struct NearSink {
  uint2* ent;
  uint32_t quota, n, run_near;
  bool over;  // an entry did not fit: the wave's entries are not valid
};

// Appends (rank, v) for the lanes with p.
__device__ __forceinline__ void near_put(NearSink& s, bool p, uint32_t rank, float v) {
  const uint64_t b = __ballot(p);
  if (!b) return;
  const uint32_t k = (uint32_t)__popcll(b);
  if (s.over || s.n + k > s.quota) {
    s.over = true;
    return;
  }
  const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
  if (p) s.ent[s.n + below] = make_uint2(rank, __float_as_uint(v));
  s.n = uniform(s.n + k);
}

// The item's entries: each lane walks its own near-zero elements that are not
// bit-identical finite pairs (slow, or in a partial vector: only those can have
// a nonzero abs_diff) and records those whose abs_diff is nonzero (NaN
// included), with their rank in the item from its own prefix and mask.
template <int DT>
__device__ __forceinline__ void near_entries(const NearItem& ni, uint64_t slow, uint32_t full, StageP stage,
                                             NearSink& s) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int lane = lane_id();
  uint32_t part = 0;  // slots of the vectors that phase A left to vec_tail
  if (full != (1u << kUnroll) - 1) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (!((full >> u) & 1u)) part |= 0x000F000Fu << (u * 4);
  }
  uint32_t cand = ni.mask & ((uint32_t)slow | part);
  while (__ballot(cand != 0)) {
    const bool act = cand != 0;
    const int p = act ? __builtin_ctz(cand) : 0;
    cand &= cand - 1;
    const int dd = p & 15, u = dd >> 2, j = dd & 3, h = p >> 4;
    const T gc = stage_elem<T>(stage, (2 * u) * 64 + lane, 2 * j + h);
    const T rc = stage_elem<T>(stage, (2 * u + 1) * 64 + lane, 2 * j + h);
    const float adf = fabsf(E::f32(gc) - E::f32(rc));
    // near-zero elements of vector u before element 2j + h
    const uint32_t lo = (ni.mask >> (u * 4)) & 0xFu, hi = (ni.mask >> (16 + u * 4)) & 0xFu;
    const uint32_t below = (uint32_t)__popc(lo & ((1u << j) - 1u)) + (uint32_t)__popc(hi & ((1u << j) - 1u)) +
                           (h ? ((lo >> j) & 1u) : 0u);
    const uint32_t pre = ((u < 2 ? ni.preA : ni.preB) >> ((u & 1) * 16)) & 0xFFFFu;
    near_put(s, act && adf != 0.0f, s.run_near + pre + below, adf);
  }
}

// Strided-sample cursor: the next sample index i, its logical position idx =
// floor(i*(n-1)/(m-1)) and rem = i*(n-1) mod (m-1).  Kept identical in every
// wave of the block (wave-uniform), advanced item by item.
struct SampleCursor {
  uint64_t i, idx;
  uint32_t rem;
};

// Cursor at the first sample whose position is >= L0 (64-bit division, once per run).
__device__ __forceinline__ SampleCursor cursor_at(const SegDesc& d, int64_t L0) {
  SampleCursor c;
  if (d.n <= d.max_samples) {
    c.i = c.idx = (uint64_t)L0;
    c.rem = 0;
    return c;
  }
  const uint64_t num = (uint64_t)d.n - 1, den = (uint64_t)d.m - 1;
  c.i = ((uint64_t)L0 * den + num - 1) / num;  // ceil(L0 * den / num)
  const uint64_t p = c.i * num;
  c.idx = p / den;
  c.rem = (uint32_t)(p - c.idx * den);
  return c;
}

// abs_diff and rel_diff of one sampled pair.
template <int DT, int MODE>
__device__ __forceinline__ void sample_pair(const SegDesc& d, typename Elem<DT>::T gc, typename Elem<DT>::T rc,
                                            float& adf, float& rel) {
  float rf;
  uint32_t kk;
  bool mm;
  elem_test<DT, MODE>(gc, rc, d, adf, kk, mm, rf);
  // abs_diff == 0 leaves rel_diff == +0 (the denominator is then finite and positive)
  rel = adf == 0.0f ? 0.0f : adf / (fabsf(rf) + 1e-12f);
}

// abs_diff and rel_diff of one sampled pair; its values join the sampled fp64 sums.
template <int DT, int MODE>
__device__ __forceinline__ void sample_value(const SegDesc& d, typename Elem<DT>::T gc, typename Elem<DT>::T rc,
                                             Acc& acc, float& adf, float& rel) {
  using E = Elem<DT>;
  sample_pair<DT, MODE>(d, gc, rc, adf, rel);
  const double g64 = E::f64(gc), r64 = E::f64(rc);
  acc.s[4] = fma(g64, g64, acc.s[4]);
  acc.s[5] = fma(r64, r64, acc.s[5]);
  acc.s[6] = fma(g64, r64, acc.s[6]);
}

// A wave's buffer of samples in LDS: the consecutive sample positions
// [at0, at0 + fill).  It is written out (coalesced) when full, at the end of a
// segment and at the end of the wave's range.  Sample values written to HBM while the scan streams its
// inputs cost far more read bandwidth than their bytes, so a wave whose samples
// fit (SampleWords::cap) writes them all at the end.
struct SampleBuf {
  uint64_t at0;  // kNone: empty
  uint32_t fill;
};

// What the buffer keeps per sample position, in two 32-bit words: the raw codes
// of the pair for element types of at most 4 bytes (abs_diff, rel_diff and the
// sampled sums are computed when the buffer is written out, every lane busy),
// else the finished abs_diff and rel_diff.
template <int DT>
struct SampleWords {
  static constexpr bool codes = sizeof(typename Elem<DT>::T) <= 4;
  // codes of at most 16 bits share one word (generated code in the low half), so the
  // buffer's second word array is not needed
  static constexpr int W = Elem<DT>::width;
  static constexpr bool one = codes && W <= 16;
  static constexpr int words = one ? 1 : 2;
  // positions per wave: two word arrays take fewer, so that a block's LDS
  // (with its level-0 histograms) stays within three blocks per CU
  static constexpr int cap = one ? 384 : 320;
};

// Writes the buffered positions out (coalesced), finishing their values first
// when the buffer holds codes.  d is the segment the positions belong to.
// kFlagMainHist: a block's level-0 histograms of its abs/rel samples, two
// 16-bit counts per LDS word (256 bins per array), and their NaN counts.
struct MainHist {
  uint32_t* h;    // [2][128] in LDS
  uint32_t* nan;  // [2] in LDS
};

// Adds every active lane's value to array k's block histogram: one aggregated
// add when the wave's values share a bin (e.g. the zeros of identical pairs),
// else one LDS atomic per lane.  Called by every lane of the wave.
__device__ __forceinline__ void main_hist_add(const MainHist& mh, int k, float v, bool act) {
  const bool isn = v != v;
  const uint64_t nb = __ballot(act && isn);
  if (nb && lane_id() == 0) atomicAdd(&mh.nan[k], (uint32_t)__popcll(nb));
  const bool ok = act && !isn;
  const uint32_t bin = fkey(v) >> 24;
  const uint64_t m = __ballot(ok);
  if (!m) return;
  const int l0 = __ffsll((long long)m) - 1;
  const uint32_t b0 = (uint32_t)__builtin_amdgcn_readlane((int)bin, l0);
  const uint64_t same = __ballot(ok && bin == b0);
  uint32_t* h = mh.h + k * 128;
  if (same == m) {
    if (lane_id() == l0) atomicAdd(&h[b0 >> 1], (uint32_t)__popcll(m) << ((b0 & 1u) << 4));
  } else if (ok) {
    atomicAdd(&h[bin >> 1], 1u << ((bin & 1u) << 4));
  }
}

template <int DT, int MODE>
__device__ __forceinline__ void sbuf_store(const SegDesc& d, SampleBuf& b, KVV_LDS uint32_t* ba, KVV_LDS uint32_t* br,
                                           float* sabs, float* srel, Acc& acc, const MainHist& mh) {
  using T = typename Elem<DT>::T;
  if (b.at0 != kNone) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool hist = (d.flags & kFlagMainHist) != 0;
    for (uint32_t k0 = 0; k0 < b.fill; k0 += 64) {
      const uint32_t k = k0 + (uint32_t)lane_id();
      const bool act = k < b.fill;
      float adf = 0.0f, rel = 0.0f;
      if (act) {
        if constexpr (SampleWords<DT>::one) {
          const uint32_t wv = ba[k];
          sample_value<DT, MODE>(d, (T)wv, (T)(wv >> SampleWords<DT>::W), acc, adf, rel);
        } else if constexpr (SampleWords<DT>::codes) {
          sample_value<DT, MODE>(d, (T)ba[k], (T)br[k], acc, adf, rel);
        } else {
          adf = __uint_as_float(ba[k]);
          rel = __uint_as_float(br[k]);
        }
        sabs[b.at0 + k] = adf;
        srel[b.at0 + k] = rel;
      }
      if (hist) {
        main_hist_add(mh, 0, adf, act);
        main_hist_add(mh, 1, rel, act);
      }
    }
  }
  b.at0 = kNone;
  b.fill = 0;
}

// Adds c consecutive sample positions [at, at + c), held by lanes 0..c-1
// (c <= 64), as the two words w0, w1 of each.
template <int DT, int MODE>
__device__ __forceinline__ void sbuf_put(const SegDesc& d, SampleBuf& b, uint64_t at, int c, uint32_t w0,
                                         uint32_t w1, KVV_LDS uint32_t* ba, KVV_LDS uint32_t* br, float* sabs,
                                         float* srel, Acc& acc, const MainHist& mh) {
  if (b.at0 != kNone && (at != b.at0 + b.fill || b.fill + (uint32_t)c > (uint32_t)SampleWords<DT>::cap))
    sbuf_store<DT, MODE>(d, b, ba, br, sabs, srel, acc, mh);
  if (b.at0 == kNone) b.at0 = at;
  const int lane = lane_id();
  if (lane < c) {
    if constexpr (SampleWords<DT>::one) {
      ba[b.fill + lane] = w0 | (w1 << SampleWords<DT>::W);
    } else {
      ba[b.fill + lane] = w0;
      br[b.fill + lane] = w1;
    }
  }
  b.fill = uniform(b.fill + (uint32_t)c);
  b.at0 = uniform(b.at0);
}

// Code of element e of a 16-byte vector.
template <int DT>
__device__ __forceinline__ typename Elem<DT>::T vec_code(const uint4& q, int e) {
  using T = typename Elem<DT>::T;
  constexpr int W = Elem<DT>::width;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (W == 64) {
    return (T)(((uint64_t)w[2 * e + 1] << 32) | w[2 * e]);
  } else {
    return (T)(w[(e * W) >> 5] >> ((e * W) & 31));
  }
}

// Samples of a segment whose every element is a sample (n <= max_samples, so
// sample index == logical index): each lane finishes the values of its own
// vectors from the stage and stores them with vector stores, no walk.  The
// sampled sums take every element's fp64 products here (the full sums may
// take phase A's packed dot form, which is only accurate to 7.2e-7).
template <int DT, int MODE>
__device__ __forceinline__ void dense_samples(const SegDesc& d, int64_t L0, int64_t L1, StageP stage, Acc& acc,
                                              float* sabs, float* srel, const MainHist& mh) {
  using E = Elem<DT>;
  constexpr int V = VecIO<DT>::V;
  constexpr int S = V >= 4 ? 4 : V;  // floats per store
  typedef float fvec __attribute__((ext_vector_type(S)));
  const int lane = lane_id();
#pragma unroll 1
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v0 = L0 + (int64_t)(u * 64 + lane) * V;
    if (v0 >= L1) break;  // this lane's later vectors lie further out
    const uint4 gq = stage_vec(stage, (2 * u) * 64 + lane);
    const uint4 rq = stage_vec(stage, (2 * u + 1) * 64 + lane);
    float* pa = sabs + d.sample_off + v0;
    float* pr = srel + d.sample_off + v0;
    // S values at a time, so few registers are live beside the prefetched item
#pragma unroll
    for (int k = 0; k < V; k += S) {
      fvec xa, xr;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        float fa, fr;
        const auto gc = vec_code<DT>(gq, k + j), rc = vec_code<DT>(rq, k + j);
        sample_pair<DT, MODE>(d, gc, rc, fa, fr);
        xa[j] = fa;
        xr[j] = fr;
        if (v0 + k + j < L1) {
          if (d.flags & kFlagMainHist) {
            // one LDS atomic per value (this loop is per lane)
            const float vv[2] = {fa, fr};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              if (vv[q] != vv[q]) {
                atomicAdd(&mh.nan[q], 1u);
              } else {
                const uint32_t bin = fkey(vv[q]) >> 24;
                atomicAdd(&mh.h[q * 128 + (bin >> 1)], 1u << ((bin & 1u) << 4));
              }
            }
          }
          const double g64 = E::f64(gc), r64 = E::f64(rc);
          acc.s[4] = fma(g64, g64, acc.s[4]);
          acc.s[5] = fma(r64, r64, acc.s[5]);
          acc.s[6] = fma(g64, r64, acc.s[6]);
        }
      }
      if (v0 + k + S <= L1) {
        *reinterpret_cast<fvec*>(pa + k) = xa;
        *reinterpret_cast<fvec*>(pr + k) = xr;
      } else {
#pragma unroll
        for (int j = 0; j < S; ++j) {
          if (v0 + k + j < L1) {
            pa[k + j] = xa[j];
            pr[k + j] = xr[j];
          }
        }
      }
    }
  }
}

// Samples of a vector item (GCR:346-347): the wave walks its cursor 64 samples
// per step (lane l takes sample cursor.i + l); every sample of the item lies in
// the wave's own stage slots.  Positions inside the item are 32-bit offsets
// from L0.  The values go through the wave's line buffer.  When n <=
// max_samples every element is a sample (the host sets the stride to 1).
template <int DT, int MODE>
__device__ __forceinline__ void sample_item(const SegDesc& d, int64_t L0, int64_t L1, StageP stage, Acc& acc,
                                            float* sabs, float* srel, SampleCursor& cur, SampleBuf& sb,
                                            KVV_LDS uint32_t* ba, KVV_LDS uint32_t* br, const MainHist& mh) {
  using IO = VecIO<DT>;
  using T = typename IO::T;
  constexpr int V = IO::V;
  constexpr int LV = V == 16 ? 4 : (V == 8 ? 3 : (V == 4 ? 2 : 1));  // log2(V)
  const int lane = lane_id();
  const uint32_t den = (uint32_t)(d.m - 1);
  const uint32_t len = (uint32_t)(L1 - L0);
  // lane * s_div only matters while it stays inside the item; clamping keeps the
  // 32-bit offsets exact for the lanes that can be in range
  const uint32_t sdiv = d.s_div < (1ull << 20) ? (uint32_t)d.s_div : (1u << 20);
  const uint32_t smod = (uint32_t)d.s_mod;
  for (;;) {
    if (cur.i >= (uint64_t)d.m || cur.idx >= (uint64_t)L1) return;
    const uint64_t left = (uint64_t)d.m - cur.i;
    const uint32_t t = cur.rem + (uint32_t)lane * smod;  // < 64 * den < 2^30
    const uint32_t q = __umulhi(t, d.s_magic) >> d.s_shift;
    const uint32_t rem = t - q * den;
    const uint32_t off = (uint32_t)(cur.idx - (uint64_t)L0) + (uint32_t)lane * sdiv + q;
    const bool in = (uint64_t)lane < left && off < len;
    // the in-range lanes are a prefix; the cursor moves past the last of them
    const int c = (int)__popcll(__ballot(in));
    if (c == 0) return;
    uint32_t w0 = 0, w1 = 0;
    if (in) {
      const uint32_t vi = off >> LV;
      const int u = (int)(vi >> 6), tt = (int)(vi & 63u), e = (int)(off & (V - 1));
      const T gc = stage_elem<T>(stage, (2 * u) * 64 + tt, e);
      const T rc = stage_elem<T>(stage, (2 * u + 1) * 64 + tt, e);
      if constexpr (SampleWords<DT>::codes) {
        w0 = (uint32_t)gc;
        w1 = (uint32_t)rc;
      } else {
        float adf, rel;
        sample_value<DT, MODE>(d, gc, rc, acc, adf, rel);
        w0 = __float_as_uint(adf);
        w1 = __float_as_uint(rel);
      }
    }
    sbuf_put<DT, MODE>(d, sb, d.sample_off + cur.i, c, w0, w1, ba, br, sabs, srel, acc, mh);
    const uint32_t offl = (uint32_t)__builtin_amdgcn_readlane((int)off, c - 1);
    uint32_t nr = (uint32_t)__builtin_amdgcn_readlane((int)rem, c - 1) + smod;
    uint64_t nidx = (uint64_t)L0 + offl + d.s_div;
    if (nr >= den) {
      nr -= den;
      nidx += 1;
    }
    cur.i = uniform(cur.i + (uint64_t)c);
    cur.idx = uniform(nidx);
    cur.rem = uniform(nr);
    if (c < 64) return;
  }
}

// Elements of a partial last vector (numel not a multiple of the vector width),
// from the stage.
template <int DT, int MODE>
__device__ __forceinline__ void vec_tail(const SegDesc& d, int64_t L0, int64_t L1, uint32_t R0, uint32_t full,
                                         StageP stage, Acc& acc, uint32_t* wc) {
  using T = typename Elem<DT>::T;
  constexpr int V = VecIO<DT>::V;
  const int lane = lane_id();
#pragma unroll 1
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = L0 + (int64_t)(u * 64 + lane) * V;
    const bool part = !((full >> u) & 1u) && v < L1;
    if (__ballot(part) == 0) continue;
    for (int e = 0; e < V; ++e) {
      const bool act = part && v + e < L1;
      const T gc = stage_elem<T>(stage, (2 * u) * 64 + lane, e);
      const T rc = stage_elem<T>(stage, (2 * u + 1) * 64 + lane, e);
      slow_elem<DT, MODE>(gc, rc, act, R0 + (uint32_t)((u * 64 + lane) * V + e), d, acc, wc);
    }
  }
}

// Scalar path: any strides, one element per thread per step.
template <int DT, int MODE>
__device__ __forceinline__ void scan_item_scalar(const SegDesc& d, int64_t L0, int64_t L1, int64_t base, Acc& acc,
                                                 uint32_t* wc) {
  for (int64_t at = L0; at < L1; at += 64) {
    const int64_t idx = at + lane_id();
    const bool act = idx < L1;
    int64_t og = 0, orr = 0;
    if (act) elem_offsets(d, idx, og, orr);
    const auto gc = act ? load_elem<DT>(d.g, og) : (typename Elem<DT>::T)0;
    const auto rc = act ? load_elem<DT>(d.r, orr) : (typename Elem<DT>::T)0;
    slow_elem<DT, MODE>(gc, rc, act, (uint32_t)(idx - base), d, acc, wc);
  }
}

// ------------------------------------------------------------ run records
// Run slot of the run that starts at item `it` of segment d, in batch wave
// range k: runs start at the segment's first item and at every wave range
// that starts inside it (the launch's ranges are nonempty until its items end).
__device__ __forceinline__ int64_t run_slot(const SegDesc& d, int64_t it, int64_t k) {
  return it == d.item_begin ? d.run_slot0 : d.run_slot0 + 1 + (k - d.run_k0);
}

// Reduces the wave's accumulators and LDS counters into the run's columns (lane
// c writes u32 column c, lane 32 + c u64 column c) and resets them for the next
// run.  `base` is the logical index of the run's first element (the origin of
// the accumulators' 32-bit offsets).
static_assert(kColU32 == 32 && kColU64 <= 32, "one lane per run column");
// Where a run record goes: the run columns in global memory, or (a wave's part
// of a block record) an LDS record of kColU32 + kColU64 words.
struct ColSink {
  const RunCols* out;
  int64_t slot;
  __device__ void put32(int c, uint32_t v) const { out->u32[c * out->stride + slot] = v; }
  __device__ void put64(int c, uint64_t v) const { out->u64[c * out->stride + slot] = v; }
};
struct LdsRecord {
  KVV_LDS uint32_t* u32;
  KVV_LDS uint64_t* u64;
  __device__ void put32(int c, uint32_t v) const { u32[c] = v; }
  __device__ void put64(int c, uint64_t v) const { u64[c] = v; }
};
template <class Sink>
__device__ inline void flush_run(Acc& acc, uint32_t* wc, const Sink& out, int64_t base) {
  const int lane = lane_id();
  const uint32_t nfast = wave_sum(acc.nfast);
  const uint32_t nmm = wave_sum(acc.nmm);
  const uint32_t nnear = wave_sum(acc.nnear_fast);
  const uint32_t fmm32 = wave_min(acc.first_mm), fvi32 = wave_min(acc.first_viol);
  const uint32_t mma = wave_max(acc.mm_abs), mmr = wave_max(acc.mm_rel);
  // bit-identical pairs have abs_diff = rel_diff = +0, whose key is 0x80000000 in both modes
  uint32_t gak = acc.gabs_k, grk = acc.grel_k;
  uint32_t gai32 = acc.gabs_i, gri32 = acc.grel_i;
  if (better32(0x80000000u, acc.first_fast, gak, gai32)) {
    gak = 0x80000000u;
    gai32 = acc.first_fast;
  }
  if (better32(0x80000000u, acc.first_fast, grk, gri32)) {
    grk = 0x80000000u;
    gri32 = acc.first_fast;
  }
  wave_argmax32(gak, gai32);
  wave_argmax32(grk, gri32);
  auto absolute = [base](uint32_t r) -> uint64_t { return r == kNone32 ? kNone : (uint64_t)(base + (int64_t)r); };
  double sm[7];
  sm[0] = wave_sum(acc.e_sq + acc.s[0]);
  sm[1] = wave_sum(acc.e_sq + acc.s[1]);
  sm[2] = wave_sum(acc.e_sq + acc.s[2]);
#pragma unroll
  for (int i = 3; i < 7; ++i) sm[i] = wave_sum(acc.s[i]);
  if (lane < kColU32) {
    uint32_t v;
    if (lane < LC_COUNT) {
      v = wc[lane] + (lane == LC_HIST0 ? nfast : 0u) + (lane == LC_NEAR ? nnear : 0u);
      wc[lane] = 0;
    } else {
      v = lane == CU_MISM ? nmm : lane == CU_MMABS ? mma : lane == CU_MMREL ? mmr : lane == CU_GABSK ? gak : grk;
    }
    out.put32(lane, v);
  } else if (lane < 32 + kColU64) {
    const int c = lane - 32;
    uint64_t v;
    if (c == CL_FIRSTMM) v = absolute(fmm32);
    else if (c == CL_FIRSTVIOL) v = absolute(fvi32);
    else if (c == CL_GABSI) v = absolute(gai32);
    else if (c == CL_GRELI) v = absolute(gri32);
    else {
      double x = sm[0];
#pragma unroll
      for (int i = 1; i < 7; ++i) x = (c - CL_S0 == i) ? sm[i] : x;
      v = (uint64_t)__double_as_longlong(x);
    }
    out.put64(c, v);
  }
  acc.init();
}

// The last wave of a block to finish folds the block's kWaves wave records
// (LDS, waves in order, so fp64 sums are reproducible) into one run record.
__device__ inline void fold_block_record(const LdsRecord* rec, const RunCols& out, int64_t slot) {
  const int lane = lane_id();
  if (lane < kColU32) {
    if (lane == CU_GABSK || lane == CU_GRELK) {
      const int ci = lane == CU_GABSK ? CL_GABSI : CL_GRELI;
      uint32_t bk = rec[0].u32[lane];
      uint64_t bi = rec[0].u64[ci];
      for (int w = 1; w < kWaves; ++w) {
        const uint32_t k = rec[w].u32[lane];
        const uint64_t i = rec[w].u64[ci];
        if (better(k, i, bk, bi)) {
          bk = k;
          bi = i;
        }
      }
      out.u32[lane * out.stride + slot] = bk;
      out.u64[ci * out.stride + slot] = bi;
    } else {
      const bool mx = lane == CU_MMABS || lane == CU_MMREL;
      uint32_t v = rec[0].u32[lane];
      for (int w = 1; w < kWaves; ++w) {
        const uint32_t x = rec[w].u32[lane];
        v = mx ? (x > v ? x : v) : v + x;
      }
      out.u32[lane * out.stride + slot] = v;
    }
  } else if (lane < 32 + kColU64) {
    const int c = lane - 32;
    if (c == CL_GABSI || c == CL_GRELI) return;  // written with their keys
    if (c == CL_FIRSTMM || c == CL_FIRSTVIOL) {
      uint64_t v = rec[0].u64[c];
      for (int w = 1; w < kWaves; ++w) v = rec[w].u64[c] < v ? rec[w].u64[c] : v;
      out.u64[c * out.stride + slot] = v;
    } else {
      double v = __longlong_as_double((long long)rec[0].u64[c]);
      for (int w = 1; w < kWaves; ++w) v += __longlong_as_double((long long)rec[w].u64[c]);
      out.u64[c * out.stride + slot] = (uint64_t)__double_as_longlong(v);
    }
  }
}

// ------------------------------------------------------------ scan kernel
// LDS of one scan block: per wave, its item's vectors (SW uint4: kUnroll
// vectors of each tensor per lane), its queue of stage positions (NQ entries:
// 64 lanes x the dtype's queue slots), its replicated ULP-bucket counters (RW
// words), its sample buffer (SBW words for each of its consecutive sample
// positions) and its counters.  Waves never touch each other's part.
template <int SW, int NQ, int RW, int SBW>
struct ScanShared {
  uint32_t done;  // waves of the block that have left their record (single-segment launches)
  uint4 stage[kWaves][SW];
  uint16_t queue[kWaves][NQ];
  uint32_t rep[kWaves][RW];
  uint32_t sbuf[kWaves][SBW][SBW == 1 ? 384 : 320];
  uint32_t wcnt[kWaves][WC_COUNT];
  // kFlagMainHist: the block's level-0 histograms (2 x 128 words) and NaN counts (2)
  uint32_t hist0[2 * 128 + 2];
};

template <int DT, int KIND>
struct ScanLds {
  static constexpr bool vec = KIND != K_SCALAR;
  using QG = QueueGeom<DT>;
  // (the scalar kind stages nothing, but its waves leave their run records there)
  using type = ScanShared<vec ? 2 * kUnroll * 64 : (kColU32 * 4 + kColU64 * 8 + 15) / 16, vec ? 64 * QG::slots : 2,
                          vec ? QG::rep_words : 1, SampleWords<DT>::words>;
};

// Per-item near-zero count of the wave (feeds the compacted-rank prefix of near_kernel).
__device__ __forceinline__ void near_item_count(const ScanArgs& a, int64_t item, Acc& acc, const uint32_t* wc,
                                                uint32_t& near_prev) {
  uint32_t mine = acc.nnear_fast;
  if (lane_id() == 0) mine += wc[LC_NEAR];
  const uint32_t now = wave_sum(mine);
  if (lane_id() == 0) a.item_near[item] = now - near_prev;
  near_prev = now;
}

// Phase A variant by wave-uniform conditions (near-zero counting; the quick or
// careful dot form), then the lowest bit-identical index while it can still be
// an argmax.  `careful` counts the items left in the careful form.
template <int DT>
__device__ __forceinline__ uint64_t phase_a_any(const SegDesc& d, int64_t L0, uint32_t R0, StageP stage,
                                                uint32_t full, Acc& acc, uint32_t& careful) {
  if (!d.fast) {
    // no element can take the fast path: all elements of the full vectors are slow
    uint64_t all = 0;
    for (int p = 0; p < VecIO<DT>::NE; ++p) {
      int u, e;
      slot_of<Elem<DT>::width>(p, u, e);
      if ((full >> u) & 1u) all |= 1ull << p;
    }
    return all;
  }
  const bool track =
      __ballot(acc.first_fast == kNone32 && (acc.gabs_k <= 0x80000000u || acc.grel_k <= 0x80000000u)) != 0;
  PhaseA o;
  if (d.flags & KVV_FLAG_NEAR_ZERO) {
    o = phase_a<DT, true>(d, stage, full);
  } else if constexpr (DotForm<DT>::on) {
    bool redone = false;
    if (d.flags & kFlagCaptureElems) {
      // the sampled sums of such a segment are its full sums: exact squares
      o = phase_a<DT, false>(d, stage, full);
    } else if (__ballot(full != (1u << kUnroll) - 1) != 0) {
      // a partial last vector (its elements are left to vec_tail): per-vector form
      o = phase_a<DT, false>(d, stage, full);
    } else if (careful) {
      --careful;
      o = phase_a_dot<DT, true>(d, stage, full, redone);
    } else {
      o = phase_a_dot<DT, false>(d, stage, full, redone);
      if (redone) careful = 8;
    }
  } else {
    o = phase_a<DT, false>(d, stage, full);
  }
  acc.e_sq += o.esq;
  acc.nfast += o.nfast;
  acc.nnear_fast += o.nnear;
  const uint64_t slow = o.slow;
  if (track) track_first_fast<DT>(R0, full, slow, acc);
  return slow;
}

// A wave of a single-segment launch leaves its run record in its own stage
// region (its items are done) and checks in; the last wave of the block folds
// the block's records into the block's run slot (runs are per block there).
template <class SM>
__device__ inline void block_record_part(const ScanArgs& a, SM& sm, Acc& acc, uint32_t* wc, int w, int64_t base) {
  auto rec_of = [&sm](int x) {
    KVV_LDS uint64_t* r = (KVV_LDS uint64_t*)(KVV_LDS uint4*)sm.stage[x];
    return LdsRecord{(KVV_LDS uint32_t*)(r + kColU64), r};
  };
  flush_run(acc, wc, rec_of(w), base);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  uint32_t old = 0;
  if (lane_id() == 0) old = atomicAdd(&sm.done, 1u);
  old = uniform(old);
  if (old != kWaves - 1) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  LdsRecord rec[kWaves];
  for (int x = 0; x < kWaves; ++x) rec[x] = rec_of(x);
  fold_block_record(rec, a.runs, blockIdx.x);
  if (a.slots) {
    // kFlagMainHist: the block's level-0 histograms and NaN counts join the group's
    const int lane = lane_id();
    const uint32_t* hb = &sm.hist0[0];
    for (int i = lane; i < 256; i += 64) {
      const uint32_t wv = hb[i];
      uint32_t* dst = a.slots + (size_t)(i >> 7) * kSlotWords + kH0R + (blockIdx.x % kH0Copies) * 256 + 2 * (i & 127);
      if (wv & 0xFFFFu) atomicAdd(dst, wv & 0xFFFFu);
      if (wv >> 16) atomicAdd(dst + 1, wv >> 16);
    }
    if (lane < 2 && hb[256 + lane]) atomicAdd(a.slots + (size_t)lane * kSlotWords + kMisc, hb[256 + lane]);
  }
}

// NZ: a single fp16/bf16 pair whose near-zero diagnostics are taken as entries
// (kFlagNearEntries); the vector kinds with the dtype's isclose test only.
template <int DT, int MODE, int KIND, bool BATCH, bool NZ = false>
__global__ __launch_bounds__(kBlock, BATCH ? 3 : 1) void scan_kernel(ScanArgs a) {
  static_assert(!NZ || (!BATCH && KIND != K_SCALAR && MODE == KVV_MODE_ISCLOSE && Elem<DT>::width == 16 &&
                        Elem<DT>::is_float), "near-zero entries: single fp16/bf16 pairs, vector kinds");
  __shared__ typename ScanLds<DT, KIND>::type sm;
  // the wave index, and all that derives from it (item range, segment, run), is
  // wave-uniform: segment fields are then read with scalar loads, which the
  // item loop's waits on the prefetched vector loads do not cover
  const int tid = threadIdx.x, w = (int)uniform((uint32_t)(tid >> 6)), lane = tid & 63;
  uint32_t* wc = sm.wcnt[w];
  if (lane < WC_COUNT) wc[lane] = 0;
  // the dense path's replicated ULP-bucket counters (fp32 isclose, vector kinds)
  constexpr bool kLean = DT == KVV_F32 && MODE == KVV_MODE_ISCLOSE && KIND != K_SCALAR;
  KVV_LDS uint32_t* const rep = (KVV_LDS uint32_t*)sm.rep[w];
  if constexpr (kLean) {
    for (int i = lane; i < kBuckets * kRep; i += 64) rep[i] = 0;
  }
  if constexpr (!BATCH) {
    if (tid == 0) sm.done = 0;
  }
  uint32_t* const hist_base = &sm.hist0[0];
  const MainHist mh{hist_base, hist_base + 256};
  if constexpr (!BATCH) {
    if (a.slots)
      for (int i = tid; i < 258; i += kBlock) hist_base[i] = 0;
    __syncthreads();
  }
  // the select histograms and counters of this call (and a near-zero sample
  // built from entries) start at zero: the later launches accumulate into
  // them, and nothing in this kernel touches them
  auto clear = [&](uint4* p, int64_t n4) {
    const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
    const int64_t z0 = (int64_t)blockIdx.x * per;
    const int64_t z1 = z0 + per < n4 ? z0 + per : n4;
    for (int64_t i = z0 + tid; i < z1; i += kBlock) p[i] = make_uint4(0, 0, 0, 0);
  };
  if (a.zero_n4) clear(a.zero_ptr, a.zero_n4);
  if (a.zero2_n4) clear(a.zero2_ptr, a.zero2_n4);
  // each wave owns a contiguous range of items; the waves of a block never wait
  // for each other
  int64_t i0, i1;
  if (BATCH) {
    // the host's wave ranges (shares weighted by item cost and dispatch round)
    const int64_t k = (int64_t)blockIdx.x * kWaves + w;
    i0 = a.item_lo + a.starts[k];
    i1 = a.item_lo + a.starts[k + 1];
  } else if (a.rounds > 1) {
    // the grid is dispatched one block per CU at a time, and earlier rounds'
    // waves are served faster: each round's waves get a share of the items in
    // proportion to its rate
    int r = (int)(blockIdx.x / (uint32_t)a.round_blocks);
    r = r < a.rounds - 1 ? r : a.rounds - 1;
    const int64_t q = ((int64_t)blockIdx.x - (int64_t)r * a.round_blocks) * kWaves + w;
    i0 = a.item_lo + a.round_first[r] + q * a.round_ipw[r];
    i1 = i0 + a.round_ipw[r];
    const int64_t r1 = a.item_lo + a.round_first[r + 1];
    if (i0 > r1) i0 = r1;
    if (i1 > r1) i1 = r1;
  } else {
    i0 = a.item_lo + ((int64_t)blockIdx.x * kWaves + w) * a.items_per_wave;
    i1 = i0 + a.items_per_wave;
    if (i1 > a.item_lo + a.items) i1 = a.item_lo + a.items;
  }
  Acc acc;
  acc.init();
  const uint32_t wave_id = blockIdx.x * kWaves + (uint32_t)w;  // wave ranges ascend with it
  NearSink sink;
  if constexpr (NZ) {
    sink.ent = a.ent + (size_t)wave_id * a.ent_quota;
    sink.quota = a.ent_quota;
    sink.n = 0;
    sink.run_near = 0;
    sink.over = false;
  }
  if (i0 >= i1) {
    if constexpr (NZ) {
      if (lane == 0) {
        a.near_wave[wave_id] = 0;
        a.ent_fill[wave_id] = 0;
        a.wave_range[wave_id] = make_uint2(0u, 0u);
      }
    }
    // a single-segment launch folds one record per block: an empty wave still
    // leaves its (empty) part
    if constexpr (!BATCH) block_record_part(a, sm, acc, wc, w, a.seg0.item_begin);
    return;
  }
  int s = 0;
  if constexpr (BATCH) {
    int lo = 0, hi = a.nseg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.table[mid].item_begin <= i0) lo = mid; else hi = mid - 1;
    }
    s = (int)uniform((uint32_t)lo);
  }
  // the segment table through the constant address space: with a uniform index
  // its fields are scalar loads
  typedef const __attribute__((address_space(4))) SegDesc CSegDesc;
  const CSegDesc* ctable = (const CSegDesc*)a.table;
  uint32_t careful = 0;
  SampleBuf sb;
  sb.at0 = kNone;
  sb.fill = 0;
  KVV_LDS uint32_t* ba = (KVV_LDS uint32_t*)sm.sbuf[w][0];
  KVV_LDS uint32_t* br = (KVV_LDS uint32_t*)sm.sbuf[w][SampleWords<DT>::words - 1];
  // one pass per run of items of one segment (a single-segment launch has one);
  // the prefetched registers are dead between runs, where the record is written
  for (int64_t it = i0;;) {
    const SegDesc& d = BATCH ? *(const SegDesc*)&ctable[s] : a.seg0;
    const int64_t run_start = it;
    const int64_t seg_end = d.item_begin + d.item_count;
    const int64_t run_end = i1 < seg_end ? i1 : seg_end;
    const int64_t base = (run_start - d.item_begin) * (int64_t)d.item_elems;  // the run's first element
    const bool dense = d.m == d.n;
    SampleCursor cur = cursor_at(d, base);
    // the run's first element, where its captures start (such a segment has at most 2^24 elements)
    if ((d.flags & kFlagCaptureElems) && lane == 0) wc[WC_CBASE] = (uint32_t)base;
    uint32_t near_prev = 0;
    uint4 gv[kUnroll], rv[kUnroll];
    uint32_t full = 0;
    RowCursor rcur = row_cursor_at(d, run_start - d.item_begin);
    if constexpr (KIND != K_SCALAR) {
      const int64_t L1 = base + d.item_elems < d.n ? base + d.item_elems : d.n;
      full = load_item<DT, KIND>(d, base, L1, gv, rv, &rcur);
    }
    for (; it < run_end; ++it) {
      const int64_t L0 = (it - d.item_begin) * (int64_t)d.item_elems;
      const int64_t L1 = L0 + d.item_elems < d.n ? L0 + d.item_elems : d.n;
      const uint32_t R0 = (uint32_t)(L0 - base);
      if constexpr (KIND == K_SCALAR) {
        scan_item_scalar<DT, MODE>(d, L0, L1, base, acc, wc);
        sample_range<DT, MODE>(d, L0, L1, acc, a.sample_abs, a.sample_rel);
      } else {
        if (full != (1u << kUnroll) - 1) patch_partial<DT, KIND>(d, L0, L1, full, gv, rv);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          sm.stage[w][(2 * u) * 64 + lane] = gv[u];
          sm.stage[w][(2 * u + 1) * 64 + lane] = rv[u];
        }
        const uint32_t full_now = full;
        StageP stage = (StageP)sm.stage[w];
        // the next item of the run: its loads fly while this one finishes
        if (it + 1 < run_end) {
          const int64_t N1 = L1 + d.item_elems < d.n ? L1 + d.item_elems : d.n;
          full = load_item<DT, KIND>(d, L1, N1, gv, rv, &rcur);
        }
        // (an input-select segment's samples and sampled sums come from the input-select kernels)
        if (!dense && !(d.flags & kFlagInputSelect))
          sample_item<DT, MODE>(d, L0, L1, stage, acc, a.sample_abs, a.sample_rel, cur, sb, ba, br, mh);
        NearItem ni{};
        if constexpr (NZ) ni = near_item<DT>(d, stage, L0, L1, full_now);
        const uint64_t slow = phase_a_any<DT>(d, L0, R0, stage, full_now, acc, careful);
        if constexpr (NZ) near_entries<DT>(ni, slow, full_now, stage, sink);
        // what is left for the queue after an in-place pass over an item of mostly slow pairs
        uint64_t left = slow;
        if (__ballot(slow != 0)) {
          if (kLean && !(d.flags & kFlagNearAny)) left = phase_b_lean<DT, MODE>(d, R0, slow, full_now, stage, acc, rep, wc);
          else if (phase_b_dense<DT, MODE>(d, R0, slow, stage, acc, wc)) left = 0;
        }
        if (__ballot(left != 0)) {
          constexpr int QS = QueueGeom<DT>::slots;
          uint32_t nq = queue_all<QS>(left, sm.queue[w]);
          // more than the queue holds: QS slots of every lane at a time
          const bool split = nq > 64u * QS;
#pragma unroll 1
          for (int p0 = 0;; p0 += QS) {
            if (split) nq = queue_part<QS>((uint32_t)(left >> p0), p0, sm.queue[w]);
            if (nq) phase_b<DT, MODE>(d, R0, nq, stage, sm.queue[w], acc, wc);
            if (!split || p0 + QS >= VecIO<DT>::NE) break;
          }
        }
        // (every lane enters: slow_elem's wave-wide steps then see the whole wave)
        if (__ballot(full_now != (1u << kUnroll) - 1)) vec_tail<DT, MODE>(d, L0, L1, R0, full_now, stage, acc, wc);
        if constexpr (NZ) {
          // every near-zero element of the item joins the run's count
          if (lane == 0) acc.nnear_fast += ni.total;
          sink.run_near = uniform(sink.run_near + ni.total);
        }
        if (dense && !(d.flags & kFlagInputSelect))
          dense_samples<DT, MODE>(d, L0, L1, stage, acc, a.sample_abs, a.sample_rel, mh);
      }
      if (d.flags & KVV_FLAG_NEAR_ZERO) near_item_count(a, it, acc, wc, near_prev);
    }
    // the run's buffered samples join its record
    if constexpr (KIND != K_SCALAR) sbuf_store<DT, MODE>(d, sb, ba, br, a.sample_abs, a.sample_rel, acc, mh);
    if constexpr (kLean) fold_rep(rep, wc);
    if (BATCH && (d.flags & kFlagCaptureElems)) {
      // the run's record (its first element and captured counts) and its values below the thresholds
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t f0 = wc[WC_CFILL], f1 = wc[WC_CFILL + 1];
      if (lane < 2) {
        const uint32_t b = wc[WC_BELOW + lane];
        if (b) atomicAdd(d.cap_state + IS_BELOW + lane, b);
      }
      if (lane == 0) a.cap_runs[run_slot(d, run_start, wave_id)] = make_uint4(wc[WC_CBASE], f0, f1, 0u);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (lane < 4) wc[WC_BELOW + lane] = 0;
    }
    if constexpr (BATCH) {
      flush_run(acc, wc, ColSink{&a.runs, run_slot(d, run_start, wave_id)}, base);
      if (it >= i1) break;
      while (it >= ctable[s].item_begin + ctable[s].item_count) ++s;
      s = (int)uniform((uint32_t)s);
    } else {
      if constexpr (NZ) {
        if (lane == 0) {
          a.near_wave[wave_id] = sink.run_near;
          a.ent_fill[wave_id] = sink.over ? kNone32 : sink.n;
          a.wave_range[wave_id] = make_uint2((uint32_t)(i0 - a.item_lo), (uint32_t)(i1 - a.item_lo));
        }
      }
      block_record_part(a, sm, acc, wc, w, base);
      break;
    }
  }
}

// ------------------------------------------------------------ run records
__device__ __forceinline__ double clamp_cos(double c) {
  if (c != c) return c;
  return c < -1.0 ? -1.0 : (c > 1.0 ? 1.0 : c);
}

// GCR:364-371 zero conventions.
__device__ __forceinline__ double cosine_of(double gr, double gg, double rr) {
  const double gn = sqrt(gg), rn = sqrt(rr);
  if (gn == 0.0 && rn == 0.0) return 1.0;
  if (gn == 0.0 || rn == 0.0) return 0.0;
  return clamp_cos(gr / (gn * rn));
}

// ------------------------------------------------------------ near-zero sample
// GCR:525-529 compacts abs_diff over |ref| <= near_zero_abs in row-major order
// and samples that compacted array with the same i*(c-1)//(m-1) stride.  Each
// block re-reads one item; thread t owns a contiguous slice so that a block
// prefix sum gives every near-zero element its global compacted rank.
struct NearArgs {
  SegDesc seg0;
  const SegDesc* table;
  int32_t nseg;
  int32_t seg_lo;          // absolute index of table[0] (near_cm is indexed by absolute segment)
  const uint64_t* near_cm; // near-zero count and sample count per segment, from the fold
  int64_t item_lo, items;
  const kvv_result* res;
  const uint64_t* item_near_off;
  const uint32_t* item_near;
  float* near_sample;
  double* item_near_sum;   // sum of the sampled values of each item
};

template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void near_kernel(NearArgs a) {
  __shared__ uint32_t scan[kBlock];
  __shared__ double dsum[kWaves];
  const int64_t item = a.item_lo + blockIdx.x;
  int s = 0;
  if (a.table) {
    int lo = 0, hi = a.nseg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.table[mid].item_begin <= item) lo = mid; else hi = mid - 1;
    }
    s = lo;
  }
  const SegDesc& d = a.table ? a.table[s] : a.seg0;
  const int tid = threadIdx.x;
  if (!(d.flags & KVV_FLAG_NEAR_ZERO)) return;
  const uint32_t cnt = a.item_near[item];
  if (cnt == 0) {
    if (tid == 0) a.item_near_sum[item] = 0.0;
    return;
  }
  const uint64_t c = a.near_cm[2 * (a.seg_lo + s)];
  const uint64_t mm = a.near_cm[2 * (a.seg_lo + s) + 1];
  const uint64_t off = a.item_near_off[item];
  const int64_t L0 = (item - d.item_begin) * (int64_t)d.item_elems;
  const int64_t L1 = L0 + d.item_elems < d.n ? L0 + d.item_elems : d.n;
  const int64_t per = (d.item_elems + kBlock - 1) / kBlock;
  const int64_t e0 = L0 + tid * per < L1 ? L0 + tid * per : L1;
  const int64_t e1 = e0 + per < L1 ? e0 + per : L1;
  // pass 1: count this thread's near-zero elements
  uint32_t mine = 0;
  for (int64_t idx = e0; idx < e1; ++idx) {
    int64_t og, orr;
    elem_offsets(d, idx, og, orr);
    mine += fabsf(Elem<DT>::f32(load_elem<DT>(d.r, orr))) <= d.nz_abs;
  }
  // exclusive block scan (Hillis-Steele in LDS; one item per block)
  scan[tid] = mine;
  __syncthreads();
  for (int o = 1; o < kBlock; o <<= 1) {
    const uint32_t v = tid >= o ? scan[tid - o] : 0u;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  uint64_t rank = off + scan[tid] - mine;
  // rank j is sampled iff j == floor(i*(c-1)/(mm-1)) for some i
  const bool all = c <= mm;
  uint64_t i_next = 0, j_next = 0;
  if (!all) {
    const uint64_t num = c - 1, den = mm - 1;
    i_next = (rank * den + num - 1) / num;
    j_next = i_next < mm ? i_next * num / den : ~0ull;
  }
  double sum = 0.0;
  for (int64_t idx = e0; idx < e1 && mine; ++idx) {
    int64_t og, orr;
    elem_offsets(d, idx, og, orr);
    float adf, rf;
    uint32_t k;
    bool mmk;
    elem_test<DT, MODE>(load_elem<DT>(d.g, og), load_elem<DT>(d.r, orr), d, adf, k, mmk, rf);
    if (!(fabsf(rf) <= d.nz_abs)) continue;
    if (all) {
      a.near_sample[d.sample_off + rank] = adf;
      sum += (double)adf;
    } else if (rank == j_next) {
      a.near_sample[d.sample_off + i_next] = adf;
      sum += (double)adf;
      ++i_next;
      j_next = i_next < mm ? i_next * (c - 1) / (mm - 1) : ~0ull;
    }
    ++rank;
  }
  sum = wave_sum(sum);
  if ((tid & 63) == 0) dsum[tid >> 6] = sum;
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
    for (int i = 0; i < kWaves; ++i) t += dsum[i];
    a.item_near_sum[item] = t;
  }
}

#include "kvv_tail.h"
#include "kvv_isel.h"

}  // namespace kvv
