// Verdict kernels for gfx950.
//
//   scan_kernel     one HBM pass over both tensors: elementwise test, counts,
//                   maxima with argmax, ULP histogram, fp64 sums, finite
//                   pattern, and the strided sample (re-read from cache).
//                   Per-block partial "run records" go to the workspace.
//   reduce_kernel   one block per segment: combines its run records in a fixed
//                   order (bit-reproducible) and writes the kvv_result.
//   near_kernel     tolerant-policy near-zero diagnostics: the rank-strided
//                   sample of the compacted near-zero abs_diff array.
//   select_kernel   exact order statistics of the samples: 4 passes of an
//                   8-bit radix select with shared histograms.
//   finalize_kernel torch.quantile's rank/lerp arithmetic and the near-zero mean.
#pragma once

#include "kvv_device.h"

namespace kvv {

constexpr int kUnroll = 4;            // 16-byte vectors per thread per item
constexpr int kSelChunk = 16384;      // sample values per select block
constexpr int kArrays = 3;            // abs, rel, near-zero abs
constexpr int kSelPasses = 4;
constexpr int kHistPerSeg = kArrays * kSelPasses * 2 * 256;

enum Layout { L_CONTIG = 0, L_ROWS = 1, L_GENERIC = 2 };

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
  int64_t row_len;        // L_ROWS: contiguous inner length
  Dims dims;              // L_ROWS: outer dims; L_GENERIC: all dims
};

// Partial verdict of a contiguous run of items handled by one block.
struct RunRec {
  uint64_t cnt[LC_COUNT];
  uint64_t mismatch;
  uint64_t first_mm, first_viol;
  uint64_t gabs_i, grel_i;
  uint32_t mm_abs, mm_rel, gabs_k, grel_k;
  double s[7];  // gg rr gr dd | sampled gg rr gr
};

struct ScanArgs {
  SegDesc seg0;            // the segment when table == nullptr
  const SegDesc* table;    // batch: segments of this launch, ascending item_begin
  int32_t nseg;
  int32_t pad;
  int64_t item_lo;         // items of this launch: [item_lo, item_lo + items)
  int64_t items;
  int64_t items_per_block;
  RunRec* runs;            // indexed by global item
  uint32_t* run_valid;     // 1 where a run starts at that item
  float* sample_abs;
  float* sample_rel;
  uint32_t* item_near;     // near-zero count per item (KVV_FLAG_NEAR_ZERO)
};

struct Acc {
  uint32_t mism;
  uint32_t mm_abs, mm_rel;
  uint32_t gabs_k, grel_k;
  uint32_t nfast;          // bit-identical finite pairs (ULP bucket 0, never a mismatch)
  uint32_t nnear_fast;     // ... of which near zero
  uint64_t first_mm, first_viol;
  uint64_t gabs_i, grel_i;
  uint64_t first_fast;     // lowest index of such a pair (an abs/rel argmax candidate of value 0)
  double e_sq;             // sum of g*g over those pairs (there g == r, so it feeds gg, rr and gr)
  double s[7];             // full path: gg rr gr dd | sampled gg rr gr
  __device__ void init() {
    mism = 0;
    mm_abs = mm_rel = 0;
    gabs_k = grel_k = 0;
    nfast = nnear_fast = 0;
    first_mm = first_viol = kNone;
    gabs_i = grel_i = kNone;
    first_fast = kNone;
    e_sq = 0.0;
#pragma unroll
    for (int i = 0; i < 7; ++i) s[i] = 0.0;
  }
};

__device__ __forceinline__ void lds_inc(uint32_t* col, int c) {
  __hip_atomic_fetch_add(&col[c * kBlock], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
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

// ------------------------------------------------------------ per element
// The reference's arithmetic, in float32 with every operation rounded on its
// own (the library is built with -ffp-contract=off):
//   float branch (GCR:722-727)  abs_diff = |g - r|,
//       mismatch = !( r == g || (isfinite(abs_diff) && abs_diff <= atol + |rtol * g|) )
//   integer branch (GCR:716-719) abs_diff = |int32(g) - int32(r)| (wrapping),
//       mismatch = abs_diff > max_abs_diff
//   rel_diff = float(abs_diff) / (|float(r)| + 1e-12f)        (GCR:730)
template <int DT, int MODE>
__device__ __forceinline__ void elem_diff(typename Elem<DT>::T gc, typename Elem<DT>::T rc, const SegDesc& d,
                                          float& adf, float& rel, uint32_t& abs_key, bool& mm, float& rf) {
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
  rel = adf / (fabsf(rf) + 1e-12f);
}

template <int DT, int MODE>
__device__ __forceinline__ void process_elem(typename Elem<DT>::T gc, typename Elem<DT>::T rc, uint64_t idx,
                                             const SegDesc& d, Acc& acc, uint32_t* col) {
  using E = Elem<DT>;
  float adf, rel, rf;
  uint32_t abs_key;
  bool mm;
  elem_diff<DT, MODE>(gc, rc, d, adf, rel, abs_key, mm, rf);
  const uint32_t rel_key = fkey(rel);
  if (mm) {
    acc.mism++;
    if (acc.first_mm == kNone) acc.first_mm = idx;
    acc.mm_abs = abs_key > acc.mm_abs ? abs_key : acc.mm_abs;
    acc.mm_rel = rel_key > acc.mm_rel ? rel_key : acc.mm_rel;
  }
  // Within a thread indices only grow, so "strictly greater, or first seen" is the argmax rule.
  if (abs_key > acc.gabs_k || acc.gabs_i == kNone) {
    acc.gabs_k = abs_key;
    acc.gabs_i = idx;
  }
  if (rel_key > acc.grel_k || acc.grel_i == kNone) {
    acc.grel_k = rel_key;
    acc.grel_i = idx;
  }
  bool nan_pair = false;
  if constexpr (E::is_float) {
    const bool ng = E::isnan(gc), nr = E::isnan(rc);
    const bool ig = E::isinf(gc), ir = E::isinf(rc);
    if (ng | nr | ig | ir) {
      // finite-pattern rule of GCR:414-437 at a non-finite position
      const bool ok = (ng && nr) || (ig && ir && E::sign(gc) == E::sign(rc));
      if (!ok) {
        lds_inc(col, LC_VIOL);
        if (acc.first_viol == kNone) acc.first_viol = idx;
      }
      if (ng) lds_inc(col, LC_NAN_G);
      if (nr) lds_inc(col, LC_NAN_R);
      if (ig) lds_inc(col, E::sign(gc) ? LC_NINF_G : LC_PINF_G);
      if (ir) lds_inc(col, E::sign(rc) ? LC_NINF_R : LC_PINF_R);
      if (ng | nr) {
        lds_inc(col, LC_NANPAIR);
        nan_pair = true;
      }
    }
  }
  if (!nan_pair) lds_inc(col, LC_HIST0 + ulp_bucket(pair_distance<DT>(gc, rc)));
  const double g64 = E::f64(gc), r64 = E::f64(rc);
  const double d64 = g64 - r64;
  acc.s[0] = fma(g64, g64, acc.s[0]);
  acc.s[1] = fma(r64, r64, acc.s[1]);
  acc.s[2] = fma(g64, r64, acc.s[2]);
  acc.s[3] = fma(d64, d64, acc.s[3]);
  if (d.flags & KVV_FLAG_NEAR_ZERO) {
    const bool near = fabsf(rf) <= d.nz_abs;
    if (near) {
      lds_inc(col, LC_NEAR);
      if (adf > d.nz_bad) lds_inc(col, LC_NEARBAD);
    } else if (mm) {
      lds_inc(col, LC_FARMM);
    }
  }
}

template <int DT>
__device__ __forceinline__ typename Elem<DT>::T load_elem(const void* base, int64_t off) {
  return reinterpret_cast<const typename Elem<DT>::T*>(base)[off];
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
  float adf, rel, rf;
  uint32_t k;
  bool mm;
  elem_diff<DT, MODE>(gc, rc, d, adf, rel, k, mm, rf);
  sabs[d.sample_off + i] = adf;
  srel[d.sample_off + i] = rel;
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
    for (int64_t idx = L0 + threadIdx.x; idx < L1; idx += kBlock) sample_one<DT, MODE>(d, idx, idx, acc, sabs, srel);
    return;
  }
  const uint64_t num = (uint64_t)d.n - 1, den = (uint64_t)d.m - 1;
  uint64_t i = ((uint64_t)L0 * den + num - 1) / num + threadIdx.x;
  for (; i < (uint64_t)d.m; i += kBlock) {
    const uint64_t idx = i * num / den;
    if (idx >= (uint64_t)L1) break;
    sample_one<DT, MODE>(d, (int64_t)idx, (int64_t)i, acc, sabs, srel);
  }
}

// Vector path: 16-byte loads of both tensors, kUnroll vectors per thread.
//
// Phase A runs over every element and only tells bit-identical finite pairs
// apart from the rest: such a pair is never a mismatch, has abs_diff = rel_diff
// = 0, ULP distance 0, and contributes g*g to the three product sums.  Phase B
// gives every other element the full treatment (process_elem), each lane
// walking its own list of such elements re-read from an LDS stage, so the
// wave pays for the longest list of any lane rather than for every element.
template <int DT, int MODE>
__device__ __forceinline__ void scan_item_vec(const SegDesc& d, int64_t L0, int64_t L1, Acc& acc, uint32_t* col,
                                              uint4* stage) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int V = 16 / sizeof(T);
  constexpr int NE = V * kUnroll;
  static_assert(NE <= 64, "per-lane element mask is 64 bits");
  union Vec {
    uint4 u;
    T e[V];
  };
  const int tid = threadIdx.x;
  Vec gv[kUnroll], rv[kUnroll];
  uint32_t full = 0;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = L0 + (int64_t)(u * kBlock + tid) * V;
    if (v + V <= L1) {
      full |= 1u << u;
      int64_t og, orr;
      if (d.layout == L_CONTIG) {
        og = orr = v;
      } else {
        elem_offsets(d, v, og, orr);
      }
      gv[u].u = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(d.g) + og);
      rv[u].u = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(d.r) + orr);
    } else {
      gv[u].u = make_uint4(0, 0, 0, 0);
      rv[u].u = make_uint4(0, 0, 0, 0);
    }
  }
  const bool fast_ok = d.fast != 0;
  const bool near_mode = (d.flags & KVV_FLAG_NEAR_ZERO) != 0;
  uint64_t slow = 0, valid = 0;
  double esq = 0.0;
  uint32_t nnear = 0;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (!((full >> u) & 1u)) continue;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const T gc = gv[u].e[e], rc = rv[u].e[e];
      const bool fast = fast_ok && gc == rc && E::finite(gc);
      const double g64 = fast ? E::f64(gc) : 0.0;
      esq = fma(g64, g64, esq);
      if (near_mode) nnear += (fast && fabsf(E::f32(gc)) <= d.nz_abs) ? 1u : 0u;
      slow |= (uint64_t)(!fast) << (u * V + e);
    }
    valid |= ((1ull << V) - 1) << (u * V);
  }
  acc.e_sq += esq;
  acc.nnear_fast += nnear;
  const uint64_t fastm = valid & ~slow;
  acc.nfast += (uint32_t)__popcll(fastm);
  if (fastm && acc.first_fast == kNone) {
    const int k = __builtin_ctzll(fastm);
    acc.first_fast = (uint64_t)(L0 + ((int64_t)(k / V) * kBlock + tid) * V + (k % V));
  }
  slow &= valid;
  if (slow) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      stage[(2 * u) * kBlock + tid] = gv[u].u;
      stage[(2 * u + 1) * kBlock + tid] = rv[u].u;
    }
    while (slow) {
      const int k = __builtin_ctzll(slow);
      slow &= slow - 1;
      const int u = k / V, e = k % V;
      const T gc = reinterpret_cast<const T*>(&stage[(2 * u) * kBlock + tid])[e];
      const T rc = reinterpret_cast<const T*>(&stage[(2 * u + 1) * kBlock + tid])[e];
      const uint64_t idx = (uint64_t)(L0 + ((int64_t)u * kBlock + tid) * V + e);
      process_elem<DT, MODE>(gc, rc, idx, d, acc, col);
    }
  }
  // a partial last vector (numel not a multiple of the vector width)
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = L0 + (int64_t)(u * kBlock + tid) * V;
    if (!((full >> u) & 1u) && v < L1) {
      for (int64_t idx = v; idx < L1; ++idx) {
        int64_t og, orr;
        elem_offsets(d, idx, og, orr);
        process_elem<DT, MODE>(load_elem<DT>(d.g, og), load_elem<DT>(d.r, orr), (uint64_t)idx, d, acc, col);
      }
    }
  }
}

// Scalar path: any strides, one element per thread per step.
template <int DT, int MODE>
__device__ __forceinline__ void scan_item_scalar(const SegDesc& d, int64_t L0, int64_t L1, Acc& acc, uint32_t* col) {
  for (int64_t idx = L0 + threadIdx.x; idx < L1; idx += kBlock) {
    int64_t og, orr;
    elem_offsets(d, idx, og, orr);
    process_elem<DT, MODE>(load_elem<DT>(d.g, og), load_elem<DT>(d.r, orr), (uint64_t)idx, d, acc, col);
  }
}

// ------------------------------------------------------------ block reductions
struct BlockScratch {
  uint64_t u[kWaves][LC_COUNT + 8];
  uint32_t k[kWaves][4];
  double s[kWaves][7];
};

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += red[i];
  return t;
}

// Reduces the block's accumulators and LDS counter columns into one RunRec
// (written by thread 0 at runs[slot]) and resets them for the next run.
__device__ void flush_run(Acc& acc, uint32_t* s_cnt, BlockScratch& bs, RunRec* out) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __syncthreads();
  for (int c = 0; c < LC_COUNT; ++c) {
    uint64_t own = s_cnt[c * kBlock + tid];
    if (c == LC_HIST0) own += acc.nfast;
    if (c == LC_NEAR) own += acc.nnear_fast;
    uint64_t v = wave_sum(own);
    s_cnt[c * kBlock + tid] = 0;
    if (lane == 0) bs.u[w][c] = v;
  }
  uint64_t mism = wave_sum((uint64_t)acc.mism);
  uint64_t fmm = wave_min(acc.first_mm), fvi = wave_min(acc.first_viol);
  uint32_t mma = wave_max(acc.mm_abs), mmr = wave_max(acc.mm_rel);
  // bit-identical pairs have abs_diff = rel_diff = +0, whose key is 0x80000000 in both modes
  uint32_t gak = acc.gabs_k, grk = acc.grel_k;
  uint64_t gai = acc.gabs_i, gri = acc.grel_i;
  if (better(0x80000000u, acc.first_fast, gak, gai)) {
    gak = 0x80000000u;
    gai = acc.first_fast;
  }
  if (better(0x80000000u, acc.first_fast, grk, gri)) {
    grk = 0x80000000u;
    gri = acc.first_fast;
  }
  wave_argmax(gak, gai);
  wave_argmax(grk, gri);
  double s[7];
  s[0] = wave_sum(acc.e_sq + acc.s[0]);
  s[1] = wave_sum(acc.e_sq + acc.s[1]);
  s[2] = wave_sum(acc.e_sq + acc.s[2]);
#pragma unroll
  for (int i = 3; i < 7; ++i) s[i] = wave_sum(acc.s[i]);
  if (lane == 0) {
    bs.u[w][LC_COUNT + 0] = mism;
    bs.u[w][LC_COUNT + 1] = fmm;
    bs.u[w][LC_COUNT + 2] = fvi;
    bs.u[w][LC_COUNT + 3] = gai;
    bs.u[w][LC_COUNT + 4] = gri;
    bs.k[w][0] = mma;
    bs.k[w][1] = mmr;
    bs.k[w][2] = gak;
    bs.k[w][3] = grk;
#pragma unroll
    for (int i = 0; i < 7; ++i) bs.s[w][i] = s[i];
  }
  __syncthreads();
  if (tid == 0) {
    RunRec rr;
    for (int c = 0; c < LC_COUNT; ++c) {
      uint64_t t = 0;
      for (int i = 0; i < kWaves; ++i) t += bs.u[i][c];
      rr.cnt[c] = t;
    }
    rr.mismatch = 0;
    rr.first_mm = rr.first_viol = kNone;
    rr.mm_abs = rr.mm_rel = 0;
    rr.gabs_k = rr.grel_k = 0;
    rr.gabs_i = rr.grel_i = kNone;
    for (int i = 0; i < 7; ++i) rr.s[i] = 0.0;
    for (int i = 0; i < kWaves; ++i) {
      rr.mismatch += bs.u[i][LC_COUNT + 0];
      rr.first_mm = bs.u[i][LC_COUNT + 1] < rr.first_mm ? bs.u[i][LC_COUNT + 1] : rr.first_mm;
      rr.first_viol = bs.u[i][LC_COUNT + 2] < rr.first_viol ? bs.u[i][LC_COUNT + 2] : rr.first_viol;
      rr.mm_abs = bs.k[i][0] > rr.mm_abs ? bs.k[i][0] : rr.mm_abs;
      rr.mm_rel = bs.k[i][1] > rr.mm_rel ? bs.k[i][1] : rr.mm_rel;
      if (better(bs.k[i][2], bs.u[i][LC_COUNT + 3], rr.gabs_k, rr.gabs_i)) {
        rr.gabs_k = bs.k[i][2];
        rr.gabs_i = bs.u[i][LC_COUNT + 3];
      }
      if (better(bs.k[i][3], bs.u[i][LC_COUNT + 4], rr.grel_k, rr.grel_i)) {
        rr.grel_k = bs.k[i][3];
        rr.grel_i = bs.u[i][LC_COUNT + 4];
      }
      for (int j = 0; j < 7; ++j) rr.s[j] += bs.s[i][j];
    }
    *out = rr;
  }
  acc.init();
  __syncthreads();
}

// ------------------------------------------------------------ scan kernel
template <int DT, int MODE>
__device__ __forceinline__ void scan_item(const SegDesc& d, int64_t item, const ScanArgs& a, Acc& acc,
                                          uint32_t* s_cnt, uint32_t* red, uint4* stage) {
  const int64_t L0 = (item - d.item_begin) * (int64_t)d.item_elems;
  const int64_t L1 = L0 + d.item_elems < d.n ? L0 + d.item_elems : d.n;
  uint32_t* col = s_cnt + threadIdx.x;
  const bool near = (d.flags & KVV_FLAG_NEAR_ZERO) != 0;
  uint32_t near_before = 0;
  if (near) near_before = col[LC_NEAR * kBlock] + acc.nnear_fast;
  if (d.vec)
    scan_item_vec<DT, MODE>(d, L0, L1, acc, col, stage);
  else
    scan_item_scalar<DT, MODE>(d, L0, L1, acc, col);
  sample_range<DT, MODE>(d, L0, L1, acc, a.sample_abs, a.sample_rel);
  if (near) {
    const uint32_t t = block_sum_u32(col[LC_NEAR * kBlock] + acc.nnear_fast - near_before, red);
    if (threadIdx.x == 0) a.item_near[item] = t;
  }
}

template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void scan_kernel(ScanArgs a) {
  __shared__ uint32_t s_cnt[LC_COUNT * kBlock];
  __shared__ uint4 stage[2 * kUnroll * kBlock];
  __shared__ BlockScratch bs;
  __shared__ uint32_t red[kWaves];
  const int tid = threadIdx.x;
  for (int c = 0; c < LC_COUNT; ++c) s_cnt[c * kBlock + tid] = 0;
  const int64_t i0 = a.item_lo + (int64_t)blockIdx.x * a.items_per_block;
  int64_t i1 = i0 + a.items_per_block;
  if (i1 > a.item_lo + a.items) i1 = a.item_lo + a.items;
  if (i0 >= i1) return;
  Acc acc;
  acc.init();
  if (a.table == nullptr) {
    const SegDesc& d = a.seg0;
    for (int64_t it = i0; it < i1; ++it) {
      if (tid == 0) a.run_valid[it] = (it == i0) ? 1u : 0u;
      scan_item<DT, MODE>(d, it, a, acc, s_cnt, red, stage);
    }
    flush_run(acc, s_cnt, bs, &a.runs[i0]);
    return;
  }
  // batch: segments sorted by item_begin; find the one holding i0
  int lo = 0, hi = a.nseg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.table[mid].item_begin <= i0) lo = mid; else hi = mid - 1;
  }
  int s = lo;
  int64_t run_start = i0;
  for (int64_t it = i0; it < i1; ++it) {
    while (it >= a.table[s].item_begin + a.table[s].item_count) ++s;
    if (it != run_start && it == a.table[s].item_begin) {
      flush_run(acc, s_cnt, bs, &a.runs[run_start]);
      run_start = it;
    }
    if (tid == 0) a.run_valid[it] = (it == run_start) ? 1u : 0u;
    scan_item<DT, MODE>(a.table[s], it, a, acc, s_cnt, red, stage);
  }
  flush_run(acc, s_cnt, bs, &a.runs[run_start]);
}

// ------------------------------------------------------------ reduce kernel
struct ReduceArgs {
  SegDesc seg0;
  const SegDesc* table;
  const RunRec* runs;
  const uint32_t* run_valid;
  kvv_result* out;
  uint32_t* hist;        // kHistPerSeg per segment
  uint32_t* nan_cnt;     // kArrays per segment
  const uint32_t* item_near;
  uint64_t* item_near_off;
};



constexpr int kReduceBlock = 1024;
constexpr int kMaxRuns = 4096;   // runs per segment: at most one per scan block (host caps the grid)
constexpr int kFields = LC_COUNT + 14;

// Field f of a run record folded into a wave-level partial: counts add,
// first indices take the minimum, keys the maximum, (key, index) pairs the
// argmax, fp64 sums add.  Every lane visits its runs in item order and the
// butterfly order is fixed, so the result does not depend on timing.
struct FieldAcc {
  uint64_t u;
  uint32_t k;
  double x;
};

__device__ __forceinline__ void field_init(int f, FieldAcc& a) {
  a.k = 0;
  a.x = 0.0;
  a.u = (f == LC_COUNT + 1 || f == LC_COUNT + 2 || f == LC_COUNT + 5 || f == LC_COUNT + 6) ? kNone : 0;
}

__device__ __forceinline__ void field_add(int f, FieldAcc& a, const RunRec& r) {
  if (f < LC_COUNT) {
    a.u += r.cnt[f];
  } else {
    switch (f - LC_COUNT) {
      case 0: a.u += r.mismatch; break;
      case 1: a.u = r.first_mm < a.u ? r.first_mm : a.u; break;
      case 2: a.u = r.first_viol < a.u ? r.first_viol : a.u; break;
      case 3: a.k = r.mm_abs > a.k ? r.mm_abs : a.k; break;
      case 4: a.k = r.mm_rel > a.k ? r.mm_rel : a.k; break;
      case 5: if (better(r.gabs_k, r.gabs_i, a.k, a.u)) { a.k = r.gabs_k; a.u = r.gabs_i; } break;
      case 6: if (better(r.grel_k, r.grel_i, a.k, a.u)) { a.k = r.grel_k; a.u = r.grel_i; } break;
      default: a.x += r.s[f - LC_COUNT - 7]; break;
    }
  }
}

__device__ __forceinline__ void field_wave_reduce(int f, FieldAcc& a) {
  const int g = f - LC_COUNT;
  if (f < LC_COUNT || g == 0) {
    a.u = wave_sum(a.u);
  } else if (g == 1 || g == 2) {
    a.u = wave_min(a.u);
  } else if (g == 3 || g == 4) {
    a.k = wave_max(a.k);
  } else if (g == 5 || g == 6) {
    wave_argmax(a.k, a.u);
  } else {
    a.x = wave_sum(a.x);
  }
}

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

// One block per segment: lists the segment's runs in item order, then folds
// the run records field by field (one wave per field group).
__global__ __launch_bounds__(kReduceBlock) void reduce_kernel(ReduceArgs a) {
  constexpr int kW = kReduceBlock / 64;
  __shared__ uint32_t runs[kMaxRuns];
  __shared__ uint64_t wsum[kW];
  __shared__ FieldAcc fres[kFields];
  __shared__ uint32_t s_nruns;
  const int seg = blockIdx.x;
  const SegDesc& d = a.table ? a.table[seg] : a.seg0;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < kHistPerSeg; i += kReduceBlock) a.hist[(size_t)seg * kHistPerSeg + i] = 0;
  if (tid < kArrays) a.nan_cnt[seg * kArrays + tid] = 0;
  // 1. run list (and, in near-zero mode, the exclusive prefix of per-item near counts)
  const int64_t per = (d.item_count + kReduceBlock - 1) / kReduceBlock;
  const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
  const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
  const bool near = (d.flags & KVV_FLAG_NEAR_ZERO) != 0;
  uint64_t nvalid = 0, nnear = 0;
  for (int64_t k = k0; k < k1; ++k) {
    nvalid += a.run_valid[d.item_begin + k] ? 1 : 0;
    if (near) nnear += a.item_near[d.item_begin + k];
  }
  uint64_t base_runs = 0, base_near = 0;
  for (int pass = 0; pass < (near ? 2 : 1); ++pass) {
    const uint64_t mine = pass == 0 ? nvalid : nnear;
    uint64_t incl = mine;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    __syncthreads();
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint64_t base = 0;
    for (int i = 0; i < w; ++i) base += wsum[i];
    (pass == 0 ? base_runs : base_near) = base + incl - mine;
  }
  {
    uint64_t at = base_runs, nr = base_near;
    for (int64_t k = k0; k < k1; ++k) {
      const int64_t it = d.item_begin + k;
      if (a.run_valid[it] && at < kMaxRuns) runs[at++] = (uint32_t)k;
      if (near) {
        a.item_near_off[it] = nr;
        nr += a.item_near[it];
      }
    }
  }
  if (tid == kReduceBlock - 1) s_nruns = (uint32_t)(base_runs + nvalid);
  __syncthreads();
  const uint32_t nruns = s_nruns < kMaxRuns ? s_nruns : kMaxRuns;
  // 2. field-parallel fold
  for (int f = w; f < kFields; f += kW) {
    FieldAcc fa;
    field_init(f, fa);
    for (uint32_t r = lane; r < nruns; r += 64) field_add(f, fa, a.runs[d.item_begin + runs[r]]);
    field_wave_reduce(f, fa);
    if (lane == 0) fres[f] = fa;
  }
  __syncthreads();
  if (tid != 0) return;
  RunRec r;
  for (int c = 0; c < LC_COUNT; ++c) r.cnt[c] = fres[c].u;
  r.mismatch = fres[LC_COUNT + 0].u;
  r.first_mm = fres[LC_COUNT + 1].u;
  r.first_viol = fres[LC_COUNT + 2].u;
  r.mm_abs = fres[LC_COUNT + 3].k;
  r.mm_rel = fres[LC_COUNT + 4].k;
  r.gabs_k = fres[LC_COUNT + 5].k;
  r.gabs_i = fres[LC_COUNT + 5].u;
  r.grel_k = fres[LC_COUNT + 6].k;
  r.grel_i = fres[LC_COUNT + 6].u;
  for (int i = 0; i < 7; ++i) r.s[i] = fres[LC_COUNT + 7 + i].x;
  kvv_result o;
  __builtin_memset(&o, 0, sizeof(o));
  o.numel = d.n;
  o.mismatch_count = (int64_t)r.mismatch;
  o.first_mismatch_index = r.first_mm == kNone ? -1 : (int64_t)r.first_mm;
  const bool imode = d.mode == KVV_MODE_MAX_ABS_DIFF;
  if (r.mismatch) {
    o.mismatch_max_abs = imode ? (double)ikey_value(r.mm_abs) : (double)fkey_value(r.mm_abs);
    o.mismatch_max_rel = (double)fkey_value(r.mm_rel);
  }
  o.sample_count = d.m;
  o.sample_sum_gg = r.s[4];
  o.sample_sum_rr = r.s[5];
  o.sample_sum_gr = r.s[6];
  o.sample_cosine = cosine_of(r.s[6], r.s[4], r.s[5]);
  {
    const double gn = sqrt(r.s[4]), rn = sqrt(r.s[5]);
    o.sample_norm_ratio = (gn == 0.0 && rn == 0.0) ? 1.0 : (gn == 0.0 ? 0.0 : (rn == 0.0 ? __builtin_inf() : gn / rn));
  }
  o.finite_violations = (int64_t)r.cnt[LC_VIOL];
  o.first_finite_violation = r.first_viol == kNone ? -1 : (int64_t)r.first_viol;
  o.nan_gen = (int64_t)r.cnt[LC_NAN_G];
  o.nan_ref = (int64_t)r.cnt[LC_NAN_R];
  o.posinf_gen = (int64_t)r.cnt[LC_PINF_G];
  o.posinf_ref = (int64_t)r.cnt[LC_PINF_R];
  o.neginf_gen = (int64_t)r.cnt[LC_NINF_G];
  o.neginf_ref = (int64_t)r.cnt[LC_NINF_R];
  o.near_zero_count = (int64_t)r.cnt[LC_NEAR];
  o.far_count = d.n - (int64_t)r.cnt[LC_NEAR];
  o.far_mismatch_count = (int64_t)r.cnt[LC_FARMM];
  o.near_zero_bad_count = (int64_t)r.cnt[LC_NEARBAD];
  {
    const int64_t c = o.near_zero_count;
    o.near_zero_sample_count = c < d.max_samples ? c : d.max_samples;
  }
  if (d.n > 0) {
    o.max_abs = imode ? (double)ikey_value(r.gabs_k) : (double)fkey_value(r.gabs_k);
    o.max_abs_index = (int64_t)r.gabs_i;
    o.max_rel = (double)fkey_value(r.grel_k);
    o.max_rel_index = (int64_t)r.grel_i;
  } else {
    o.max_abs_index = o.max_rel_index = -1;
  }
  for (int b = 0; b < kBuckets; ++b) o.ulp_hist[b] = r.cnt[LC_HIST0 + b];
  o.nan_pairs = (int64_t)r.cnt[LC_NANPAIR];
  o.sum_gg = r.s[0];
  o.sum_rr = r.s[1];
  o.sum_gr = r.s[2];
  o.sum_dd = r.s[3];
  {
    const double dn = sqrt(r.s[3]), rn = sqrt(r.s[1]);
    o.rel_l2 = rn == 0.0 ? (dn == 0.0 ? 0.0 : __builtin_inf()) : dn / rn;
  }
  o.cosine = cosine_of(r.s[2], r.s[0], r.s[1]);
  o.p99_abs = o.p99_rel = __builtin_nan("");
  o.near_zero_p99_abs = o.near_zero_mean_abs = __builtin_nan("");
  a.out[d.out_index] = o;
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
  int32_t pad;
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
  const uint64_t c = (uint64_t)a.res[d.out_index].near_zero_count;
  const uint64_t mm = (uint64_t)a.res[d.out_index].near_zero_sample_count;
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
    float adf, rel, rf;
    uint32_t k;
    bool mmk;
    elem_diff<DT, MODE>(load_elem<DT>(d.g, og), load_elem<DT>(d.r, orr), d, adf, rel, k, mmk, rf);
    mine += fabsf(rf) <= d.nz_abs;
  }
  // exclusive block scan (Hillis-Steele in LDS; one item per block, cheap)
  scan[tid] = mine;
  __syncthreads();
  for (int o = 1; o < kBlock; o <<= 1) {
    const uint32_t v = tid >= o ? scan[tid - o] : 0u;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  uint64_t rank = off + scan[tid] - mine;
  // next sampled rank >= rank: rank j is sampled iff j == floor(i*(c-1)/(mm-1)) for some i
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
    float adf, rel, rf;
    uint32_t k;
    bool mmk;
    elem_diff<DT, MODE>(load_elem<DT>(d.g, og), load_elem<DT>(d.r, orr), d, adf, rel, k, mmk, rf);
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

// ------------------------------------------------------------ order statistics
struct SelectArgs {
  SegDesc seg0;
  const SegDesc* table;
  const int64_t* chunk_seg;   // batch: owning segment of each chunk (per array layout)
  int32_t nseg;
  int32_t narrays;            // 2, or 3 with near-zero
  int64_t total_chunks;       // chunks per array over all segments
  const kvv_result* res;
  const float* arr[kArrays];
  uint32_t* hist;
  uint32_t* nan_cnt;
  int32_t pass;
  int32_t pad;
};

__device__ __forceinline__ int64_t group_count(const SegDesc& d, const kvv_result& r, int arr) {
  return arr < 2 ? d.m : r.near_zero_sample_count;
}

// torch.quantile(q=0.99) ranks: rank = f32(0.99) * f32(m-1) rounded to float32;
// lower = trunc(rank), upper = ceil(rank).
__device__ __forceinline__ void q99_ranks(int64_t m, uint64_t& lo, uint64_t& hi, float& w) {
  const float rank = 0.99f * (float)(m - 1);
  lo = (uint64_t)rank;
  hi = (uint64_t)ceilf(rank);
  w = rank - (float)lo;
}

// Block-cooperative search (kBlock == 256 threads, one per bin): the bin of a
// 256-bin histogram that holds 0-based rank `resid`, and how many values lie in
// lower bins.  A rank past the end (only when NaNs were left out) gives bin 255.
__device__ void block_find_bin(const uint32_t* h, uint64_t resid, uint32_t& bin, uint64_t& below, uint64_t* sh) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint64_t c = h[tid];
  uint64_t incl = c;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  __syncthreads();
  if (lane == 63) sh[w] = incl;
  if (tid == 0) {
    sh[kWaves] = 255;
    sh[kWaves + 1] = 0;
  }
  __syncthreads();
  uint64_t base = 0;
  for (int i = 0; i < w; ++i) base += sh[i];
  incl += base;
  const uint64_t excl = incl - c;
  if (c > 0 && excl <= resid && resid < incl) {
    sh[kWaves] = (uint64_t)tid;
    sh[kWaves + 1] = excl;
  }
  __syncthreads();
  bin = (uint32_t)sh[kWaves];
  below = sh[kWaves + 1];
}

// High bits fixed so far (`passes` digits) and the residual rank of target rr.
__device__ void block_select_state(const uint32_t* h, int passes, int rr, uint64_t rank, uint32_t& prefix,
                                   uint64_t& resid, uint64_t* sh) {
  prefix = 0;
  resid = rank;
  for (int p = 0; p < passes; ++p) {
    uint32_t bin;
    uint64_t below;
    block_find_bin(h + (p * 2 + rr) * 256, resid, bin, below, sh);
    prefix = (prefix << 8) | bin;
    resid -= below;
  }
}

__global__ __launch_bounds__(kBlock) void select_kernel(SelectArgs a) {
  __shared__ uint32_t lh[2][256];
  __shared__ uint64_t sh[kWaves + 2];
  __shared__ uint32_t s_nan;
  const int tid = threadIdx.x;
  const int64_t gb = blockIdx.x;
  const int arr = (int)(gb / a.total_chunks);
  const int64_t chunk = gb - (int64_t)arr * a.total_chunks;
  const int s = a.table ? (int)a.chunk_seg[chunk] : 0;
  const SegDesc& d = a.table ? a.table[s] : a.seg0;
  const int64_t count = group_count(d, a.res[d.out_index], arr);
  const int64_t c0 = (chunk - d.chunk_begin) * (int64_t)kSelChunk;
  if (c0 >= count) return;
  const int64_t c1 = c0 + kSelChunk < count ? c0 + kSelChunk : count;
  uint32_t* h = a.hist + (size_t)s * kHistPerSeg + (size_t)arr * (kSelPasses * 2 * 256);
  const int pass = a.pass;
  uint32_t p0 = 0, p1 = 0;
  {
    uint64_t lo, hi, r;
    float w;
    q99_ranks(count, lo, hi, w);
    block_select_state(h, pass, 0, lo, p0, r, sh);
    block_select_state(h, pass, 1, hi, p1, r, sh);
  }
  for (int i = tid; i < 512; i += kBlock) (&lh[0][0])[i] = 0;
  if (tid == 0) s_nan = 0;
  __syncthreads();
  const int shift = 24 - 8 * pass;
  const float* v = a.arr[arr] + d.sample_off;
  uint32_t nans = 0;
  for (int64_t i = c0 + tid; i < c1; i += kBlock) {
    const float x = v[i];
    if (__builtin_isnan(x)) {
      ++nans;
      continue;
    }
    const uint32_t k = fkey(x);
    const uint32_t dig = (k >> shift) & 255u;
    const uint32_t top = pass == 0 ? 0u : (k >> (shift + 8));
    if (top == p0) atomicAdd(&lh[0][dig], 1u);
    if (top == p1) atomicAdd(&lh[1][dig], 1u);
  }
  if (pass == 0) {
    nans = wave_sum(nans);
    if ((tid & 63) == 0 && nans) atomicAdd(&s_nan, nans);
  }
  __syncthreads();
  uint32_t* hp = h + pass * 2 * 256;
  for (int i = tid; i < 512; i += kBlock) {
    const uint32_t c = (&lh[0][0])[i];
    if (c) atomicAdd(&hp[i], c);
  }
  if (pass == 0 && tid == 0 && s_nan) atomicAdd(&a.nan_cnt[s * kArrays + arr], s_nan);
}

struct FinalArgs {
  SegDesc seg0;
  const SegDesc* table;
  int32_t narrays;
  int32_t pad;
  kvv_result* res;
  const uint32_t* hist;
  const uint32_t* nan_cnt;
  const double* item_near_sum;
};

// One block per segment: the exact order statistics of each sample array and
// torch.quantile's interpolation, plus the near-zero sample mean.
__global__ __launch_bounds__(kBlock) void finalize_kernel(FinalArgs a) {
  __shared__ uint64_t sh[kWaves + 2];
  __shared__ double part[kBlock];
  const int s = blockIdx.x;
  const SegDesc& d = a.table ? a.table[s] : a.seg0;
  const int tid = threadIdx.x;
  kvv_result& r = a.res[d.out_index];
  for (int arr = 0; arr < a.narrays; ++arr) {
    const int64_t count = group_count(d, r, arr);
    double out = __builtin_nan("");
    if (count > 0 && a.nan_cnt[s * kArrays + arr] == 0) {
      const uint32_t* h = a.hist + (size_t)s * kHistPerSeg + (size_t)arr * (kSelPasses * 2 * 256);
      uint64_t lo, hi, resid;
      float w;
      q99_ranks(count, lo, hi, w);
      uint32_t klo, khi;
      block_select_state(h, kSelPasses, 0, lo, klo, resid, sh);
      block_select_state(h, kSelPasses, 1, hi, khi, resid, sh);
      const float va = fkey_value(klo), vb = fkey_value(khi);
      // torch's lerp: small weights from the lower end, large ones from the upper end, one rounding each
      const float diff = vb - va;
      const float q = fabsf(w) < 0.5f ? fmaf(w, diff, va) : fmaf(w - 1.0f, diff, vb);
      out = (double)q;
    }
    __syncthreads();
    if (tid == 0) {
      if (arr == 0) r.p99_abs = out;
      if (arr == 1) r.p99_rel = out;
      if (arr == 2) r.near_zero_p99_abs = out;
    }
    if (arr == 2 && count > 0) {
      // fixed-order sum of the per-item sampled sums: contiguous chunks, then chunks in order
      const int64_t per = (d.item_count + kBlock - 1) / kBlock;
      const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
      const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
      double t = 0.0;
      for (int64_t k = k0; k < k1; ++k) t += a.item_near_sum[d.item_begin + k];
      part[tid] = t;
      __syncthreads();
      if (tid == 0) {
        double sum = 0.0;
        for (int i = 0; i < kBlock; ++i) sum += part[i];
        r.near_zero_mean_abs = (double)(float)(sum / (double)count);
      }
    }
  }
}

}  // namespace kvv
