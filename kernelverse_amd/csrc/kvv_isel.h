// Input select (included by kvv_kernels.h, namespace kvv): the p99 order
// statistics of abs_diff and rel_diff (GCR:396-402) over a segment's strided
// sample (GCR:338-348), read straight from the two input tensors instead of
// from sample arrays.
//
// Used by batch launches with many large groups (C4-like batches), for
// contiguous segments: the main pass then writes no sample arrays for them
// (8 bytes per sample, more than a bf16 pair's own 4) and walks no sample
// positions.  Most segments capture their order statistics (the capture path
// below); a segment whose capture misses is selected from its inputs by
// isel_fallback_kernel, one block per segment, in four steps:
//
//   hist    per chunk of samples: 11-bit histograms of the top key digit
//           (bits 31..21) of abs_diff and rel_diff, added into the segment's
//           histograms (nonzero bins only); exact zeros (identical pairs) are
//           only counted.  The chunk's sums of g^2, r^2 and g*r over its
//           samples (the sampled cosine and norm ratio, GCR:351-393) are left
//           for the run fold, which adds them up in chunk order (a capture
//           segment keeps the capture pass's);
//   find    the bins of the two order statistics of each array and the count
//           below them;
//   gather  per chunk: the values that fall in those bins (zeros aside) are
//           appended, through a per-wave LDS stage, to the segment's sample
//           region, whose space the workspace holds anyway;
//   final   the order statistics among the zeros and the appended values (in
//           LDS when at most kSmall were appended, else by streaming digit
//           passes), interpolated like torch.quantile.
//
// abs_diff and rel_diff are computed exactly as the main pass's samples are
// (sample_pair), so the result equals the selection over sample arrays.

constexpr int kIselStage = 512;          // per-wave LDS stage of the gather, values per array

struct IselArgs {
  SegDesc* table;          // (the pivot launch writes the capture thresholds of its segments)
  const int2* chunks;      // chunk launches: work list of (segment, chunk of the segment), one per block,
  const uint32_t* nchunks; // ... of this length (the blocks past it have no work)
  double* sums;            // sampled sums per chunk (3 each, at the segment's isel_chunk0 + chunk)
  const int32_t* segs;     // segment launches: segment per block,
  const uint32_t* nsegs;   // ... this many (null: one for every block)
  uint32_t* state;         // kIselStateWords per input-select segment (SegDesc::isel_slot)
  float* buf[2];           // the sample arrays: space for the appended abs_diff, rel_diff
  kvv_result* res;
  const uint4* cap_runs;   // capture final: the run records of the main pass
  // capture final: the fallback's segment list, to which it adds the segments that miss
  int32_t* fb_segs;
  uint32_t* fb_scount;
  int32_t group;           // fallback launch: the dtype group whose segments it takes
};

// abs_diff and the rel_diff denominator of one pair, as elem_test / sample_pair
// compute them.  rel_diff = abs_diff / den; abs_diff == 0 gives +0 (den is then
// finite and positive).
template <int DT, int MODE>
__device__ __forceinline__ void diff_parts(typename Elem<DT>::T gc, typename Elem<DT>::T rc, float& adf, float& den) {
  using E = Elem<DT>;
  const float rf = E::f32(rc);
  if constexpr (MODE == KVV_MODE_ISCLOSE) {
    adf = fabsf(E::f32(gc) - rf);
  } else {
    const uint32_t diff = (uint32_t)E::i32(gc) - (uint32_t)E::i32(rc);
    const int32_t sd = (int32_t)diff;
    adf = (float)(sd < 0 ? (int32_t)(0u - diff) : sd);
  }
  den = fabsf(rf) + 1e-12f;
}

// Calls f(abs_diff, den, act, g, r) for every element of [e0, e1) of the
// contiguous segment d (e0 a multiple of the vector width), 16-byte vectors of
// both tensors, kIselUnroll per thread and round.  Every thread of the block
// takes part in every call (act marks real elements), so f may use wave-wide
// operations.
constexpr int kIselUnroll = 4;
template <int DT, int MODE, typename F>
__device__ __forceinline__ void chunk_pass(const SegDesc& d, int64_t e0, int64_t e1, F&& f) {
  using T = typename Elem<DT>::T;
  constexpr int V = VecIO<DT>::V;
  const int tid = threadIdx.x;
  const int64_t j0 = e0 / V, j1 = e1 / V;  // full vectors
  // global address space: flat loads would also count against the LDS counter
  typedef const __attribute__((address_space(1))) u32x4* G4;
  const G4 g4 = (G4)d.g;
  const G4 r4 = (G4)d.r;
#pragma unroll 1
  for (int64_t v0 = j0; v0 < j1; v0 += kIselUnroll * kBlock) {
    uint4 gq[kIselUnroll], rq[kIselUnroll];
#pragma unroll
    for (int u = 0; u < kIselUnroll; ++u) {
      const int64_t j = v0 + u * kBlock + tid;
      if (j < j1) {
        const u32x4 x = __builtin_nontemporal_load(g4 + j), y = __builtin_nontemporal_load(r4 + j);
        gq[u] = make_uint4(x.x, x.y, x.z, x.w);
        rq[u] = make_uint4(y.x, y.y, y.z, y.w);
      } else {
        gq[u] = rq[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int u = 0; u < kIselUnroll; ++u) {
      const bool act = v0 + u * kBlock + tid < j1;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float adf, den;
        const T gc = vec_code<DT>(gq[u], e), rc = vec_code<DT>(rq[u], e);
        diff_parts<DT, MODE>(gc, rc, adf, den);
        f(adf, den, act, gc, rc);
      }
    }
  }
  // the segment's last partial vector: fewer than V elements, one round
  if (j1 * V < e1) {
    const int64_t i = j1 * V + tid;
    const bool act = i < e1;
    const T gc = act ? load_elem<DT>(d.g, i) : (T)0;
    const T rc = act ? load_elem<DT>(d.r, i) : (T)0;
    float adf, den;
    diff_parts<DT, MODE>(gc, rc, adf, den);
    f(adf, den, act, gc, rc);
  }
}

// Logical index of sample i of a segment with m < n: i*s_div + floor(i*s_mod/(m-1))
// (GCR:346-347).  i*s_mod < 2^48, so the quotient from doubles is off by at
// most one, which the remainder corrects.
__device__ __forceinline__ int64_t sample_index(const SegDesc& d, int64_t i, double inv_den) {
  const int64_t den = d.m - 1;
  const int64_t t = i * (int64_t)d.s_mod;
  int64_t q = (int64_t)((double)t * inv_den);
  const int64_t rem = t - q * den;
  q += rem < 0 ? -1 : (rem >= den ? 1 : 0);
  return i * (int64_t)d.s_div + q;
}

// Calls f(abs_diff, den, act, g, r) for samples [i0, i1) of segment d (m < n,
// contiguous): kIselSampleUnroll samples per thread and round, element loads.
// A thread's samples are kBlock apart; its index steps from one to the next
// with the quotient and remainder of kBlock * s_mod / (m - 1).
constexpr int kIselSampleUnroll = 8;
template <int DT, int MODE, typename F>
__device__ __forceinline__ void sample_pass(const SegDesc& d, int64_t i0, int64_t i1, F&& f) {
  using T = typename Elem<DT>::T;
  typedef const __attribute__((address_space(1))) T* GT;
  const GT g = (GT)d.g;
  const GT r = (GT)d.r;
  const int tid = threadIdx.x;
  const uint32_t den = (uint32_t)(d.m - 1);  // m <= 2^24
  const uint64_t step_t = (uint64_t)kBlock * d.s_mod;
  const uint32_t step_q = (uint32_t)(step_t / den), step_r = (uint32_t)(step_t % den);
  const int64_t step_idx = (int64_t)kBlock * (int64_t)d.s_div + step_q;
  // the thread's first sample: index and remainder of i * s_mod / (m - 1)
  int64_t idx = sample_index(d, i0 + tid, 1.0 / (double)den);
  uint32_t rem = (uint32_t)(((uint64_t)(i0 + tid) * d.s_mod) % den);
#pragma unroll 1
  for (int64_t b = i0; b < i1; b += kIselSampleUnroll * kBlock) {
    T gc[kIselSampleUnroll], rc[kIselSampleUnroll];
#pragma unroll
    for (int u = 0; u < kIselSampleUnroll; ++u) {
      const int64_t i = b + u * kBlock + tid;
      gc[u] = rc[u] = (T)0;
      if (i < i1) {
        gc[u] = g[idx];
        rc[u] = r[idx];
      }
      rem += step_r;
      const bool carry = rem >= den;
      rem -= carry ? den : 0u;
      idx += step_idx + (carry ? 1 : 0);
    }
#pragma unroll
    for (int u = 0; u < kIselSampleUnroll; ++u) {
      float adf, den;
      diff_parts<DT, MODE>(gc[u], rc[u], adf, den);
      f(adf, den, b + u * kBlock + tid < i1, gc[u], rc[u]);
    }
  }
}

// The strided samples of a segment with n - 1 <= (17/16)(m - 1) (a segment a
// little past the sample cap: nearly every element a sample), elements of 1 or
// 2 bytes (whose element loads fill few bytes of a cache line each; wider
// elements measured faster with them), 16-byte vector access: windows of
// kStageSamples samples, whose
// elements the block first stages in LDS (`wg`, `wr`: kStageElems each) with
// vector loads; each thread then reads its samples from there.  Otherwise as
// sample_pass (the same samples, in the same order per thread).
constexpr int kStageSamples = kIselSampleUnroll * kBlock;
constexpr int kStageElems = 2304;  // >= kStageSamples * 17/16 + 32: a window's elements and vector slack
template <int DT>
__device__ __forceinline__ bool staged_ok(const SegDesc& d) {
  return sizeof(typename Elem<DT>::T) <= 2 && d.vec && d.m < d.n && 16 * (d.n - 1) <= 17 * (d.m - 1);
}
template <int DT, int MODE, typename F>
__device__ __forceinline__ void sample_pass_staged(const SegDesc& d, int64_t i0, int64_t i1, F&& f, uint4* wg,
                                                   uint4* wr) {
  using T = typename Elem<DT>::T;
  constexpr int V = VecIO<DT>::V;
  typedef const __attribute__((address_space(1))) u32x4* G4;
  typedef const __attribute__((address_space(1))) T* GT;
  const G4 g4 = (G4)d.g;
  const G4 r4 = (G4)d.r;
  const int tid = threadIdx.x;
  const uint32_t den = (uint32_t)(d.m - 1);  // m <= 2^24
  const double inv_den = 1.0 / (double)den;
  const uint64_t step_t = (uint64_t)kBlock * d.s_mod;
  const uint32_t step_q = (uint32_t)(step_t / den), step_r = (uint32_t)(step_t % den);
  const int64_t step_idx = (int64_t)kBlock * (int64_t)d.s_div + step_q;
  int64_t idx = sample_index(d, i0 + tid, inv_den);
  uint32_t rem = (uint32_t)(((uint64_t)(i0 + tid) * d.s_mod) % den);
  const T* sg = reinterpret_cast<const T*>(wg);
  const T* sr = reinterpret_cast<const T*>(wr);
  const int64_t nfull = d.n / V;  // vectors wholly inside the tensor
#pragma unroll 1
  for (int64_t s0 = i0; s0 < i1; s0 += kStageSamples) {
    const int64_t s1 = s0 + kStageSamples < i1 ? s0 + kStageSamples : i1;
    // the window: the vectors from the one holding the first sample to the one holding the last
    const int64_t w0 = sample_index(d, s0, inv_den) / V;
    const int64_t w1 = sample_index(d, s1 - 1, inv_den) / V + 1;
    for (int64_t j = w0 + tid; j < w1; j += kBlock) {
      uint4 x, y;
      if (j < nfull) {
        const u32x4 a = __builtin_nontemporal_load(g4 + j), b = __builtin_nontemporal_load(r4 + j);
        x = make_uint4(a.x, a.y, a.z, a.w);
        y = make_uint4(b.x, b.y, b.z, b.w);
      } else {
        // the tensor's partial last vector: its elements one by one
        T eg[V], er[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const int64_t k = j * V + e;
          eg[e] = k < d.n ? ((GT)d.g)[k] : (T)0;
          er[e] = k < d.n ? ((GT)d.r)[k] : (T)0;
        }
        __builtin_memcpy(&x, eg, 16);
        __builtin_memcpy(&y, er, 16);
      }
      wg[j - w0] = x;
      wr[j - w0] = y;
    }
    __syncthreads();
    const int64_t e0 = w0 * V;
    T gc[kIselSampleUnroll], rc[kIselSampleUnroll];
#pragma unroll
    for (int u = 0; u < kIselSampleUnroll; ++u) {
      const int64_t i = s0 + u * kBlock + tid;
      gc[u] = rc[u] = (T)0;
      if (i < s1) {
        gc[u] = sg[idx - e0];
        rc[u] = sr[idx - e0];
      }
      rem += step_r;
      const bool carry = rem >= den;
      rem -= carry ? den : 0u;
      idx += step_idx + (carry ? 1 : 0);
    }
#pragma unroll
    for (int u = 0; u < kIselSampleUnroll; ++u) {
      float adf, dn;
      diff_parts<DT, MODE>(gc[u], rc[u], adf, dn);
      f(adf, dn, s0 + u * kBlock + tid < s1, gc[u], rc[u]);
    }
    __syncthreads();  // (the next window overwrites the stage)
  }
}

// Calls f over the block's chunk: contiguous elements when every element is a
// sample, else the strided sample positions.
template <int DT, int MODE, typename F>
__device__ __forceinline__ void unit_pass(const SegDesc& d, int64_t e0, int64_t e1, F&& f) {
  if (d.m == d.n) chunk_pass<DT, MODE>(d, e0, e1, f);
  else sample_pass<DT, MODE>(d, e0, e1, f);
}

// Entry b of a chunk work list: its segment and element range.
__device__ __forceinline__ void chunk_range(const IselArgs& a, uint32_t b, const SegDesc*& d, int64_t& e0,
                                            int64_t& e1, int64_t& gchunk) {
  const int2 ck = a.chunks[b];
  d = &a.table[ck.x];
  const int64_t len = isel_chunk_len(*d);
  e0 = (int64_t)ck.y * len;
  e1 = e0 + len < d->m ? e0 + len : d->m;
  gchunk = d->isel_chunk0 + ck.y;
}

// The input-select passes take their work lists in block-strided loops: a
// launch sized for every chunk (or segment) costs little when the lists are
// short, which they are when every capture succeeds.
constexpr int kIselWorkBlocks = 1024;

// ------------------------------------------------------------ capture path
// An input-select segment (kFlagCapture) is selected in one read of its
// inputs (its samples are its elements, or strided positions among them):
//
//   isel_pivot_kernel      one block per segment, before the main pass: the
//                          abs/rel keys of kPivotSamples values (kPivotRuns
//                          runs of kPivotRun consecutive samples, spread over
//                          the segment), and a lower bound of their order
//                          statistic at kPivotRank from two 2048-bin
//                          histogram passes over the range of their keys,
//                          which becomes the capture threshold (cap_key);
//   main pass              every nonzero sampled value whose key reaches its
//                          threshold is written, compacted, into its run's
//                          part of the segment's sample region (from the run's
//                          first sample on); the others
//                          are counted (IS_BELOW); each run leaves a record;
//   isel_cap_final_kernel  one block per segment and array: the runs'
//                          captured values are moved together, then an order
//                          statistic of rank t lies among the zeros
//                          (t < zeros), the values below the thresholds
//                          (missed) or the captured ones (rank
//                          t - zeros - below there).  If either array misses
//                          one, the segment is added to the fallback's list,
//                          and isel_fallback_kernel selects it from its
//                          inputs.
//
// The threshold rank leaves 88 of the 4096 pivot values above it: 1 % of them
// (41) plus six standard deviations of that count (6.4 each) and a margin, so
// the p99 ranks lie above the thresholds unless the pivot runs misrepresent
// the segment, and about 2 % of the values are captured.
constexpr int kPivotRuns = 64, kPivotRun = 64, kPivotSamples = kPivotRuns * kPivotRun;
constexpr uint32_t kPivotRank = kPivotSamples - 88;
static_assert(kPivotSamples == 16 * kBlock && kPivotRun == 64 && kSmall < kIselChunk,
              "pivot values: 16 per thread, one run per wave and step, fewer than a capture segment's");

// Capture thresholds.  A NaN among the pivot values (the p99 is then NaN)
// captures the NaNs only.  cap_rel_lo and cap_rel_hi bound where rel_diff =
// fl(abs_diff / den), den = fl(|ref| + 1e-12), reaches cap_key[1] without the
// division (the threshold value v, u = 2^-24 the rounding unit):
// * below: abs_diff < fl(cap_rel_lo * den) gives fl(abs_diff / den) < v,
//   since cap_rel_lo <= v * (1 - 2^-20) and every product stays a normal float
//   (v >= 2^-80, den >= 1e-12; larger v are capped at 2^127, past which only
//   the division tells).  fl(cap_rel_lo * |ref|) is never above that product.
// * above: abs_diff >= H = fl(cap_rel_hi * |ref| + cap_rel_hic), with
//   cap_rel_hi = fl(v * (1 + 2^-20)) and cap_rel_hic = fl(cap_rel_hi * 1e-12),
//   gives H >= cap_rel_hi * (|ref| + 1e-12) * (1 - u)^2 >= cap_rel_hi * den *
//   (1 - u)^3, so abs_diff / den > v * (1 + 2^-20) * (1 - u)^4 > v and the
//   rounded quotient is at least v.  Taken for 2^-80 <= v < 2^100 (products
//   normal or, where they overflow, H infinite and the test false); else
//   cap_rel_hi is +inf and only the division tells.
__device__ inline void set_thresholds(SegDesc& d, uint32_t ka, bool nan_a, uint32_t kr, bool nan_r) {
  const uint32_t k0 = nan_a ? 0xFFFFFFFFu : ka, k1 = nan_r ? 0xFFFFFFFFu : kr;
  d.cap_key[0] = k0 > kZeroKey ? k0 : kZeroKey + 1u;
  d.cap_key[1] = k1 > kZeroKey ? k1 : kZeroKey + 1u;
  const float v = fkey_value(d.cap_key[1]);
  float lo, hi = __builtin_inff();
  if (d.cap_key[1] == 0xFFFFFFFFu) {
    lo = __builtin_inff();
  } else if (v < 0x1p-80f) {
    lo = 0.0f;
  } else {
    lo = fminf(v * (1.0f - 0x1p-20f), 0x1p127f);
    if (v < 0x1p100f) hi = v * (1.0f + 0x1p-20f);
  }
  d.cap_rel_lo = lo;
  d.cap_rel_hi = hi;
  d.cap_rel_hic = hi * 1e-12f;
}

// Counts of bins [tid * 8, tid * 8 + 8) of both block histograms.
__device__ __forceinline__ void hist_bins8(const SelectLds& L, uint32_t cA[8], uint32_t cB[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cA[i] = L.h[0][threadIdx.x * 8 + i];
    cB[i] = L.h[1][threadIdx.x * 8 + i];
  }
}

template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void isel_pivot_kernel(IselArgs a) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  SegDesc& d = a.table[a.segs[blockIdx.x]];
  uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  if (!(d.flags & kFlagCapture)) {
    // the input-select passes accumulate into the whole state
    for (int i = tid; i < kIselStateWords; i += kBlock) st[i] = 0;
    return;
  }
  // the capture counters (the histograms are cleared if the segment falls back)
  for (int i = IS_ZEROS + tid; i < kIselStateWords; i += kBlock) st[i] = 0;
  // pivot value i = k * kBlock + tid is element i % 64 of run i / 64, which starts
  // at floor(run * (m - kPivotRun) / (kPivotRuns - 1)): a wave reads one run per step
  using T = typename Elem<DT>::T;
  const uint64_t span = (uint64_t)(d.m - kPivotRun);
  const double inv_den = 1.0 / (double)(d.m - 1);
  uint32_t key[2][16];
  uint32_t low[2] = {0u, 0u}, nan[2] = {0u, 0u};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = k * kBlock + tid;
    // (sample positions: the element of sample j is j itself when every element is a sample)
    const int64_t j = (int64_t)((uint64_t)(i / kPivotRun) * span / (uint64_t)(kPivotRuns - 1)) + i % kPivotRun;
    const int64_t e = d.m == d.n ? j : sample_index(d, j, inv_den);
    const T gc = load_elem<DT>(d.g, e), rc = load_elem<DT>(d.r, e);
    float adf, den;
    diff_parts<DT, MODE>(gc, rc, adf, den);
    key[0][k] = fkey(adf);
    key[1][k] = fkey(adf / den);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      low[x] += key[x][k] <= kZeroKey ? 1u : 0u;
      nan[x] += key[x][k] == 0xFFFFFFFFu ? 1u : 0u;
    }
  }
  // counts over the block: values at or below zero (their keys go first), NaNs
  uint32_t lo_a = block_sum_nan(low[0], L), lo_r = block_sum_nan(low[1], L);
  const bool na = block_sum_nan(nan[0], L) != 0, nr = block_sum_nan(nan[1], L) != 0;
  // the order statistic at kPivotRank among the values above zero, by two
  // passes of 2048 bins over the range of those values' keys (then over the
  // range of the rank's bin): spread over the range, the adds of values that
  // share their leading key bits do not meet in a few LDS words
  uint32_t resid[2] = {kPivotRank >= lo_a ? kPivotRank - lo_a : 0u, kPivotRank >= lo_r ? kPivotRank - lo_r : 0u};
  const bool zero_a = kPivotRank < lo_a, zero_r = kPivotRank < lo_r;
  uint32_t lo[2], hi[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t kk = key[x][k];
      if (kk > kZeroKey) {
        mn = kk < mn ? kk : mn;
        mx = kk > mx ? kk : mx;
      }
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    if ((tid & 63) == 0) {
      L.sh[x * 8 + (tid >> 6)] = mn;
      L.sh[x * 8 + 4 + (tid >> 6)] = mx;
    }
  }
  __syncthreads();
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    lo[x] = L.sh[x * 8];
    hi[x] = L.sh[x * 8 + 4];
    for (int w = 1; w < kWaves; ++w) {
      lo[x] = L.sh[x * 8 + w] < lo[x] ? L.sh[x * 8 + w] : lo[x];
      hi[x] = L.sh[x * 8 + 4 + w] > hi[x] ? L.sh[x * 8 + 4 + w] : hi[x];
    }
    if (lo[x] > hi[x]) lo[x] = hi[x] = kZeroKey + 1u;  // no value above zero (the rank is then a zero)
  }
  __syncthreads();
#pragma unroll 1
  for (int lev = 0; lev < 2; ++lev) {
    int shift[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int bits = 32 - __clz(hi[x] - lo[x]);
      shift[x] = bits > 11 ? bits - 11 : 0;
    }
    for (int i = tid; i < 2 * 2048; i += kBlock) (&L.h[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const uint32_t kk = key[x][k];
        if (kk > kZeroKey && kk >= lo[x] && kk <= hi[x]) atomicAdd(&L.h[x][(kk - lo[x]) >> shift[x]], 1u);
      }
    }
    __syncthreads();
    uint32_t cA[8], cB[8], bin[2], below[2];
    hist_bins8(L, cA, cB);
    block_find2<8>(cA, cB, false, resid, bin, below, L.sh);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const uint64_t nlo = (uint64_t)lo[x] + ((uint64_t)bin[x] << shift[x]);
      const uint64_t nhi = nlo + ((uint64_t)1 << shift[x]) - 1;
      lo[x] = (uint32_t)nlo;
      hi[x] = nhi < hi[x] ? (uint32_t)nhi : hi[x];
      resid[x] -= below[x];
    }
    __syncthreads();
  }
  // the lower end of the rank's final bin: a lower bound of the order statistic
  if (tid == 0) set_thresholds(d, zero_a ? kZeroKey : lo[0], na, zero_r ? kZeroKey : lo[1], nr);
}

// LDS of the fallback's histogram step: bins 2048 + lane take the adds of a
// lane without a counted value (no branch, no shared word).
struct HistLds {
  uint32_t h[2][2048 + 64];
  uint32_t zs[kWaves];
  double ss[kWaves][3];
};

// Fallback step 1, one chunk (samples e0..e1 of d, batch-wide chunk gchunk):
// its top-digit histograms added into the segment's, its zeros counted, its
// sampled sums stored.  Called by all threads of the block.
template <int DT, int MODE>
__device__ inline void isel_hist_chunk(const IselArgs& a, const SegDesc& d, int64_t e0, int64_t e1, int64_t gchunk,
                                       HistLds& H) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  for (int i = tid; i < 2 * (2048 + 64); i += kBlock) (&H.h[0][0])[i] = 0;
  __syncthreads();
  using E = Elem<DT>;
  uint32_t zeros = 0;
  double sg = 0.0, sr = 0.0, sx = 0.0;
  unit_pass<DT, MODE>(d, e0, e1, [&](float adf, float den, bool act, typename E::T gc, typename E::T rc) {
    const bool z = adf == 0.0f;
    zeros += act && z ? 1u : 0u;
    const bool cnt = act && !z;
    const uint32_t ba = cnt ? fkey(adf) >> 21 : 2048u + lane;
    const uint32_t br = cnt ? fkey(adf / den) >> 21 : 2048u + lane;
    atomicAdd(&H.h[0][ba], 1u);
    atomicAdd(&H.h[1][br], 1u);
    // inactive lanes hold zero codes, which add 0
    const double g64 = E::f64(gc), r64 = E::f64(rc);
    sg = fma(g64, g64, sg);
    sr = fma(r64, r64, sr);
    sx = fma(g64, r64, sx);
  });
  zeros = wave_sum(zeros);
  if (lane == 0) H.zs[tid >> 6] = zeros;
  // the chunk's sampled sums, in a fixed order (bit-reproducible)
  sg = wave_sum(sg);
  sr = wave_sum(sr);
  sx = wave_sum(sx);
  if (lane == 0) {
    H.ss[tid >> 6][0] = sg;
    H.ss[tid >> 6][1] = sr;
    H.ss[tid >> 6][2] = sx;
  }
  __syncthreads();
  // (a capture segment's chunk sums are the capture pass's: the run fold may be
  // reading them while the fallback runs)
  if (tid < 3 && !(d.flags & kFlagCapture)) {
    double t = 0.0;
    for (int w = 0; w < kWaves; ++w) t += H.ss[w][tid];
    a.sums[(size_t)gchunk * 3 + tid] = t;
  }
  for (int i = tid; i < 2 * 2048; i += kBlock) {
    const uint32_t c = H.h[i >> 11][i & 2047];
    if (c) atomicAdd(&st[IS_HIST + i], c);
  }
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kWaves; ++w) t += H.zs[w];
    if (t) atomicAdd(&st[IS_ZEROS], t);
  }
  __syncthreads();
}

// Writes the wave's LDS stage out to buf, at space reserved in the segment's
// count with one atomic (fill is wave-uniform).
__device__ __forceinline__ void stage_flush(const float* stage, uint32_t& fill, uint32_t* count, float* buf) {
  const int lane = lane_id();
  uint32_t base = 0;
  if (lane == 0) base = atomicAdd(count, fill);
  base = __builtin_amdgcn_readfirstlane(base);
  for (uint32_t i = lane; i < fill; i += 64) buf[base + i] = stage[i];
  fill = 0;
}

// Appends v for the lanes with p to the wave's LDS stage; a stage without room
// for a whole wave is written out first.
__device__ __forceinline__ void stage_append(float* stage, uint32_t& fill, bool p, float v, uint32_t* count,
                                             float* buf) {
  const uint64_t b = __ballot(p);
  if (!b) return;
  if (fill + 64 > (uint32_t)kIselStage) stage_flush(stage, fill, count, buf);
  const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
  if (p) stage[fill + below] = v;
  fill += (uint32_t)__popcll(b);
}

// Fallback step 3, one chunk: its values in the target bins appended to the
// segment's sample region.  Called by all threads of the block; each wave's
// stage is its own and written out at the end of the chunk.
template <int DT, int MODE>
__device__ inline void isel_gather_chunk(const IselArgs& a, const SegDesc& d, int64_t e0, int64_t e1,
                                         float (&stage)[kWaves][2][kIselStage]) {
  const int w = threadIdx.x >> 6;
  uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  const bool nan0 = st[IS_NAN] != 0, nan1 = st[IS_NAN + 1] != 0;
  if (nan0 && nan1) return;
  const uint32_t p00 = st[IS_PFX], p01 = st[IS_PFX + 1], p10 = st[IS_PFX + 2], p11 = st[IS_PFX + 3];
  float* ba = a.buf[0] + d.sample_off;
  float* br = a.buf[1] + d.sample_off;
  uint32_t fa = 0, fr = 0;
  using T = typename Elem<DT>::T;
  unit_pass<DT, MODE>(d, e0, e1, [&](float adf, float den, bool act, T, T) {
    const float rel = adf / den;
    const uint32_t ka = fkey(adf) >> 21, kr = fkey(rel) >> 21;
    const bool cnt = act && adf != 0.0f;
    stage_append(stage[w][0], fa, cnt && !nan0 && (ka == p00 || ka == p01), adf, &st[IS_GFILL], ba);
    stage_append(stage[w][1], fr, cnt && !nan1 && (kr == p10 || kr == p11), rel, &st[IS_GFILL + 1], br);
  });
  if (fa) stage_flush(stage[w][0], fa, &st[IS_GFILL], ba);
  if (fr) stage_flush(stage[w][1], fr, &st[IS_GFILL + 1], br);
}

// The capture pass of the capture segments with strided samples, one block
// per chunk of their samples: the sampled values at or above the pivot
// thresholds are appended (through per-wave LDS stages) to the segment's
// sample region, counted in IS_FILL; the nonzero ones below are counted in
// IS_BELOW; and the chunk's sampled sums are left as the fallback's
// histogram step leaves them.  (Dense capture segments are captured by the
// main pass.)
template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void isel_capture_kernel(IselArgs a) {
  __shared__ float stage[kWaves][2][kIselStage];
  // a window of staged elements (sample_pass_staged: elements of at most 2 bytes)
  __shared__ uint4 win[2][sizeof(typename Elem<DT>::T) <= 2 ? kStageElems * 2 / 16 : 1];
  __shared__ uint32_t nb[kWaves][2];
  __shared__ double ss[kWaves][3];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t nwork = *a.nchunks;
#pragma unroll 1
  for (uint32_t b = blockIdx.x; b < nwork; b += gridDim.x) {
    const SegDesc* d;
    int64_t e0, e1, gchunk;
    chunk_range(a, b, d, e0, e1, gchunk);
    uint32_t* st = a.state + (size_t)d->isel_slot * kIselStateWords;
    float* ba = a.buf[0] + d->sample_off;
    float* br = a.buf[1] + d->sample_off;
    const uint32_t k0 = d->cap_key[0], k1 = d->cap_key[1];
    uint32_t fa = 0, fr = 0, b0 = 0, b1 = 0;
    bool nan0 = false, nan1 = false, neg = false;
    double sg = 0.0, sr = 0.0, sx = 0.0;
    using E = Elem<DT>;
    const float crlo = d->cap_rel_lo;
    auto capture = [&](float adf, float den, bool act, typename E::T gc, typename E::T rc) {
      const bool nz = act && !(adf == 0.0f);
      const bool ca = nz && fkey(adf) >= k0;
      // rel_diff is divided out only where it can reach its threshold (set_thresholds)
      float rel = 0.0f;
      bool cr = false;
      if (nz && !(adf < crlo * den)) {
        rel = adf / den;
        cr = fkey(rel) >= k1;
      }
      b0 += nz && !ca ? 1u : 0u;
      b1 += nz && !cr ? 1u : 0u;
      nan0 = nan0 || (ca && adf != adf);
      nan1 = nan1 || (cr && rel != rel);
      neg = neg || (act && adf < 0.0f);
      stage_append(stage[w][0], fa, ca, adf, &st[IS_FILL], ba);
      stage_append(stage[w][1], fr, cr, rel, &st[IS_FILL + 1], br);
      // inactive lanes hold zero codes, which add 0
      const double g64 = E::f64(gc), r64 = E::f64(rc);
      sg = fma(g64, g64, sg);
      sr = fma(r64, r64, sr);
      sx = fma(g64, r64, sx);
    };
    if (staged_ok<DT>(*d)) sample_pass_staged<DT, MODE>(*d, e0, e1, capture, win[0], win[1]);
    else unit_pass<DT, MODE>(*d, e0, e1, capture);
    if (fa) stage_flush(stage[w][0], fa, &st[IS_FILL], ba);
    if (fr) stage_flush(stage[w][1], fr, &st[IS_FILL + 1], br);
    if (__ballot(nan0) && lane == 0) st[IS_CNAN] = 1u;
    if (__ballot(nan1) && lane == 0) st[IS_CNAN + 1] = 1u;
    if (__ballot(neg) && lane == 0) st[IS_CNEG] = 1u;
    b0 = wave_sum(b0);
    b1 = wave_sum(b1);
    // the chunk's sampled sums, in a fixed order (bit-reproducible)
    sg = wave_sum(sg);
    sr = wave_sum(sr);
    sx = wave_sum(sx);
    if (lane == 0) {
      nb[w][0] = b0;
      nb[w][1] = b1;
      ss[w][0] = sg;
      ss[w][1] = sr;
      ss[w][2] = sx;
    }
    __syncthreads();
    if (tid < 3) {
      double t = 0.0;
      for (int v = 0; v < kWaves; ++v) t += ss[v][tid];
      a.sums[(size_t)gchunk * 3 + tid] = t;
    } else if (tid < 5) {
      uint32_t t = 0;
      for (int v = 0; v < kWaves; ++v) t += nb[v][tid - 3];
      if (t) atomicAdd(&st[IS_BELOW + tid - 3], t);
    }
    __syncthreads();
  }
}

#ifdef KVV_COMMON_KERNELS
// Where the order statistics of capture array x lie: rank t among the zeros
// (the smallest values: need = false), among the values below the threshold
// (a miss) or among the `cap` captured ones (need, at rank rk there).
struct CapRanks {
  bool miss, need[2];
  uint32_t rk[2];
};
__device__ __forceinline__ CapRanks cap_ranks(const SegDesc& d, uint32_t cap, uint32_t below, bool nan,
                                              const uint64_t rank[2]) {
  CapRanks c;
  // (more counted than the segment holds cannot happen; it would fall back)
  c.miss = (uint64_t)cap + below > (uint64_t)d.m;
  const uint64_t zeros = c.miss ? 0 : (uint64_t)d.m - cap - below;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    c.need[t] = !nan && !c.miss && rank[t] >= zeros + below;
    c.rk[t] = c.need[t] ? (uint32_t)(rank[t] - zeros - below) : 0u;
    c.miss = c.miss || (!nan && rank[t] >= zeros && rank[t] < zeros + below);
  }
  return c;
}

// Moves the runs' captured values of array x (each at its run's first element)
// together at the start of the region, run after run (a run's values only move
// down, over values already moved); within a run, a step of the block reads
// all its values before it writes them.
__device__ inline void cap_compact(const IselArgs& a, const SegDesc& d, int64_t nruns, int x) {
  const int tid = threadIdx.x;
  float* v = a.buf[x] + d.sample_off;
  uint32_t pos = 0;
  for (int64_t k = 0; k < nruns; ++k) {
    const uint4 rec = a.cap_runs[d.run_slot0 + k];
    const uint32_t c = x == 0 ? rec.y : rec.z;
    if (rec.x != pos) {
      constexpr int PER = 8;
      for (uint32_t o = 0; o < c; o += PER * kBlock) {
        float t[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const uint32_t j = o + i * kBlock + tid;
          t[i] = j < c ? v[rec.x + j] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const uint32_t j = o + i * kBlock + tid;
          if (j < c) v[pos + j] = t[i];
        }
        __threadfence_block();
        __syncthreads();
      }
    }
    pos += c;
  }
}

// Two blocks per segment: block 2s + x selects array x (both blocks place the
// order statistics from the same counts, so they agree on a miss; the x = 0
// block then hands the segment to the input-select passes).
__global__ __launch_bounds__(kBlock) void isel_cap_final_kernel(IselArgs a) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  const int x = (int)(blockIdx.x & 1u);
  const int seg = a.segs[blockIdx.x >> 1];
  const SegDesc& d = a.table[seg];
  if (!(d.flags & kFlagCapture)) return;
  uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  uint64_t rank64[2];
  float wgt;
  q99_ranks(d.m, rank64, wgt);
  // the captured totals: the main pass's runs' counts, or the capture pass's (already compact)
  const bool elems = (d.flags & kFlagCaptureElems) != 0;
  const int64_t nruns = elems ? segment_runs(d) : 0;
  uint32_t t0 = 0, t1 = 0;
  for (int64_t k = tid; k < nruns; k += kBlock) {
    const uint4 rec = a.cap_runs[d.run_slot0 + k];
    t0 += rec.y;
    t1 += rec.z;
  }
  uint32_t cap[2] = {block_sum_nan(t0, L), block_sum_nan(t1, L)};
  if (!elems) {
    cap[0] = st[IS_FILL];
    cap[1] = st[IS_FILL + 1];
  }
  const bool nan[2] = {st[IS_CNAN] != 0, st[IS_CNAN + 1] != 0};
  const CapRanks c0 = cap_ranks(d, cap[0], st[IS_BELOW], nan[0], rank64);
  const CapRanks c1 = cap_ranks(d, cap[1], st[IS_BELOW + 1], nan[1], rank64);
  if (st[IS_CNEG] != 0 || c0.miss || c1.miss) {
    // the fallback takes the segment over, from cleared histograms and counts
    // (not the words either block reads above)
    if (x != 0) return;
    __syncthreads();
    for (int i = tid; i <= IS_BASE + 3; i += kBlock)
      if (i != IS_FILL && i != IS_FILL + 1) st[i] = 0;
    if (tid == 0) a.fb_segs[atomicAdd(a.fb_scount, 1u)] = seg;
    return;
  }
  const CapRanks& c = x == 0 ? c0 : c1;
  uint32_t key[2] = {kZeroKey, kZeroKey};
  if (c.need[0] || c.need[1]) {
    if (elems) cap_compact(a, d, nruns, x);
    const uint32_t r2[2] = {c.need[0] ? c.rk[0] : c.rk[1], c.need[1] ? c.rk[1] : c.rk[0]};
    uint32_t k[2];
    range_keys(a.buf[x] + d.sample_off, cap[x], r2, k, L);
    if (c.need[0]) key[0] = k[0];
    if (c.need[1]) key[1] = k[1];
  }
  if (tid == 0) store_p99(a.res[d.out_index], x, key, wgt, nan[x]);
}

#endif  // KVV_COMMON_KERNELS

// ------------------------------------------------------------ fallback
// Fallback step 2: the bins of both order statistics of each array and the
// count below them.  Called by all threads of the block.
__device__ inline void isel_find_seg(const IselArgs& a, const SegDesc& d, SelectLds& L) {
  const int tid = threadIdx.x;
  uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  uint64_t rank64[2];
  float wgt;
  q99_ranks(d.m, rank64, wgt);
  const uint32_t zeros = st[IS_ZEROS];
#pragma unroll 1
  for (int x = 0; x < 2; ++x) {
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t bin = tid * 8 + i;
      c[i] = st[IS_HIST + x * 2048 + bin] + (bin == (kZeroKey >> 21) ? zeros : 0u);
    }
    const uint32_t resid[2] = {(uint32_t)rank64[0], (uint32_t)rank64[1]};
    uint32_t bin[2], below[2];
    block_find2<8>(c, c, true, resid, bin, below, L.sh);
    if (tid == 0) {
      st[IS_NAN + x] = st[IS_HIST + x * 2048 + 2047] != 0 ? 1u : 0u;  // the bin of the NaN keys
      st[IS_PFX + 2 * x] = bin[0];
      st[IS_PFX + 2 * x + 1] = bin[1];
      st[IS_BASE + 2 * x] = below[0];
      st[IS_BASE + 2 * x + 1] = below[1];
    }
    __syncthreads();
  }
}

// Fallback step 4: the order statistics among the zeros and the appended
// values, interpolated like torch.quantile.  Called by all threads.
__device__ inline void isel_final_seg(const IselArgs& a, const SegDesc& d, SelectLds& L) {
  const int tid = threadIdx.x;
  const uint32_t* st = a.state + (size_t)d.isel_slot * kIselStateWords;
  uint64_t rank64[2];
  float wgt;
  q99_ranks(d.m, rank64, wgt);
  const uint32_t z = st[IS_ZEROS];
#pragma unroll 1
  for (int x = 0; x < 2; ++x) {
    const bool nan = st[IS_NAN + x] != 0;
    uint32_t key[2] = {kZeroKey, kZeroKey};
    if (!nan) {
      const uint32_t p[2] = {st[IS_PFX + 2 * x], st[IS_PFX + 2 * x + 1]};
      const uint32_t b[2] = {st[IS_BASE + 2 * x], st[IS_BASE + 2 * x + 1]};
      const uint32_t filled = st[IS_GFILL + x];
      // The appended values are those of the target bins (one, or two adjacent
      // non-empty ones) without the zeros, which are the smallest values of the
      // zero bin.  Rank of each order statistic among the appended values:
      uint32_t rk[2];
      bool need[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t in_bin = (uint32_t)rank64[t] - b[t];
        // appended values of the bins before this rank's bin (the first bin's, less its zeros)
        const uint32_t before = b[t] - b[0] - (p[t] != p[0] && p[0] == (kZeroKey >> 21) ? z : 0u);
        if (p[t] == (kZeroKey >> 21)) {
          need[t] = in_bin >= z;
          rk[t] = need[t] ? before + in_bin - z : 0u;
        } else {
          need[t] = true;
          rk[t] = before + in_bin;
        }
      }
      if (need[0] || need[1]) {
        if (!need[0]) rk[0] = rk[1];
        if (!need[1]) rk[1] = rk[0];
        uint32_t k[2];
        const float* v = a.buf[x] + d.sample_off;
        if (filled <= (uint32_t)kSmall) small_keys(v, filled, rk, k, L);
        else stream_keys(v, filled, rk, k, L);
        if (need[0]) key[0] = k[0];
        if (need[1]) key[1] = k[1];
      }
    }
    if (tid == 0) store_p99(a.res[d.out_index], x, key, wgt, nan);
    __syncthreads();
  }
}

// The block's writes to global memory (state words, appended values) reach the
// block's later reads: the steps of one segment run in one block.
__device__ __forceinline__ void fallback_step_sync() {
  __threadfence();
  __syncthreads();
  __threadfence();
}

union FallbackLds {
  HistLds h;
  float stage[kWaves][2][kIselStage];
  SelectLds s;
};

// The fallback of one dtype group's segments (a.group) on the list a.segs
// (a.nsegs long: the input-select segments that do not capture, then those
// whose capture missed): one block per segment, block-strided over the list,
// taking the four steps over the segment's chunks in turn.  Launched once per
// group after the capture final; its blocks find the list empty unless a
// capture missed.
template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void isel_fallback_kernel(IselArgs a) {
  __shared__ FallbackLds U;
  const uint32_t nwork = *a.nsegs;
#pragma unroll 1
  for (uint32_t wi = blockIdx.x; wi < nwork; wi += gridDim.x) {
    const SegDesc& d = a.table[a.segs[wi]];
    if (d.isel_group != a.group) continue;
    const int64_t len = isel_chunk_len(d);
    const int64_t nck = (d.m + len - 1) / len;
#pragma unroll 1
    for (int64_t ck = 0; ck < nck; ++ck) {
      const int64_t e0 = ck * len, e1 = e0 + len < d.m ? e0 + len : d.m;
      isel_hist_chunk<DT, MODE>(a, d, e0, e1, (int64_t)d.isel_chunk0 + ck, U.h);
    }
    fallback_step_sync();
    isel_find_seg(a, d, U.s);
    fallback_step_sync();
#pragma unroll 1
    for (int64_t ck = 0; ck < nck; ++ck) {
      const int64_t e0 = ck * len, e1 = e0 + len < d.m ? e0 + len : d.m;
      isel_gather_chunk<DT, MODE>(a, d, e0, e1, U.stage);
    }
    fallback_step_sync();
    isel_final_seg(a, d, U.s);
    fallback_step_sync();
  }
}
