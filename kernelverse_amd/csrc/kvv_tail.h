// Launches after the main pass (included by kvv_kernels.h, namespace kvv):
//
//   * the fold of a segment's run records into its kvv_result, in a fixed
//     order (bit-reproducible fp64 sums);
//   * the exact order statistics of torch.quantile(q=0.99) over the strided
//     sample arrays (abs_diff, rel_diff and, for the tolerant policy, the
//     near-zero abs_diff), GCR:396-402 (torch.quantile) and GCR:525-548.
//
// One kernel, tail_kernel, plays both roles: its first `reduce_blocks` blocks
// fold run records (one segment each), the others select.  A (segment, array)
// group of at most kSmall samples is selected by one block entirely in
// registers and LDS (4 digit passes of 8 bits).  A larger group is selected by
// all of its chunk blocks in three launches.  Level 0 histograms the top 8
// bits of every value's ordering key into the group's global histogram.  Level
// 1 locates both ranks' level-0 bins, histograms bits 23..12 of the values
// under those prefixes, and keeps those values' keys in the round's own span
// of the sample array, grouped by (rank, level-1 digit), with a table of where
// every cell of 8 groups starts and each cell's smallest and largest key.  The
// final launch (one block per large group) locates the 20-bit prefixes, takes
// the key from the cell bounds when the target's cell holds one value, else
// reads only the kept keys of the target groups and counts their last 12 bits
// in LDS, then interpolates like torch.quantile and writes the result.  The
// main pass (or a clearing launch) cleared the histograms.
//
// A launch with at least as many large groups as the device has CUs (a big
// batch) needs no global histograms or level launches: a contiguous pair's
// abs/rel are selected from its inputs (kvv_isel.h), any other large group by
// one block ("level" 4, select_group_stream) that streams the group once per
// digit.

struct TailArgs {
  SegDesc seg0;               // the segment when table == nullptr
  const SegDesc* table;
  const int64_t* chunk_seg;   // batch: owning segment of each select chunk
  int32_t nseg;
  int32_t reduce_blocks;      // leading blocks that fold run records (reduce_roles per segment), 0 for none
  int32_t reduce_roles;       // 5, or 6 with the near-zero prefix; 0: one wave per segment (reduce_segment_wave)
  int32_t level;              // select level of the launch: 0 (with the fold and small groups), 1, 2 = final
  int32_t arr_lo;             // select blocks cover arrays [arr_lo, arr_lo + narr)
  int32_t narr;
  int32_t pad;
  int64_t total_chunks;       // select blocks per array
  kvv_result* res;
  RunCols runs;
  const float* arr[kArrays];
  uint32_t* slots;            // kArrays * kSlotWords words per large segment
  uint16_t* subtab;           // level-1 candidate tables: kSubTab per select round, per array
  uint32_t* submm;            // per select round and array: min and max kept key of each of its kCells cells
  int64_t total_sub;          // select rounds per array (total_chunks * rounds)
  const uint32_t* item_near;
  uint64_t* item_near_off;
  const double* item_near_sum;
  const double* isel_sums;    // input-select segments: sampled sums per chunk (3 each)
  uint64_t* near_cm;          // near-zero count and sample count per segment (device copies of the fold's)
  // near-zero entries (kFlagNearEntries, single pairs): what the main pass's waves left, and the
  // blocks of the first launch that place them in the near-zero sample
  const uint2* ent;
  const uint32_t* near_wave;
  const uint32_t* ent_fill;
  const uint2* wave_range;    // each wave's items (relative to the segment), for waves whose entries did not fit
  uint32_t ent_quota;
  int32_t nwaves;
  int32_t scatter_blocks;
  int32_t pad3;
  double* near_psum;          // per scatter block: the sum of its sampled entries
};

struct ReduceLds {
  uint64_t pu[kBlock];   // per-thread partial folds
  uint32_t pk[kBlock];
  double pd[kBlock];
  uint64_t tu[32];       // per-field totals
  double td[8];
  uint64_t wsum[kWaves];
};

// Block histograms hold two 16-bit bin counts per word: a block counts at most
// max(kSelChunk * kMaxSelRounds, kSmall) values, so a count never carries into
// its neighbour.
// Sample counts stay below 2^24 (the host caps max_samples), so ranks and
// histogram sums fit 32 bits.
struct SelectLds {
  uint32_t h[2][2048];
  double part[kBlock];
  uint32_t sh[16];
  uint32_t misc[4];
  uint32_t fill[2];  // input select: compacted values per array
};
static_assert(kSelChunk * kMaxSelRounds <= 65535 && kSmall <= 65535, "16-bit block bin counts");
static_assert(kSlotWords % 4 == 0, "slots are cleared in 16-byte stores");

union TailLds {
  ReduceLds r;
  SelectLds s;
};

// ------------------------------------------------------------ run-record fold
// kvv_result of one segment from its run columns, split over five blocks
// (roles) that each own a disjoint set of output fields: 0-2 the counts (finite
// pattern and near-zero, ULP histogram, mismatches), 3 the first indices and
// argmaxima, 4 the fp64 sums; role 5 (tolerant policy) writes the near-zero
// prefix of the per-item counts.  Inside a role,
// F fields x P parts cover the block; part p of a field folds slots
// [p*S, (p+1)*S) of the segment (S a multiple of 4, so every thread issues
// aligned 16-byte loads, all at once), and the parts are folded in order.
template <int F, int P>
__device__ __forceinline__ void role_split(int64_t nruns, int& f, int& p, int64_t& j0, int64_t& j1) {
  const int tid = threadIdx.x;
  f = tid / P;
  p = tid % P;
  int64_t span = (nruns + P - 1) / P;
  span = (span + 3) & ~int64_t(3);
  j0 = (int64_t)p * span;
  j1 = j0 + span < nruns ? j0 + span : nruns;
  if (f >= F) j0 = j1 = 0;
}

__device__ __forceinline__ int64_t segment_runs(const SegDesc& d) { return d.item_count > 0 ? d.run_n : 0; }

// Folds a u32 column part [j0, j1) (sum or max), 4 slots per load, 8 loads in flight.
template <bool MAX>
__device__ __forceinline__ uint64_t fold_u32(const uint32_t* col, int64_t j0, int64_t j1) {
  uint64_t t = 0;
  for (int64_t j = j0; j < j1; j += 32) {
    uint4 q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = j + 4 * i < j1 ? *reinterpret_cast<const uint4*>(col + j + 4 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = j + 4 * i + e < j1;
        const uint64_t x = in ? v[e] : 0u;
        if (MAX) t = x > t ? x : t; else t += x;
      }
    }
  }
  return t;
}

// Count columns [F0, F0 + F) of the segment, folded by one block; the outputs
// of those counts are written by the same block.
template <int F0, int F>
__device__ inline void reduce_counts(const TailArgs& a, const SegDesc& d, int seg, int64_t nruns, ReduceLds& L) {
  constexpr int P = kBlock / F;
  int f, p;
  int64_t j0, j1;
  role_split<F, P>(nruns, f, p, j0, j1);
  const int col_i = F0 + (f < F ? f : 0);
  const uint32_t* col = a.runs.u32 + (size_t)col_i * a.runs.stride + d.run_slot0;
  const bool is_max = col_i == CU_MMABS || col_i == CU_MMREL;
  L.pu[threadIdx.x] = is_max ? fold_u32<true>(col, j0, j1) : fold_u32<false>(col, j0, j1);
  __syncthreads();
  const int tid = threadIdx.x, lane = tid & 63;
  // field i's parts are folded by wave i mod 4: a few parts per lane, then the lanes (DPP)
  for (int i = tid >> 6; i < F; i += kWaves) {
    const int c = F0 + i;
    const bool mx = c == CU_MMABS || c == CU_MMREL;
    uint64_t t = 0;
    for (int q = lane; q < P; q += 64) {
      const uint64_t v = L.pu[i * P + q];
      t = mx ? (v > t ? v : t) : t + v;
    }
    t = mx ? wave_max(t) : wave_sum(t);
    if (lane == 0) L.tu[c] = t;
  }
  __syncthreads();
  kvv_result& o = a.res[d.out_index];
  const double qnan = __builtin_nan("");
  auto cnt = [&](int c) { return L.tu[c]; };
  if (F0 == 0) {  // finite pattern and near-zero counts
    switch (tid) {
      case 0:
        o.finite_violations = (int64_t)cnt(LC_VIOL);
        o.nan_gen = (int64_t)cnt(LC_NAN_G);
        o.nan_ref = (int64_t)cnt(LC_NAN_R);
        o.posinf_gen = (int64_t)cnt(LC_PINF_G);
        break;
      case 1:
        o.posinf_ref = (int64_t)cnt(LC_PINF_R);
        o.neginf_gen = (int64_t)cnt(LC_NINF_G);
        o.neginf_ref = (int64_t)cnt(LC_NINF_R);
        o.nan_pairs = (int64_t)cnt(LC_NANPAIR);
        break;
      case 2: {
        const int64_t c = (int64_t)cnt(LC_NEAR);
        o.near_zero_count = c;
        o.far_count = d.n - c;
        o.far_mismatch_count = (int64_t)cnt(LC_FARMM);
        o.near_zero_bad_count = (int64_t)cnt(LC_NEARBAD);
        const int64_t nm = c < d.max_samples ? c : d.max_samples;
        o.near_zero_sample_count = nm;
        if (a.near_cm) {
          // the later launches read these from device memory (the record may be host memory)
          a.near_cm[2 * seg] = (uint64_t)c;
          a.near_cm[2 * seg + 1] = (uint64_t)nm;
        }
        // the near-zero selection writes these when it has a sample to work on
        if (!(d.flags & kFlagNearAny) || nm == 0) o.near_zero_p99_abs = o.near_zero_mean_abs = qnan;
        break;
      }
      default:
        break;
    }
  } else if (F0 == LC_HIST0) {  // ULP histogram
    if (tid < kBuckets) o.ulp_hist[tid] = cnt(LC_HIST0 + tid);
  } else {  // mismatches, and the fields of no column
    if (tid != 0) return;
    const bool imode = d.mode == KVV_MODE_MAX_ABS_DIFF;
    o.numel = d.n;
    const uint64_t mm = cnt(CU_MISM);
    o.mismatch_count = (int64_t)mm;
    const uint32_t ka = (uint32_t)cnt(CU_MMABS), kr = (uint32_t)cnt(CU_MMREL);
    o.mismatch_max_abs = mm ? (imode ? (double)ikey_value(ka) : (double)fkey_value(ka)) : 0.0;
    o.mismatch_max_rel = mm ? (double)fkey_value(kr) : 0.0;
    o.sample_count = d.m;
    // an empty sample has no selection to write its quantiles
    if (d.m == 0) o.p99_abs = o.p99_rel = qnan;
    o.status = 0;  // (a wave whose near-zero entries did not fit is re-read by the first tail launch)
    o.reserved = 0;
  }
}

__device__ inline void reduce_extrema(const TailArgs& a, const SegDesc& d, int64_t nruns, ReduceLds& L) {
  // fields: 0 first mismatch, 1 first finite violation (min); 2 abs, 3 rel (argmax)
  constexpr int F = 4, P = kBlock / F;
  int f, p;
  int64_t j0, j1;
  role_split<F, P>(nruns, f, p, j0, j1);
  const int tid = threadIdx.x;
  const uint64_t* ci = a.runs.u64 + (size_t)(f < 2 ? f : CL_GABSI + (f - 2)) * a.runs.stride + d.run_slot0;
  const uint32_t* ck = a.runs.u32 + (size_t)(CU_GABSK + (f >= 2 ? f - 2 : 0)) * a.runs.stride + d.run_slot0;
  uint32_t bk = 0;
  uint64_t bi = kNone;
  for (int64_t j = j0; j < j1; j += 16) {
    uint4 qi[8];
    uint4 qk[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) qi[i] = j + 2 * i < j1 ? *reinterpret_cast<const uint4*>(ci + j + 2 * i) : make_uint4(0, 0, 0, 0);
    if (f >= 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) qk[i] = j + 4 * i < j1 ? *reinterpret_cast<const uint4*>(ck + j + 4 * i) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (j + e >= j1) continue;
      const uint4 wi = qi[e >> 1];
      const uint64_t idx = (e & 1) ? (((uint64_t)wi.w << 32) | wi.z) : (((uint64_t)wi.y << 32) | wi.x);
      if (f < 2) {
        bi = idx < bi ? idx : bi;
      } else {
        const uint4 wk = qk[e >> 2];
        const uint32_t k = (e & 3) == 0 ? wk.x : ((e & 3) == 1 ? wk.y : ((e & 3) == 2 ? wk.z : wk.w));
        if (better(k, idx, bk, bi)) {
          bk = k;
          bi = idx;
        }
      }
    }
  }
  // F * P is the block: wave f holds field f's parts, folded in registers (DPP)
  static_assert(F == kWaves && P == 64, "one wave per field");
  uint32_t tk = bk;
  uint64_t ti = bi;
  if (f < 2) ti = wave_min(ti); else wave_argmax(tk, ti);
  if ((tid & 63) == 0) {
    kvv_result& o = a.res[d.out_index];
    const bool imode = d.mode == KVV_MODE_MAX_ABS_DIFF;
    if (f == 0) {
      o.first_mismatch_index = ti == kNone ? -1 : (int64_t)ti;
    } else if (f == 1) {
      o.first_finite_violation = ti == kNone ? -1 : (int64_t)ti;
    } else if (d.n == 0) {
      if (f == 2) {
        o.max_abs = 0.0;
        o.max_abs_index = -1;
      } else {
        o.max_rel = 0.0;
        o.max_rel_index = -1;
      }
    } else if (f == 2) {
      o.max_abs = imode ? (double)ikey_value(tk) : (double)fkey_value(tk);
      o.max_abs_index = (int64_t)ti;
    } else {
      o.max_rel = (double)fkey_value(tk);
      o.max_rel_index = (int64_t)ti;
    }
  }
}

__device__ inline void reduce_sums(const TailArgs& a, const SegDesc& d, int64_t nruns, ReduceLds& L) {
  constexpr int F = 7, P = kBlock / F;
  static_assert(P <= 64, "one part per lane in the combine");
  int f, p;
  int64_t j0, j1;
  role_split<F, P>(nruns, f, p, j0, j1);
  const int tid = threadIdx.x;
  const uint64_t* col = a.runs.u64 + (size_t)(CL_S0 + (f < F ? f : 0)) * a.runs.stride + d.run_slot0;
  double t = 0.0;
  for (int64_t j = j0; j < j1; j += 16) {
    uint4 q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = j + 2 * i < j1 ? *reinterpret_cast<const uint4*>(col + j + 2 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (j + e >= j1) continue;
      const uint4 w = q[e >> 1];
      const uint64_t bits = (e & 1) ? (((uint64_t)w.w << 32) | w.z) : (((uint64_t)w.y << 32) | w.x);
      t += __longlong_as_double((long long)bits);
    }
  }
  L.pd[tid] = t;
  __syncthreads();
  // field i's parts summed by wave i mod 4 in a fixed tree (DPP): reproducible
  for (int i = tid >> 6; i < F; i += kWaves) {
    const int q = tid & 63;
    double u = q < P ? L.pd[i * P + q] : 0.0;
    u = wave_sum(u);
    if (q == 0) L.td[i] = u;
  }
  __syncthreads();
  auto sum = [&](int i) { return L.td[i]; };
  kvv_result& o = a.res[d.out_index];
  if (tid == 0) {
    // the sampled sums; an input-select segment's are its chunks', in chunk order
    double sg = sum(4), sr = sum(5), sx = sum(6);
    if (d.flags & kFlagCaptureElems) {
      // every element is a sample: the sampled sums are the full ones (exact fp64 squares)
      sg = sum(0);
      sr = sum(1);
      sx = sum(2);
    } else if (d.flags & kFlagInputSelect) {
      sg = sr = sx = 0.0;
      const int64_t nck = (d.m + isel_chunk_len(d) - 1) / isel_chunk_len(d);
      for (int64_t c = 0; c < nck; ++c) {
        const double* p = a.isel_sums + (size_t)(d.isel_chunk0 + c) * 3;
        sg += p[0];
        sr += p[1];
        sx += p[2];
      }
    }
    o.sample_sum_gg = sg;
    o.sample_sum_rr = sr;
    o.sample_sum_gr = sx;
    o.sample_cosine = cosine_of(sx, sg, sr);
    const double gn = sqrt(sg), rn = sqrt(sr);
    o.sample_norm_ratio = (gn == 0.0 && rn == 0.0) ? 1.0 : (gn == 0.0 ? 0.0 : (rn == 0.0 ? __builtin_inf() : gn / rn));
  } else if (tid == 1) {
    o.sum_gg = sum(0);
    o.sum_rr = sum(1);
    o.sum_gr = sum(2);
    o.sum_dd = sum(3);
    const double dn = sqrt(sum(3)), rn = sqrt(sum(1));
    o.rel_l2 = rn == 0.0 ? (dn == 0.0 ? 0.0 : __builtin_inf()) : dn / rn;
    o.cosine = cosine_of(sum(2), sum(0), sum(1));
  }
}

// The fold of a batch segment of at most 64 runs by one wave (lane k reads run
// k of every column): the outputs of the count, extrema and sum roles above,
// from wave reductions (the f64 sums in a fixed DPP tree: reproducible).
// Batches without near-zero diagnostics only.
template <bool BATCH>
__device__ inline void reduce_segment_wave(const TailArgs& a, int seg) {
  const SegDesc& d = BATCH ? a.table[seg] : a.seg0;
  const int64_t nruns = segment_runs(d);
  const int lane = lane_id();
  const bool in = lane < nruns;
  const size_t at = (size_t)d.run_slot0 + (size_t)(in ? lane : 0);
  const size_t stride = a.runs.stride;
  uint32_t cu[kColU32];
#pragma unroll
  for (int c = 0; c < kColU32; ++c) cu[c] = in ? a.runs.u32[(size_t)c * stride + at] : 0u;
  uint64_t cl[kColU64];
#pragma unroll
  for (int c = 0; c < kColU64; ++c) cl[c] = in ? a.runs.u64[(size_t)c * stride + at] : 0u;
  // every count of a segment is at most its element count: below 2^32 the
  // sums stay in 32-bit lanes (half the DPP moves of 64-bit ones)
  const bool n32 = d.n < ((int64_t)1 << 32);
  uint64_t cnt[kColU32];
#pragma unroll
  for (int c = 0; c < kColU32; ++c) {
    if (c == CU_GABSK || c == CU_GRELK) continue;
    if (c == CU_MMABS || c == CU_MMREL) cnt[c] = wave_max(cu[c]);
    else cnt[c] = n32 ? (uint64_t)wave_sum(cu[c]) : wave_sum((uint64_t)cu[c]);
  }
  uint64_t fmm = in ? cl[CL_FIRSTMM] : kNone, fviol = in ? cl[CL_FIRSTVIOL] : kNone;
  fmm = wave_min(fmm);
  fviol = wave_min(fviol);
  uint32_t ka = cu[CU_GABSK], kr = cu[CU_GRELK];
  uint64_t ia = in ? cl[CL_GABSI] : kNone, ir = in ? cl[CL_GRELI] : kNone;
  wave_argmax(ka, ia);
  wave_argmax(kr, ir);
  double sm[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) sm[i] = wave_sum(in ? __longlong_as_double((long long)cl[CL_S0 + i]) : 0.0);
  if (lane != 0) return;
  kvv_result& o = a.res[d.out_index];
  const double qnan = __builtin_nan("");
  const bool imode = d.mode == KVV_MODE_MAX_ABS_DIFF;
  // counts (as reduce_counts)
  o.finite_violations = (int64_t)cnt[LC_VIOL];
  o.nan_gen = (int64_t)cnt[LC_NAN_G];
  o.nan_ref = (int64_t)cnt[LC_NAN_R];
  o.posinf_gen = (int64_t)cnt[LC_PINF_G];
  o.posinf_ref = (int64_t)cnt[LC_PINF_R];
  o.neginf_gen = (int64_t)cnt[LC_NINF_G];
  o.neginf_ref = (int64_t)cnt[LC_NINF_R];
  o.nan_pairs = (int64_t)cnt[LC_NANPAIR];
  const int64_t nz = (int64_t)cnt[LC_NEAR];
  o.near_zero_count = nz;
  o.far_count = d.n - nz;
  o.far_mismatch_count = (int64_t)cnt[LC_FARMM];
  o.near_zero_bad_count = (int64_t)cnt[LC_NEARBAD];
  const int64_t nm = nz < d.max_samples ? nz : d.max_samples;
  o.near_zero_sample_count = nm;
  if (a.near_cm) {
    a.near_cm[2 * seg] = (uint64_t)nz;
    a.near_cm[2 * seg + 1] = (uint64_t)nm;
  }
  if (!(d.flags & kFlagNearAny) || nm == 0) o.near_zero_p99_abs = o.near_zero_mean_abs = qnan;
  for (int b = 0; b < kBuckets; ++b) o.ulp_hist[b] = cnt[LC_HIST0 + b];
  o.numel = d.n;
  const uint64_t mm = cnt[CU_MISM];
  o.mismatch_count = (int64_t)mm;
  o.mismatch_max_abs = mm ? (imode ? (double)ikey_value((uint32_t)cnt[CU_MMABS]) : (double)fkey_value((uint32_t)cnt[CU_MMABS]))
                          : 0.0;
  o.mismatch_max_rel = mm ? (double)fkey_value((uint32_t)cnt[CU_MMREL]) : 0.0;
  o.sample_count = d.m;
  if (d.m == 0) o.p99_abs = o.p99_rel = qnan;
  o.status = 0;
  o.reserved = 0;
  // extrema (as reduce_extrema)
  o.first_mismatch_index = fmm == kNone ? -1 : (int64_t)fmm;
  o.first_finite_violation = fviol == kNone ? -1 : (int64_t)fviol;
  if (d.n == 0) {
    o.max_abs = 0.0;
    o.max_abs_index = -1;
    o.max_rel = 0.0;
    o.max_rel_index = -1;
  } else {
    o.max_abs = imode ? (double)ikey_value(ka) : (double)fkey_value(ka);
    o.max_abs_index = (int64_t)ia;
    o.max_rel = (double)fkey_value(kr);
    o.max_rel_index = (int64_t)ir;
  }
  // sums (as reduce_sums)
  double sg = sm[4], sr = sm[5], sx = sm[6];
  if (d.flags & kFlagCaptureElems) {
    sg = sm[0];
    sr = sm[1];
    sx = sm[2];
  } else if (d.flags & kFlagInputSelect) {
    sg = sr = sx = 0.0;
    const int64_t nck = (d.m + isel_chunk_len(d) - 1) / isel_chunk_len(d);
    for (int64_t c = 0; c < nck; ++c) {
      const double* p = a.isel_sums + (size_t)(d.isel_chunk0 + c) * 3;
      sg += p[0];
      sr += p[1];
      sx += p[2];
    }
  }
  o.sample_sum_gg = sg;
  o.sample_sum_rr = sr;
  o.sample_sum_gr = sx;
  o.sample_cosine = cosine_of(sx, sg, sr);
  const double gn = sqrt(sg), rn = sqrt(sr);
  o.sample_norm_ratio = (gn == 0.0 && rn == 0.0) ? 1.0 : (gn == 0.0 ? 0.0 : (rn == 0.0 ? __builtin_inf() : gn / rn));
  o.sum_gg = sm[0];
  o.sum_rr = sm[1];
  o.sum_gr = sm[2];
  o.sum_dd = sm[3];
  const double dn = sqrt(sm[3]), rn2 = sqrt(sm[1]);
  o.rel_l2 = rn2 == 0.0 ? (dn == 0.0 ? 0.0 : __builtin_inf()) : dn / rn2;
  o.cosine = cosine_of(sm[2], sm[0], sm[1]);
}

// Near-zero: exclusive prefix of the per-item counts, in item order.
__device__ inline void reduce_near_prefix(const TailArgs& a, const SegDesc& d, ReduceLds& L) {
  if (!(d.flags & KVV_FLAG_NEAR_ZERO)) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t per = (d.item_count + kBlock - 1) / kBlock;
  const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
  const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
  // (8 counts per pass with their loads in flight together; one load per step,
  // and in the second loop a store between them, made every step a round trip)
  constexpr int kB = 8;
  const uint32_t* cnt = a.item_near + d.item_begin;
  uint64_t mine = 0;
  for (int64_t k = k0; k < k1; k += kB) {
    uint32_t v[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) v[q] = k + q < k1 ? cnt[k + q] : 0u;
#pragma unroll
    for (int q = 0; q < kB; ++q) mine += v[q];
  }
  uint64_t incl = mine;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) L.wsum[w] = incl;
  __syncthreads();
  uint64_t base = 0;
  for (int i = 0; i < w; ++i) base += L.wsum[i];
  uint64_t run = base + incl - mine;
  uint64_t* off = a.item_near_off + d.item_begin;
  for (int64_t k = k0; k < k1; k += kB) {
    uint32_t v[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) v[q] = k + q < k1 ? cnt[k + q] : 0u;
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      if (k + q < k1) off[k + q] = run;
      run += v[q];
    }
  }
}

template <bool BATCH>
__device__ inline void reduce_segment(const TailArgs& a, int seg, int role, ReduceLds& L) {
  // a single pair's descriptor is read from the kernel arguments (scalar loads)
  const SegDesc& d = BATCH ? a.table[seg] : a.seg0;
  const int64_t nruns = segment_runs(d);
  switch (role) {
    case 0: reduce_counts<0, LC_HIST0>(a, d, seg, nruns, L); break;
    case 1: reduce_counts<LC_HIST0, kBuckets>(a, d, seg, nruns, L); break;
    case 2: reduce_counts<CU_MISM, 3>(a, d, seg, nruns, L); break;
    case 3: reduce_extrema(a, d, nruns, L); break;
    case 4: reduce_sums(a, d, nruns, L); break;
    default: reduce_near_prefix(a, d, L); break;
  }
}

// ------------------------------------------------------------ selection
// Samples of array arr of segment s (the near-zero sample's size comes from the
// fold's device copy, written in an earlier launch).
__device__ __forceinline__ int64_t group_count(const TailArgs& a, const SegDesc& d, int s, int arr) {
  if (arr < 2) return d.m;
  // (volatile: kept a load of its own, not merged with d.m's into one generic-pointer load)
  return (int64_t)*(const volatile uint64_t*)&a.near_cm[2 * s + 1];
}

// torch.quantile(q=0.99) ranks: rank = f32(0.99) * f32(m-1) rounded to float32;
// lower = trunc(rank), upper = ceil(rank).
__device__ __forceinline__ void q99_ranks(int64_t m, uint64_t rank[2], float& w) {
  const float rk = 0.99f * (float)(m - 1);
  rank[0] = (uint64_t)rk;
  rank[1] = (uint64_t)ceilf(rk);
  w = rk - (float)rank[0];
}

// Adds 1 to bin `bin` of a packed block histogram (two 16-bit counts per
// word) for every lane with `act`: one LDS atomic per lane, no branches (the
// LDS serialises lanes that hit the same word, which costs less than merging
// them in software).
__device__ __forceinline__ void lds_hist_add(uint32_t* h, uint32_t bin, bool act) {
  if (act) atomicAdd(&h[bin >> 1], 1u << ((bin & 1u) << 4));
}

// Per-lane run-length merge in front of lds_hist_add: consecutive values of a
// lane that fall in the same bin become one add (skewed data, e.g. mostly
// identical pairs, then costs a few atomics per lane instead of one per value).
struct BinRun {
  uint32_t bin = 0, cnt = 0;
  __device__ __forceinline__ void add(uint32_t* h, uint32_t b, bool act) {
    const bool change = act && b != bin;
    if (change && cnt) atomicAdd(&h[bin >> 1], cnt << ((bin & 1u) << 4));
    bin = change ? b : bin;
    cnt = change ? 1u : cnt + (act ? 1u : 0u);
  }
  __device__ __forceinline__ void flush(uint32_t* h) {
    if (cnt) atomicAdd(&h[bin >> 1], cnt << ((bin & 1u) << 4));
  }
};

__device__ __forceinline__ uint32_t packed_count(const uint32_t* h, uint32_t bin) {
  return (h[bin >> 1] >> ((bin & 1u) << 4)) & 0xFFFFu;
}

// Block-cooperative search for the bins holding two 0-based ranks.  Thread t
// holds the counts of bins [t * PER, t * PER + PER) of histogram A in cA and of
// histogram B in cB; rank 0 searches A, rank 1 searches A when `one` (both
// ranks share a histogram) and B otherwise.  Gives each rank's bin and the count
// of lower bins; a rank past the end (only when NaNs were left out) gives the
// last bin.  One DPP scan per histogram, three barriers.  Called by all threads.
template <int PER>
__device__ inline void block_find2(const uint32_t* cA, const uint32_t* cB, bool one, const uint32_t resid[2],
                                   uint32_t bin[2], uint32_t below[2], uint32_t* sh, uint32_t* cnt = nullptr,
                                   const uint32_t* expect = nullptr, uint32_t* added = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t sA = 0, sB = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    sA += cA[i];
    sB += cB[i];
  }
  if (one) sB = sA;
  const uint32_t iA = wave_incl_scan(sA);
  const uint32_t iB = one ? iA : wave_incl_scan(sB);
  __syncthreads();
  if (lane == 63) {
    sh[w] = iA;
    sh[kWaves + w] = iB;
  }
  if (tid == 0) {
    sh[8] = sh[10] = PER * kBlock - 1;
    sh[9] = sh[11] = sh[12] = sh[13] = 0;
  }
  __syncthreads();
  uint32_t baseA = 0, baseB = 0;
  for (int i = 0; i < w; ++i) {
    baseA += sh[i];
    baseB += sh[kWaves + i];
  }
  uint32_t eA = baseA + iA - sA, eB = baseB + iB - sB;  // counts of the bins before the thread's
  // expect: totals that A and B must reach (0: none); the shortfall joins bin 0,
  // the first of thread 0, which moves every other thread's bins up by it
  uint32_t zA = 0, zB = 0;
  if (expect) {
    uint32_t tA = 0, tB = 0;
    for (int i = 0; i < kWaves; ++i) {
      tA += sh[i];
      tB += sh[kWaves + i];
    }
    zA = expect[0] ? expect[0] - tA : 0u;
    zB = one ? zA : (expect[1] ? expect[1] - tB : 0u);
    if (added) {
      added[0] = zA;
      added[1] = zB;
    }
    if (tid > 0) {
      eA += zA;
      eB += zB;
    } else {
      sA += zA;
      sB += zB;
    }
  }
  const uint32_t z0A = tid == 0 ? zA : 0u, z0B = tid == 0 ? zB : 0u;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const bool useB = rr == 1 && !one;
    const uint32_t sum = useB ? sB : sA;
    uint32_t e = useB ? eB : eA;
    const uint32_t r = resid[rr];
    if (sum > 0 && e <= r && r < e + sum) {
      uint32_t b = tid * PER, bc = 0;
      bool found = false;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t c = (useB ? cB[i] : cA[i]) + (i == 0 ? (useB ? z0B : z0A) : 0u);
        if (!found && r < e + c) {
          b = tid * PER + i;
          if (cnt) bc = c;
          found = true;
        } else if (!found) {
          e += c;
        }
      }
      sh[8 + 2 * rr] = b;
      sh[9 + 2 * rr] = e;
      if (cnt) sh[12 + rr] = bc;
    }
  }
  __syncthreads();
  bin[0] = sh[8];
  below[0] = sh[9];
  bin[1] = sh[10];
  below[1] = sh[11];
  if (cnt) {
    cnt[0] = sh[12];
    cnt[1] = sh[13];
  }
}

// torch's quantile interpolation between the order statistics (NaN when the
// sample holds a NaN); the near-zero array also gets its sample mean.  Called
// by all threads of the block.
__device__ __forceinline__ void store_p99(kvv_result& res, int arr, const uint32_t key[2], float wgt, bool has_nan) {
  double out = __builtin_nan("");
  if (!has_nan) {
    const float va = fkey_value(key[0]), vb = fkey_value(key[1]);
    // small weights from the lower end, large ones from the upper end, one rounding each
    const float diff = vb - va;
    const float q = fabsf(wgt) < 0.5f ? fmaf(wgt, diff, va) : fmaf(wgt - 1.0f, diff, vb);
    out = (double)q;
  }
  if (arr == 0) res.p99_abs = out;
  else if (arr == 1) res.p99_rel = out;
  else res.near_zero_p99_abs = out;
}

__device__ inline void finalize_group(const TailArgs& a, const SegDesc& d, int arr, int64_t count,
                                      const uint32_t key[2], float wgt, bool has_nan, SelectLds& L) {
  kvv_result& res = a.res[d.out_index];
  const int tid = threadIdx.x;
  if (tid == 0) store_p99(res, arr, key, wgt, has_nan);
  if (arr == 2) {
    // near-zero sample mean: fixed-order sum of the per-item sampled sums, or of
    // the scatter blocks' sums when the sample was built from entries
    double t = 0.0;
    if (d.flags & kFlagNearEntries) {
      for (int k = tid; k < a.scatter_blocks; k += kBlock) t += a.near_psum[k];
    } else {
      const int64_t per = (d.item_count + kBlock - 1) / kBlock;
      const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
      const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
      for (int64_t k = k0; k < k1; ++k) t += a.item_near_sum[d.item_begin + k];
    }
    L.part[tid] = t;
    __syncthreads();
    if (tid == 0) {
      double sum = 0.0;
      for (int i = 0; i < kBlock; ++i) sum += L.part[i];
      res.near_zero_mean_abs = (double)(float)(sum / (double)count);
    }
  }
}

__device__ __forceinline__ uint32_t block_sum_nan(uint32_t v, SelectLds& L) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) L.misc[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += L.misc[i];
  __syncthreads();
  return t;
}

// The keys of the order statistics of ranks rank[0] <= rank[1] among at most
// kSmall values: keys in registers, four 8-bit digit passes over block
// histograms in LDS.  Returns whether a value is NaN (the keys are then not
// searched).  Called by all threads of the block.
__device__ inline bool small_keys(const float* v, int64_t count, const uint32_t rank[2], uint32_t key[2],
                                  SelectLds& L) {
  constexpr int PER = kSmall / kBlock;
  const int tid = threadIdx.x;
  float x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t idx = (int64_t)i * kBlock + tid;
    x[i] = idx < count ? v[idx] : 0.0f;
  }
  uint32_t k[PER];
  uint32_t nans = 0, valid = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t idx = (int64_t)i * kBlock + tid;
    const bool isn = __builtin_isnan(x[i]);
    nans += (idx < count && isn) ? 1u : 0u;
    valid |= (idx < count && !isn ? 1u : 0u) << i;
    k[i] = fkey(x[i]);
  }
  key[0] = key[1] = 0u;
  const bool has_nan = block_sum_nan(nans, L) != 0;
  if (!has_nan) {
    uint32_t resid[2] = {rank[0], rank[1]};
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      const bool same = key[0] == key[1];
      if (tid < 128) L.h[0][tid] = L.h[1][tid] = 0;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const bool ok = (valid >> i) & 1u;
        const uint32_t top = pass == 0 ? 0u : (k[i] >> (shift + 8));
        const uint32_t dig = (k[i] >> shift) & 255u;
        lds_hist_add(L.h[0], dig, ok && top == key[0]);
        if (!same) lds_hist_add(L.h[1], dig, ok && top == key[1]);
      }
      __syncthreads();
      const uint32_t cA = packed_count(L.h[0], tid), cB = packed_count(L.h[1], tid);
      uint32_t bin[2], below[2];
      block_find2<1>(&cA, &cB, same, resid, bin, below, L.sh);
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        key[rr] = (key[rr] << 8) | bin[rr];
        resid[rr] -= below[rr];
      }
    }
  }
  return has_nan;
}

__device__ inline bool range_keys(const float* v, uint32_t count, const uint32_t rank[2], uint32_t key[2],
                                  SelectLds& L);

// A group of at most kSmall samples, selected by one block.
__device__ inline void select_small(const TailArgs& a, const SegDesc& d, int arr, int64_t count, SelectLds& L) {
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  const uint32_t rank[2] = {(uint32_t)rank64[0], (uint32_t)rank64[1]};
  uint32_t key[2];
  const bool has_nan = range_keys(a.arr[arr] + d.sample_off, (uint32_t)count, rank, key, L);
  finalize_group(a, d, arr, count, key, wgt, has_nan, L);
}

// BinRun with full 32-bit counts (a histogram of one bin per word).
struct BinRun32 {
  uint32_t bin = 0, cnt = 0;
  __device__ __forceinline__ void add(uint32_t* h, uint32_t b, bool act) {
    const bool change = act && b != bin;
    if (change && cnt) atomicAdd(&h[bin], cnt);
    bin = change ? b : bin;
    cnt = change ? 1u : cnt + (act ? 1u : 0u);
  }
  __device__ __forceinline__ void flush(uint32_t* h) {
    if (cnt) atomicAdd(&h[bin], cnt);
  }
};

// One digit pass of select_group_stream over the whole group: digit
// (key >> SH) & (2^W - 1) of the values whose bits above SH + W equal the
// rank's prefix (every value at the first pass), counted in 32-bit LDS bins.
template <int SH, int W, bool FIRST>
__device__ inline uint32_t group_pass(const float* v, int64_t count, const uint32_t pfx[2], bool same, SelectLds& L) {
  constexpr int PER = kStreamChunk / kBlock;
  constexpr uint32_t DM = (1u << W) - 1u;
  const int tid = threadIdx.x;
  for (int i = tid; i < 2 * 2048; i += kBlock) (&L.h[0][0])[i] = 0;
  __syncthreads();
  uint32_t nans = 0;
  BinRun32 ra, rb;
  // thread t takes 4 consecutive values of every 4 * kBlock, read with 16-byte loads
  auto load = [&](float (&x)[PER], int64_t c0) {
#pragma unroll
    for (int k = 0; k < PER / 4; ++k) {
      const int64_t i0 = c0 + (int64_t)k * (4 * kBlock) + 4 * tid;
      if (i0 + 3 < count) {
        const float4 q = *reinterpret_cast<const float4*>(v + i0);
        x[4 * k] = q.x;
        x[4 * k + 1] = q.y;
        x[4 * k + 2] = q.z;
        x[4 * k + 3] = q.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) x[4 * k + j] = i0 + j < count ? v[i0 + j] : 0.0f;
      }
    }
  };
  auto count_in = [&](const float (&x)[PER], int64_t c0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t idx = c0 + (int64_t)(i >> 2) * (4 * kBlock) + 4 * tid + (i & 3);
      const bool isn = __builtin_isnan(x[i]);
      const bool ok = idx < count && !isn;
      const uint32_t key = fkey(x[i]);
      const uint32_t dig = (key >> SH) & DM;
      if (FIRST) {
        nans += (idx < count && isn) ? 1u : 0u;
        ra.add(L.h[0], dig, ok);
      } else {
        const uint32_t top = key >> (SH + W);
        ra.add(L.h[0], dig, ok && top == pfx[0]);
        if (!same) rb.add(L.h[1], dig, ok && top == pfx[1]);
      }
    }
  };
  // one buffer: a second one in flight would double the registers (2 blocks per
  // CU instead of 5), and more resident blocks hide the load latency better
  float xa[PER];
#pragma unroll 1
  for (int64_t c0 = 0; c0 < count; c0 += kStreamChunk) {
    load(xa, c0);
    count_in(xa, c0);
  }
  ra.flush(L.h[0]);
  if (!FIRST && !same) rb.flush(L.h[1]);
  __syncthreads();
  return nans;
}

// Folds one pass's histograms into the ranks' prefixes and residual ranks.
template <int W>
__device__ inline void group_pass_ranks(bool same, uint32_t key[2], uint32_t resid[2], SelectLds& L) {
  constexpr int PER = (1 << W) / kBlock;
  const int tid = threadIdx.x;
  uint32_t cA[PER], cB[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    cA[i] = L.h[0][tid * PER + i];
    cB[i] = L.h[1][tid * PER + i];
  }
  uint32_t bin[2], below[2];
  block_find2<PER>(cA, cB, same, resid, bin, below, L.sh);
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    key[rr] = (key[rr] << W) | bin[rr];
    resid[rr] -= below[rr];
  }
  __syncthreads();
}

// The keys of the order statistics of ranks rank[0] <= rank[1] among `count`
// values, found by one block streaming them once per digit (bits 31..21,
// 20..10, 9..0).  Returns whether a value is NaN (the keys are then not
// searched).  Called by all threads of the block.
__device__ inline bool stream_keys(const float* v, int64_t count, const uint32_t rank[2], uint32_t key[2],
                                   SelectLds& L) {
  key[0] = key[1] = 0u;
  uint32_t resid[2] = {rank[0], rank[1]};
  const uint32_t none[2] = {0u, 0u};
  const uint32_t nans = group_pass<21, 11, true>(v, count, none, true, L);
  const bool has_nan = block_sum_nan(nans, L) != 0;
  if (!has_nan) {
    group_pass_ranks<11>(true, key, resid, L);
    bool same = key[0] == key[1];
    group_pass<10, 11, false>(v, count, key, same, L);
    group_pass_ranks<11>(same, key, resid, L);
    same = key[0] == key[1];
    group_pass<0, 10, false>(v, count, key, same, L);
    group_pass_ranks<10>(same, key, resid, L);
  }
  return has_nan;
}

// The keys of the order statistics of ranks rank[0] <= rank[1] among `count`
// values, by radix passes over the values' own key range: the first pass
// bins [min key, max key] into 2048 bins (shifting off the low bits the range
// needs beyond 11), each later pass bins the key range of the rank's bin, down
// to a single key (at most three passes for 32-bit keys).  Values that share a
// narrow range (e.g. the top few percent of a distribution, whose leading key
// bits agree) thus spread over the bins instead of meeting in a few LDS words.
// Values stay in registers when there are at most kSmall of them, else every
// pass reads them again.  Returns whether a value is NaN (the keys are then
// not searched).  Called by all threads of the block.
__device__ inline bool range_keys(const float* v, uint32_t count, const uint32_t rank[2], uint32_t key[2],
                                  SelectLds& L) {
  constexpr int PER = kSmall / kBlock;
  const int tid = threadIdx.x;
  const bool regs = count <= (uint32_t)kSmall;
  uint32_t k[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t idx = (uint32_t)(i * kBlock + tid);
    k[i] = regs && idx < count ? fkey(v[idx]) : 0u;
  }
  // f(key) for every value of this thread
  auto visit = [&](auto&& f) {
    if (regs) {
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if ((uint32_t)(i * kBlock + tid) < count) f(k[i]);
    } else {
      // eight loads in flight per thread
      for (uint32_t i0 = 0; i0 < count; i0 += 8 * kBlock) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t idx = i0 + (uint32_t)(i * kBlock + tid);
          t[i] = idx < count ? v[idx] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i0 + (uint32_t)(i * kBlock + tid) < count) f(fkey(t[i]));
      }
    }
  };
  uint32_t mn = 0xFFFFFFFFu, mx = 0u, nans = 0u, zeros = 0u;
  visit([&](uint32_t kk) {
    mn = kk < mn ? kk : mn;
    mx = kk > mx ? kk : mx;
    nans += kk == 0xFFFFFFFFu ? 1u : 0u;
    zeros += kk == kZeroKey ? 1u : 0u;
  });
  key[0] = key[1] = 0u;
  // NaNs and exact zeros counted together (each at most the block's count, below 2^16 when
  // the values are in registers; else only the NaN count is used)
  const uint32_t nz = block_sum_nan(regs ? nans | (zeros << 16) : nans, L);
  if ((regs ? nz & 0xFFFFu : nz) != 0) return true;
  mn = wave_min(mn);
  mx = wave_max(mx);
  if ((tid & 63) == 0) {
    L.misc[tid >> 6] = mn;
    L.sh[tid >> 6] = mx;
  }
  __syncthreads();
  mn = L.misc[0];
  mx = L.sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    mn = L.misc[w] < mn ? L.misc[w] : mn;
    mx = L.sh[w] > mx ? L.sh[w] : mx;
  }
  __syncthreads();
  // both ranks among the exact zeros, the least values (the p99 of mostly identical pairs): no pass
  if (regs && mn == kZeroKey && rank[1] < (nz >> 16)) {
    key[0] = key[1] = kZeroKey;
    return false;
  }
  uint32_t lo[2] = {mn, mn}, hi[2] = {mx, mx}, resid[2] = {rank[0], rank[1]};
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    if (lo[0] == hi[0] && lo[1] == hi[1]) break;
    const bool same = lo[0] == lo[1] && hi[0] == hi[1];
    int shift[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int bits = 32 - __clz(hi[t] - lo[t]);
      shift[t] = bits > 11 ? bits - 11 : 0;
    }
    for (int i = tid; i < 2 * 2048; i += kBlock) (&L.h[0][0])[i] = 0;
    __syncthreads();
    // a lane's consecutive values of one bin are added once (repeated values,
    // e.g. the zeros of mostly identical data, would serialise on one word)
    uint32_t rb[2] = {0u, 0u}, rn[2] = {0u, 0u};
    visit([&](uint32_t kk) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if ((t == 0 || !same) && lo[t] != hi[t] && kk >= lo[t] && kk <= hi[t]) {
          const uint32_t bin = (kk - lo[t]) >> shift[t];
          if (bin != rb[t]) {
            if (rn[t]) atomicAdd(&L.h[t][rb[t]], rn[t]);
            rb[t] = bin;
            rn[t] = 0;
          }
          ++rn[t];
        }
      }
    });
#pragma unroll
    for (int t = 0; t < 2; ++t)
      if (rn[t]) atomicAdd(&L.h[t][rb[t]], rn[t]);
    __syncthreads();
    uint32_t cA[8], cB[8], bin[2], below[2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      cA[i] = L.h[0][tid * 8 + i];
      cB[i] = L.h[1][tid * 8 + i];
    }
    block_find2<8>(cA, cB, same, resid, bin, below, L.sh);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (lo[t] == hi[t]) continue;
      const uint64_t nlo = (uint64_t)lo[t] + ((uint64_t)bin[t] << shift[t]);
      const uint64_t nhi = nlo + ((uint64_t)1 << shift[t]) - 1;
      lo[t] = (uint32_t)nlo;
      hi[t] = nhi < hi[t] ? (uint32_t)nhi : hi[t];
      resid[t] -= below[t];
    }
    __syncthreads();
  }
  key[0] = lo[0];
  key[1] = lo[1];
  return false;
}

// A whole large group selected by one block (stream_keys).  Used when a launch
// holds enough groups to fill the device by itself: no global histograms, no
// further launches.
__device__ inline void select_group_stream(const TailArgs& a, const SegDesc& d, int arr, int64_t count,
                                           SelectLds& L) {
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  const uint32_t rank[2] = {(uint32_t)rank64[0], (uint32_t)rank64[1]};
  uint32_t key[2];
  const bool has_nan = stream_keys(a.arr[arr] + d.sample_off, count, rank, key, L);
  finalize_group(a, d, arr, count, key, wgt, has_nan, L);
}

// Prefixes and residual ranks of the two order statistics of a large group
// after the digit levels below LEVEL, from the group's global histograms.  All
// histogram words the block needs are loaded in one go.
// zeros_add: values the level-0 histogram does not hold but the array does, all
// +0 (a near-zero sample built from entries: its zeros were never histogrammed).
// zeros (LEVEL 2): the exact zeros under the +0 prefix, which level 1 left out
// of its histograms and candidates: the +0 bin's level-0 count minus the
// level-1 counts under it.  They join digit 0 here, and the final read-off
// adds them to the target group when that is the zeros' group.
// h0pre: the thread's level-0 words (the histogram and its copies), when the
// caller loaded them itself (ahead of its own loads, so they land first).
template <int LEVEL>
__device__ inline void group_state(const uint32_t* slot, const uint64_t rank64[2], uint32_t pfx[2], uint32_t resid[2],
                                   SelectLds& L, uint32_t zeros_add = 0, uint32_t* pfx0 = nullptr,
                                   uint32_t* zeros = nullptr, const uint32_t* h0pre = nullptr) {
  static_assert(LEVEL == 1 || LEVEL == 2, "prefixes after one or two digit levels");
  const int tid = threadIdx.x;
  uint32_t h1a[16], h1b[16];
  uint32_t h0w = (h0pre ? h0pre[0] : slot[kH0 + tid]) + (tid == (int)(0x80000000u >> 24) ? zeros_add : 0u);
#pragma unroll
  for (int r = 0; r < kH0Copies; ++r) h0w += h0pre ? h0pre[r + 1] : slot[kH0R + r * 256 + tid];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (LEVEL >= 2) {
      h1a[i] = slot[kH1 + tid * 16 + i];
      h1b[i] = slot[kH1 + 4096 + tid * 16 + i];
    }
  }
  resid[0] = (uint32_t)rank64[0];
  resid[1] = (uint32_t)rank64[1];
  uint32_t bin[2], below[2], bcnt[2];
  block_find2<1>(&h0w, &h0w, true, resid, bin, below, L.sh, bcnt);
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    pfx[rr] = bin[rr];
    resid[rr] -= below[rr];
    if (pfx0) pfx0[rr] = bin[rr];
  }
  if (LEVEL >= 2) {
    // the level-1 histogram under the +0 prefix must reach that bin's level-0 count
    const bool za = pfx[0] == (kZeroKey >> 24);
    const bool zb = pfx[0] != pfx[1] && pfx[1] == (kZeroKey >> 24);
    const uint32_t expect[2] = {za ? bcnt[0] : 0u, zb ? bcnt[1] : 0u};
    uint32_t added[2];
    block_find2<16>(h1a, h1b, pfx[0] == pfx[1], resid, bin, below, L.sh, nullptr, expect, added);
    if (zeros) *zeros = za ? added[0] : added[1];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      pfx[rr] = (pfx[rr] << 12) | bin[rr];
      resid[rr] -= below[rr];
    }
  }
}

// The near-zero sample's implicit zeros when it was built from entries: its
// values minus the sampled entries the scatter counted (slot word kMisc + 1).
__device__ __forceinline__ uint32_t entry_zeros(const SegDesc& d, int arr, int64_t count, const uint32_t* slot) {
  if (arr != 2 || !(d.flags & kFlagNearEntries)) return 0u;
  return (uint32_t)(count - (int64_t)slot[kMisc + 1]);
}

// Exclusive prefix, in place, of a packed block histogram of `nwords` words
// (two 16-bit counts each, nwords a multiple of kBlock): afterwards each half
// holds the number of values in lower bins.  Returns the total.  Called by all
// threads of the block.
__device__ inline uint32_t block_offsets16(uint32_t* h, int nwords, SelectLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int per = nwords / kBlock;  // consecutive words per thread (8 or 16)
  uint32_t sum = 0;
  for (int k = 0; k < per; ++k) {
    const uint32_t v = h[tid * per + k];
    sum += (v & 0xFFFFu) + (v >> 16);
  }
  const uint32_t incl = wave_incl_scan(sum);
  __syncthreads();
  if (lane == 63) L.misc[w] = incl;
  __syncthreads();
  uint32_t base = incl - sum;
  for (int i = 0; i < w; ++i) base += L.misc[i];
  const uint32_t total = L.misc[0] + L.misc[1] + L.misc[2] + L.misc[3];
  for (int k = 0; k < per; ++k) {
    const uint32_t v = h[tid * per + k];
    const uint32_t lo = base, hi = base + (v & 0xFFFFu);
    base = hi + (v >> 16);
    h[tid * per + k] = lo | (hi << 16);
  }
  __syncthreads();
  return total;
}

// One chunk of a large group at digit level LEVEL: 0 = bits 31..24 of every
// value, 1 = bits 23..12 of the values under either rank's level-0 prefix,
// whose keys are then kept, grouped by (rank, level-1 digit), in the round's
// own span of the sample array (its values are all in registers by then) with
// the round's table of group starts.  The chunk is d.sel_rounds consecutive
// rounds of kSelChunk samples, each read with 16-byte loads (thread t takes 4
// consecutive values of every 4 * kBlock).  Level 0 histograms the rounds into
// one block histogram added to the group's once; level 1 adds each round's.
template <int LEVEL>
__device__ inline void select_chunk(const TailArgs& a, const SegDesc& d, int arr, int64_t count, int64_t c,
                                    SelectLds& L) {
  static_assert(LEVEL == 0 || LEVEL == 1, "two histogram levels");
  constexpr int PER = kSelChunk / kBlock;  // values per thread and round
  constexpr int NV = PER / 4;
  constexpr int DS = LEVEL == 0 ? 24 : 12;               // digit = (key >> DS) & DM
  constexpr uint32_t DM = LEVEL == 0 ? 255u : 4095u;
  const int tid = threadIdx.x;
  const int rounds = d.sel_rounds;
  uint32_t* slot = a.slots + ((size_t)d.lslot * kArrays + arr) * kSlotWords;
  float* v = const_cast<float*>(a.arr[arr]) + d.sample_off;
  auto load_round = [&](float (&x)[PER], int64_t c0, int64_t c1) {
    if (c1 - c0 == kSelChunk) {
      // a full round (every round but a group's last): only 16-byte loads, all
      // in flight together.  (With the partial form's element loads in the same
      // code, each 16-byte load waited for the one before: their registers are shared.)
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const float4 q = *reinterpret_cast<const float4*>(v + c0 + (int64_t)k * (4 * kBlock) + 4 * tid);
        x[4 * k] = q.x;
        x[4 * k + 1] = q.y;
        x[4 * k + 2] = q.z;
        x[4 * k + 3] = q.w;
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t i0 = c0 + (int64_t)k * (4 * kBlock) + 4 * tid;
      if (i0 + 3 < c1) {
        const float4 q = *reinterpret_cast<const float4*>(v + i0);
        x[4 * k] = q.x;
        x[4 * k + 1] = q.y;
        x[4 * k + 2] = q.z;
        x[4 * k + 3] = q.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) x[4 * k + j] = i0 + j < c1 ? v[i0 + j] : 0.0f;
      }
    }
  };
  // level 1: the group's state words are loaded first, then the first round's
  // values, so the state (its sums and block scans) is worked out while the
  // values are still in flight
  uint32_t h0v[kH0Copies + 1];
  uint32_t nan_count = 0, zadd = 0;
  if (LEVEL == 1) {
    nan_count = slot[kMisc];
    zadd = entry_zeros(d, arr, count, slot);
    h0v[0] = slot[kH0 + tid];
#pragma unroll
    for (int r = 0; r < kH0Copies; ++r) h0v[r + 1] = slot[kH0R + r * 256 + tid];
    asm volatile("" ::: "memory");  // (keeps the value loads below behind these)
  }
  int64_t c0 = c * rounds * (int64_t)kSelChunk;
  int64_t c1 = c0 + kSelChunk < count ? c0 + kSelChunk : count;
  float x[PER];
  load_round(x, c0, c1);
  uint32_t pfx[2] = {0u, 0u};
  bool same = true;
  if (LEVEL == 1) {
    uint64_t rank64[2];
    float wgt;
    q99_ranks(count, rank64, wgt);
    uint32_t resid[2];
    group_state<1>(slot, rank64, pfx, resid, L, zadd, nullptr, nullptr, h0v);
    // a NaN among the samples makes the quantile NaN: nothing to locate (the final read-off checks the same count)
    if (nan_count != 0) return;
    same = pfx[0] == pfx[1];
  }
  // the keys under each rank's 8-bit prefix, [lo, lo + span); the +0 prefix
  // leaves out the exact zeros (identical pairs): the final read-off takes their
  // count from the two histograms instead of keeping them as candidates
  const uint32_t lo0 = (pfx[0] << 24) + (pfx[0] == (kZeroKey >> 24) ? 1u : 0u);
  const uint32_t lo1 = (pfx[1] << 24) + (pfx[1] == (kZeroKey >> 24) ? 1u : 0u);
  const uint32_t span0 = (1u << 24) - (lo0 & 1u), span1 = (1u << 24) - (lo1 & 1u);
  // level 1: bins (rank, digit), the second rank's 4096 only when its prefix differs
  const int nwords = LEVEL == 0 ? 128 : (same ? 2048 : 4096);
  uint32_t* h = &L.h[0][0];
  // level 1: each wave's kept keys of the round (at most its PER * 64 values),
  // then a spare word per lane; the round's cell bounds
  uint32_t* klist = nullptr;
  uint32_t *cmin = nullptr, *cmax = nullptr;
  if constexpr (LEVEL == 1) {
    __shared__ uint32_t kl[kWaves][PER * 64 + 64];
    __shared__ uint32_t cb[2][kCells];
    klist = kl[tid >> 6];
    cmin = cb[0];
    cmax = cb[1];
  }
  if (LEVEL == 0) {
    for (int i = tid; i < nwords; i += kBlock) h[i] = 0;
    __syncthreads();
  }
  uint32_t nans = 0;
  BinRun run0;
#pragma unroll 1
  for (int r = 0; r < rounds; ++r) {
    if (r > 0) {
      c0 = (c * rounds + r) * (int64_t)kSelChunk;
      if (c0 >= count) break;
      c1 = c0 + kSelChunk < count ? c0 + kSelChunk : count;
      load_round(x, c0, c1);
    }
    if (LEVEL == 1) {
      for (int i = tid; i < nwords; i += kBlock) h[i] = 0;
      __syncthreads();
    }
    uint32_t keep = 0;
    // position i of the thread lies inside the round when its offset in the round is below lim
    const int lim = (int)(c1 - c0) - 4 * tid;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const bool in = (i >> 2) * (4 * kBlock) + (i & 3) < lim;
      const uint32_t key = fkey(x[i]);
      if (LEVEL == 0) {
        const bool isn = __builtin_isnan(x[i]);
        nans += in && isn ? 1u : 0u;
        run0.add(h, (key >> DS) & DM, in && !isn);
      } else {
        // under a rank's prefix: key - lo < span (exact zeros left out of the +0
        // prefix); no NaN reaches level 1 (a NaN count returns above)
        const bool m0 = key - lo0 < span0;
        const bool m1 = !same && key - lo1 < span1;
        keep |= (in && (m0 || m1) ? 1u : 0u) << i;
      }
    }
    uint32_t wkept = 0;
    if (LEVEL == 1) {
      // the wave's kept keys, compacted in lane order into its LDS list; the
      // histogram and the scatter below then run over the list, every lane busy
      // (a walk over each thread's 32 values left most lanes idle)
      const uint32_t nk = (uint32_t)__popc(keep);
      const uint32_t incl = wave_incl_scan(nk);
      wkept = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
      // (branch-free: a value that is not kept goes to the lane's spare word)
      const uint32_t spare = PER * 64 + (uint32_t)(tid & 63);
      uint32_t o = incl - nk;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t b = (keep >> i) & 1u;
        klist[b ? o : spare] = fkey(x[i]);
        o += b;
      }
      __builtin_amdgcn_wave_barrier();
      for (uint32_t e = (uint32_t)(tid & 63); e < wkept; e += 64) {
        const uint32_t key = klist[e];
        lds_hist_add(h, ((key >> 24) == pfx[0] ? 0u : 4096u) | ((key >> 12) & 4095u), true);
      }
      __syncthreads();
      // this round's histogram joins the group's
      for (int i = tid; i < nwords; i += kBlock) {
        const uint32_t wv = h[i];
        uint32_t* dst = slot + kH1 + 2 * i;  // rank 1's bins follow rank 0's (words 2048.. -> bins 4096..)
        if (wv & 0xFFFFu) atomicAdd(dst, wv & 0xFFFFu);
        if (wv >> 16) atomicAdd(dst + 1, wv >> 16);
      }
      __syncthreads();
      // the kept keys, grouped by bin, into the round's span of the sample array
      const uint32_t total = block_offsets16(h, nwords, L);
      const int64_t sub = (d.chunk_begin + c) * (int64_t)rounds + r;
      uint16_t* tab = a.subtab + ((size_t)arr * a.total_sub + (size_t)sub) * kSubTab;
      for (int i = tid; i <= kCells; i += kBlock) {
        const int bin = i << kCellShift;
        tab[i] = (uint16_t)(bin < 2 * nwords ? (h[bin >> 1] & 0xFFFFu) : total);
      }
      // the smallest and largest kept key of each cell
      for (int i = tid; i < kCells; i += kBlock) {
        cmin[i] = 0xFFFFFFFFu;
        cmax[i] = 0u;
      }
      __syncthreads();  // (the offsets are read before the scatter advances them)
      uint32_t* out = reinterpret_cast<uint32_t*>(v + c0);
      for (uint32_t e = (uint32_t)(tid & 63); e < wkept; e += 64) {
        const uint32_t key = klist[e];
        const uint32_t bin = ((key >> 24) == pfx[0] ? 0u : 4096u) | ((key >> 12) & 4095u);
        const uint32_t sh = (bin & 1u) << 4;
        const uint32_t old = atomicAdd(&h[bin >> 1], 1u << sh);
        out[(old >> sh) & 0xFFFFu] = key;
        atomicMin(&cmin[bin >> kCellShift], key);
        atomicMax(&cmax[bin >> kCellShift], key);
      }
      __syncthreads();
      uint2* mm = reinterpret_cast<uint2*>(a.submm + ((size_t)arr * a.total_sub + (size_t)sub) * kSubMM);
      for (int i = tid; i < kCells; i += kBlock) mm[i] = make_uint2(cmin[i], cmax[i]);
    }
  }
  if (LEVEL == 0) {
    run0.flush(h);
    nans = block_sum_nan(nans, L);
    __syncthreads();
    // add the block histogram to the group's: bins 2w and 2w+1 of word w
    for (int i = tid; i < nwords; i += kBlock) {
      const uint32_t wv = h[i];
      uint32_t* dst = slot + kH0 + 2 * i;
      if (wv & 0xFFFFu) atomicAdd(dst, wv & 0xFFFFu);
      if (wv >> 16) atomicAdd(dst + 1, wv >> 16);
    }
    if (tid == 0 && nans) atomicAdd(&slot[kMisc], nans);
  }
}

// The final read-off of a large group (one block): the 20-bit prefixes and
// residual ranks from the group's two histograms, then the last 12 bits from
// the kept keys of the target (rank, level-1 digit) groups only: each round's
// table bounds the cell of 8 groups around the target (when the cell holds a
// single value over all rounds, that value is the key and nothing is read),
// a block prefix over the rounds
// spreads those keys over all threads, and the keys under the prefix are
// counted in LDS (per-thread run merging: the target often holds one repeated
// value).  Ranks under different prefixes take one pass each.
__device__ inline void select_final(const TailArgs& a, const SegDesc& d, int arr, int64_t count, SelectLds& L) {
  const int tid = threadIdx.x;
  const uint32_t* slot = a.slots + ((size_t)d.lslot * kArrays + arr) * kSlotWords;
  const bool has_nan = slot[kMisc] != 0;
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  uint32_t pfx[2], resid[2], p0[2], zeros;
  group_state<2>(slot, rank64, pfx, resid, L, entry_zeros(d, arr, count, slot), p0, &zeros);
  uint32_t key0 = 0u, key1 = 0u;
  if (!has_nan) {
    const int rounds = d.sel_rounds;
    const int64_t nsub = (count + kSelChunk - 1) / kSelChunk;
    const uint16_t* tab0 = a.subtab + ((size_t)arr * a.total_sub + (size_t)d.chunk_begin * rounds) * kSubTab;
    const uint32_t* keys = reinterpret_cast<const uint32_t*>(a.arr[arr] + d.sample_off);
    uint32_t* H = &L.h[0][0];                              // 4096 bins, one per word
    uint32_t* pre = reinterpret_cast<uint32_t*>(L.part);   // round prefix (256 + 1) and starts (255)
    uint32_t* beg = pre + 257;
    const int passes = pfx[0] == pfx[1] ? 1 : 2;
#pragma unroll 1
    for (int rr = 0; rr < passes; ++rr) {
      for (int i = tid; i < 4096; i += kBlock) H[i] = 0;
      const uint32_t pr = rr == 0 ? pfx[0] : pfx[1];
      const uint32_t group = (p0[0] != p0[1] && rr == 1 ? 4096u : 0u) | (pr & 4095u);
      const int cell = (int)(group >> kCellShift);
      // one value throughout the target's cell (e.g. equal power-of-two steps): that is the key
      const uint32_t* mm0 = a.submm + ((size_t)arr * a.total_sub + (size_t)d.chunk_begin * rounds) * kSubMM;
      uint32_t lo_key = 0xFFFFFFFFu, hi_key = 0u;
      for (int64_t k = tid; k < nsub; k += kBlock) {
        const uint2 b = *reinterpret_cast<const uint2*>(mm0 + (size_t)k * kSubMM + 2 * cell);
        const uint32_t a0 = b.x, a1 = b.y;
        lo_key = a0 < lo_key ? a0 : lo_key;
        hi_key = a1 > hi_key ? a1 : hi_key;
      }
      lo_key = wave_min(lo_key);
      hi_key = wave_max(hi_key);
      __syncthreads();
      if ((tid & 63) == 0) {
        L.misc[tid >> 6] = lo_key;
        L.sh[tid >> 6] = hi_key;
      }
      __syncthreads();
      for (int w = 0; w < kWaves; ++w) {
        lo_key = L.misc[w] < lo_key ? L.misc[w] : lo_key;
        hi_key = L.sh[w] > hi_key ? L.sh[w] : hi_key;
      }
      const bool zg = zeros != 0u && pr == (kZeroKey >> 12);  // the target group holds the zeros
      if (zg) {
        lo_key = kZeroKey < lo_key ? kZeroKey : lo_key;
        hi_key = kZeroKey > hi_key ? kZeroKey : hi_key;
      }
      __syncthreads();
      if (lo_key == hi_key) {
        if (passes == 1 || rr == 0) key0 = lo_key;
        if (passes == 1 || rr == 1) key1 = lo_key;
        continue;
      }
      BinRun32 run;
#pragma unroll 1
      for (int64_t s0 = 0; s0 < nsub; s0 += 255) {
        const int nb = nsub - s0 < 255 ? (int)(nsub - s0) : 255;
        uint32_t lo = 0, len = 0;
        if (tid < nb) {
          const uint16_t* t = tab0 + (size_t)(s0 + tid) * kSubTab;
          // the round's own span bounds every read below, whatever the table holds
          const CellSpan cs = cell_span(t[cell], t[cell + 1], count, s0 + tid, kSelChunk);
          lo = cs.lo;
          len = cs.len;
        }
        const uint32_t incl = wave_incl_scan(len);
        __syncthreads();  // (pre/beg of the previous batch are read)
        if ((tid & 63) == 63) L.misc[tid >> 6] = incl;
        __syncthreads();
        uint32_t base = incl - len;
        for (int w = 0; w < (tid >> 6); ++w) base += L.misc[w];
        if (tid < nb) {
          pre[tid] = base;
          beg[tid] = lo;
        }
        if (tid == 0) pre[nb] = L.misc[0] + L.misc[1] + L.misc[2] + L.misc[3];
        __syncthreads();
        const uint32_t total = pre[nb];
        // 8 positions per thread at a time: their loads are all in flight together
#pragma unroll 1
        for (uint32_t f0 = 0; f0 < total; f0 += 8 * kBlock) {
          uint32_t kk[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const uint32_t f = f0 + (uint32_t)(u * kBlock + tid);
            kk[u] = 0u;
            if (f < total) {
              int lo_k = 0, hi_k = nb - 1;  // the round holding flat position f: pre[k] <= f < pre[k + 1]
              while (lo_k < hi_k) {
                const int mid = (lo_k + hi_k + 1) >> 1;
                if (pre[mid] <= f) lo_k = mid; else hi_k = mid - 1;
              }
              kk[u] = keys[(size_t)(s0 + lo_k) * kSelChunk + beg[lo_k] + (f - pre[lo_k])];
            }
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const uint32_t f = f0 + (uint32_t)(u * kBlock + tid);
            run.add(H, kk[u] & 4095u, f < total && (kk[u] >> 12) == pr);
          }
        }
      }
      run.flush(H);
      if (zg && tid == 0) atomicAdd(&H[0], zeros);
      __syncthreads();
      uint32_t hc[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) hc[i] = H[tid * 16 + i];
      const uint32_t r_this = rr == 0 ? resid[0] : resid[1];
      uint32_t rs[2] = {r_this, passes == 1 ? resid[1] : r_this};
      uint32_t bin[2], below[2];
      block_find2<16>(hc, hc, true, rs, bin, below, L.sh);
      if (passes == 1) {
        key0 = (pfx[0] << 12) | bin[0];
        key1 = (pfx[1] << 12) | bin[1];
      } else if (rr == 0) {
        key0 = (pfx[0] << 12) | bin[0];
      } else {
        key1 = (pfx[1] << 12) | bin[0];
      }
      __syncthreads();
    }
  }
  const uint32_t key[2] = {key0, key1};
  finalize_group(a, d, arr, count, key, wgt, has_nan, L);
  // this block was the slot's last reader: it leaves the slot clear for the next
  // call on the workspace (KVV_FLAG_WS_KEPT skips the clearing launch then)
  __syncthreads();
  uint4* z = reinterpret_cast<uint4*>(const_cast<uint32_t*>(slot));
  for (int i = tid; i < kSlotWords / 4; i += kBlock) z[i] = make_uint4(0u, 0u, 0u, 0u);
}

// ------------------------------------------------------------ near-zero entries
// Where a sampled near-zero value goes: the near-zero sample (GCR:525-529 samples
// the compacted array abs_diff[|ref| <= near_zero_abs] with the stride
// i*(c-1)//(m-1) of GCR:346-347, or takes every rank when c <= max_samples).
// The main pass zeroed the sample, so only nonzero values (NaN included) are
// placed: the near-zero elements without one are its zeros.  Each placed value
// joins the block's level-0 histogram (an LDS 256-bin histogram), its count,
// NaN count and fp64 sum.
struct NearPlace {
  uint64_t c, m, num, den;
  bool strided;
  float* sample;
  uint32_t* hist;  // LDS, 256 bins; null when the near-zero sample is a small group
  double sum;
  uint32_t cnt, nan;

  // Rank j (0-based, in the compacted array) holding value v.
  __device__ __forceinline__ void put(uint64_t j, float v) {
    uint64_t i = j;
    bool take = j < c;
    if (strided) {
      // the first sample index i with i*(c-1) >= j*(m-1); rank j is sampled when
      // i*(c-1) < (j+1)*(m-1) too (then floor(i*(c-1)/(m-1)) == j).  The
      // estimate from doubles is off by at most one.
      const uint64_t t = j * den;
      i = (uint64_t)((double)t * (1.0 / (double)num));
      if (i * num < t) ++i;
      if (i > 0 && (i - 1) * num >= t) --i;
      if (i * num < t) ++i;
      take = i < m && i * num < t + den;
    }
    if (take) {
      sample[i] = v;
      sum += (double)v;
      ++cnt;
      if (v != v) ++nan;
      else if (hist) atomicAdd(&hist[fkey(v) >> 24], 1u);
    }
  }
};

// A wave whose entries did not fit its share of the pool: its items are read
// again (one item per block iteration, thread t taking the 8 consecutive
// elements 8t..8t+7 of the item, so thread order is row-major order) and every
// near-zero element at a sampled rank with a nonzero abs_diff is placed.
// `base` is the number of near-zero elements before the wave.  Called by all
// threads of the block; fp16/bf16 single pairs of a vector layout only.
__device__ inline void near_refill(const TailArgs& a, const SegDesc& d, int w, uint64_t base, NearPlace& np,
                                   SelectLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint2 wr = a.wave_range[w];
  const bool bf = d.dtype == KVV_BF16;
  auto f32 = [bf](uint32_t code) -> float {
    return bf ? __uint_as_float(code << 16) : Elem<KVV_F16>::f32((uint16_t)code);
  };
#pragma unroll 1
  for (uint32_t it = wr.x; it < wr.y; ++it) {
    const int64_t L0 = (int64_t)it * d.item_elems;
    const int64_t L1 = L0 + d.item_elems < d.n ? L0 + d.item_elems : d.n;
    const int64_t e0 = L0 + 8 * (int64_t)tid;
    const int ne = e0 >= L1 ? 0 : (L1 - e0 >= 8 ? 8 : (int)(L1 - e0));
    uint32_t gq[4] = {0u, 0u, 0u, 0u}, rq[4] = {0u, 0u, 0u, 0u};
    if (ne > 0) {
      int64_t og, orr;
      elem_offsets(d, e0, og, orr);  // a vector layout: 8 consecutive elements never cross a row
      const uint16_t* gp = reinterpret_cast<const uint16_t*>(d.g) + og;
      const uint16_t* rp = reinterpret_cast<const uint16_t*>(d.r) + orr;
      if (ne == 8) {
        const uint4 x = nt_load16(gp), y = nt_load16(rp);
        gq[0] = x.x; gq[1] = x.y; gq[2] = x.z; gq[3] = x.w;
        rq[0] = y.x; rq[1] = y.y; rq[2] = y.z; rq[3] = y.w;
      } else {
        for (int k = 0; k < ne; ++k) {
          gq[k >> 1] |= (uint32_t)gp[k] << ((k & 1) * 16);
          rq[k >> 1] |= (uint32_t)rp[k] << ((k & 1) * 16);
        }
      }
    }
    uint32_t mask = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float rf = f32((rq[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu);
      mask |= (k < ne && fabsf(rf) <= d.nz_abs ? 1u : 0u) << k;
    }
    // exclusive block prefix of the threads' near-zero counts (row-major ranks)
    const uint32_t cntt = (uint32_t)__popc(mask);
    const uint32_t incl = wave_incl_scan(cntt);
    __syncthreads();  // (the previous item's totals are read)
    if (lane == 63) L.misc[wv] = incl;
    __syncthreads();
    uint32_t before = incl - cntt;
    for (int q = 0; q < wv; ++q) before += L.misc[q];
    const uint32_t total = L.misc[0] + L.misc[1] + L.misc[2] + L.misc[3];
    uint64_t j = base + before;
    while (mask) {
      const int k = __builtin_ctz(mask);
      mask &= mask - 1;
      const float gf = f32((gq[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu);
      const float rf = f32((rq[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu);
      const float adf = fabsf(gf - rf);
      if (!(adf == 0.0f)) np.put(j, adf);
      ++j;
    }
    base += total;
  }
}

// Scatter block b of the first tail launch (a single pair with
// kFlagNearEntries) handles waves [w0, w1): the entries of each wave get their
// rank in the compacted near-zero array (GCR:525-529: abs_diff over |ref| <=
// near_zero_abs, row-major) -- the near-zero elements before the wave plus the
// entry's rank within it -- and are placed (NearPlace); a wave whose entries did
// not fit is read again (near_refill).  The block adds its placed values'
// histogram to copy b mod 16 of the near-zero sample's level-0 histogram (the
// zeros join when the next level reads it), their count and NaN count to the
// slot, and leaves their fp64 sum for the mean.
__device__ inline void near_scatter(const TailArgs& a, int b, SelectLds& L) {
  const SegDesc& d = a.seg0;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nw = a.nwaves;
  const int per = (nw + a.scatter_blocks - 1) / a.scatter_blocks;
  const int w0 = b * per < nw ? b * per : nw;
  const int w1 = w0 + per < nw ? w0 + per : nw;
  // the near-zero count c, and the near-zero elements of the waves before w0: the
  // per-wave counts in 16-byte loads, all of a thread's in flight at once (the
  // array holds 256-byte aligned words; a partial last vector is read by element)
  uint64_t tot = 0, before = 0;
  {
    constexpr int kQ = 4;  // 16-byte loads per thread and pass: 4 x 256 x 4 = 4096 waves
    const uint4* q = reinterpret_cast<const uint4*>(a.near_wave);
    const int nq = nw >> 2;
#pragma unroll 1
    for (int v0 = tid; v0 < nq; v0 += kQ * kBlock) {
      uint4 x[kQ];
#pragma unroll
      for (int k = 0; k < kQ; ++k) x[k] = v0 + k * kBlock < nq ? q[v0 + k * kBlock] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int k = 0; k < kQ; ++k) {
        const int w = 4 * (v0 + k * kBlock);
        const uint32_t e[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tot += e[j];
          before += w + j < w0 ? e[j] : 0u;
        }
      }
    }
    for (int w = 4 * nq + tid; w < nw; w += kBlock) {
      const uint64_t x = a.near_wave[w];
      tot += x;
      before += w < w0 ? x : 0u;
    }
  }
  tot = wave_sum(tot);
  before = wave_sum(before);
  uint64_t* red = reinterpret_cast<uint64_t*>(L.part);
  if (lane == 0) {
    red[wv] = tot;
    red[kWaves + wv] = before;
  }
  for (int i = tid; i < 256; i += kBlock) L.h[0][i] = 0;
  __syncthreads();
  uint64_t c = 0, base = 0;
  for (int i = 0; i < kWaves; ++i) {
    c += red[i];
    base += red[kWaves + i];
  }
  const uint64_t ms = (uint64_t)d.max_samples;
  const uint64_t m = c < ms ? c : ms;
  if (b == 0 && tid == 0) {
    // the near-zero count and sample count, for the selection's launches
    a.near_cm[0] = c;
    a.near_cm[1] = m;
  }
  NearPlace np;
  np.c = c;
  np.m = m;
  np.strided = c > ms;
  np.num = np.strided ? c - 1 : 1;
  np.den = np.strided ? m - 1 : 1;
  np.sample = const_cast<float*>(a.arr[2]) + d.sample_off;
  // the near-zero sample's slot is used only when that sample itself is a large
  // group: a group of at most kSmall values is selected by select_small straight
  // from the array, and only select_final (large groups) clears the slot again,
  // which a kept workspace relies on
  const bool large = d.lslot >= 0 && m > (uint64_t)kSmall;
  uint32_t* slot = large ? a.slots + ((size_t)d.lslot * kArrays + 2) * kSlotWords : nullptr;
  np.hist = large ? &L.h[0][0] : nullptr;
  np.sum = 0.0;
  np.cnt = np.nan = 0;
#pragma unroll 1
  for (int w = w0; w < w1; ++w) {
    const uint32_t fill = a.ent_fill[w];
    if (fill == kNone32) {
      near_refill(a, d, w, base, np, L);
    } else {
      // the wave's entries, 8 per thread per pass with their loads in flight together
      const uint2* ent = a.ent + (size_t)w * a.ent_quota;
      constexpr int kEnt = 8;
#pragma unroll 1
      for (uint32_t k0 = tid; k0 < fill; k0 += kEnt * kBlock) {
        uint2 xs[kEnt];
#pragma unroll
        for (int u = 0; u < kEnt; ++u) {
          const uint32_t k = k0 + (uint32_t)u * kBlock;
          xs[u] = k < fill ? ent[k] : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kEnt; ++u)
          if (k0 + (uint32_t)u * kBlock < fill) np.put(base + xs[u].x, __uint_as_float(xs[u].y));
      }
    }
    base += a.near_wave[w];
  }
  const double sum = wave_sum(np.sum);
  const uint32_t cnt = wave_sum(np.cnt), nan = wave_sum(np.nan);
  __syncthreads();  // (the rank bases in L.part and the refill's L.misc are read)
  if (lane == 0) {
    L.part[wv] = sum;
    L.sh[wv] = cnt;
    L.sh[kWaves + wv] = nan;
  }
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
    for (int i = 0; i < kWaves; ++i) t += L.part[i];
    a.near_psum[b] = t;
    uint32_t tc = 0, tn = 0;
    for (int i = 0; i < kWaves; ++i) {
      tc += L.sh[i];
      tn += L.sh[kWaves + i];
    }
    if (large && tc) atomicAdd(&slot[kMisc + 1], tc);
    if (large && tn) atomicAdd(&slot[kMisc], tn);
  }
  if (large) {
    // copy b mod 16: thousands of scatter blocks would otherwise serialise on the busiest bins
    uint32_t* h0 = slot + kH0R + (b % kH0Copies) * 256;
    for (int i = tid; i < 256; i += kBlock)
      if (L.h[0][i]) atomicAdd(&h0[i], L.h[0][i]);
  }
}

#ifdef KVV_COMMON_KERNELS
// Clears n4 16-byte words (the select slots of a single pair whose main pass
// adds into them); a kernel rather than a memset, so a captured graph replays it.
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(uint4* p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kBlock)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The near-zero entries of a single pair (kFlagNearEntries), placed by their own
// launch between the main pass and the first tail launch: block b handles its
// run of waves (near_scatter); block 0 also leaves the near-zero count and
// sample count for the selection that follows (the fold writes the same values).
// Its few registers let many blocks share a CU: the work is latency-bound loads.
__global__ __launch_bounds__(kBlock) void near_scatter_kernel(TailArgs a) {
  __shared__ SelectLds lds;
  near_scatter(a, (int)blockIdx.x, lds);
}

// LEVEL 0: the first launch: leading blocks fold run records, the others run
// select level 0 and select small groups.  LEVEL 3: the first launch of a
// single pair whose main pass did level 0 of its abs/rel samples
// (kFlagMainHist): as LEVEL 0, with select level 1 for its large groups.  LEVEL 1: select level 1.  LEVEL 2: the final
// read-off, by the first chunk block of each large group.
// "Level" 4 selects the large groups of a many-group launch (select_group_stream).
// BATCH: the segments come from the device table; otherwise the single pair's
// descriptor is a kernel argument, read with scalar loads.
template <int LEVEL, bool BATCH>
__global__ __launch_bounds__(kBlock) void tail_kernel(TailArgs a) {
  __shared__ TailLds lds;
  constexpr bool kFirst = LEVEL == 0 || LEVEL == 3;
  const int64_t b = blockIdx.x;
  if (kFirst && b < a.reduce_blocks) {
    if (a.reduce_roles == 0) {
      // (batches of few runs per segment: a wave per segment)
      const int seg = (int)b * kWaves + (int)(threadIdx.x >> 6);
      if (seg < a.nseg) reduce_segment_wave<BATCH>(a, seg);
    } else {
      reduce_segment<BATCH>(a, (int)(b / a.reduce_roles), (int)(b % a.reduce_roles), lds.r);
    }
    return;
  }
  const int64_t sb = b - a.reduce_blocks;
  const int arr = a.arr_lo + (int)(sb / a.total_chunks);
  const int64_t chunk = sb - (int64_t)(arr - a.arr_lo) * a.total_chunks;
  const int s = BATCH ? (int)a.chunk_seg[chunk] : 0;
  const SegDesc& d = BATCH ? a.table[s] : a.seg0;
  const int64_t count = group_count(a, d, s, arr);
  const int64_t c = chunk - d.chunk_begin;
  if (count <= 0) return;
  if (LEVEL == 4) {
    // many-group launches: a large group without global histograms, one block
    // (abs/rel of an input-select segment are selected by the isel_* kernels)
    if (arr < 2 && (d.flags & kFlagInputSelect)) return;
    if (count > kSmall && d.lslot < 0 && c == 0) select_group_stream(a, d, arr, count, lds.s);
    return;
  }
  if (count <= kSmall || d.lslot < 0) {
    if (kFirst && c == 0 && count <= kSmall) select_small(a, d, arr, count, lds.s);
    return;
  }
  if constexpr (LEVEL == 0) {
    // (a near-zero sample built from entries had its level 0 from near_scatter_kernel)
    if (arr == 2 && (d.flags & kFlagNearEntries)) return;
    if (c * d.sel_rounds * (int64_t)kSelChunk >= count) return;
    select_chunk<0>(a, d, arr, count, c, lds.s);
  } else if constexpr (LEVEL == 1 || LEVEL == 3) {
    if (c * d.sel_rounds * (int64_t)kSelChunk >= count) return;
    select_chunk<1>(a, d, arr, count, c, lds.s);
  } else if constexpr (LEVEL == 2) {
    if (c == 0) select_final(a, d, arr, count, lds.s);
  }
}
#endif  // KVV_COMMON_KERNELS
