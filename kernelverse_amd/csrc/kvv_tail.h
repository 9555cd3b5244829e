// Launches after the main pass (included by kvv_kernels.h, namespace kvv):
//
//   * the fold of a segment's run records into its kvv_result, in a fixed
//     order (bit-reproducible fp64 sums);
//   * the exact order statistics of torch.quantile(q=0.99) over the strided
//     sample arrays (abs_diff, rel_diff and, for the tolerant policy, the
//     near-zero abs_diff), GCR:318-343 and GCR:525-548.
//
// One kernel, tail_kernel, plays both roles: its first `reduce_blocks` blocks
// fold run records (one segment each), the others select.  A (segment, array)
// group of at most kSmall samples is selected by one block entirely in
// registers and LDS (4 digit passes of 8 bits).  A larger group is selected by
// all of its chunk blocks in three launches, one per digit level of the
// ordering key: bits 31..24, 23..12 and 11..0.  Each level histograms, in LDS,
// the digit of the values whose higher digits match the prefix found so far,
// and adds the block histogram to the group's global histogram; the next
// level's blocks locate the ranks in it.  A fourth launch (one block per large
// group) reads the full keys off the three histograms, interpolates like
// torch.quantile and writes the result.  The main pass cleared the histograms.

struct TailArgs {
  SegDesc seg0;               // the segment when table == nullptr
  const SegDesc* table;
  const int64_t* chunk_seg;   // batch: owning segment of each select chunk
  int32_t nseg;
  int32_t reduce_blocks;      // leading blocks that fold run records (one per segment), 0 for none
  int32_t level;              // select digit level 0, 1 or 2 (small groups are done at level 0)
  int32_t arr_lo;             // select blocks cover arrays [arr_lo, arr_lo + narr)
  int32_t narr;
  int32_t pad;
  int64_t total_chunks;       // select blocks per array
  kvv_result* res;
  const RunRec* runs;
  const float* arr[kArrays];
  uint32_t* slots;            // kArrays * kSlotWords words per large segment
  const uint32_t* item_near;
  uint64_t* item_near_off;
  const double* item_near_sum;
};

struct ReduceLds {
  RunAcc wred[kWaves];
  RunAcc fin;
  uint64_t wsum[kWaves];
};

// Block histograms hold two 16-bit bin counts per word: a block counts at most
// kSelChunk (= kSmall) values, so a count never carries into its neighbour.
// Sample counts stay below 2^24 (the host caps max_samples), so ranks and
// histogram sums fit 32 bits.
struct SelectLds {
  uint32_t h[2][2048];
  double part[kBlock];
  uint32_t sh[16];
  uint32_t misc[4];
};
static_assert(kSelChunk == kSmall && kSelChunk <= 65535, "16-bit block bin counts");

union TailLds {
  ReduceLds r;
  SelectLds s;
};

// ------------------------------------------------------------ run-record fold
// kvv_result of one segment from its run records: each thread folds a strided
// subset, waves fold lanes in order, then one thread per field folds the waves
// in order, and the output fields are written by several threads at once.
__device__ inline void reduce_segment(const TailArgs& a, int seg, ReduceLds& L) {
  const SegDesc& d = a.table ? a.table[seg] : a.seg0;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // runs of this segment: its first item plus the block starts strictly inside it
  int64_t nruns = 0, b_first = 0;
  if (d.item_count > 0) {
    const int64_t rel0 = d.item_begin - d.run_base;                    // >= 0
    b_first = rel0 / d.run_ipb + 1;                                     // first block start after item_begin
    const int64_t rel_end = d.item_begin + d.item_count - d.run_base;  // exclusive
    const int64_t b_end = (rel_end + d.run_ipb - 1) / d.run_ipb;       // block starts < rel_end
    nruns = 1 + (b_end > b_first ? b_end - b_first : 0);
  }
  RunAcc acc;
  run_init(acc);
  // two records in flight per step
  for (int64_t j = tid; j < nruns; j += 2 * kBlock) {
    const RunRec r0 = a.runs[run_item(d, j, b_first)];
    const bool two = j + kBlock < nruns;
    RunRec r1;
    if (two) r1 = a.runs[run_item(d, j + kBlock, b_first)];
    run_merge(acc, r0);
    if (two) run_merge(acc, r1);
  }
  run_wave_reduce(acc);
  if (lane == 0) L.wred[w] = acc;
  // near-zero: exclusive prefix of the per-item counts, in item order
  if (d.flags & KVV_FLAG_NEAR_ZERO) {
    const int64_t per = (d.item_count + kBlock - 1) / kBlock;
    const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
    const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
    uint64_t mine = 0;
    for (int64_t k = k0; k < k1; ++k) mine += a.item_near[d.item_begin + k];
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
    for (int64_t k = k0; k < k1; ++k) {
      a.item_near_off[d.item_begin + k] = run;
      run += a.item_near[d.item_begin + k];
    }
  }
  __syncthreads();
  // fold the wave records: thread f takes field f, waves in order
  if (tid < LC_COUNT) {
    uint64_t t = 0;
    for (int i = 0; i < kWaves; ++i) t += L.wred[i].cnt[tid];
    L.fin.cnt[tid] = t;
  } else if (tid < LC_COUNT + 14) {
    RunAcc& f = L.fin;
    const int g = tid - LC_COUNT;
    if (g == 0) {
      uint64_t t = 0;
      for (int i = 0; i < kWaves; ++i) t += L.wred[i].mismatch;
      f.mismatch = t;
    } else if (g == 1 || g == 2) {
      uint64_t t = kNone;
      for (int i = 0; i < kWaves; ++i) {
        const uint64_t v = g == 1 ? L.wred[i].first_mm : L.wred[i].first_viol;
        t = v < t ? v : t;
      }
      if (g == 1) f.first_mm = t; else f.first_viol = t;
    } else if (g == 3 || g == 4) {
      uint32_t t = 0;
      for (int i = 0; i < kWaves; ++i) {
        const uint32_t v = g == 3 ? L.wred[i].mm_abs : L.wred[i].mm_rel;
        t = v > t ? v : t;
      }
      if (g == 3) f.mm_abs = t; else f.mm_rel = t;
    } else if (g == 5 || g == 6) {
      uint32_t bk = 0;
      uint64_t bi = kNone;
      for (int i = 0; i < kWaves; ++i) {
        const uint32_t k = g == 5 ? L.wred[i].gabs_k : L.wred[i].grel_k;
        const uint64_t x = g == 5 ? L.wred[i].gabs_i : L.wred[i].grel_i;
        if (better(k, x, bk, bi)) {
          bk = k;
          bi = x;
        }
      }
      if (g == 5) {
        f.gabs_k = bk;
        f.gabs_i = bi;
      } else {
        f.grel_k = bk;
        f.grel_i = bi;
      }
    } else {
      double t = 0.0;
      for (int i = 0; i < kWaves; ++i) t += L.wred[i].s[g - 7];
      f.s[g - 7] = t;
    }
  }
  __syncthreads();
  const RunAcc& r = L.fin;
  kvv_result& o = a.res[d.out_index];
  const bool imode = d.mode == KVV_MODE_MAX_ABS_DIFF;
  const double qnan = __builtin_nan("");
  switch (tid) {
    case 0:
      o.numel = d.n;
      o.mismatch_count = (int64_t)r.mismatch;
      o.first_mismatch_index = r.first_mm == kNone ? -1 : (int64_t)r.first_mm;
      o.mismatch_max_abs = r.mismatch ? (imode ? (double)ikey_value(r.mm_abs) : (double)fkey_value(r.mm_abs)) : 0.0;
      o.mismatch_max_rel = r.mismatch ? (double)fkey_value(r.mm_rel) : 0.0;
      o.status = 0;
      o.reserved = 0;
      break;
    case 1: {
      o.sample_count = d.m;
      o.sample_sum_gg = r.s[4];
      o.sample_sum_rr = r.s[5];
      o.sample_sum_gr = r.s[6];
      o.sample_cosine = cosine_of(r.s[6], r.s[4], r.s[5]);
      const double gn = sqrt(r.s[4]), rn = sqrt(r.s[5]);
      o.sample_norm_ratio = (gn == 0.0 && rn == 0.0) ? 1.0 : (gn == 0.0 ? 0.0 : (rn == 0.0 ? __builtin_inf() : gn / rn));
      break;
    }
    case 2:
      o.finite_violations = (int64_t)r.cnt[LC_VIOL];
      o.first_finite_violation = r.first_viol == kNone ? -1 : (int64_t)r.first_viol;
      o.nan_gen = (int64_t)r.cnt[LC_NAN_G];
      o.nan_ref = (int64_t)r.cnt[LC_NAN_R];
      o.posinf_gen = (int64_t)r.cnt[LC_PINF_G];
      o.posinf_ref = (int64_t)r.cnt[LC_PINF_R];
      o.neginf_gen = (int64_t)r.cnt[LC_NINF_G];
      o.neginf_ref = (int64_t)r.cnt[LC_NINF_R];
      break;
    case 3: {
      const int64_t c = (int64_t)r.cnt[LC_NEAR];
      o.near_zero_count = c;
      o.far_count = d.n - c;
      o.far_mismatch_count = (int64_t)r.cnt[LC_FARMM];
      o.near_zero_bad_count = (int64_t)r.cnt[LC_NEARBAD];
      const int64_t nm = c < d.max_samples ? c : d.max_samples;
      o.near_zero_sample_count = nm;
      // the near-zero selection writes these when it has a sample to work on
      if (!(d.flags & KVV_FLAG_NEAR_ZERO) || nm == 0) o.near_zero_p99_abs = o.near_zero_mean_abs = qnan;
      break;
    }
    case 4:
      if (d.n > 0) {
        o.max_abs = imode ? (double)ikey_value(r.gabs_k) : (double)fkey_value(r.gabs_k);
        o.max_abs_index = (int64_t)r.gabs_i;
        o.max_rel = (double)fkey_value(r.grel_k);
        o.max_rel_index = (int64_t)r.grel_i;
      } else {
        o.max_abs = o.max_rel = 0.0;
        o.max_abs_index = o.max_rel_index = -1;
      }
      break;
    case 5: {
      o.nan_pairs = (int64_t)r.cnt[LC_NANPAIR];
      o.sum_gg = r.s[0];
      o.sum_rr = r.s[1];
      o.sum_gr = r.s[2];
      o.sum_dd = r.s[3];
      const double dn = sqrt(r.s[3]), rn = sqrt(r.s[1]);
      o.rel_l2 = rn == 0.0 ? (dn == 0.0 ? 0.0 : __builtin_inf()) : dn / rn;
      o.cosine = cosine_of(r.s[2], r.s[0], r.s[1]);
      break;
    }
    case 6:
      // an empty sample has no selection to write its quantiles
      if (d.m == 0) o.p99_abs = o.p99_rel = qnan;
      break;
    default:
      if (tid >= 64 && tid < 64 + kBuckets) o.ulp_hist[tid - 64] = r.cnt[LC_HIST0 + tid - 64];
      break;
  }
}

// ------------------------------------------------------------ selection
__device__ __forceinline__ int64_t group_count(const SegDesc& d, const kvv_result& r, int arr) {
  return arr < 2 ? d.m : r.near_zero_sample_count;
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
                                   uint32_t bin[2], uint32_t below[2], uint32_t* sh) {
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
    sh[9] = sh[11] = 0;
  }
  __syncthreads();
  uint32_t baseA = 0, baseB = 0;
  for (int i = 0; i < w; ++i) {
    baseA += sh[i];
    baseB += sh[kWaves + i];
  }
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const bool useB = rr == 1 && !one;
    const uint32_t sum = useB ? sB : sA;
    uint32_t e = useB ? baseB + iB - sB : baseA + iA - sA;
    const uint32_t r = resid[rr];
    if (sum > 0 && e <= r && r < e + sum) {
      uint32_t b = tid * PER;
      bool found = false;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t c = useB ? cB[i] : cA[i];
        if (!found && r < e + c) {
          b = tid * PER + i;
          found = true;
        } else if (!found) {
          e += c;
        }
      }
      sh[8 + 2 * rr] = b;
      sh[9 + 2 * rr] = e;
    }
  }
  __syncthreads();
  bin[0] = sh[8];
  below[0] = sh[9];
  bin[1] = sh[10];
  below[1] = sh[11];
}

// torch's quantile interpolation between the order statistics (NaN when the
// sample holds a NaN); the near-zero array also gets its sample mean.  Called
// by all threads of the block.
__device__ inline void finalize_group(const TailArgs& a, const SegDesc& d, int arr, int64_t count,
                                      const uint32_t key[2], float wgt, bool has_nan, SelectLds& L) {
  kvv_result& res = a.res[d.out_index];
  const int tid = threadIdx.x;
  if (tid == 0) {
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
  if (arr == 2) {
    // near-zero sample mean: fixed-order sum of the per-item sampled sums
    const int64_t per = (d.item_count + kBlock - 1) / kBlock;
    const int64_t k0 = tid * per < d.item_count ? tid * per : d.item_count;
    const int64_t k1 = k0 + per < d.item_count ? k0 + per : d.item_count;
    double t = 0.0;
    for (int64_t k = k0; k < k1; ++k) t += a.item_near_sum[d.item_begin + k];
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

// A group of at most kSmall samples: keys in registers, four 8-bit digit
// passes over block histograms in LDS.
__device__ inline void select_small(const TailArgs& a, const SegDesc& d, int arr, int64_t count, SelectLds& L) {
  constexpr int PER = kSmall / kBlock;
  const int tid = threadIdx.x;
  const float* v = a.arr[arr] + d.sample_off;
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
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  uint32_t key[2] = {0u, 0u};
  const bool has_nan = block_sum_nan(nans, L) != 0;
  if (!has_nan) {
    uint32_t resid[2] = {(uint32_t)rank64[0], (uint32_t)rank64[1]};
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
  finalize_group(a, d, arr, count, key, wgt, has_nan, L);
}

// Prefixes and residual ranks of the two order statistics of a large group
// after the digit levels below LEVEL, from the group's global histograms.  All
// histogram words the block needs are loaded in one go.
template <int LEVEL>
__device__ inline void group_state(const uint32_t* slot, const uint64_t rank64[2], uint32_t pfx[2], uint32_t resid[2],
                                   SelectLds& L) {
  const int tid = threadIdx.x;
  uint32_t h0w = 0, h1a[16], h1b[16], h2a[16], h2b[16];
  if (LEVEL >= 1) h0w = slot[kH0 + tid];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (LEVEL >= 2) {
      h1a[i] = slot[kH1 + tid * 16 + i];
      h1b[i] = slot[kH1 + 4096 + tid * 16 + i];
    }
    if (LEVEL >= 3) {
      h2a[i] = slot[kH2 + tid * 16 + i];
      h2b[i] = slot[kH2 + 4096 + tid * 16 + i];
    }
  }
  pfx[0] = pfx[1] = 0u;
  resid[0] = (uint32_t)rank64[0];
  resid[1] = (uint32_t)rank64[1];
  uint32_t bin[2], below[2];
  if (LEVEL >= 1) {
    block_find2<1>(&h0w, &h0w, true, resid, bin, below, L.sh);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      pfx[rr] = bin[rr];
      resid[rr] -= below[rr];
    }
  }
  if (LEVEL >= 2) {
    block_find2<16>(h1a, h1b, pfx[0] == pfx[1], resid, bin, below, L.sh);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      pfx[rr] = (pfx[rr] << 12) | bin[rr];
      resid[rr] -= below[rr];
    }
  }
  if (LEVEL >= 3) {
    block_find2<16>(h2a, h2b, pfx[0] == pfx[1], resid, bin, below, L.sh);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      pfx[rr] = (pfx[rr] << 12) | bin[rr];
      resid[rr] -= below[rr];
    }
  }
}

// One chunk of a large group at digit level LEVEL: 0 = bits 31..24, 1 = 23..12,
// 2 = 11..0.
template <int LEVEL>
__device__ inline void select_chunk(const TailArgs& a, const SegDesc& d, int arr, int64_t count, int64_t c,
                                    SelectLds& L) {
  constexpr int PER = kSelChunk / kBlock;
  constexpr int HS = LEVEL == 2 ? 12 : 24;                     // prefix = key >> HS
  constexpr int DS = LEVEL == 0 ? 24 : (LEVEL == 1 ? 12 : 0);  // digit = (key >> DS) & DM
  constexpr uint32_t DM = LEVEL == 0 ? 255u : 4095u;
  const int tid = threadIdx.x;
  const int64_t c0 = c * (int64_t)kSelChunk;
  const int64_t c1 = c0 + kSelChunk < count ? c0 + kSelChunk : count;
  uint32_t* slot = a.slots + ((size_t)d.lslot * kArrays + arr) * kSlotWords;
  const float* v = a.arr[arr] + d.sample_off;
  float x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t idx = c0 + (int64_t)i * kBlock + tid;
    x[i] = idx < c1 ? v[idx] : 0.0f;
  }
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  uint32_t pfx[2], resid[2];
  group_state<LEVEL>(slot, rank64, pfx, resid, L);
  const bool same = pfx[0] == pfx[1];
  const int nwords = LEVEL == 0 ? 128 : (same ? 2048 : 4096);
  for (int i = tid; i < nwords; i += kBlock) (&L.h[0][0])[i] = 0;
  __syncthreads();
  uint32_t nans = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t idx = c0 + (int64_t)i * kBlock + tid;
    const bool isn = __builtin_isnan(x[i]);
    const bool ok = idx < c1 && !isn;
    if (LEVEL == 0) nans += (idx < c1 && isn) ? 1u : 0u;
    const uint32_t key = fkey(x[i]);
    const uint32_t dig = (key >> DS) & DM;
    if (LEVEL == 0) {
      lds_hist_add(L.h[0], dig, ok);
    } else {
      const uint32_t top = key >> HS;
      lds_hist_add(L.h[0], dig, ok && top == pfx[0]);
      if (!same) lds_hist_add(L.h[1], dig, ok && top == pfx[1]);
    }
  }
  if (LEVEL == 0) nans = block_sum_nan(nans, L);
  __syncthreads();
  // add the block histogram to the group's: bins 2w and 2w+1 of word w
  uint32_t* gh = slot + (LEVEL == 0 ? kH0 : (LEVEL == 1 ? kH1 : kH2));
  for (int i = tid; i < nwords; i += kBlock) {
    const uint32_t wv = (&L.h[0][0])[i];
    const int rr = LEVEL == 0 ? 0 : i / 2048;
    const int bw = LEVEL == 0 ? i : i % 2048;
    uint32_t* dst = gh + rr * 4096 + 2 * bw;
    if (wv & 0xFFFFu) atomicAdd(dst, wv & 0xFFFFu);
    if (wv >> 16) atomicAdd(dst + 1, wv >> 16);
  }
  if (LEVEL == 0 && tid == 0 && nans) atomicAdd(&slot[kMisc], nans);
}

// After the last level: one block per large group reads the full keys off the
// histograms and finishes the group.
__device__ inline void select_final(const TailArgs& a, const SegDesc& d, int arr, int64_t count, SelectLds& L) {
  const uint32_t* slot = a.slots + ((size_t)d.lslot * kArrays + arr) * kSlotWords;
  const bool has_nan = slot[kMisc] != 0;
  uint64_t rank64[2];
  float wgt;
  q99_ranks(count, rank64, wgt);
  uint32_t key[2], resid[2];
  group_state<3>(slot, rank64, key, resid, L);
  finalize_group(a, d, arr, count, key, wgt, has_nan, L);
}

#ifdef KVV_COMMON_KERNELS
// Level 0 also folds run records (leading blocks) and selects small groups.
template <int LEVEL>
__global__ __launch_bounds__(kBlock) void tail_kernel(TailArgs a) {
  __shared__ TailLds lds;
  const int64_t b = blockIdx.x;
  if (LEVEL == 0 && b < a.reduce_blocks) {
    reduce_segment(a, (int)b, lds.r);
    return;
  }
  const int64_t sb = b - a.reduce_blocks;
  const int arr = a.arr_lo + (int)(sb / a.total_chunks);
  const int64_t chunk = sb - (int64_t)(arr - a.arr_lo) * a.total_chunks;
  const int s = a.table ? (int)a.chunk_seg[chunk] : 0;
  const SegDesc& d = a.table ? a.table[s] : a.seg0;
  const int64_t count = group_count(d, a.res[d.out_index], arr);
  const int64_t c = chunk - d.chunk_begin;
  if (count <= 0) return;
  if (count <= kSmall || d.lslot < 0) {
    if (LEVEL == 0 && c == 0) select_small(a, d, arr, count, lds.s);
    return;
  }
  if (LEVEL == 3) {
    if (c == 0) select_final(a, d, arr, count, lds.s);
    return;
  }
  if (c * (int64_t)kSelChunk >= count) return;
  select_chunk<LEVEL>(a, d, arr, count, c, lds.s);
}
#endif  // KVV_COMMON_KERNELS
