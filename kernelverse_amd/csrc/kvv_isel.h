// Input select (included by kvv_kernels.h, namespace kvv): the p99 order
// statistics of abs_diff and rel_diff (GCR:396-402) over a segment's strided
// sample (GCR:338-348), read straight from the two input tensors instead of
// from sample arrays.
//
// Used by batch launches with many large groups (C4-like batches), for
// contiguous segments: the main pass then writes no sample arrays for them
// (8 bytes per sample, more than a bf16 pair's own 4) and walks no sample
// positions, and the selection reads the samples twice instead of the sample
// arrays three times, spread over chunks instead of one block per group.
// Four launches after the main pass:
//
//   isel_hist_kernel    one block per chunk of samples: 11-bit
//                       histograms of the top key digit (bits 31..21) of
//                       abs_diff and rel_diff, added into the segment's global
//                       histograms (nonzero bins only); exact zeros (identical
//                       pairs) are only counted.  The block also sums g^2,
//                       r^2 and g*r over its samples (the sampled cosine and
//                       norm ratio, GCR:351-393), which the run fold adds up
//                       in chunk order;
//   isel_find_kernel    one block per segment: the bins of the two order
//                       statistics of each array and the count below them;
//   isel_gather_kernel  one block per chunk: the values that fall in those bins
//                       (zeros aside) are appended, through a per-wave LDS
//                       stage, to the segment's sample region, whose space the
//                       workspace holds anyway;
//   isel_final_kernel   one block per segment: the order statistics among the
//                       zeros and the appended values (in LDS when at most
//                       kSmall were appended, else by streaming digit passes),
//                       interpolated like torch.quantile.
//
// abs_diff and rel_diff are computed exactly as the main pass's samples are
// (sample_pair), so the result equals the selection over sample arrays.

constexpr int kIselStage = 512;          // per-wave LDS stage of the gather, values per array

// Per-segment state (u32 words), cleared by the main pass.
enum IselWord {
  IS_HIST = 0,                 // [2][2048] top-digit histograms of abs_diff, rel_diff (zeros aside)
  IS_ZEROS = 2 * 2048,         // exact zeros (abs_diff == rel_diff == +0)
  IS_FILL,                     // [2] values appended per array
  IS_NAN = IS_FILL + 2,        // [2] the array holds a NaN
  IS_PFX = IS_NAN + 2,         // [2][2] bin of each order statistic
  IS_BASE = IS_PFX + 4,        // [2][2] values below each of those bins
  kIselStateWords = 4160       // 16,640 bytes: a multiple of 256
};
static_assert(IS_BASE + 4 <= kIselStateWords && (kIselStateWords * 4) % 256 == 0, "input-select state");

struct IselArgs {
  const SegDesc* table;
  const int2* chunks;      // chunk launches: (segment, chunk of the segment) per block
  int64_t chunk_lo;        // chunk launches: batch-wide number of the launch's first chunk
  double* sums;            // sampled sums per chunk (3 each)
  const int32_t* segs;     // segment launches: segment per block
  uint32_t* state;         // kIselStateWords per input-select segment (SegDesc::isel_slot)
  float* buf[2];           // the sample arrays: space for the appended abs_diff, rel_diff
  kvv_result* res;
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

// Calls f over the block's chunk: contiguous elements when every element is a
// sample, else the strided sample positions.
template <int DT, int MODE, typename F>
__device__ __forceinline__ void unit_pass(const SegDesc& d, int64_t e0, int64_t e1, F&& f) {
  if (d.m == d.n) chunk_pass<DT, MODE>(d, e0, e1, f);
  else sample_pass<DT, MODE>(d, e0, e1, f);
}

__device__ __forceinline__ void chunk_range(const IselArgs& a, const SegDesc*& d, int64_t& e0, int64_t& e1) {
  const int2 ck = a.chunks[blockIdx.x];
  d = &a.table[ck.x];
  const int64_t len = isel_chunk_len(*d);
  e0 = (int64_t)ck.y * len;
  e1 = e0 + len < d->m ? e0 + len : d->m;
}

template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void isel_hist_kernel(IselArgs a) {
  // bins 2048 + lane: a lane without a counted value adds there (no branch, no shared word)
  __shared__ uint32_t h[2][2048 + 64];
  __shared__ uint32_t zs[kWaves];
  __shared__ double ss[kWaves][3];
  const int tid = threadIdx.x, lane = tid & 63;
  const SegDesc* d;
  int64_t e0, e1;
  chunk_range(a, d, e0, e1);
  for (int i = tid; i < 2 * (2048 + 64); i += kBlock) (&h[0][0])[i] = 0;
  __syncthreads();
  using E = Elem<DT>;
  uint32_t zeros = 0;
  double sg = 0.0, sr = 0.0, sx = 0.0;
  unit_pass<DT, MODE>(*d, e0, e1, [&](float adf, float den, bool act, typename E::T gc, typename E::T rc) {
    const bool z = adf == 0.0f;
    zeros += act && z ? 1u : 0u;
    const bool cnt = act && !z;
    const uint32_t ba = cnt ? fkey(adf) >> 21 : 2048u + lane;
    const uint32_t br = cnt ? fkey(adf / den) >> 21 : 2048u + lane;
    atomicAdd(&h[0][ba], 1u);
    atomicAdd(&h[1][br], 1u);
    // inactive lanes hold zero codes, which add 0
    const double g64 = E::f64(gc), r64 = E::f64(rc);
    sg = fma(g64, g64, sg);
    sr = fma(r64, r64, sr);
    sx = fma(g64, r64, sx);
  });
  zeros = wave_sum(zeros);
  if (lane == 0) zs[tid >> 6] = zeros;
  // the chunk's sampled sums, in a fixed order (bit-reproducible)
  sg = wave_sum(sg);
  sr = wave_sum(sr);
  sx = wave_sum(sx);
  if (lane == 0) {
    ss[tid >> 6][0] = sg;
    ss[tid >> 6][1] = sr;
    ss[tid >> 6][2] = sx;
  }
  __syncthreads();
  if (tid < 3) {
    double t = 0.0;
    for (int w = 0; w < kWaves; ++w) t += ss[w][tid];
    a.sums[(size_t)(a.chunk_lo + blockIdx.x) * 3 + tid] = t;
  }
  uint32_t* st = a.state + (size_t)d->isel_slot * kIselStateWords;
  for (int i = tid; i < 2 * 2048; i += kBlock) {
    const uint32_t c = h[i >> 11][i & 2047];
    if (c) atomicAdd(&st[IS_HIST + i], c);
  }
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kWaves; ++w) t += zs[w];
    if (t) atomicAdd(&st[IS_ZEROS], t);
  }
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

template <int DT, int MODE>
__global__ __launch_bounds__(kBlock) void isel_gather_kernel(IselArgs a) {
  __shared__ float stage[kWaves][2][kIselStage];
  const int w = threadIdx.x >> 6;
  const SegDesc* d;
  int64_t e0, e1;
  chunk_range(a, d, e0, e1);
  uint32_t* st = a.state + (size_t)d->isel_slot * kIselStateWords;
  const bool nan0 = st[IS_NAN] != 0, nan1 = st[IS_NAN + 1] != 0;
  if (nan0 && nan1) return;
  const uint32_t p00 = st[IS_PFX], p01 = st[IS_PFX + 1], p10 = st[IS_PFX + 2], p11 = st[IS_PFX + 3];
  float* ba = a.buf[0] + d->sample_off;
  float* br = a.buf[1] + d->sample_off;
  uint32_t fa = 0, fr = 0;
  using T = typename Elem<DT>::T;
  unit_pass<DT, MODE>(*d, e0, e1, [&](float adf, float den, bool act, T, T) {
    const float rel = adf / den;
    const uint32_t ka = fkey(adf) >> 21, kr = fkey(rel) >> 21;
    const bool cnt = act && adf != 0.0f;
    stage_append(stage[w][0], fa, cnt && !nan0 && (ka == p00 || ka == p01), adf, &st[IS_FILL], ba);
    stage_append(stage[w][1], fr, cnt && !nan1 && (kr == p10 || kr == p11), rel, &st[IS_FILL + 1], br);
  });
  if (fa) stage_flush(stage[w][0], fa, &st[IS_FILL], ba);
  if (fr) stage_flush(stage[w][1], fr, &st[IS_FILL + 1], br);
}

#ifdef KVV_COMMON_KERNELS
__global__ __launch_bounds__(kBlock) void isel_find_kernel(IselArgs a) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  const SegDesc& d = a.table[a.segs[blockIdx.x]];
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

__global__ __launch_bounds__(kBlock) void isel_final_kernel(IselArgs a) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  const SegDesc& d = a.table[a.segs[blockIdx.x]];
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
      const uint32_t filled = st[IS_FILL + x];
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
#endif  // KVV_COMMON_KERNELS
