// bsattn_select.hip -- block selection for large candidate sets (more than
// one wave's worth of candidates) and wide GQA groups.
//
// k_select: one 1024-thread workgroup per (kv head, sequence).  Thread t owns
// blocks [t*PER, t*PER + PER) of the score row (read as whole vectors), with
// their keys in registers (PER = 1, 2, 4, 8 or 12, the smallest that covers
// the batch: every pass over the keys costs in proportion to PER); the K-th
// largest key is found by a range-adaptive radix select (a 2048-bin LDS
// histogram of the keys' range, refined inside the bin that holds the K-th
// key, which one wave resolves once it holds at most 64 keys).  Ties at the
// K-th key go to the lowest indices (a workgroup scan over the owners'
// segments), and the output is compacted in ascending block order.
//
// Wide groups (G >= 8): the block scores are first computed with MFMA
// (k_score_mfma), which does not reproduce the canonical summation order.
// Each approximate score s~ comes with a bound e >= |s~ - s| (s = canonical
// score), so with s_K, s_K+1 the K-th and (K+1)-th largest approximate
// scores, a block with s~ - e > s_K+1 + e is certainly selected, one with
// s~ + e < s_K - e certainly is not, and only the blocks in between (the
// band) are rescored in the canonical order; the remaining places go to the
// best of the band by (exact score, index) (one wave decides a band of at
// most 64 blocks).  The selection is therefore the
// canonical one, bit for bit.  (A block whose approximate score is not
// finite has no bound; if there is one, every candidate is rescored.)
//
// Bound: products of fp16 / bf16 pairs are exact or within one rounding in
// fp32; the canonical order adds 11 roundings and any fp32 accumulation of
// 128 products at most 128 more, so |s~ - s| <= 2^-14 * A with
// A = max over the group of sum |q_d| |k_d|.  Inputs below fp16's normal
// range that an MFMA might flush change a dot by at most
// 2^-14 * (||q||_1 + ||k||_1), which is added.  A + ||k||_1 is one MFMA on
// the magnitudes: max over the group of sum (|q_d| + 1) |k_d|, with |q_d| + 1
// rounded to nearest in the cache's type (>= 1, so within 2^-11 of itself in
// fp16, 2^-8 in bf16) and the product widened by 2^-10 (fp16) or 2^-7 (bf16)
// of itself to cover that rounding.  The bound used per (sequence, kv head)
// is the maximum over its blocks, widened by 2^-8 of itself to cover the
// roundings of the comparisons.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bsattn_device.h"

namespace bsattn {

constexpr int kMfmaTiles = 4;     // 16-block tiles per MFMA-scoring wave
constexpr int kMfmaChunk = 4 * 16 * kMfmaTiles;  // candidate blocks per MFMA-scoring workgroup
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelPerMax = 12;    // blocks per thread: mbps <= 12288
static_assert(kSelPerMax * kSelThreads / kMfmaChunk <= 64, "one wave reads every chunk bound");

__device__ __forceinline__ u32x4 abs16x8(u32x4 v) {
  return u32x4{v[0] & 0x7FFF7FFFu, v[1] & 0x7FFF7FFFu, v[2] & 0x7FFF7FFFu, v[3] & 0x7FFF7FFFu};
}

// a pair of non-negative fp16 / bf16 values x -> x + 1, rounded to nearest
template <int DT>
__device__ __forceinline__ uint32_t abs_plus_one(uint32_t x) {
  if constexpr (DT == 0) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, x) + f16x2{(_Float16)1.0f, (_Float16)1.0f});
  } else {
    return cvt_pk<1>(__uint_as_float(x << 16) + 1.0f, __uint_as_float(x & 0xFFFF0000u) + 1.0f);
  }
}

// fmaxf over each 16-lane row (every lane of the row gets it)
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xF, 0xF, false)));  // row_ror:1
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xF, 0xF, false)));  // row_ror:2
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, false)));  // row_ror:4
  return fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false)));  // row_ror:8
}

// integer sum over each 16-lane row (every lane of the row gets it)
__device__ __forceinline__ int row_sum16(int x) {
  x += __builtin_amdgcn_mov_dpp(x, 0x121, 0xF, 0xF, false);  // row_ror:1
  x += __builtin_amdgcn_mov_dpp(x, 0x122, 0xF, 0xF, false);  // row_ror:2
  x += __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false);  // row_ror:4
  return x + __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
}

// a workgroup barrier that orders LDS only: global loads still in flight stay
// in flight (__syncthreads() also waits for every outstanding global access)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// fmaxf over the whole wave
__device__ __forceinline__ float wave_max_f32(float x) {
  return __uint_as_float(wave_allreduce_u32(__float_as_uint(x), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}

// ---------------------------------------------------------------------------
// MFMA scoring (G >= 8): workgroup (chunk, kv head, sequence) handles
// kMfmaChunk candidate blocks; each wave takes kMfmaTiles 16-block tiles
// (the query operand is loaded once per wave):
//   S[head][block] = Q[head][:] . Summ[block][:]   (A = Q, B = summary rows^T)
// so that lane (block n, group g) holds heads 4g .. 4g+3 of block n and the
// maximum over the group is taken in-lane and across the four lane groups;
// plus (|Q| + 1) . |Summ|^T for the bound.  Writes the approximate score
// (max over the group) of every candidate and the chunk's bound to
// err[seq row][chunk].  The query loads are issued before the rows: loads
// complete in issue order, so each tile's MFMAs wait only for that tile's
// rows, and the tiles are computed while the later rows arrive.
// grid (chunks, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_score_mfma(Geometry geo, SeqBatch sb,
                                                    const uint16_t* __restrict__ q,
                                                    float* __restrict__ scores,
                                                    float* __restrict__ err, int err_stride,
                                                    int floor_rank) {
  __shared__ float s_e[4];
  __shared__ int s_bad[4];
  __shared__ float s_tm[4 * kMfmaTiles];  // each tile's largest approximate score (-inf: no candidate)
  __shared__ float s_sc[kMfmaChunk];      // the chunk's approximate scores (-inf: no candidate)
  const int chunk = blockIdx.x, h = blockIdx.y, bi = blockIdx.z;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // (the entries of wave w are written below by the same wave)
  s_sc[threadIdx.x] = -INFINITY;
  if (lane < kMfmaTiles) s_tm[wave * kMfmaTiles + lane] = -INFINITY;
  const int n = lane & 15, g = lane >> 4;
  const int seq = sb.ids[bi];
  const int c0 = geo.ns;
  u32x4 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = u32x4{0u, 0u, 0u, 0u};
  if (n < G) {
    const uint16_t* src = q + q_row(sb, bi, h * G + n) + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *(const u32x4*)(src + 32 * s);
  }
  // this wave's kMfmaTiles consecutive 16-block tiles; every summary load is
  // issued before the sequence length is known (rows are clamped into the
  // table; rows past the candidates are read and not used)
  const int jw = c0 + chunk * kMfmaChunk + wave * 16 * kMfmaTiles;
  u32x4 af[kMfmaTiles][4];
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    const int jr = min(jw + 16 * t + n, geo.mbps - 1);
    const uint16_t* row = summary_row(geo, seq, h, jr) + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) af[t][s] = *(const u32x4*)(row + 32 * s);
  }
  const int len = entry_len(geo, sb, bi, seq);
  const int nb = len > 0 ? (len + geo.tb - 1) / geo.tb : 0;
  const int c1 = nb - geo.nr;
  float* erow = err + ((size_t)bi * geo.hkv + h) * 2 * err_stride;
  if (!ranked_select(geo, c1 - c0)) {
    if (threadIdx.x == 0) {
      erow[chunk] = 0.0f;
      erow[err_stride + chunk] = INFINITY;
    }
    return;
  }
  constexpr uint32_t one2 = DT == 0 ? 0x3C003C00u : 0x3F803F80u;
  const u32x4 ones = u32x4{one2, one2, one2, one2};
  // |q| and |q| + 1 (zero past the group)
  u32x4 qa[4], qm[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qa[s] = abs16x8(qf[s]);
#pragma unroll
    for (int i = 0; i < 4; ++i) qm[s][i] = n < G ? abs_plus_one<DT>(qa[s][i]) : 0u;
  }
  // ||q_head||_1 (|Q| . 1), maximum over the group
  f32x4 q1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) q1 = mfma16x16x32<DT>(qa[s], ones, q1);
  float q1h = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (4 * g + i < G) q1h = fmaxf(q1h, q1[i]);
  const float q1max = max_over_groups(q1h);
  float emax = 0.0f;
  bool wbad = false;
  float st[kMfmaTiles];  // each tile's scores, stored after the last tile
  float* srow = score_row(geo, scores, bi, h);
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    // every tile, also past the candidates (masked below): each row load is
    // then waited for here, and nothing after the loop waits for memory
    const int j0 = jw + 16 * t;
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f}, a = d;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      d = mfma16x16x32<DT>(qf[s], af[t][s], d);
      a = mfma16x16x32<DT>(qm[s], abs16x8(af[t][s]), a);
    }
    // lane (block j0 + n, group g), entry i: head 4g + i
    float sc = -INFINITY, am = 0.0f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i < G) {
        sc = fmaxf(sc, d[i]);
        am = fmaxf(am, a[i]);
        bad = bad || __builtin_isnan(d[i]) || __builtin_isinf(d[i]);
      }
    sc = max_over_groups(sc);
    am = max_over_groups(am);
    // any non-finite head score makes the block's approximate score NaN
    const uint64_t bm = __ballot(bad);
    const bool any_bad = (((bm | (bm >> 16) | (bm >> 32) | (bm >> 48)) >> n) & 1ull) != 0ull;
    const int j = j0 + n;
    float tv = -INFINITY;
    st[t] = any_bad ? __builtin_nanf("") : sc;
    if (j < c1) {
      if (g == 0) s_sc[wave * 16 * kMfmaTiles + 16 * t + n] = st[t];
      if (!any_bad) {
        emax = fmaxf(emax, am);
        tv = sc;
      }
    }
    wbad = wbad || __ballot(j < c1 && any_bad) != 0ull;
    tv = row_max16(tv);
    if (lane == 0) s_tm[wave * kMfmaTiles + t] = tv;
  }
  // the scores, once every row load has been consumed (a store after each
  // tile slowed the rows' arrival)
  if (g == 0) {
#pragma unroll
    for (int t = 0; t < kMfmaTiles; ++t)
      if (jw + 16 * t + n < c1) srow[jw + 16 * t + n] = st[t];
  }
  emax = wave_max_f32(emax);
  if (lane == 0) {
    s_e[wave] = emax;
    s_bad[wave] = wbad;
  }
  __syncthreads();
  if (wave == 0) {
    // the chunk's floor, a score that floor_rank of its candidates reach:
    // the floor_rank-th largest of its tile maxima (distinct blocks), or,
    // when fewer tiles hold candidates, its floor_rank-th largest score (with
    // repeats).  -inf if a score is not finite (no certificate), +inf if the
    // chunk has fewer candidates
    const int total = min(max(c1 - (c0 + chunk * kMfmaChunk), 0), kMfmaChunk);
    float fl = INFINITY;
    if (s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3]) {
      fl = -INFINITY;
    } else if ((total + 15) / 16 >= floor_rank) {
      // rank of each tile maximum in descending order, ties by tile index;
      // the ranks of the 16 maxima are 0 .. 15, each once
      const int me = lane & 15;
      const float mine = s_tm[me];
      int rank = 0;
#pragma unroll
      for (int i = 0; i < 4 * kMfmaTiles; ++i) {
        const float o = s_tm[i];
        rank += (o > mine || (o == mine && i < me)) ? 1 : 0;
      }
      const uint64_t at = __ballot(lane < 16 && rank == floor_rank - 1);
      fl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), (int)__ffsll((unsigned long long)at) - 1));
    } else if (total >= floor_rank) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = s_sc[lane + 64 * i];
      for (int r = 0; r < floor_rank; ++r) {
        float lm = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        const float m = wave_max_f32(lm);
        fl = m;
        // remove one occurrence: the lowest lane holding it, its first slot
        const int src = __ffsll((unsigned long long)__ballot(lm == m)) - 1;
        if (lane == src) {
          if (v[0] == m) v[0] = -INFINITY;
          else if (v[1] == m) v[1] = -INFINITY;
          else if (v[2] == m) v[2] = -INFINITY;
          else v[3] = -INFINITY;
        }
      }
    }
    if (lane == 0) {
      constexpr float slack = DT == 0 ? 1.0f + 0x1p-10f : 1.0f + 0x1p-7f;  // |q| + 1 rounded
      erow[chunk] = 0x1p-14f * (fmaxf(fmaxf(s_e[0], s_e[1]), fmaxf(s_e[2], s_e[3])) * slack + q1max);
      erow[err_stride + chunk] = fl;
    }
  }
}

// ---------------------------------------------------------------------------
// workgroup primitives (1024 threads).  The cross-wave exchanges are
// double-buffered: call n uses buffer n & 1 (ph counts the calls, uniformly
// over the workgroup), so a call's writes never meet the previous call's
// reads, and the barrier of call n + 1 orders call n's reads before call
// n + 2's writes.  One barrier per call.
// ---------------------------------------------------------------------------
constexpr int kHistBins = 2048;
constexpr int kSmall = 64;  // keys resolved by one wave

struct SelScratch {
  uint32_t hist[kHistBins];
  uint32_t small[kSmall];
  int misc[8];
  __align__(16) uint32_t xch[2][2][kSelWaves];
};

// exclusive prefix sum of v over the workgroup in thread order; *total
__device__ __forceinline__ int wg_scan_excl(int v, SelScratch& ss, int& ph, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int x = wave_scan_incl(v);
  uint32_t* buf = ss.xch[ph & 1][0];
  ++ph;
  if (lane == 63) buf[w] = (uint32_t)x;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int t = (int)buf[i];
    off += (i < w) ? t : 0;
    tot += t;
  }
  *total = tot;
  return off + x - v;
}

// workgroup minimum of a and maximum of b (one exchange)
__device__ __forceinline__ void wg_minmax(uint32_t& a, uint32_t& b, SelScratch& ss, int& ph) {
  a = wave_min_u32(a);
  b = wave_max_u32(b);
  uint32_t(*buf)[kSelWaves] = ss.xch[ph & 1];
  ++ph;
  if ((threadIdx.x & 63) == 0) {
    buf[0][threadIdx.x >> 6] = a;
    buf[1][threadIdx.x >> 6] = b;
  }
  __syncthreads();
  a = buf[0][0];
  b = buf[1][0];
#pragma unroll
  for (int i = 1; i < kSelWaves; ++i) {
    a = min(a, buf[0][i]);
    b = max(b, buf[1][i]);
  }
}

// The K-th largest of the workgroup's nvalid valid keys (bit p of vmask:
// kr[p] valid), 1 <= K <= nvalid.  Range-adaptive radix select: the keys in
// [lo, hi] are histogrammed into 2048 LDS bins, the bin holding the K-th
// largest becomes the new range, until the range is one value or its bin
// holds at most 64 keys, which one wave then resolves by a bitwise search of
// their offsets.  The first pass bins by score value (scores cluster in a
// few binary exponents, so key bits would crowd them into a few bins); later
// passes bin by key bits, dividing the range by 2048 each time.
// *gt = valid keys > the result, *eq = valid keys equal to it.
template <int PER>
__device__ uint32_t wg_kth(const uint32_t (&kr)[PER], uint32_t vmask, int nvalid, int K,
                           SelScratch& ss, int& ph, int* gt, int* eq) {
  const int tid = threadIdx.x, lane = tid & 63;
  for (int b = tid; b < kHistBins; b += kSelThreads) ss.hist[b] = 0u;
  if (tid == 0) ss.misc[3] = 0;
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
  for (int p = 0; p < PER; ++p)
    if ((vmask >> p) & 1u) {
      lo = min(lo, kr[p]);
      hi = max(hi, kr[p]);
    }
  wg_minmax(lo, hi, ss, ph);  // its barrier also orders the zeroing above
  int need = K, above = 0, rcnt = nvalid;
  bool by_value = true;
  uint32_t tau;
#pragma unroll 1
  while (true) {
    if (lo == hi) {  // every remaining key has one value
      tau = lo;
      *gt = above;
      *eq = rcnt;
      break;
    }
    const float vlo = key_value(lo), span = key_value(hi) - vlo;
    const bool use_v = by_value && __builtin_isfinite(vlo) && __builtin_isfinite(span) && span > 0.0f;
    const float scale = use_v ? (float)(kHistBins - 1) / span : 0.0f;
    const int sh = use_v ? 0 : max(0, 32 - __clz(hi - lo) - 11);  // (hi - lo) >> sh < 2048
    auto bin = [&](uint32_t key) -> int {
      return use_v ? min(kHistBins - 1, (int)((key_value(key) - vlo) * scale)) : (int)((key - lo) >> sh);
    };
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if (((vmask >> p) & 1u) && kr[p] >= lo && kr[p] <= hi) atomicAdd(&ss.hist[bin(kr[p])], 1u);
    __syncthreads();
    // thread t owns bins 2047 - 2t and 2046 - 2t, so a scan in thread order
    // counts the keys in higher bins
    const int b0 = kHistBins - 1 - 2 * tid, b1 = b0 - 1;
    const int h0 = (int)ss.hist[b0], h1 = (int)ss.hist[b1];
    int tot;
    const int before = wg_scan_excl(h0 + h1, ss, ph, &tot);
    if (before < need && need <= before + h0) {
      ss.misc[0] = b0;
      ss.misc[1] = before;
      ss.misc[2] = h0;
    } else if (before + h0 < need && need <= before + h0 + h1) {
      ss.misc[0] = b1;
      ss.misc[1] = before + h0;
      ss.misc[2] = h1;
    }
    __syncthreads();
    const int bstar = ss.misc[0], abv = ss.misc[1], cnt = ss.misc[2];
    above += abv;
    need -= abv;
    rcnt = cnt;
    if (!use_v && sh == 0) {  // one-value bin
      tau = lo + (uint32_t)bstar;
      *gt = above;
      *eq = cnt;
      break;
    }
    if (cnt <= kSmall) {
      // gather the bin's keys; one wave finds the need-th largest
#pragma unroll
      for (int p = 0; p < PER; ++p)
        if (((vmask >> p) & 1u) && kr[p] >= lo && kr[p] <= hi && bin(kr[p]) == bstar)
          ss.small[atomicAdd(&ss.misc[3], 1)] = kr[p];
      __syncthreads();
      if (tid < 64) {
        const bool valid = lane < cnt;
        const uint32_t x = valid ? ss.small[lane] : 0u;
        const uint32_t mn = wave_min_u32(valid ? x : 0xFFFFFFFFu), mx = wave_max_u32(x);
        const uint32_t off = x - mn;
        uint32_t t = 0u;
        for (int bit = mx == mn ? -1 : 31 - __clz(mx - mn); bit >= 0; --bit) {
          const uint32_t cand = t | (1u << bit);
          if (__popcll(__ballot(valid && off >= cand)) >= need) t = cand;
        }
        const int gcount = __popcll(__ballot(valid && off > t));
        const int ecount = __popcll(__ballot(valid && off == t));
        if (lane == 0) {
          ss.misc[4] = (int)(mn + t);
          ss.misc[5] = gcount;
          ss.misc[6] = ecount;
        }
      }
      __syncthreads();
      tau = (uint32_t)ss.misc[4];
      *gt = above + ss.misc[5];
      *eq = ss.misc[6];
      break;
    }
    // refine to the bin's keys; the histogram is cleared for the next pass
    // (every read of it is behind the barriers above)
    for (int b = tid; b < kHistBins; b += kSelThreads) ss.hist[b] = 0u;
    if (tid == 0) ss.misc[3] = 0;
    if (use_v) {
      uint32_t nlo = 0xFFFFFFFFu, nhi = 0u;
#pragma unroll
      for (int p = 0; p < PER; ++p)
        if (((vmask >> p) & 1u) && kr[p] >= lo && kr[p] <= hi && bin(kr[p]) == bstar) {
          nlo = min(nlo, kr[p]);
          nhi = max(nhi, kr[p]);
        }
      wg_minmax(nlo, nhi, ss, ph);
      lo = nlo;
      hi = nhi;
    } else {
      const uint32_t nlo = lo + ((uint32_t)bstar << sh);
      const uint32_t span_k = (1u << sh) - 1u;
      hi = (hi - nlo < span_k) ? hi : nlo + span_k;
      lo = nlo;
      __syncthreads();
    }
    by_value = false;
  }
  __syncthreads();  // ss is reused by the caller
  return tau;
}

// Marks the K largest of the nvalid valid keys (ties at the K-th to the
// lowest index, i.e. thread order then p); all of them when K >= nvalid.
template <int PER>
__device__ uint32_t wg_topk_mask(const uint32_t (&kr)[PER], uint32_t vmask, int nvalid, int K,
                                 SelScratch& ss, int& ph) {
  if (K <= 0) return 0u;
  if (nvalid <= K) return vmask;
  int gt, eq;
  const uint32_t tau = wg_kth(kr, vmask, nvalid, K, ss, ph, &gt, &eq);
  const int krem = K - gt;
  uint32_t take = 0u;
  if (eq == krem) {  // every key equal to the K-th is taken
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if (((vmask >> p) & 1u) && kr[p] >= tau) take |= 1u << p;
    return take;
  }
  int ties = 0;
#pragma unroll
  for (int p = 0; p < PER; ++p) ties += ((vmask >> p) & 1u) && kr[p] == tau;
  int tie_total;
  int rank = wg_scan_excl(ties, ss, ph, &tie_total);
#pragma unroll
  for (int p = 0; p < PER; ++p)
    if ((vmask >> p) & 1u) {
      if (kr[p] > tau) take |= 1u << p;
      else if (kr[p] == tau) {
        if (rank < krem) take |= 1u << p;
        ++rank;
      }
    }
  return take;
}

// The krem best of one wave's keys x (lanes with valid set; lane order is
// index order) by (key desc, lane asc), 1 <= krem < number of valid lanes.
__device__ __forceinline__ bool wave_take_best(uint32_t x, bool valid, int krem) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const uint32_t mn = wave_min_u32(valid ? x : 0xFFFFFFFFu), mx = wave_max_u32(valid ? x : 0u);
  const uint32_t off = x - mn;
  uint32_t t = 0u;  // the krem-th largest offset
  for (int bit = mx == mn ? -1 : 31 - __clz(mx - mn); bit >= 0; --bit) {
    const uint32_t cand = t | (1u << bit);
    if (__popcll(__ballot(valid && off >= cand)) >= krem) t = cand;
  }
  const int gcount = __popcll(__ballot(valid && off > t));
  const uint64_t eqm = __ballot(valid && off == t);
  return valid && (off > t || (off == t && gcount + __popcll(eqm & below) < krem));
}

// 8 consecutive query elements held in LDS as fp32 (16-byte aligned)
__device__ __forceinline__ void query8(const float* src, float (&v)[8]) {
  const float4 a = ((const float4*)src)[0], b = ((const float4*)src)[1];
  v[0] = a.x;
  v[1] = a.y;
  v[2] = a.z;
  v[3] = a.w;
  v[4] = b.x;
  v[5] = b.y;
  v[6] = b.z;
  v[7] = b.w;
}

// thread's PER consecutive score-row entries as whole vectors
template <int PER>
__device__ __forceinline__ void load_scores(const float* __restrict__ src, float (&v)[PER]) {
  if constexpr (PER % 4 == 0) {
#pragma unroll
    for (int i = 0; i < PER / 4; ++i) {
      const float4 x = ((const float4*)src)[i];
      v[4 * i] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else if constexpr (PER == 2) {
    const float2 x = *(const float2*)src;
    v[0] = x.x;
    v[1] = x.y;
  } else {
    v[0] = src[0];
  }
}

// ---------------------------------------------------------------------------
// The selection over the keys the workgroup's threads hold (kr[p] of slot p
// valid where vmask has bit p; jr[p] its block index; thread order then p
// is block order; nvalid valid keys in all): the K largest by (exact key,
// index), as a mask over the thread's slots.  BAND: the keys are
// approximate MFMA scores with bound e (see the top of this file), and the
// band around the K-th is rescored in the canonical order (the query rows
// in s_qf); the argument needs only that the keys held include the row's
// top K.
// ---------------------------------------------------------------------------
template <int DT, int G, bool BAND, int PER>
__device__ uint32_t select_core(const Geometry& geo, int seq, int h, const uint32_t (&kr)[PER],
                                const int (&jr)[PER], uint32_t vmask, int nvalid, int K, float e,
                                SelScratch& ss, int& ph, uint32_t* s_band, const float* s_qf) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (nvalid <= K) return vmask;
  if constexpr (!BAND) {
    return wg_topk_mask(kr, vmask, nvalid, K, ss, ph);
  } else {
    // K-th largest approximate key
    int gt, eq;
    const uint32_t t1 = wg_kth(kr, vmask, nvalid, K, ss, ph, &gt, &eq);
    // one exchange: the largest key below t1 and whether every approximate
    // score is finite
    uint32_t fin = 1u, below = 0u;
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if ((vmask >> p) & 1u) {
        if (kr[p] < t1) below = max(below, kr[p]);
        if (!__builtin_isfinite(key_value(kr[p]))) fin = 0u;
      }
    wg_minmax(fin, below, ss, ph);
    const uint32_t t2 = gt + eq <= K ? below : t1;  // the (K+1)-th largest
    const float lb = key_value(t1) - e, ub = key_value(t2) + e;
    // a candidate whose approximate score is not finite has no bound (its
    // exact score may exceed any other), and non-finite limits certify
    // nothing: then every candidate is rescored
    const bool bounds_ok = fin != 0u && __builtin_isfinite(lb) && __builtin_isfinite(ub);
    // classify: certainly in (take), band (rescored), certainly out
    uint32_t band = 0u, take = 0u;
    int nin = 0, nband = 0;
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if ((vmask >> p) & 1u) {
        const float v = key_value(kr[p]);  // the approximate score (NaN -> -inf)
        const bool sure = bounds_ok && __builtin_isfinite(v);
        if (sure && v - e > ub) {
          take |= 1u << p;
          ++nin;
        } else if (!(sure && v + e < lb)) {
          band |= 1u << p;
          ++nband;
        }
      }
    // both counts in one scan (each total <= 12288 fits 16 bits)
    int packed_total;
    const int packed_pos = wg_scan_excl((nin << 16) | nband, ss, ph, &packed_total);
    const int nin_total = packed_total >> 16, nband_total = packed_total & 0xFFFF;
    const int bpos = packed_pos & 0xFFFF;
    const int krem = K - nin_total;
    if (nband_total <= krem) return take | band;
    // band list, then the canonical score of every band block
    int w = bpos;
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if (band & (1u << p)) s_band[w++] = (uint32_t)jr[p];
    __syncthreads();
    const int c = tid & 15;
    for (int bk = tid >> 4; bk < nband_total; bk += kSelThreads / 16) {
      const int j = (int)s_band[bk];
      float sv[8];
      unpack8<DT>(*(const u32x4*)(summary_row(geo, seq, h, j) + 8 * c), sv);
      float best = 0.0f;
#pragma unroll 4
      for (int gq = 0; gq < G; ++gq) {
        float qv[8];
        query8(s_qf + gq * kHeadDim + 8 * c, qv);
        const float acc = canonical_dot16<DT>(qv, sv);
        if (gq == 0 || acc > best) best = acc;
      }
      if (c == 0) s_band[bk] = score_key(best);  // the slot's index is no longer needed
    }
    __syncthreads();
    if (nband_total <= 64) {
      // one wave picks the krem best of the band (band slots are in block
      // order) and leaves a 0/1 flag in each slot
      if (tid < 64) {
        const bool valid = lane < nband_total;
        const uint32_t x = valid ? s_band[lane] : 0u;
        const bool t = wave_take_best(x, valid, krem);
        if (valid) s_band[lane] = t ? 1u : 0u;
      }
      __syncthreads();
      w = bpos;
#pragma unroll
      for (int p = 0; p < PER; ++p)
        if (band & (1u << p)) take |= (s_band[w++] != 0u ? 1u : 0u) << p;
      return take;
    }
    uint32_t br[PER];
    w = bpos;
#pragma unroll
    for (int p = 0; p < PER; ++p) br[p] = (band & (1u << p)) ? s_band[w++] : 0u;
    return take | wg_topk_mask(br, band, nband_total, krem, ss, ph);
  }
}

// ---------------------------------------------------------------------------
// Banded selection after a certified floor.  The survivors (approximate
// score v in [lim, vmax]) are histogrammed into kWaveBins bins of value;
// bin(v) = min(kWaveBins - 1, floor(fl(fl(v - lim) * scale))) is monotone in
// v, and fl(v - lim) * scale stays within 2^-12 of the exact (v - lim) *
// scale (u below), so two keys D bins apart have u more than D - 1 - 2^-11
// apart, i.e. values more than that over scale.  With b* the bin of the
// K-th largest approximate score t1 and D chosen so that
// (D - 1 - 2^-11) / scale > 2e:
//   bin(x) >= b* + D:  v_x - e > t1 + e >= t2 + e, certainly selected;
//   bin(x) <= b* - D:  v_x + e < t1 - e, certainly not;
// the keys of the bins in between (the band, which holds the K-th) are
// rescored in the canonical order, and the remaining places go to the band's
// best by (exact key, index).
// Every pass runs on few lanes: each wave first packs its own survivors
// (bin, block) into its first lanes through LDS, in block order, so that a
// survivor is one lane and not a slot of every thread's PER; then
//   barrier 1: the histogram; each wave finds b* for itself, counts its
//              certainly-selected keys and hands its band keys slots of an
//              unordered band list (LDS counter);
//   barrier 2: the band list; waves take its entries 4 at a time (16 lanes
//              each) and rescore them;
//   barrier 3: the exact keys; the same lanes rank their entry among all of
//              them (4 per lane, then a row sum) and mark it selected or not;
//   barrier 4: the marks; each wave counts the selected band blocks of the
//              waves before it and writes its selected blocks.
// (Barriers 3 and 4 are skipped when the band fills the remaining places.)
// Each pass is a few instructions per wave: a 16-wave workgroup runs four
// waves per SIMD, so work that every wave repeats costs sixteen times its
// own instruction count on each SIMD.  Returns
// false, having written nothing to out, when a wave holds more than 64
// survivors, the band exceeds kFastBand or the bound spans too many bins (the
// caller then runs the general passes over the same survivors); each
// decision is uniform over the workgroup, as every wave reads the same LDS
// words.
// ---------------------------------------------------------------------------
constexpr int kFastBins = kWaveBins;  // find_kth_bin's histogram
constexpr int kFastBand = 64;
static_assert(kFastBins <= kHistBins, "the histogram lives in SelScratch");

struct FastScratch {
  float wmax[kSelWaves];                // each wave's largest valid approximate score
  __align__(16) int win[kSelWaves];     // each wave's certainly-selected count
  __align__(16) int bj[kFastBand];      // band list: block
  __align__(16) uint32_t bk[kFastBand];  // band list: exact key
  int pk[kFastBand];                    // band list: selected
  int bcnt;                             // band slots handed out
  int over;                             // a wave held more than 64 survivors
};

template <int DT, int G, int PER>
__device__ bool select_banded(const Geometry& geo, int seq, int h, const float (&sc)[PER], uint32_t vmask,
                              int K, float e, float lim, float scale, SelScratch& ss, FastScratch& fs,
                              uint32_t* s_band, const float* s_qf, int32_t* out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const float y = 2.0f * e * scale * 1.001f;  // D = floor(y) + 3 > 2e * scale + 1 + 2^-11
  if (!(y < 512.0f)) return false;
  const int D = (int)y + 3;
  // the wave's survivors, packed in block order: bin << 16 | block - the
  // wave's first block.  A survivor's rank in the wave is at most its offset,
  // so the words stay inside the wave's own blocks of s_band (< mbps words)
  const int ct = __popc(vmask);
  const int incl = wave_scan_incl(ct);
  const int n_w = __builtin_amdgcn_readlane(incl, 63);
  uint32_t* wl = s_band + wave * 64 * PER;
  int w = incl - ct;
#pragma unroll
  for (int p = 0; p < PER; ++p)
    if ((vmask >> p) & 1u) {
      const int bn = min(kFastBins - 1, (int)((sc[p] - lim) * scale));
      wl[w++] = ((uint32_t)bn << 16) | (uint32_t)(lane * PER + p);
    }
  if (n_w > 64 && lane == 0) fs.over = 1;
  wave_lds_order();
  const bool has = lane < n_w;
  const uint32_t word = has ? wl[lane] : 0u;
  const int bin = (int)(word >> 16);
  const int j = wave * 64 * PER + (int)(word & 0xFFFFu);
  if (has) atomicAdd(&ss.hist[bin], 1u);
  lds_barrier();
  if (fs.over) return false;
  int bstar, abv, cnt;
  find_kth_bin(ss.hist, K, bstar, abv, cnt);
  const bool in = has && bin >= bstar + D;
  const bool band = has && !in && bin > bstar - D;
  const uint64_t inb = __ballot(in), bandb = __ballot(band);
  if (lane == 0) fs.win[wave] = __popcll(inb);
  // each band key's summary row, requested by its owner now and read by the
  // rescoring lanes after the band list is out (then from the cache); every
  // lane loads (the others the first candidate's row), so that the load is
  // not waited for where a branch joins
  const uint16_t* pfr = summary_row(geo, seq, h, band ? j : geo.ns);
  const uint32_t pf0 = *(const uint32_t*)pfr, pf1 = *(const uint32_t*)(pfr + 64);
  int slot = 0;
  if (bandb) {
    int b0 = 0;
    if (lane == 0) b0 = atomicAdd(&fs.bcnt, __popcll(bandb));
    slot = __builtin_amdgcn_readlane(b0, 0) + __popcll(bandb & below);
    if (band && slot < kFastBand) fs.bj[slot] = j;
  }
  lds_barrier();
  const int nband = fs.bcnt;
  u32x4 w4[kSelWaves / 4];
#pragma unroll
  for (int i = 0; i < kSelWaves / 4; ++i) w4[i] = *(const u32x4*)(fs.win + 4 * i);
  int nin = 0, in_before = 0;  // certainly-selected keys: all, and in the waves before this one
#pragma unroll
  for (int v = 0; v < kSelWaves; ++v) {
    nin += (int)w4[v >> 2][v & 3];
    in_before += v < wave ? (int)w4[v >> 2][v & 3] : 0;
  }
  const int krem = K - nin;  // >= 1, and nband >= 1: the K-th is in the band
  if (nband > kFastBand || nband < 1 || krem < 1) return false;
  const bool rescore = nband > krem;
  if (rescore) {
    // band entry gi = 4 * wave + lane / 16 on 16 lanes: its canonical score,
    // then (after the barrier) its rank among the entries by (exact key
    // desc, block asc), as distinct 64-bit keys
    const bool holder = 4 * wave < nband;
    const int gi = 4 * wave + (lane >> 4), c = lane & 15;
    const int ge = min(gi, nband - 1);
    if (holder) {
      const int jb = fs.bj[ge];
      float sv[8];
      unpack8<DT>(*(const u32x4*)(summary_row(geo, seq, h, jb) + 8 * c), sv);
      float best = 0.0f;
#pragma unroll 4
      for (int gq = 0; gq < G; ++gq) {
        float qv[8];
        query8(s_qf + gq * kHeadDim + 8 * c, qv);
        const float acc = canonical_dot16<DT>(qv, sv);
        if (gq == 0 || acc > best) best = acc;
      }
      if (c == 0 && gi < nband) fs.bk[gi] = score_key(best);
    }
    lds_barrier();
    if (holder) {
      const uint64_t me = ((uint64_t)fs.bk[ge] << 32) | (uint32_t)~fs.bj[ge];
      int r = 0;
#pragma unroll
      for (int m = 0; m < kFastBand / 16; ++m) {
        const int L = c + 16 * m;  // < kFastBand: stale past nband, not counted
        const uint64_t o = ((uint64_t)fs.bk[L] << 32) | (uint32_t)~fs.bj[L];
        r += (L < nband && o > me) ? 1 : 0;
      }
      r = row_sum16(r);
      if (c == 0 && gi < nband) fs.pk[gi] = r < krem ? 1 : 0;
    }
    lds_barrier();
  }
  // without rescoring the band fills the remaining places: every entry is taken
  const int bjl = fs.bj[lane];
  const bool pkl = lane < nband && (!rescore || fs.pk[lane] != 0);
  const int pick_before = __popcll(__ballot(pkl && bjl / (64 * PER) < wave));
  const bool take = in || (band && (!rescore || fs.pk[slot] != 0));
  const int pos = geo.ns + in_before + pick_before + __popcll(__ballot(take) & below);
  asm volatile("" ::"v"(pf0), "v"(pf1));  // the prefetch's registers, consumed before the store
  if (take && pos < geo.ns + K) out[pos] = j;
  return true;
}

// ---------------------------------------------------------------------------
// block-wide selection; grid (Hkv, n), 1024 threads.  Thread t owns blocks
// j = t*PER + p, p < PER, of its score row (the candidates are ns <= j <
// ns + nc), so thread order then p is block order.
// BAND: scores are the approximate MFMA scores with bounds in err (see the
// top of this file); dynamic LDS then holds the band (u32 per candidate).
// The scoring also left each chunk's floor (its floor_rank-th largest
// approximate score): every chunk with a finite floor holds floor_rank
// candidates at or above it, so when those chunks hold at least K of them,
// the row's K-th largest exact score is at least tau - e (tau = the least
// floor), and a candidate with s~ < tau - 2e is certainly out.  The
// remaining candidates (a few percent of a row of iid scores) are compacted
// into LDS, one per thread, and the selection runs over them.
// ---------------------------------------------------------------------------
template <int DT, int G, bool BAND, int PER>
__global__ __launch_bounds__(kSelThreads) void k_select(Geometry geo, SeqBatch sb,
                                                        const uint16_t* __restrict__ q,
                                                        const float* __restrict__ scores,
                                                        const float* __restrict__ err,
                                                        int err_stride, int err_count, int floor_rank,
                                                        int32_t* __restrict__ idx_out) {
  extern __shared__ uint32_t s_band[];
  __shared__ SelScratch ss;
  __shared__ FastScratch fs;
  __shared__ __align__(16) float s_qf[BAND ? G * kHeadDim : 4];  // the group's query rows (fp32)
  __shared__ float s_lim[2];  // e, tau - 2e
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = blockIdx.x, bi = blockIdx.y;
  const int seq = sb.ids[bi];
  const int c0 = geo.ns, K = geo.top_k;
  // the arguments of the first phase, loaded in one round of scalar loads:
  // left to itself the compiler issues each where it is first needed, and
  // every one of them then waits behind the round before it
  asm volatile("" ::"s"(seq), "s"(sb.len[bi]), "s"(sb.qoff[bi]), "s"(sb.qhs), "s"(geo.hkv), "s"(geo.sstride),
               "s"(geo.tb), "s"(c0), "s"(geo.nr), "s"(K), "s"(geo.nsel_max), "s"(geo.meta), "s"(q), "s"(scores),
               "s"(err), "s"(err_stride), "s"(err_count), "s"(idx_out));
  // scores (and the chunk bounds and floors) are loaded before the sequence
  // length is known: the row reads stay inside the score buffer (its slack
  // covers the last row), and entries that are not candidates are never used
  const int i0 = tid * PER;
  float sc[PER];
  load_scores<PER>(score_row(geo, scores, bi, h) + i0, sc);
  float ev = 0.0f, fl = INFINITY;
  if (BAND && tid < 64 && lane < err_count) {
    const float* erow = err + ((size_t)bi * geo.hkv + h) * 2 * err_stride;
    ev = erow[lane];
    fl = erow[err_stride + lane];
  }
  // the query rows of the group (one word per thread), also issued before
  // the length is known
  static_assert(!BAND || G * kHeadDim / 2 <= kSelThreads, "one query word per thread");
  uint32_t qw = 0u;
  if (BAND && tid < G * kHeadDim / 2)
    qw = ((const uint32_t*)(q + q_row(sb, bi, h * G + tid / (kHeadDim / 2))))[tid % (kHeadDim / 2)];
  const int len = entry_len(geo, sb, bi, seq);
  const int nb = len > 0 ? (len + geo.tb - 1) / geo.tb : 0;
  const int nc = nb - geo.nr - c0;
  int32_t* out = idx_out + ((size_t)bi * geo.hkv + h) * geo.nsel_max;
  if (!ranked_select(geo, nc)) {  // every block kept, or (top_k 0) sinks and recent only
    for (int p = tid; p < geo.nsel_max; p += kSelThreads)
      out[p] = selected_block(p, nb, nc > K, geo.ns, geo.nr, K, nullptr);
    return;
  }
  int jr[PER];
  uint32_t vmask = 0u;
  float vm = -INFINITY;  // the largest valid approximate score (NaN skipped)
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const bool v = i0 + p >= c0 && i0 + p < c0 + nc;
    jr[p] = i0 + p;
    vmask |= (uint32_t)v << p;
    if (v) vm = fmaxf(vm, sc[p]);
  }
  // the keys (score order as unsigned integers), where the passes need them
  auto keys = [&](uint32_t (&kr)[PER]) {
#pragma unroll
    for (int p = 0; p < PER; ++p) kr[p] = ((vmask >> p) & 1u) ? score_key(sc[p]) : 0u;
  };
  int ph = 0;
  uint32_t take;
  int total;
  if constexpr (!BAND) {
    uint32_t kr[PER];
    keys(kr);
    take = select_core<DT, G, BAND, PER>(geo, seq, h, kr, jr, vmask, nc, K, 0.0f, ss, ph, s_band, s_qf);
    const int pos = wg_scan_excl(__popc(take), ss, ph, &total);
    int w = geo.ns + pos;
#pragma unroll
    for (int p = 0; p < PER; ++p)
      if (take & (1u << p)) out[w++] = jr[p];
  } else {
    if (tid < G * kHeadDim / 2) {
      s_qf[2 * tid] = to_f32<DT>((uint16_t)(qw & 0xFFFFu));
      s_qf[2 * tid + 1] = to_f32<DT>((uint16_t)(qw >> 16));
    }
    // for the banded selection: its histogram cleared, its counters, and
    // each wave's largest approximate score
    for (int b = tid; b < kFastBins; b += kSelThreads) ss.hist[b] = 0u;
    if (tid == 0) {
      fs.bcnt = 0;
      fs.over = 0;
    }
    vm = wave_max_f32(vm);
    if (lane == 0) fs.wmax[tid >> 6] = vm;
    if (tid < 64) {
      // the bound: maximum over the chunks' bounds (NaN bounds are skipped);
      // the floor: least chunk floor, if the chunks with one hold K
      const float e = wave_max_f32(ev) * (1.0f + 0x1p-8f) + 0x1p-120f;
      const float tau = __uint_as_float(wave_allreduce_u32(__float_as_uint(fl), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fminf(__uint_as_float(a), __uint_as_float(b)));
      }));
      const int nfl = __popcll(__ballot(fl < INFINITY));
      if (tid == 0) {
        s_lim[0] = e;
        s_lim[1] = (int64_t)nfl * floor_rank >= K ? tau - 2.0f * e : -INFINITY;
      }
    }
    __syncthreads();
    const float e = s_lim[0], lim = s_lim[1];
    // certainly out: below lim (-inf: no floor.  A NaN candidate's chunk
    // has floor -inf, so with a finite lim every candidate score is a number)
    if (lim > -INFINITY) {
#pragma unroll
      for (int p = 0; p < PER; ++p)
        if (((vmask >> p) & 1u) && sc[p] < lim) vmask &= ~(1u << p);
    }
    float vmax = fs.wmax[0];
#pragma unroll
    for (int w = 1; w < kSelWaves; ++w) vmax = fmaxf(vmax, fs.wmax[w]);
    const float scale = (float)(kFastBins - 1) / (vmax - lim);
    if (lim > -INFINITY && __builtin_isfinite(vmax) && vmax > lim && __builtin_isfinite(scale) &&
        select_banded<DT, G, PER>(geo, seq, h, sc, vmask, K, e, lim, scale, ss, fs, s_band, s_qf, out)) {
      total = K;
    } else {
      uint32_t kr[PER];
      keys(kr);
      int nv;
      const int cpos = wg_scan_excl(__popc(vmask), ss, ph, &nv);
      if (nv <= kSelThreads) {
        // one candidate per thread, in block order: keys through the band
        // buffer (mbps >= nc >= nv words), blocks through the histogram
        // (2048 words), both free until the selection
        int w = cpos;
#pragma unroll
        for (int p = 0; p < PER; ++p)
          if ((vmask >> p) & 1u) {
            s_band[w] = kr[p];
            ss.hist[w++] = (uint32_t)jr[p];
          }
        __syncthreads();
        const uint32_t k1[1] = {tid < nv ? s_band[tid] : 0u};
        const int j1[1] = {tid < nv ? (int)ss.hist[tid] : -1};
        __syncthreads();  // read before the selection reuses both
        take = select_core<DT, G, BAND, 1>(geo, seq, h, k1, j1, tid < nv ? 1u : 0u, nv, K, e, ss, ph, s_band, s_qf);
        const int pos = wg_scan_excl(__popc(take), ss, ph, &total);
        if (take) out[geo.ns + pos] = j1[0];
      } else {
        take = select_core<DT, G, BAND, PER>(geo, seq, h, kr, jr, vmask, nv, K, e, ss, ph, s_band, s_qf);
        const int pos = wg_scan_excl(__popc(take), ss, ph, &total);
        int w = geo.ns + pos;
#pragma unroll
        for (int p = 0; p < PER; ++p)
          if (take & (1u << p)) out[w++] = jr[p];
      }
    }
  }
  // sinks, the chosen candidates in block order (above), recent blocks
  for (int p = tid; p < geo.ns; p += kSelThreads) out[p] = p;
  for (int r = tid; r < geo.nr; r += kSelThreads) out[geo.ns + total + r] = nb - geo.nr + r;
  for (int p = geo.ns + total + geo.nr + tid; p < geo.nsel_max; p += kSelThreads) out[p] = -1;
}

// ===========================================================================
// launcher: scoring + block-wide selection for batches whose largest
// candidate set exceeds one wave's selection (or whose top_k does)
// ===========================================================================
int mfma_err_stride(const Geometry& g) { return (g.mbps + kMfmaChunk - 1) / kMfmaChunk; }

template <int DT, int G, bool BAND>
static void select_per(const Geometry& g, const SeqBatch& b, const uint16_t* q, const float* scores,
                       const float* err, int stride, int chunks, int floor_rank, int max_nc, int32_t* idx,
                       hipStream_t s, Timing* prof) {
  const int per = (g.ns + max_nc + kSelThreads - 1) / kSelThreads;  // blocks 0 .. ns + max_nc - 1
  const dim3 grid(g.hkv, b.n), blk(kSelThreads);
  const size_t lds = BAND ? (size_t)g.mbps * 4 : 0;
  if (per <= 1)
    launch(k_select<DT, G, BAND, 1>, grid, blk, lds, s, prof, kProfTopk, g, b, q, scores, err, stride, chunks, floor_rank, idx);
  else if (per <= 2)
    launch(k_select<DT, G, BAND, 2>, grid, blk, lds, s, prof, kProfTopk, g, b, q, scores, err, stride, chunks, floor_rank, idx);
  else if (per <= 4)
    launch(k_select<DT, G, BAND, 4>, grid, blk, lds, s, prof, kProfTopk, g, b, q, scores, err, stride, chunks, floor_rank, idx);
  else if (per <= 8)
    launch(k_select<DT, G, BAND, 8>, grid, blk, lds, s, prof, kProfTopk, g, b, q, scores, err, stride, chunks, floor_rank, idx);
  else
    launch(k_select<DT, G, BAND, kSelPerMax>, grid, blk, lds, s, prof, kProfTopk, g, b, q, scores, err, stride,
           chunks, floor_rank, idx);
}

template <int DT, int G>
static void select_wide(const Geometry& g, const SeqBatch& b, const uint16_t* q, float* scores,
                        float* err, int max_nc, int32_t* idx, hipStream_t s, Timing* prof) {
  const int chunks = (max_nc + kMfmaChunk - 1) / kMfmaChunk;
  const int stride = mfma_err_stride(g);
  // each chunk's floor_rank-th largest score, so that the chunks hold K
  const int floor_rank = std::min(8, std::max(1, (g.top_k + chunks - 1) / chunks));
  launch(k_score_mfma<DT, G>, dim3(chunks, g.hkv, b.n), dim3(256), 0, s, prof, kProfScore, g, b, q,
         scores, err, stride, floor_rank);
  select_per<DT, G, true>(g, b, q, scores, err, stride, chunks, floor_rank, max_nc, idx, s, prof);
}

hipError_t launch_select_large(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                               float* err, int max_nc, int32_t* idx, hipStream_t s, Timing* prof,
                               bool scores_ready) {
  const uint16_t* qq = (const uint16_t*)q;
  if (!scores_ready && g.group >= 8) {
    if (g.dtype == 0) {
      if (g.group == 8) select_wide<0, 8>(g, b, qq, scores, err, max_nc, idx, s, prof);
      else select_wide<0, 16>(g, b, qq, scores, err, max_nc, idx, s, prof);
    } else {
      if (g.group == 8) select_wide<1, 8>(g, b, qq, scores, err, max_nc, idx, s, prof);
      else select_wide<1, 16>(g, b, qq, scores, err, max_nc, idx, s, prof);
    }
    return hipGetLastError();
  }
  // exact scores already in `scores`
  if (g.dtype == 0) select_per<0, 1, false>(g, b, qq, scores, nullptr, 0, 0, 1, max_nc, idx, s, prof);
  else select_per<1, 1, false>(g, b, qq, scores, nullptr, 0, 0, 1, max_nc, idx, s, prof);
  return hipGetLastError();
}

}  // namespace bsattn
