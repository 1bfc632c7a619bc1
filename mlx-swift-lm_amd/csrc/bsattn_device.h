// bsattn_device.h -- device-side helpers shared by the 16-bit kernels
// (bsattn_kernels.hip) and the affine-quantized kernels (bsattn_quant.hip):
// element conversions, the MFMA wrapper, fragment-major tile addressing,
// the wave-level top-K selection and cross-lane-group reductions.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bsattn_internal.h"

namespace bsattn {


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// element conversions (dtype 0 = fp16, 1 = bf16); RNE on the way down
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float to_f32(uint16_t b) {
  if constexpr (DT == 0) return (float)__builtin_bit_cast(_Float16, b);
  else return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float f) {
  if constexpr (DT == 0) return __builtin_bit_cast(uint16_t, (_Float16)f);
  else return f32_to_bf16_rne(f);
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)from_f32<DT>(lo) | ((uint32_t)from_f32<DT>(hi) << 16);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
// An empty use of a uniform value at this point: its load is issued here
// rather than sunk into a later branch behind other waits.
__device__ __forceinline__ void issue_here(int x) { asm volatile("" ::"s"(x)); }

// tokens batch entry bi attends to, and the element offset of its q / out
// row for query head `head`
__device__ __forceinline__ int entry_len(const Geometry& g, const SeqBatch& sb, int bi, int seq) {
  const int l = sb.len[bi];
  return l >= 0 ? l : g.meta[seq];
}
__device__ __forceinline__ size_t q_row(const SeqBatch& sb, int bi, int head) {
  return (size_t)sb.qoff[bi] + (size_t)head * sb.qhs;
}

__device__ __forceinline__ const int32_t* block_table(const Geometry& g, int seq) {
  return g.meta + g.bt_off + (size_t)seq * g.mbps;
}

// ---------------------------------------------------------------------------
// fragment-major tile addressing (element offsets inside a K or V tile)
//  K: fragment (t, s) for QK token tile t and k-step s; lane (m, g) holds
//     dims 32*s + 8*g .. +7 of token tok_of(m / 4, 4*t + m % 4).
//  V: fragment (dt, s2) for dim tile dt and PV k-step s2; lane (n, g) holds
//     tokens 32*s2 + 8*g .. +7 of dim 16*dt + n.
// tok_of(g, e) = 32*(e/8) + 8*g + e%8 is the token whose score lands in
// accumulator entry e of lane group g (see k_attend).
// ---------------------------------------------------------------------------
__host__ __device__ inline int tok_of(int g, int e) { return 32 * (e >> 3) + 8 * g + (e & 7); }

__host__ __device__ inline int k_elem(int tok, int d) {
  const int e = 8 * (tok >> 5) + (tok & 7);  // accumulator entry of the token
  const int t = e >> 2, m = 4 * ((tok >> 3) & 3) + (e & 3);
  const int s = d >> 5, g = (d >> 3) & 3;
  return (((t * 4 + s) * 64 + m + 16 * g) << 3) + (d & 7);
}

__host__ __device__ inline int v_elem(int tb, int tok, int d) {
  const int ks2 = tb >> 5;
  const int s2 = tok >> 5, g = (tok >> 3) & 3;
  const int dt = d >> 4, n = d & 15;
  return (((dt * ks2 + s2) * 64 + n + 16 * g) << 3) + (tok & 7);
}

// ---------------------------------------------------------------------------
// metadata patch: meta[idx[i]] = val[i]
// Block-score row of (batch entry bi, kv head h): sstride floats, entry j =
// block j (only candidate blocks are written).
__device__ __forceinline__ float* score_row(const Geometry& g, float* scores, int bi, int h) {
  return scores + ((size_t)bi * g.hkv + h) * g.sstride;
}
__device__ __forceinline__ const float* score_row(const Geometry& g, const float* scores, int bi,
                                                  int h) {
  return scores + ((size_t)bi * g.hkv + h) * g.sstride;
}

__device__ __forceinline__ uint16_t* summary_row(const Geometry& g, int seq, int h, int j) {
  return g.summ + (((size_t)seq * g.hkv + h) * g.mbps + j) * kHeadDim;
}

__device__ __forceinline__ uint32_t score_key(float s) {
  if (__builtin_isnan(s)) return 0u;
  if (s == 0.0f) s = 0.0f;
  const uint32_t b = __float_as_uint(s);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int DT>
__device__ __forceinline__ void unpack8(const u32x4 raw, float* out) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    out[e] = to_f32<DT>((uint16_t)((e & 1) ? (raw[e >> 1] >> 16) : (raw[e >> 1] & 0xFFFFu)));
}

// dims 8c .. 8c+7 of one token's key kr and value vr into slot `slot` of the
// (page, kv head h) slab: 16 contiguous bytes of the K tile, eight scattered
// elements of the V tile.  THROUGH: device-scope stores, which write through
// the XCD's L2 at once (for a kernel that writes the token early and runs on:
// the partial lines are then not left to the write-back at its end)
template <bool THROUGH = false>
__device__ __forceinline__ void put_token(const Geometry& g, int page, int h, int slot, int c,
                                          const u32x4 kr, const u32x4 vr) {
  uint8_t* slab = g.pool + ((size_t)page * g.hkv + h) * g.slab_bytes;
  uint16_t* Kt = (uint16_t*)(slab + g.k_off);
  uint16_t* Vt = (uint16_t*)(slab + g.v_off);
  if constexpr (THROUGH) {
    uint64_t* kd = (uint64_t*)(Kt + k_elem(slot, 8 * c));
    __hip_atomic_store(kd, (uint64_t)kr[0] | ((uint64_t)kr[1] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(kd + 1, (uint64_t)kr[2] | ((uint64_t)kr[3] << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *(u32x4*)(Kt + k_elem(slot, 8 * c)) = kr;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = vr[e >> 1];
    const uint16_t x = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xFFFFu));
    uint16_t* vd = Vt + v_elem(g.tb, slot, 8 * c + e);
    if constexpr (THROUGH) __hip_atomic_store(vd, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *vd = x;
  }
}

// dims 8c .. 8c+7 of a full block's summary: the mean of its tb keys (held in
// LDS as blk[token][c]), summed in token order, each add and the final scale
// rounded once in fp32 (the order summary16 follows)
template <int DT>
__device__ __forceinline__ u32x4 fold_block(const u32x4 (*blk)[16], int tb, int c) {
  float acc[8];
  unpack8<DT>(blk[0][c], acc);
  for (int t = 1; t < tb; ++t) {
    float x[8];
    unpack8<DT>(blk[t][c], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __fadd_rn(acc[e], x[e]);
  }
  const float inv = 1.0f / (float)tb;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack2<DT>(__fmul_rn(acc[2 * e], inv), __fmul_rn(acc[2 * e + 1], inv));
  return o;
}

// Candidates are ranked only when they outnumber top_k.
__host__ __device__ inline bool ranked_select(const Geometry& g, int nc) {
  return nc > g.top_k && g.top_k > 0;
}

// x of the lane K places up in the same 16-lane DPP row (row_shl:K); lanes
// whose source falls outside the row get 0
template <int K>
__device__ __forceinline__ float row_shl(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + K, 0xF, 0xF, true));
}

// Canonical dot product of one 128-dim pair held by the 16 lanes of a DPP
// row (lane c = chunk c: dims 8c .. 8c+7): fused left fold of the chunk's 8
// products, then the pairwise tree over chunks, (c, c+1), then (c, c+2),
// (c, c+4), (c, c+8), which lane 0 of the row accumulates through row
// shifts (fp32 addition is commutative, so the order of each pair does not
// matter).  Only lane 0 of the row (c == 0) holds the result.
// Each step is one fused multiply-add, fma(a, b, acc) = round(a*b + acc):
// the normative order (the oracle folds with fmaf the same way).  A product
// of two 16-bit values is exact in fp32 unless it leaves fp32's range (bf16
// only), so this is also the rounded sum of the rounded product there.
template <int DT>
__device__ __forceinline__ float canonical_dot16(const float* a, const float* b) {
  float acc = __fmul_rn(a[0], b[0]);
#pragma unroll
  for (int e = 1; e < 8; ++e) acc = __builtin_fmaf(a[e], b[e], acc);
  acc = __fadd_rn(acc, row_shl<1>(acc));
  acc = __fadd_rn(acc, row_shl<2>(acc));
  acc = __fadd_rn(acc, row_shl<4>(acc));
  acc = __fadd_rn(acc, row_shl<8>(acc));
  return acc;
}

// ---------------------------------------------------------------------------
// wave-level top-K of one (sequence, kv head): the same selection as the
// oracle (K largest keys, ties to the lower index), computed by one wave with
// no workgroup barriers.  Lane l holds candidates c0 + l + 64*k, k < S (S a
// power of two; padded keys are 0 and never counted).  The K-th largest key
// tau is found by a range-adaptive histogram select in LDS (kWaveBins bins
// over the score range, refined inside the bin that holds the K-th key until
// it holds at most 64 keys, which a bitwise search of their offsets
// resolves); keys > tau are taken, and of the keys == tau the lowest indices.
// Candidates c0 .. c0+nc-1, nc <= 64 * S, nc > K > 0.  Writes the K chosen
// block indices, ascending, to sel_blk and their pages (from bt) to sel_page
// when sel_page is not null.  ws: kWaveScratch words of LDS, 16-B aligned.
// ---------------------------------------------------------------------------
constexpr int kSelKeysPerLane = 16;
constexpr int kSelMaxK = 256;  // top_k limit of the in-kernel selection
constexpr int kWaveBins = 1024;
constexpr int kWaveScratch = kWaveBins + 64;

// inverse of score_key; key 0 (NaN) -> -inf
__device__ __forceinline__ float key_value(uint32_t key) {
  if (key == 0u) return -INFINITY;
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// cross-lane moves on the VALU: DPP within 16-lane rows, permlane swaps
// across rows (no LDS round trips)
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, true);
}
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowRor4 = 0x124, kDppRowRor8 = 0x128;
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

template <typename Op>
__device__ __forceinline__ uint32_t wave_allreduce_u32(uint32_t x, Op op) {
  x = op(x, dpp_u32<kDppQuadXor1>(x));
  x = op(x, dpp_u32<kDppQuadXor2>(x));
  x = op(x, dpp_u32<kDppRowRor4>(x));
  x = op(x, dpp_u32<kDppRowRor8>(x));
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = op((uint32_t)a[0], (uint32_t)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return op((uint32_t)b[0], (uint32_t)b[1]);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return wave_allreduce_u32(x, [](uint32_t a, uint32_t b) { return min(a, b); });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return wave_allreduce_u32(x, [](uint32_t a, uint32_t b) { return max(a, b); });
}
__device__ __forceinline__ int wave_sum_i32(int x) {
  return (int)wave_allreduce_u32((uint32_t)x, [](uint32_t a, uint32_t b) { return a + b; });
}
// inclusive prefix sum over the wave's lanes
__device__ __forceinline__ int wave_scan_incl(int v) {
  uint32_t x = (uint32_t)v;
  x += dpp_u32<kDppRowShr1>(x);
  x += dpp_u32<kDppRowShr2>(x);
  x += dpp_u32<kDppRowShr4>(x);
  x += dpp_u32<kDppRowShr8>(x);
  x += dpp_u32<kDppRowBcast15, 0xA>(x);
  x += dpp_u32<kDppRowBcast31, 0xC>(x);
  return (int)x;
}
// orders this wave's LDS accesses (a wave's LDS instructions complete in
// issue order; this keeps the compiler from moving them across)
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The bin of a kWaveBins-bin LDS histogram (bins filled, read-only here)
// that holds the need-th largest key: lane l owns bins kWaveBins-1 - 16l - j,
// j < 16 (descending), so a scan of the lanes' sums counts the keys in
// higher bins; the owning lane's 16 bins are then scanned by 16 lanes.
// b_star: the bin; abv: keys in higher bins; cnt: keys in b_star.
__device__ __forceinline__ void find_kth_bin(const uint32_t* hist, int need, int& b_star, int& abv, int& cnt) {
  constexpr int BPL = kWaveBins / 64;
  const int lane = threadIdx.x & 63;
  const u32x4* r4 = (const u32x4*)(hist + kWaveBins - BPL * (lane + 1));
  int lsum = 0;
#pragma unroll
  for (int i = 0; i < BPL / 4; ++i) {
    const u32x4 v = r4[i];
    lsum += (int)(v[0] + v[1] + v[2] + v[3]);
  }
  const int incl = wave_scan_incl(lsum);
  const int excl = incl - lsum;
  const int src = __ffsll((unsigned long long)__ballot(excl < need && need <= incl)) - 1;
  const int base = __builtin_amdgcn_readlane(excl, src);
  const int ct = lane < BPL ? (int)hist[kWaveBins - 1 - BPL * src - lane] : 0;
  const int ci = wave_scan_incl(ct);
  const int js = __ffsll((unsigned long long)__ballot(lane < BPL && base + ci - ct < need && need <= base + ci)) - 1;
  b_star = kWaveBins - 1 - BPL * src - js;
  abv = base + __builtin_amdgcn_readlane(ci - ct, js);
  cnt = __builtin_amdgcn_readlane(ct, js);
}

template <int S>
__device__ __forceinline__ uint32_t wave_kth_key(const uint32_t (&key)[S], int nc, int K, uint32_t* ws) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
  for (int k = 0; k < S; ++k)
    if (lane + 64 * k < nc) {
      lo = min(lo, key[k]);
      hi = max(hi, key[k]);
    }
  lo = wave_min_u32(lo);
  hi = wave_max_u32(hi);
  int need = K;
  bool by_value = true;
  uint32_t* hist = ws;
  uint32_t* small = ws + kWaveBins;
#pragma unroll 1
  while (true) {
    if (lo == hi) return lo;
    // the first pass bins by score value (keys crowd in a few binary
    // exponents), later passes by key bits
    const float vlo = key_value(lo), span = key_value(hi) - vlo;
    const bool use_v = by_value && __builtin_isfinite(vlo) && __builtin_isfinite(span) && span > 0.0f;
    // bins need only be monotone in the key: an approximate reciprocal will do
    const float scale = use_v ? (float)(kWaveBins - 1) * __builtin_amdgcn_rcpf(span) : 0.0f;
    const int sh = use_v ? 0 : max(0, 32 - __clz(hi - lo) - 10);  // (hi - lo) >> sh < 1024
    auto bin = [&](uint32_t k) -> int {
      return use_v ? min(kWaveBins - 1, (int)((key_value(k) - vlo) * scale)) : (int)((k - lo) >> sh);
    };
    u32x4* h4 = (u32x4*)hist + lane * (kWaveBins / 256);
#pragma unroll
    for (int i = 0; i < kWaveBins / 256; ++i) h4[i] = u32x4{0u, 0u, 0u, 0u};
    wave_lds_order();
    int bk[S];  // each key's bin in this pass, -1 outside the range
#pragma unroll
    for (int k = 0; k < S; ++k) {
      bk[k] = lane + 64 * k < nc && key[k] >= lo && key[k] <= hi ? bin(key[k]) : -1;
      if (bk[k] >= 0) atomicAdd(&hist[bk[k]], 1u);
    }
    wave_lds_order();
    int b_star, abv, cnt;
    find_kth_bin(hist, need, b_star, abv, cnt);
    need -= abv;
    if (!use_v && sh == 0) return lo + (uint32_t)b_star;  // one-value bin
    if (cnt <= 64) {
      // the bin's keys, in any order; a bitwise search of their offsets
      int base = 0;
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const bool in = bk[k] == b_star;
        const uint64_t m = __ballot(in);
        if (in) small[base + __popcll(m & below)] = key[k];
        base += __popcll(m);
      }
      wave_lds_order();
      const bool valid = lane < cnt;
      const uint32_t x = valid ? small[lane] : 0u;
      if (cnt <= 16) {
        // few keys: each lane counts the keys above and at its own; the
        // need-th largest is the key with gt < need <= ge
        int gt = 0, ge = 0;
        for (int jj = 0; jj < cnt; ++jj) {
          const uint32_t xj = (uint32_t)__builtin_amdgcn_readlane((int)x, jj);
          gt += xj > x;
          ge += xj >= x;
        }
        const int src = __ffsll((unsigned long long)__ballot(valid && gt < need && need <= ge)) - 1;
        wave_lds_order();  // the scratch may be reused right after
        return (uint32_t)__builtin_amdgcn_readlane((int)x, src);
      }
      const uint32_t mn = wave_min_u32(valid ? x : 0xFFFFFFFFu), mx = wave_max_u32(x);
      const uint32_t off = x - mn;
      uint32_t t = 0u;
      for (int bit = mx == mn ? -1 : 31 - __clz(mx - mn); bit >= 0; --bit) {
        const uint32_t cand = t | (1u << bit);
        if (__popcll(__ballot(valid && off >= cand)) >= need) t = cand;
      }
      wave_lds_order();  // the scratch may be reused right after
      return mn + t;
    }
    if (use_v) {
      uint32_t nlo = 0xFFFFFFFFu, nhi = 0u;
#pragma unroll
      for (int k = 0; k < S; ++k)
        if (bk[k] == b_star) {
          nlo = min(nlo, key[k]);
          nhi = max(nhi, key[k]);
        }
      lo = wave_min_u32(nlo);
      hi = wave_max_u32(nhi);
    } else {
      const uint32_t nlo = lo + ((uint32_t)b_star << sh);
      const uint32_t span_k = (1u << sh) - 1u;
      hi = (hi - nlo < span_k) ? hi : nlo + span_k;
      lo = nlo;
    }
    by_value = false;
    wave_lds_order();
  }
}

// Raw scores and block-table entries of the candidates c0 + lane + 64*k,
// k < kSelKeysPerLane, loaded before the sequence length is known (the
// score and block-table rows are mbps wide; the remaining slots read 0).
struct WaveCand {
  float score[kSelKeysPerLane];
  int page[kSelKeysPerLane];
};
__device__ __forceinline__ void wave_cand_load(const float* __restrict__ srow,
                                               const int32_t* __restrict__ bt, int c0, int mbps,
                                               WaveCand& wc) {
  const int lane = threadIdx.x & 63;
  // unconditional loads, every score before any page: loads complete in
  // issue order, and a load under a branch is waited for where the branch
  // joins.  Slots past the table read its last row; the selection reads
  // only slots below nc <= mbps - c0.
#pragma unroll
  for (int k = 0; k < kSelKeysPerLane; ++k) wc.score[k] = srow[min(c0 + lane + 64 * k, mbps - 1)];
#pragma unroll
  for (int k = 0; k < kSelKeysPerLane; ++k) wc.page[k] = bt != nullptr ? bt[min(c0 + lane + 64 * k, mbps - 1)] : 0;
}

template <int S>
__device__ __forceinline__ void wave_topk_s(const WaveCand& wc, int c0, int nc, int K, int* sel_blk,
                                            int* sel_page, uint32_t* ws) {
  const int lane = threadIdx.x & 63;
  uint32_t key[S];
#pragma unroll
  for (int k = 0; k < S; ++k) key[k] = lane + 64 * k < nc ? score_key(wc.score[k]) : 0u;
  const uint32_t tau = wave_kth_key<S>(key, nc, K, ws);
  // keys > tau are taken; of the keys == tau, the krem lowest indices
  int gt_total = 0;
  {
    uint64_t m[S];
#pragma unroll
    for (int k = 0; k < S; ++k) m[k] = __ballot(lane + 64 * k < nc && key[k] > tau);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < S; ++k) gt_total += __popcll(m[k]);
  }
  const int krem = K - gt_total;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int sel_before = 0, ties_before = 0;
#pragma unroll
  for (int k = 0; k < S; ++k) {
    const int i = lane + 64 * k;
    const bool real = i < nc;
    const bool eq = real && key[k] == tau;
    const uint64_t eqm = __ballot(eq);
    const bool take = (real && key[k] > tau) || (eq && ties_before + __popcll(eqm & below) < krem);
    const uint64_t tm = __ballot(take);
    if (take) {
      const int pos = sel_before + __popcll(tm & below);
      sel_blk[pos] = c0 + i;
      if (sel_page) sel_page[pos] = wc.page[k];
    }
    sel_before += __popcll(tm);
    ties_before += __popcll(eqm);
  }
}

// S = smallest power of two with 64 * S >= nc (nc <= 64 * kSelKeysPerLane)
__device__ __forceinline__ void wave_topk(const WaveCand& wc, int c0, int nc, int K, int* sel_blk,
                                          int* sel_page, uint32_t* ws) {
  if (nc <= 64) wave_topk_s<1>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if (nc <= 128) wave_topk_s<2>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if (nc <= 256) wave_topk_s<4>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if (nc <= 512) wave_topk_s<8>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else wave_topk_s<16>(wc, c0, nc, K, sel_blk, sel_page, ws);
}

// ---------------------------------------------------------------------------
// workgroup-wide top-K inside the attention workgroup, for candidate sets
// up to 64 * W * kWgKeys: the same selection as wave_topk (K largest keys,
// ties to the lower index), with the candidates spread over all W waves so
// that no wave holds more than kWgKeys per lane.  Slot k of wave w, lane l
// holds candidate c0 + 64 (W k + w) + l, so S = ceil(nc / (64 W)) slots
// carry every candidate and the waves share them evenly.  The histogram
// passes of wave_kth_key run on one LDS histogram that all waves fill;
// every wave then reads the whole histogram and reaches the same decision,
// so only the fills and the small-set compaction need barriers.
// ---------------------------------------------------------------------------
constexpr int kWgKeys = 8;
// LDS words: histogram, small set, small-set count, per-wave lo / hi, and
// per-(slot, wave) counts of keys above / at the threshold
constexpr int kWgScratch = kWaveBins + 64 + 4 + 2 * 16 + 2 * 64;

template <int NK>
struct WgCandT {
  float score[NK];
  int page[NK];
};
using WgCand = WgCandT<kWgKeys>;
// keys per lane the attention workgroup's selection holds: its W waves
// cover the fused selection's 2048 candidates (8 at 4 waves, 4 at 9)
template <int W>
constexpr int attend_keys() {
  return W <= 4 ? kWgKeys : 4;
}
template <int W, int NK = kWgKeys>
__device__ __forceinline__ void wg_cand_load(const float* __restrict__ srow,
                                             const int32_t* __restrict__ bt, int c0, int mbps,
                                             int wave, WgCandT<NK>& wc) {
  const int lane = threadIdx.x & 63;
  // unconditional loads, every score before any page: loads complete in
  // issue order (the selection needs the scores first, the pages only once
  // it is done), and a load under a branch is waited for where the branch
  // joins.  Slots past the table read its last row; the selection reads
  // only slots below nc <= mbps - c0.
#pragma unroll
  for (int k = 0; k < NK; ++k) wc.score[k] = srow[min(c0 + 64 * (W * k + wave) + lane, mbps - 1)];
#pragma unroll
  for (int k = 0; k < NK; ++k)
    wc.page[k] = bt != nullptr ? bt[min(c0 + 64 * (W * k + wave) + lane, mbps - 1)] : 0;
}

template <int S, int W>
__device__ __forceinline__ uint32_t wg_kth_key(const uint32_t (&key)[S], const bool (&real)[S], int K,
                                               uint32_t* ws) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint32_t* hist = ws;
  uint32_t* small = ws + kWaveBins;
  uint32_t* small_n = small + 64;
  uint32_t* xlo = small_n + 4;
  uint32_t* xhi = xlo + 16;
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
  for (int k = 0; k < S; ++k)
    if (real[k]) {
      lo = min(lo, key[k]);
      hi = max(hi, key[k]);
    }
  lo = wave_min_u32(lo);
  hi = wave_max_u32(hi);
  if (lane == 0) {
    xlo[wave] = lo;
    xhi[wave] = hi;
  }
  __syncthreads();
  lo = xlo[0];
  hi = xhi[0];
#pragma unroll
  for (int w = 1; w < W; ++w) {
    lo = min(lo, xlo[w]);
    hi = max(hi, xhi[w]);
  }
  int need = K;
  bool by_value = true;
#pragma unroll 1
  while (true) {
    if (lo == hi) return lo;
    const float vlo = key_value(lo), span = key_value(hi) - vlo;
    const bool use_v = by_value && __builtin_isfinite(vlo) && __builtin_isfinite(span) && span > 0.0f;
    // bins need only be monotone in the key: an approximate reciprocal will do
    const float scale = use_v ? (float)(kWaveBins - 1) * __builtin_amdgcn_rcpf(span) : 0.0f;
    const int sh = use_v ? 0 : max(0, 32 - __clz(hi - lo) - 10);
    auto bin = [&](uint32_t k) -> int {
      return use_v ? min(kWaveBins - 1, (int)((key_value(k) - vlo) * scale)) : (int)((k - lo) >> sh);
    };
    // every wave's previous reads of the histogram and exchange words are
    // done before they are cleared (barrier at the end of the pass)
    for (int i = threadIdx.x; i < kWaveBins / 4; i += 64 * W) ((u32x4*)hist)[i] = u32x4{0u, 0u, 0u, 0u};
    if (threadIdx.x == 0) *small_n = 0u;
    __syncthreads();
    int bk[S];  // each key's bin in this pass, -1 outside the range
#pragma unroll
    for (int k = 0; k < S; ++k) {
      bk[k] = real[k] && key[k] >= lo && key[k] <= hi ? bin(key[k]) : -1;
      if (bk[k] >= 0) atomicAdd(&hist[bk[k]], 1u);
    }
    __syncthreads();
    int b_star, abv, cnt;
    find_kth_bin(hist, need, b_star, abv, cnt);
    need -= abv;
    if (!use_v && sh == 0) return lo + (uint32_t)b_star;  // one-value bin
    if (cnt <= 64) {
      // the bin's keys from every wave, in any order
      int mine_n = 0;
      uint64_t m[S];
#pragma unroll
      for (int k = 0; k < S; ++k) {
        m[k] = __ballot(bk[k] == b_star);
        mine_n += __popcll(m[k]);
      }
      uint32_t base = 0u;
      if (lane == 0 && mine_n > 0) base = atomicAdd(small_n, (uint32_t)mine_n);
      base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
      for (int k = 0; k < S; ++k) {
        if ((m[k] >> lane) & 1ull) small[base + __popcll(m[k] & below)] = key[k];
        base += __popcll(m[k]);
      }
      __syncthreads();
      const bool valid = lane < cnt;
      const uint32_t x = valid ? small[lane] : 0u;
      uint32_t tau;
      if (cnt <= 16) {
        int gt = 0, ge = 0;
        for (int jj = 0; jj < cnt; ++jj) {
          const uint32_t xj = (uint32_t)__builtin_amdgcn_readlane((int)x, jj);
          gt += xj > x;
          ge += xj >= x;
        }
        const int s2 = __ffsll((unsigned long long)__ballot(valid && gt < need && need <= ge)) - 1;
        tau = (uint32_t)__builtin_amdgcn_readlane((int)x, s2);
      } else {
        const uint32_t mn = wave_min_u32(valid ? x : 0xFFFFFFFFu), mx = wave_max_u32(x);
        const uint32_t off = x - mn;
        uint32_t t = 0u;
        for (int bit = mx == mn ? -1 : 31 - __clz(mx - mn); bit >= 0; --bit) {
          const uint32_t cand = t | (1u << bit);
          if (__popcll(__ballot(valid && off >= cand)) >= need) t = cand;
        }
        tau = mn + t;
      }
      __syncthreads();  // the scratch may be reused right after
      return tau;
    }
    if (use_v) {
      uint32_t nlo = 0xFFFFFFFFu, nhi = 0u;
#pragma unroll
      for (int k = 0; k < S; ++k)
        if (bk[k] == b_star) {
          nlo = min(nlo, key[k]);
          nhi = max(nhi, key[k]);
        }
      nlo = wave_min_u32(nlo);
      nhi = wave_max_u32(nhi);
      if (lane == 0) {
        xlo[wave] = nlo;
        xhi[wave] = nhi;
      }
      __syncthreads();
      lo = xlo[0];
      hi = xhi[0];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        lo = min(lo, xlo[w]);
        hi = max(hi, xhi[w]);
      }
    } else {
      const uint32_t nlo = lo + ((uint32_t)b_star << sh);
      const uint32_t span_k = (1u << sh) - 1u;
      hi = (hi - nlo < span_k) ? hi : nlo + span_k;
      lo = nlo;
    }
    by_value = false;
    __syncthreads();
  }
}

// Top-K of candidates c0 .. c0+nc-1 (nc <= 64 * W * S, nc > K > 0) held as
// wg_cand_load left them; writes the K chosen block indices, ascending, to
// sel_blk and their pages to sel_page.  Every wave of the workgroup calls
// it (it contains workgroup barriers); ws: kWgScratch words of LDS.
template <int S, int W, int NK>
__device__ __forceinline__ void wg_topk_s(const WgCandT<NK>& wc, int c0, int nc, int K, int* sel_blk,
                                          int* sel_page, uint32_t* ws) {
  static_assert(S <= NK && S * W <= 64, "slots beyond the loaded keys or the (slot, wave) counts");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t key[S];
  bool real[S];
#pragma unroll
  for (int k = 0; k < S; ++k) {
    real[k] = 64 * (W * k + wave) + lane < nc;
    key[k] = real[k] ? score_key(wc.score[k]) : 0u;
  }
  const uint32_t tau = wg_kth_key<S, W>(key, real, K, ws);
  // per-(slot, wave) counts of keys above and at tau, in candidate order
  uint32_t* cgt = ws + kWaveBins + 64 + 4 + 32;
  uint32_t* ceq = cgt + 64;
  uint64_t gtm[S], eqm[S];
#pragma unroll
  for (int k = 0; k < S; ++k) {
    gtm[k] = __ballot(real[k] && key[k] > tau);
    eqm[k] = __ballot(real[k] && key[k] == tau);
    if (lane == 0) {
      cgt[W * k + wave] = (uint32_t)__popcll(gtm[k]);
      ceq[W * k + wave] = (uint32_t)__popcll(eqm[k]);
    }
  }
  __syncthreads();
  // exclusive prefix over the S * W (slot, wave) groups, one group per lane
  const int gi = lane < S * W ? (int)cgt[lane] : 0, ei = lane < S * W ? (int)ceq[lane] : 0;
  const int ginc = wave_scan_incl(gi), einc = wave_scan_incl(ei);
  const int gt_total = __builtin_amdgcn_readlane(ginc, 63);
  const int krem = K - gt_total;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int k = 0; k < S; ++k) {
    const int f = W * k + wave;
    const int gpre = __builtin_amdgcn_readlane(ginc - gi, f);
    const int epre = __builtin_amdgcn_readlane(einc - ei, f);
    const bool gt = (gtm[k] >> lane) & 1ull, eq = (eqm[k] >> lane) & 1ull;
    const int eb = epre + __popcll(eqm[k] & below);
    const bool take = gt || (eq && eb < krem);
    if (take) {
      const int pos = gpre + __popcll(gtm[k] & below) + min(eb, krem);
      sel_blk[pos] = c0 + 64 * f + lane;
      if (sel_page) sel_page[pos] = wc.page[k];
    }
  }
}

// S = smallest power of two with 64 * W * S >= nc (nc <= 64 * W * NK; the
// callers' hosts keep nc within 64 * W * min(NK, 64 / W), so the S = 8 path
// of a workgroup of more than 8 waves is never taken)
template <int W, int NK>
__device__ __forceinline__ void wg_topk(const WgCandT<NK>& wc, int c0, int nc, int K, int* sel_blk,
                                        int* sel_page, uint32_t* ws) {
  if (nc <= 64 * W) wg_topk_s<1, W, NK>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if (nc <= 128 * W) wg_topk_s<2, W, NK>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if constexpr (NK < 8 || 8 * W > 64) wg_topk_s<4, W, NK>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else if (nc <= 256 * W) wg_topk_s<4, W, NK>(wc, c0, nc, K, sel_blk, sel_page, ws);
  else wg_topk_s<8, W, NK>(wc, c0, nc, K, sel_blk, sel_page, ws);
}

// ---------------------------------------------------------------------------
// The attention workgroup's top-K where each wave needs only its own slot's
// block.  The candidates spread over the W waves as for wg_topk (slot k of
// wave w, lane l holds candidate c0 + 64 g + l, group g = W k + w), and the
// selection is the same (K largest keys, ties to the lower index), with three
// workgroup barriers where wg_topk and the read of its output take seven:
//  1. the waves' key bounds, the histogram cleared behind the same barrier;
//  2. the histogram fill;
//  3. once the bin that holds the K-th key is known: every group's masks of
//     keys above that bin and in it, the page of every candidate that can be
//     taken (above the bin or in it) at a fixed position and, when the bin
//     holds more keys than are still needed and they need not be equal, the
//     bin's keys with their candidate offsets.
// Each wave then finds, per group, its taken blocks (the bin's keys by rank,
// key descending and index ascending; equal keys by index), counts them,
// finds the group and lane of its rank-th selected block, and reads its
// page.  A K-th bin of more than 64 keys takes another histogram pass (two
// barriers more).
// ---------------------------------------------------------------------------
template <int W>
constexpr int slot_scratch_words() {
  return kWaveBins + 2 * 64 + 4 + 2 * 16 + 4 * 64 + 64 * W * attend_keys<W>();
}

template <int S, int W, int NK>
__device__ __forceinline__ void wg_topk_slot_s(const WgCandT<NK>& wc, int c0, int nc, int K, int rank,
                                               int* j_out, int* page_out, int* row, uint32_t* ws) {
  static_assert(S <= NK && S * W <= 64, "slots beyond the loaded keys or the 64 groups");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint32_t* hist = ws;
  uint32_t* small = ws + kWaveBins;  // the K-th bin's keys
  int* small_at = (int*)(small + 64);  // their offsets 64 g + l from c0
  uint32_t* small_n = (uint32_t*)(small_at + 64);
  uint32_t* xlo = small_n + 4;
  uint32_t* xhi = xlo + 16;
  uint64_t* gmask = (uint64_t*)(xhi + 16);
  uint64_t* bmask = gmask + 64;
  int* gpage = (int*)(bmask + 64);
  uint32_t key[S];
  bool real[S];
#pragma unroll
  for (int k = 0; k < S; ++k) {
    real[k] = 64 * (W * k + wave) + lane < nc;
    key[k] = real[k] ? score_key(wc.score[k]) : 0u;
  }
  // 1. bounds; the histogram is cleared behind the same barrier
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
  for (int k = 0; k < S; ++k)
    if (real[k]) {
      lo = min(lo, key[k]);
      hi = max(hi, key[k]);
    }
  lo = wave_min_u32(lo);
  hi = wave_max_u32(hi);
  if (lane == 0) {
    xlo[wave] = lo;
    xhi[wave] = hi;
  }
  for (int i = threadIdx.x; i < kWaveBins / 4; i += 64 * W) ((u32x4*)hist)[i] = u32x4{0u, 0u, 0u, 0u};
  if (threadIdx.x == 0) *small_n = 0u;
  __syncthreads();
  lo = xlo[0];
  hi = xhi[0];
#pragma unroll
  for (int w = 1; w < W; ++w) {
    lo = min(lo, xlo[w]);
    hi = max(hi, xhi[w]);
  }
  // need: the keys still to take from the current range [lo, hi] (every key
  // above it is taken); the loop ends with the bin b_star that holds the
  // need-th largest of them, bk the keys' bins (-1 outside the range) and
  // by_rank set when that bin's keys must be ranked (cnt of them, more than
  // need, not known to be equal)
  int need = K, cnt = 0, b_star = 0;
  int bk[S];
  bool by_value = true, by_rank = false;
#pragma unroll 1
  while (true) {
    if (lo == hi) {  // every key in the range is equal
#pragma unroll
      for (int k = 0; k < S; ++k) bk[k] = real[k] && key[k] == lo ? 0 : -1;
      b_star = 0;
      break;
    }
    const float vlo = key_value(lo), span = key_value(hi) - vlo;
    const bool use_v = by_value && __builtin_isfinite(vlo) && __builtin_isfinite(span) && span > 0.0f;
    // bins need only be monotone in the key: an approximate reciprocal will do
    const float scale = use_v ? (float)(kWaveBins - 1) * __builtin_amdgcn_rcpf(span) : 0.0f;
    const int sh = use_v ? 0 : max(0, 32 - __clz(hi - lo) - 10);
    // a key in a value range is a finite score (NaN keys sit below every
    // finite one), so its bin is taken from the score itself
    auto bin = [&](int k) -> int {
      return use_v ? min(kWaveBins - 1, (int)((wc.score[k] - vlo) * scale)) : (int)((key[k] - lo) >> sh);
    };
    // 2. the histogram
#pragma unroll
    for (int k = 0; k < S; ++k) {
      bk[k] = real[k] && key[k] >= lo && key[k] <= hi ? bin(k) : -1;
      if (bk[k] >= 0) atomicAdd(&hist[bk[k]], 1u);
    }
    __syncthreads();
    int abv;
    find_kth_bin(hist, need, b_star, abv, cnt);
    need -= abv;
    if (!use_v && sh == 0) break;  // one-value bin
    if (cnt <= 64) {
      by_rank = cnt > need;
      break;
    }
    // another pass over the K-th bin: its bounds, then a cleared histogram
    if (use_v) {
      uint32_t nlo = 0xFFFFFFFFu, nhi = 0u;
#pragma unroll
      for (int k = 0; k < S; ++k)
        if (bk[k] == b_star) {
          nlo = min(nlo, key[k]);
          nhi = max(nhi, key[k]);
        }
      nlo = wave_min_u32(nlo);
      nhi = wave_max_u32(nhi);
      if (lane == 0) {
        xlo[wave] = nlo;
        xhi[wave] = nhi;
      }
      __syncthreads();  // every wave has read the histogram; the bounds are in
      lo = xlo[0];
      hi = xhi[0];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        lo = min(lo, xlo[w]);
        hi = max(hi, xhi[w]);
      }
    } else {
      const uint32_t nlo = lo + ((uint32_t)b_star << sh);
      const uint32_t span_k = (1u << sh) - 1u;
      hi = (hi - nlo < span_k) ? hi : nlo + span_k;
      lo = nlo;
      __syncthreads();  // every wave has read the histogram
    }
    for (int i = threadIdx.x; i < kWaveBins / 4; i += 64 * W) ((u32x4*)hist)[i] = u32x4{0u, 0u, 0u, 0u};
    by_value = false;
    __syncthreads();  // cleared; every wave has read the bounds
  }
  // 3. the groups' masks of keys above the K-th bin and in it, every
  // candidate's page, and the bin's keys when they are ranked
  uint64_t inm[S];
  int mine_n = 0;
#pragma unroll
  for (int k = 0; k < S; ++k) {
    const int g = W * k + wave;
    const uint64_t gtm = __ballot(real[k] && (key[k] > hi || bk[k] > b_star));
    inm[k] = __ballot(bk[k] == b_star);
    mine_n += __popcll(inm[k]);
    if (lane == 0) {
      gmask[g] = gtm;
      bmask[g] = inm[k];
    }
    // only a candidate that can be taken is ever looked up
    if (((gtm | inm[k]) >> lane) & 1ull) gpage[64 * g + lane] = wc.page[k];
  }
  if (by_rank) {
    uint32_t base = 0u;
    if (lane == 0 && mine_n > 0) base = atomicAdd(small_n, (uint32_t)mine_n);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
    for (int k = 0; k < S; ++k) {
      if ((inm[k] >> lane) & 1ull) {
        const uint32_t at = base + __popcll(inm[k] & below);
        small[at] = key[k];
        small_at[at] = 64 * (W * k + wave) + lane;
      }
      base += __popcll(inm[k]);
    }
  }
  __syncthreads();
  // lane g: group g's masks; the K-th bin's keys are taken by index (gm
  // above, em at the bin) or, when ranked, moved into gm by rank
  constexpr int NG = S * W;
  uint64_t gm = lane < NG ? gmask[lane] : 0ull, em = lane < NG ? bmask[lane] : 0ull;
  if (by_rank) {
    const bool valid = lane < cnt;
    const uint32_t x = valid ? small[lane] : 0u;
    const int xa = valid ? small_at[lane] : 0;
    int r = 0;
    for (int jj = 0; jj < cnt; ++jj) {
      const uint32_t xj = (uint32_t)__builtin_amdgcn_readlane((int)x, jj);
      const int aj = __builtin_amdgcn_readlane(xa, jj);
      r += (xj > x || (xj == x && aj < xa)) ? 1 : 0;
    }
    uint64_t tk = __ballot(valid && r < need);
    uint64_t bits = 0ull;
    while (tk != 0ull) {
      const int jj = __ffsll((unsigned long long)tk) - 1;
      tk &= tk - 1ull;
      const int aj = __builtin_amdgcn_readlane(xa, jj);
      if ((aj >> 6) == lane) bits |= 1ull << (aj & 63);
    }
    gm |= bits;
    em = 0ull;
  }
  // equal keys at the K-th bin are split by index only when the bin holds
  // more of them than are needed; otherwise every key of the bin is taken
  const bool split_eq = !by_rank && cnt != need;
  if (!split_eq) {
    gm |= em;
    em = 0ull;
  }
  const int ng = __popcll(gm);
  int t_eq = 0;
  if (split_eq) {
    const int ne = __popcll(em);
    const int krem = K - wave_sum_i32(ng);
    const int e_excl = wave_scan_incl(ne) - ne;
    t_eq = min(max(krem - e_excl, 0), ne);
  }
  const int taken = ng + t_eq;
  const int t_excl = wave_scan_incl(taken) - taken;
  auto group_take = [&](uint64_t gms, uint64_t ems, int tq) -> uint64_t {
    // taken lanes of a group: above, or the tq lowest of the K-th bin's
    const bool eb = (ems >> lane) & 1ull;
    const bool take = ((gms >> lane) & 1ull) || (eb && __popcll(ems & below) < tq);
    return __ballot(take);
  };
  if (rank >= 0) {
    const int src = __ffsll((unsigned long long)__ballot(lane < NG && t_excl <= rank && rank < t_excl + taken)) - 1;
    const int r_in = rank - __builtin_amdgcn_readlane(t_excl, src);
    const uint64_t gms = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(gm >> 32), src) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)gm, src);
    const uint64_t ems = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(em >> 32), src) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)em, src);
    const uint64_t tm = group_take(gms, ems, __builtin_amdgcn_readlane(t_eq, src));
    const bool mine = ((tm >> lane) & 1ull) && __popcll(tm & below) == r_in;
    const int b = __ffsll((unsigned long long)__ballot(mine)) - 1;
    *j_out = c0 + 64 * src + b;
    *page_out = gpage[64 * src + b];
  }
  if (row != nullptr) {  // the whole selection, ascending (one wave)
    for (int g = 0; g < NG; ++g) {
      const uint64_t gms = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(gm >> 32), g) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)gm, g);
      const uint64_t ems = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(em >> 32), g) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)em, g);
      const uint64_t tm = group_take(gms, ems, __builtin_amdgcn_readlane(t_eq, g));
      if ((tm >> lane) & 1ull) row[__builtin_amdgcn_readlane(t_excl, g) + __popcll(tm & below)] = c0 + 64 * g + lane;
    }
  }
}

// S = smallest power of two with 64 * W * S >= nc (nc <= 64 * W * NK)
template <int W, int NK>
__device__ __forceinline__ void wg_topk_slot(const WgCandT<NK>& wc, int c0, int nc, int K, int rank, int* j_out,
                                             int* page_out, int* row, uint32_t* ws) {
  if (nc <= 64 * W) wg_topk_slot_s<1, W, NK>(wc, c0, nc, K, rank, j_out, page_out, row, ws);
  else if (nc <= 128 * W) wg_topk_slot_s<2, W, NK>(wc, c0, nc, K, rank, j_out, page_out, row, ws);
  else if constexpr (NK < 8 || 8 * W > 64) wg_topk_slot_s<4, W, NK>(wc, c0, nc, K, rank, j_out, page_out, row, ws);
  else if (nc <= 256 * W) wg_topk_slot_s<4, W, NK>(wc, c0, nc, K, rank, j_out, page_out, row, ws);
  else wg_topk_slot_s<8, W, NK>(wc, c0, nc, K, rank, j_out, page_out, row, ws);
}

// Block in output slot p of the selection for nb blocks: sinks [0, ns),
// then the K ranked candidates (sel), then recent [nb - nr, nb); when the
// candidates do not outnumber K (ranked false) every block is kept.  sel is
// read only when ranked and K > 0.
__device__ __forceinline__ int selected_block(int p, int nb, bool ranked, int ns, int nr, int K,
                                              const int* sel) {
  if (!ranked) return p < nb ? p : -1;
  if (p < ns) return p;
  if (p < ns + K) return sel[p - ns];
  if (p < ns + K + nr) return nb - nr + (p - ns - K);
  return -1;
}

// ---------------------------------------------------------------------------
// wave-level helpers
// ---------------------------------------------------------------------------
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two floats -> packed fp16 / bf16 (v_cvt_pk_*_f32, round to nearest even)
template <int DT>
__device__ __forceinline__ uint32_t cvt_pk(float a, float b) {
  if constexpr (DT == 0) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// {x[l], x[l ^ 16]} and {x[l], x[l ^ 32]} on the VALU (v_permlane*_swap)
__device__ __forceinline__ float max_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ---------------------------------------------------------------------------
// affine-quantized slab (b = 4 or 8 bits; Tb tokens), byte offsets:
//   K codes  [Tb * 128 * b / 8]: per 16-token QK tile t, b/4 fragments of
//            1 KiB; lane (m, g) of the tile's fragments holds, for k-step s,
//            the 8 codes of dims 32*s + 8*g .. +7 of the tile's row m token
//            (int4: one word per k-step, all four in one fragment; int8:
//            two words per k-step, k-steps 2f, 2f+1 in fragment f);
//   V codes  [same]: fragments (dim-tile group, PV k-step s2); lane (n, g)
//            holds, per 16-dim tile dt, the codes of tokens 32*s2 + 8*g .. +7
//            of dim 16*dt + n (int4: one word per dt, four dt per fragment;
//            int8: two words per dt, two dt per fragment);
//   scale / bias [Tb][8 x fp16]: (k scale g0, g1, k bias g0, g1, v scale g0,
//            g1, v bias g0, g1) of a token, at entry sb_entry(tok): lane group
//            g reads its Tb/4 tokens tok_of(g, e) as one contiguous run.
// Inside a 32-bit word, int4 element e (dim or token order) sits in nibble
// q_nib(e), so that (w >> 4k) & 0x000F000F holds elements 2k and 2k+1; int8
// element e sits in byte e.
// ---------------------------------------------------------------------------
__host__ __device__ inline int q_nib(int e) { return (e >> 1) + 4 * (e & 1); }

// byte offset of the code of (tok, d) in the K-code tile; *shift = its bit
// offset inside that byte
__host__ __device__ inline int kq_byte(int bits, int tok, int d, int* shift) {
  const int ea = 8 * (tok >> 5) + (tok & 7);
  const int t = ea >> 2, m = 4 * ((tok >> 3) & 3) + (ea & 3);
  const int s = d >> 5, g = (d >> 3) & 3, e = d & 7;
  const int lane = m + 16 * g;
  if (bits == 4) {
    const int nb = q_nib(e);
    *shift = 4 * (nb & 1);
    return (t * 64 + lane) * 16 + 4 * s + (nb >> 1);
  }
  *shift = 0;
  return ((t * 2 + (s >> 1)) * 64 + lane) * 16 + 4 * (2 * (s & 1) + (e >> 2)) + (e & 3);
}

__host__ __device__ inline int vq_byte(int bits, int tb, int tok, int d, int* shift) {
  const int ks2 = tb >> 5, s2 = tok >> 5, g = (tok >> 3) & 3, e = tok & 7;
  const int dt = d >> 4, lane = (d & 15) + 16 * g;
  if (bits == 4) {
    const int nb = q_nib(e);
    *shift = 4 * (nb & 1);
    return (((dt >> 2) * ks2 + s2) * 64 + lane) * 16 + 4 * (dt & 3) + (nb >> 1);
  }
  *shift = 0;
  return (((dt >> 1) * ks2 + s2) * 64 + lane) * 16 + 4 * (2 * (dt & 1) + (e >> 2)) + (e & 3);
}

__host__ __device__ inline int sb_entry(int tb, int tok) {
  return ((tok >> 3) & 3) * (tb >> 2) + 8 * (tok >> 5) + (tok & 7);
}

// int4 word (element e in nibble q_nib(e)) -> 8 fp16 values 1 + c/16, in
// element order: pair k = elements 2k, 2k+1 = nibbles k, k+4 (the prefill
// kernel's per-workgroup dequantisation)
__device__ __forceinline__ u32x4 nib_to_f16(uint32_t w) {
  constexpr uint32_t M = 0x03C003C0u, ONE = 0x3C003C00u;
  return u32x4{((w << 6) & M) | ONE, ((w << 2) & M) | ONE, ((w >> 2) & M) | ONE,
               ((w >> 6) & M) | ONE};
}


// two int8 words (element e in byte e) -> 8 fp16 values 1024 + c: each
// byte becomes the low byte of an fp16 whose high byte is 0x64
__device__ __forceinline__ u32x4 byte_to_f16(uint32_t lo, uint32_t hi) {
  constexpr uint32_t H = 0x64646464u;
  return u32x4{__builtin_amdgcn_perm(H, lo, 0x04010400u), __builtin_amdgcn_perm(H, lo, 0x04030402u),
               __builtin_amdgcn_perm(H, hi, 0x04010400u), __builtin_amdgcn_perm(H, hi, 0x04030402u)};
}

template <int KB>
struct QCode {
  static constexpr float OFF = KB == 4 ? 1.0f : 1024.0f;  // value of code 0
  static constexpr float INV_UNIT = KB == 4 ? 16.0f : 1.0f;  // 1 / value step
  static constexpr int KF = KB / 4;                          // K fragments per token tile
  static constexpr int DPF = 16 / KB;                        // dim tiles per V fragment
  static constexpr int WPR = kHeadDim * KB / 32;             // MLX words per token row
};

// ---------------------------------------------------------------------------
// attention workgroup plumbing shared by the 16-bit and quantized kernels.
// A workgroup is W waves = W consecutive selected slots of one (sequence,
// kv head); wave w of split `split` handles slot split * W + w.
// ---------------------------------------------------------------------------
// Block (j) and physical page of this wave's slot, -1 when the slot is empty.
// SEL 1 / 2: the selection is computed here from the block scores (1: wave 0
// runs wave_topk over up to 64 * kSelKeysPerLane candidates; 2: every wave
// runs wg_topk_slot over up to 64 * W * attend_keys<W>()), the candidates' block-table
// entries loaded alongside their scores, blocks and pages shared through
// s_sel / s_selp; forced slots load their page before the selection is
// known.  Split 0 then writes the selected indices to idx (if not null).
// Otherwise the block is jg (given_index); -1 and indices past the
// sequence's last block contribute nothing.  Contains a workgroup barrier
// when SEL.
// Block index of a slot in the given-index table (-1 past the table).
__device__ __forceinline__ int given_index(const Geometry& geo, const int32_t* __restrict__ idx,
                                           int bi, int h, int slot) {
  return slot < geo.nsel_max ? idx[((size_t)bi * geo.hkv + h) * geo.nsel_max + slot] : -1;
}

template <int TB, int W, int SEL>
__device__ __forceinline__ void attend_pick(const Geometry& geo, int bi, int h, int seq, int len,
                                            int slot, bool first, int wave, int lane,
                                            int32_t* __restrict__ idx, int jg,
                                            const WaveCand* wc, const WgCandT<attend_keys<W>()>* wgc, int* s_sel,
                                            int* s_selp, uint32_t* s_ws, int& j_out,
                                            int& page_out) {
  int j = -1, page = -1;
  if constexpr (SEL) {
    const int nb = len > 0 ? (len + TB - 1) / TB : 0;
    const int c0 = geo.ns, nc = nb - geo.nr - c0, K = geo.top_k;
    const bool ranked = nc > K;
    const int32_t* bt = block_table(geo, seq);
    // sink / recent / every-block slots are known from the length alone
    const bool picked = ranked && K > 0 && slot >= geo.ns && slot < geo.ns + K;
    if (!picked) {
      j = selected_block(slot, nb, ranked, geo.ns, geo.nr, K, s_sel);
      if (j >= 0) page = uniform(bt[j]);
    }
    if constexpr (SEL == 2) {
      // each wave finds its own slot's block; the first wave of split 0
      // also writes the whole selection for the index row
      if (ranked && K > 0) {
        int jr = -1, pr = -1;
        wg_topk_slot<W>(*wgc, c0, nc, K, picked ? slot - geo.ns : -1, &jr, &pr,
                        idx != nullptr && first ? s_sel : nullptr, s_ws);
        if (picked) {
          j = jr;
          page = pr;
        }
        wave_lds_order();
      }
    } else if (ranked && K > 0) {  // wave 0 selects, the workgroup reads it through LDS
      if (wave == 0) wave_topk(*wc, c0, nc, K, s_sel, s_selp, s_ws);
      __syncthreads();
      if (picked) {
        j = s_sel[slot - geo.ns];
        page = s_selp[slot - geo.ns];
      }
    }
    if (idx != nullptr && first) {
      int32_t* row = idx + ((size_t)bi * geo.hkv + h) * geo.nsel_max;
      for (int p = lane; p < geo.nsel_max; p += 64)
        row[p] = selected_block(p, nb, ranked, geo.ns, geo.nr, K, s_sel);
    }
  } else {
    // the page is requested before the length check: every j in [0, mbps)
    // has an in-bounds table entry; other j read entry 0 and are dropped
    j = uniform(jg);
    const bool in_table = j >= 0 && j < geo.mbps;
    const int pg = uniform(block_table(geo, seq)[in_table ? j : 0]);
    issue_here(pg);
    if (!in_table || (int64_t)j * TB >= len) j = -1;
    if (j >= 0) page = uniform(pg);
  }
  j_out = uniform(j);
  page_out = uniform(page);
}

// Stores one 16-dim tile of this wave's O (MFMA accumulator layout: lane
// (dim n, group g) holds heads 4g .. 4g+3) into s_o[head][dim] (OD < 128:
// a buffer of OD dims, dt counted within it).
template <int G, int OD = kHeadDim>
__device__ __forceinline__ void store_o_tile(float (*s_o)[OD], int dt, int n, int g,
                                             const f32x4& o) {
  if constexpr (G >= 4) {
    if (4 * g < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_o[4 * g + i][16 * dt + n] = o[i];
    }
  } else {
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < G; ++i) s_o[i][16 * dt + n] = o[i];
    }
  }
}

// Per-wave (m, l, o) of an empty slot.
template <int G, int OD = kHeadDim>
__device__ __forceinline__ void store_empty(float* s_m, float* s_l, float (*s_o)[OD], int lane) {
  if (lane < G) {
    s_m[lane] = -INFINITY;
    s_l[lane] = 0.f;
  }
  for (int e = lane; e < G * OD; e += 64) s_o[e / OD][e % OD] = 0.f;
}

// One output element of a merged split: the normalised output (nsplit ==
// 1) or the unnormalised partial (o, m, l) of split `split` of nsplit for
// k_combine.  Wide groups (G >= 8: G heads of partials per split, megabytes
// per launch) store them nontemporally: left dirty in the L2s they are
// written back while the next layer's scoring streams its summaries; narrow
// groups' small partials are cheaper cached, for the combine right after.
// (A runtime choice between the two stores compiles to the cached one.)
template <int DT, int G>
__device__ __forceinline__ void merge_emit(const Geometry& geo, const SeqBatch& sb, int bi, int h,
                                           int split, int nsplit, int head, int d, float M,
                                           float L, float a, uint16_t* __restrict__ out,
                                           float* __restrict__ partials) {
  constexpr bool nt = G >= 8;
  if (nsplit == 1) {
    out[q_row(sb, bi, h * G + head) + d] = from_f32<DT>(L > 0.f ? a / L : 0.f);
  } else {
    const size_t row = (size_t)bi * geo.hq + h * G + head;
    float* pp = partials + (row * nsplit + split) * (kHeadDim + 2);
    if constexpr (nt) {
      __builtin_nontemporal_store(a, pp + d);
      if (d == 0) {
        __builtin_nontemporal_store(M, pp + kHeadDim);
        __builtin_nontemporal_store(L, pp + kHeadDim + 1);
      }
    } else {
      pp[d] = a;
      if (d == 0) {
        pp[kHeadDim] = M;
        pp[kHeadDim + 1] = L;
      }
    }
  }
}

// Thread head < G: the maximum M of head `head` over the W waves, each
// wave's weight exp2(m_w - M) (s_f) and the merged sum L (s_ML).
template <int G, int W>
__device__ __forceinline__ void merge_weights(const float (*s_m)[16], const float (*s_l)[16],
                                              float (*s_f)[16], float (*s_ML)[16]) {
  if (threadIdx.x < G) {
    const int head = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][head]);
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float mw = s_m[w][head];
      const float f = (M == -INFINITY || mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      s_f[w][head] = f;
      L += f * s_l[w][head];
    }
    s_ML[0][head] = M;
    s_ML[1][head] = L;
  }
}

// Dims d0 .. d0 + OD - 1 of the merged split from the waves' outputs in
// s_o[w][head][d - d0], with the weights of merge_weights (behind a
// barrier): each element is sum_w s_f[w][head] * o_w, summed from wave 0 up.
template <int DT, int G, int W, int OD>
__device__ __forceinline__ void merge_dims(const Geometry& geo, const SeqBatch& sb, int bi, int h,
                                           int split, int nsplit, const float (*s_f)[16],
                                           const float (*s_ML)[16], const float (*s_o)[G][OD],
                                           int d0, uint16_t* __restrict__ out,
                                           float* __restrict__ partials) {
  for (int e = threadIdx.x; e < G * OD; e += 64 * W) {
    const int head = e / OD, d = e % OD;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) a += s_f[w][head] * s_o[w][head][d];
    merge_emit<DT, G>(geo, sb, bi, h, split, nsplit, head, d0 + d, s_ML[0][head], s_ML[1][head], a,
                      out, partials);
  }
}

// Merges the W waves' (m, l, o) (after a workgroup barrier) and writes the
// normalised output (nsplit == 1) or the unnormalised partial (o, m, l) of
// split `split` of nsplit for k_combine.
template <int DT, int G, int W>
__device__ __forceinline__ void attend_merge(const Geometry& geo, const SeqBatch& sb, int bi, int h,
                                             int split, int nsplit,
                                             const float (*s_m)[16], const float (*s_l)[16],
                                             const float (*s_o)[G][kHeadDim],
                                             uint16_t* __restrict__ out,
                                             float* __restrict__ partials) {
  // per head: the maximum M over the waves, each wave's weight exp2(m_w - M)
  // and the merged sum L.  With one element per thread every thread computes
  // them for its own head (the same operations in the same order everywhere,
  // so no barrier is needed to share them); otherwise once (thread h < G)
  // behind a barrier.
  if constexpr (G * kHeadDim <= 64 * W) {
    const int e = threadIdx.x;
    if (e < G * kHeadDim) {
      const int head = e / kHeadDim, d = e % kHeadDim;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][head]);
      float L = 0.f, a = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float mw = s_m[w][head];
        const float f = (M == -INFINITY || mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        L += f * s_l[w][head];
        a += f * s_o[w][head][d];
      }
      merge_emit<DT, G>(geo, sb, bi, h, split, nsplit, head, d, M, L, a, out, partials);
    }
  } else {
    __shared__ float s_f[W][16], s_ML[2][16];
    merge_weights<G, W>(s_m, s_l, s_f, s_ML);
    __syncthreads();
    merge_dims<DT, G, W, kHeadDim>(geo, sb, bi, h, split, nsplit, s_f, s_ML, s_o, 0, out, partials);
  }
}

// ---------------------------------------------------------------------------
// host-side launch helper
// ---------------------------------------------------------------------------
// Launches `kernel`; with a profiling slot for its kind, the dispatch itself
// records the slot's start/stop events (hipExtLaunchKernel).
template <typename F, typename... Args>
static void launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Timing* prof,
                   int kind, Args... args) {
  if (prof && prof[kind].start) {
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, prof[kind].start, prof[kind].stop,
                          0u, args...);
    prof[kind].used = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
  }
}

}  // namespace bsattn
