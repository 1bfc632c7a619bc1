// bsattn_kernels.hip -- gfx950 (CDNA4) kernels of the block-sparse decode
// path: append, block summary, block scoring, top-K select, gathered
// split-K attention and the split combine.
//
// Page slab layout (one slab per (physical page, kv head), Tb tokens): the
// K and V tiles are stored in MFMA-fragment-major order, i.e. as the
// sequence of 1 KiB register fragments (64 lanes x 16 B) the attention
// kernel feeds to v_mfma_f32_16x16x32, so every load instruction of the
// gather reads 1 KiB of contiguous memory.  k_elem / v_elem give the element
// offset of (token, dim).  Summaries: [seq][kv head][block][D], by logical
// block, written when a block fills.
//
// Bit-exact parts (summary, score, selection) use __fadd_rn / __fmul_rn so
// the compiler cannot contract or reorder them; the order is the one the
// oracle states (sequential token fold; 16 chunks of 8 dims, then the
// pairwise tree over chunks; max over the GQA group scanning upward).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bsattn_device.h"

namespace bsattn {

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_patch(int32_t* meta, PatchBatch pb) {
  const int t = threadIdx.x;
  if (t < pb.n) meta[pb.idx[t]] = pb.val[t];
}

// ---------------------------------------------------------------------------
// block summary of one (block, kv head) by the 16 lanes that own its dims
// 8c .. 8c+7: sequential fp32 fold over the block's tokens from token 0,
// times 1/Tb, rounded to the cache dtype.  Each lane reads 16 contiguous
// bytes per token (its chunk of the fragment-major K tile).
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void summary16(const Geometry& geo, const uint16_t* __restrict__ Kt, int c,
                                          uint16_t* __restrict__ dst) {
  float acc[8];
  unpack8<DT>(*(const u32x4*)(Kt + k_elem(0, 8 * c)), acc);
#pragma unroll 8
  for (int t = 1; t < geo.tb; ++t) {
    float x[8];
    unpack8<DT>(*(const u32x4*)(Kt + k_elem(t, 8 * c)), x);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __fadd_rn(acc[e], x[e]);
  }
  const float inv = 1.0f / (float)geo.tb;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack2<DT>(__fmul_rn(acc[2 * e], inv), __fmul_rn(acc[2 * e + 1], inv));
  *(u32x4*)(dst + 8 * c) = o;
}

// ---------------------------------------------------------------------------
// append: 16 tokens x 16 lanes (8 dims each) per workgroup.  With
// fuse_summary (one token per sequence: the workgroup's token 0), a token
// that fills its block also writes the block's summary: the whole workgroup
// loads the block's other keys into LDS in one round of loads (the new key
// comes from the registers of the lanes that wrote it), and its 16 lanes then
// fold the block in token order from LDS, as summary16 does from memory.
// grid (ceil(L/16), Hkv, n)
// ---------------------------------------------------------------------------
// Body of one append workgroup: tokens blockIdx.x * 16 .. +15 of entry bi,
// kv head h, starting at position base.  page_given >= 0 is the page of the
// (single) token's block, passed by a caller that patches the block table in
// the same launch; otherwise the page is read from the block table.
template <int DT>
__device__ __forceinline__ void append_body(const Geometry& geo, int seq, int bi, int h, int L,
                                            int base, int page_given,
                                            const uint16_t* __restrict__ k,
                                            const uint16_t* __restrict__ v, bool fuse_summary,
                                            u32x4 (*s_blk)[16]) {
  const int tg = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int tok = blockIdx.x * 16 + tg;
  const int32_t* bt = block_table(geo, seq);
  // the workgroup's token 0 (the only one) fills its block: uniform.  Then
  // the keys of the block's other tokens (written by earlier launches) are
  // requested first, all at once and without a branch (token indices
  // clamped; blocks of 32 or 64 tokens: at most four keys per thread), so
  // that they arrive with the token's own
  const int blk0 = base / geo.tb;
  const bool fills = fuse_summary && base - blk0 * geo.tb == geo.tb - 1;
  u32x4 pre[4];
  if (fills) {
    const int page = page_given >= 0 ? page_given : bt[blk0];
    const uint16_t* Kt =
        (const uint16_t*)(geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes + geo.k_off);
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = *(const u32x4*)(Kt + k_elem(min(tg + 16 * i, geo.tb - 2), 8 * c));
  }
  u32x4 kr = u32x4{0u, 0u, 0u, 0u};
  if (tok < L) {
    const int pos = base + tok;
    const int blk = pos / geo.tb, slot = pos - blk * geo.tb;
    const int page = page_given >= 0 ? page_given : bt[blk];
    const size_t src = (((size_t)bi * geo.hkv + h) * L + tok) * kHeadDim + 8 * c;
    kr = *(const u32x4*)(k + src);
    const u32x4 vr = *(const u32x4*)(v + src);
    put_token(geo, page, h, slot, c, kr, vr);
  }
  if (!fills) return;
  const int blk = blk0;
  // keys 0 .. Tb-2 (loaded above); key Tb-1 is kr of tg 0
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (tg + 16 * i < geo.tb - 1) s_blk[tg + 16 * i][c] = pre[i];
  if (tg == 0) s_blk[geo.tb - 1][c] = kr;
  __syncthreads();
  if (tg != 0) return;
  *(u32x4*)(summary_row(geo, seq, h, blk) + 8 * c) = fold_block<DT>(s_blk, geo.tb, c);
}

template <int DT>
__global__ __launch_bounds__(256) void k_append(Geometry geo, AppendBatch ab,
                                                const uint16_t* __restrict__ k,
                                                const uint16_t* __restrict__ v, bool fuse_summary,
                                                bool device_len) {
  __shared__ u32x4 s_blk[64][16];  // the filled block's keys, [token][8-dim chunk]
  const int bi = blockIdx.z, h = blockIdx.y;
  const int seq = ab.seq[bi];
  // device_len: the position is the device-side length (one token; a
  // sequence without a reserved page for it takes nothing)
  int base = ab.old_len[bi];
  if (device_len) {
    base = geo.meta[seq];
    if (base >= geo.meta[geo.cap_off + seq]) return;
  }
  append_body<DT>(geo, seq, bi, h, ab.L, base, -1, k, v, fuse_summary, s_blk);
}

// ---------------------------------------------------------------------------
// block summaries of the blocks completed by an append: 4 (block, kv head)
// pairs per 64-thread workgroup, 16 lanes each.  Summaries are stored by
// logical block: summ[seq][kv head][block][D].
// grid (max_count, ceil(Hkv / 4), n)
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(64) void k_summary(Geometry geo, SummaryBatch sb) {
  const int bi = blockIdx.z;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 4), c = threadIdx.x & 15;
  if ((int)blockIdx.x >= sb.count[bi] || h >= geo.hkv) return;
  const int seq = sb.seq[bi];
  const int j = sb.first[bi] + blockIdx.x;
  const int page = block_table(geo, seq)[j];
  const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  summary16<DT>(geo, (const uint16_t*)(slab + geo.k_off), c, summary_row(geo, seq, h, j));
}

// ---------------------------------------------------------------------------
// block scoring: workgroup (chunk, kv head, sequence) scores CH (64 or 32)
// candidate blocks of one (sequence, kv head); 16 lanes per block, 8 dims
// per lane; summaries are contiguous by logical block, so every load issues
// up front with no indirection.  Small launches take CH = 32 (twice the
// workgroups, half the serial work per thread).  grid (chunks, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int G, int CH>
__device__ __forceinline__ void score_body(const Geometry& geo, const SeqBatch& sb,
                                           const uint16_t* __restrict__ q,
                                           float* __restrict__ scores, int chunk, int h, int bi) {
  constexpr int P = CH / 16;
  const int tid = threadIdx.x;
  const int seq = sb.ids[bi];
  const int c = tid & 15;
  const int j0 = geo.ns + chunk * CH + (tid >> 4);
  // the query first: loads complete in issue order, so each row's dots
  // below wait only for that row and run while the later rows arrive
  u32x4 qr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qr[g] = *(const u32x4*)(q + q_row(sb, bi, h * G + g) + 8 * c);
  // every row load is issued before the sequence length is known and
  // without a branch: rows are clamped into the table (a row past the
  // candidates is read and not used)
  const uint16_t* sbase = summary_row(geo, seq, h, 0) + 8 * c;
  u32x4 raw[P];
#pragma unroll
  for (int p = 0; p < P; ++p)
    raw[p] = *(const u32x4*)(sbase + (size_t)min(j0 + 16 * p, geo.mbps - 1) * kHeadDim);
  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) unpack8<DT>(qr[g], qv[g]);
  const int len = entry_len(geo, sb, bi, seq);
  const int nb = len > 0 ? (len + geo.tb - 1) / geo.tb : 0;
  const int c1 = nb - geo.nr;
  if (!ranked_select(geo, c1 - geo.ns)) return;
  float* srow = score_row(geo, scores, bi, h);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = j0 + 16 * p;
    if (j < c1) {  // rows are 16-lane aligned: a row enters or skips as a whole
      float sv[8];
      unpack8<DT>(raw[p], sv);
      float best = 0.0f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float acc = canonical_dot16<DT>(qv[g], sv);
        if (g == 0 || acc > best) best = acc;
      }
      if (c == 0) srow[j] = best;
    }
  }
}

template <int DT, int G, int CH>
__global__ __launch_bounds__(256) void k_score(Geometry geo, SeqBatch sb,
                                               const uint16_t* __restrict__ q,
                                               float* __restrict__ scores) {
  score_body<DT, G, CH>(geo, sb, q, scores, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ---------------------------------------------------------------------------
// One decode step's append and scoring in one launch (attentionWithCacheUpdate
// with one new token per sequence): workgroups x = 0 append entry bi's token
// to kv head h (writing the summary of the block it completes), the rest
// score candidate chunk x - 1.  The host patches of this step (lengths,
// capacities, table entries of new pages) are applied here by workgroup
// (0, 0, 0) for the launches that follow; nothing in this launch reads them:
// the append takes its position and page from the arguments, the scoring
// takes each entry's length from sb, and the block an append completes is
// the newest block, which is forced (recent >= 1) and never scored.
// grid (chunks + 1, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int G, int CH>
__global__ __launch_bounds__(256) void k_append_score(Geometry geo, SeqBatch sb, StepPages sp,
                                                      PatchBatch pb, const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ v,
                                                      const uint16_t* __restrict__ q,
                                                      float* __restrict__ scores) {
  __shared__ u32x4 s_blk[64][16];
  const int h = blockIdx.y, bi = blockIdx.z;
  if (blockIdx.x == 0) {
    if (h == 0 && bi == 0 && (int)threadIdx.x < pb.n) geo.meta[pb.idx[threadIdx.x]] = pb.val[threadIdx.x];
    append_body<DT>(geo, sb.ids[bi], bi, h, 1, sb.len[bi] - 1, sp.page[bi], k, v, true, s_blk);
    return;
  }
  score_body<DT, G, CH>(geo, sb, q, scores, blockIdx.x - 1, h, bi);
}

// ---------------------------------------------------------------------------
// top-K select for batches whose candidate sets fit one wave (at most
// 64 * kSelKeysPerLane candidates, top_k <= kSelMaxK): one workgroup per
// (kv head, sequence), one wave selects.  Larger sets go to k_select
// (bsattn_select.hip).  grid (Hkv, n)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_topk(Geometry geo, SeqBatch sb,
                                             const float* __restrict__ scores,
                                             int32_t* __restrict__ idx_out) {
  __shared__ int s_sel[kSelMaxK];
  __shared__ __align__(16) uint32_t s_ws[kWaveScratch];
  const int lane = threadIdx.x;
  const int h = blockIdx.x, bi = blockIdx.y;
  const int seq = sb.ids[bi];
  const int c0 = geo.ns;
  WaveCand wc;
  wave_cand_load(score_row(geo, scores, bi, h), nullptr, c0, geo.mbps, wc);
  const int len = entry_len(geo, sb, bi, seq);
  const int nb = len > 0 ? (len + geo.tb - 1) / geo.tb : 0;
  const int nc = nb - geo.nr - c0;
  const bool ranked = ranked_select(geo, nc);
  int32_t* out = idx_out + ((size_t)bi * geo.hkv + h) * geo.nsel_max;
  if (ranked) wave_topk(wc, c0, nc, geo.top_k, s_sel, nullptr, s_ws);
  // (top_k 0 with candidates: sinks and recent only, no selection)
  for (int p = lane; p < geo.nsel_max; p += 64)
    out[p] = selected_block(p, nb, nc > geo.top_k, geo.ns, geo.nr, geo.top_k, s_sel);
}

// ---------------------------------------------------------------------------
// gathered attention.  Workgroup = W waves = W consecutive selected slots of
// one (sequence, kv head); each wave does one block with MFMA 16x16x32:
//   S^T[token][head] = K[token][:] . Q[head][:]       (A = K rows, B = Q^T)
//   O[head][dim]     = P[head][token] . V[token][dim] (A = P,      B = V)
// The contraction index may be permuted freely as long as A and B agree:
//  - QK, k-step s, lane group g: head dims 32*s + 8*g .. +7;
//  - the QK tile rows are ordered so that the S accumulator of lane (head n,
//    group g) holds tokens tok_of(g, e), e = 0..Tb/4-1, which is the
//    A-operand layout PV needs (no shuffles).
// The tiles are stored fragment-major, so each K/V load is 1 KiB contiguous,
// and every K/V load of a wave is issued before the first wait (a scheduling
// barrier keeps the compiler from interleaving them with the MFMAs).
// bf16: P is split into hi + lo bf16 parts (two MFMAs) for ~16-bit P.
// SEL 1 / 2: the selection is computed here from the block scores instead
// of being read from idx (1: wave 0 runs wave_topk; 2: all W waves run
// wg_topk, each holding a share of the candidates), loading the candidates'
// block-table entries alongside their scores and sharing blocks and pages
// through LDS; split 0 then writes the selected indices to idx (if not
// null).  SEL 0: the blocks are read from idx.
// With more than one split, each workgroup writes an unnormalised partial
// (o, m, l) for k_combine.  grid (nsplit, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int TB, int G, int W, int SEL>
__global__ __launch_bounds__(64 * W, W > 4 ? 1 : 3) void k_attend(Geometry geo, SeqBatch sb,
                                                   const uint16_t* __restrict__ q,
                                                   int32_t* __restrict__ idx,
                                                   const float* __restrict__ scores,
                                                   float sl2, uint16_t* __restrict__ out,
                                                   float* __restrict__ partials) {
  constexpr int NT = TB / 16;   // QK token tiles
  constexpr int EPL = TB / 4;   // scores per lane
  constexpr int KS2 = TB / 32;  // PV k-steps
  __shared__ float s_m[W][16], s_l[W][16];
  __shared__ float s_o[W][G][kHeadDim];
  __shared__ int s_sel[SEL ? kSelMaxK : 1];
  __shared__ int s_selp[SEL ? kSelMaxK : 1];
  __shared__ __align__(16) uint32_t s_ws[SEL == 2 ? slot_scratch_words<W>() : SEL ? kWaveScratch : 4];
  const int split = blockIdx.x, h = blockIdx.y, bi = blockIdx.z;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int seq = sb.ids[bi];
  const int slot = split * W + wave;
  // given indices: the slot's block index heads the longest dependent chain
  // (index -> page -> K/V), so it is requested before the length and Q
  const int jg = SEL ? -1 : given_index(geo, idx, bi, h, slot);
  u32x4 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = u32x4{0u, 0u, 0u, 0u};
  if (n < G) {
    const uint16_t* src = q + q_row(sb, bi, h * G + n) + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *(const u32x4*)(src + 32 * s);
  }
  // the selecting wave loads every candidate's score and page before the
  // sequence length is known
  WaveCand wc;
  WgCandT<attend_keys<W>()> wgc;
  if constexpr (SEL == 1) {
    if (wave == 0)
      wave_cand_load(score_row(geo, scores, bi, h), block_table(geo, seq), geo.ns,
                     geo.mbps, wc);
  } else if constexpr (SEL == 2) {
    wg_cand_load<W, attend_keys<W>()>(score_row(geo, scores, bi, h), block_table(geo, seq), geo.ns,
                                      geo.mbps, wave,
                    wgc);
  }
  const int len = uniform(entry_len(geo, sb, bi, seq));
  int j, page;
  attend_pick<TB, W, SEL>(geo, bi, h, seq, len, slot, split == 0 && wave == 0, wave, lane, idx, jg, &wc,
                          &wgc, s_sel, s_selp, s_ws, j, page);
  if (j >= 0) {
    const int valid = min(TB, len - j * TB);
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
    // fragment-major tiles: fragment f of lane l is 16 B at (f * 64 + l) * 16
    const u32x4* Kf = (const u32x4*)(slab + geo.k_off) + lane;
    const u32x4* Vf = (const u32x4*)(slab + geo.v_off) + lane;
    u32x4 kf[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[t][s] = __builtin_nontemporal_load(Kf + (t * 4 + s) * 64);
    u32x4 vf[8][KS2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) vf[dt][s2] = __builtin_nontemporal_load(Vf + (dt * KS2 + s2) * 64);
    __builtin_amdgcn_sched_barrier(0);
    // S^T = K . Q^T
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[t] = mfma16x16x32<DT>(kf[t][s], qf[s], acc[t]);
    }
    // softmax over this block (log2 domain); lanes of padded heads (n >= G)
    // see S = 0 and produce rows of O that are never stored
    float pv[EPL];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) pv[4 * t + i] = acc[t][i] * sl2;
    if (valid < TB) {
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        if (tok_of(g, e) >= valid) pv[e] = -INFINITY;
    }
    float mx = pv[0];
#pragma unroll
    for (int e = 1; e < EPL; ++e) mx = fmaxf(mx, pv[e]);
    mx = max_over_groups(mx);
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      pv[e] = __builtin_amdgcn_exp2f(pv[e] - mx);
      ps += pv[e];
    }
    ps = sum_over_groups(ps);
    // P operand (A): lane (head n, group g), k-step s2, elements 2*jj, 2*jj+1
    // -> tokens tok_of(g, 8*s2 + 2*jj (+1)) = 32*s2 + 8*g + 2*jj (+1)
    u32x4 pf[KS2];
    u32x4 pl[KS2];
#pragma unroll
    for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float p0 = pv[8 * s2 + 2 * jj], p1 = pv[8 * s2 + 2 * jj + 1];
        const uint32_t hi = cvt_pk<DT>(p0, p1);
        pf[s2][jj] = hi;
        if constexpr (DT == 1)
          pl[s2][jj] = cvt_pk<1>(p0 - __uint_as_float(hi << 16), p1 - __uint_as_float(hi & 0xFFFF0000u));
      }
    // zero V of tokens past the end of a partial block (stale page data)
    if (valid < TB) {
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int t0 = 32 * s2 + 8 * g + 2 * jj;
          const uint32_t m = (t0 < valid ? 0x0000FFFFu : 0u) | (t0 + 1 < valid ? 0xFFFF0000u : 0u);
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) vf[dt][s2][jj] &= m;
        }
    }
    // O = P . V; lane (dim n, group g) holds O rows (heads) 4g .. 4g+3
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) {
        o = mfma16x16x32<DT>(pf[s2], vf[dt][s2], o);
        if constexpr (DT == 1) o = mfma16x16x32<DT>(pl[s2], vf[dt][s2], o);
      }
      store_o_tile<G>(s_o[wave], dt, n, g, o);
    }
    if (g == 0 && n < G) {
      s_m[wave][n] = mx;
      s_l[wave][n] = ps;
    }
  } else {
    store_empty<G>(s_m[wave], s_l[wave], s_o[wave], lane);
  }
  __syncthreads();
  attend_merge<DT, G, W>(geo, sb, bi, h, split, (int)gridDim.x, s_m, s_l, s_o, out, partials);
}

// ---------------------------------------------------------------------------
// combine split partials: one workgroup per (q head, sequence).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_reduce_128(float v, bool is_max, float* s_red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, u) : v + u;
  }
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = is_max ? fmaxf(s_red[0], s_red[1]) : s_red[0] + s_red[1];
  __syncthreads();
  return v;
}

template <int DT>
__global__ __launch_bounds__(128) void k_combine(Geometry geo, SeqBatch sb,
                                                 const float* __restrict__ partials,
                                                 uint16_t* __restrict__ out, int nsplit) {
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[2];
  const int hq = blockIdx.x, bi = blockIdx.y, d = threadIdx.x;
  const size_t row = (size_t)bi * geo.hq + hq;
  const int ns = nsplit;
  const float* pp = partials + row * ns * (kHeadDim + 2);
  float M = -INFINITY;
  for (int sp = d; sp < ns; sp += 128) M = fmaxf(M, pp[sp * (kHeadDim + 2) + kHeadDim]);
  M = block_reduce_128(M, true, s_red);
  float wl = 0.f;
  for (int sp = d; sp < ns; sp += 128) {
    const float m = pp[sp * (kHeadDim + 2) + kHeadDim];
    const float w = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - M);
    s_w[sp] = w;
    wl += w * pp[sp * (kHeadDim + 2) + kHeadDim + 1];
  }
  wl = block_reduce_128(wl, false, s_red);  // also orders the s_w writes
  const float inv = wl > 0.f ? 1.f / wl : 0.f;
  float a = 0.f;
  for (int sp = 0; sp < ns; ++sp) a += s_w[sp] * pp[sp * (kHeadDim + 2) + d];
  out[q_row(sb, bi, hq) + d] = from_f32<DT>(a * inv);
}

// The same combine for nsplit <= NS <= 128 with every load issued first:
// thread t loads (m, l) of split t, then o[d] of every split into registers
// (split indices clamped to nsplit - 1, so no load sits under a branch).
// Loads complete in issue order, so the weights (one exp2 per split, shared
// through LDS) wait only for (m, l) while the o loads arrive; M, the sum and
// o are reduced in the order of k_combine, with the same result.
template <int DT, int NS>
__global__ __launch_bounds__(128) void k_combine_x(Geometry geo, SeqBatch sb,
                                                   const float* __restrict__ partials,
                                                   uint16_t* __restrict__ out, int nsplit) {
  static_assert(NS <= 128, "one split's (m, l) per thread");
  __shared__ float s_w[NS];
  __shared__ float s_red[2];
  const int hq = blockIdx.x, bi = blockIdx.y, d = threadIdx.x;
  const float* pp = partials + ((size_t)bi * geo.hq + hq) * nsplit * (kHeadDim + 2);
  const float* pd = pp + min(d, nsplit - 1) * (kHeadDim + 2);
  const float md = pd[kHeadDim], ld = pd[kHeadDim + 1];
  float o[NS];
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) o[sp] = pp[min(sp, nsplit - 1) * (kHeadDim + 2) + d];
  const bool mine = d < nsplit;
  const float M = block_reduce_128(mine ? fmaxf(-INFINITY, md) : -INFINITY, true, s_red);
  const float w = (!mine || md == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(md - M);
  if (d < NS) s_w[d] = w;
  const float wl = block_reduce_128(mine ? 0.f + w * ld : 0.f, false, s_red);  // also orders the s_w writes
  const float inv = wl > 0.f ? 1.f / wl : 0.f;
  float a = 0.f;
#pragma unroll
  for (int sp = 0; sp < NS; ++sp)
    if (sp < nsplit) a += s_w[sp] * o[sp];
  out[q_row(sb, bi, hq) + d] = from_f32<DT>(a * inv);
}

// The same combine for nsplit <= NS in one round of loads: every thread
// (dim d) loads all splits' (m, l, o[d]) at once (the m / l loads of a wave
// share one address) and reduces them in registers, with no LDS or barriers.
template <int DT, int NS>
__global__ __launch_bounds__(128) void k_combine_r(Geometry geo, SeqBatch sb,
                                                   const float* __restrict__ partials,
                                                   uint16_t* __restrict__ out, int nsplit) {
  const int hq = blockIdx.x, bi = blockIdx.y, d = threadIdx.x;
  const float* pp = partials + ((size_t)bi * geo.hq + hq) * nsplit * (kHeadDim + 2);
  float m[NS], l[NS], o[NS];
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) {
    const bool v = sp < nsplit;
    m[sp] = v ? pp[sp * (kHeadDim + 2) + kHeadDim] : -INFINITY;
    l[sp] = v ? pp[sp * (kHeadDim + 2) + kHeadDim + 1] : 0.f;
    o[sp] = v ? pp[sp * (kHeadDim + 2) + d] : 0.f;
  }
  float M = m[0];
#pragma unroll
  for (int sp = 1; sp < NS; ++sp) M = fmaxf(M, m[sp]);
  float L = 0.f, a = 0.f;
#pragma unroll
  for (int sp = 0; sp < NS; ++sp) {
    const float w = (m[sp] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[sp] - M);
    L += w * l[sp];
    a += w * o[sp];
  }
  out[q_row(sb, bi, hq) + d] = from_f32<DT>(a * (L > 0.f ? 1.f / L : 0.f));
}

// ---------------------------------------------------------------------------
// export: pages -> [n, Hkv, T, D]; grid (ceil(T/16), Hkv, n)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_export(Geometry geo, SeqBatch sb, int T,
                                                uint16_t* __restrict__ ko,
                                                uint16_t* __restrict__ vo) {
  const int bi = blockIdx.z, h = blockIdx.y;
  const int tok = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  if (tok >= T) return;
  const int seq = sb.ids[bi];
  const int blk = tok / geo.tb, slot = tok - blk * geo.tb;
  const int page = block_table(geo, seq)[blk];
  const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  const size_t dst = (((size_t)bi * geo.hkv + h) * T + tok) * kHeadDim + 8 * c;
  *(u32x4*)(ko + dst) = *(const u32x4*)((const uint16_t*)(slab + geo.k_off) + k_elem(slot, 8 * c));
  const uint16_t* Vt = (const uint16_t*)(slab + geo.v_off);
  u32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = (uint32_t)Vt[v_elem(geo.tb, slot, 8 * c + 2 * e)] |
           ((uint32_t)Vt[v_elem(geo.tb, slot, 8 * c + 2 * e + 1)] << 16);
  *(u32x4*)(vo + dst) = w;
}

// summaries of one sequence -> [Hkv, nfull, D]; grid (nfull, Hkv)
__global__ __launch_bounds__(128) void k_export_summaries(Geometry geo, int seq, int nfull,
                                                          uint16_t* __restrict__ out) {
  const int j = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  out[((size_t)h * nfull + j) * kHeadDim + d] = summary_row(geo, seq, h, j)[d];
}

// ===========================================================================
// launchers
// ===========================================================================
hipError_t launch_patch(const Geometry& g, const PatchBatch& pb, hipStream_t s) {
  hipLaunchKernelGGL(k_patch, dim3(1), dim3(256), 0, s, g.meta, pb);
  return hipGetLastError();
}

hipError_t launch_append(const Geometry& g, const AppendBatch& ab, const void* k, const void* v,
                         bool fuse_summary, hipStream_t s, Timing* prof) {
  dim3 grid((ab.L + 15) / 16, g.hkv, ab.n);
  const uint16_t *kk = (const uint16_t*)k, *vv = (const uint16_t*)v;
  if (g.dtype == 0) launch(k_append<0>, grid, dim3(256), 0, s, prof, kProfAppend, g, ab, kk, vv, fuse_summary, false);
  else launch(k_append<1>, grid, dim3(256), 0, s, prof, kProfAppend, g, ab, kk, vv, fuse_summary, false);
  return hipGetLastError();
}

// advances the device-side length of each listed sequence by one token when
// a reserved page held it (after k_append's device-length step)
__global__ __launch_bounds__(64) void k_advance(Geometry geo, AppendBatch ab) {
  for (int i = threadIdx.x; i < ab.n; i += 64) {
    const int seq = ab.seq[i];
    const int len = geo.meta[seq];
    if (len < geo.meta[geo.cap_off + seq]) geo.meta[seq] = len + 1;
  }
}

hipError_t launch_append_step(const Geometry& g, const AppendBatch& ab, const void* k, const void* v,
                              hipStream_t s, Timing* prof) {
  dim3 grid(1, g.hkv, ab.n);
  const uint16_t *kk = (const uint16_t*)k, *vv = (const uint16_t*)v;
  if (g.dtype == 0) launch(k_append<0>, grid, dim3(256), 0, s, prof, kProfAppend, g, ab, kk, vv, true, true);
  else launch(k_append<1>, grid, dim3(256), 0, s, prof, kProfAppend, g, ab, kk, vv, true, true);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, g, ab);
  return hipGetLastError();
}

hipError_t launch_summary(const Geometry& g, const SummaryBatch& sb, int max_count,
                          hipStream_t s, Timing* prof) {
  if (g.kv_bits != 0) return launch_summary_q(g, sb, max_count, s, prof);
  dim3 grid(max_count, (g.hkv + 3) / 4, sb.n);
  if (g.dtype == 0)
    launch(k_summary<0>, grid, dim3(64), 0, s, prof, kProfSummary, g, sb);
  else
    launch(k_summary<1>, grid, dim3(64), 0, s, prof, kProfSummary, g, sb);
  return hipGetLastError();
}

template <int DT, int CH>
static void score_dispatch(const Geometry& g, const SeqBatch& b, int max_nc, const uint16_t* q,
                           float* sc, hipStream_t s, Timing* prof) {
  const dim3 grid((max_nc + CH - 1) / CH, g.hkv, b.n), blk(256);
  switch (g.group) {
    case 1: launch(k_score<DT, 1, CH>, grid, blk, 0, s, prof, kProfScore, g, b, q, sc); break;
    case 2: launch(k_score<DT, 2, CH>, grid, blk, 0, s, prof, kProfScore, g, b, q, sc); break;
    case 4: launch(k_score<DT, 4, CH>, grid, blk, 0, s, prof, kProfScore, g, b, q, sc); break;
    case 8: launch(k_score<DT, 8, CH>, grid, blk, 0, s, prof, kProfScore, g, b, q, sc); break;
    default: launch(k_score<DT, 16, CH>, grid, blk, 0, s, prof, kProfScore, g, b, q, sc); break;
  }
}

template <int DT, int CH>
static void append_score_dispatch(const Geometry& g, const SeqBatch& b, const StepPages& sp,
                                  const PatchBatch& pb, int chunks, const uint16_t* k,
                                  const uint16_t* v, const uint16_t* q, float* sc, hipStream_t s,
                                  Timing* prof) {
  const dim3 grid(chunks + 1, g.hkv, b.n), blk(256);
  switch (g.group) {
    case 1: launch(k_append_score<DT, 1, CH>, grid, blk, 0, s, prof, kProfScore, g, b, sp, pb, k, v, q, sc); break;
    case 2: launch(k_append_score<DT, 2, CH>, grid, blk, 0, s, prof, kProfScore, g, b, sp, pb, k, v, q, sc); break;
    case 4: launch(k_append_score<DT, 4, CH>, grid, blk, 0, s, prof, kProfScore, g, b, sp, pb, k, v, q, sc); break;
    case 8: launch(k_append_score<DT, 8, CH>, grid, blk, 0, s, prof, kProfScore, g, b, sp, pb, k, v, q, sc); break;
    default: launch(k_append_score<DT, 16, CH>, grid, blk, 0, s, prof, kProfScore, g, b, sp, pb, k, v, q, sc); break;
  }
}

int candidates(const Geometry& g, int len) {
  const int nb = len > 0 ? (len + g.tb - 1) / g.tb : 0;
  return nb - g.nr - g.ns;
}

static bool wave_selectable(const Geometry& g, int max_nc) {
  return max_nc <= 64 * kSelKeysPerLane && g.top_k <= kSelMaxK;
}

// exact (canonical) scores of every ranked candidate
hipError_t launch_score(const Geometry& g, const SeqBatch& b, const void* q, float* scores, int max_nc,
                        hipStream_t s, Timing* prof) {
  if (!ranked_select(g, max_nc)) return hipSuccess;
  // 32-candidate chunks while the 64-candidate grid has at most 1024
  // workgroups (8 sequences x 8 kv heads at 32k tokens: 512 -> 1024
  // workgroups, ~0.4 us faster; 4 x 8 at 131k tokens, 1024 -> 2048: 0.2 us
  // per layer-step faster; grids of thousands of workgroups are issue-bound
  // and keep 64)
  const bool small = (int64_t)((max_nc + 63) / 64) * g.hkv * b.n <= 1024;
  const uint16_t* qq = (const uint16_t*)q;
  if (g.dtype == 0) {
    if (small) score_dispatch<0, 32>(g, b, max_nc, qq, scores, s, prof);
    else score_dispatch<0, 64>(g, b, max_nc, qq, scores, s, prof);
  } else {
    if (small) score_dispatch<1, 32>(g, b, max_nc, qq, scores, s, prof);
    else score_dispatch<1, 64>(g, b, max_nc, qq, scores, s, prof);
  }
  return hipGetLastError();
}

hipError_t launch_select(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                         float* err, int32_t* idx, int max_nc, hipStream_t s, Timing* prof) {
  const bool small = wave_selectable(g, max_nc);
  if (!small && g.group >= 8)  // MFMA scores + exact rescoring of the band
    return launch_select_large(g, b, q, scores, err, max_nc, idx, s, prof, false);
  hipError_t e = launch_score(g, b, q, scores, max_nc, s, prof);
  if (e != hipSuccess) return e;
  if (!small) return launch_select_large(g, b, q, scores, err, max_nc, idx, s, prof, true);
  launch(k_topk, dim3(g.hkv, b.n), dim3(64), 0, s, prof, kProfTopk, g, b, (const float*)scores, idx);
  return hipGetLastError();
}

template <int DT, int TB, int SEL, int W>
static void attend_dispatch_w(const Geometry& g, dim3 grid, const SeqBatch& b, const uint16_t* q,
                              int32_t* idx, const float* sc, float sl2, uint16_t* out, float* part,
                              hipStream_t s, Timing* prof) {
  const dim3 blk(64 * W);
  const int kd = kProfAttend;
  if constexpr (W != kWaves) {  // the wide workgroup serves groups of up to 4 heads
    switch (g.group) {
      case 1: launch(k_attend<DT, TB, 1, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      case 2: launch(k_attend<DT, TB, 2, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      default: launch(k_attend<DT, TB, 4, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    }
  } else {
    switch (g.group) {
      case 1: launch(k_attend<DT, TB, 1, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      case 2: launch(k_attend<DT, TB, 2, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      case 4: launch(k_attend<DT, TB, 4, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      case 8: launch(k_attend<DT, TB, 8, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      default: launch(k_attend<DT, TB, 16, W, SEL>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    }
  }
}

template <int DT, int TB, int SEL>
static void attend_dispatch(const Geometry& g, int waves, dim3 grid, const SeqBatch& b, const uint16_t* q,
                            int32_t* idx, const float* sc, float sl2, uint16_t* out, float* part,
                            hipStream_t s, Timing* prof) {
  if constexpr (SEL != 1) {  // one selecting wave runs in kWaves-wave workgroups only
    if (waves == kWavesWide) {
      attend_dispatch_w<DT, TB, SEL, kWavesWide>(g, grid, b, q, idx, sc, sl2, out, part, s, prof);
      return;
    }
  }
  attend_dispatch_w<DT, TB, SEL, kWaves>(g, grid, b, q, idx, sc, sl2, out, part, s, prof);
}

int attend_waves(const Geometry& g, int nseq) {
  // the wide workgroup: groups of up to 4 heads, and splits that fit one
  // workgroup per CU (quantized 16-head groups of 32-token blocks, whose
  // wide workgroup holds half its outputs in LDS at a time and fits 72
  // VGPRs: two per CU); then only where no CU
  // holds more waves than with kWaves-wave workgroups spread over the CUs.
  // (Its fused selection holds 64 * kWavesWide * attend_keys = 2304
  // candidates, more than the 2048 a decode selects inside the attention
  // kernel; beyond those it takes the given-index kernel, as kWaves does.)
  const bool two = g.kv_bits != 0 && g.group == 16 && g.tb == 32;
  if (kWaves != 4 || (g.group > 4 && !two) || g.cus <= 0) return kWaves;
  const int64_t pairs = (int64_t)std::min(std::max(nseq, 1), kMaxBatch) * g.hkv;
  const int64_t wide = pairs * ((g.nsel_max + kWavesWide - 1) / kWavesWide);
  const int64_t per_cu = (wide + g.cus - 1) / g.cus;
  if (per_cu > (two ? 2 : 1)) return kWaves;
  const int64_t base = pairs * g.nsplit;
  const int64_t base_waves = (int64_t)kWaves * ((base + g.cus - 1) / g.cus);
  return kWavesWide * per_cu < base_waves ? kWavesWide : kWaves;
}

template <int SEL>
static hipError_t attend_impl(const Geometry& g, const SeqBatch& b, const void* q, int32_t* idx,
                              const float* scores, int waves, float scale, void* out, float* partials,
                              hipStream_t s, Timing* prof) {
  const float sl2 = scale * 1.4426950408889634f;
  // splits of this launch: the partial workspace holds g.nsplit (kWaves-wave) splits, the most
  const int nsplit = (g.nsel_max + waves - 1) / waves;
  dim3 grid(nsplit, g.hkv, b.n);
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* oo = (uint16_t*)out;
  if (g.kv_bits != 0) {
    hipError_t e = launch_attend_q(g, b, q, idx, scores, SEL, waves, sl2, out, partials, s, prof);
    if (e != hipSuccess) return e;
  } else if (g.dtype == 0) {
    if (g.tb == 64) attend_dispatch<0, 64, SEL>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
    else attend_dispatch<0, 32, SEL>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
  } else {
    if (g.tb == 64) attend_dispatch<1, 64, SEL>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
    else attend_dispatch<1, 32, SEL>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  return launch_combine(g, b, partials, nsplit, out, s, prof);
}

template <int DT>
static void combine_dispatch(const Geometry& g, const SeqBatch& b, const float* partials, int nsplit,
                             uint16_t* oo, hipStream_t s, Timing* prof) {
  const dim3 grid(g.hq, b.n), blk(128);
  const int kc = kProfCombine;
  // one round of loads: up to 16 splits with every split's (m, l) in each
  // thread (8 sequences x 32 heads, 9 splits: 4.1 against 4.3 us for the
  // loop), up to 64 with one exp2 per split shared through LDS (17 splits:
  // 4.0 against 4.3 us, 34: 4.1 against 4.6 us; 34 splits take the 40-split
  // form, 6 clamped loads per thread rather than 14); the loop beyond
  if (nsplit <= 8) launch(k_combine_r<DT, 8>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else if (nsplit <= 16) launch(k_combine_r<DT, 16>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else if (nsplit <= 32) launch(k_combine_x<DT, 32>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else if (nsplit <= 40) launch(k_combine_x<DT, 40>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else if (nsplit <= 48) launch(k_combine_x<DT, 48>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else if (nsplit <= 64) launch(k_combine_x<DT, 64>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
  else launch(k_combine<DT>, grid, blk, 0, s, prof, kc, g, b, partials, oo, nsplit);
}

hipError_t launch_combine(const Geometry& g, const SeqBatch& b, const float* partials, int nsplit,
                          void* out, hipStream_t s, Timing* prof) {
  uint16_t* oo = (uint16_t*)out;
  if (g.dtype == 0) combine_dispatch<0>(g, b, partials, nsplit, oo, s, prof);
  else combine_dispatch<1>(g, b, partials, nsplit, oo, s, prof);
  return hipGetLastError();
}

hipError_t launch_attend(const Geometry& g, const SeqBatch& b, const void* q, const int32_t* idx,
                         int waves, float scale, void* out, float* partials, hipStream_t s, Timing* prof) {
  return attend_impl<0>(g, b, q, const_cast<int32_t*>(idx), nullptr, waves, scale, out, partials, s,
                            prof);
}

int fused_select_limit(int top_k) {
  return top_k <= kSelMaxK ? 64 * std::max(kWaves * kWgKeys, kSelKeysPerLane) : 0;
}

hipError_t launch_decode_attend(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                                int32_t* idx_out, int max_nc, int waves, float scale, void* out,
                                float* partials, hipStream_t s, Timing* prof) {
  // every wave of the workgroup takes a share of the candidates (measured
  // faster than one wave selecting, also for 510 candidates: the per-key
  // work of each pass shrinks W-fold for a few workgroup barriers); with
  // few waves per workgroup, one wave's larger capacity is used beyond that
  // (both callers keep max_nc within fused_select_limit, so the one-wave
  // selection, which runs in kWaves-wave workgroups only, is not reached)
  if (max_nc <= 64 * kWaves * kWgKeys)
    return attend_impl<2>(g, b, q, idx_out, scores, waves, scale, out, partials, s, prof);
  return attend_impl<1>(g, b, q, idx_out, scores, kWaves, scale, out, partials, s, prof);
}

hipError_t launch_decode(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                         int32_t* idx_out, int max_nc, int waves, float scale, void* out,
                         float* partials, hipStream_t s, Timing* prof) {
  hipError_t e = launch_score(g, b, q, scores, max_nc, s, prof);
  if (e != hipSuccess) return e;
  return launch_decode_attend(g, b, q, scores, idx_out, max_nc, waves, scale, out, partials, s, prof);
}

hipError_t launch_append_decode(const Geometry& g, const SeqBatch& b, const StepPages& sp,
                                const PatchBatch& pb, const void* k, const void* v, const void* q,
                                float* scores, int32_t* idx_out, int max_nc, bool fused, int waves,
                                float scale, void* out, float* partials, hipStream_t s, Timing* prof) {
  // the fused decode appends, scores and attends in one launch
  if (fused)
    return launch_fused_append_decode(g, b, sp, pb, k, v, q, idx_out, scale, out, partials, s, prof);
  // the scoring chunk size follows launch_score
  const bool small = (int64_t)((max_nc + 63) / 64) * g.hkv * b.n <= 1024;
  const int ch = small ? 32 : 64;
  const int chunks = ranked_select(g, max_nc) ? (max_nc + ch - 1) / ch : 0;
  const uint16_t *kk = (const uint16_t*)k, *vv = (const uint16_t*)v, *qq = (const uint16_t*)q;
  if (g.dtype == 0) {
    if (small) append_score_dispatch<0, 32>(g, b, sp, pb, chunks, kk, vv, qq, scores, s, prof);
    else append_score_dispatch<0, 64>(g, b, sp, pb, chunks, kk, vv, qq, scores, s, prof);
  } else {
    if (small) append_score_dispatch<1, 32>(g, b, sp, pb, chunks, kk, vv, qq, scores, s, prof);
    else append_score_dispatch<1, 64>(g, b, sp, pb, chunks, kk, vv, qq, scores, s, prof);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_decode_attend(g, b, q, scores, idx_out, max_nc, waves, scale, out, partials, s, prof);
}

hipError_t launch_export(const Geometry& g, const SeqBatch& b, int T, void* k_out, void* v_out,
                         hipStream_t s) {
  dim3 grid((T + 15) / 16, g.hkv, b.n);
  hipLaunchKernelGGL(k_export, grid, dim3(256), 0, s, g, b, T, (uint16_t*)k_out, (uint16_t*)v_out);
  return hipGetLastError();
}

hipError_t launch_export_summaries(const Geometry& g, int seq, int nfull, void* out,
                                   hipStream_t s) {
  hipLaunchKernelGGL(k_export_summaries, dim3(nfull, g.hkv), dim3(128), 0, s, g, seq, nfull,
                     (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace bsattn
