// bsattn_decode.hip -- fused block-sparse decode for 16-bit caches on gfx950:
// block scoring, top-K selection, gather + attention and (with one split)
// the final output in one launch.
//
// Layout of a launch: S splits per (batch entry, kv head) pair, one
// workgroup of W waves per (pair, split), about 256 workgroups in all (one
// per CU: a CU pulls at most ~45 GB/s of random 32 KiB slabs, so the gather
// needs every CU, and a single wave of workgroups leaves no CU with a
// second one to finish).  Every workgroup of a pair scores all of the pair's
// candidate blocks itself (the summaries are read once from HBM and the
// other splits' reads hit the L2: the splits of a pair are placed on one
// XCD, workgroup i running on XCD i % 8), runs the workgroup-wide top-K over
// the scores in LDS, and then gathers its share of the selected blocks:
// slot (r * W + wave) * S + split, round r < R.  A wave keeps an online
// softmax over its rounds; the W waves merge through LDS into the output
// (S == 1) or into split partials for k_combine.
//
// Scoring is the canonical order of the oracle (16 lanes per block, 8 dims
// per lane, left fold of the 8 products, pairwise tree over the 16 chunks,
// maximum over the GQA group scanning upward), so the selection is
// bit-identical to the separate scoring + selection kernels'.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "bsattn_device.h"

namespace bsattn {

// k_decode modes: score + select + attend (fused), attend over given
// indices (given), append each entry's new token, then score + select +
// attend (fused append)
constexpr int kModeFused = 0, kModeGiven = 1, kModeFusedAppend = 2;

// the fused append's extra arguments: the page of each entry's newest block,
// metadata words to patch for the launches that follow, and the new tokens'
// keys and values ([n][Hkv][128])
struct AppendArgs {
  StepPages sp;
  PatchBatch pb;
  const uint16_t* k;
  const uint16_t* v;
};
struct NoAppend {};
template <int MODE>
using ModeArgs = std::conditional_t<MODE == kModeFusedAppend, AppendArgs, NoAppend>;

// candidate blocks of a pair the fused kernel scores and selects from
constexpr int kFusedMaxCand = 2048;
// scoring rounds: round r, lane group lg (16 lanes) takes candidate
// lg + 4 W r; the summaries of kScoreChunk rounds are loaded per step
constexpr int kScoreChunk = 8;
// gather rounds per wave
constexpr int kMaxRounds = 8;

template <int DT, int G>
__device__ __forceinline__ float group_score(const float (&qv)[G][8], const u32x4 raw) {
  float sv[8];
  unpack8<DT>(raw, sv);
  float best = 0.0f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float acc = canonical_dot16<DT>(qv[g], sv);
    if (g == 0 || acc > best) best = acc;
  }
  return best;
}

// Loads the summaries of scoring chunk `ch` (rounds kScoreChunk * ch + i)
// for lane group lg: rows below `lim` (exclusive); the rest are not scored.
template <int W>
__device__ __forceinline__ void load_score_chunk(const uint16_t* __restrict__ srow0, int c0, int lg,
                                                 int ch, int lim, u32x4 (&raw)[kScoreChunk]) {
  // no branch around a load (a load under one is waited for where the
  // branch joins): rows from lim on all read row lim - 1 (one cached line
  // per lane group; never scored)
  const int last = max(lim - 1, 0);
#pragma unroll
  for (int i = 0; i < kScoreChunk; ++i) {
    const int j = c0 + lg + 4 * W * (kScoreChunk * ch + i);
    raw[i] = *(const u32x4*)(srow0 + (size_t)min(j, last) * kHeadDim);
  }
}

template <int DT, int G, int W>
__device__ __forceinline__ void score_chunk(const float (&qv)[G][8], const u32x4 (&raw)[kScoreChunk],
                                            int lg, int c, int ch, int nc, float* s_score) {
#pragma unroll
  for (int i = 0; i < kScoreChunk; ++i) {
    const int cand = lg + 4 * W * (kScoreChunk * ch + i);
    if (cand < nc) {  // a whole 16-lane row enters or skips
      const float best = group_score<DT, G>(qv, raw[i]);
      if (c == 0) s_score[cand] = best;
    }
  }
}

// Adds one 16-dim tile of a block's O (accumulator layout: lane (dim n,
// group g) holds heads 4g .. 4g+3) to the wave's running O in s_o, whose
// heads are first rescaled by a[i] (the online-softmax factor of head 4g+i).
// The tile was written by this wave (store_o_tile) in program order.
template <int G>
__device__ __forceinline__ void rescale_add_o_tile(float (*s_o)[kHeadDim], int dt, int n, int g,
                                                   const f32x4& o, const float (&a)[4]) {
  if constexpr (G >= 4) {
    if (4 * g < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* p = &s_o[4 * g + i][16 * dt + n];
        *p = *p * a[i] + o[i];
      }
    }
  } else {
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        float* p = &s_o[i][16 * dt + n];
        *p = *p * a[i] + o[i];
      }
    }
  }
}

// grid: 8 * ceil(npairs / 8) * S workgroups of 64 W threads.
// GIVEN: the blocks come from idx ([n][Hkv][nsel_max], -1 padded: the
// given-index attention, bsattn_attend), with the same slots, rounds and
// merge order as the fused decode, so decode == select + attend bit for
// bit.  Otherwise the kernel scores and selects, and writes the selection
// to idx when it is not null.
// len_first: read the entry's length before the summaries (only its rows
// are loaded); otherwise every row below the block-table width is loaded
// at once (no wait for the length; for batches whose rows are all in use).
template <int DT, int TB, int G, int W, int MODE>
__global__ __launch_bounds__(64 * W) void k_decode(Geometry geo, SeqBatch sb,
                                                   const uint16_t* __restrict__ q,
                                                   int32_t* __restrict__ idx, float sl2,
                                                   uint16_t* __restrict__ out,
                                                   float* __restrict__ partials, int S, int R,
                                                   int len_first, ModeArgs<MODE> ap) {
  constexpr bool GIVEN = MODE == kModeGiven, APPEND = MODE == kModeFusedAppend;
  constexpr int NT = TB / 16;   // QK token tiles
  constexpr int EPL = TB / 4;   // scores per lane
  constexpr int KS2 = TB / 32;  // PV k-steps
  __shared__ float s_score[GIVEN ? 1 : kFusedMaxCand];
  __shared__ int s_sel[GIVEN ? 1 : kSelMaxK], s_selp[GIVEN ? 1 : kSelMaxK];
  __shared__ __align__(16) uint32_t s_ws[GIVEN ? 4 : kWgScratch];
  __shared__ float s_m[W][16], s_l[W][16];
  __shared__ float s_o[W][G][kHeadDim];
  __shared__ int s_jr[W][kMaxRounds], s_pr[W][kMaxRounds];
  __shared__ u32x4 s_blk[APPEND ? TB : 1][16];  // keys of a block the append fills

  // (pair, split); the S splits of a pair share workgroup index mod 8 (XCD)
  const int L = blockIdx.x, xcd = L & 7, r8 = L >> 3;
  const int pair = (r8 / S) * 8 + xcd, split = r8 % S;
  if (pair >= sb.n * geo.hkv) return;
  const int bi = pair / geo.hkv, h = pair - bi * geo.hkv;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;  // MFMA: column n, lane group g
  const int c = lane & 15;                  // scoring: chunk c of the 16-lane row
  const int lg = wave * 4 + g;              // scoring lane group
  const int seq = uniform(sb.ids[bi]);
  const int32_t* bt = block_table(geo, seq);
  const uint16_t* srow0 = summary_row(geo, seq, h, 0) + 8 * c;
  const int c0 = geo.ns;

  // --- loads that need nothing else: the new token (append), q in both
  // layouts, the first summaries (unless the length comes first), the length
  [[maybe_unused]] u32x4 tk, tv;
  if constexpr (APPEND) {
    // dims 8c .. 8c+7 of the token's key and value, in every lane (no
    // branch, so that no wait lands on the loads that follow)
    const size_t src = ((size_t)bi * geo.hkv + h) * kHeadDim + 8 * c;
    tk = *(const u32x4*)(ap.k + src);
    tv = *(const u32x4*)(ap.v + src);
  }
  u32x4 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = u32x4{0u, 0u, 0u, 0u};
  if (n < G) {
    const uint16_t* src = q + q_row(sb, bi, h * G + n) + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *(const u32x4*)(src + 32 * s);
  }
  // append, further loads whose results wait until after the scoring: when
  // the token completes its block, split 0 folds the block's summary, whose
  // other keys (written by earlier launches) are requested now; workgroup 0
  // requests the metadata words it patches for the launches that follow
  // (nothing in this launch reads a patched word: lengths come from sb, the
  // newest block's page from ap.sp, and the scored candidates end before the
  // newest block, since recent >= 1)
  constexpr int NP = APPEND ? ((TB - 1) * 16 + 64 * W - 1) / (64 * W) : 1;
  [[maybe_unused]] u32x4 pre[NP];
  [[maybe_unused]] int pidx = 0, pval = 0;
  [[maybe_unused]] bool fills = false;
  if constexpr (APPEND) {
    fills = split == 0 && sb.len[bi] % TB == 0;
    if (fills) {
      const uint16_t* Kt = (const uint16_t*)(geo.pool + ((size_t)ap.sp.page[bi] * geo.hkv + h) * geo.slab_bytes +
                                             geo.k_off);
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int e = min((int)threadIdx.x + 64 * W * i, (TB - 1) * 16 - 1);
        pre[i] = *(const u32x4*)(Kt + k_elem(e >> 4, 8 * (e & 15)));
      }
    }
    if (L == 0) {
      const int t = min((int)threadIdx.x, kMaxPatch - 1);
      pidx = ap.pb.idx[t];
      pval = ap.pb.val[t];
    }
  }
  // block and page of each of this wave's rounds (-1: nothing), kept in the
  // wave's own row of s_jr / s_pr (written and read by this wave only, in
  // program order)
  int len;
  // append: newest block, and whether this wave gathers it
  [[maybe_unused]] int jn = -1;
  [[maybe_unused]] bool owner = false;
  if constexpr (GIVEN) {
    // indices from idx; the block-table entry is requested before the
    // length check (every j in [0, mbps) has one; others read entry 0 and
    // are dropped)
    int jr[kMaxRounds], pr[kMaxRounds];
#pragma unroll
    for (int rr = 0; rr < kMaxRounds; ++rr) {
      const int slot = (rr * W + wave) * S + split;
      jr[rr] = rr < R ? uniform(given_index(geo, idx, bi, h, slot)) : -1;
      const bool in_table = jr[rr] >= 0 && jr[rr] < geo.mbps;
      pr[rr] = rr < R ? uniform(bt[in_table ? jr[rr] : 0]) : -1;
      if (!in_table) jr[rr] = -1;
    }
    len = uniform(entry_len(geo, sb, bi, seq));
    if (lane == 0) {
#pragma unroll
      for (int rr = 0; rr < kMaxRounds; ++rr) {
        s_jr[wave][rr] = (int64_t)jr[rr] * TB >= len ? -1 : jr[rr];
        s_pr[wave][rr] = pr[rr];
      }
    }
  } else {
    float qv[G][8];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) unpack8<DT>(*(const u32x4*)(q + q_row(sb, bi, h * G + gg) + 8 * c), qv[gg]);
    // two scoring chunks in flight (A: even chunks, B: odd).  Without
    // len_first the first two chunks are loaded and scored over every row
    // below the block-table width before the length is waited for (rows past
    // the sequence score too and are never read): the length load, a scalar
    // chain through the metadata, then overlaps the scoring.
    u32x4 rawA[kScoreChunk], rawB[kScoreChunk];
    const int len_req = entry_len(geo, sb, bi, seq);
    int ch0 = 0;  // first chunk left to score
    WgCand wgc;
    if (!len_first) {
      const int rows = geo.mbps - c0;
      load_score_chunk<W>(srow0, c0, lg, 0, geo.mbps, rawA);
      load_score_chunk<W>(srow0, c0, lg, 1, geo.mbps, rawB);
      score_chunk<DT, G, W>(qv, rawA, lg, c, 0, rows, s_score);
      score_chunk<DT, G, W>(qv, rawB, lg, c, 1, rows, s_score);
      ch0 = 2;
    }
    len = uniform(len_req);
    const int nb = len > 0 ? (len + TB - 1) / TB : 0;
    const int nc = nb - geo.nr - c0, K = geo.top_k;
    const bool ranked = nc > K;           // sinks, the K picked, recent
    const bool select = ranked && K > 0;  // (top_k 0: sinks and recent only)
    const int lim = len_first ? c0 + max(nc, 0) : geo.mbps;
    // append: the token goes to the newest block jn, on page ap.sp.page[bi]
    // (its block-table entry may be patched by this launch).  The block's
    // slot is the last one (sinks, picked, recent; or every block in order);
    // lanes 0..15 of the wave that gathers it store the token, and that wave
    // waits for the store before its gather of the block
    jn = APPEND ? (len - 1) / TB : -1;
    if constexpr (APPEND) {
      const int slot_n = ranked ? geo.ns + K + geo.nr - 1 : nb - 1;
      owner = split == slot_n % S && wave == (slot_n / S) % W;
    }
    // the token's store, the patches, and the keys of a completed block into
    // LDS (the new key from the registers of lanes 0..15); called after the
    // scoring, whose waits have covered those loads, or, when nothing is
    // scored, at the end of this branch (where it waits for them)
    auto append_stage = [&]() {
      if constexpr (APPEND) {
        if (owner && lane < 16) put_token<true>(geo, ap.sp.page[bi], h, len - 1 - jn * TB, c, tk, tv);
        if (L == 0 && (int)threadIdx.x < ap.pb.n) geo.meta[pidx] = pval;
        if (fills) {
#pragma unroll
          for (int i = 0; i < NP; ++i) {
            const int e = threadIdx.x + 64 * W * i;
            if (e < (TB - 1) * 16) s_blk[e >> 4][e & 15] = pre[i];
          }
          if (threadIdx.x < 16) s_blk[TB - 1][threadIdx.x] = tk;
        }
      }
    };
    // block-table entries of the selection's keys: slot k of wave w, lane l
    // holds candidate c0 + 64 (W k + w) + l
    // (unconditional: slots from lim on read entry lim - 1 and are never
    // selected)
#pragma unroll
    for (int k = 0; k < kWgKeys; ++k) wgc.page[k] = bt[min(c0 + 64 * (W * k + wave) + lane, max(lim - 1, 0))];
    // slots known from the length alone (sinks, recent, every block when
    // nothing is ranked): their pages are requested now
    {
      int jr[kMaxRounds], pr[kMaxRounds];
#pragma unroll
      for (int rr = 0; rr < kMaxRounds; ++rr) {
        const int slot = (rr * W + wave) * S + split;
        const bool picked = ranked && slot >= geo.ns && slot < geo.ns + K;
        jr[rr] = rr < R && !picked ? selected_block(slot, nb, ranked, geo.ns, geo.nr, K, nullptr) : -1;
        if constexpr (APPEND) pr[rr] = jr[rr] == jn ? ap.sp.page[bi] : jr[rr] >= 0 ? uniform(bt[jr[rr]]) : -1;
        else pr[rr] = jr[rr] >= 0 ? uniform(bt[jr[rr]]) : -1;
      }
      if (lane == 0) {
#pragma unroll
        for (int rr = 0; rr < kMaxRounds; ++rr) {
          s_jr[wave][rr] = jr[rr];
          s_pr[wave][rr] = pr[rr];
        }
      }
    }
    // scoring (exact, canonical order) of every candidate into LDS, then
    // the workgroup's top-K
    if (select) {
      const int nch = (nc + 4 * W * kScoreChunk - 1) / (4 * W * kScoreChunk);
      if (ch0 < nch) load_score_chunk<W>(srow0, c0, lg, ch0, lim, rawA);
      if (ch0 + 1 < nch) load_score_chunk<W>(srow0, c0, lg, ch0 + 1, lim, rawB);
#pragma unroll 1
      for (int ch = ch0; ch < nch; ch += 2) {
        score_chunk<DT, G, W>(qv, rawA, lg, c, ch, nc, s_score);
        if (ch + 2 < nch) load_score_chunk<W>(srow0, c0, lg, ch + 2, lim, rawA);
        if (ch + 1 < nch) {
          score_chunk<DT, G, W>(qv, rawB, lg, c, ch + 1, nc, s_score);
          if (ch + 3 < nch) load_score_chunk<W>(srow0, c0, lg, ch + 3, lim, rawB);
        }
      }
      append_stage();
      __syncthreads();
#pragma unroll
      for (int k = 0; k < kWgKeys; ++k) {
        const int i = 64 * (W * k + wave) + lane;
        wgc.score[k] = i < nc ? s_score[i] : 0.0f;
      }
      wg_topk<W>(wgc, c0, nc, K, s_sel, s_selp, s_ws);
      __syncthreads();
      if (lane == 0) {
#pragma unroll 1
        for (int rr = 0; rr < R; ++rr) {
          const int slot = (rr * W + wave) * S + split;
          if (slot >= geo.ns && slot < geo.ns + K) {
            s_jr[wave][rr] = s_sel[slot - geo.ns];
            s_pr[wave][rr] = s_selp[slot - geo.ns];
          }
        }
      }
    }
    if (idx != nullptr && split == 0 && wave == 0) {
      int32_t* row = idx + ((size_t)bi * geo.hkv + h) * geo.nsel_max;
      for (int p = lane; p < geo.nsel_max; p += 64)
        row[p] = selected_block(p, nb, ranked, geo.ns, geo.nr, K, s_sel);
    }
    if (!select) append_stage();
  }

  // --- gather + attention: this wave's slots, online softmax over rounds;
  // the running O lives in the wave's own s_o tile (rescaled and added per
  // round), the running maximum and sum in registers
  float m_run = -INFINITY, l_run = 0.f;  // per head n (all lane groups agree)
  bool any = false;
  wave_lds_order();  // lane 0's s_jr / s_pr writes before every lane's reads
#pragma unroll 1
  for (int rr = 0; rr < R; ++rr) {
    const int j = uniform(s_jr[wave][rr]), page = uniform(s_pr[wave][rr]);
    if (j < 0) continue;
    // the newest block of an append: this wave stored its token; the store is
    // complete before the block is read
    if constexpr (APPEND)
      if (j == jn) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int valid = min(TB, len - j * TB);
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
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
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      pv[e] = __builtin_amdgcn_exp2f(pv[e] - m_new);
      ps += pv[e];
    }
    ps = sum_over_groups(ps);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    // factors of the running O's heads: lane (dim n, group g) holds heads
    // 4g .. 4g+3 of an O tile, whose factors sit in lanes 4g + i
    float a4[4] = {0.f, 0.f, 0.f, 0.f};
    if (any) {
#pragma unroll
      for (int i = 0; i < 4; ++i) a4[i] = __shfl(alpha, 4 * g + i, 64);
    }
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
    if (valid < TB) {  // V of tokens past the end of a partial block is stale
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int t0 = 32 * s2 + 8 * g + 2 * jj;
          const uint32_t msk = (t0 < valid ? 0x0000FFFFu : 0u) | (t0 + 1 < valid ? 0xFFFF0000u : 0u);
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) vf[dt][s2][jj] &= msk;
        }
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) {
        o = mfma16x16x32<DT>(pf[s2], vf[dt][s2], o);
        if constexpr (DT == 1) o = mfma16x16x32<DT>(pl[s2], vf[dt][s2], o);
      }
      if (any) rescale_add_o_tile<G>(s_o[wave], dt, n, g, o, a4);
      else store_o_tile<G>(s_o[wave], dt, n, g, o);
    }
    any = true;
  }
  if (any) {
    if (g == 0 && n < G) {
      s_m[wave][n] = m_run;
      s_l[wave][n] = l_run;
    }
  } else {
    store_empty<G>(s_m[wave], s_l[wave], s_o[wave], lane);
  }
  __syncthreads();
  attend_merge<DT, G, W>(geo, sb, bi, h, split, S, s_m, s_l, s_o, out, partials);
  if constexpr (APPEND) {
    // the completed block's summary: 16 lanes fold its keys from LDS (written
    // before the barriers of the merge) in token order
    if (fills && threadIdx.x < 16)
      *(u32x4*)(summary_row(geo, seq, h, jn) + 8 * threadIdx.x) = fold_block<DT>(s_blk, TB, threadIdx.x);
  }
}

// ===========================================================================
// launcher
// ===========================================================================
namespace {

struct FusedPlan {
  int S, W, R;
};

// S splits for about 256 workgroups (at most the partial workspace's
// g.nsplit), then the fewest rounds R and waves W in {4, 8, 12} that cover
// the selection (12 only for 32-token blocks: a 64-token wave holds 32 KiB
// of K / V fragments in flight and needs more than the ~170 registers of
// three waves per SIMD).
FusedPlan fused_plan(const Geometry& g, int n) {
  FusedPlan p{};
  const int pairs = n * g.hkv;
  p.S = std::max(1, std::min(g.nsplit, (256 + pairs / 2) / pairs));
  const int wmax = g.tb == 32 ? 12 : 8;
  const int per = (g.nsel_max + p.S - 1) / p.S;  // slots per split
  p.R = (per + wmax - 1) / wmax;
  const int w = (per + p.R - 1) / p.R;
  p.W = w <= 4 ? 4 : w <= 8 ? 8 : 12;
  return p;
}

template <int DT, int TB, int G, int MD>
void decode_w(const Geometry& g, const FusedPlan& p, dim3 grid, const SeqBatch& b, const uint16_t* q,
              int32_t* idx, float sl2, uint16_t* out, float* part, int lf, const ModeArgs<MD>& ap,
              hipStream_t s, Timing* prof) {
  const int kd = kProfAttend;
  switch (p.W) {
    case 4: launch(k_decode<DT, TB, G, 4, MD>, grid, dim3(256), 0, s, prof, kd, g, b, q, idx, sl2, out, part, p.S, p.R, lf, ap); break;
    case 8: launch(k_decode<DT, TB, G, 8, MD>, grid, dim3(512), 0, s, prof, kd, g, b, q, idx, sl2, out, part, p.S, p.R, lf, ap); break;
    default:  // fused_plan gives W = 12 for 32-token blocks only
      if constexpr (TB == 32)
        launch(k_decode<DT, TB, G, 12, MD>, grid, dim3(768), 0, s, prof, kd, g, b, q, idx, sl2, out, part, p.S, p.R, lf, ap);
      break;
  }
}

template <int DT, int TB, int MD>
void decode_g(const Geometry& g, const FusedPlan& p, dim3 grid, const SeqBatch& b, const uint16_t* q,
              int32_t* idx, float sl2, uint16_t* out, float* part, int lf, const ModeArgs<MD>& ap,
              hipStream_t s, Timing* prof) {
  switch (g.group) {
    case 1: decode_w<DT, TB, 1, MD>(g, p, grid, b, q, idx, sl2, out, part, lf, ap, s, prof); break;
    case 2: decode_w<DT, TB, 2, MD>(g, p, grid, b, q, idx, sl2, out, part, lf, ap, s, prof); break;
    default: decode_w<DT, TB, 4, MD>(g, p, grid, b, q, idx, sl2, out, part, lf, ap, s, prof); break;
  }
}

// nseq: the call's sequences, which the splits are planned for (a launch of
// a multi-token decode holds several entries per sequence)
template <int MD>
hipError_t decode_impl(const Geometry& g, const SeqBatch& b, int nseq, const void* q, int32_t* idx,
                       bool len_first, float scale, void* out, float* partials,
                       const ModeArgs<MD>& ap, hipStream_t s, Timing* prof) {
  const FusedPlan p = fused_plan(g, nseq);
  const int pairs = b.n * g.hkv;
  const dim3 grid(8 * ((pairs + 7) / 8) * p.S);
  const float sl2 = scale * 1.4426950408889634f;
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* oo = (uint16_t*)out;
  const int lf = len_first ? 1 : 0;
  if (g.dtype == 0) {
    if (g.tb == 64) decode_g<0, 64, MD>(g, p, grid, b, qq, idx, sl2, oo, partials, lf, ap, s, prof);
    else decode_g<0, 32, MD>(g, p, grid, b, qq, idx, sl2, oo, partials, lf, ap, s, prof);
  } else {
    if (g.tb == 64) decode_g<1, 64, MD>(g, p, grid, b, qq, idx, sl2, oo, partials, lf, ap, s, prof);
    else decode_g<1, 32, MD>(g, p, grid, b, qq, idx, sl2, oo, partials, lf, ap, s, prof);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.S == 1) return e;
  return launch_combine(g, b, partials, p.S, out, s, prof);
}

}  // namespace

bool fused_decode_ok(const Geometry& g, int nseq, int max_nc) {
  if (g.kv_bits != 0 || g.group > 4 || max_nc > kFusedMaxCand || g.top_k > kSelMaxK) return false;
  const FusedPlan p = fused_plan(g, nseq);
  // every split of a pair scores all of the pair's candidates: worth it with
  // one split (no redundancy, and no combine), or with few candidates.  (A CU
  // pulls ~20 GB/s while every CU loads: the 128 KiB of summaries of a
  // 510-candidate pair take it ~6 us, against ~5 us for a scoring kernel that
  // spreads them over every CU.)
  if (p.S > 1 && max_nc > 256) return false;
  if (p.R > kMaxRounds) return false;
  // every candidate fits the workgroup selection's keys
  return max_nc <= 64 * p.W * kWgKeys;
}

hipError_t launch_fused_decode(const Geometry& g, const SeqBatch& b, int nseq, const void* q,
                               int32_t* idx_out, bool len_first, float scale, void* out, float* partials,
                               hipStream_t s, Timing* prof) {
  return decode_impl<kModeFused>(g, b, nseq, q, idx_out, len_first, scale, out, partials, NoAppend{}, s, prof);
}

hipError_t launch_fused_append_decode(const Geometry& g, const SeqBatch& b, const StepPages& sp,
                                      const PatchBatch& pb, const void* k, const void* v, const void* q,
                                      int32_t* idx_out, float scale, void* out, float* partials,
                                      hipStream_t s, Timing* prof) {
  const AppendArgs ap{sp, pb, (const uint16_t*)k, (const uint16_t*)v};
  return decode_impl<kModeFusedAppend>(g, b, b.n, q, idx_out, true, scale, out, partials, ap, s, prof);
}

hipError_t launch_fused_attend(const Geometry& g, const SeqBatch& b, int nseq, const void* q,
                               const int32_t* idx, float scale, void* out, float* partials, hipStream_t s,
                               Timing* prof) {
  return decode_impl<kModeGiven>(g, b, nseq, q, const_cast<int32_t*>(idx), false, scale, out, partials,
                                 NoAppend{}, s, prof);
}

}  // namespace bsattn
