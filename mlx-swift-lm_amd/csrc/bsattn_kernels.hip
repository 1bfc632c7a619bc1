// bsattn_kernels.hip -- gfx950 (CDNA4) kernels of the block-sparse decode
// path: append, block summary, block scoring, top-K select, gathered
// split-K attention and the split combine.
//
// Page slab layout (one slab per (physical page, kv head), Tb tokens):
//   K tile  [Tb][D]   token-major  (a token's key = 256 contiguous bytes)
//   V tile  [D][Tb]   dim-major    (a dim's Tb values contiguous)
// Summaries: [page][kv head][D], written when a block fills.
//
// Bit-exact parts (summary, score, selection) use __fadd_rn / __fmul_rn so
// the compiler cannot contract or reorder them; the order is the one the
// oracle states (sequential token fold; 16 chunks of 8 dims, then an xor
// butterfly 1, 2, 4, 8; max over the GQA group scanning upward).
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

// 256-thread inclusive scan; s_tmp holds 4 ints.
__device__ __forceinline__ int block_scan_incl(int v, int* s_tmp, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_tmp[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int t = s_tmp[i];
    off += (i < w) ? t : 0;
    tot += t;
  }
  __syncthreads();
  if (total) *total = tot;
  return off + x;
}

__device__ __forceinline__ const int32_t* block_table(const Geometry& g, int seq) {
  return g.meta + g.bt_off + (size_t)seq * g.mbps;
}

// ---------------------------------------------------------------------------
// metadata patch: meta[idx[i]] = val[i]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_patch(int32_t* meta, PatchBatch pb) {
  const int t = threadIdx.x;
  if (t < pb.n) meta[pb.idx[t]] = pb.val[t];
}

// ---------------------------------------------------------------------------
// append: 16 tokens x 16 lanes (8 dims each) per workgroup
// grid (ceil(L/16), Hkv, n)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_append(Geometry geo, AppendBatch ab,
                                                const uint16_t* __restrict__ k,
                                                const uint16_t* __restrict__ v) {
  const int bi = blockIdx.z, h = blockIdx.y;
  const int tok = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  if (tok >= ab.L) return;
  const int seq = ab.seq[bi];
  const int pos = ab.old_len[bi] + tok;
  const int blk = pos / geo.tb, slot = pos - blk * geo.tb;
  const int page = block_table(geo, seq)[blk];
  const size_t src = (((size_t)bi * geo.hkv + h) * ab.L + tok) * kHeadDim + 8 * c;
  const u32x4 kr = *(const u32x4*)(k + src);
  const u32x4 vr = *(const u32x4*)(v + src);
  uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  *(u32x4*)((uint16_t*)(slab + geo.k_off) + slot * kHeadDim + 8 * c) = kr;
  uint16_t* Vt = (uint16_t*)(slab + geo.v_off);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = vr[e >> 1];
    Vt[(8 * c + e) * geo.tb + slot] = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xFFFFu));
  }
}

// ---------------------------------------------------------------------------
// block summary: one workgroup per (block, kv head, sequence), one thread
// per dim; sequential fp32 fold over the block's tokens, times 1/Tb.
// grid (max_count, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(128) void k_summary(Geometry geo, SummaryBatch sb) {
  const int bi = blockIdx.z, h = blockIdx.y;
  if ((int)blockIdx.x >= sb.count[bi]) return;
  const int seq = sb.seq[bi];
  const int j = sb.first[bi] + blockIdx.x;
  const int page = block_table(geo, seq)[j];
  const int d = threadIdx.x;
  const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  const uint16_t* Kt = (const uint16_t*)(slab + geo.k_off);
  float acc = to_f32<DT>(Kt[d]);
  for (int t = 1; t < geo.tb; ++t) acc = __fadd_rn(acc, to_f32<DT>(Kt[t * kHeadDim + d]));
  geo.summ[((size_t)page * geo.hkv + h) * kHeadDim + d] =
      from_f32<DT>(__fmul_rn(acc, 1.0f / (float)geo.tb));
}

// ---------------------------------------------------------------------------
// block scoring: 16 lanes per (block, kv head) row, 8 dims per lane.
// grid (ceil(max_cand / per_wg), n); needs 16 % Hkv == 0.
// ---------------------------------------------------------------------------
constexpr int kScoreIters = 8;

template <int DT, int G>
__global__ __launch_bounds__(256) void k_score(Geometry geo, SeqBatch sb,
                                               const uint16_t* __restrict__ q,
                                               float* __restrict__ scores) {
  const int bi = blockIdx.y;
  const int seq = sb.ids[bi];
  const int len = geo.meta[seq];
  const int nb = (len + geo.tb - 1) / geo.tb;
  const int c0 = geo.ns, c1 = nb - geo.nr;
  if (c1 - c0 <= geo.top_k) return;  // every candidate is kept; no ranking
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int hkv = geo.hkv;
  const int h = r % hkv;
  const int bpi = 16 / hkv;
  const int bofs = r / hkv;
  float qv[G][8];
  const uint16_t* qrow = q + ((size_t)bi * geo.hq + h * G) * kHeadDim + 8 * c;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const u32x4 raw = *(const u32x4*)(qrow + (size_t)g * kHeadDim);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      qv[g][e] = to_f32<DT>((uint16_t)((e & 1) ? (raw[e >> 1] >> 16) : (raw[e >> 1] & 0xFFFFu)));
  }
  const int32_t* bt = block_table(geo, seq);
  float* srow = scores + ((size_t)bi * hkv + h) * geo.mbps;
  const int jbase = c0 + blockIdx.x * (bpi * kScoreIters);
  for (int it = 0; it < kScoreIters; ++it) {
    const int j = jbase + it * bpi + bofs;
    if (j >= c1) break;  // whole 16-lane row leaves together
    const int page = bt[j];
    const u32x4 raw = *(const u32x4*)(geo.summ + ((size_t)page * hkv + h) * kHeadDim + 8 * c);
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      s[e] = to_f32<DT>((uint16_t)((e & 1) ? (raw[e >> 1] >> 16) : (raw[e >> 1] & 0xFFFFu)));
    float best = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = __fmul_rn(qv[g][0], s[0]);
#pragma unroll
      for (int e = 1; e < 8; ++e) acc = __fadd_rn(acc, __fmul_rn(qv[g][e], s[e]));
      acc = __fadd_rn(acc, __shfl_xor(acc, 1, 64));
      acc = __fadd_rn(acc, __shfl_xor(acc, 2, 64));
      acc = __fadd_rn(acc, __shfl_xor(acc, 4, 64));
      acc = __fadd_rn(acc, __shfl_xor(acc, 8, 64));
      if (g == 0 || acc > best) best = acc;
    }
    if (c == 0) srow[j] = best;
  }
}

// ---------------------------------------------------------------------------
// top-K select: one workgroup per (kv head, sequence).  MSB-first radix
// select (4 x 8 bits) of the K-th largest key, then ties by ascending
// index, then compaction of forced + chosen blocks in ascending order.
// dynamic LDS: keys[mbps] (u32) + flags[mbps] (u8)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t score_key(float s) {
  if (__builtin_isnan(s)) return 0u;
  if (s == 0.0f) s = 0.0f;
  const uint32_t b = __float_as_uint(s);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__global__ __launch_bounds__(256) void k_topk(Geometry geo, SeqBatch sb,
                                              const float* __restrict__ scores,
                                              int32_t* __restrict__ idx_out) {
  extern __shared__ uint32_t smem[];
  uint32_t* keys = smem;
  uint8_t* flags = (uint8_t*)(smem + geo.mbps);
  __shared__ uint32_t hist[256];
  __shared__ int s_tmp[4];
  __shared__ int s_sel[2];
  const int tid = threadIdx.x;
  const int h = blockIdx.x, bi = blockIdx.y;
  const int seq = sb.ids[bi];
  const int len = geo.meta[seq];
  const int nb = len > 0 ? (len + geo.tb - 1) / geo.tb : 0;
  int32_t* out = idx_out + ((size_t)bi * geo.hkv + h) * geo.nsel_max;
  const int c0 = geo.ns, c1 = nb - geo.nr, nc = c1 - c0;
  for (int j = tid; j < nb; j += 256)
    flags[j] = (j < geo.ns || j >= nb - geo.nr || (nc > 0 && nc <= geo.top_k)) ? 1 : 0;
  __syncthreads();
  if (nc > geo.top_k && geo.top_k > 0) {
    const float* sc = scores + ((size_t)bi * geo.hkv + h) * geo.mbps;
    for (int i = tid; i < nc; i += 256) keys[i] = score_key(sc[c0 + i]);
    uint32_t prefix = 0u, mask = 0u;
    int krem = geo.top_k;
    for (int sh = 24; sh >= 0; sh -= 8) {
      hist[tid] = 0u;
      __syncthreads();
      for (int i = tid; i < nc; i += 256) {
        const uint32_t key = keys[i];
        if (((key ^ prefix) & mask) == 0u) atomicAdd(&hist[(key >> sh) & 255u], 1u);
      }
      __syncthreads();
      const int cnt = (int)hist[255 - tid];
      const int incl = block_scan_incl(cnt, s_tmp, nullptr);
      if (incl >= krem && incl - cnt < krem) {
        s_sel[0] = 255 - tid;
        s_sel[1] = incl - cnt;
      }
      __syncthreads();
      prefix |= (uint32_t)s_sel[0] << sh;
      mask |= 0xFFu << sh;
      krem -= s_sel[1];
      __syncthreads();
    }
    const uint32_t tau = prefix;
    const int per = (nc + 255) / 256;
    const int lo = min(tid * per, nc), hi = min(lo + per, nc);
    int nties = 0;
    for (int i = lo; i < hi; ++i) {
      const uint32_t key = keys[i];
      if (key > tau) flags[c0 + i] = 1;
      else if (key == tau) ++nties;
    }
    int rank = block_scan_incl(nties, s_tmp, nullptr) - nties;
    for (int i = lo; i < hi; ++i)
      if (keys[i] == tau) {
        if (rank < krem) flags[c0 + i] = 1;
        ++rank;
      }
  }
  __syncthreads();
  const int per = (nb + 255) / 256;
  const int lo = min(tid * per, nb), hi = min(lo + per, nb);
  int cnt = 0;
  for (int j = lo; j < hi; ++j) cnt += flags[j];
  int total = 0;
  int pos = block_scan_incl(cnt, s_tmp, &total) - cnt;
  for (int j = lo; j < hi; ++j)
    if (flags[j]) {
      if (pos < geo.nsel_max) out[pos] = j;
      ++pos;
    }
  for (int p = total + tid; p < geo.nsel_max; p += 256) out[p] = -1;
}

// ---------------------------------------------------------------------------
// gathered attention.  Workgroup = 4 waves = 4 consecutive selected slots of
// one (sequence, kv head); each wave does one block with MFMA 16x16x32:
//   S^T[token][head] = K[token][:] . Q[head][:]   (A = K rows, B = Q^T)
//   O[head][dim]     = P[head][token] . V[token][dim]  (A = P, B = V)
// Token order inside the QK tiles is chosen so that the S accumulator of
// lane (head n, group g) holds tokens TPG*g .. TPG*g+TPG-1, which is exactly
// the A-operand layout the PV product needs (no shuffles).  Any permutation
// of the contraction index is legal as long as A and B agree; the head-dim
// chunk of lane group g at k-step s is dims 32*g + 8*s .. +7.
// bf16: P is split into hi + lo bf16 parts (two MFMAs) for ~16-bit P.
// grid (nsplit, Hkv, n)
// ---------------------------------------------------------------------------
template <int DT, int TB, int G>
__global__ __launch_bounds__(256) void k_attend(Geometry geo, SeqBatch sb,
                                                const uint16_t* __restrict__ q,
                                                const int32_t* __restrict__ idx,
                                                float sl2, uint16_t* __restrict__ out,
                                                float* __restrict__ partials) {
  constexpr int NT = TB / 16;   // QK token tiles
  constexpr int TPG = TB / 4;   // tokens per lane group
  constexpr int KS2 = TB / 32;  // PV k-steps
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ float s_o[kWaves][G][kHeadDim];
  const int split = blockIdx.x, h = blockIdx.y, bi = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int seq = sb.ids[bi];
  const int slot = split * kWaves + wave;
  int j = -1;
  if (slot < geo.nsel_max) j = idx[((size_t)bi * geo.hkv + h) * geo.nsel_max + slot];
  j = uniform(j);
  const int len = uniform(geo.meta[seq]);
  // -1 and indices past the sequence's last block contribute nothing
  if (j >= geo.mbps || (int64_t)j * TB >= len) j = -1;
  if (j >= 0) {
    const int page = uniform(block_table(geo, seq)[j]);
    const int valid = min(TB, len - j * TB);
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
    const uint16_t* Kt = (const uint16_t*)(slab + geo.k_off);
    const uint16_t* Vt = (const uint16_t*)(slab + geo.v_off);
    u32x4 kf[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tok = TPG * (n >> 2) + 4 * t + (n & 3);
      const u32x4* src = (const u32x4*)(Kt + tok * kHeadDim + 32 * g);
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[t][s] = src[s];
    }
    u32x4 vf[8][KS2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x4* src = (const u32x4*)(Vt + (16 * dt + n) * TB + TPG * g);
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) vf[dt][s2] = src[s2];
    }
    u32x4 qf[4];
    if (n < G) {
      const u32x4* src = (const u32x4*)(q + ((size_t)bi * geo.hq + h * G + n) * kHeadDim + 32 * g);
#pragma unroll
      for (int s = 0; s < 4; ++s) qf[s] = src[s];
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qf[s] = u32x4{0u, 0u, 0u, 0u};
    }
    // S^T = K . Q^T
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[t] = mfma16x16x32<DT>(kf[t][s], qf[s], acc[t]);
    }
    // softmax over this block (log2 domain)
    float pv[TPG];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * t + i;
        float x = acc[t][i] * sl2;
        if (TPG * g + e >= valid) x = -INFINITY;
        pv[e] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < TPG; ++e) {
      const float p = (n < G) ? __builtin_amdgcn_exp2f(pv[e] - mx) : 0.f;
      pv[e] = p;
      ps += p;
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    // P operand (A): lane (head n, group g), k-step s2 -> tokens TPG*g + 8*s2 + 0..7
    u32x4 pf[KS2];
    u32x4 pl[KS2];
#pragma unroll
    for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float p0 = pv[8 * s2 + 2 * jj], p1 = pv[8 * s2 + 2 * jj + 1];
        if constexpr (DT == 0) {
          pf[s2][jj] = pack2<0>(p0, p1);
          pl[s2][jj] = 0u;
        } else {
          const uint16_t h0 = f32_to_bf16_rne(p0), h1 = f32_to_bf16_rne(p1);
          pf[s2][jj] = (uint32_t)h0 | ((uint32_t)h1 << 16);
          pl[s2][jj] = pack2<1>(p0 - to_f32<1>(h0), p1 - to_f32<1>(h1));
        }
      }
    // zero V of tokens past the end of a partial block (stale page data)
    if (valid < TB) {
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int t0 = TPG * g + 8 * s2 + 2 * jj;
          const uint32_t m = (t0 < valid ? 0x0000FFFFu : 0u) | (t0 + 1 < valid ? 0xFFFF0000u : 0u);
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) vf[dt][s2][jj] &= m;
        }
    }
    // O = P . V
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) {
        o = mfma16x16x32<DT>(pf[s2], vf[dt][s2], o);
        if constexpr (DT == 1) o = mfma16x16x32<DT>(pl[s2], vf[dt][s2], o);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int head = 4 * g + i;
        if (head < G) s_o[wave][head][16 * dt + n] = o[i];
      }
    }
    if (g == 0 && n < G) {
      s_m[wave][n] = mx;
      s_l[wave][n] = ps;
    }
  } else {
    if (lane < G) {
      s_m[wave][lane] = -INFINITY;
      s_l[wave][lane] = 0.f;
    }
    for (int e = lane; e < G * kHeadDim; e += 64) s_o[wave][e / kHeadDim][e % kHeadDim] = 0.f;
  }
  __syncthreads();
  const int nsplit = geo.nsplit;
  for (int e = threadIdx.x; e < G * kHeadDim; e += 256) {
    const int head = e / kHeadDim, d = e % kHeadDim;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][head]);
    float L = 0.f, a = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = s_m[w][head];
        const float f = (mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        L += f * s_l[w][head];
        a += f * s_o[w][head][d];
      }
    }
    const size_t row = (size_t)bi * geo.hq + h * G + head;
    if (nsplit == 1) {
      out[row * kHeadDim + d] = from_f32<DT>(L > 0.f ? a / L : 0.f);
    } else {
      float* pp = partials + (row * nsplit + split) * (kHeadDim + 2);
      pp[d] = a;
      if (d == 0) {
        pp[kHeadDim] = M;
        pp[kHeadDim + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// combine split partials: one workgroup per (q head, sequence)
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(128) void k_combine(Geometry geo, const float* __restrict__ partials,
                                                 uint16_t* __restrict__ out) {
  const int hq = blockIdx.x, bi = blockIdx.y, d = threadIdx.x;
  const size_t row = (size_t)bi * geo.hq + hq;
  const int ns = geo.nsplit;
  const float* pp = partials + row * ns * (kHeadDim + 2);
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, pp[s * (kHeadDim + 2) + kHeadDim]);
  float L = 0.f, a = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < ns; ++s) {
      const float m = pp[s * (kHeadDim + 2) + kHeadDim];
      if (m == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(m - M);
      L += f * pp[s * (kHeadDim + 2) + kHeadDim + 1];
      a += f * pp[s * (kHeadDim + 2) + d];
    }
  }
  out[row * kHeadDim + d] = from_f32<DT>(L > 0.f ? a / L : 0.f);
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
  *(u32x4*)(ko + dst) = *(const u32x4*)((const uint16_t*)(slab + geo.k_off) + slot * kHeadDim + 8 * c);
  const uint16_t* Vt = (const uint16_t*)(slab + geo.v_off);
  u32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = (uint32_t)Vt[(8 * c + 2 * e) * geo.tb + slot] |
           ((uint32_t)Vt[(8 * c + 2 * e + 1) * geo.tb + slot] << 16);
  *(u32x4*)(vo + dst) = w;
}

// summaries of one sequence -> [Hkv, nfull, D]; grid (nfull, Hkv)
__global__ __launch_bounds__(128) void k_export_summaries(Geometry geo, int seq, int nfull,
                                                          uint16_t* __restrict__ out) {
  const int j = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int page = block_table(geo, seq)[j];
  out[((size_t)h * nfull + j) * kHeadDim + d] = geo.summ[((size_t)page * geo.hkv + h) * kHeadDim + d];
}

// ===========================================================================
// launchers
// ===========================================================================
hipError_t launch_patch(const Geometry& g, const PatchBatch& pb, hipStream_t s) {
  hipLaunchKernelGGL(k_patch, dim3(1), dim3(256), 0, s, g.meta, pb);
  return hipGetLastError();
}

hipError_t launch_append(const Geometry& g, const AppendBatch& ab, const void* k, const void* v,
                         hipStream_t s) {
  dim3 grid((ab.L + 15) / 16, g.hkv, ab.n);
  hipLaunchKernelGGL(k_append, grid, dim3(256), 0, s, g, ab, (const uint16_t*)k,
                     (const uint16_t*)v);
  return hipGetLastError();
}

hipError_t launch_append_quantized(const Geometry&, const AppendBatch&, const uint32_t*,
                                   const void*, const void*, const uint32_t*, const void*,
                                   const void*, hipStream_t) {
  return hipErrorNotSupported;
}

hipError_t launch_summary(const Geometry& g, const SummaryBatch& sb, int max_count,
                          hipStream_t s) {
  dim3 grid(max_count, g.hkv, sb.n);
  if (g.dtype == 0)
    hipLaunchKernelGGL(k_summary<0>, grid, dim3(128), 0, s, g, sb);
  else
    hipLaunchKernelGGL(k_summary<1>, grid, dim3(128), 0, s, g, sb);
  return hipGetLastError();
}

template <int DT>
static void score_dispatch(const Geometry& g, dim3 grid, const SeqBatch& b, const uint16_t* q,
                           float* sc, hipStream_t s) {
  switch (g.group) {
    case 1: hipLaunchKernelGGL((k_score<DT, 1>), grid, dim3(256), 0, s, g, b, q, sc); break;
    case 2: hipLaunchKernelGGL((k_score<DT, 2>), grid, dim3(256), 0, s, g, b, q, sc); break;
    case 4: hipLaunchKernelGGL((k_score<DT, 4>), grid, dim3(256), 0, s, g, b, q, sc); break;
    case 8: hipLaunchKernelGGL((k_score<DT, 8>), grid, dim3(256), 0, s, g, b, q, sc); break;
    default: hipLaunchKernelGGL((k_score<DT, 16>), grid, dim3(256), 0, s, g, b, q, sc); break;
  }
}

hipError_t launch_score(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                        int max_cand, hipStream_t s) {
  const int per_wg = (16 / g.hkv) * kScoreIters;
  dim3 grid((max_cand + per_wg - 1) / per_wg, b.n);
  if (g.dtype == 0) score_dispatch<0>(g, grid, b, (const uint16_t*)q, scores, s);
  else score_dispatch<1>(g, grid, b, (const uint16_t*)q, scores, s);
  return hipGetLastError();
}

hipError_t launch_topk(const Geometry& g, const SeqBatch& b, const float* scores, int32_t* idx,
                       hipStream_t s) {
  const size_t lds = (size_t)g.mbps * 5;
  hipLaunchKernelGGL(k_topk, dim3(g.hkv, b.n), dim3(256), lds, s, g, b, scores, idx);
  return hipGetLastError();
}

template <int DT, int TB>
static void attend_dispatch(const Geometry& g, dim3 grid, const SeqBatch& b, const uint16_t* q,
                            const int32_t* idx, float sl2, uint16_t* out, float* part,
                            hipStream_t s) {
  switch (g.group) {
    case 1: hipLaunchKernelGGL((k_attend<DT, TB, 1>), grid, dim3(256), 0, s, g, b, q, idx, sl2, out, part); break;
    case 2: hipLaunchKernelGGL((k_attend<DT, TB, 2>), grid, dim3(256), 0, s, g, b, q, idx, sl2, out, part); break;
    case 4: hipLaunchKernelGGL((k_attend<DT, TB, 4>), grid, dim3(256), 0, s, g, b, q, idx, sl2, out, part); break;
    case 8: hipLaunchKernelGGL((k_attend<DT, TB, 8>), grid, dim3(256), 0, s, g, b, q, idx, sl2, out, part); break;
    default: hipLaunchKernelGGL((k_attend<DT, TB, 16>), grid, dim3(256), 0, s, g, b, q, idx, sl2, out, part); break;
  }
}

hipError_t launch_attend(const Geometry& g, const SeqBatch& b, const void* q, const int32_t* idx,
                         float scale, void* out, float* partials, hipStream_t s) {
  const float sl2 = scale * 1.4426950408889634f;
  dim3 grid(g.nsplit, g.hkv, b.n);
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* oo = (uint16_t*)out;
  if (g.dtype == 0) {
    if (g.tb == 64) attend_dispatch<0, 64>(g, grid, b, qq, idx, sl2, oo, partials, s);
    else attend_dispatch<0, 32>(g, grid, b, qq, idx, sl2, oo, partials, s);
  } else {
    if (g.tb == 64) attend_dispatch<1, 64>(g, grid, b, qq, idx, sl2, oo, partials, s);
    else attend_dispatch<1, 32>(g, grid, b, qq, idx, sl2, oo, partials, s);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || g.nsplit == 1) return e;
  if (g.dtype == 0)
    hipLaunchKernelGGL(k_combine<0>, dim3(g.hq, b.n), dim3(128), 0, s, g, partials, oo);
  else
    hipLaunchKernelGGL(k_combine<1>, dim3(g.hq, b.n), dim3(128), 0, s, g, partials, oo);
  return hipGetLastError();
}

hipError_t launch_export(const Geometry& g, const SeqBatch& b, int T, void* k_out, void* v_out,
                         hipStream_t s) {
  dim3 grid((T + 15) / 16, g.hkv, b.n);
  hipLaunchKernelGGL(k_export, grid, dim3(256), 0, s, g, b, T, (uint16_t*)k_out, (uint16_t*)v_out);
  return hipGetLastError();
}

hipError_t launch_export_quantized(const Geometry&, const SeqBatch&, int, uint32_t*, void*, void*,
                                   uint32_t*, void*, void*, hipStream_t) {
  return hipErrorNotSupported;
}

hipError_t launch_export_summaries(const Geometry& g, int seq, int nfull, void* out,
                                   hipStream_t s) {
  hipLaunchKernelGGL(k_export_summaries, dim3(nfull, g.hkv), dim3(128), 0, s, g, seq, nfull,
                     (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace bsattn
