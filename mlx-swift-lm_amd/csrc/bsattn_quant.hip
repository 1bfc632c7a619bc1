// bsattn_quant.hip -- gfx950 kernels of the block-sparse decode path over an
// MLX-style affine-quantized KV cache (b = 4 or 8 bits, group 64 along the
// head dim, fp16 scale and bias per group: w = scale * code + bias).
//
// The slab layout (bsattn_device.h) stores the codes in the order the
// attention kernel's MFMA operands need them, so every gather load is a
// contiguous 1 KiB fragment, and the scales / biases of a lane group's
// tokens as one contiguous run.  Dequantisation is fused into the MFMAs:
//   - a code c becomes the exact fp16 value 1024 + u c with bit operations
//     only (int8: u = 1; int4: u = 1 or 16 by the element's place in its
//     word, the other operand of a unit-16 element taking 1/16, so that
//     every product is the other operand times c plus 1024 times it);
//   - QK per group g of 64 dims: raw_g = sum_d q'_d (1024 + u_d c_d), so
//     sum_d q_d c_d = raw_g - 1024 Q'_g with Q'_g = sum_d q'_d (one MFMA
//     against an all-ones operand; q' = q with the 1/16 applied), and
//     s = sum_g k_scale_g * sum_d q_d c_d + k_bias_g * Q_g (Q_g = sum_d q_d);
//   - PV per group: P_g = p * v_scale_g (fp16, times 1/16 at unit-16
//     tokens) is the A operand against the codes; the same P_g and
//     p * v_bias_g against an all-ones operand give sum_t P_g and
//     sum_t p v_bias_g in the accumulator layout of O, so
//     o = raw - 1024 sum P_g + sum p v_bias_g needs no shuffles (the PV
//     accumulator starts at sum p v_bias_g - 1024 sum P_g).
// Summaries of a quantized cache are fp16 means of the dequantized keys
// (fmaf(scale, code, bias), sequential fold), so scoring and selection are
// the 16-bit kernels' own.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bsattn_device.h"

namespace bsattn {

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ float lo_f(uint32_t w) { return h2f(w & 0xFFFFu); }
__device__ __forceinline__ float hi_f(uint32_t w) { return h2f(w >> 16); }

// Codes as the decode kernel's MFMA operands: int8 code c is the fp16
// 1024 + c (byte_to_f16); an int4 word (element e in nibble q_nib(e)) gives
// pairs 0 and 2 (elements 0, 1, 4, 5) as 1024 + c and pairs 1 and 3
// (elements 2, 3, 6, 7) as 1024 + 16 c: pair k's nibbles k and k + 4 sit at
// bits 4 (k & 1) and 16 + 4 (k & 1) once the word is shifted by 8 (k >> 1),
// inside the fp16 mantissa under the exponent of 1024, so a word costs one
// shift and four v_and_or_b32 (base: 0x64006400 in a VGPR).  The other
// operand of each unit-16 element is scaled by 1/16 (kUnit16), so every
// product is q c (or p c) plus 1024 times the other operand, and
// sum (1024 + u c) x = sum x c u + 1024 sum x removes the offset with the sum
// of the same scaled operand.
__device__ __forceinline__ u32x4 nib_to_f16_dec(uint32_t w, uint32_t base) {
  const uint32_t w8 = w >> 8;
  return u32x4{(w & 0x000F000Fu) | base, (w & 0x00F000F0u) | base, (w8 & 0x000F000Fu) | base,
               (w8 & 0x00F000F0u) | base};
}
constexpr float kDecOff = 1024.0f;  // value of code 0 in the decode operands
constexpr float kUnit16 = 0.0625f;  // scale of the other operand at unit-16 int4 elements

// 0x64006400 (two fp16 1024.0) in a VGPR the compiler cannot fold into the
// v_and_or_b32 (a DPP identity move: unlike an inline-asm move, the
// compiler sees its register write, so the MFMA hazard wait states around
// it are inserted)
__device__ __forceinline__ uint32_t f16_pair_1024() {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)0x64006400, 0xE4, 0xF, 0xF, false);
}

// A operand of QK token tile t, k-step s, from the tile's K fragments
template <int KB>
__device__ __forceinline__ u32x4 k_operand(const u32x4* kf, int s, uint32_t base) {
  if constexpr (KB == 4) return nib_to_f16_dec(kf[0][s], base);
  else return byte_to_f16(kf[s >> 1][2 * (s & 1)], kf[s >> 1][2 * (s & 1) + 1]);
}

// B operand of PV dim tile dt, k-step s2, from the V fragments
template <int KB, int KS2>
__device__ __forceinline__ u32x4 v_operand(const u32x4* vf, int dt, int s2, uint32_t base) {
  constexpr int DPF = QCode<KB>::DPF;
  const u32x4& f = vf[(dt / DPF) * KS2 + s2];
  if constexpr (KB == 4) return nib_to_f16_dec(f[dt & 3], base);
  else return byte_to_f16(f[2 * (dt & 1)], f[2 * (dt & 1) + 1]);
}

// x * 1/16 on both fp16 halves (exact unless the result is below fp16's
// normal range)
__device__ __forceinline__ uint32_t f16x2_unit16(uint32_t x) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, x) * f16x2{(_Float16)kUnit16, (_Float16)kUnit16});
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// DPP inside each 16-lane row (bank b = lanes 4b .. 4b+3 of the row); r and
// t are constants once the calling loops are unrolled.
// row_ror: lane n reads lane (n - r) mod 16 of its row (r in {4, 8, 12}).
__device__ __forceinline__ uint32_t row_ror(uint32_t x, int r) {
  switch (r) {
    case 4: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x124, 0xF, 0xF, false);
    case 8: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, false);
    case 12: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x12C, 0xF, 0xF, false);
    default: return x;
  }
}
__device__ __forceinline__ float row_ror(float x, int r) {
  return __uint_as_float(row_ror(__float_as_uint(x), r));
}
// old with bank t (1..3) replaced by src's bank 0
__device__ __forceinline__ float bank_from0(float old, float src, int t) {
  const int o = __float_as_int(old), s = __float_as_int(src);
  switch (t) {
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(o, s, 0x124, 0xF, 0x2, false));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(o, s, 0x128, 0xF, 0x4, false));
    case 3: return __int_as_float(__builtin_amdgcn_update_dpp(o, s, 0x12C, 0xF, 0x8, false));
    default: return src;
  }
}

// ---------------------------------------------------------------------------
// quantize 8 consecutive dims of one row (lane c of the 16 lanes holding the
// row; lanes c & ~7 .. +7 hold one 64-dim group) by mlx's affine rule, in
// fp32 with correctly rounded divisions:
//   scale = max((max - min) / (2^b - 1), 1e-7), negated unless
//   |min| > |max|; edge = min if |min| > |max| else max;
//   q0 = rint(edge / scale); q0 != 0: scale = edge / q0, bias = edge;
//   q0 == 0 (an all-zero group): bias = 0;
//   code = clamp(rint((x - bias) / scale), 0, 2^b - 1) from the fp32 scale
//   and bias, which are stored rounded to fp16.
// (Signed zeros cannot matter: q0 == 0 only when edge is a zero, and then
// bias is +0.)
// ---------------------------------------------------------------------------
template <int KB>
__device__ __forceinline__ void quantize8(const uint16_t* __restrict__ src, int c, uint8_t* codes,
                                          uint16_t* scale_out, uint16_t* bias_out) {
  const u32x4 raw = *(const u32x4*)src;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (e & 1) ? hi_f(raw[e >> 1]) : lo_f(raw[e >> 1]);
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    mn = fminf(mn, x[e]);
    mx = fmaxf(mx, x[e]);
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, off, 64));
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  }
  constexpr float nbins = (float)((1 << KB) - 1);
  float scale = fmaxf(__fdiv_rn(__fsub_rn(mx, mn), nbins), (float)1e-7);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = __builtin_rintf(__fdiv_rn(edge, scale));
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = __fdiv_rn(edge, q0);
    bias = edge;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float qv = __builtin_rintf(__fdiv_rn(__fsub_rn(x[e], bias), scale));
    qv = qv < 0.0f ? 0.0f : qv;
    qv = qv > nbins ? nbins : qv;
    codes[e] = (uint8_t)qv;
  }
  if ((c & 7) == 0) {
    *scale_out = __builtin_bit_cast(uint16_t, (_Float16)scale);
    *bias_out = __builtin_bit_cast(uint16_t, (_Float16)bias);
  }
}

// ---------------------------------------------------------------------------
// append: workgroup x covers the 8-aligned positions [P0, P0 + 8),
// P0 = 8 * (old_len / 8 + x), of one (sequence, kv head); the tokens
// appended there are [max(P0, old), min(P0 + 8, old + L)).  Stage 1 puts
// their codes and scales / biases in LDS (quantizing fp16 input, or
// unpacking the MLX layout: element i of a row in word i / (32/b), bits
// b * (i % (32/b)) up, LSB first; scales / biases [.., D / 64]); stage 2
// writes whole 32-bit words: K words belong to one token, a V word to one dim
// and the 8 (int4) or 4 (int8) tokens of this group, merged with the codes
// already there when the group is only partly new.
// grid (L / 8 + 2, Hkv, n), 128 threads
// ---------------------------------------------------------------------------
template <int KB, bool QUANTIZE>
__global__ __launch_bounds__(128) void k_append_q(Geometry geo, AppendBatch ab,
                                                  const uint16_t* __restrict__ k16,
                                                  const uint16_t* __restrict__ v16,
                                                  const uint32_t* __restrict__ kw,
                                                  const uint16_t* __restrict__ ks,
                                                  const uint16_t* __restrict__ kb,
                                                  const uint32_t* __restrict__ vw,
                                                  const uint16_t* __restrict__ vs,
                                                  const uint16_t* __restrict__ vb) {
  constexpr int WPR = QCode<KB>::WPR;
  __shared__ uint8_t s_kc[8][kHeadDim];
  __shared__ uint8_t s_vc[8][kHeadDim];
  __shared__ uint32_t s_sb[8][4];
  const int bi = blockIdx.z, h = blockIdx.y;
  const int old = ab.old_len[bi], L = ab.L;
  const int P0 = 8 * (old / 8 + (int)blockIdx.x);
  const int lo = max(P0, old), hi = min(P0 + 8, old + L);
  if (lo >= hi) return;
  const int seq = ab.seq[bi];
  const int tid = threadIdx.x;
  {
    const int i = tid >> 4, c = tid & 15;  // token P0 + i, dims 8c .. 8c+7
    const int pos = P0 + i;
    if (pos >= lo && pos < hi) {
      const size_t row = ((size_t)bi * geo.hkv + h) * L + (pos - old);
      uint16_t* sbh = (uint16_t*)s_sb[i];
      if constexpr (QUANTIZE) {
        const int grp = c >> 3;
        quantize8<KB>(k16 + row * kHeadDim + 8 * c, c, &s_kc[i][8 * c], sbh + grp, sbh + 2 + grp);
        quantize8<KB>(v16 + row * kHeadDim + 8 * c, c, &s_vc[i][8 * c], sbh + 4 + grp, sbh + 6 + grp);
      } else {
        if constexpr (KB == 4) {
          const uint32_t a = kw[row * WPR + c], b = vw[row * WPR + c];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            s_kc[i][8 * c + e] = (uint8_t)((a >> (4 * e)) & 15u);
            s_vc[i][8 * c + e] = (uint8_t)((b >> (4 * e)) & 15u);
          }
        } else {
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const uint32_t a = kw[row * WPR + 2 * c + w], b = vw[row * WPR + 2 * c + w];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              s_kc[i][8 * c + 4 * w + e] = (uint8_t)(a >> (8 * e));
              s_vc[i][8 * c + 4 * w + e] = (uint8_t)(b >> (8 * e));
            }
          }
        }
        if (c < 2) {
          sbh[c] = ks[row * 2 + c];
          sbh[2 + c] = kb[row * 2 + c];
          sbh[4 + c] = vs[row * 2 + c];
          sbh[6 + c] = vb[row * 2 + c];
        }
      }
    }
  }
  __syncthreads();
  const int blk = P0 / geo.tb, slot0 = P0 - blk * geo.tb;
  const int page = block_table(geo, seq)[blk];
  uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  uint8_t* Kc = slab + geo.k_off;
  uint8_t* Vc = slab + geo.v_off;
  // K: 8 tokens x WPR words
  for (int u = tid; u < 8 * WPR; u += 128) {
    const int i = u / WPR, wd = u - i * WPR;
    const int pos = P0 + i;
    if (pos < lo || pos >= hi) continue;
    int sh;
    uint32_t word = 0u;
    if constexpr (KB == 4) {
#pragma unroll
      for (int e = 0; e < 8; ++e) word |= (uint32_t)s_kc[i][8 * wd + e] << (4 * q_nib(e));
      *(uint32_t*)(Kc + kq_byte(4, slot0 + i, 8 * wd, &sh)) = word;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) word |= (uint32_t)s_kc[i][4 * wd + e] << (8 * e);
      *(uint32_t*)(Kc + kq_byte(8, slot0 + i, 4 * wd, &sh)) = word;
    }
  }
  // V: thread = dim; words of this group's tokens
  {
    const int d = tid;
    constexpr int TPW = 32 / KB;  // tokens per word
#pragma unroll
    for (int w = 0; w < 8 / TPW; ++w) {
      const int t0 = P0 + w * TPW;
      if (t0 + TPW <= lo || t0 >= hi) continue;
      int sh;
      uint32_t* dst = (uint32_t*)(Vc + vq_byte(KB, geo.tb, slot0 + w * TPW, d, &sh));
      const bool whole = t0 >= lo && t0 + TPW <= hi;
      uint32_t word = whole ? 0u : *dst;
#pragma unroll
      for (int e = 0; e < TPW; ++e) {
        const int pos = t0 + e;
        if (pos < lo || pos >= hi) continue;
        const int at = KB == 4 ? 4 * q_nib(e) : 8 * e;
        const uint32_t mask = ((1u << KB) - 1u) << at;
        word = (word & ~mask) | ((uint32_t)s_vc[pos - P0][d] << at);
      }
      *dst = word;
    }
  }
  // scales / biases: 16 B per token
  if (tid < 8) {
    const int pos = P0 + tid;
    if (pos >= lo && pos < hi) {
      u32x4* dst = (u32x4*)(slab + geo.sb_off) + sb_entry(geo.tb, slot0 + tid);
      *dst = u32x4{s_sb[tid][0], s_sb[tid][1], s_sb[tid][2], s_sb[tid][3]};
    }
  }
}

// ---------------------------------------------------------------------------
// block summary of a quantized block: thread per dim, sequential fp32 fold
// of the dequantized keys fmaf(scale, code, bias) from token 0, times 1/Tb,
// to fp16.  grid (max_count, Hkv, n)
// ---------------------------------------------------------------------------
template <int KB>
__global__ __launch_bounds__(128) void k_summary_q(Geometry geo, SummaryBatch sb) {
  const int bi = blockIdx.z, h = blockIdx.y;
  if ((int)blockIdx.x >= sb.count[bi]) return;
  const int seq = sb.seq[bi];
  const int j = sb.first[bi] + blockIdx.x;
  const int page = block_table(geo, seq)[j];
  const int d = threadIdx.x, grp = d >> 6;
  const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  const uint8_t* Kc = slab + geo.k_off;
  const uint16_t* Sb = (const uint16_t*)(slab + geo.sb_off);
  float acc = 0.0f;
  for (int t = 0; t < geo.tb; ++t) {
    int sh;
    const int code = (Kc[kq_byte(KB, t, d, &sh)] >> sh) & ((1 << KB) - 1);
    const uint16_t* f = Sb + 8 * sb_entry(geo.tb, t);
    const float w = __builtin_fmaf(h2f(f[grp]), (float)code, h2f(f[2 + grp]));
    acc = (t == 0) ? w : __fadd_rn(acc, w);
  }
  summary_row(geo, seq, h, j)[d] =
      __builtin_bit_cast(uint16_t, (_Float16)__fmul_rn(acc, 1.0f / (float)geo.tb));
}

// ---------------------------------------------------------------------------
// gathered attention over quantized blocks: the 16-bit kernel's structure
// (one block per wave, W waves per workgroup, selection fused when SEL,
// split partials merged by k_combine), with the dequantisation folded into
// the MFMAs as described at the top of this file.  q / out are fp16.
// grid (nsplit, Hkv, n).  Workgroups per CU the register budget is sized
// for: two 9-wave ones for 16-head groups over given indices (launched
// for 32-token blocks, 72 VGPRs), five 4-wave ones for wide groups of
// 32-token blocks over given indices, otherwise one (9 waves) or two (4).
// ---------------------------------------------------------------------------
template <int TB, int G, int W, int SEL, int KB>
__global__ __launch_bounds__(64 * W, W > 4 ? (G > 8 && SEL == 0 ? 2 : 1) : G > 4 && SEL == 0 && TB == 32 ? 5 : 2) void k_attend_q(Geometry geo, SeqBatch sb,
                                                     const uint16_t* __restrict__ q,
                                                     int32_t* __restrict__ idx,
                                                     const float* __restrict__ scores,
                                                     float sl2, uint16_t* __restrict__ out,
                                                     float* __restrict__ partials) {
  using QC = QCode<KB>;
  constexpr int NT = TB / 16;   // QK token tiles
  constexpr int EPL = TB / 4;   // scores per lane
  constexpr int KS2 = TB / 32;  // PV k-steps
  constexpr int KF = QC::KF;
  constexpr int NVF = (8 / QC::DPF) * KS2;  // V fragments
  // HALF (16-head groups): the waves' outputs are merged in two halves of
  // 64 dims through one half-width buffer (4 KB less LDS per wave: over
  // given indices a 4-wave workgroup fits 32 KB, five to a CU, and two
  // 9-wave workgroups fit a CU)
  constexpr bool HALF = G > 8;
  constexpr int OD = HALF ? kHeadDim / 2 : kHeadDim;
  __shared__ float s_m[W][16], s_l[W][16];
  __shared__ float s_o[W][G][OD];
  __shared__ int s_sel[SEL ? kSelMaxK : 1];
  __shared__ int s_selp[SEL ? kSelMaxK : 1];
  __shared__ __align__(16) uint32_t s_ws[SEL == 2 ? slot_scratch_words<W>() : SEL ? kWaveScratch : 4];
  // wide groups: each wave's block of TB scale / bias entries, one per lane
  // through LDS (4 registers held while K and V are in flight, not EPL x 4)
  __shared__ __align__(16) u32x4 s_sb[G > 4 ? W : 1][G > 4 ? TB : 1];
  const int split = blockIdx.x, h = blockIdx.y, bi = blockIdx.z;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int seq = sb.ids[bi];
  // given indices: the slot's block index heads the longest dependent chain
  // (index -> page -> K/V), so it is requested before the length and Q
  const int jg = SEL ? -1 : given_index(geo, idx, bi, h, split * W + wave);
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
  f32x4 oh[HALF ? 4 : 1];  // HALF: O's dims 64 .. 127, stored after the first merge
  attend_pick<TB, W, SEL>(geo, bi, h, seq, len, split * W + wave, split == 0 && wave == 0, wave, lane,
                          idx, jg, &wc, &wgc, s_sel, s_selp, s_ws, j, page);
  if (j >= 0) {
    const int valid = min(TB, len - j * TB);
    const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
    const u32x4* Kf = (const u32x4*)(slab + geo.k_off) + lane;
    const u32x4* Vf = (const u32x4*)(slab + geo.v_off) + lane;
    const u32x4* Sf = (const u32x4*)(slab + geo.sb_off) + g * EPL;
    constexpr bool CMP = G <= 4;
    // wide groups: entry lane of the block's scales / biases (lanes past TB
    // repeat one), requested ahead of K and V
    u32x4 sbx;
    if constexpr (!CMP) sbx = ((const u32x4*)(slab + geo.sb_off))[lane & (TB - 1)];
    u32x4 kf[NT][KF];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int f = 0; f < KF; ++f) kf[t][f] = __builtin_nontemporal_load(Kf + (t * KF + f) * 64);
    u32x4 vf[NVF];
#pragma unroll
    for (int i = 0; i < NVF; ++i) vf[i] = __builtin_nontemporal_load(Vf + i * 64);
    // CMP (groups of at most 4 heads): the real heads of a QK tile's scores
    // are the lanes of bank 0 (n < 4) of each row, so tile t is rotated into
    // bank t and the per-score work runs on 4 registers instead of EPL;
    // lane (n, g) then holds head n & 3, tile n >> 2, entries 4 (n >> 2) + i
    const int tcp = n >> 2;
    u32x4 sbv[CMP ? 4 : 1];  // CMP: this lane's scale / bias entries
    if constexpr (CMP) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sbv[i] = tcp < NT ? Sf[4 * tcp + i] : u32x4{0u, 0u, 0u, 0u};
    }
    // entry e of this lane (wide groups: from LDS)
    auto sbe = [&](int e) __attribute__((always_inline)) -> u32x4 {
      if constexpr (CMP) return sbv[e];
      else return s_sb[wave][g * EPL + e];
    };
    __builtin_amdgcn_sched_barrier(0);
    const u32x4 ones = u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
    const uint32_t base = f16_pair_1024();
    // the QK operand: q, with int4's unit-16 elements (2, 3, 6, 7 of every
    // k-step) scaled by 1/16
    u32x4 qk[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qk[s] = qf[s];
      if constexpr (KB == 4) {
        qk[s][1] = f16x2_unit16(qf[s][1]);
        qk[s][3] = f16x2_unit16(qf[s][3]);
      }
    }
    // per dim group g, for head n (every accumulator entry): the sum of the
    // QK operand (qs, for the code offset) and of q (qb, for the biases)
    f32x4 qs0 = mfma_f16(ones, qk[0], f32x4{0.f, 0.f, 0.f, 0.f});
    qs0 = mfma_f16(ones, qk[1], qs0);
    f32x4 qs1 = mfma_f16(ones, qk[2], f32x4{0.f, 0.f, 0.f, 0.f});
    qs1 = mfma_f16(ones, qk[3], qs1);
    f32x4 qb0 = qs0, qb1 = qs1;
    if constexpr (KB == 4) {
      qb0 = mfma_f16(ones, qf[0], f32x4{0.f, 0.f, 0.f, 0.f});
      qb0 = mfma_f16(ones, qf[1], qb0);
      qb1 = mfma_f16(ones, qf[2], f32x4{0.f, 0.f, 0.f, 0.f});
      qb1 = mfma_f16(ones, qf[3], qb1);
    }
    if constexpr (!CMP) {
      // lane (n, g) reads entries g * EPL + e (token tok_of(g, e)), stored by
      // their lanes here; those of tokens past the block's valid ones are
      // zero, so that no stale scale / bias reaches PV
      if (lane < TB)
        s_sb[wave][lane] = tok_of(lane / EPL, lane % EPL) < valid ? sbx : u32x4{0u, 0u, 0u, 0u};
      wave_lds_order();
    }
    // A operands: P_g = p * v_scale_g and p * v_bias_g per dim group
    u32x4 pa0[KS2], pa1[KS2], pb0[KS2], pb1[KS2];
    float mx, ps;
    if constexpr (CMP) {
      // raw_g = K-codes-as-fp16 . Q^T per dim group, every tile
      f32x4 r0[NT], r1[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        r0[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        r1[t] = r0[t];
        r0[t] = mfma_f16(k_operand<KB>(kf[t], 0, base), qk[0], r0[t]);
        r0[t] = mfma_f16(k_operand<KB>(kf[t], 1, base), qk[1], r0[t]);
        r1[t] = mfma_f16(k_operand<KB>(kf[t], 2, base), qk[2], r1[t]);
        r1[t] = mfma_f16(k_operand<KB>(kf[t], 3, base), qk[3], r1[t]);
      }
      f32x4 c0 = r0[0], c1 = r1[0];
#pragma unroll
      for (int t = 1; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c0[i] = bank_from0(c0[i], r0[t][i], t);
          c1[i] = bank_from0(c1[i], r1[t][i], t);
        }
      // of head n & 3 after the rotations
      float q0c = qs0[0], q1c = qs1[0], q0 = qb0[0], q1 = qb1[0];
#pragma unroll
      for (int t = 1; t < 4; ++t) {
        q0c = bank_from0(q0c, qs0[0], t);
        q1c = bank_from0(q1c, qs1[0], t);
        if constexpr (KB == 4) {
          q0 = bank_from0(q0, qb0[0], t);
          q1 = bank_from0(q1, qb1[0], t);
        }
      }
      if constexpr (KB != 4) {
        q0 = q0c;
        q1 = q1c;
      }
      q0c *= kDecOff;
      q1c *= kDecOff;
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4& f = sbv[i];
        const float d0 = c0[i] - q0c;  // sum_d q_d c_d, group 0
        const float d1 = c1[i] - q1c;
        float sc = lo_f(f[0]) * d0;
        sc = __builtin_fmaf(lo_f(f[1]), q0, sc);
        sc = __builtin_fmaf(hi_f(f[0]), d1, sc);
        sc = __builtin_fmaf(hi_f(f[1]), q1, sc);
        pv[i] = sc * sl2;
      }
      // tokens past the end (and, for 32-token blocks, the banks past the
      // block's two tiles): no score, and no stale scale / bias reaches PV
      if (NT < 4 || valid < TB) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tok_of(g, 4 * tcp + i) >= valid) {
            pv[i] = -INFINITY;
            sbv[i] = u32x4{0u, 0u, 0u, 0u};
          }
      }
      // per head: over the lane's entries, the row's 4 banks, the 4 rows
      float m = fmaxf(fmaxf(pv[0], pv[1]), fmaxf(pv[2], pv[3]));
      m = fmaxf(m, row_ror(m, 4));
      m = fmaxf(m, row_ror(m, 8));
      mx = max_over_groups(m);
      ps = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(pv[i] - mx);
        ps += pv[i];
      }
      ps += row_ror(ps, 4);
      ps += row_ror(ps, 8);
      ps = sum_over_groups(ps);
      // compact pairs (entries 2 pp, 2 pp + 1), then each A operand pair jj
      // of k-step s2 (tokens of tile 2 s2 + jj / 2, entries 2 (jj % 2) ..)
      // is rotated from its tile's bank into bank 0 (rows of the other banks
      // are heads past the group, never stored)
      // (pair 1's tokens meet int4's unit-16 V elements: P_g takes 1/16)
      uint32_t ca0[2], ca1[2], cb0[2], cb1[2];
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const float p0 = pv[2 * pp], p1 = pv[2 * pp + 1];
        const float u = KB == 4 && pp == 1 ? kUnit16 : 1.0f;
        const u32x4 &f0 = sbv[2 * pp], &f1 = sbv[2 * pp + 1];
        ca0[pp] = cvt_pk<0>(p0 * u * lo_f(f0[2]), p1 * u * lo_f(f1[2]));
        ca1[pp] = cvt_pk<0>(p0 * u * hi_f(f0[2]), p1 * u * hi_f(f1[2]));
        cb0[pp] = cvt_pk<0>(p0 * lo_f(f0[3]), p1 * lo_f(f1[3]));
        cb1[pp] = cvt_pk<0>(p0 * hi_f(f0[3]), p1 * hi_f(f1[3]));
      }
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = (16 - 4 * (2 * s2 + (jj >> 1))) & 15, pp = jj & 1;
          pa0[s2][jj] = row_ror(ca0[pp], r);
          pa1[s2][jj] = row_ror(ca1[pp], r);
          pb0[s2][jj] = row_ror(cb0[pp], r);
          pb1[s2][jj] = row_ror(cb1[pp], r);
        }
    } else {
      const float q0 = qb0[0], q1 = qb1[0];
      const float q0c = qs0[0] * kDecOff, q1c = qs1[0] * kDecOff;
      // raw_g = K-codes-as-fp16 . Q^T per dim group
      float pv[EPL];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 r0 = f32x4{0.f, 0.f, 0.f, 0.f}, r1 = r0;
        r0 = mfma_f16(k_operand<KB>(kf[t], 0, base), qk[0], r0);
        r0 = mfma_f16(k_operand<KB>(kf[t], 1, base), qk[1], r0);
        r1 = mfma_f16(k_operand<KB>(kf[t], 2, base), qk[2], r1);
        r1 = mfma_f16(k_operand<KB>(kf[t], 3, base), qk[3], r1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 f = sbe(4 * t + i);
          const float d0 = r0[i] - q0c;  // sum_d q_d c_d, group 0
          const float d1 = r1[i] - q1c;
          float sc = lo_f(f[0]) * d0;
          sc = __builtin_fmaf(lo_f(f[1]), q0, sc);
          sc = __builtin_fmaf(hi_f(f[0]), d1, sc);
          sc = __builtin_fmaf(hi_f(f[1]), q1, sc);
          pv[4 * t + i] = sc * sl2;
        }
      }
      if (valid < TB) {
        // tokens past the end: no score (their scales / biases are zero)
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          if (tok_of(g, e) >= valid) pv[e] = -INFINITY;
      }
      mx = pv[0];
#pragma unroll
      for (int e = 1; e < EPL; ++e) mx = fmaxf(mx, pv[e]);
      mx = max_over_groups(mx);
      ps = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(pv[e] - mx);
        ps += pv[e];
      }
      ps = sum_over_groups(ps);
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int e0 = 8 * s2 + 2 * jj, e1 = e0 + 1;
          const float p0 = pv[e0], p1 = pv[e1];
          const float u = KB == 4 && (jj & 1) ? kUnit16 : 1.0f;  // int4's unit-16 V elements
          const u32x4 f0 = sbe(e0), f1 = sbe(e1);
          pa0[s2][jj] = cvt_pk<0>(p0 * u * lo_f(f0[2]), p1 * u * lo_f(f1[2]));
          pa1[s2][jj] = cvt_pk<0>(p0 * u * hi_f(f0[2]), p1 * u * hi_f(f1[2]));
          pb0[s2][jj] = cvt_pk<0>(p0 * lo_f(f0[3]), p1 * lo_f(f1[3]));
          pb1[s2][jj] = cvt_pk<0>(p0 * hi_f(f0[3]), p1 * hi_f(f1[3]));
        }
    }
    // sum_t P_g and sum_t p v_bias_g, in O's accumulator layout
    f32x4 ps0 = f32x4{0.f, 0.f, 0.f, 0.f}, ps1 = ps0, vb0 = ps0, vb1 = ps0;
#pragma unroll
    for (int s2 = 0; s2 < KS2; ++s2) {
      ps0 = mfma_f16(pa0[s2], ones, ps0);
      ps1 = mfma_f16(pa1[s2], ones, ps1);
      vb0 = mfma_f16(pb0[s2], ones, vb0);
      vb1 = mfma_f16(pb1[s2], ones, vb1);
    }
    // O = P_g . V codes, corrected per dim group: each tile's accumulator
    // starts at sum_t p v_bias_g - kDecOff sum_t P_g (the codes' offset)
    f32x4 oc0, oc1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      oc0[i] = __builtin_fmaf(-kDecOff, ps0[i], vb0[i]);
      oc1[i] = __builtin_fmaf(-kDecOff, ps1[i], vb1[i]);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 o = dt < 4 ? oc0 : oc1;
#pragma unroll
      for (int s2 = 0; s2 < KS2; ++s2) o = mfma_f16(dt < 4 ? pa0[s2] : pa1[s2], v_operand<KB, KS2>(vf, dt, s2, base), o);
      if (!HALF || dt < 4) store_o_tile<G, OD>(s_o[wave], dt, n, g, o);
      else oh[dt & 3] = o;
    }
    if (g == 0 && n < G) {
      s_m[wave][n] = mx;
      s_l[wave][n] = ps;
    }
  } else {
    store_empty<G, OD>(s_m[wave], s_l[wave], s_o[wave], lane);
    if constexpr (HALF) {
#pragma unroll
      for (int t = 0; t < 4; ++t) oh[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __syncthreads();
  if constexpr (HALF) {
    __shared__ float s_f[W][16], s_ML[2][16];
    merge_weights<G, W>(s_m, s_l, s_f, s_ML);
    __syncthreads();
    merge_dims<0, G, W, OD>(geo, sb, bi, h, split, (int)gridDim.x, s_f, s_ML, s_o, 0, out, partials);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) store_o_tile<G, OD>(s_o[wave], t, n, g, oh[t]);
    __syncthreads();
    merge_dims<0, G, W, OD>(geo, sb, bi, h, split, (int)gridDim.x, s_f, s_ML, s_o, OD, out, partials);
  } else {
    attend_merge<0, G, W>(geo, sb, bi, h, split, (int)gridDim.x, s_m, s_l, s_o, out, partials);
  }
}

// ---------------------------------------------------------------------------
// export in the MLX layout: kw / vw [n, Hkv, T, D*b/32] uint32 (LSB first),
// scales / biases [n, Hkv, T, D/64] fp16.  grid (ceil(T/16), Hkv, n)
// ---------------------------------------------------------------------------
template <int KB>
__global__ __launch_bounds__(256) void k_export_q(Geometry geo, SeqBatch sb, int T,
                                                  uint32_t* __restrict__ kw, uint16_t* __restrict__ ks,
                                                  uint16_t* __restrict__ kb, uint32_t* __restrict__ vw,
                                                  uint16_t* __restrict__ vs, uint16_t* __restrict__ vb) {
  constexpr int WPR = QCode<KB>::WPR;
  constexpr int EPW = 32 / KB;  // elements per MLX word
  const int bi = blockIdx.z, h = blockIdx.y;
  const int tok = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  if (tok >= T) return;
  const int seq = sb.ids[bi];
  const int blk = tok / geo.tb, slot = tok - blk * geo.tb;
  const int page = block_table(geo, seq)[blk];
  const uint8_t* slab = geo.pool + ((size_t)page * geo.hkv + h) * geo.slab_bytes;
  const size_t row = ((size_t)bi * geo.hkv + h) * T + tok;
  constexpr uint32_t mask = (1u << KB) - 1u;
#pragma unroll
  for (int w = 0; w < WPR / 16; ++w) {
    const int wd = (WPR / 16) * c + w;
    uint32_t a = 0u, b = 0u;
#pragma unroll
    for (int e = 0; e < EPW; ++e) {
      const int d = wd * EPW + e;
      int sh;
      a |= ((uint32_t)(slab[geo.k_off + kq_byte(KB, slot, d, &sh)] >> sh) & mask) << (KB * e);
      b |= ((uint32_t)(slab[geo.v_off + vq_byte(KB, geo.tb, slot, d, &sh)] >> sh) & mask) << (KB * e);
    }
    kw[row * WPR + wd] = a;
    vw[row * WPR + wd] = b;
  }
  if (c < 2) {
    const uint16_t* f = (const uint16_t*)(slab + geo.sb_off) + 8 * sb_entry(geo.tb, slot);
    ks[row * 2 + c] = f[c];
    kb[row * 2 + c] = f[2 + c];
    vs[row * 2 + c] = f[4 + c];
    vb[row * 2 + c] = f[6 + c];
  }
}

// ===========================================================================
// launchers
// ===========================================================================
hipError_t launch_append_q16(const Geometry& g, const AppendBatch& ab, const void* k,
                             const void* v, hipStream_t s, Timing* prof) {
  const dim3 grid(ab.L / 8 + 2, g.hkv, ab.n);
  const uint16_t *k16 = (const uint16_t*)k, *v16 = (const uint16_t*)v;
  if (g.kv_bits == 4)
    launch(k_append_q<4, true>, grid, dim3(128), 0, s, prof, kProfAppend, g, ab, k16, v16,
             (const uint32_t*)nullptr, (const uint16_t*)nullptr, (const uint16_t*)nullptr,
             (const uint32_t*)nullptr, (const uint16_t*)nullptr, (const uint16_t*)nullptr);
  else
    launch(k_append_q<8, true>, grid, dim3(128), 0, s, prof, kProfAppend, g, ab, k16, v16,
             (const uint32_t*)nullptr, (const uint16_t*)nullptr, (const uint16_t*)nullptr,
             (const uint32_t*)nullptr, (const uint16_t*)nullptr, (const uint16_t*)nullptr);
  return hipGetLastError();
}

hipError_t launch_append_quantized(const Geometry& g, const AppendBatch& ab, const uint32_t* kw,
                                   const void* ks, const void* kb, const uint32_t* vw,
                                   const void* vs, const void* vb, hipStream_t s, Timing* prof) {
  const dim3 grid(ab.L / 8 + 2, g.hkv, ab.n);
  const uint16_t* nul = nullptr;
  if (g.kv_bits == 4)
    launch(k_append_q<4, false>, grid, dim3(128), 0, s, prof, kProfAppend, g, ab, nul, nul, kw,
             (const uint16_t*)ks, (const uint16_t*)kb, vw, (const uint16_t*)vs, (const uint16_t*)vb);
  else
    launch(k_append_q<8, false>, grid, dim3(128), 0, s, prof, kProfAppend, g, ab, nul, nul, kw,
             (const uint16_t*)ks, (const uint16_t*)kb, vw, (const uint16_t*)vs, (const uint16_t*)vb);
  return hipGetLastError();
}

hipError_t launch_summary_q(const Geometry& g, const SummaryBatch& sb, int max_count,
                            hipStream_t s, Timing* prof) {
  const dim3 grid(max_count, g.hkv, sb.n);
  if (g.kv_bits == 4) launch(k_summary_q<4>, grid, dim3(128), 0, s, prof, kProfSummary, g, sb);
  else launch(k_summary_q<8>, grid, dim3(128), 0, s, prof, kProfSummary, g, sb);
  return hipGetLastError();
}

template <int TB, int SEL, int KB>
static void attend_q_group(const Geometry& g, int waves, dim3 grid, const SeqBatch& b, const uint16_t* q,
                           int32_t* idx, const float* sc, float sl2, uint16_t* out, float* part,
                           hipStream_t s, Timing* prof) {
  const int kd = kProfAttend;
  if constexpr (SEL != 1) {  // the wide workgroup: groups of up to 4 or of 16 heads, never one selecting wave
    if (waves == kWavesWide) {
      constexpr int W = kWavesWide;
      const dim3 blk(64 * W);
      switch (g.group) {
        case 1: launch(k_attend_q<TB, 1, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
        case 2: launch(k_attend_q<TB, 2, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
        case 16: launch(k_attend_q<TB, 16, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
        default: launch(k_attend_q<TB, 4, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
      }
      return;
    }
  }
  constexpr int W = kWaves;
  const dim3 blk(64 * W);
  switch (g.group) {
    case 1: launch(k_attend_q<TB, 1, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    case 2: launch(k_attend_q<TB, 2, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    case 4: launch(k_attend_q<TB, 4, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    case 8: launch(k_attend_q<TB, 8, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
    default: launch(k_attend_q<TB, 16, W, SEL, KB>, grid, blk, 0, s, prof, kd, g, b, q, idx, sc, sl2, out, part); break;
  }
}

template <int SEL>
static void attend_q_sel(const Geometry& g, int waves, dim3 grid, const SeqBatch& b, const uint16_t* q,
                         int32_t* idx, const float* sc, float sl2, uint16_t* out, float* part,
                         hipStream_t s, Timing* prof) {
  if (g.kv_bits == 4) {
    if (g.tb == 64) attend_q_group<64, SEL, 4>(g, waves, grid, b, q, idx, sc, sl2, out, part, s, prof);
    else attend_q_group<32, SEL, 4>(g, waves, grid, b, q, idx, sc, sl2, out, part, s, prof);
  } else {
    if (g.tb == 64) attend_q_group<64, SEL, 8>(g, waves, grid, b, q, idx, sc, sl2, out, part, s, prof);
    else attend_q_group<32, SEL, 8>(g, waves, grid, b, q, idx, sc, sl2, out, part, s, prof);
  }
}

// grid (splits of `waves`, Hkv, n); the caller combines the splits
hipError_t launch_attend_q(const Geometry& g, const SeqBatch& b, const void* q, int32_t* idx,
                           const float* scores, int sel_mode, int waves, float sl2, void* out,
                           float* partials, hipStream_t s, Timing* prof) {
  const dim3 grid((g.nsel_max + waves - 1) / waves, g.hkv, b.n);
  const uint16_t* qq = (const uint16_t*)q;
  uint16_t* oo = (uint16_t*)out;
  if (sel_mode == 1) attend_q_sel<1>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
  else if (sel_mode == 2) attend_q_sel<2>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
  else attend_q_sel<0>(g, waves, grid, b, qq, idx, scores, sl2, oo, partials, s, prof);
  return hipGetLastError();
}

hipError_t launch_export_quantized(const Geometry& g, const SeqBatch& b, int T, uint32_t* kw,
                                   void* ks, void* kb, uint32_t* vw, void* vs, void* vb,
                                   hipStream_t s) {
  const dim3 grid((T + 15) / 16, g.hkv, b.n);
  if (g.kv_bits == 4)
    hipLaunchKernelGGL(k_export_q<4>, grid, dim3(256), 0, s, g, b, T, kw, (uint16_t*)ks,
                       (uint16_t*)kb, vw, (uint16_t*)vs, (uint16_t*)vb);
  else
    hipLaunchKernelGGL(k_export_q<8>, grid, dim3(256), 0, s, g, b, T, kw, (uint16_t*)ks,
                       (uint16_t*)kb, vw, (uint16_t*)vs, (uint16_t*)vb);
  return hipGetLastError();
}

}  // namespace bsattn
