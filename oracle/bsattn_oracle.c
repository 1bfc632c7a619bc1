/*
 * bsattn_oracle.c -- CPU oracle for block-sparse decode attention.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Built with
 * -ffp-contract=off so every fp32 operation below rounds exactly once, in the
 * order written; the HIP kernels reproduce the same order where bit-exactness
 * is required (block summaries, block scores, hence selected indices).
 *
 * Reference semantics followed:
 *  - dense decode attention: attentionWithCacheUpdate
 *    (Libraries/MLXLMCommon/AttentionUtils.swift:37-77) -> softmax(q k^T * scale) v
 *    with GQA head h attending kv head h / (Hq/Hkv)
 *    (Libraries/MLXLMCommon/KVCache.swift:1547-1555 reshapes [B,Hkv,G,L,D]);
 *  - cache layout [B, Hkv, T, D], appended at `offset`
 *    (KVCache.swift:328-371);
 *  - affine quantized storage: codes packed in uint32 along the head dim,
 *    scales/biases per group of `groupSize` (KVCache.swift:776-889), value
 *    w = scale * q + bias (KVCache.swift:1569-1613 via quantizedMM).
 * Block summary / scoring / top-K / paged gather have no reference function;
 * their arithmetic is stated at each function.
 */
#include "bsattn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* numeric formats                                                     */
/* ------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t a = x & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
  if (a >= 0x47800000u) return (uint16_t)(sign | 0x7C00u); /* >= 2^16: inf */
  uint32_t e = a >> 23;
  if (e < 113) { /* |x| < 2^-14: fp16 subnormal (or zero) */
    if (e == 0) return (uint16_t)sign; /* fp32 subnormal: far below 2^-24 */
    uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126 - e; /* >= 14 */
    if (shift > 24) return (uint16_t)sign;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = ((e - 112) << 10) | ((a >> 13) & 0x3FFu);
  uint32_t rem = a & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 0) {
    /* zero / subnormal: m * 2^-24, exact in fp32 */
    float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
  return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t r = x + 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* double -> fp16 with a single rounding: split off the exactly
 * representable fp16 neighbours and compare. */
static uint16_t f64_to_16(double x, int dtype) {
  if (isnan(x)) return dtype == ORC_F16 ? 0x7E00 : 0x7FC0;
  /* overflow threshold = largest finite + half an ulp (ties go to inf) */
  double lim = dtype == ORC_F16 ? 65520.0 : 0x1.FFp+127;
  if (fabs(x) >= lim) return (uint16_t)((x < 0 ? 0x8000 : 0) | (dtype == ORC_F16 ? 0x7C00 : 0x7F80));
  if (fabs(x) > (dtype == ORC_F16 ? 65504.0 : 0x1.FEp+127))
    return (uint16_t)((x < 0 ? 0x8000 : 0) | (dtype == ORC_F16 ? 0x7BFF : 0x7F7F));
  float f = (float)x; /* may double-round; fix up below */
  uint16_t h = dtype == ORC_F16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f);
  /* candidates h-1, h, h+1 (same sign direction); choose nearest to x,
   * ties to even */
  double best_err = -1.0;
  uint16_t best = h;
  for (int d = -1; d <= 1; d++) {
    uint16_t c = (uint16_t)(h + d);
    double v = dtype == ORC_F16 ? (double)orc_f16_to_f32(c) : (double)orc_bf16_to_f32(c);
    if (isnan(v)) continue;
    if ((c & 0x8000) != (h & 0x8000) && v != 0.0) continue;
    double err = fabs(v - x);
    if (best_err < 0 || err < best_err || (err == best_err && !(c & 1))) {
      best_err = err;
      best = c;
    }
  }
  return best;
}

uint16_t orc_f64_to_f16(double x) { return f64_to_16(x, ORC_F16); }
uint16_t orc_f64_to_bf16(double x) { return f64_to_16(x, ORC_BF16); }

static float to_f32(uint16_t h, int dtype) {
  return dtype == ORC_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}
static uint16_t from_f32(float f, int dtype) {
  return dtype == ORC_F16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f);
}

void orc_to_f32(const uint16_t* in, int64_t n, int dtype, float* out) {
  for (int64_t i = 0; i < n; i++) out[i] = to_f32(in[i], dtype);
}
void orc_from_f32(const float* in, int64_t n, int dtype, uint16_t* out) {
  for (int64_t i = 0; i < n; i++) out[i] = from_f32(in[i], dtype);
}

/* ------------------------------------------------------------------ */
/* counter-based RNG: splitmix64 finaliser chained over (seed, stream, */
/* index); Box-Muller in double                                        */
/* ------------------------------------------------------------------ */

uint64_t orc_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t orc_hash3(uint64_t seed, uint64_t stream, uint64_t index) {
  return orc_splitmix64(orc_splitmix64(orc_splitmix64(seed) + stream) + index);
}

double orc_normal(uint64_t seed, uint64_t stream, uint64_t index) {
  uint64_t p = index >> 1;
  uint64_t a = orc_hash3(seed, stream, 2 * p);
  uint64_t b = orc_hash3(seed, stream, 2 * p + 1);
  double u1 = (double)((a >> 11) + 1) * 0x1.0p-53; /* (0, 1] */
  double u2 = (double)(b >> 11) * 0x1.0p-53;       /* [0, 1) */
  double r = sqrt(-2.0 * log(u1));
  double t = 6.283185307179586476925286766559 * u2;
  return (index & 1) ? r * sin(t) : r * cos(t);
}

void orc_fill_normal(uint64_t seed, uint64_t stream, uint64_t start, int64_t n,
                     int64_t row_len, const double* row_mult, int dtype,
                     uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) {
    double v = orc_normal(seed, stream, start + (uint64_t)i);
    if (row_mult) v *= row_mult[i / row_len];
    out[i] = f64_to_16(v, dtype);
  }
}

void orc_choose_positions(uint64_t seed, uint64_t stream, uint64_t key,
                          int32_t n, int32_t count, int32_t* out) {
  int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
  for (int32_t i = 0; i < n; i++) perm[i] = i;
  for (int32_t i = 0; i < count && i < n; i++) {
    uint64_t h = orc_hash3(seed, stream, (key << 32) | (uint64_t)i);
    int32_t j = i + (int32_t)(h % (uint64_t)(n - i));
    int32_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
    out[i] = perm[i];
  }
  free(perm);
}

int64_t orc_uniform_int(uint64_t seed, uint64_t stream, uint64_t index,
                        int64_t lo, int64_t hi) {
  uint64_t span = (uint64_t)(hi - lo) + 1u;
  return lo + (int64_t)(orc_hash3(seed, stream, index) % span);
}

/* ------------------------------------------------------------------ */
/* block summary                                                       */
/*   summary[d] = round_dtype( (sum_{t=0..Tb-1} k[t][d]) * (1/Tb) )    */
/*   the sum is an fp32 left fold starting from k[0][d]; 1/Tb is a     */
/*   power of two so the scaling is exact (outside underflow).         */
/* ------------------------------------------------------------------ */

void orc_block_summary(const uint16_t* keys, int64_t ld, int Tb, int D,
                       int dtype, uint16_t* out) {
  float inv = 1.0f / (float)Tb;
  for (int d = 0; d < D; d++) {
    float acc = to_f32(keys[d], dtype);
    for (int t = 1; t < Tb; t++) acc = acc + to_f32(keys[(int64_t)t * ld + d], dtype);
    out[d] = from_f32(acc * inv, dtype);
  }
}

int orc_summaries(const uint16_t* keys, int T, int D, int Tb, int dtype,
                  uint16_t* out) {
  int nfull = T / Tb;
  for (int j = 0; j < nfull; j++)
    orc_block_summary(keys + (int64_t)j * Tb * D, D, Tb, D, dtype, out + (int64_t)j * D);
  return nfull;
}

/* ------------------------------------------------------------------ */
/* MLX affine codec                                                    */
/*   The reference quantizes with mlx-swift's quantized(_:groupSize:   */
/*   bits:) (KVCache.swift:416-417 in toQuantized, :856-857 in         */
/*   updateQuantized).  That lives in the un-vendored dependency       */
/*   mlx-swift 0.31.x (Package.swift:39) -> mlx; restated here is its  */
/*   published affine rule (mlx ops `affine_quantize`, CPU backend     */
/*   `quantize`), all in fp32, per group of gs elements along D:       */
/*     mn, mx  = min / max of the group                                */
/*     scale   = max((mx - mn) / (2^bits - 1), 1e-7)                   */
/*     side    = |mn| > |mx|;  scale = side ? scale : -scale           */
/*     edge    = side ? mn : mx            (the larger-magnitude end)  */
/*     q0      = rint(edge / scale)                                    */
/*     q0 != 0: scale = edge / q0, bias = edge;  q0 == 0: bias = 0     */
/*     code    = clamp(rint((x - bias) / scale), 0, 2^bits - 1)        */
/*   with the fp32 scale and bias; they are stored rounded (RNE) to    */
/*   fp16.  rint rounds half to even.  The edge therefore maps to a    */
/*   code exactly (0 for mx, 2^bits - 1 ... for mn), and a group that  */
/*   straddles 0 has 0 = bias + scale * (-q0) in exact arithmetic.     */
/*   Element i of a row lives in word i / (32/bits), bit               */
/*   bits * (i % (32/bits)), least significant first.                  */
/*   dequant: w = fmaf(scale, code, bias) in fp32 (MLX's w = s*q + b). */
/* ------------------------------------------------------------------ */

int orc_code_at(const uint32_t* row_codes, int i, int bits) {
  int per = 32 / bits;
  return (int)((row_codes[i / per] >> (bits * (i % per))) & ((1u << bits) - 1u));
}

void orc_affine_params(const float* x, int gs, int bits, float* scale_out,
                       float* bias_out) {
  const float nbins = (float)((1 << bits) - 1);
  const float eps = (float)1e-7;
  float mn = INFINITY, mx = -INFINITY;
  for (int i = 0; i < gs; i++) {
    mx = mx < x[i] ? x[i] : mx; /* std::max(mx, x) */
    mn = x[i] < mn ? x[i] : mn; /* std::min(mn, x) */
  }
  int side = fabsf(mn) > fabsf(mx);
  float scale = (mx - mn) / nbins;
  scale = scale < eps ? eps : scale;
  scale = side ? scale : -scale;
  float edge = side ? mn : mx;
  float q0 = rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  *scale_out = scale;
  *bias_out = bias;
}

void orc_quantize_affine(const uint16_t* x, int64_t rows, int D, int bits,
                         int gs, uint32_t* codes, uint16_t* scales,
                         uint16_t* biases) {
  int per = 32 / bits;
  int words = D / per;
  int ng = D / gs;
  float nbins = (float)((1 << bits) - 1);
  float xf[256];
  if (gs > 256 || D % gs != 0 || gs % per != 0) abort();
  for (int64_t r = 0; r < rows; r++) {
    const uint16_t* xr = x + r * D;
    uint32_t* cr = codes + r * words;
    memset(cr, 0, sizeof(uint32_t) * (size_t)words);
    for (int g = 0; g < ng; g++) {
      for (int i = 0; i < gs; i++) xf[i] = orc_f16_to_f32(xr[g * gs + i]);
      float sf, bf;
      orc_affine_params(xf, gs, bits, &sf, &bf);
      scales[r * ng + g] = orc_f32_to_f16(sf);
      biases[r * ng + g] = orc_f32_to_f16(bf);
      for (int i = 0; i < gs; i++) {
        int e = g * gs + i;
        float q = rintf((xf[i] - bf) / sf);
        q = q < 0.0f ? 0.0f : q; /* std::max(q, 0) */
        q = q > nbins ? nbins : q;
        cr[e / per] |= ((uint32_t)q) << (bits * (e % per));
      }
    }
  }
}

void orc_dequantize_affine(const uint32_t* codes, const uint16_t* scales,
                           const uint16_t* biases, int64_t rows, int D,
                           int bits, int gs, float* out) {
  int words = D * bits / 32;
  int ng = D / gs;
  for (int64_t r = 0; r < rows; r++)
    for (int i = 0; i < D; i++) {
      float s = orc_f16_to_f32(scales[r * ng + i / gs]);
      float b = orc_f16_to_f32(biases[r * ng + i / gs]);
      out[r * D + i] = fmaf(s, (float)orc_code_at(codes + r * words, i, bits), b);
    }
}

void orc_block_summary_q(const uint32_t* codes, const uint16_t* scales,
                         const uint16_t* biases, int Tb, int D, int bits,
                         int gs, uint16_t* out) {
  int words = D * bits / 32;
  int ng = D / gs;
  float inv = 1.0f / (float)Tb;
  for (int d = 0; d < D; d++) {
    float acc = 0.0f;
    for (int t = 0; t < Tb; t++) {
      float s = orc_f16_to_f32(scales[t * ng + d / gs]);
      float b = orc_f16_to_f32(biases[t * ng + d / gs]);
      float w = fmaf(s, (float)orc_code_at(codes + (int64_t)t * words, d, bits), b);
      acc = (t == 0) ? w : acc + w;
    }
    out[d] = orc_f32_to_f16(acc * inv);
  }
}

int orc_summaries_q(const uint32_t* codes, const uint16_t* scales,
                    const uint16_t* biases, int T, int D, int Tb, int bits,
                    int gs, uint16_t* out) {
  int words = D * bits / 32, ng = D / gs, nfull = T / Tb;
  for (int j = 0; j < nfull; j++)
    orc_block_summary_q(codes + (int64_t)j * Tb * words,
                        scales + (int64_t)j * Tb * ng, biases + (int64_t)j * Tb * ng,
                        Tb, D, bits, gs, out + (int64_t)j * D);
  return nfull;
}

/* ------------------------------------------------------------------ */
/* block scoring                                                       */
/*   dot(a, b): chunk c (c = 0..D/8-1) covers dims 8c..8c+7;           */
/*     p_c = fma(a7, b7, ... fma(a2, b2, fma(a1, b1, a0*b0)))  (fp32,  */
/*     each step one rounding of the exact a*b + acc).  A product of   */
/*     two 16-bit values is exact in fp32 unless it leaves fp32's range */
/*     (bf16 only), so elsewhere this is the unfused chain too;          */
/*   then a pairwise tree: p_c <- p_c + p_{c^1}, then + p_{c^2}, ...   */
/*   with the lower chunk on the left (fp32 addition is commutative,   */
/*   so every lane of an xor-butterfly holds the same bits).           */
/*   score[j] = max_g dot(q_g, summary_j), scanning g upward and        */
/*   replacing only on strictly greater.                               */
/* ------------------------------------------------------------------ */

float orc_dot_canonical(const uint16_t* a, const uint16_t* b, int D, int dtype) {
  float p[64];
  int nc = D / 8;
  for (int c = 0; c < nc; c++) {
    float acc = to_f32(a[8 * c], dtype) * to_f32(b[8 * c], dtype);
    for (int j = 1; j < 8; j++)
      acc = fmaf(to_f32(a[8 * c + j], dtype), to_f32(b[8 * c + j], dtype), acc);
    p[c] = acc;
  }
  for (int stride = 1; stride < nc; stride <<= 1)
    for (int c = 0; c < nc; c += 2 * stride) p[c] = p[c] + p[c + stride];
  return p[0];
}

void orc_score_blocks(const uint16_t* q, int G, const uint16_t* summ, int n,
                      int D, int dtype, float* out) {
  for (int j = 0; j < n; j++) {
    float best = orc_dot_canonical(q, summ + (int64_t)j * D, D, dtype);
    for (int g = 1; g < G; g++) {
      float s = orc_dot_canonical(q + (int64_t)g * D, summ + (int64_t)j * D, D, dtype);
      if (s > best) best = s;
    }
    out[j] = best;
  }
}

/* ------------------------------------------------------------------ */
/* top-K selection                                                     */
/*   key(s): NaN -> 0 (lowest); -0 -> +0; otherwise the IEEE bits made */
/*   monotone (negative: ~bits, non-negative: bits | 0x80000000).      */
/*   Blocks: nb = ceil(len/Tb); forced = [0, min(ns,nb)) and           */
/*   [max(0, nb-nr), nb); candidates = [ns, nb-nr) (all full blocks).  */
/*   If there are <= K candidates all are taken, else the K largest by */
/*   (key desc, index asc).  Output = forced U taken, ascending.       */
/* ------------------------------------------------------------------ */

uint32_t orc_score_key(float s) {
  if (isnan(s)) return 0u;
  if (s == 0.0f) s = 0.0f;
  uint32_t b = f2u(s);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef struct { uint32_t key; int32_t idx; } kv_t;

static int cmp_kv(const void* x, const void* y) {
  const kv_t* a = (const kv_t*)x;
  const kv_t* b = (const kv_t*)y;
  if (a->key != b->key) return a->key > b->key ? -1 : 1;
  return a->idx < b->idx ? -1 : (a->idx > b->idx ? 1 : 0);
}

int orc_select(const float* scores, int len, int Tb, int ns, int nr, int K,
               int32_t* out) {
  int nsel_max = ns + nr + K;
  for (int i = 0; i < nsel_max; i++) out[i] = -1;
  if (len <= 0) return 0;
  int nb = (len + Tb - 1) / Tb;
  char* take = (char*)calloc((size_t)nb, 1);
  for (int j = 0; j < ns && j < nb; j++) take[j] = 1;
  for (int j = nb - nr; j < nb; j++)
    if (j >= 0) take[j] = 1;
  int c0 = ns, c1 = nb - nr;
  int nc = c1 - c0;
  if (nc > 0) {
    if (nc <= K) {
      for (int j = c0; j < c1; j++) take[j] = 1;
    } else {
      kv_t* kv = (kv_t*)malloc(sizeof(kv_t) * (size_t)nc);
      for (int j = c0; j < c1; j++) {
        kv[j - c0].key = orc_score_key(scores[j]);
        kv[j - c0].idx = j;
      }
      qsort(kv, (size_t)nc, sizeof(kv_t), cmp_kv);
      for (int i = 0; i < K; i++) take[kv[i].idx] = 1;
      free(kv);
    }
  }
  int n = 0;
  for (int j = 0; j < nb; j++)
    if (take[j]) out[n++] = j;
  free(take);
  return n;
}

/* ------------------------------------------------------------------ */
/* attention (fp64): s_t = scale * q.k_t, p = softmax(s), o = sum p v  */
/* over the tokens of the selected blocks (block j covers tokens       */
/* [j*Tb, min((j+1)*Tb, T))).  An empty selection gives zeros.         */
/* ------------------------------------------------------------------ */

static void attend_rows(const double* qd, int G, const float* kf, const float* vf,
                        const int32_t* tok, int ntok, int D, double scale,
                        double* out) {
  double* s = (double*)malloc(sizeof(double) * (size_t)(ntok > 0 ? ntok : 1));
  for (int g = 0; g < G; g++) {
    double* o = out + (int64_t)g * D;
    for (int d = 0; d < D; d++) o[d] = 0.0;
    if (ntok == 0) continue;
    double m = -INFINITY;
    for (int i = 0; i < ntok; i++) {
      const float* k = kf + (int64_t)tok[i] * D;
      double acc = 0.0;
      for (int d = 0; d < D; d++) acc += qd[(int64_t)g * D + d] * (double)k[d];
      s[i] = acc * scale;
      if (s[i] > m) m = s[i];
    }
    double l = 0.0;
    for (int i = 0; i < ntok; i++) {
      double p = exp(s[i] - m);
      l += p;
      const float* v = vf + (int64_t)tok[i] * D;
      for (int d = 0; d < D; d++) o[d] += p * (double)v[d];
    }
    for (int d = 0; d < D; d++) o[d] /= l;
  }
  free(s);
}

static int gather_tokens(const int32_t* idx, int n_idx, int T, int Tb, int32_t* tok) {
  int n = 0;
  for (int i = 0; i < n_idx; i++) {
    int j = idx[i];
    if (j < 0) continue; /* -1 entries are skipped */
    for (int t = j * Tb; t < (j + 1) * Tb && t < T; t++) tok[n++] = t;
  }
  return n;
}

void orc_attend(const uint16_t* q, int G, const uint16_t* keys,
                const uint16_t* values, int T, int D, int Tb,
                const int32_t* idx, int n_idx, double scale, int dtype,
                double* out) {
  int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_idx * Tb + 1));
  int ntok = gather_tokens(idx, n_idx, T, Tb, tok);
  double* qd = (double*)malloc(sizeof(double) * (size_t)G * D);
  for (int64_t i = 0; i < (int64_t)G * D; i++) qd[i] = to_f32(q[i], dtype);
  /* convert only the gathered rows */
  float* kf = (float*)malloc(sizeof(float) * (size_t)(ntok + 1) * D);
  float* vf = (float*)malloc(sizeof(float) * (size_t)(ntok + 1) * D);
  int32_t* loc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(ntok + 1));
  for (int i = 0; i < ntok; i++) {
    for (int d = 0; d < D; d++) {
      kf[(int64_t)i * D + d] = to_f32(keys[(int64_t)tok[i] * D + d], dtype);
      vf[(int64_t)i * D + d] = to_f32(values[(int64_t)tok[i] * D + d], dtype);
    }
    loc[i] = i;
  }
  attend_rows(qd, G, kf, vf, loc, ntok, D, scale, out);
  free(tok); free(qd); free(kf); free(vf); free(loc);
}

void orc_attend_q(const uint16_t* q, int G, const uint32_t* kc,
                  const uint16_t* ks, const uint16_t* kb, const uint32_t* vc,
                  const uint16_t* vs, const uint16_t* vb, int T, int D, int Tb,
                  int bits, int gs, const int32_t* idx, int n_idx,
                  double scale, double* out) {
  int words = D * bits / 32, ng = D / gs;
  int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_idx * Tb + 1));
  int ntok = gather_tokens(idx, n_idx, T, Tb, tok);
  double* qd = (double*)malloc(sizeof(double) * (size_t)G * D);
  for (int64_t i = 0; i < (int64_t)G * D; i++) qd[i] = orc_f16_to_f32(q[i]);
  float* kf = (float*)malloc(sizeof(float) * (size_t)(ntok + 1) * D);
  float* vf = (float*)malloc(sizeof(float) * (size_t)(ntok + 1) * D);
  int32_t* loc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(ntok + 1));
  for (int i = 0; i < ntok; i++) {
    int64_t t = tok[i];
    orc_dequantize_affine(kc + t * words, ks + t * ng, kb + t * ng, 1, D, bits, gs,
                          kf + (int64_t)i * D);
    orc_dequantize_affine(vc + t * words, vs + t * ng, vb + t * ng, 1, D, bits, gs,
                          vf + (int64_t)i * D);
    loc[i] = i;
  }
  attend_rows(qd, G, kf, vf, loc, ntok, D, scale, out);
  free(tok); free(qd); free(kf); free(vf); free(loc);
}

void orc_dense(const uint16_t* q, int G, const uint16_t* keys,
               const uint16_t* values, int T, int D, double scale, int dtype,
               double* out) {
  for (int g = 0; g < G; g++) {
    double* o = out + (int64_t)g * D;
    for (int d = 0; d < D; d++) o[d] = 0.0;
    if (T == 0) continue;
    double m = -INFINITY;
    double* s = (double*)malloc(sizeof(double) * (size_t)T);
    for (int t = 0; t < T; t++) {
      double acc = 0.0;
      for (int d = 0; d < D; d++)
        acc += (double)to_f32(q[(int64_t)g * D + d], dtype) *
               (double)to_f32(keys[(int64_t)t * D + d], dtype);
      s[t] = acc * scale;
      if (s[t] > m) m = s[t];
    }
    double l = 0.0;
    for (int t = 0; t < T; t++) {
      double p = exp(s[t] - m);
      l += p;
      for (int d = 0; d < D; d++) o[d] += p * (double)to_f32(values[(int64_t)t * D + d], dtype);
    }
    for (int d = 0; d < D; d++) o[d] /= l;
    free(s);
  }
}

void orc_block_mass(const uint16_t* q, const float* keys_f32, int T, int D,
                    int Tb, double scale, double* mass) {
  int nb = (T + Tb - 1) / Tb;
  double* s = (double*)malloc(sizeof(double) * (size_t)T);
  double m = -INFINITY;
  for (int t = 0; t < T; t++) {
    double acc = 0.0;
    for (int d = 0; d < D; d++) acc += (double)orc_f16_to_f32(q[d]) * (double)keys_f32[(int64_t)t * D + d];
    s[t] = acc * scale;
    if (s[t] > m) m = s[t];
  }
  double l = 0.0;
  for (int j = 0; j < nb; j++) mass[j] = 0.0;
  for (int t = 0; t < T; t++) {
    double p = exp(s[t] - m);
    l += p;
    mass[t / Tb] += p;
  }
  for (int j = 0; j < nb; j++) mass[j] /= l;
  free(s);
}

/* ------------------------------------------------------------------ */

int orc_decode_head(const uint16_t* q, int G, const uint16_t* keys,
                    const uint16_t* values, int T, int D, int Tb, int ns,
                    int nr, int K, double scale, int dtype, int32_t* idx_out,
                    double* out) {
  int nb = (T + Tb - 1) / Tb;
  uint16_t* summ = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(nb + 1) * D);
  float* sc = (float*)malloc(sizeof(float) * (size_t)(nb + 1));
  int nfull = orc_summaries(keys, T, D, Tb, dtype, summ);
  orc_score_blocks(q, G, summ, nfull, D, dtype, sc);
  int n = orc_select(sc, T, Tb, ns, nr, K, idx_out);
  orc_attend(q, G, keys, values, T, D, Tb, idx_out, n, scale, dtype, out);
  free(summ);
  free(sc);
  return n;
}

/* ------------------------------------------------------------------ */
/* one decode layer-step of every (sequence, kv head), given the block  */
/* summaries: score -> select -> attend, the (b, h) pairs spread over   */
/* OpenMP threads (each pair is independent).  The CPU baseline; the    */
/* per-pair arithmetic is the functions above.                          */
/* ------------------------------------------------------------------ */

int orc_omp_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_layer_step(const uint16_t* q, const uint16_t* summ, const uint16_t* keys,
                    const uint16_t* values, const uint32_t* kc, const uint16_t* ks,
                    const uint16_t* kb, const uint32_t* vc, const uint16_t* vs,
                    const uint16_t* vb, int B, int Hq, int Hkv, int T, int D, int Tb,
                    int bits, int gs, int ns, int nr, int K, double scale, int dtype,
                    int32_t* idx_out, double* out) {
  const int G = Hq / Hkv, nfull = T / Tb, nsel = ns + nr + K;
  const int words = bits ? D * bits / 32 : 0, ng = bits ? D / gs : 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (int p = 0; p < B * Hkv; p++) {
    const int b = p / Hkv, h = p % Hkv;
    const uint16_t* qq = q + ((int64_t)b * Hq + (int64_t)h * G) * D;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(nfull + 1));
    orc_score_blocks(qq, G, summ + (int64_t)p * nfull * D, nfull, D, bits ? ORC_F16 : dtype, sc);
    int32_t* idx = idx_out + (int64_t)p * nsel;
    int n = orc_select(sc, T, Tb, ns, nr, K, idx);
    double* o = out + ((int64_t)b * Hq + (int64_t)h * G) * D;
    if (bits) {
      const int64_t t0 = (int64_t)p * T;
      orc_attend_q(qq, G, kc + t0 * words, ks + t0 * ng, kb + t0 * ng, vc + t0 * words,
                   vs + t0 * ng, vb + t0 * ng, T, D, Tb, bits, gs, idx, n, scale, o);
    } else {
      const int64_t t0 = (int64_t)p * T * D;
      orc_attend(qq, G, keys + t0, values + t0, T, D, Tb, idx, n, scale, dtype, o);
    }
    free(sc);
  }
}
