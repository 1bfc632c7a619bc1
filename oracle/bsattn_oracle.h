/*
 * bsattn_oracle.h -- CPU oracle for block-sparse decode attention.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path
 * is compared against; nothing in the product library links, loads or calls
 * it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may use it.
 *
 * The reference (TheTom/mlx-swift-lm, Swift over mlx-swift) has no
 * block-sparse path: its decode attention is the dense
 * `attentionWithCacheUpdate` (Libraries/MLXLMCommon/AttentionUtils.swift:37-77)
 * over `KVCacheSimple` (Libraries/MLXLMCommon/KVCache.swift:315-442) or the
 * quantized variant (KVCache.swift:728-889, 1533-1621).  Scoring, top-K,
 * gather and append therefore follow the arithmetic written out below; the
 * dense and quantized-layout semantics follow the cited reference lines.
 *
 * Element storage: fp16 / bf16 values are passed as raw uint16 bit patterns.
 * dtype codes: 0 = fp16, 1 = bf16.
 */
#ifndef BSATTN_ORACLE_H
#define BSATTN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F16 = 0, ORC_BF16 = 1 };

/* ---- numeric formats (round-to-nearest-even) ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f64_to_f16(double x); /* direct double -> fp16 RNE */
uint16_t orc_f64_to_bf16(double x); /* direct double -> bf16 RNE */
void orc_to_f32(const uint16_t* in, int64_t n, int dtype, float* out);
void orc_from_f32(const float* in, int64_t n, int dtype, uint16_t* out);

/* ---- counter-based RNG ---- */
uint64_t orc_splitmix64(uint64_t x);
uint64_t orc_hash3(uint64_t seed, uint64_t stream, uint64_t index);
double orc_normal(uint64_t seed, uint64_t stream, uint64_t index);
/* out[i] = round_dtype(normal(seed, stream, start + i) * row_mult[i / row_len])
 * row_mult may be NULL (all 1). */
void orc_fill_normal(uint64_t seed, uint64_t stream, uint64_t start, int64_t n,
                     int64_t row_len, const double* row_mult, int dtype,
                     uint16_t* out);
/* Choose `count` distinct positions in [0, n) (partial Fisher-Yates keyed by
 * (seed, stream, key)); written to out[0..count) in selection order. */
void orc_choose_positions(uint64_t seed, uint64_t stream, uint64_t key,
                          int32_t n, int32_t count, int32_t* out);
/* Uniform integer in [lo, hi] from hash3(seed, stream, index). */
int64_t orc_uniform_int(uint64_t seed, uint64_t stream, uint64_t index,
                        int64_t lo, int64_t hi);

/* ---- block summary (mean of a full block's keys) ---- */
/* keys [Tb][D] (row stride ld elements); out [D] */
void orc_block_summary(const uint16_t* keys, int64_t ld, int Tb, int D,
                       int dtype, uint16_t* out);
/* summaries of all full blocks of one (sequence, kv-head): keys [T][D] */
int orc_summaries(const uint16_t* keys, int T, int D, int Tb, int dtype,
                  uint16_t* out /* [T/Tb][D] */);

/* ---- MLX affine codec (group along the head dim, LSB-first pack) ---- */
/* fp32 scale and bias of one group of gs values (before their fp16 cast) */
void orc_affine_params(const float* x, int gs, int bits, float* scale_out,
                       float* bias_out);
void orc_quantize_affine(const uint16_t* x_f16, int64_t rows, int D, int bits,
                         int gs, uint32_t* codes, uint16_t* scales,
                         uint16_t* biases);
/* w = fmaf(scale, code, bias) in fp32 */
void orc_dequantize_affine(const uint32_t* codes, const uint16_t* scales,
                           const uint16_t* biases, int64_t rows, int D,
                           int bits, int gs, float* out);
int orc_code_at(const uint32_t* row_codes, int i, int bits);
/* summary of a full block from dequantized keys; out fp16 [D] */
void orc_block_summary_q(const uint32_t* codes, const uint16_t* scales,
                         const uint16_t* biases, int Tb, int D, int bits,
                         int gs, uint16_t* out);
int orc_summaries_q(const uint32_t* codes, const uint16_t* scales,
                    const uint16_t* biases, int T, int D, int Tb, int bits,
                    int gs, uint16_t* out);

/* ---- block scoring ---- */
/* dot product in the canonical order (D/8 chunks of 8 folded left to
 * right, then a pairwise tree over chunks: (c, c^1), then (c, c^2) ...) */
float orc_dot_canonical(const uint16_t* a, const uint16_t* b, int D, int dtype);
/* s[j] = max over g of dot(q[g], summ[j]) (first-greater wins) */
void orc_score_blocks(const uint16_t* q, int G, const uint16_t* summ, int n,
                      int D, int dtype, float* out);

/* ---- top-K selection ---- */
uint32_t orc_score_key(float s);
/* Selects blocks for one (sequence, kv-head) of `len` tokens.  scores[j]
 * is read for candidate blocks only.  Writes ascending block indices into
 * out[0..n_sel) and -1 into out[n_sel .. ns+nr+K).  Returns n_sel. */
int orc_select(const float* scores, int len, int Tb, int ns, int nr, int K,
               int32_t* out);

/* ---- attention over selected blocks (fp64) ---- */
/* q [G][D]; keys/values [T][D] (dtype); idx = selected block ids (-1 entries skipped);
 * out [G][D] in double.  T = tokens in the sequence. */
void orc_attend(const uint16_t* q, int G, const uint16_t* keys,
                const uint16_t* values, int T, int D, int Tb,
                const int32_t* idx, int n_idx, double scale, int dtype,
                double* out);
/* quantized K/V in MLX layout: codes [T][D*bits/32], scales/biases [T][D/gs]
 * fp16.  q is fp16. */
void orc_attend_q(const uint16_t* q, int G, const uint32_t* kc,
                  const uint16_t* ks, const uint16_t* kb, const uint32_t* vc,
                  const uint16_t* vs, const uint16_t* vb, int T, int D, int Tb,
                  int bits, int gs, const int32_t* idx, int n_idx,
                  double scale, double* out);
/* dense decode attention over all T tokens (what attentionWithCacheUpdate
 * computes for L = 1): direct loop, independent of the block machinery. */
void orc_dense(const uint16_t* q, int G, const uint16_t* keys,
               const uint16_t* values, int T, int D, double scale, int dtype,
               double* out);
/* per-block softmax mass of dense attention for one q head: mass[nb] */
void orc_block_mass(const uint16_t* q, const float* keys_f32, int T, int D,
                    int Tb, double scale, double* mass);

/* ---- one (sequence, kv-head) end to end: summary -> score -> select ->
 * attend.  Returns n_sel. ---- */
int orc_decode_head(const uint16_t* q, int G, const uint16_t* keys,
                    const uint16_t* values, int T, int D, int Tb, int ns,
                    int nr, int K, double scale, int dtype, int32_t* idx_out,
                    double* out);

/* ---- one decode layer-step of B sequences x Hkv kv heads, T tokens each,
 * given the block summaries summ [B][Hkv][T/Tb][D]: score -> select ->
 * attend per (sequence, kv head), pairs spread over OpenMP threads.  16-bit
 * caches pass keys / values [B][Hkv][T][D] (dtype); quantized ones (bits 4 /
 * 8, dtype fp16) pass kc / vc [B][Hkv][T][D*bits/32] and ks / kb / vs / vb
 * [B][Hkv][T][D/gs] instead.  idx_out [B][Hkv][ns+nr+K], out [B][Hq][D]. */
int orc_omp_threads(void);
void orc_layer_step(const uint16_t* q, const uint16_t* summ, const uint16_t* keys,
                    const uint16_t* values, const uint32_t* kc, const uint16_t* ks,
                    const uint16_t* kb, const uint32_t* vc, const uint16_t* vs,
                    const uint16_t* vb, int B, int Hq, int Hkv, int T, int D, int Tb,
                    int bits, int gs, int ns, int nr, int K, double scale, int dtype,
                    int32_t* idx_out, double* out);

#ifdef __cplusplus
}
#endif
#endif
