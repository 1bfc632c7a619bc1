/*
 * bsattn.h -- C ABI of the MI355X (gfx950) block-sparse decode-attention
 * library (libbsattn.so).
 *
 * One `bsattn_cache` is one layer's KV cache for up to `max_seqs`
 * sequences: a paged pool of `block_size`-token pages in HBM, a per-sequence
 * block table, and one mean-pooled summary key per full block and KV head.
 * It stands in for the reference's per-layer `KVCache` object
 * (Libraries/MLXLMCommon/KVCache.swift:38-77) and its decode attention
 * (`attentionWithCacheUpdate`, Libraries/MLXLMCommon/AttentionUtils.swift:37-77).
 *
 * ABI rules
 *  - every call returns an int status: BSATTN_OK (0) or a negative code; the
 *    message of the last failure on the calling thread is bsattn_last_error();
 *    no C++ exception crosses the ABI;
 *  - tensors are caller-owned device pointers, dense, in the reference's
 *    [batch, heads, tokens, head_dim] order; fp16/bf16 data is raw 16-bit;
 *  - work is enqueued on the caller's hipStream_t (`stream`, NULL = the
 *    default stream) and nothing synchronizes the host except where stated;
 *  - a handle is thread-compatible, not thread-safe, and is used with one
 *    stream at a time (the reference guards a cache the same way:
 *    Libraries/MLXLMCommon/ModelContainer.swift:32-33).
 */
#ifndef BSATTN_H
#define BSATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSATTN_VERSION 1

/* status codes */
#define BSATTN_OK 0
#define BSATTN_ERR_INVALID (-1)  /* bad argument / unsupported shape */
#define BSATTN_ERR_HIP (-2)      /* a HIP runtime call failed */
#define BSATTN_ERR_NO_PAGES (-3) /* the page pool is exhausted */
#define BSATTN_ERR_RANGE (-4)    /* sequence id or length out of range */
#define BSATTN_ERR_NOMEM (-5)    /* a host allocation failed; the cache is unchanged */
#define BSATTN_ERR_INTERNAL (-6) /* an unexpected internal failure */

/* element types of q / k / v / output / summaries */
#define BSATTN_F16 0
#define BSATTN_BF16 1

typedef struct bsattn_cache bsattn_cache;

/* Cache geometry.  Mirrors the knobs of QuantizedKVCache
 * (groupSize / bits: KVCache.swift:728-744) plus the block-sparse ones. */
typedef struct bsattn_desc {
  int32_t max_seqs;           /* sequences (batch rows) the cache can hold */
  int32_t num_q_heads;        /* Hq */
  int32_t num_kv_heads;       /* Hkv; Hq % Hkv == 0, Hq / Hkv <= 16 */
  int32_t head_dim;           /* D; 128 */
  int32_t block_size;         /* tokens per block (= page): 32 or 64 */
  int32_t dtype;              /* BSATTN_F16 or BSATTN_BF16 */
  int32_t kv_bits;            /* 0: K/V stored in dtype; 4 or 8: affine (dtype f16) */
  int32_t group_size;         /* affine group along head_dim: 64 */
  int32_t top_k;              /* scored blocks kept per (sequence, kv head) */
  int32_t sink_blocks;        /* leading blocks always kept */
  int32_t recent_blocks;      /* trailing blocks always kept; >= 1 */
  int32_t max_blocks_per_seq; /* block-table width */
  int64_t num_pages;          /* physical pages; 0 = max_seqs * max_blocks_per_seq */
  int32_t device;             /* HIP device ordinal */
  int32_t reserved[3];        /* must be 0 */
} bsattn_desc;

/* Derived sizes, for callers sizing buffers. */
typedef struct bsattn_info {
  int32_t nsel_max;        /* sink + recent + top_k: width of index outputs */
  int32_t num_splits;      /* attention partials per (sequence, q head): the most a call uses */
  int64_t page_bytes;      /* bytes of one page across all kv heads, incl. summaries */
  int64_t pool_bytes;      /* device bytes held by the handle */
  int64_t free_pages;      /* pages not owned by any sequence */
} bsattn_info;

int32_t bsattn_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* bsattn_last_error(void);

/* Creates an empty cache.  Replaces constructing a KVCacheSimple /
 * QuantizedKVCache in LanguageModel.newCache
 * (Libraries/MLXLMCommon/LanguageModel.swift:215-230). */
int bsattn_cache_create(const bsattn_desc* desc, bsattn_cache** out);
int bsattn_cache_destroy(bsattn_cache* cache);
int bsattn_cache_info(const bsattn_cache* cache, bsattn_info* out);

/* Permutes the pages no sequence holds, from a seed (Fisher-Yates keyed by
 * splitmix64 over (seed, stream 5, index)), so that later appends take their
 * pages in a shuffled physical order.  Results never depend on the physical
 * order; this reproduces the scattered layouts a long-running pool reaches.
 * No reference counterpart (the reference's caches are contiguous,
 * KVCache.swift:328-371).  Host only: nothing is enqueued. */
int bsattn_shuffle_free_pages(bsattn_cache* cache, uint64_t seed);

/* Physical pages of sequence `seq`, in logical order (its block table row,
 * reserved pages included), into out[0, cap); *n_out = the count, also when
 * cap is too small (then BSATTN_ERR_RANGE).  Introspection for tests and
 * integrators; no reference counterpart.  Host only. */
int bsattn_seq_pages(const bsattn_cache* cache, int32_t seq, int32_t* out, int32_t cap,
                     int32_t* n_out);

/* Tokens held by sequence `seq` (the reference's `offset`,
 * KVCache.swift:40). */
int bsattn_seq_len(const bsattn_cache* cache, int32_t seq, int32_t* out_len);

/* Appends n_tokens tokens to each listed sequence: k, v are
 * [n_seqs, Hkv, n_tokens, D] in dtype.  Blocks that become full get their
 * summary written.  seq_ids (host, n_seqs distinct ids) may be NULL for
 * rows 0..n_seqs-1.  On a quantized cache the keys/values are quantized on
 * append.  Replaces KVCacheSimple.update(keys:values:)
 * (KVCache.swift:328-371) and QuantizedKVCache.updateQuantized
 * (KVCache.swift:816-889). */
int bsattn_append(bsattn_cache* cache, const void* k, const void* v,
                  const int32_t* seq_ids, int32_t n_seqs, int32_t n_tokens,
                  void* stream);

/* Appends already-quantized tokens in MLX layout: *_w [n, Hkv, L, D*bits/32]
 * uint32, *_s / *_b [n, Hkv, L, D/group_size] fp16.  Same layout as the
 * (wq, scales, biases) tuples of QuantizedKVCache.state
 * (KVCache.swift:906-925). */
int bsattn_append_quantized(bsattn_cache* cache, const uint32_t* k_w,
                            const void* k_s, const void* k_b,
                            const uint32_t* v_w, const void* v_s,
                            const void* v_b, const int32_t* seq_ids,
                            int32_t n_seqs, int32_t n_tokens, void* stream);

/* Selector-index API (no reference counterpart; additive).  Scores every
 * candidate block with max over the GQA group of q . summary, keeps sink and
 * recent blocks and the top_k best (ties -> lower index).  q is
 * [n_seqs, Hq, 1, D]; idx_out (device) is [n_seqs, Hkv, nsel_max] int32:
 * ascending block indices, padded with -1. */
int bsattn_select(bsattn_cache* cache, const void* q, const int32_t* seq_ids,
                  int32_t n_seqs, int32_t* idx_out, void* stream);

/* Attention of q [n_seqs, Hq, 1, D] over the blocks listed in idx
 * ([n_seqs, Hkv, nsel_max], -1 padded; device) -> out [n_seqs, Hq, 1, D]
 * in dtype.  softmax(q k^T * scale) v over the gathered tokens, GQA head h
 * reading kv head h / (Hq/Hkv) (as the dense path of AttentionUtils.swift:68-75
 * and KVCache.swift:1533-1621 computes over all tokens). */
int bsattn_attend(bsattn_cache* cache, const void* q, const int32_t* seq_ids,
                  int32_t n_seqs, const int32_t* idx, float scale, void* out,
                  void* stream);

/* bsattn_select then bsattn_attend.  idx_out may be NULL (library
 * workspace).  The decode branch of attentionWithCacheUpdate
 * (AttentionUtils.swift:68-75) after the cache update. */
int bsattn_decode(bsattn_cache* cache, const void* q, const int32_t* seq_ids,
                  int32_t n_seqs, float scale, void* out, int32_t* idx_out,
                  void* stream);

/* bsattn_decode without any allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it).  No counterpart in the reference.  The same kernels and results, bit
 * for bit, as bsattn_decode; its workspaces (block scores, score bounds,
 * indices, split partials) live in a fixed 16 MiB device scratch that every
 * call on one GPU shares (each GPU holds its own until the process ends),
 * and nothing is allocated on the device or the host.  At most 64
 * sequences per call; a call whose workspaces exceed the scratch fails with
 * BSATTN_ERR_RANGE.  Calls on one GPU that may overlap (other streams, other
 * threads, other caches) race on the scratch: serialize them.  Profiling is
 * not recorded.  Like bsattn_decode it sizes its launches from the held
 * pages and reads the device-side lengths, so it may follow
 * bsattn_append_step without bsattn_sync (e.g. a captured
 * [bsattn_append_step, bsattn_decode_noalloc] step; make one call before
 * capture so that the scratch's address is looked up outside it). */
int bsattn_decode_noalloc(bsattn_cache* cache, const void* q, const int32_t* seq_ids,
                          int32_t n_seqs, float scale, void* out, int32_t* idx_out,
                          void* stream);

/* One decode step of attentionWithCacheUpdate (AttentionUtils.swift:37-77
 * with L = 1: cache.update(keys:values:), KVCache.swift:328-371, then the
 * decode attention, AttentionUtils.swift:68-75) in one call: appends one
 * token per listed sequence (k, v [n_seqs, Hkv, 1, D]) and decodes q
 * [n_seqs, Hq, 1, D] over the caches that now hold it -> out; idx_out as
 * in bsattn_decode.  Same results, bit for bit, as bsattn_append followed
 * by bsattn_decode; on a 16-bit cache whose batch takes the fused decode
 * the whole step is one launch (the append inside the decode kernel),
 * otherwise the append and the block scoring share one launch. */
int bsattn_append_decode(bsattn_cache* cache, const void* k, const void* v,
                         const void* q, const int32_t* seq_ids, int32_t n_seqs,
                         float scale, void* out, int32_t* idx_out, void* stream);

/* Decode of n_query (1..16) query tokens per sequence whose n_query keys /
 * values were appended last: the speculative-verify pass of
 * Evaluate.swift:862-870 (L = numDraft + 1 under a causal mask).  q / out
 * are [n_seqs, Hq, n_query, D]; query i of a sequence holding T tokens
 * attends to its first T - n_query + 1 + i tokens, selecting its own blocks
 * there, i.e. exactly what n_query single-token decodes would compute one
 * after another.  idx_out (may be NULL) is [n_seqs, n_query, Hkv,
 * nsel_max]. */
int bsattn_decode_multi(bsattn_cache* cache, const void* q,
                        const int32_t* seq_ids, int32_t n_seqs,
                        int32_t n_query, float scale, void* out,
                        int32_t* idx_out, void* stream);

/* Dense causal attention of the last n_query tokens of each listed sequence
 * (a prefill chunk whose keys / values were appended): q / out
 * [n_seqs, Hq, n_query, D]; query i of a sequence holding T tokens attends to
 * tokens [0, T - n_query + i], as attentionWithCacheUpdate with L > 1 and
 * the causal mask (AttentionUtils.swift:46-52, BaseKVCache.makeMask,
 * KVCache.swift:160-174) computes over the whole cache (for a quantized
 * cache: quantizedScaledDotProductAttention with the causal mask,
 * KVCache.swift:1533-1621). */
int bsattn_prefill(bsattn_cache* cache, const void* q, const int32_t* seq_ids,
                   int32_t n_seqs, int32_t n_query, float scale, void* out,
                   void* stream);

/* Graph-capturable decode loop.  bsattn_reserve takes the pages for
 * n_tokens more tokens of each listed sequence now; bsattn_append_step then
 * appends one token per listed sequence (k / v [n_seqs, Hkv, 1, D]) at the
 * sequence's device-side length, writes the summary of a block it
 * completes and advances that length, with no host bookkeeping, so a
 * [bsattn_append_step, bsattn_decode] pair can be captured into a HIP graph
 * and replayed once per step (a sequence whose reservation is used up
 * takes no further tokens).  Until bsattn_sync copies the device-side
 * lengths back (synchronizing the stream), calls that need exact token
 * counts fail with BSATTN_ERR_INVALID; bsattn_decode / select / attend size
 * their launches from the held pages and run.  16-bit caches.  (No
 * reference counterpart: the reference's cache update is host-driven,
 * KVCache.swift:328-371.) */
int bsattn_reserve(bsattn_cache* cache, const int32_t* seq_ids,
                   int32_t n_seqs, int32_t n_tokens, void* stream);
int bsattn_append_step(bsattn_cache* cache, const void* k, const void* v,
                       const int32_t* seq_ids, int32_t n_seqs, void* stream);
int bsattn_sync(bsattn_cache* cache, void* stream);

/* Drops the last n_tokens of each listed sequence (clamped to its length);
 * writes the number trimmed per sequence to trimmed (host, may be NULL).
 * KVCacheSimple.trim (KVCache.swift:396-402). */
int bsattn_trim(bsattn_cache* cache, const int32_t* seq_ids, int32_t n_seqs,
                int32_t n_tokens, int32_t* trimmed, void* stream);

/* Empties the listed sequences and returns their pages to the pool. */
int bsattn_reset(bsattn_cache* cache, const int32_t* seq_ids, int32_t n_seqs,
                 void* stream);

/* Deep copy (KVCacheSimple.copy, KVCache.swift:429-437). */
int bsattn_copy(const bsattn_cache* src, bsattn_cache** out, void* stream);

/* Writes the listed sequences' keys and values in the reference layout
 * [n_seqs, Hkv, T, D] (device); all listed sequences must hold T tokens.
 * The `state` getter of KVCacheSimple (KVCache.swift:373-384).  On a
 * quantized cache use bsattn_export_quantized. */
int bsattn_export(const bsattn_cache* cache, const int32_t* seq_ids,
                  int32_t n_seqs, void* k_out, void* v_out, void* stream);

/* Quantized state in MLX layout (see bsattn_append_quantized).
 * QuantizedKVCache.state getter (KVCache.swift:906-925). */
int bsattn_export_quantized(const bsattn_cache* cache, const int32_t* seq_ids,
                            int32_t n_seqs, uint32_t* k_w, void* k_s,
                            void* k_b, uint32_t* v_w, void* v_s, void* v_b,
                            void* stream);

/* Block summaries of one sequence: out [Hkv, T / block_size, D] (device,
 * dtype; fp16 for quantized caches). */
int bsattn_export_summaries(const bsattn_cache* cache, int32_t seq, void* out,
                            void* stream);

/* Opt-in kernel timing (no reference counterpart; the reference times with
 * wall-clock Date deltas, Libraries/MLXLMCommon/Evaluate.swift:1773-1777).
 * While enabled, every eager launch of the handle's kernels carries HIP
 * start/stop events attached to its dispatch (launches captured into a
 * graph are not timed).  bsattn_profile_read waits for the recorded events
 * and returns the summed kernel time and launch count of one kernel kind
 * since profiling was last enabled.  Enabling (or disabling) resets the sums. */
#define BSATTN_KERNEL_SCORE 0   /* block scoring */
#define BSATTN_KERNEL_TOPK 1    /* top-K selection (bsattn_select) */
#define BSATTN_KERNEL_ATTEND 2  /* gather + attention (selection fused in bsattn_decode) */
#define BSATTN_KERNEL_COMBINE 3 /* split combine */
#define BSATTN_KERNEL_APPEND 4  /* token append */
#define BSATTN_KERNEL_SUMMARY 5 /* block summary refresh */
#define BSATTN_KERNEL_PREFILL 6 /* dense causal prefill attention */
int bsattn_profile_enable(bsattn_cache* cache, int32_t enable);
int bsattn_profile_read(bsattn_cache* cache, int32_t kernel, double* total_ms,
                        int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* BSATTN_H */
