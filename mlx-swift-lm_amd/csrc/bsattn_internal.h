// bsattn_internal.h -- shared between the kernels (bsattn_kernels.hip) and
// the cache manager / C ABI (bsattn_capi.cpp).  Plain structs passed by
// value as kernel arguments; no device code here.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace bsattn {

constexpr int kHeadDim = 128;
constexpr int kMaxBatch = 64;   // sequences per launch (host splits larger calls)
constexpr int kMaxQueries = 16; // query tokens per sequence in one multi-token decode
constexpr int kMaxPatch = 240;  // metadata words patched per launch
#ifndef BSATTN_WAVES
#define BSATTN_WAVES 4
#endif
constexpr int kWaves = BSATTN_WAVES;  // waves per attention workgroup (one block each)
// The wide attention workgroup, one per CU: a call whose selected blocks
// fill every CU with one such workgroup (8 sequences x 8 kv heads x 34
// blocks = 4 splits of 9 waves = 256 workgroups) reads them with no CU
// holding more waves than another, where 4-wave workgroups (576) put 3 on
// some CUs and 2 on the rest.
constexpr int kWavesWide = 9;
constexpr int kMaxSplits = 512;       // attention splits per (sequence, kv head)
// device scratch of the no-allocation decode (bsattn_noalloc.hip), per GPU
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
// floats after the last block-score row: the workgroup selection reads a
// thread's candidates as whole vectors, up to 12 x 1024 entries from a row
// start, and the entries past the row are never candidates
constexpr int kScoreSlack = 12 * 1024;

// Static geometry of one cache, copied into every launch.
struct Geometry {
  int32_t hq, hkv, group;     // group = hq / hkv
  int32_t tb;                 // tokens per block
  int32_t dtype;              // 0 f16, 1 bf16
  int32_t kv_bits;            // 0, 4, 8
  int32_t gsize;              // affine group size
  int32_t top_k, ns, nr, nsel_max, nsplit;  // nsplit: splits of kWaves (the partial workspace's)
  int32_t cus;                // compute units of the device
  int32_t mbps;               // block-table width
  int32_t sstride;            // block-score row stride (mbps rounded up to 64)
  int32_t bt_off;             // offset of the block table inside meta
  int32_t cap_off;            // offset of the per-sequence capacities (tokens of held pages)
  int64_t slab_bytes;         // bytes of one (page, kv head) slab
  // byte offsets inside a slab: K tile (or K codes), V tile (or V codes),
  // per-token scales / biases (quantized caches only)
  int64_t k_off, v_off, sb_off;
  uint8_t* pool;              // [num_pages][hkv] slabs
  uint16_t* summ;             // [max_seqs][hkv][mbps][D], by logical block
  int32_t* meta;              // [max_seqs] lengths, [max_seqs][mbps] pages, [max_seqs] capacities
};

// A launch's batch entries: entry i is a query of sequence ids[i] that sees
// its first len[i] tokens (-1: all of them; a multi-token decode has one
// entry per query token, each seeing the tokens up to its own position);
// its q and output rows start at element qoff[i] (from the launch's q / out
// pointers), heads qhs elements apart.
struct SeqBatch {
  int32_t n;
  int32_t qhs;
  int32_t ids[kMaxBatch];
  int32_t len[kMaxBatch];
  int32_t qoff[kMaxBatch];
};

struct AppendBatch {
  int32_t n, L;
  int32_t seq[kMaxBatch];
  int32_t old_len[kMaxBatch];
};

struct SummaryBatch {
  int32_t n;
  int32_t seq[kMaxBatch];
  int32_t first[kMaxBatch];
  int32_t count[kMaxBatch];
};

struct PatchBatch {
  int32_t n;
  int32_t idx[kMaxPatch];
  int32_t val[kMaxPatch];
};

// page of the block that receives entry i's new token (launch_append_decode)
struct StepPages {
  int32_t page[kMaxBatch];
};

// Opt-in per-kernel profiling: a launcher given a Timing array records the
// start/stop events of slot `kind` around that kernel's dispatch (when the
// slot's events are set) and marks the slot used.
enum ProfKind {
  kProfScore = 0, kProfTopk = 1, kProfAttend = 2, kProfCombine = 3, kProfAppend = 4,
  kProfSummary = 5, kProfPrefill = 6, kProfKinds = 7
};
struct Timing {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};

// address of the no-allocation scratch on `device`, which must be current
// (looked up once per device; bsattn_noalloc.hip)
hipError_t noalloc_scratch(int device, void** out);

// launchers (bsattn_kernels.hip); return hipError_t of the launch
hipError_t launch_patch(const Geometry& g, const PatchBatch& pb, hipStream_t s);
// fuse_summary (one token per sequence): blocks completed by the append get
// their summary from the append kernel itself (no launch_summary needed)
hipError_t launch_append(const Geometry& g, const AppendBatch& ab, const void* k,
                         const void* v, bool fuse_summary, hipStream_t s, Timing* prof);
// quantized caches (bsattn_quant.hip): append from fp16 (quantize on append)
// or from the MLX layout; block summaries of dequantized keys; attention
// one token per listed sequence at its device-side length, then the lengths
// advanced (no host bookkeeping: capturable in a HIP graph)
hipError_t launch_append_step(const Geometry& g, const AppendBatch& ab, const void* k, const void* v,
                              hipStream_t s, Timing* prof);
hipError_t launch_append_q16(const Geometry& g, const AppendBatch& ab, const void* k,
                             const void* v, hipStream_t s, Timing* prof);
hipError_t launch_append_quantized(const Geometry& g, const AppendBatch& ab,
                                   const uint32_t* kw, const void* ks, const void* kb,
                                   const uint32_t* vw, const void* vs, const void* vb,
                                   hipStream_t s, Timing* prof);
hipError_t launch_summary_q(const Geometry& g, const SummaryBatch& sb, int max_count,
                            hipStream_t s, Timing* prof);
hipError_t launch_attend_q(const Geometry& g, const SeqBatch& b, const void* q, int32_t* idx,
                           const float* scores, int sel_mode, int waves, float sl2, void* out,
                           float* partials, hipStream_t s, Timing* prof);
hipError_t launch_summary(const Geometry& g, const SummaryBatch& sb, int max_count,
                          hipStream_t s, Timing* prof);
// candidate blocks (neither sink nor recent) of a sequence of `len` tokens
int candidates(const Geometry& g, int len);
// scoring + top-K for a batch whose largest candidate count is max_nc;
// err: bound and floor workspace of 2 * mfma_err_stride(g) floats per
// (sequence, kv head)
hipError_t launch_select(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                         float* err, int32_t* idx, int max_nc, hipStream_t s, Timing* prof);
int mfma_err_stride(const Geometry& g);
// block-wide selection (bsattn_select.hip); scores_ready: exact scores are
// in `scores`, else (group >= 8) MFMA scores with the band rescored exactly
hipError_t launch_select_large(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                               float* err, int max_nc, int32_t* idx, hipStream_t s, Timing* prof,
                               bool scores_ready);
// Waves per attention workgroup (kWaves or kWavesWide) for one call over
// nseq sequences, from the geometry and nseq alone.  Every launch of a call
// takes the same count, and calls that must agree bit for bit (decode and
// select + attend, append + decode and the one-call step, a multi-token
// decode and its single-token decodes) pass the same nseq, so their splits,
// and the order their partials merge in, are the same.
int attend_waves(const Geometry& g, int nseq);
hipError_t launch_attend(const Geometry& g, const SeqBatch& b, const void* q,
                         const int32_t* idx, int waves, float scale, void* out, float* partials,
                         hipStream_t s, Timing* prof);
// decode = scoring + attention with the top-K selection done inside the
// attention kernel; valid while every sequence has at most
// fused_select_limit(top_k) candidate blocks.  idx_out may be null.
int fused_select_limit(int top_k);
hipError_t launch_decode(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                         int32_t* idx_out, int max_nc, int waves, float scale, void* out,
                         float* partials, hipStream_t s, Timing* prof);
hipError_t launch_decode_attend(const Geometry& g, const SeqBatch& b, const void* q, float* scores,
                                int32_t* idx_out, int max_nc, int waves, float scale, void* out,
                                float* partials, hipStream_t s, Timing* prof);
// one decode step of a 16-bit cache with one new token per entry (b.len =
// the lengths after it): fused (requires fused_decode_ok): one launch of the
// fused decode kernel that also applies the patches pb and the appends (k / v
// [n, Hkv, 1, D] into the pages sp), plus the combine when it splits;
// otherwise the patches, the appends and the scoring in one launch, then the
// selection + attention (+ combine) launches of launch_decode (requires
// max_nc <= fused_select_limit(top_k)).  Every cache has recent
// >= 1, so the block an append completes is forced, never scored.
hipError_t launch_append_decode(const Geometry& g, const SeqBatch& b, const StepPages& sp,
                                const PatchBatch& pb, const void* k, const void* v, const void* q,
                                float* scores, int32_t* idx_out, int max_nc, bool fused, int waves,
                                float scale, void* out, float* partials, hipStream_t s, Timing* prof);
// split combine of nsplit partials per (entry, q head) into out
hipError_t launch_combine(const Geometry& g, const SeqBatch& b, const float* partials, int nsplit,
                          void* out, hipStream_t s, Timing* prof);
// fused decode (bsattn_decode.hip): scoring, selection, gather + attention
// (+ combine) for 16-bit caches with GQA groups up to 4; fused_decode_ok
// tells whether the launches of a call over nseq sequences (its splits are
// planned for them, whatever a launch's entry count) with at most max_nc
// candidate blocks per entry fit it.  len_first: each workgroup reads its
// entry's length before the summaries (for ragged batches; otherwise every
// row of the block-table width is read at once).  idx_out may be null.
bool fused_decode_ok(const Geometry& g, int nseq, int max_nc);
// exact (canonical) block scores of every ranked candidate into `scores`
hipError_t launch_score(const Geometry& g, const SeqBatch& b, const void* q, float* scores, int max_nc,
                        hipStream_t s, Timing* prof);

hipError_t launch_fused_decode(const Geometry& g, const SeqBatch& b, int nseq, const void* q,
                               int32_t* idx_out, bool len_first, float scale, void* out, float* partials,
                               hipStream_t s, Timing* prof);
// the same kernel's gather + attention over given indices (used by
// bsattn_attend exactly where decode takes the fused path, so that
// decode == select + attend bit for bit)
hipError_t launch_fused_attend(const Geometry& g, const SeqBatch& b, int nseq, const void* q,
                               const int32_t* idx, float scale, void* out, float* partials, hipStream_t s,
                               Timing* prof);
// one launch per decode step: each entry's new token (k, v: [n][Hkv][128]) is
// stored at position b.len[i] - 1 on page sp.page[i] before the fused decode
// gathers it, the block it fills gets its summary, and the metadata patches
// pb are applied for the launches that follow (requires recent >= 1)
hipError_t launch_fused_append_decode(const Geometry& g, const SeqBatch& b, const StepPages& sp,
                                      const PatchBatch& pb, const void* k, const void* v, const void* q,
                                      int32_t* idx_out, float scale, void* out, float* partials,
                                      hipStream_t s, Timing* prof);
// dense causal attention of the last L tokens of each sequence
hipError_t launch_prefill(const Geometry& g, const SeqBatch& b, int L, const void* q, float scale,
                          void* out, hipStream_t s, Timing* prof);
hipError_t launch_export(const Geometry& g, const SeqBatch& b, int T, void* k_out,
                         void* v_out, hipStream_t s);
hipError_t launch_export_quantized(const Geometry& g, const SeqBatch& b, int T,
                                   uint32_t* kw, void* ks, void* kb, uint32_t* vw,
                                   void* vs, void* vb, hipStream_t s);
hipError_t launch_export_summaries(const Geometry& g, int seq, int nfull, void* out,
                                   hipStream_t s);

}  // namespace bsattn
