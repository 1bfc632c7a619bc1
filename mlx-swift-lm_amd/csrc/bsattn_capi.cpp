// bsattn_capi.cpp -- the C ABI of include/bsattn.h: page-pool manager,
// per-sequence block tables, argument checking and kernel sequencing.
//
// The host copy of lengths / block tables is authoritative; the device copy
// (`meta`) is brought up to date in stream order by small patch launches
// whose payload travels in the kernel arguments, so no host staging buffer
// can be overwritten while a copy is still pending.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/bsattn.h"
#include "bsattn_internal.h"

using namespace bsattn;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) noexcept {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  try {
    g_err = buf;
  } catch (...) {
    g_err.clear();  // no memory for the message: the status code still says what failed
  }
  return code;
}

// Handler of every entry point's function-try-block: no C++ exception
// crosses the ABI.  Host state is only changed after the allocations a call
// needs have succeeded, so a failed call leaves the cache as it was.
int on_exception() noexcept {
  try {
    throw;
  } catch (const std::bad_alloc&) {
    return fail(BSATTN_ERR_NOMEM, "host memory allocation failed");
  } catch (const std::length_error&) {
    return fail(BSATTN_ERR_NOMEM, "host container size limit exceeded");
  } catch (const std::exception& e) {
    return fail(BSATTN_ERR_INTERNAL, "internal error: %s", e.what());
  } catch (...) {
    return fail(BSATTN_ERR_INTERNAL, "internal error: unknown exception");
  }
}

int hip_fail(hipError_t e, const char* what) {
  return fail(BSATTN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(call, what)              \
  do {                                   \
    hipError_t e_ = (call);              \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

}  // namespace

struct bsattn_cache {
  bsattn_desc d{};
  Geometry geo{};
  int64_t num_pages = 0;
  size_t pool_bytes = 0, summ_bytes = 0, meta_words = 0;
  // per-launch workspaces, rows = batch entries of one launch
  float* scores = nullptr;    // [rows][hkv][sstride] + kScoreSlack
  int32_t* idx_ws = nullptr;  // [rows][hkv][nsel_max]
  float* partials = nullptr;  // [rows][hq][nsplit][D + 2]
  float* err_ws = nullptr;    // [rows][hkv][2][mfma_err_stride]: MFMA score bounds, chunk floors
  std::vector<int32_t> len;
  // set by bsattn_append_step: the device-side lengths may be ahead of `len`
  // until bsattn_sync
  bool stale = false;
  std::vector<std::vector<int32_t>> pages;
  std::vector<int32_t> free_pages;  // stack; back() is handed out next
  // opt-in per-kernel timing (bsattn_profile_*)
  bool profiling = false;
  std::vector<hipEvent_t> event_pool;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[kProfKinds];
  double prof_ms[kProfKinds] = {};
  int64_t prof_count[kProfKinds] = {};
};

namespace {

struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int validate_desc(const bsattn_desc& d) {
  if (d.max_seqs < 1) return fail(BSATTN_ERR_INVALID, "max_seqs must be >= 1 (got %d)", d.max_seqs);
  if (d.num_kv_heads < 1 || d.num_q_heads < 1 || d.num_q_heads % d.num_kv_heads != 0)
    return fail(BSATTN_ERR_INVALID, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                d.num_q_heads, d.num_kv_heads);
  const int G = d.num_q_heads / d.num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16)
    return fail(BSATTN_ERR_INVALID, "GQA group %d unsupported (1, 2, 4, 8 or 16)", G);
  if (16 % d.num_kv_heads != 0)
    return fail(BSATTN_ERR_INVALID, "num_kv_heads %d unsupported (must divide 16)", d.num_kv_heads);
  if (d.head_dim != kHeadDim) return fail(BSATTN_ERR_INVALID, "head_dim %d unsupported (128)", d.head_dim);
  if (d.block_size != 32 && d.block_size != 64)
    return fail(BSATTN_ERR_INVALID, "block_size %d unsupported (32 or 64)", d.block_size);
  if (d.dtype != BSATTN_F16 && d.dtype != BSATTN_BF16)
    return fail(BSATTN_ERR_INVALID, "dtype %d unknown", d.dtype);
  if (d.kv_bits != 0) {
    if (d.kv_bits != 4 && d.kv_bits != 8)
      return fail(BSATTN_ERR_INVALID, "kv_bits %d unsupported (0, 4 or 8)", d.kv_bits);
    if (d.dtype != BSATTN_F16)
      return fail(BSATTN_ERR_INVALID, "quantized caches take fp16 queries, keys and values");
    if (d.group_size != 64)
      return fail(BSATTN_ERR_INVALID, "group_size %d unsupported (64)", d.group_size);
  }
  if (d.top_k < 0 || d.sink_blocks < 0) return fail(BSATTN_ERR_INVALID, "top_k and sink_blocks must be >= 0");
  if (d.recent_blocks < 1) return fail(BSATTN_ERR_INVALID, "recent_blocks must be >= 1 (the partial block is never scored)");
  if (d.max_blocks_per_seq < 1 || d.max_blocks_per_seq > 12288)
    return fail(BSATTN_ERR_INVALID, "max_blocks_per_seq %d out of range [1, 12288]", d.max_blocks_per_seq);
  const int64_t nsel = (int64_t)d.top_k + d.sink_blocks + d.recent_blocks;
  if (nsel > (int64_t)kMaxSplits * kWaves)
    return fail(BSATTN_ERR_INVALID, "sink + recent + top_k = %lld exceeds %d", (long long)nsel, kMaxSplits * kWaves);
  if (d.num_pages < 0) return fail(BSATTN_ERR_INVALID, "num_pages must be >= 0");
  for (int r : d.reserved)
    if (r != 0) return fail(BSATTN_ERR_INVALID, "reserved fields must be 0");
  return BSATTN_OK;
}

// Seq list -> vector (validated, distinct)
int seq_list(const bsattn_cache* c, const int32_t* ids, int32_t n, std::vector<int32_t>& out) {
  if (n < 1) return fail(BSATTN_ERR_INVALID, "n_seqs must be >= 1 (got %d)", n);
  if (n > c->d.max_seqs) return fail(BSATTN_ERR_RANGE, "n_seqs %d exceeds max_seqs %d", n, c->d.max_seqs);
  out.resize(n);
  std::vector<char> seen(c->d.max_seqs, 0);
  for (int i = 0; i < n; ++i) {
    const int s = ids ? ids[i] : i;
    if (s < 0 || s >= c->d.max_seqs) return fail(BSATTN_ERR_RANGE, "sequence id %d out of range [0, %d)", s, c->d.max_seqs);
    if (seen[s]) return fail(BSATTN_ERR_INVALID, "sequence id %d listed twice", s);
    seen[s] = 1;
    out[i] = s;
  }
  return BSATTN_OK;
}

int flush_patches(bsattn_cache* c, std::vector<std::pair<int32_t, int32_t>>& p, hipStream_t s) {
  for (size_t i = 0; i < p.size(); i += kMaxPatch) {
    PatchBatch pb{};
    pb.n = (int32_t)std::min<size_t>(kMaxPatch, p.size() - i);
    for (int k = 0; k < pb.n; ++k) {
      pb.idx[k] = p[i + k].first;
      pb.val[k] = p[i + k].second;
    }
    HIP_TRY(launch_patch(c->geo, pb, s), "patch launch");
  }
  p.clear();
  return BSATTN_OK;
}

// device-side capacity of a sequence: tokens its pages hold
void cap_patch(const bsattn_cache* c, int seq, std::vector<std::pair<int32_t, int32_t>>& patches) {
  patches.emplace_back(c->geo.cap_off + seq, (int32_t)c->pages[seq].size() * c->d.block_size);
}

int release_pages(bsattn_cache* c, int seq, int keep_blocks,
                  std::vector<std::pair<int32_t, int32_t>>& patches) {
  auto& pg = c->pages[seq];
  while ((int)pg.size() > keep_blocks) {
    c->free_pages.push_back(pg.back());
    pg.pop_back();
  }
  cap_patch(c, seq, patches);
  return BSATTN_OK;
}

// Reserve pages for new lengths; on failure nothing changes.  A sequence may
// already hold more pages than its new length needs (bsattn_reserve took them
// ahead): it needs none, and its surplus is not counted against the others.
int reserve_pages(bsattn_cache* c, const std::vector<int32_t>& seqs, int L,
                  std::vector<std::pair<int32_t, int32_t>>& patches) {
  const int tb = c->d.block_size;
  int64_t need = 0;
  for (int s : seqs) {
    const int64_t newlen = (int64_t)c->len[s] + L;
    if (newlen > (int64_t)c->d.max_blocks_per_seq * tb)
      return fail(BSATTN_ERR_RANGE, "sequence %d would hold %lld tokens > max_blocks_per_seq * block_size = %d",
                  s, (long long)newlen, c->d.max_blocks_per_seq * tb);
    need += std::max<int64_t>(0, (newlen + tb - 1) / tb - (int64_t)c->pages[s].size());
  }
  if (need > (int64_t)c->free_pages.size())
    return fail(BSATTN_ERR_NO_PAGES, "page pool exhausted: need %lld pages, %zu free", (long long)need,
                c->free_pages.size());
  // every allocation first (may throw), then the bookkeeping (cannot)
  patches.reserve(patches.size() + (size_t)need + seqs.size());
  for (int s : seqs) c->pages[s].reserve((c->len[s] + L + tb - 1) / tb);
  for (int s : seqs) {
    const int newlen = c->len[s] + L;
    const int nblk = (newlen + tb - 1) / tb;
    auto& pg = c->pages[s];
    while ((int)pg.size() < nblk) {
      const int32_t p = c->free_pages.back();
      c->free_pages.pop_back();
      patches.emplace_back(c->geo.bt_off + s * c->d.max_blocks_per_seq + (int)pg.size(), p);
      pg.push_back(p);
    }
    cap_patch(c, s, patches);
  }
  return BSATTN_OK;
}

// Profiling slots for one C-ABI call: null unless profiling is on and the
// stream is not being captured into a graph.
Timing* prof_slots(bsattn_cache* c, hipStream_t s, Timing* tm) {
  if (!c->profiling) return nullptr;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
  for (int k = 0; k < kProfKinds; ++k) {
    hipEvent_t ev[2];
    for (auto& e : ev) {
      if (!c->event_pool.empty()) {
        e = c->event_pool.back();
        c->event_pool.pop_back();
      } else if (hipEventCreate(&e) != hipSuccess) {
        e = nullptr;
      }
    }
    tm[k].start = ev[0];
    tm[k].stop = ev[1];
    tm[k].used = false;
  }
  return tm;
}

void prof_collect(bsattn_cache* c, Timing* tm) {
  if (!tm) return;
  for (int k = 0; k < kProfKinds; ++k) {
    if (tm[k].used && tm[k].start && tm[k].stop) {
      c->pending[k].emplace_back(tm[k].start, tm[k].stop);
    } else {
      if (tm[k].start) c->event_pool.push_back(tm[k].start);
      if (tm[k].stop) c->event_pool.push_back(tm[k].stop);
    }
  }
}

int prof_drain(bsattn_cache* c) {
  for (int k = 0; k < kProfKinds; ++k) {
    for (auto& pr : c->pending[k]) {
      float ms = 0.f;
      hipError_t e = hipEventSynchronize(pr.second);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, pr.first, pr.second);
      if (e != hipSuccess) return hip_fail(e, "profile events");
      c->prof_ms[k] += ms;
      c->prof_count[k] += 1;
      c->event_pool.push_back(pr.first);
      c->event_pool.push_back(pr.second);
    }
    c->pending[k].clear();
  }
  return BSATTN_OK;
}

void prof_release(bsattn_cache* c) {
  for (int k = 0; k < kProfKinds; ++k) {
    for (auto& pr : c->pending[k]) {
      c->event_pool.push_back(pr.first);
      c->event_pool.push_back(pr.second);
    }
    c->pending[k].clear();
  }
  for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
  c->event_pool.clear();
}

}  // namespace

extern "C" {

int32_t bsattn_version(void) { return BSATTN_VERSION; }

const char* bsattn_last_error(void) { return g_err.c_str(); }

int bsattn_cache_create(const bsattn_desc* desc, bsattn_cache** out) try {
  if (!desc || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  *out = nullptr;
  int rc = validate_desc(*desc);
  if (rc) return rc;
  DeviceGuard dg(desc->device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", desc->device);
  bsattn_cache* c = new (std::nothrow) bsattn_cache();
  if (!c) return fail(BSATTN_ERR_NOMEM, "host allocation failed");
  c->d = *desc;
  const bsattn_desc& d = c->d;
  c->num_pages = d.num_pages ? d.num_pages : (int64_t)d.max_seqs * d.max_blocks_per_seq;
  Geometry& g = c->geo;
  g.hq = d.num_q_heads;
  g.hkv = d.num_kv_heads;
  g.group = d.num_q_heads / d.num_kv_heads;
  g.tb = d.block_size;
  g.dtype = d.dtype;
  g.kv_bits = d.kv_bits;
  g.gsize = d.group_size;
  g.top_k = d.top_k;
  g.ns = d.sink_blocks;
  g.nr = d.recent_blocks;
  g.nsel_max = d.top_k + d.sink_blocks + d.recent_blocks;
  g.nsplit = (g.nsel_max + kWaves - 1) / kWaves;
  {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, desc->device) != hipSuccess) cus = 0;
    g.cus = cus;  // 0: attention workgroups keep kWaves waves
  }
  g.mbps = d.max_blocks_per_seq;
  g.sstride = (g.mbps + 63) & ~63;
  g.bt_off = d.max_seqs;
  g.cap_off = d.max_seqs * (1 + d.max_blocks_per_seq);
  // slab: K tile then V tile (16-bit elements, or b-bit codes), then for
  // quantized caches 16 B of scales / biases per token
  g.k_off = 0;
  g.v_off = (int64_t)d.block_size * kHeadDim * (d.kv_bits ? d.kv_bits : 16) / 8;
  g.sb_off = 2 * g.v_off;
  g.slab_bytes = g.sb_off + (d.kv_bits ? (int64_t)d.block_size * 16 : 0);
  c->pool_bytes = (size_t)c->num_pages * g.hkv * g.slab_bytes;
  c->summ_bytes = (size_t)d.max_seqs * g.hkv * g.mbps * kHeadDim * 2;
  c->meta_words = (size_t)d.max_seqs * (2 + d.max_blocks_per_seq);
  // host bookkeeping before any device allocation, so a failure here leaks nothing
  try {
    c->len.assign(d.max_seqs, 0);
    c->pages.assign(d.max_seqs, {});
    c->free_pages.resize(c->num_pages);
  } catch (...) {
    delete c;
    throw;
  }
  for (int64_t i = 0; i < c->num_pages; ++i) c->free_pages[i] = (int32_t)(c->num_pages - 1 - i);
  auto cleanup = [&](int code) {
    (void)hipFree(g.pool);
    (void)hipFree(g.summ);
    (void)hipFree(g.meta);
    (void)hipFree(c->scores);
    (void)hipFree(c->idx_ws);
    (void)hipFree(c->partials);
    (void)hipFree(c->err_ws);
    delete c;
    return code;
  };
  hipError_t e;
  if ((e = hipMalloc((void**)&g.pool, c->pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(pool)"));
  if ((e = hipMalloc((void**)&g.summ, c->summ_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(summaries)"));
  if ((e = hipMalloc((void**)&g.meta, c->meta_words * 4)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(meta)"));
  // per-launch workspaces: one row per batch entry of a launch
  const size_t rows = (size_t)std::min(kMaxBatch, d.max_seqs * kMaxQueries);
  if ((e = hipMalloc((void**)&c->scores, (rows * g.hkv * g.sstride + kScoreSlack) * 4)) != hipSuccess)
    return cleanup(hip_fail(e, "hipMalloc(scores)"));
  if ((e = hipMalloc((void**)&c->idx_ws, rows * g.hkv * g.nsel_max * 4)) != hipSuccess)
    return cleanup(hip_fail(e, "hipMalloc(indices)"));
  if ((e = hipMalloc((void**)&c->partials, rows * g.hq * g.nsplit * (kHeadDim + 2) * 4)) != hipSuccess)
    return cleanup(hip_fail(e, "hipMalloc(partials)"));
  if ((e = hipMalloc((void**)&c->err_ws, rows * g.hkv * 2 * mfma_err_stride(g) * 4)) != hipSuccess)
    return cleanup(hip_fail(e, "hipMalloc(bounds)"));
  // zeroed pages: never-written token slots hold finite values
  if ((e = hipMemset(g.pool, 0, c->pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(pool)"));
  if ((e = hipMemset(g.summ, 0, c->summ_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(summaries)"));
  if ((e = hipMemset(g.meta, 0, c->meta_words * 4)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(meta)"));
  if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(hip_fail(e, "hipDeviceSynchronize"));
  *out = c;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_cache_destroy(bsattn_cache* c) try {
  if (!c) return BSATTN_OK;
  DeviceGuard dg(c->d.device);
  (void)hipDeviceSynchronize();
  prof_release(c);
  (void)hipFree(c->geo.pool);
  (void)hipFree(c->geo.summ);
  (void)hipFree(c->geo.meta);
  (void)hipFree(c->scores);
  (void)hipFree(c->idx_ws);
  (void)hipFree(c->partials);
  (void)hipFree(c->err_ws);
  delete c;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_cache_info(const bsattn_cache* c, bsattn_info* out) try {
  if (!c || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  out->nsel_max = c->geo.nsel_max;
  out->num_splits = c->geo.nsplit;
  out->page_bytes = (int64_t)c->geo.hkv * (c->geo.slab_bytes + kHeadDim * 2);
  out->pool_bytes = (int64_t)(c->pool_bytes + c->summ_bytes + c->meta_words * 4);
  out->free_pages = (int64_t)c->free_pages.size();
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

// Calls that need the exact token counts refuse while device-side appends
// (bsattn_append_step) may have advanced them past the host's view.
static int check_synced(const bsattn_cache* c) {
  if (c->stale)
    return fail(BSATTN_ERR_INVALID, "device-side lengths may be ahead of the host's view "
                                    "(bsattn_append_step): call bsattn_sync first");
  return BSATTN_OK;
}

int bsattn_shuffle_free_pages(bsattn_cache* c, uint64_t seed) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  // Fisher-Yates over the free list with index hash splitmix64 chained over
  // (seed, stream 5, i); the stack's back is handed out first
  auto mix = [](uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  auto& f = c->free_pages;
  const size_t n = f.size();
  for (size_t i = 0; i + 1 < n; ++i) {
    const uint64_t hsh = mix(mix(mix(seed) + 5u) + (uint64_t)i);
    std::swap(f[n - 1 - i], f[n - 1 - i - (size_t)(hsh % (uint64_t)(n - i))]);
  }
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_seq_pages(const bsattn_cache* c, int32_t seq, int32_t* out, int32_t cap, int32_t* n_out) try {
  if (!c || !n_out || (cap > 0 && !out)) return fail(BSATTN_ERR_INVALID, "null argument");
  if (seq < 0 || seq >= c->d.max_seqs) return fail(BSATTN_ERR_RANGE, "sequence id %d out of range", seq);
  const auto& pg = c->pages[seq];
  *n_out = (int32_t)pg.size();
  if ((int64_t)pg.size() > (int64_t)cap)
    return fail(BSATTN_ERR_RANGE, "sequence %d holds %zu pages, buffer takes %d", seq, pg.size(), cap);
  std::copy(pg.begin(), pg.end(), out);
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_seq_len(const bsattn_cache* c, int32_t seq, int32_t* out_len) try {
  if (!c || !out_len) return fail(BSATTN_ERR_INVALID, "null argument");
  if (seq < 0 || seq >= c->d.max_seqs) return fail(BSATTN_ERR_RANGE, "sequence id %d out of range", seq);
  int rc = check_synced(c);
  if (rc) return rc;
  *out_len = c->len[seq];
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_reserve(bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs, int32_t n_tokens,
                   void* stream) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  if (n_tokens < 0) return fail(BSATTN_ERR_INVALID, "n_tokens must be >= 0");
  std::vector<int32_t> seqs;
  int rc = check_synced(c);
  if (rc) return rc;
  rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  std::vector<std::pair<int32_t, int32_t>> patches;
  rc = reserve_pages(c, seqs, n_tokens, patches);
  if (rc) return rc;
  return flush_patches(c, patches, (hipStream_t)stream);
} catch (...) {
  return on_exception();
}

int bsattn_append_step(bsattn_cache* c, const void* k, const void* v, const int32_t* seq_ids,
                       int32_t n_seqs, void* stream) try {
  if (!c || !k || !v) return fail(BSATTN_ERR_INVALID, "null argument");
  if (c->d.kv_bits != 0)
    return fail(BSATTN_ERR_INVALID, "device-side appends are provided for 16-bit caches");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  hipStream_t s = (hipStream_t)stream;
  const size_t row = (size_t)c->geo.hkv * kHeadDim;  // elements per sequence
  for (int i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
    AppendBatch ab{};
    ab.n = std::min(kMaxBatch, n_seqs - i0);
    ab.L = 1;
    for (int i = 0; i < ab.n; ++i) ab.seq[i] = seqs[i0 + i];
    Timing tm[kProfKinds];
    Timing* prof = prof_slots(c, s, tm);
    hipError_t e = launch_append_step(c->geo, ab, (const uint16_t*)k + i0 * row,
                                      (const uint16_t*)v + i0 * row, s, prof);
    prof_collect(c, prof);
    if (e != hipSuccess) return hip_fail(e, "append step launch");
  }
  c->stale = true;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_sync(bsattn_cache* c, void* stream) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  std::vector<int32_t> dev(c->d.max_seqs);
  HIP_TRY(hipMemcpy(dev.data(), c->geo.meta, dev.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy(lengths)");
  c->len = dev;
  c->stale = false;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

// Shared append flow: reserve pages, patch lengths / block tables, then per
// batch of sequences launch `kernels(batch, first row)` (token writes) and the
// summaries of the blocks that become full.
extern "C++" template <typename F>
int append_impl(bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs, int32_t n_tokens,
                       hipStream_t s, F kernels) {
  if (n_tokens < 1) return fail(BSATTN_ERR_INVALID, "n_tokens must be >= 1 (got %d)", n_tokens);
  std::vector<int32_t> seqs;
  int rc = check_synced(c);
  if (rc) return rc;
  rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  std::vector<std::pair<int32_t, int32_t>> patches;
  rc = reserve_pages(c, seqs, n_tokens, patches);
  if (rc) return rc;
  const int tb = c->d.block_size;
  for (int s_ : seqs) patches.emplace_back(s_, c->len[s_] + n_tokens);
  rc = flush_patches(c, patches, s);
  if (rc) return rc;
  for (int i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
    AppendBatch ab{};
    SummaryBatch sb{};
    ab.n = std::min(kMaxBatch, n_seqs - i0);
    ab.L = n_tokens;
    int max_count = 0;
    for (int i = 0; i < ab.n; ++i) {
      const int sq = seqs[i0 + i];
      ab.seq[i] = sq;
      ab.old_len[i] = c->len[sq];
      const int first = c->len[sq] / tb;
      const int last = (c->len[sq] + n_tokens) / tb;  // exclusive: full blocks after
      sb.seq[i] = sq;
      sb.first[i] = first;
      sb.count[i] = last - first;
      max_count = std::max(max_count, last - first);
    }
    sb.n = ab.n;
    Timing tm[kProfKinds];
    Timing* prof = prof_slots(c, s, tm);
    // one token into a 16-bit cache: the append kernel writes the summaries
    const bool fused = n_tokens == 1 && c->d.kv_bits == 0;
    hipError_t e = kernels(ab, (size_t)i0, fused, prof);
    if (e == hipSuccess && max_count > 0 && !fused) e = launch_summary(c->geo, sb, max_count, s, prof);
    prof_collect(c, prof);
    if (e != hipSuccess) return hip_fail(e, "append launch");
  }
  for (int s_ : seqs) c->len[s_] += n_tokens;
  return BSATTN_OK;
}

int bsattn_append(bsattn_cache* c, const void* k, const void* v, const int32_t* seq_ids,
                  int32_t n_seqs, int32_t n_tokens, void* stream) try {
  if (!c || !k || !v) return fail(BSATTN_ERR_INVALID, "null argument");
  hipStream_t s = (hipStream_t)stream;
  const size_t row = (size_t)c->geo.hkv * n_tokens * kHeadDim;  // elements per sequence
  const bool quant = c->d.kv_bits != 0;
  return append_impl(c, seq_ids, n_seqs, n_tokens, s, [&](const AppendBatch& ab, size_t i0, bool fused,
                                                           Timing* prof) {
    const uint16_t* kk = (const uint16_t*)k + i0 * row;
    const uint16_t* vv = (const uint16_t*)v + i0 * row;
    return quant ? launch_append_q16(c->geo, ab, kk, vv, s, prof)
                 : launch_append(c->geo, ab, kk, vv, fused, s, prof);
  });
} catch (...) {
  return on_exception();
}

int bsattn_append_quantized(bsattn_cache* c, const uint32_t* k_w, const void* k_s, const void* k_b,
                            const uint32_t* v_w, const void* v_s, const void* v_b,
                            const int32_t* seq_ids, int32_t n_seqs, int32_t n_tokens,
                            void* stream) try {
  if (!c || !k_w || !k_s || !k_b || !v_w || !v_s || !v_b) return fail(BSATTN_ERR_INVALID, "null argument");
  if (c->d.kv_bits == 0) return fail(BSATTN_ERR_INVALID, "not a quantized cache (kv_bits 0): use bsattn_append");
  hipStream_t s = (hipStream_t)stream;
  const size_t rows = (size_t)c->geo.hkv * n_tokens;  // token rows per sequence
  const size_t words = kHeadDim * c->d.kv_bits / 32, groups = kHeadDim / c->d.group_size;
  return append_impl(c, seq_ids, n_seqs, n_tokens, s, [&](const AppendBatch& ab, size_t i0, bool,
                                                           Timing* prof) {
    const size_t wo = i0 * rows * words, go = i0 * rows * groups;
    return launch_append_quantized(c->geo, ab, k_w + wo, (const uint16_t*)k_s + go,
                                   (const uint16_t*)k_b + go, v_w + wo, (const uint16_t*)v_s + go,
                                   (const uint16_t*)v_b + go, s, prof);
  });
} catch (...) {
  return on_exception();
}

// One query of a launch: the sequence, the tokens it sees (-1: all), the
// element offset of its q / out rows.
struct Entry {
  int32_t seq, len;
  int64_t qoff;
};

// Entries of n_query query tokens per listed sequence, q / out laid out
// [n, Hq, n_query, D]: query i of a sequence holding T tokens (the n_query
// new ones included) sees its first T - n_query + 1 + i tokens.
static std::vector<Entry> entries(const bsattn_cache* c, const std::vector<int32_t>& seqs, int n_query) {
  std::vector<Entry> es;
  es.reserve(seqs.size() * n_query);
  const int64_t hq = c->geo.hq;
  for (size_t b = 0; b < seqs.size(); ++b)
    for (int i = 0; i < n_query; ++i)
      es.push_back({seqs[b], n_query == 1 ? -1 : c->len[seqs[b]] - n_query + 1 + i,
                    ((int64_t)b * hq * n_query + i) * kHeadDim});
  return es;
}

// Tokens an entry may see, for sizing launches: its own count, or every
// token its pages hold (the device-side length, which graph-replayed appends
// advance, never exceeds that); the kernels read the actual length.
static int visible(const bsattn_cache* c, const Entry& e) {
  return e.len >= 0 ? e.len : (int)c->pages[e.seq].size() * c->d.block_size;
}

// the launch batch for entries [e0, e0 + n); q / out offsets relative to entry e0
static SeqBatch make_batch(const Entry* es, int e0, int n, int qhs) {
  SeqBatch b{};
  b.n = n;
  b.qhs = qhs;
  for (int i = 0; i < n; ++i) {
    b.ids[i] = es[e0 + i].seq;
    b.len[i] = es[e0 + i].len;
    b.qoff[i] = (int32_t)(es[e0 + i].qoff - es[e0].qoff);
  }
  return b;
}

// Whether the fused decode of entries [e0, e0 + n) should read each entry's
// length before its block summaries: when the rows the entries' held pages
// cover are well below the block-table width, loading every row at once would
// fetch mostly unused summaries.
// (Entries with their own token count carry it in the launch arguments, so
// knowing it first costs nothing.)
static bool len_first(const bsattn_cache* c, const Entry* es, int e0, int n) {
  const int tb = c->d.block_size;
  int64_t held = 0;
  bool given = true;
  for (int i = 0; i < n; ++i) {
    held += (visible(c, es[e0 + i]) + tb - 1) / tb;
    given = given && es[e0 + i].len >= 0;
  }
  return given || 4 * held < 3 * (int64_t)n * c->d.max_blocks_per_seq;
}

// Device workspaces of one launch (rows = the launch's batch entries):
// block scores [rows][hkv][sstride] + kScoreSlack, MFMA score bounds
// and floors [rows][hkv][2][mfma_err_stride], indices [rows][hkv][nsel_max], split
// partials [rows][hq][nsplit][D + 2].
struct Workspace {
  float* scores;
  float* err;
  int32_t* idx;
  float* partials;
};

static Workspace cache_workspace(const bsattn_cache* c) {
  return Workspace{c->scores, c->err_ws, c->idx_ws, c->partials};
}

// Selection, attention or both for the entries, in launches of at most
// kMaxBatch entries: the fused decode kernel where it applies, else scoring
// and selection inside the attention kernel when every entry's candidates
// fit it, else separate selection.  The workspaces are per launch (launches
// on one stream run in order).  nseq: the call's sequences (n / nseq query
// tokens each), from which every launch's splits are planned.  profile:
// time the launches when profiling is on.
enum class Op { Select, Attend, Decode };
static int run_entries(bsattn_cache* c, Op op, const void* q, const Entry* es, int n, int nseq, int qhs,
                       const int32_t* idx_in, int32_t* idx_out, float scale, void* out, hipStream_t s,
                       const Workspace& ws, bool profile = true) {
  const Geometry& g = c->geo;
  const size_t idx_row = (size_t)g.hkv * g.nsel_max;
  const int waves = attend_waves(g, nseq);
  for (int e0 = 0; e0 < n; e0 += kMaxBatch) {
    const SeqBatch b = make_batch(es, e0, std::min(kMaxBatch, n - e0), qhs);
    int max_nc = 0;
    for (int i = 0; i < b.n; ++i) max_nc = std::max(max_nc, candidates(g, visible(c, es[e0 + i])));
    const uint16_t* qq = (const uint16_t*)q + es[e0].qoff;
    uint16_t* oo = out ? (uint16_t*)out + es[e0].qoff : nullptr;
    int32_t* io = idx_out ? idx_out + e0 * idx_row : nullptr;
    Timing tm[kProfKinds];
    Timing* prof = profile ? prof_slots(c, s, tm) : nullptr;
    hipError_t e = hipSuccess;
    if (op == Op::Select) {
      e = launch_select(g, b, qq, ws.scores, ws.err, io, max_nc, s, prof);
    } else if (op == Op::Attend) {
      if (fused_decode_ok(g, nseq, max_nc))
        e = launch_fused_attend(g, b, nseq, qq, idx_in + e0 * idx_row, scale, oo, ws.partials, s, prof);
      else
        e = launch_attend(g, b, qq, idx_in + e0 * idx_row, waves, scale, oo, ws.partials, s, prof);
    } else if (fused_decode_ok(g, nseq, max_nc)) {
      e = launch_fused_decode(g, b, nseq, qq, io, len_first(c, es, e0, b.n), scale, oo, ws.partials, s, prof);
    } else if (max_nc > fused_select_limit(g.top_k)) {
      int32_t* sel = io ? io : ws.idx;
      e = launch_select(g, b, qq, ws.scores, ws.err, sel, max_nc, s, prof);
      if (e == hipSuccess) e = launch_attend(g, b, qq, sel, waves, scale, oo, ws.partials, s, prof);
    } else {
      e = launch_decode(g, b, qq, ws.scores, io, max_nc, waves, scale, oo, ws.partials, s, prof);
    }
    prof_collect(c, prof);
    if (e != hipSuccess) return hip_fail(e, op == Op::Select ? "select launch" : op == Op::Attend ? "attend launch" : "decode launch");
  }
  return BSATTN_OK;
}

int bsattn_select(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                  int32_t* idx_out, void* stream) try {
  if (!c || !q || !idx_out) return fail(BSATTN_ERR_INVALID, "null argument");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const std::vector<Entry> es = entries(c, seqs, 1);
  return run_entries(c, Op::Select, q, es.data(), (int)es.size(), (int)seqs.size(), kHeadDim, nullptr, idx_out,
                     0.0f, nullptr,
                     (hipStream_t)stream, cache_workspace(c));
} catch (...) {
  return on_exception();
}

int bsattn_attend(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                  const int32_t* idx, float scale, void* out, void* stream) try {
  if (!c || !q || !idx || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const std::vector<Entry> es = entries(c, seqs, 1);
  return run_entries(c, Op::Attend, q, es.data(), (int)es.size(), (int)seqs.size(), kHeadDim, idx, nullptr,
                     scale, out,
                     (hipStream_t)stream, cache_workspace(c));
} catch (...) {
  return on_exception();
}

int bsattn_decode(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                  float scale, void* out, int32_t* idx_out, void* stream) try {
  if (!c || !q || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const std::vector<Entry> es = entries(c, seqs, 1);
  return run_entries(c, Op::Decode, q, es.data(), (int)es.size(), (int)seqs.size(), kHeadDim, nullptr, idx_out,
                     scale, out,
                     (hipStream_t)stream, cache_workspace(c));
} catch (...) {
  return on_exception();
}

int bsattn_decode_noalloc(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                          float scale, void* out, int32_t* idx_out, void* stream) try {
  // no device or host allocation on the way: the entries live on the stack,
  // the workspaces in the device's fixed scratch, profiling is not recorded.
  // Like bsattn_decode, the launches are sized from each sequence's held
  // pages and the kernels read the device-side lengths, so the call follows
  // bsattn_append_step without a bsattn_sync (a captured [append_step,
  // decode_noalloc] loop).
  if (!c || !q || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (n_seqs < 1 || n_seqs > kMaxBatch || n_seqs > c->d.max_seqs)
    return fail(BSATTN_ERR_RANGE, "n_seqs %d out of range [1, %d] for the no-allocation decode", n_seqs,
                std::min(kMaxBatch, c->d.max_seqs));
  const Geometry& g = c->geo;
  Entry es[kMaxBatch];
  for (int i = 0; i < n_seqs; ++i) {
    const int sq = seq_ids ? seq_ids[i] : i;
    if (sq < 0 || sq >= c->d.max_seqs)
      return fail(BSATTN_ERR_RANGE, "sequence id %d out of range [0, %d)", sq, c->d.max_seqs);
    for (int j = 0; j < i; ++j)
      if (es[j].seq == sq) return fail(BSATTN_ERR_INVALID, "sequence id %d listed twice", sq);
    es[i] = Entry{sq, -1, (int64_t)i * g.hq * kHeadDim};
  }
  // workspaces of one launch of n_seqs rows, each 256-byte aligned
  const size_t rows = (size_t)n_seqs;
  size_t used = 0;
  auto take = [&used](size_t bytes) {
    const size_t at = used;
    used += (bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t o_sc = take((rows * g.hkv * g.sstride + kScoreSlack) * 4);
  const size_t o_err = take(rows * g.hkv * 2 * mfma_err_stride(g) * 4);
  const size_t o_idx = take(rows * g.hkv * g.nsel_max * 4);
  const size_t o_part = take(rows * g.hq * g.nsplit * (kHeadDim + 2) * 4);
  if (used > kNoAllocScratchBytes)
    return fail(BSATTN_ERR_RANGE,
                "the decode of %d sequences needs %zu bytes of workspace; the no-allocation scratch holds %zu "
                "(decode fewer sequences per call, or use bsattn_decode)",
                n_seqs, used, kNoAllocScratchBytes);
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  void* base = nullptr;
  HIP_TRY(noalloc_scratch(c->d.device, &base), "hipGetSymbolAddress(scratch)");
  char* b = (char*)base;
  const Workspace ws{(float*)(b + o_sc), (float*)(b + o_err), (int32_t*)(b + o_idx), (float*)(b + o_part)};
  return run_entries(c, Op::Decode, q, es, n_seqs, n_seqs, kHeadDim, nullptr, idx_out, scale, out,
                     (hipStream_t)stream, ws, false);
} catch (...) {
  return on_exception();
}

int bsattn_append_decode(bsattn_cache* c, const void* k, const void* v, const void* q,
                         const int32_t* seq_ids, int32_t n_seqs, float scale, void* out,
                         int32_t* idx_out, void* stream) try {
  if (!c || !k || !v || !q || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  const Geometry& g = c->geo;
  const int tb = c->d.block_size;
  int max_nc = 0;
  // (create requires recent_blocks >= 1: the block a token completes is never scored)
  bool one_launch = c->d.kv_bits == 0 && n_seqs <= kMaxBatch;
  for (int sq : seqs) {
    if ((int64_t)c->len[sq] + 1 > (int64_t)c->d.max_blocks_per_seq * tb) one_launch = false;
    else max_nc = std::max(max_nc, candidates(g, c->len[sq] + 1));
  }
  // fused: the append launch, then the fused decode kernel (scoring inside);
  // otherwise append + scoring in one launch, then selection + attention
  const bool fused = one_launch && fused_decode_ok(g, n_seqs, max_nc);
  one_launch = one_launch && (fused || max_nc <= fused_select_limit(g.top_k));
  if (!one_launch) {
    rc = bsattn_append(c, k, v, seq_ids, n_seqs, 1, stream);
    if (rc) return rc;
    return bsattn_decode(c, q, seq_ids, n_seqs, scale, out, idx_out, stream);
  }
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  hipStream_t s = (hipStream_t)stream;
  std::vector<std::pair<int32_t, int32_t>> patches;
  rc = reserve_pages(c, seqs, 1, patches);
  if (rc) return rc;
  for (int sq : seqs) patches.emplace_back(sq, c->len[sq] + 1);
  if (patches.size() > (size_t)kMaxPatch) {  // applied by a launch of their own
    rc = flush_patches(c, patches, s);
    if (rc) return rc;
  }
  PatchBatch pb{};
  pb.n = (int32_t)patches.size();
  for (int i = 0; i < pb.n; ++i) {
    pb.idx[i] = patches[i].first;
    pb.val[i] = patches[i].second;
  }
  SeqBatch b{};
  StepPages sp{};
  b.n = n_seqs;
  b.qhs = kHeadDim;
  for (int i = 0; i < n_seqs; ++i) {
    const int sq = seqs[i];
    b.ids[i] = sq;
    b.len[i] = c->len[sq] + 1;
    b.qoff[i] = (int32_t)((int64_t)i * g.hq * kHeadDim);
    sp.page[i] = c->pages[sq][c->len[sq] / tb];
  }
  Timing tm[kProfKinds];
  Timing* prof = prof_slots(c, s, tm);
  hipError_t e = launch_append_decode(g, b, sp, pb, k, v, q, c->scores, idx_out, max_nc, fused,
                                     attend_waves(g, n_seqs), scale, out, c->partials, s, prof);
  prof_collect(c, prof);
  if (e != hipSuccess) return hip_fail(e, "append-decode launch");
  for (int sq : seqs) c->len[sq] += 1;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_decode_multi(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                        int32_t n_query, float scale, void* out, int32_t* idx_out, void* stream) try {
  if (!c || !q || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (n_query < 1 || n_query > kMaxQueries)
    return fail(BSATTN_ERR_INVALID, "n_query %d out of range [1, %d]", n_query, kMaxQueries);
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  for (int sq : seqs)
    if (c->len[sq] < n_query)
      return fail(BSATTN_ERR_INVALID, "sequence %d holds %d tokens, fewer than its %d queries", sq, c->len[sq],
                  n_query);
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const std::vector<Entry> es = entries(c, seqs, n_query);
  return run_entries(c, Op::Decode, q, es.data(), (int)es.size(), (int)seqs.size(), n_query * kHeadDim, nullptr,
                     idx_out, scale, out, (hipStream_t)stream, cache_workspace(c));
} catch (...) {
  return on_exception();
}

int bsattn_prefill(bsattn_cache* c, const void* q, const int32_t* seq_ids, int32_t n_seqs,
                   int32_t n_query, float scale, void* out, void* stream) try {
  if (!c || !q || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (n_query < 1) return fail(BSATTN_ERR_INVALID, "n_query must be >= 1");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  for (int sq : seqs)
    if (c->len[sq] < n_query)
      return fail(BSATTN_ERR_INVALID, "sequence %d holds %d tokens, fewer than its %d queries", sq, c->len[sq],
                  n_query);
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  hipStream_t s = (hipStream_t)stream;
  // q / out [n, Hq, L, D]: a launch takes whole sequences whose row offsets fit int32
  const int64_t per_seq = (int64_t)c->geo.hq * n_query * kHeadDim;
  const int step = (int)std::max<int64_t>(1, std::min<int64_t>(kMaxBatch, INT32_MAX / per_seq));
  const int n = (int)seqs.size();
  for (int i0 = 0; i0 < n; i0 += step) {
    SeqBatch b{};
    b.n = std::min(step, n - i0);
    b.qhs = n_query * kHeadDim;
    for (int i = 0; i < b.n; ++i) {
      b.ids[i] = seqs[i0 + i];
      b.len[i] = -1;
      b.qoff[i] = (int32_t)(i * per_seq);
    }
    Timing tm[kProfKinds];
    Timing* prof = prof_slots(c, s, tm);
    hipError_t e = launch_prefill(c->geo, b, n_query, (const uint16_t*)q + i0 * per_seq, scale,
                                  (uint16_t*)out + i0 * per_seq, s, prof);
    prof_collect(c, prof);
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
  }
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_trim(bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs, int32_t n_tokens,
                int32_t* trimmed, void* stream) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (n_tokens < 0) return fail(BSATTN_ERR_INVALID, "n_tokens must be >= 0");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  std::vector<std::pair<int32_t, int32_t>> patches;
  patches.reserve(2 * seqs.size());  // the loop below then cannot throw
  for (int i = 0; i < n_seqs; ++i) {
    const int sq = seqs[i];
    const int t = std::min(c->len[sq], n_tokens);
    if (trimmed) trimmed[i] = t;
    c->len[sq] -= t;
    release_pages(c, sq, (c->len[sq] + c->d.block_size - 1) / c->d.block_size, patches);
    patches.emplace_back(sq, c->len[sq]);
  }
  return flush_patches(c, patches, (hipStream_t)stream);
} catch (...) {
  return on_exception();
}

int bsattn_reset(bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs, void* stream) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  std::vector<std::pair<int32_t, int32_t>> patches;
  patches.reserve(2 * seqs.size());  // the loop below then cannot throw
  for (int sq : seqs) {
    c->len[sq] = 0;
    release_pages(c, sq, 0, patches);
    patches.emplace_back(sq, 0);
  }
  return flush_patches(c, patches, (hipStream_t)stream);
} catch (...) {
  return on_exception();
}

int bsattn_copy(const bsattn_cache* src, bsattn_cache** out, void* stream) try {
  if (!src || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(src)) return rs;
  int rc = bsattn_cache_create(&src->d, out);
  if (rc) return rc;
  bsattn_cache* c = *out;
  *out = nullptr;
  try {
    c->len = src->len;
    c->pages = src->pages;
    c->free_pages = src->free_pages;
  } catch (...) {
    bsattn_cache_destroy(c);
    throw;
  }
  DeviceGuard dg(src->d.device);
  if (!dg.ok) {
    bsattn_cache_destroy(c);
    return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", src->d.device);
  }
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if ((e = hipMemcpyAsync(c->geo.pool, src->geo.pool, src->pool_bytes, hipMemcpyDeviceToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(c->geo.summ, src->geo.summ, src->summ_bytes, hipMemcpyDeviceToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(c->geo.meta, src->geo.meta, src->meta_words * 4, hipMemcpyDeviceToDevice, s)) != hipSuccess) {
    bsattn_cache_destroy(c);
    return hip_fail(e, "copy");
  }
  *out = c;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_export(const bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs, void* k_out,
                  void* v_out, void* stream) try {
  if (!c || !k_out || !v_out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (c->d.kv_bits != 0) return fail(BSATTN_ERR_INVALID, "quantized cache: use bsattn_export_quantized");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  const int T = c->len[seqs[0]];
  for (int sq : seqs)
    if (c->len[sq] != T) return fail(BSATTN_ERR_INVALID, "listed sequences hold different token counts");
  if (T == 0) return BSATTN_OK;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const size_t row = (size_t)c->geo.hkv * T * kHeadDim * 2;
  for (int i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
    SeqBatch b{};
    b.n = std::min(kMaxBatch, n_seqs - i0);
    for (int i = 0; i < b.n; ++i) {
      b.ids[i] = seqs[i0 + i];
      b.len[i] = -1;
    }
    HIP_TRY(launch_export(c->geo, b, T, (char*)k_out + i0 * row, (char*)v_out + i0 * row,
                          (hipStream_t)stream),
            "export launch");
  }
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_export_quantized(const bsattn_cache* c, const int32_t* seq_ids, int32_t n_seqs,
                            uint32_t* k_w, void* k_s, void* k_b, uint32_t* v_w, void* v_s,
                            void* v_b, void* stream) try {
  if (!c || !k_w || !k_s || !k_b || !v_w || !v_s || !v_b) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (c->d.kv_bits == 0) return fail(BSATTN_ERR_INVALID, "not a quantized cache (kv_bits 0): use bsattn_export");
  std::vector<int32_t> seqs;
  int rc = seq_list(c, seq_ids, n_seqs, seqs);
  if (rc) return rc;
  const int T = c->len[seqs[0]];
  for (int sq : seqs)
    if (c->len[sq] != T) return fail(BSATTN_ERR_INVALID, "listed sequences hold different token counts");
  if (T == 0) return BSATTN_OK;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  const size_t rows = (size_t)c->geo.hkv * T;
  const size_t words = kHeadDim * c->d.kv_bits / 32, groups = kHeadDim / c->d.group_size;
  for (int i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
    SeqBatch b{};
    b.n = std::min(kMaxBatch, n_seqs - i0);
    for (int i = 0; i < b.n; ++i) {
      b.ids[i] = seqs[i0 + i];
      b.len[i] = -1;
    }
    const size_t wo = (size_t)i0 * rows * words, go = (size_t)i0 * rows * groups;
    HIP_TRY(launch_export_quantized(c->geo, b, T, k_w + wo, (uint16_t*)k_s + go, (uint16_t*)k_b + go,
                                    v_w + wo, (uint16_t*)v_s + go, (uint16_t*)v_b + go,
                                    (hipStream_t)stream),
            "export launch");
  }
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_export_summaries(const bsattn_cache* c, int32_t seq, void* out, void* stream) try {
  if (!c || !out) return fail(BSATTN_ERR_INVALID, "null argument");
  if (int rs = check_synced(c)) return rs;
  if (seq < 0 || seq >= c->d.max_seqs) return fail(BSATTN_ERR_RANGE, "sequence id %d out of range", seq);
  const int nfull = c->len[seq] / c->d.block_size;
  if (nfull == 0) return BSATTN_OK;
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  HIP_TRY(launch_export_summaries(c->geo, seq, nfull, out, (hipStream_t)stream), "export summaries launch");
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_profile_enable(bsattn_cache* c, int32_t enable) try {
  if (!c) return fail(BSATTN_ERR_INVALID, "null argument");
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  int rc = prof_drain(c);
  if (rc) return rc;
  for (int k = 0; k < kProfKinds; ++k) {
    c->prof_ms[k] = 0.0;
    c->prof_count[k] = 0;
  }
  c->profiling = enable != 0;
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

int bsattn_profile_read(bsattn_cache* c, int32_t kernel, double* total_ms, int64_t* launches) try {
  if (!c || !total_ms || !launches) return fail(BSATTN_ERR_INVALID, "null argument");
  if (kernel < 0 || kernel >= kProfKinds) return fail(BSATTN_ERR_INVALID, "unknown kernel id %d", kernel);
  DeviceGuard dg(c->d.device);
  if (!dg.ok) return fail(BSATTN_ERR_HIP, "hipSetDevice(%d) failed", c->d.device);
  int rc = prof_drain(c);
  if (rc) return rc;
  *total_ms = c->prof_ms[kernel];
  *launches = c->prof_count[kernel];
  return BSATTN_OK;
} catch (...) {
  return on_exception();
}

}  // extern "C"
