/* decode_client.c -- a plain C client of libbsattn (no Python, no torch):
 * reads a decode problem from a file, runs create -> append -> decode ->
 * select through the C ABI on one device and writes the outputs and the
 * selected block indices.  It is what a non-Python binding (the Swift
 * system-library shim) does, and the GPU tests compare its results with the
 * Python binding's and the oracle's.
 *
 * Input:  int32 B, Hq, Hkv, T, Tb, dtype, top_k, sink, recent; float scale;
 *         then K, V [B, Hkv, T, 128] and q [B, Hq, 128] as 16-bit words.
 * Output: out [B, Hq, 128] 16-bit words, then idx [B, Hkv, nsel] int32 from
 *         bsattn_decode, then idx [B, Hkv, nsel] int32 from bsattn_select. */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "bsattn.h"

#define D 128

static int check(int rc, const char* what) {
  if (rc != BSATTN_OK) {
    fprintf(stderr, "%s failed (%d): %s\n", what, rc, bsattn_last_error());
    exit(1);
  }
  return rc;
}

static void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
    exit(1);
  }
}

static void* read_exact(FILE* f, size_t bytes) {
  void* p = malloc(bytes ? bytes : 1);
  if (!p || fread(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "short input (%zu bytes wanted)\n", bytes);
    exit(1);
  }
  return p;
}

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: %s <problem.bin> <result.bin>\n", argv[0]);
    return 2;
  }
  FILE* in = fopen(argv[1], "rb");
  if (!in) {
    perror(argv[1]);
    return 1;
  }
  int32_t h[9];
  float scale;
  if (fread(h, sizeof(int32_t), 9, in) != 9 || fread(&scale, sizeof(float), 1, in) != 1) {
    fprintf(stderr, "short header\n");
    return 1;
  }
  const int32_t B = h[0], Hq = h[1], Hkv = h[2], T = h[3];
  const size_t kv_bytes = (size_t)B * Hkv * T * D * 2, q_bytes = (size_t)B * Hq * D * 2;
  void* hk = read_exact(in, kv_bytes);
  void* hv = read_exact(in, kv_bytes);
  void* hq = read_exact(in, q_bytes);
  fclose(in);

  bsattn_desc desc = {0};
  desc.max_seqs = B;
  desc.num_q_heads = Hq;
  desc.num_kv_heads = Hkv;
  desc.head_dim = D;
  desc.block_size = h[4];
  desc.dtype = h[5];
  desc.kv_bits = 0;
  desc.group_size = 64;
  desc.top_k = h[6];
  desc.sink_blocks = h[7];
  desc.recent_blocks = h[8];
  desc.max_blocks_per_seq = (T + h[4] - 1) / h[4] + 2;
  desc.num_pages = 0;
  desc.device = 0;
  bsattn_cache* cache = NULL;
  check(bsattn_cache_create(&desc, &cache), "bsattn_cache_create");
  bsattn_info info;
  check(bsattn_cache_info(cache, &info), "bsattn_cache_info");
  const size_t idx_bytes = (size_t)B * Hkv * info.nsel_max * sizeof(int32_t);

  void *dk, *dv, *dq, *dout;
  int32_t *didx, *dsel;
  hip_check(hipMalloc(&dk, kv_bytes), "hipMalloc k");
  hip_check(hipMalloc(&dv, kv_bytes), "hipMalloc v");
  hip_check(hipMalloc(&dq, q_bytes), "hipMalloc q");
  hip_check(hipMalloc(&dout, q_bytes), "hipMalloc out");
  hip_check(hipMalloc((void**)&didx, idx_bytes), "hipMalloc idx");
  hip_check(hipMalloc((void**)&dsel, idx_bytes), "hipMalloc sel");
  hip_check(hipMemcpy(dk, hk, kv_bytes, hipMemcpyHostToDevice), "copy k");
  hip_check(hipMemcpy(dv, hv, kv_bytes, hipMemcpyHostToDevice), "copy v");
  hip_check(hipMemcpy(dq, hq, q_bytes, hipMemcpyHostToDevice), "copy q");

  /* every sequence gets all T tokens in one call; null stream = default */
  check(bsattn_append(cache, dk, dv, NULL, B, T, NULL), "bsattn_append");
  for (int32_t b = 0; b < B; ++b) {
    int32_t len = -1;
    check(bsattn_seq_len(cache, b, &len), "bsattn_seq_len");
    if (len != T) {
      fprintf(stderr, "sequence %d holds %d tokens, expected %d\n", b, len, T);
      return 1;
    }
  }
  check(bsattn_decode(cache, dq, NULL, B, scale, dout, didx, NULL), "bsattn_decode");
  check(bsattn_select(cache, dq, NULL, B, dsel, NULL), "bsattn_select");
  hip_check(hipDeviceSynchronize(), "synchronize");

  void* hout = malloc(q_bytes);
  int32_t* hidx = (int32_t*)malloc(idx_bytes);
  int32_t* hsel = (int32_t*)malloc(idx_bytes);
  hip_check(hipMemcpy(hout, dout, q_bytes, hipMemcpyDeviceToHost), "copy out");
  hip_check(hipMemcpy(hidx, didx, idx_bytes, hipMemcpyDeviceToHost), "copy idx");
  hip_check(hipMemcpy(hsel, dsel, idx_bytes, hipMemcpyDeviceToHost), "copy sel");
  FILE* o = fopen(argv[2], "wb");
  if (!o || fwrite(hout, 1, q_bytes, o) != q_bytes || fwrite(hidx, 1, idx_bytes, o) != idx_bytes ||
      fwrite(hsel, 1, idx_bytes, o) != idx_bytes) {
    fprintf(stderr, "cannot write %s\n", argv[2]);
    return 1;
  }
  fclose(o);

  check(bsattn_cache_destroy(cache), "bsattn_cache_destroy");
  hip_check(hipFree(dk), "free");
  hip_check(hipFree(dv), "free");
  hip_check(hipFree(dq), "free");
  hip_check(hipFree(dout), "free");
  hip_check(hipFree(didx), "free");
  hip_check(hipFree(dsel), "free");
  free(hk);
  free(hv);
  free(hq);
  free(hout);
  free(hidx);
  free(hsel);
  printf("ok: B=%d Hq=%d Hkv=%d T=%d nsel=%d\n", B, Hq, Hkv, T, info.nsel_max);
  return 0;
}
