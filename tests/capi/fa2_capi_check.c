/*
 * fa2_capi_check.c - a plain C host of the library's C ABI (include/fa2_fwd.h): no Python, no
 * torch in the process. It is what a non-Python caller of the replaced Triton launch
 * (fa2/kernel.py:247-259) does: device buffers from hipMalloc, one fa2_attn_fwd or
 * fa2_attn_fwd_ex call on a stream, errors through the return code and fa2_last_error().
 *
 *   fa2_capi_check run B H_q H_kv N_q N_kv D dtype causal pack block_m block_n splits lse seed out
 *       fills q, k, v with seeded values in [-2, 2) (a 64-bit LCG, rounded to the 16-bit type),
 *       runs one forward and writes a binary file for tests/test_gpu_capi.py: 16 int32 header
 *       words (the arguments, the return code, the split count used), then the 16-bit bits of
 *       q, k, v and out, then (lse = 1) the fp32 log-sum-exp. Exit status 0 when the call
 *       returned FA2_OK.
 *   fa2_capi_check errors
 *       checks that rejected arguments come back as FA2_EINVAL / FA2_EALIGN with a message, and
 *       that the policy queries answer; exit status 0 when they all do.
 *
 * Test infrastructure only: built next to this file by csrc/build.py and run by the tests.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fa2_fwd.h"

#define HIP_OK(x)                                                                  \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(3);                                                                     \
    }                                                                              \
  } while (0)

/* fp32 -> 16-bit bits, round to nearest even; inputs here are normal numbers or zero. */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static uint16_t to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((u >> 23) & 0xffu) - 127 + 15;
  uint32_t mant = u & 0x7fffffu;
  if ((u & 0x7fffffffu) == 0) return (uint16_t)sign;
  if (exp <= 0 || exp >= 31) return (uint16_t)(sign | (exp <= 0 ? 0u : 0x7c00u));
  uint32_t h = ((uint32_t)exp << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;  /* may carry into the exponent */
  return (uint16_t)(sign | h);
}

static uint64_t g_state;
static float next_value(void) {  /* [-2, 2) */
  g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((g_state >> 40) & 0xffffffu) / 16777216.0f * 4.0f - 2.0f;
}

/* Host staging buffers are pinned (hipHostMalloc): the HIP runtime would otherwise lock pageable
 * memory for large copies, and locking memory that already exists is refused on some systems. */
static void* host_alloc(size_t bytes) {
  void* h = NULL;
  HIP_OK(hipHostMalloc(&h, bytes ? bytes : 16, 0));
  return h;
}

static uint16_t* fill(size_t n, int dtype) {
  uint16_t* h = (uint16_t*)host_alloc(n * 2);
  for (size_t i = 0; i < n; ++i) h[i] = dtype ? to_bf16(next_value()) : to_f16(next_value());
  return h;
}

static void* device_alloc(size_t bytes) {
  void* d = NULL;
  HIP_OK(hipMalloc(&d, bytes ? bytes : 16));
  return d;
}

static void* upload(const void* h, size_t bytes) {
  void* d = device_alloc(bytes);
  if (bytes) HIP_OK(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice));
  return d;
}

static int run(int argc, char** argv) {
  if (argc != 17) {
    fprintf(stderr, "run needs 15 arguments\n");
    return 2;
  }
  int32_t a[14];
  for (int i = 0; i < 14; ++i) a[i] = (int32_t)atoi(argv[2 + i]);
  const int32_t B = a[0], hq = a[1], hkv = a[2], nq = a[3], nkv = a[4], d = a[5], dtype = a[6],
                causal = a[7], pack = a[8], block_m = a[9], block_n = a[10], splits_req = a[11],
                want_lse = a[12], seed = a[13];
  const char* path = argv[16];
  g_state = 0x9e3779b97f4a7c15ull ^ (uint64_t)seed;

  const size_t nq_el = (size_t)B * hq * nq * d, nkv_el = (size_t)B * hkv * nkv * d;
  uint16_t* hq_ = fill(nq_el, dtype);
  uint16_t* hk_ = fill(nkv_el, dtype);
  uint16_t* hv_ = fill(nkv_el, dtype);
  void* dq = upload(hq_, nq_el * 2);
  void* dk = upload(hk_, nkv_el * 2);
  void* dv = upload(hv_, nkv_el * 2);
  void* dout = device_alloc(nq_el * 2);
  float* dlse = NULL;
  if (want_lse) dlse = (float*)device_alloc((size_t)B * hq * nq * 4);

  /* contiguous [b, h, n, d] element strides */
  const int64_t sq[4] = {(int64_t)hq * nq * d, (int64_t)nq * d, d, 1};
  const int64_t skv[4] = {(int64_t)hkv * nkv * d, (int64_t)nkv * d, d, 1};
  const float qk_scale = (float)(1.0 / sqrt((double)d) * 1.4426950408889634);  /* fa2/kernel.py:240-244 */

  int32_t splits = splits_req;
  if (splits == 0) {  /* the library's own pick; 256 CUs on MI355X */
    int cus = 0;
    HIP_OK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    splits = fa2_num_splits(B, hq, hkv, nq, nkv, d, causal, block_m, block_n, cus);
  }
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  int rc;
  if (splits == 1 && !want_lse) {
    rc = fa2_attn_fwd(dq, dk, dv, dout, sq, skv, skv, sq, B, hq, hkv, nq, nkv, d, dtype, causal,
                      pack, block_m, block_n, qk_scale, stream);
  } else {
    const size_t ws_bytes = fa2_workspace_bytes(B, hq, nq, d, splits);
    void* ws = NULL;
    if (ws_bytes) HIP_OK(hipMalloc(&ws, ws_bytes));  /* hipMalloc returns 256-byte alignment */
    rc = fa2_attn_fwd_ex(dq, dk, dv, dout, sq, skv, skv, sq, B, hq, hkv, nq, nkv, d, dtype, causal,
                         pack, block_m, block_n, qk_scale, dlse, splits, ws, ws_bytes, stream);
    HIP_OK(hipStreamSynchronize(stream));
    if (ws) HIP_OK(hipFree(ws));
  }
  if (rc != FA2_OK) fprintf(stderr, "fa2 call returned %d: %s\n", rc, fa2_last_error());
  HIP_OK(hipStreamSynchronize(stream));
  HIP_OK(hipStreamDestroy(stream));

  uint16_t* hout = (uint16_t*)host_alloc(nq_el * 2);
  HIP_OK(hipMemcpy(hout, dout, nq_el * 2, hipMemcpyDeviceToHost));
  float* hlse = NULL;
  if (want_lse) {
    hlse = (float*)host_alloc((size_t)B * hq * nq * 4);
    HIP_OK(hipMemcpy(hlse, dlse, (size_t)B * hq * nq * 4, hipMemcpyDeviceToHost));
  }
  FILE* f = fopen(path, "wb");
  if (!f) {
    fprintf(stderr, "cannot write %s\n", path);
    return 2;
  }
  int32_t header[16] = {B, hq, hkv, nq, nkv, d, dtype, causal, pack, block_m, block_n, splits,
                        want_lse, rc, seed, 0};
  fwrite(header, 4, 16, f);
  fwrite(hq_, 2, nq_el, f);
  fwrite(hk_, 2, nkv_el, f);
  fwrite(hv_, 2, nkv_el, f);
  fwrite(hout, 2, nq_el, f);
  if (want_lse) fwrite(hlse, 4, (size_t)B * hq * nq, f);
  fclose(f);
  HIP_OK(hipFree(dq));
  HIP_OK(hipFree(dk));
  HIP_OK(hipFree(dv));
  HIP_OK(hipFree(dout));
  if (dlse) HIP_OK(hipFree(dlse));
  HIP_OK(hipHostFree(hq_));
  HIP_OK(hipHostFree(hk_));
  HIP_OK(hipHostFree(hv_));
  HIP_OK(hipHostFree(hout));
  if (hlse) HIP_OK(hipHostFree(hlse));
  printf("fa2_capi_check: %s rc=%d splits=%d\n", fa2_version(), rc, splits);
  return rc == FA2_OK ? 0 : 1;
}

static int expect(int rc, int want, const char* what, const char* needle) {
  const char* msg = fa2_last_error();
  const int ok = rc == want && strstr(msg, needle) != NULL;
  printf("%-44s rc=%d (want %d) \"%s\" %s\n", what, rc, want, msg, ok ? "ok" : "FAILED");
  return ok ? 0 : 1;
}

static int errors(void) {
  /* fake but 16-byte aligned pointers: every call below is rejected before any launch */
  void* q = (void*)0x1000;
  void* k = (void*)0x2000;
  const int64_t s[4] = {8192, 2048, 64, 1}, s_bad[4] = {8192, 2048, 60, 1};
  int bad = 0;
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 32, 48, 0, 1, 1, 128, 0, 0.18f, NULL),
                FA2_EINVAL, "head_dim 48", "head_dim");
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s, s, s, 1, 5, 2, 32, 32, 64, 0, 1, 1, 128, 0, 0.18f, NULL),
                FA2_EINVAL, "H_q % H_kv", "divisible");
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 16, 64, 0, 1, 1, 128, 0, 0.18f, NULL),
                FA2_EINVAL, "causal with N_q != N_kv", "N_q == N_kv");
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 32, 64, 0, 1, 2, 127, 0, 0.18f, NULL),
                FA2_EINVAL, "pack with BLOCK_M % group", "BLOCK_M");
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 32, 64, 0, 1, 1, 128, 0, -1.0f, NULL),
                FA2_EINVAL, "qk_scale <= 0", "qk_scale");
  bad += expect(fa2_attn_fwd((char*)q + 8, k, k, q, s, s, s, s, 1, 4, 2, 32, 32, 64, 0, 1, 1, 128, 0,
                             0.18f, NULL),
                FA2_EALIGN, "unaligned q", "aligned");
  bad += expect(fa2_attn_fwd(q, k, k, q, s, s_bad, s, s, 1, 4, 2, 32, 32, 64, 0, 1, 1, 128, 0, 0.18f, NULL),
                FA2_EALIGN, "k stride not a multiple of 8", "multiples of 8");
  bad += expect(fa2_attn_fwd_ex(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 256, 64, 0, 0, 1, 128, 0, 0.18f, NULL,
                                4, NULL, 0, NULL),
                FA2_EINVAL, "split-KV without a workspace", "workspace");
  bad += expect(fa2_attn_fwd_ex(q, k, k, q, s, s, s, s, 1, 4, 2, 32, 32, 64, 0, 1, 1, 128, 0, 0.18f, NULL,
                                2, NULL, 0, NULL),
                FA2_EINVAL, "split-KV with causal", "causal");
  int32_t bm = 0, bn = 0, nw = 0, ns = 0;
  if (fa2_default_config(128, &bm, &bn, &nw, &ns) != FA2_OK || bm != 128 || bn <= 0 || nw != bm / 32) {
    printf("fa2_default_config(128) FAILED\n");
    ++bad;
  }
  if (fa2_should_pack_gqa(1, 4, 128) != 1 || fa2_should_pack_gqa(1000, 7, 128) != 0) {
    printf("fa2_should_pack_gqa FAILED\n");
    ++bad;
  }
  if (fa2_workspace_bytes(16, 32, 1, 128, 1) != 0 || fa2_workspace_bytes(16, 32, 1, 128, 2) == 0) {
    printf("fa2_workspace_bytes FAILED\n");
    ++bad;
  }
  printf("fa2_capi_check errors: %s (%s)\n", bad ? "FAILED" : "all ok", fa2_version());
  return bad ? 1 : 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && strcmp(argv[1], "run") == 0) return run(argc, argv);
  if (argc >= 2 && strcmp(argv[1], "errors") == 0) return errors();
  fprintf(stderr, "usage: %s run ... | errors\n", argv[0]);
  return 2;
}
