// fa2_fwd.hip - C ABI of the gfx950 FlashAttention-2 forward (declared in include/fa2_fwd.h).
//
// Host half of the reference's launch wrapper `attention()` (fa2/kernel.py:210-260):
// argument checks, the kernel-instance choice and the grid, then one asynchronous
// launch on the caller's stream. Python keeps the tensor-level checks and exceptions;
// this file re-checks every value the kernel relies on so that a non-Python host cannot
// launch it out of bounds.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "attn_fwd_launch.hpp"
#include "fa2_fwd.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

using fa2::Params;

constexpr int kDims[4] = {16, 32, 64, 128};
// 128 rows x stride x 2 bytes must stay below 2^31.
constexpr int64_t kMaxRowStride = int64_t(1) << 22;

// Per (dtype, head_dim) launchers, each compiled in its own translation unit.
int launch_r64(int dtype, int di, const Params& p, int waves, bool causal, unsigned grid,
               hipStream_t s) {
  switch (dtype * 4 + di) {
    case 2: return fa2::launch_attn_fwd_r64<0, 64>(p, waves, 32, causal, grid, s);
    case 3: return fa2::launch_attn_fwd_r64<0, 128>(p, waves, 32, causal, grid, s);
    case 6: return fa2::launch_attn_fwd_r64<1, 64>(p, waves, 32, causal, grid, s);
    default: return fa2::launch_attn_fwd_r64<1, 128>(p, waves, 32, causal, grid, s);
  }
}

int launch(int dtype, int di, const Params& p, int waves, int block_n, bool causal, unsigned grid,
           hipStream_t s) {
  switch (dtype * 4 + di) {
    case 0: return fa2::launch_attn_fwd<0, 16>(p, waves, block_n, causal, grid, s);
    case 1: return fa2::launch_attn_fwd<0, 32>(p, waves, block_n, causal, grid, s);
    case 2: return fa2::launch_attn_fwd<0, 64>(p, waves, block_n, causal, grid, s);
    case 3: return fa2::launch_attn_fwd<0, 128>(p, waves, block_n, causal, grid, s);
    case 4: return fa2::launch_attn_fwd<1, 16>(p, waves, block_n, causal, grid, s);
    case 5: return fa2::launch_attn_fwd<1, 32>(p, waves, block_n, causal, grid, s);
    case 6: return fa2::launch_attn_fwd<1, 64>(p, waves, block_n, causal, grid, s);
    default: return fa2::launch_attn_fwd<1, 128>(p, waves, block_n, causal, grid, s);
  }
}

int dim_index(int d) {
  for (int i = 0; i < 4; ++i)
    if (kDims[i] == d) return i;
  return -1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

const char* fa2_last_error(void) { return g_err; }

const char* fa2_version(void) { return "fa2-mi355x 0.1.0 (gfx950, mfma_f32_32x32x16)"; }

int fa2_default_config(int32_t head_dim, int32_t* block_m, int32_t* block_n,
                       int32_t* num_waves, int32_t* num_stages) {
  if (dim_index(head_dim) < 0)
    return fail(FA2_EINVAL, "head_dim must be one of 16, 32, 64, 128, got %d", head_dim);
  // gfx950 defaults: 4 wave64s of 32 query rows, 64-key K/V tiles, one tile in LDS
  // while the next is in flight in registers.
  if (block_m) *block_m = 128;
  if (block_n) *block_n = 64;
  if (num_waves) *num_waves = 4;
  if (num_stages) *num_stages = 2;
  return FA2_OK;
}

int fa2_should_pack_gqa(int32_t n_q, int32_t group, int32_t block_m) {
  if (group <= 1 || block_m <= 0 || block_m % group) return 0;
  // _tile_efficiency(rows, bm) = rows / (ceil(rows / bm) * bm), fa2/kernel.py:198-199
  auto eff = [block_m](double rows) {
    const double tiles = std::ceil(rows / block_m);
    return tiles > 0 ? rows / (tiles * block_m) : 0.0;
  };
  return eff((double)n_q) < 0.9 * eff((double)n_q * group) ? 1 : 0;
}

int fa2_attn_fwd(const void* q, const void* k, const void* v, void* out,
                 const int64_t q_stride[4], const int64_t k_stride[4],
                 const int64_t v_stride[4], const int64_t o_stride[4],
                 int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                 int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                 int32_t block_m, int32_t block_n, float qk_scale, void* stream) {
  g_err[0] = '\0';
  // ---- shape checks (fa2/kernel.py:218-228)
  if (batch < 0 || h_q <= 0 || h_kv <= 0 || n_q < 0 || n_kv < 0)
    return fail(FA2_EINVAL, "bad sizes: batch=%d h_q=%d h_kv=%d n_q=%d n_kv=%d", batch, h_q,
                h_kv, n_q, n_kv);
  if (h_q % h_kv) return fail(FA2_EINVAL, "GQA needs H_q divisible by H_kv (%d %% %d)", h_q, h_kv);
  const int di = dim_index(head_dim);
  if (di < 0)
    return fail(FA2_EINVAL, "head_dim must be a power of two in [16, 128], got %d", head_dim);
  if (dtype != FA2_DTYPE_F16 && dtype != FA2_DTYPE_BF16)
    return fail(FA2_EINVAL, "dtype must be FA2_DTYPE_F16 or FA2_DTYPE_BF16, got %d", dtype);
  if (causal && n_q != n_kv)
    return fail(FA2_EINVAL, "causal attention here assumes N_q == N_kv (%d != %d)", n_q, n_kv);
  // ---- program shape (fa2/kernel.py:230-238)
  const int group = h_q / h_kv;
  if (pack != 1 && pack != group)
    return fail(FA2_EINVAL, "pack must be 1 or the GQA group %d, got %d", group, pack);
  if (block_m < 1 || block_m > 256)
    return fail(FA2_EINVAL, "BLOCK_M must be in [1, 256], got %d", block_m);
  if (block_m % pack)
    return fail(FA2_EINVAL,
                "pack_gqa needs BLOCK_M (%d) to be a multiple of the GQA group (%d)", block_m,
                pack);
  if (block_n < 0 || block_n > 128)
    return fail(FA2_EINVAL, "BLOCK_N must be in [1, 128] (0 = default), got %d", block_n);
  if (!(qk_scale > 0.f) || !std::isfinite(qk_scale))
    return fail(FA2_EINVAL, "qk_scale (sm_scale * log2 e) must be positive and finite, got %g",
                (double)qk_scale);
  if (batch == 0 || n_q == 0) return FA2_OK;  // empty output: nothing to launch
  // ---- the 16-byte load/store rule
  if (!q || !k || !v || !out) return fail(FA2_EINVAL, "null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(FA2_EALIGN, "q, k, v and out must be 16-byte aligned");
  const int64_t* strides[4] = {q_stride, k_stride, v_stride, o_stride};
  for (int t = 0; t < 4; ++t) {
    if (!strides[t]) return fail(FA2_EINVAL, "null stride array");
    if (strides[t][3] != 1)
      return fail(FA2_EALIGN, "the head_dim stride must be 1 (tensor %d has %lld)", t,
                  (long long)strides[t][3]);
    for (int j = 0; j < 3; ++j)
      if (strides[t][j] % 8 || strides[t][j] < 0)
        return fail(FA2_EALIGN, "strides must be multiples of 8 elements (tensor %d dim %d: %lld)",
                    t, j, (long long)strides[t][j]);
  }
  // K/V tiles are addressed with 32-bit byte offsets from the tile's first row.
  if (k_stride[2] > kMaxRowStride || v_stride[2] > kMaxRowStride)
    return fail(FA2_EINVAL, "k/v sequence stride above %lld elements is not supported",
                (long long)kMaxRowStride);

  // block_m rows -> wave64s of 32 rows, rounded up to 1, 2, 4 or 8 (rows past block_m are
  // computed on zeros and dropped); block_n -> the next supported K/V tile width.
  int waves = 1;
  while (waves * 32 < block_m) waves *= 2;
  const int bn_req = block_n ? block_n : 64;
  const int bn = bn_req <= 32 ? 32 : bn_req <= 64 ? 64 : 128;

  Params p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(out);
  p.sqb = q_stride[0]; p.sqh = q_stride[1]; p.sqn = q_stride[2];
  p.skb = k_stride[0]; p.skh = k_stride[1]; p.skn = k_stride[2];
  p.svb = v_stride[0]; p.svh = v_stride[1]; p.svn = v_stride[2];
  p.sob = o_stride[0]; p.soh = o_stride[1]; p.son = o_stride[2];
  p.h_q = h_q;
  p.n_q = n_q;
  p.n_kv = n_kv;
  p.group = group;
  p.pack = pack;
  p.block_m = block_m;
  const int64_t rows = (int64_t)n_q * pack;
  const int64_t n_tiles = (rows + block_m - 1) / block_m;
  const int64_t n_bh = (int64_t)batch * (h_q / pack);
  if (n_tiles * n_bh > 0x7fffffffLL)
    return fail(FA2_EINVAL, "grid of %lld programs is too large", (long long)(n_tiles * n_bh));
  p.n_tiles = (int32_t)n_tiles;
  p.n_bh = (int32_t)n_bh;
  p.qk_scale = qk_scale;

  // Programs of 128 or 256 rows over 32-key tiles at head_dim 64/128 run the kernel with 64
  // query rows per wave (half the LDS traffic per FLOP); everything else the 32-row kernel.
  const bool r64 = head_dim >= 64 && (block_m == 128 || block_m == 256) && bn == 32;
  const int e = r64 ? launch_r64(dtype, di, p, block_m / 64, causal != 0,
                                 (unsigned)(n_tiles * n_bh), static_cast<hipStream_t>(stream))
                    : launch(dtype, di, p, waves, bn, causal != 0, (unsigned)(n_tiles * n_bh),
                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(FA2_ELAUNCH, "kernel launch failed: %s", hipGetErrorString((hipError_t)e));
  return FA2_OK;
}

}  // extern "C"
