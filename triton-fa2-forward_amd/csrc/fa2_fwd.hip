// fa2_fwd.hip - C ABI of the gfx950 FlashAttention-2 forward (declared in include/fa2_fwd.h).
//
// Host half of the reference's launch wrapper `attention()` (fa2/kernel.py:210-260):
// argument checks, the kernel-instance choice and the grid, then one asynchronous
// launch on the caller's stream. Python keeps the tensor-level checks and exceptions;
// this file re-checks every value the kernel relies on so that a non-Python host cannot
// launch it out of bounds.
#include <hip/hip_runtime.h>

#include "attn_fwd_host.hpp"

namespace {

// The product's kernel instances, per (dtype, head_dim) each compiled in its own translation
// unit. This library has no timing variants (the measurement library fa2_ablate.hip has them).
int launch(int dtype, int di, const Params& p, int waves, int block_n, bool causal, unsigned grid,
           hipStream_t s, int variant, hipEvent_t stop) {
  if (variant != 0) return (int)hipErrorInvalidValue;
  switch (dtype * 4 + di) {
    case 0: return fa2::launch_attn_fwd<0, 16>(p, waves, block_n, causal, grid, s, stop);
    case 1: return fa2::launch_attn_fwd<0, 32>(p, waves, block_n, causal, grid, s, stop);
    case 2: return fa2::launch_attn_fwd<0, 64>(p, waves, block_n, causal, grid, s, stop);
    case 3: return fa2::launch_attn_fwd<0, 128>(p, waves, block_n, causal, grid, s, stop);
    case 4: return fa2::launch_attn_fwd<1, 16>(p, waves, block_n, causal, grid, s, stop);
    case 5: return fa2::launch_attn_fwd<1, 32>(p, waves, block_n, causal, grid, s, stop);
    case 6: return fa2::launch_attn_fwd<1, 64>(p, waves, block_n, causal, grid, s, stop);
    default: return fa2::launch_attn_fwd<1, 128>(p, waves, block_n, causal, grid, s, stop);
  }
}

}  // namespace

extern "C" {

const char* fa2_last_error(void) { return g_err; }

const char* fa2_version(void) { return "fa2-mi355x 0.1.0 (gfx950, mfma_f32_32x32x16)"; }

int fa2_default_config(int32_t head_dim, int32_t* block_m, int32_t* block_n,
                       int32_t* num_waves, int32_t* num_stages) {
  if (dim_index(head_dim) < 0)
    return fail(FA2_EINVAL, "head_dim must be one of 16, 32, 64, 128, got %d", head_dim);
  // gfx950 defaults: 4 wave64s of 32 query rows, default_block_n keys per K/V tile, two K
  // and two V tiles in LDS.
  if (block_m) *block_m = 128;
  if (block_n) *block_n = default_block_n(head_dim);
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
  return fa2_attn_fwd_ex(q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                         n_q, n_kv, head_dim, dtype, causal, pack, block_m, block_n, qk_scale,
                         nullptr, 1, nullptr, 0, stream);
}

size_t fa2_workspace_bytes(int32_t batch, int32_t h_q, int32_t n_q, int32_t head_dim,
                           int32_t num_splits) {
  if (num_splits <= 1 || batch <= 0 || h_q <= 0 || n_q <= 0 || dim_index(head_dim) < 0) return 0;
  const size_t rows = (size_t)batch * h_q * n_q;
  return workspace_layout(rows, head_dim, num_splits).total;
}

size_t fa2_workspace_bytes_for(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                               int32_t n_kv, int32_t head_dim, int32_t dtype, int32_t causal,
                               int32_t num_splits) {
  if (batch <= 0 || h_q <= 0 || h_kv <= 0 || n_q <= 0 || n_kv <= 0 || dim_index(head_dim) < 0)
    return 0;
  size_t bytes = fa2_workspace_bytes(batch, h_q, n_q, head_dim, num_splits);
  if (key_table_pays(batch, h_q, h_kv, n_q, n_kv, head_dim, dtype, causal != 0))
    bytes += key_table_bytes(batch, h_kv, n_kv);
  return bytes;
}

int32_t fa2_num_splits(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                       int32_t head_dim, int32_t causal, int32_t block_m, int32_t block_n,
                       int32_t num_cus) {
  if (causal || batch <= 0 || h_q <= 0 || h_kv <= 0 || h_q % h_kv || n_q <= 0 || n_kv <= 0 ||
      block_m <= 0 || num_cus <= 0 || dim_index(head_dim) < 0)
    return 1;
  // The grid of the smaller of the two GQA layouts, so that a packed and an unpacked launch
  // of the same problem split the same way and stay equal bit for bit.
  const int group = h_q / h_kv;
  int64_t programs = ((int64_t)n_q + block_m - 1) / block_m * ((int64_t)batch * h_q);
  if (block_m % group == 0)
    programs = std::min(programs, ((int64_t)n_q * group + block_m - 1) / block_m * ((int64_t)batch * h_kv));
  const int bn = tile_n(block_n, head_dim);
  const int64_t tiles = ((int64_t)n_kv + bn - 1) / bn;
  // Split until every CU has a workgroup, with at least kMinSplitTiles tiles per split and at
  // most kMaxSplits splits. (Filling the second workgroup slot of each CU as well measured
  // slower on MI355X: the fp32 partial outputs cost more than the extra overlap gains.)
  int s = 1;
  while (programs * s < num_cus && s * 2 <= kMaxSplits && tiles / (s * 2) >= kMinSplitTiles) s *= 2;
  return s;
}

int fa2_attn_fwd_ex(const void* q, const void* k, const void* v, void* out,
                    const int64_t q_stride[4], const int64_t k_stride[4],
                    const int64_t v_stride[4], const int64_t o_stride[4],
                    int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                    int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                    int32_t block_m, int32_t block_n, float qk_scale, float* lse,
                    int32_t num_splits, void* workspace, size_t workspace_bytes, void* stream) {
  const LaunchArgs a{q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                     n_q, n_kv, head_dim, dtype, causal, pack, block_m, block_n, qk_scale, lse,
                     num_splits, workspace, workspace_bytes, 0, nullptr, 0, false};
  return attn_fwd_impl(a, launch, stream);
}

}  // extern "C"

// ---- the no-allocation entry point. Its workspace is the library's own device array, defined in
// fa2_scratch.hip: a translation unit of its own, so that its 32 MiB belong to a code object that
// only this entry point's address lookup loads.

extern "C" {

int fa2_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* out,
                         const int64_t q_stride[4], const int64_t k_stride[4],
                         const int64_t v_stride[4], const int64_t o_stride[4],
                         int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                         int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                         int32_t block_m, int32_t block_n, float qk_scale, float* lse,
                         int32_t num_splits, void* stream) {
  g_err[0] = '\0';
  // the split-KV partials are required; the key-norm table (where it pays) is optional and is
  // left off when it would not fit beside them
  const size_t need = fa2_workspace_bytes(batch, h_q, n_q, head_dim, num_splits);
  if (need > (size_t)FA2_NOALLOC_SCRATCH_BYTES)
    return fail(FA2_EINVAL,
                "split-KV with %d splits needs %zu bytes of scratch; fa2_attn_fwd_noalloc holds "
                "%zu (use fa2_attn_fwd_ex with a workspace, or fewer splits)",
                num_splits, need, (size_t)FA2_NOALLOC_SCRATCH_BYTES);
  size_t use = fa2_workspace_bytes_for(batch, h_q, h_kv, n_q, n_kv, head_dim, dtype, causal,
                                       num_splits);
  if (use > (size_t)FA2_NOALLOC_SCRATCH_BYTES) use = need;
  void* ws = nullptr;
  if (use > 0) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(FA2_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (stream) {
      hipDevice_t sdev = -1;
      e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
      if (e != hipSuccess)
        return fail(FA2_ELAUNCH, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
      if (sdev != dev)
        return fail(FA2_EINVAL,
                    "the stream runs on device %d but device %d is current; make it current",
                    sdev, dev);
    }
    if (dev < 0 || dev >= fa2::kScratchDevices)
      return fail(FA2_EINVAL, "device %d is past the %d devices the scratch table covers", dev,
                  fa2::kScratchDevices);
    e = fa2::noalloc_scratch(dev, &ws);
    if (e != hipSuccess || !ws)
      return fail(FA2_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
  }
  const LaunchArgs a{q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                     n_q, n_kv, head_dim, dtype, causal, pack, block_m, block_n, qk_scale, lse,
                     num_splits, ws, use, 0, nullptr, 0, false, false};
  return attn_fwd_impl(a, launch, stream);
}

}  // extern "C"
