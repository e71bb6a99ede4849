// fa2_ablate.hip - C ABI of the measurement library libfa2_ablate.so (include/fa2_ablate.h):
// the forward kernel's timing variants behind the same argument checks and launch sequence as
// the product (attn_fwd_host.hpp, compiled into this library separately).
#include <hip/hip_runtime.h>

#include "attn_fwd_ablate.hpp"
#include "attn_fwd_host.hpp"
#include "fa2_ablate.h"

namespace {

int launch_ablate(int dtype, int di, const Params& p, int waves, int block_n, bool causal,
                  unsigned grid, hipStream_t s, int variant) {
  // the variants exist at the default configuration only (4 waves of 32 rows, the default tile)
  if (waves != 4 || block_n != default_block_n(kDims[di])) return (int)hipErrorInvalidValue;
  switch (dtype * 4 + di) {
    case 0: return fa2::launch_attn_fwd_ablate<0, 16>(p, variant, causal, grid, s);
    case 1: return fa2::launch_attn_fwd_ablate<0, 32>(p, variant, causal, grid, s);
    case 2: return fa2::launch_attn_fwd_ablate<0, 64>(p, variant, causal, grid, s);
    case 3: return fa2::launch_attn_fwd_ablate<0, 128>(p, variant, causal, grid, s);
    case 4: return fa2::launch_attn_fwd_ablate<1, 16>(p, variant, causal, grid, s);
    case 5: return fa2::launch_attn_fwd_ablate<1, 32>(p, variant, causal, grid, s);
    case 6: return fa2::launch_attn_fwd_ablate<1, 64>(p, variant, causal, grid, s);
    default: return fa2::launch_attn_fwd_ablate<1, 128>(p, variant, causal, grid, s);
  }
}

}  // namespace

extern "C" {

const char* fa2_ablate_last_error(void) { return g_err; }

int fa2_ablate_attn_fwd(const void* q, const void* k, const void* v, void* out,
                        const int64_t q_stride[4], const int64_t k_stride[4],
                        const int64_t v_stride[4], const int64_t o_stride[4], int32_t batch,
                        int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                        int32_t dtype, int32_t causal, int32_t pack, float qk_scale,
                        int32_t variant, void* stream) {
  // FA2_ABLATE_STATIC_ORDER is the host's: the launch keeps the static order (no dynamic tail)
  const bool static_order = (variant & FA2_ABLATE_STATIC_ORDER) != 0;
  variant &= ~FA2_ABLATE_STATIC_ORDER;
  // the timeline instance writes its records: only fa2_ablate_timeline, with a buffer, runs it
  if (!fa2::ablation_variant_built(variant) || (variant & fa2::kVariantTimeline)) {
    g_err[0] = '\0';
    return fail(FA2_EINVAL, "variant 0x%x is not one of the built timing variants",
                (unsigned)variant);
  }
  return attn_fwd_impl(q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                       n_q, n_kv, head_dim, dtype, causal, pack, 128, 0, qk_scale, nullptr, 1,
                       nullptr, 0, variant, launch_ablate, stream, nullptr, 0, static_order);
}

int fa2_ablate_timeline(const void* q, const void* k, const void* v, void* out,
                        const int64_t q_stride[4], const int64_t k_stride[4],
                        const int64_t v_stride[4], const int64_t o_stride[4], int32_t batch,
                        int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                        int32_t dtype, int32_t causal, int32_t pack, float qk_scale,
                        uint64_t* records, int64_t record_words, void* stream) {
  g_err[0] = '\0';
  if (!records) return fail(FA2_EINVAL, "null timeline buffer");
  if (reinterpret_cast<uintptr_t>(records) & 7u)
    return fail(FA2_EALIGN, "the timeline buffer must be 8-byte aligned");
  return attn_fwd_impl(q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                       n_q, n_kv, head_dim, dtype, causal, pack, 128, 0, qk_scale, nullptr, 1,
                       nullptr, 0, fa2::kVariantTimeline, launch_ablate, stream, records,
                       record_words);
}

int fa2_ablate_tail_schedule(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                             int32_t head_dim, int32_t causal, int32_t pack,
                             int32_t* static_blocks, int32_t* tail_programs,
                             int32_t* tail_workgroups) {
  g_err[0] = '\0';
  if (!static_blocks || !tail_programs || !tail_workgroups) return fail(FA2_EINVAL, "null output");
  *static_blocks = *tail_programs = *tail_workgroups = 0;
  if (batch < 1 || h_q < 1 || h_kv < 1 || n_q < 1 || h_q % h_kv)
    return fail(FA2_EINVAL, "bad sizes: batch=%d h_q=%d h_kv=%d n_q=%d", batch, h_q, h_kv, n_q);
  if (dim_index(head_dim) < 0)
    return fail(FA2_EINVAL, "head_dim must be a power of two in [16, 128], got %d", head_dim);
  const int group = h_q / h_kv;
  if (pack != 1 && pack != group)
    return fail(FA2_EINVAL, "pack must be 1 or the GQA group %d, got %d", group, pack);
  if (128 % pack)
    return fail(FA2_EINVAL, "pack_gqa needs BLOCK_M (128) to be a multiple of the group (%d)", pack);
  // attn_fwd_impl's grid at block_m 128 (4 waves) and the default K/V tile
  const int64_t n_tiles = ((int64_t)n_q * pack + 127) / 128;
  const int64_t n_bh = (int64_t)batch * (h_q / pack);
  const int64_t units = n_bh / (group / pack);
  const TailSchedule ts =
      tail_schedule(causal != 0, 1, 4, units, group / pack, n_tiles,
                    unit_chunk(units, n_q, head_dim), head_dim, tile_n(0, head_dim));
  *static_blocks = ts.static_blocks;
  *tail_programs = ts.tail_programs;
  *tail_workgroups = ts.tail_wgs;
  return 0;
}

int fa2_ablate_mfma_ceiling(int32_t mode, int32_t workgroups, int32_t iters, float* out,
                            int64_t out_words, void* stream) {
  g_err[0] = '\0';
  if (mode < FA2_ABLATE_CEIL_MFMA || mode > FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC)
    return fail(FA2_EINVAL, "unknown ceiling mode %d", (int)mode);
  if (workgroups < 1 || workgroups > FA2_ABLATE_CEIL_MAX_WORKGROUPS)
    return fail(FA2_EINVAL, "workgroups %d outside [1, %d]", (int)workgroups,
                FA2_ABLATE_CEIL_MAX_WORKGROUPS);
  if (iters < 1 || iters > FA2_ABLATE_CEIL_MAX_ITERS)
    return fail(FA2_EINVAL, "iters %d outside [1, %d]", (int)iters, FA2_ABLATE_CEIL_MAX_ITERS);
  if (!out) return fail(FA2_EINVAL, "null output");
  if (reinterpret_cast<uintptr_t>(out) & 3u)
    return fail(FA2_EALIGN, "the output must be 4-byte aligned");
  if (out_words < (int64_t)workgroups * 256)
    return fail(FA2_EINVAL, "the output holds %lld floats; %d workgroups write %lld",
                (long long)out_words, (int)workgroups, (long long)workgroups * 256);
  const int rc = fa2::launch_mfma_ceiling(mode, out, workgroups, iters,
                                          static_cast<hipStream_t>(stream));
  if (rc != 0)
    return fail(FA2_ELAUNCH, "ceiling launch failed: %s", hipGetErrorString((hipError_t)rc));
  return 0;
}

int fa2_ablate_hbm_read(const void* src, int64_t bytes, uint32_t* out, int64_t out_words,
                        int32_t workgroups, void* stream) {
  g_err[0] = '\0';
  if (!src || !out) return fail(FA2_EINVAL, "null buffer");
  if ((reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(out) & 3u))
    return fail(FA2_EALIGN, "src must be 16-byte and out 4-byte aligned");
  if (bytes < 16 || bytes % 16) return fail(FA2_EINVAL, "bytes (%lld) must be a positive multiple of 16", (long long)bytes);
  if (workgroups < 1 || workgroups > FA2_ABLATE_CEIL_MAX_WORKGROUPS)
    return fail(FA2_EINVAL, "workgroups %d outside [1, %d]", (int)workgroups,
                FA2_ABLATE_CEIL_MAX_WORKGROUPS);
  if (out_words < (int64_t)workgroups * 256)
    return fail(FA2_EINVAL, "the output holds %lld words; %d workgroups write %lld",
                (long long)out_words, (int)workgroups, (long long)workgroups * 256);
  const int rc = fa2::launch_hbm_read(src, bytes / 16, out, workgroups, static_cast<hipStream_t>(stream));
  if (rc != 0)
    return fail(FA2_ELAUNCH, "read launch failed: %s", hipGetErrorString((hipError_t)rc));
  return 0;
}

}  // extern "C"
