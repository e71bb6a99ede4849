// attn_fwd_ablate.hpp - the timing variants of the forward kernel, built only into the
// measurement library libfa2_ablate.so (fa2_ablate.hip, attn_fwd_ablate_inst.hip), never into
// libfa2_fwd.so. Counterpart of the reference's knockout copy of its kernel (bench/ablation.py:
// 1-20, 56-202): here the switches are VARIANT bits of the one kernel template, so every variant
// is the product's code with one kind of work changed or removed.
#pragma once

#include <hip/hip_runtime.h>

#include "attn_fwd_common.hpp"
#include "attn_fwd_params.hpp"

namespace fa2 {

// The variants built, by the reference's names (bench/ablation.py:42-53): VARIANT bit sets.
constexpr int kAblationVariants[] = {
    0,                                            // copy: the product kernel, bit for bit
    kVariantScaleFirst,                           // scale_first
    kVariantMaskEveryTile,                        // mask_every_tile
    kVariantScaleFirst | kVariantMaskEveryTile,   // before_fixes
    kVariantNoExp,                                // no_exp
    kVariantNoSoftmax,                            // no_softmax
    kVariantKvL2,                                 // kv_l2
    kVariantNoSoftmax | kVariantKvL2,             // matmul_only
    kVariantNoKvStaging,                          // no_kv_staging (not in the reference)
    kVariantSplitKeys,                            // split_keys (not in the reference)
    kVariantNoQLoad,                              // no_q_load (not in the reference)
    kVariantNoStore,                              // no_store (not in the reference)
    kVariantTimeline,                             // copy + per-workgroup timeline records
};

constexpr bool ablation_variant_built(int variant) {
  for (int v : kAblationVariants)
    if (v == variant) return true;
  return false;
}

// Launches attn_fwd_kernel<DT, D, 4, default_block_n(D), causal, variant> on `grid` programs of
// 128 rows; variant must be one of kAblationVariants. Returns a hipError_t value.
template <int DT, int D>
int launch_attn_fwd_ablate(const Params& p, int variant, bool causal, unsigned grid,
                           hipStream_t stream, hipEvent_t stop);

#define FA2_DECLARE_ABLATE(DT, D)                                                          \
  extern template int launch_attn_fwd_ablate<DT, D>(const Params&, int, bool, unsigned, \
                                                    hipStream_t, hipEvent_t);
FA2_DECLARE_ABLATE(0, 16)
FA2_DECLARE_ABLATE(0, 32)
FA2_DECLARE_ABLATE(0, 64)
FA2_DECLARE_ABLATE(0, 128)
FA2_DECLARE_ABLATE(1, 16)
FA2_DECLARE_ABLATE(1, 32)
FA2_DECLARE_ABLATE(1, 64)
FA2_DECLARE_ABLATE(1, 128)
#undef FA2_DECLARE_ABLATE

// Launches mfma_ceiling_kernel<mode> (mfma_ceiling.hip) on `workgroups` workgroups of 256
// threads, `iters` x 16 MFMAs per wave; mode is one of FA2_ABLATE_CEIL_*. Returns a hipError_t
// value.
int launch_mfma_ceiling(int mode, float* out, int workgroups, int iters, hipStream_t stream);

// Launches hbm_read_kernel (mfma_ceiling.hip): `workgroups` x 256 threads read n16 16-byte words
// of src, grid-stride, each thread writing one word of out. Returns a hipError_t value.
int launch_hbm_read(const void* src, int64_t n16, uint32_t* out, int workgroups, hipStream_t stream);

}  // namespace fa2
