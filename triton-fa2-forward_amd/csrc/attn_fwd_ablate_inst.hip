// attn_fwd_ablate_inst.hip - the timing-variant instances of one (dtype, head_dim) pair for the
// measurement library. Compiled once per pair with -DFA2_DT=<0|1> -DFA2_D=<16|32|64|128>.
#include "attn_fwd_ablate.hpp"
#include "attn_fwd_kernel.hpp"
#include "attn_fwd_launch.hpp"

#if !defined(FA2_DT) || !defined(FA2_D)
#error "compile with -DFA2_DT=<0|1> -DFA2_D=<16|32|64|128>"
#endif

namespace fa2 {

namespace {

template <int DT, int D, int VARIANT>
int launch_variant(const Params& p, bool causal, unsigned grid, hipStream_t s, hipEvent_t stop) {
  constexpr int BN = default_block_n(D);
  if constexpr ((VARIANT & kVariantSplitKeys) != 0) {
    // the key split: 8 waves, two groups of 4 on the same 128 rows; head_dim 128 only
    if constexpr (D != 128) {
      return (int)hipErrorInvalidValue;
    } else {
      if (causal)
        return launch_with_stop(attn_fwd_kernel<DT, D, 8, BN, true, VARIANT>, grid, 512, s, stop,
                                p);
      return launch_with_stop(attn_fwd_kernel<DT, D, 8, BN, false, VARIANT>, grid, 512, s, stop,
                              p);
    }
  } else {
    if (causal)
      return launch_with_stop(attn_fwd_kernel<DT, D, 4, BN, true, VARIANT>, grid, 256, s, stop, p);
    return launch_with_stop(attn_fwd_kernel<DT, D, 4, BN, false, VARIANT>, grid, 256, s, stop, p);
  }
}

template <int DT, int D, int... V>
int dispatch(const Params& p, int variant, bool causal, unsigned grid, hipStream_t s,
             hipEvent_t stop) {
  int rc = (int)hipErrorInvalidValue;
  (void)((variant == V ? (rc = launch_variant<DT, D, V>(p, causal, grid, s, stop), true) : false) ||
         ...);
  return rc;
}

}  // namespace

template <int DT, int D>
int launch_attn_fwd_ablate(const Params& p, int variant, bool causal, unsigned grid,
                           hipStream_t s, hipEvent_t stop) {
  return dispatch<DT, D, kAblationVariants[0], kAblationVariants[1], kAblationVariants[2],
                  kAblationVariants[3], kAblationVariants[4], kAblationVariants[5],
                  kAblationVariants[6], kAblationVariants[7], kAblationVariants[8],
                  kAblationVariants[9], kAblationVariants[10], kAblationVariants[11],
                  kAblationVariants[12]>(
      p, variant, causal, grid, s, stop);
}

static_assert(sizeof(kAblationVariants) / sizeof(int) == 13, "dispatch lists every variant");

template int launch_attn_fwd_ablate<FA2_DT, FA2_D>(const Params&, int, bool, unsigned,
                                                   hipStream_t, hipEvent_t);

}  // namespace fa2
