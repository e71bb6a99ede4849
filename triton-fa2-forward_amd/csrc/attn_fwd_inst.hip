// attn_fwd_inst.hip - the kernel instances of one (dtype, head_dim) pair.
// Compiled once per pair with -DFA2_DT=<0 fp16 | 1 bf16> -DFA2_D=<16|32|64|128>.
#include "attn_fwd_kernel.hpp"
#include "attn_fwd_launch.hpp"

#if !defined(FA2_DT) || !defined(FA2_D)
#error "compile with -DFA2_DT=<0|1> -DFA2_D=<16|32|64|128>"
#endif

namespace fa2 {

namespace {

template <int DT, int D, int NW, int BN>
int launch_shape(const Params& p, bool causal, unsigned grid, hipStream_t s, hipEvent_t stop) {
  if (causal) return launch_with_stop(attn_fwd_kernel<DT, D, NW, BN, true>, grid, NW * 64, s, stop, p);
  return launch_with_stop(attn_fwd_kernel<DT, D, NW, BN, false>, grid, NW * 64, s, stop, p);
}

template <int DT, int D, int NW>
int launch_bn(const Params& p, int block_n, bool causal, unsigned grid, hipStream_t s,
              hipEvent_t stop) {
  switch (block_n) {
    case 32: return launch_shape<DT, D, NW, 32>(p, causal, grid, s, stop);
    case 64: return launch_shape<DT, D, NW, 64>(p, causal, grid, s, stop);
    default: return launch_shape<DT, D, NW, 128>(p, causal, grid, s, stop);
  }
}

}  // namespace

template <int DT, int D>
int launch_attn_fwd(const Params& p, int waves, int block_n, bool causal, unsigned grid,
                    hipStream_t s, hipEvent_t stop) {
  if (p.key_norm2) {  // the host writes a key-norm table only for the default configuration
    constexpr int BN = default_block_n(D);
    if (waves != 4 || block_n != BN) return (int)hipErrorInvalidValue;
    if (causal)
      return launch_with_stop(attn_fwd_kernel<DT, D, 4, BN, true, kVariantKeyBound>, grid, 256, s,
                              stop, p);
    return launch_with_stop(attn_fwd_kernel<DT, D, 4, BN, false, kVariantKeyBound>, grid, 256, s,
                            stop, p);
  }
  switch (waves) {
    case 1: return launch_bn<DT, D, 1>(p, block_n, causal, grid, s, stop);
    case 2: return launch_bn<DT, D, 2>(p, block_n, causal, grid, s, stop);
    case 4: return launch_bn<DT, D, 4>(p, block_n, causal, grid, s, stop);
    default: return launch_bn<DT, D, 8>(p, block_n, causal, grid, s, stop);
  }
}

template int launch_attn_fwd<FA2_DT, FA2_D>(const Params&, int, int, bool, unsigned, hipStream_t,
                                            hipEvent_t);

}  // namespace fa2
