// attn_fwd_launch.hpp - per (dtype, head_dim) launchers of the forward kernel.
//
// Each instantiation lives in its own translation unit (attn_fwd_inst.hip compiled once per
// dtype x head_dim), so the library's many kernel instances build in parallel.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "attn_fwd_params.hpp"

namespace fa2 {

// One kernel launch on `stream`; with a `stop` event, through hipExtLaunchKernel, which signals
// the event from the kernel's own completion instead of a marker of its own in the stream.
// Returns a hipError_t value.
template <class Kernel>
int launch_with_stop(Kernel kernel, unsigned grid, unsigned block, hipStream_t stream,
                     hipEvent_t stop, const Params& p) {
  if (stop)
    hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream, nullptr, stop, 0, p);
  else
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream, p);
  return (int)hipGetLastError();
}

// Launches attn_fwd_kernel<DT, D, waves, block_n, causal> on `grid` programs.
// waves in {1, 2, 4, 8}, block_n in {32, 64, 128}; `stop` (or null) is signalled when the kernel
// ends. Returns a hipError_t value.
template <int DT, int D>
int launch_attn_fwd(const Params& p, int waves, int block_n, bool causal, unsigned grid,
                    hipStream_t stream, hipEvent_t stop);

// gfx950 default K/V tile: 64 keys (sweep.py on the BASELINE.json configs, MI355X: best for
// C2, C3, C5 at head_dim 128, and for C4 at head_dim 64 with the software-pipelined loop that
// 64-key tiles get there; a tie with 128 at head_dim 32); 128 keys at head_dim 16 (+2.4% causal,
// +3.6% full on a B2 H16 N16384 shape).
constexpr int default_block_n(int head_dim) { return head_dim == 16 ? 128 : 64; }

// Launches the split-KV combine pass (attn_fwd_combine.hip).
int launch_combine(int dtype, int head_dim, const CombineParams& c, hipStream_t stream);

// Launches the key-norm pass (attn_key_norm.hip) on `grid` = batch * h_kv * chunks workgroups.
int launch_key_norm(int dtype, int head_dim, const KeyNormParams& k, unsigned grid,
                    hipStream_t stream);

// Devices the no-allocation scratch table covers (fa2_scratch.hip).
constexpr int kScratchDevices = 64;
// The device address of fa2_attn_fwd_noalloc's scratch array on device `dev`, which must be the
// current device: looked up once per device (hipGetSymbolAddress) and kept. Returns a hipError_t.
hipError_t noalloc_scratch(int dev, void** out);

#define FA2_DECLARE_LAUNCH(DT, D)                                                          \
  extern template int launch_attn_fwd<DT, D>(const Params&, int, int, bool, unsigned, \
                                             hipStream_t, hipEvent_t);
FA2_DECLARE_LAUNCH(0, 16)
FA2_DECLARE_LAUNCH(0, 32)
FA2_DECLARE_LAUNCH(0, 64)
FA2_DECLARE_LAUNCH(0, 128)
FA2_DECLARE_LAUNCH(1, 16)
FA2_DECLARE_LAUNCH(1, 32)
FA2_DECLARE_LAUNCH(1, 64)
FA2_DECLARE_LAUNCH(1, 128)
#undef FA2_DECLARE_LAUNCH

}  // namespace fa2
