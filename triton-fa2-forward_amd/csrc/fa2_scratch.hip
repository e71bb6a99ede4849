// fa2_scratch.hip - the device array behind fa2_attn_fwd_noalloc (include/fa2_fwd.h), in a
// translation unit of its own. Each translation unit of the library is its own device code
// object, so the array's FA2_NOALLOC_SCRATCH_BYTES belong to this code object alone, which no
// kernel launch loads: only noalloc_scratch's address lookup does.
//
// One copy per GPU, alive until the process ends; every call on a GPU shares it, so calls that
// overlap on one GPU (two streams, two threads) race. Nothing in it needs clearing between calls:
// the split-KV partials and the key-norm table are written in full before they are read.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "attn_fwd_launch.hpp"
#include "fa2_fwd.h"

static __device__ __align__(256) unsigned char scratch[FA2_NOALLOC_SCRATCH_BYTES];

namespace fa2 {

namespace {
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kScratchDevices];
}  // namespace

hipError_t noalloc_scratch(int dev, void** out) {
  *out = nullptr;
  if (dev < 0 || dev >= kScratchDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      // the array's host-side name is only a stand-in: its address on this device comes from
      // the runtime, and only that address ever reaches a kernel
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return e != hipSuccess ? e : hipErrorInvalidSymbol;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return hipSuccess;
}

}  // namespace fa2
