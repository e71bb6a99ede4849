// mfma_ceiling.hip - what the matrix cores sustain on this chip, for the measurement library
// (fa2_ablate_mfma_ceiling, include/fa2_ablate.h, checks the arguments and calls
// launch_mfma_ceiling).
//
// MI355X holds its socket power near the limit by lowering the graphics clock, and the energy of
// an MFMA depends on its operands' bits: constant operands run at the top clock, random ones do
// not. This kernel issues v_mfma_f32_32x32x16_bf16 back to back (two independent accumulators,
// no other dependency) in the attention kernel's launch shape: 256-thread workgroups, 64 KiB of
// dynamic LDS each, so two workgroups (two waves per SIMD) per CU. Modes add, per MFMA, the
// attention kernel's other work, on data that depends on nothing:
//   FA2_ABLATE_CEIL_MFMA              random operands in registers;
//   FA2_ABLATE_CEIL_MFMA_CONST        the same with constant operands (1.0);
//   FA2_ABLATE_CEIL_MFMA_LDS          random operands, one 1 KiB ds_read_b128 per MFMA (the K and
//                                     V operand traffic of 32-row waves);
//   FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX  that plus the softmax's vector work per MFMA at head_dim
//                                     128 (one FMA and one exp2 per score and lane register,
//                                     half a bf16 pack, half a dot2 row sum);
//   FA2_ABLATE_CEIL_MFMA_EXP          random operands in registers, one exp2 per MFMA;
//   FA2_ABLATE_CEIL_MFMA_FMA2         random operands in registers, two FMAs per MFMA
//   FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC  the LDS_SOFTMAX mix with the two accumulators held in
//                                     VGPRs, where the attention kernel holds its own
//   FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC  the VACC mix with one 1 KiB read per two MFMAs: the
//                                     operand reads of 64-row waves, where every K and V
//                                     operand feeds the MFMAs of two 32-row blocks; four
//                                     accumulators instead of two
//   FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE  the same with 128 KiB of LDS per workgroup: one
//                                     workgroup, one wave per SIMD, per CU (the occupancy that
//                                     64-row waves at head_dim 128 would have)
//   FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE  the VACC mix with head_dim 64's softmax per MFMA (a
//                                     tile's 16 MFMAs carry its 32 scores per lane: two FMAs, two
//                                     exp2, one bf16 pack, one dot2 sum) at its occupancy: 48 KiB
//                                     of LDS, three workgroups (three waves per SIMD) per CU
// (EXP and FMA2 price an exp2 against FMAs in the issue cycles beside the MFMAs). For every other
// mode the compiler keeps the accumulators in AGPRs, since nothing but MFMAs touches them in the
// loop; with vector work beside the MFMAs the two placements do not issue alike, so VACC gives
// the mix ceiling of the kernel's own placement. Its MFMAs are inline asm in the VGPR form
// (the compiler's own choice is one form for all of a kernel's MFMAs), and the compiler's hazard
// recognizer does not see them: 2 wait states separate the vector writes of their operands
// (before the loop) from the first, and the results are read once, after 12 wait states, gfx950's
// waits around a 32x32x16 MFMA.
// The output is meaningless; every lane writes one float so that nothing is optimised away.
//
// hbm_read_kernel is the memory-side counterpart (fa2_ablate_hbm_read): a streaming read of a
// buffer, 16 bytes per lane per load, four loads in flight per lane, grid-stride, for the rate
// HBM sustains on a plain read (the bound of the few-queries, split-KV regime).
#include <hip/hip_runtime.h>

#include "attn_fwd_ablate.hpp"
#include "attn_fwd_common.hpp"
#include "fa2_ablate.h"

namespace fa2 {
namespace {

constexpr int kCeilThreads = 256;
constexpr size_t kCeilLdsBytes = 64 * 1024;  // two workgroups per CU, as attn_fwd_kernel
constexpr int kCeilChunks = 16;              // operands read: 16 chunks of 1 KiB

// 32-bit integer hash ("lowbias32", C. Wellons, public domain)
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// two bf16 with random sign and mantissa in +-[0.5, 2), or two 1.0
__device__ __forceinline__ uint32_t bf16_pair(uint32_t x, bool random) {
  if (!random) return 0x3f803f80u;
  const uint32_t r = mix32(x);
  const uint32_t lo = (r & 0x8000u) | ((126u + (r >> 7 & 1u)) << 7) | (r & 0x7fu);
  const uint32_t h = r >> 16;
  const uint32_t hi = (h & 0x8000u) | ((126u + (h >> 7 & 1u)) << 7) | (h & 0x7fu);
  return lo | hi << 16;
}

template <int MODE>
__global__ __launch_bounds__(kCeilThreads) void mfma_ceiling_kernel(float* out, int iters) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr bool kRandom = MODE != FA2_ABLATE_CEIL_MFMA_CONST;
  constexpr bool kHalf = MODE == FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC ||
                        MODE == FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE;
  constexpr bool kSm64 = MODE == FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE;
  constexpr bool kVacc = MODE == FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC || kHalf || kSm64;
  constexpr bool kLds = MODE == FA2_ABLATE_CEIL_MFMA_LDS ||
                        MODE == FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX || kVacc;
  constexpr bool kSoftmax = MODE == FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX || kVacc;
  constexpr bool kExp = MODE == FA2_ABLATE_CEIL_MFMA_EXP;
  constexpr bool kFma2 = MODE == FA2_ABLATE_CEIL_MFMA_FMA2;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < kCeilChunks * 256; i += kCeilThreads)
    reinterpret_cast<uint32_t*>(lds)[i] = bf16_pair(i + 4096u * blockIdx.x, kRandom);
  __syncthreads();
  const char FA2_LDS* chunks = (const char FA2_LDS*)lds + lane * 16;
  const uint32_t seed = 1u << 24 | (blockIdx.x * kCeilThreads + threadIdx.x) * 4u;
  u32x4 b = {bf16_pair(seed, kRandom), bf16_pair(seed + 1, kRandom),
             bf16_pair(seed + 2, kRandom), bf16_pair(seed + 3, kRandom)};
  u32x4 a[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = *(const volatile u32x4 FA2_LDS*)(chunks + i * 1024);
  float sv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sv[j] = (float)(mix32(seed + 8 + j) & 0xffffu) * (1.0f / 65536.0f);
  float lsum = 0.f, eprev = 0.f;
  // independent accumulators: two, or four in the half-read modes (a 64-row wave has four S and
  // eight O tiles in flight, and one wave per SIMD must not wait on one MFMA's result)
  constexpr int kAcc = kHalf ? 4 : 2;
  f32x16 acc[4] = {};
  // 2 wait states between the vector writes of the accumulators and b and the first asm MFMA
  if constexpr (kVacc)
    asm volatile("s_nop 1" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(b));
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      // the operand of MFMA i: a[i & 3], or a[(i >> 1) & 3] when every read feeds two MFMAs
      constexpr int kShift = kHalf ? 1 : 0;
      const int ai = (i >> kShift) & 3;
      if constexpr (kVacc) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                     : "+v"(acc[i % kAcc])
                     : "v"(a[ai]), "v"(b));
      } else {
        acc[i % kAcc] = Elem<1>::mma(a[ai], b, acc[i % kAcc]);
      }
      // the read for the operand four ahead, into the register just consumed (after its last
      // MFMA)
      if constexpr (kLds) {
        if (!kHalf || (i & 1))
          a[ai] = *(const volatile u32x4 FA2_LDS*)(chunks + (((i >> kShift) + 4) & 15) * 1024);
      }
      if constexpr (kSm64) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i & 7], 0.0625f, -4.0f));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[(i + 4) & 7], 0.0625f, -4.0f));
        sv[i & 7] = e0;
        sv[(i + 4) & 7] = e1;
        lsum = Elem<1>::sum2(Elem<1>::pack2(e0, e1), lsum);
      } else if constexpr (kSoftmax) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i & 7], 0.0625f, -4.0f));
        sv[i & 7] = e;
        if (i & 1) lsum = Elem<1>::sum2(Elem<1>::pack2(eprev, e), lsum);
        eprev = e;
      }
      if constexpr (kExp) sv[i & 7] = __builtin_amdgcn_exp2f(sv[i & 7] * -1.0f);
      if constexpr (kFma2) {
        sv[i & 7] = __builtin_fmaf(sv[i & 7], 0.9990234375f, 0.0009765625f);
        sv[(i + 4) & 7] = __builtin_fmaf(sv[(i + 4) & 7], 0.9990234375f, 0.0009765625f);
      }
    }
  }
  if constexpr (kVacc)
    asm volatile("s_nop 7\n\ts_nop 3" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
  f32x16 s = acc[0] + acc[1];
  if constexpr (kAcc == 4) s += acc[2] + acc[3];
  float t = lsum;
  if constexpr (kExp || kFma2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) t += sv[j];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) t += s[i];
  out[(size_t)blockIdx.x * kCeilThreads + threadIdx.x] = t;
}

template <int MODE>
int launch_ceiling(float* out, int workgroups, int iters, hipStream_t s) {
  // 128 KiB leaves room for one workgroup per CU (160 KiB of LDS)
  // (48 KiB: three per CU)
  constexpr size_t lds = MODE == FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE ? 2 * kCeilLdsBytes
                         : MODE == FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE ? 48 * 1024
                                                                             : kCeilLdsBytes;
  hipLaunchKernelGGL(mfma_ceiling_kernel<MODE>, dim3(workgroups), dim3(kCeilThreads), lds, s,
                     out, iters);
  return (int)hipGetLastError();
}

__global__ __launch_bounds__(kCeilThreads) void hbm_read_kernel(const u32x4* src, int64_t n16,
                                                                uint32_t* out) {
  const int64_t stride = (int64_t)gridDim.x * kCeilThreads;
  int64_t i = (int64_t)blockIdx.x * kCeilThreads + threadIdx.x;
  u32x4 x = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    x ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) x ^= src[i];
  out[(int64_t)blockIdx.x * kCeilThreads + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

}  // namespace

int launch_hbm_read(const void* src, int64_t n16, uint32_t* out, int workgroups, hipStream_t s) {
  hipLaunchKernelGGL(hbm_read_kernel, dim3(workgroups), dim3(kCeilThreads), 0, s,
                     static_cast<const u32x4*>(src), n16, out);
  return (int)hipGetLastError();
}

int launch_mfma_ceiling(int mode, float* out, int workgroups, int iters, hipStream_t s) {
  switch (mode) {
    case FA2_ABLATE_CEIL_MFMA: return launch_ceiling<FA2_ABLATE_CEIL_MFMA>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_CONST:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_CONST>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_LDS:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_LDS>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_EXP:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_EXP>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_MFMA_FMA2:
      return launch_ceiling<FA2_ABLATE_CEIL_MFMA_FMA2>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC:
      return launch_ceiling<FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE:
      return launch_ceiling<FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE>(out, workgroups, iters, s);
    case FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE:
      return launch_ceiling<FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE>(out, workgroups, iters, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace fa2
