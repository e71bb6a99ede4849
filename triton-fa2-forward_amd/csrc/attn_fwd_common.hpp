// attn_fwd_common.hpp - types and device helpers shared by the forward kernels:
// the MFMA / conversion traits per element type, the LDS swizzle keys, lane-pair reductions,
// the transposing LDS read and the HBM -> LDS buffer loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_fwd_params.hpp"

namespace fa2 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

#define FA2_LDS __attribute__((address_space(3)))
#define FA2_GLOBAL __attribute__((address_space(1)))

// Lazy-rescale threshold in exp2 units: the reference max lags the true max by at most this.
constexpr float kRescaleTau = 8.0f;
// Score bound from key norms: a wave whose rows all satisfy |q| |k|max qk_scale <= m + tau after
// their first tile never moves its reference max again, so it skips the row max. P <= 2^tau then:
// 2^15 stays inside fp16's range (65504); bf16 has fp32's exponent range, so 2^32 is safe there
// and l and O stay far from fp32 overflow (l <= 2^32 per key).
template <int DT>
constexpr float kBoundTau = DT == 1 ? 32.0f : 15.0f;
// A row whose bound exceeds m + tau by at most this much skips too: its reference is raised by
// the next whole number (to bound - tau or just above it) before its first P, so P <= 2^tau
// still holds and the row's largest P is at least 2^-lift. A whole number scales every P by an
// exact power of two, so P's rounding to the input type is unchanged (a row of one key still
// gets its value exactly) until fp16's subnormal range, which then starts up to 4 binades nearer
// the row's largest P (keys there are rounded to 2^-25 absolute instead of 2^-29 of it); bf16
// has fp32's exponent range. Compile-time switch FA2_BOUND_LIFT (1 on, 0 off) so that an A/B of
// two builds can compare them (ab.py).
#ifndef FA2_BOUND_LIFT
#define FA2_BOUND_LIFT 1
#endif
#ifndef FA2_BOUND_LIFT_F16
#define FA2_BOUND_LIFT_F16 4
#endif
template <int DT>
constexpr float kBoundLift = FA2_BOUND_LIFT ? (DT == 1 ? 8.0f : (float)FA2_BOUND_LIFT_F16) : 0.0f;
// ... and only rows whose bound is at most this: every score of the row lies in [-bound, bound],
// and a lifted reference is at most bound - tau + 1, so P >= 2^(-2 bound + tau - 1) >= 2^-24,
// fp16's smallest subnormal: no key's weight vanishes that the unlifted row would keep.
template <int DT>
constexpr float kBoundLiftMax = DT == 1 ? INFINITY : (kBoundTau<DT> + 23.0f) / 2.0f;
// qk_scale raised by 2^-10: covers the fp32 rounding of the squared norms and of the MFMA's
// score sums (at most ~2^-17 relative at head_dim 128) in the bound |q| |k|max qk_scale.
__host__ __device__ constexpr float qk_scale_bound(float qk_scale) {
  return qk_scale * (1.0f + 1.0f / 1024.0f);
}
// ln 2: a base-2 log-sum-exp times this is the natural one
constexpr float kLn2 = 0.6931471805599453f;
// Kernel variant bits (attn_fwd_kernel's VARIANT; FA2_VARIANT_* in the C ABI)
constexpr int kVariantScaleFirst = 1;
constexpr int kVariantMaskEveryTile = 2;
// Not a timing variant: the instance that reads the key-norm table and skips the row max where
// the table proves it unneeded (launched by the production path when a table was written).
constexpr int kVariantKeyBound = 4;
// Work-skipping knockouts, built only into the measurement library (fa2_ablate.hip), never into
// the product: the reference's ablation switches that remove one kind of work so that its cost is
// the time difference (bench/ablation.py:6-10). Their outputs are wrong by design.
constexpr int kVariantNoExp = 8;       // exp2 replaced by its argument (alpha too)
constexpr int kVariantNoSoftmax = 16;  // no mask, row max, exp, sum or rescale: O = (Q K^T) V
constexpr int kVariantKvL2 = 32;       // every tile loads the first K/V tile again (L2 hits)
// K/V tiles from the third on are not loaded: every tile's products read whichever of the first
// two tiles its LDS buffer holds. What staging K/V through LDS costs beyond the first tiles.
constexpr int kVariantNoKvStaging = 256;
// Measurement library only, and computes attention (in another summation order): twice the waves
// per workgroup, in two groups that take the two halves of each program's key range with K/V
// buffers of their own, and merge through LDS (one workgroup per CU).
constexpr int kVariantSplitKeys = 512;
// A program's fixed cost, knocked out: Q is not loaded (a lane pattern in its place), or the
// output is not stored (the accumulators only kept alive). What hiding a program's Q load or its
// store behind another program's tiles could gain at most. Outputs wrong by design.
constexpr int kVariantNoQLoad = 1024;
constexpr int kVariantNoStore = 2048;
// Measurement library only, and computes the product's attention: every workgroup also records
// its timeline (Params::timeline, kTimelineWords words); waits for its stores before the last stamp.
constexpr int kVariantTimeline = 64;
// s_getreg operands (register id | offset << 6 | (size - 1) << 11) of the whole 32-bit HW_ID
// register (id 4: wave, SIMD, CU, shader array and engine of the wave) and XCC_ID (id 20).
constexpr int kHwregHwId = 4 | (31 << 11);
constexpr int kHwregXccId = 20 | (31 << 11);

// ---------------------------------------------------------------------------------
// element type traits: the MFMA, the fp32 -> 16-bit pair conversion (RNE) and the fp32 sum of
// a converted pair
// ---------------------------------------------------------------------------------
template <int DT>
struct Elem;

template <>
struct Elem<0> {  // fp16
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + lo + hi of a packed pair, in fp32 (v_dot2c_f32_f16 against (1, 1))
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair),
                                  __builtin_bit_cast(f16x2, 0x3c003c00u), acc, false);
  }
  // acc + lo^2 + hi^2 of a packed pair, in fp32
  static __device__ __forceinline__ float sumsq2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), __builtin_bit_cast(f16x2, pair),
                                  acc, false);
  }
};

template <>
struct Elem<1> {  // bf16
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + lo + hi of a packed pair, in fp32 (v_dot2c_f32_bf16 against (1, 1))
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                           __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
  }
  // acc + lo^2 + hi^2 of a packed pair, in fp32
  static __device__ __forceinline__ float sumsq2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                           __builtin_bit_cast(bf16x2, pair), acc, false);
  }
};

// ---------------------------------------------------------------------------------
// index helpers
// ---------------------------------------------------------------------------------

// Swap bits 2 and 3 of a row index inside a 32-row block (an involution).
__device__ __forceinline__ constexpr int pi_row(int x) {
  return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1);
}

// XOR key of the K tile's 16-byte chunks. u = pi_row(row % 32) % 16, i.e. the lane index
// (mod 16) that reads this row. Chosen (exhaustive search over linear keys) so that the
// b128 A-operand reads are conflict-free for 32- and 64-bank LDS models.
template <int D>
__device__ __forceinline__ int k_key(int u) {
  if constexpr (D == 128) {
    return u & 15;
  } else if constexpr (D == 64) {
    return ((u >> 1) & 1) | (((u >> 2) & 1) << 1) | (((u ^ (u >> 3)) & 1) << 2);
  } else if constexpr (D == 32) {
    return ((u >> 2) & 1) | ((((u >> 1) ^ (u >> 3)) & 1) << 1);
  } else {
    return (u >> 2) & 1;
  }
}

// XOR key of the V tile's 16-byte chunks, a function of the key row (mod 16); makes the
// ds_read_b64_tr_b16 reads conflict-free for 32- and 64-bank LDS models.
template <int D>
__device__ __forceinline__ int v_key(int row) {
  if constexpr (D == 128) {
    return ((row & 1) << 1) | ((row & 2) << 1) | ((row & 1) << 3);
  } else if constexpr (D == 64) {
    return ((row & 1) << 1) | ((row & 2) << 1);
  } else if constexpr (D == 32) {
    return row & 2;
  } else {
    return 0;
  }
}

// max / sum of a value over the lane pair (l, l^32)
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// This lane's sum of a score tile (16 values per 32-key block), in index order. It starts from
// the first value, not from 0.0f: 0 + x cannot be folded (it turns -0 into +0), so a zero start
// costs one more add per tile; the sum is the same.
template <int NB>
__device__ __forceinline__ float lane_sum(const f32x16 (&s)[NB]) {
  float r = s[0][0];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = (nb == 0 ? 1 : 0); i < 16; ++i) r += s[nb][i];
  return r;
}

__device__ __forceinline__ u32x2 lds_read_tr(const char FA2_LDS* p) {
  i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 FA2_LDS*)p);
  return __builtin_bit_cast(u32x2, v);
}

// A raw buffer resource (gfx9 layout) over [base, base + bytes): loads past `bytes` return
// zeros. Built from wave-uniform values, so it lives in SGPRs.
__device__ __forceinline__ u32x4 make_desc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  auto uniform = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
  return u32x4{uniform((uint32_t)a), uniform((uint32_t)(a >> 32) & 0xffffu), uniform(bytes),
               0x00020000u};
}

// LDS byte address of a __shared__ object, as a wave-uniform value.
__device__ __forceinline__ uint32_t lds_addr(const FA2_LDS void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// 16 bytes HBM -> LDS without VGPRs: lane l of the wave writes lds_base + 16 * l
// (buffer_load_dwordx4 ... lds, LDS destination in M0). Issued as inline asm on purpose: the
// compiler's own LDS-DMA intrinsic makes it wait for every DMA in flight before the next LDS
// read of any buffer (it cannot prove the double buffers apart), which serialises the
// prefetch. Callers wait with wait_vmcnt<N>() before a barrier instead. The LDS address is an
// operand bound to M0 ("{m0}"): the compiler itself writes M0 before the asm and knows it is
// read there (M0 is a reserved register, so a clobber of it would not be honoured).
__device__ __forceinline__ void load_lds16(u32x4 desc, uint32_t voffset, uint32_t lds_base) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voffset), "s"(desc), "{m0}"(lds_base)
               : "memory");
}

// s_waitcnt vmcnt(N), leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace fa2
