// attn_fwd_combine.hip - merges the partial outputs of a split-KV launch.
//
// Split s of a row saw keys K_s and wrote O_s = sum_{n in K_s} p_n v_n / l_s (fp32) and
// lse_s = log2 l_s, with p_n = exp2(s_n * qk_scale) rounded to the input type and l_s their sum
// (the weights the kernel normalises by). With L = max_s lse_s and w_s = exp2(lse_s - L),
//   O = sum_s w_s O_s / sum_s w_s,
// the same online-softmax merge the kernel applies tile by tile (fa2/kernel.py:95-105), applied
// once across splits; it equals the single-pass result up to rounding. The log-sum-exp output
// merges the splits' exact (unrounded) lse the same way: L' + log2 sum_s exp2(lse'_s - L').
// Memory-bound: each thread merges 4 dims of one row (16-byte loads).
#include <hip/hip_runtime.h>

#include "attn_fwd_common.hpp"
#include "attn_fwd_launch.hpp"

namespace fa2 {

namespace {

// Latency-bound at the sizes split-KV is for (the few-queries table merges 0.5 MiB): all of a
// thread's loads are issued before any arithmetic, unrolled over the largest split count with a
// uniform guard, instead of one load round per split. Measured 4.67 -> 4.46 us on the few-queries
// shape (N_q 1, 2 splits); the rest is the launch and one trip to memory.
constexpr int kCombineMaxSplits = 16;  // fa2_attn_fwd_ex accepts at most 16 splits

template <int DT, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const CombineParams c) {
  using E = Elem<DT>;
  constexpr int TPR = D / 4;  // threads per row
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t / TPR;
  if (row >= c.rows) return;
  const int d0 = (int)(t - row * TPR) * 4;
  const bool want_lse = c.lse && d0 == 0;
  float lse[kCombineMaxSplits], lsx[kCombineMaxSplits];
  f32x4 x[kCombineMaxSplits];
#pragma unroll
  for (int s = 0; s < kCombineMaxSplits; ++s) {
    if (s < c.splits) {
      lse[s] = c.part_lse[s * c.rows + row];
      x[s] = *(const f32x4*)(c.part_o + (s * c.rows + row) * D + d0);
      if (want_lse) lsx[s] = c.part_lse_exact[s * c.rows + row];
    }
  }
  float L = -INFINITY;
#pragma unroll
  for (int s = 0; s < kCombineMaxSplits; ++s)
    if (s < c.splits) L = fmaxf(L, lse[s]);
  float wsum = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kCombineMaxSplits; ++s) {
    if (s < c.splits) {
      const float w = exp2f(lse[s] - L);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = __builtin_fmaf(w, x[s][i], o[i]);
      wsum += w;
    }
  }
  const int64_t bh = row / c.n_q;
  const int pos = (int)(row - bh * c.n_q);
  const int64_t b = bh / c.h_q;
  const int head = (int)(bh - b * c.h_q);
  uint16_t* orow = c.o + b * c.sob + head * c.soh + pos * c.son + d0;
  const float inv = 1.0f / wsum;
  *(u32x2*)orow = u32x2{E::pack2(o[0] * inv, o[1] * inv), E::pack2(o[2] * inv, o[3] * inv)};
  if (want_lse) {
    float Lx = -INFINITY;
#pragma unroll
    for (int s = 0; s < kCombineMaxSplits; ++s)
      if (s < c.splits) Lx = fmaxf(Lx, lsx[s]);
    float sx = 0.f;
#pragma unroll
    for (int s = 0; s < kCombineMaxSplits; ++s)
      if (s < c.splits) sx += exp2f(lsx[s] - Lx);
    c.lse[row] = (Lx + log2f(sx)) * kLn2;
  }
}

template <int DT, int D>
int launch_d(const CombineParams& c, hipStream_t s) {
  const int64_t threads = c.rows * (D / 4);
  const unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL((attn_combine_kernel<DT, D>), dim3(grid), dim3(256), 0, s, c);
  return (int)hipGetLastError();
}

}  // namespace

int launch_combine(int dtype, int head_dim, const CombineParams& c, hipStream_t s) {
  switch (dtype * 4 + (head_dim == 16 ? 0 : head_dim == 32 ? 1 : head_dim == 64 ? 2 : 3)) {
    case 0: return launch_d<0, 16>(c, s);
    case 1: return launch_d<0, 32>(c, s);
    case 2: return launch_d<0, 64>(c, s);
    case 3: return launch_d<0, 128>(c, s);
    case 4: return launch_d<1, 16>(c, s);
    case 5: return launch_d<1, 32>(c, s);
    case 6: return launch_d<1, 64>(c, s);
    default: return launch_d<1, 128>(c, s);
  }
}

}  // namespace fa2
