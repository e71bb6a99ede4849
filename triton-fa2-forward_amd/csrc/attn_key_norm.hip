// attn_key_norm.hip - the key-norm pass: for every (batch, kv head) and every kKeyChunk keys,
// the largest squared Euclidean norm of a key, in fp32.
//
// The forward kernel uses it to bound its scores: |q . k| <= |q| |k| (Cauchy-Schwarz), so a
// row whose first tile gave it the reference max m, and for which |q| max|k| qk_scale <= m + tau,
// can never see a later score above m + tau. A wave whose rows all pass skips the per-tile row
// max from then on. One pass over K: memory-bound, ~K bytes / HBM rate.
#include <hip/hip_runtime.h>

#include "attn_fwd_common.hpp"
#include "attn_fwd_launch.hpp"

namespace fa2 {

namespace {

// One workgroup per (batch, kv head, chunk of kKeyChunk keys), 256 threads. CPR lanes read one
// key row (16 bytes each, consecutive), so a wave covers 64 / CPR rows per load instruction.
template <int DT, int D>
__global__ __launch_bounds__(256) void key_norm_kernel(const KeyNormParams k) {
  using E = Elem<DT>;
  constexpr int CPR = D / 8;             // 16-byte pieces per key row
  constexpr int ROWS = 256 / CPR;        // rows per pass of the workgroup
  constexpr int PASSES = (kKeyChunk + ROWS - 1) / ROWS;
  const int chunk = (int)(blockIdx.x % (unsigned)k.chunks);
  const int bh = (int)(blockIdx.x / (unsigned)k.chunks);
  const int b = bh / k.h_kv, h = bh - b * k.h_kv;
  const int tid = threadIdx.x;
  const int row0 = tid / CPR, col = tid % CPR;
  const uint16_t* base = k.k + b * k.skb + h * k.skh + col * 8;
  float mx = 0.f;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    const int r = pass * ROWS + row0;  // row inside the chunk
    const int n = chunk * kKeyChunk + r;
    float s = 0.f;
    if (r < kKeyChunk && n < k.n_kv) {
      const u32x4 x = *(const u32x4*)(base + (int64_t)n * k.skn);
      s = E::sumsq2(x[0], s);
      s = E::sumsq2(x[1], s);
      s = E::sumsq2(x[2], s);
      s = E::sumsq2(x[3], s);
    }
    // the CPR lanes of one row are consecutive and CPR-aligned: xor offsets below CPR stay inside
#pragma unroll
    for (int off = CPR / 2; off >= 1; off /= 2) s += __shfl_xor(s, off, 64);
    mx = fmaxf(mx, s);
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  __shared__ float red[4];
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) k.out[(int64_t)bh * k.chunks + chunk] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int DT, int D>
int launch_d(const KeyNormParams& k, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((key_norm_kernel<DT, D>), dim3(grid), dim3(256), 0, s, k);
  return (int)hipGetLastError();
}

}  // namespace

int launch_key_norm(int dtype, int head_dim, const KeyNormParams& k, unsigned grid,
                    hipStream_t s) {
  switch (dtype * 4 + (head_dim == 16 ? 0 : head_dim == 32 ? 1 : head_dim == 64 ? 2 : 3)) {
    case 0: return launch_d<0, 16>(k, grid, s);
    case 1: return launch_d<0, 32>(k, grid, s);
    case 2: return launch_d<0, 64>(k, grid, s);
    case 3: return launch_d<0, 128>(k, grid, s);
    case 4: return launch_d<1, 16>(k, grid, s);
    case 5: return launch_d<1, 32>(k, grid, s);
    case 6: return launch_d<1, 64>(k, grid, s);
    default: return launch_d<1, 128>(k, grid, s);
  }
}

}  // namespace fa2
