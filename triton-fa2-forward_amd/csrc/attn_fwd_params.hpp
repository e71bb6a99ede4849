// attn_fwd_params.hpp - argument block of the forward kernel, shared by host and device code.
#pragma once

#include <stdint.h>

namespace fa2 {

// Kernel arguments: the reference's launch arguments (fa2/kernel.py:248-259) with the
// d strides dropped (they must be 1) and the grid decomposition precomputed.
struct Params {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t sqb, sqh, sqn;
  int64_t skb, skh, skn;
  int64_t svb, svh, svn;
  int64_t sob, soh, son;
  int32_t h_q, n_q, n_kv;
  int32_t group;    // h_q / h_kv
  int32_t pack;     // query heads per program: 1 or group
  int32_t block_m;  // (position, head) rows per program
  int32_t n_tiles;  // programs along the packed rows: ceil(n_q * pack / block_m)
  int32_t n_bh;     // programs along batch x head groups: batch * h_q / pack
  float qk_scale;   // sm_scale * log2(e)
};

}  // namespace fa2
