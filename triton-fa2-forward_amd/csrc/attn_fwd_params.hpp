// attn_fwd_params.hpp - argument block of the forward kernel, shared by host and device code.
#pragma once

#include <stdint.h>

namespace fa2 {

// Number of XCDs (each with its own L2) that the hardware deals workgroups to round-robin.
constexpr int kXcds = 8;
// Compute units (8 XCDs x 32). With two workgroups per CU, the dispatcher's first round places
// block b and block b + kCus on the same CU (measured with the hardware CU id).
constexpr int kCus = 256;

// Keys per entry of the key-norm table (attn_key_norm.hip): one workgroup of the key-norm pass
// each (C3: 1024 workgroups), and at most three entries per 128-row causal program's own rows.
constexpr int kKeyChunk = 64;

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
  // Causal grids whose (batch, kv head) units split evenly over the XCDs: each XCD runs its
  // units unit_chunk at a time (a divisor of its unit count), q-tile-major inside a chunk.
  int32_t unit_chunk;
  // Dynamic tail (causal grids; the host's tail_schedule): the workgroups from static_blocks on
  // each take one ticket from *tickets with an agent-scope atomic increment that wraps at
  // tail_wgs - 1, so that the word is zero again once the launch has run. Ticket t below
  // tail_programs runs program static_blocks + t of the static order; the others exit at once.
  // No tail: static_blocks = INT32_MAX (read beside the grid fields, so that the check costs the
  // prologue no load of its own) and workgroup b runs program b.
  int32_t static_blocks;
  int32_t tail_wgs;
  int32_t tail_programs;
  float qk_scale;   // sm_scale * log2(e)
  // Optional outputs beyond the reference's:
  float* lse;        // [B, H_q, N_q] natural-log log-sum-exp of the scaled scores, or null;
                     // when set, the kernel also sums the unrounded P (part_lse_exact)
  // Split-KV: the key range of every program is cut into `splits` pieces of `split_tiles`
  // K/V tiles, one workgroup each; each writes its normalised partial output and base-2
  // log-sum-exp, which a combine pass merges (splits == 1: the kernel writes o itself).
  float* part_o;     // [splits][B * H_q * N_q][D] fp32
  float* part_lse;   // [splits][B * H_q * N_q] fp32, base 2, of the weights part_o is
                     // normalised by (P rounded to the input type): the merge weights
  float* part_lse_exact;  // the same of the unrounded P (written when lse is requested)
  int64_t part_rows; // B * H_q * N_q
  int32_t splits;
  int32_t split_tiles;
  // Optional key-norm table (null: off), written by the key-norm pass before the kernel: for
  // every (batch, kv head) and every kKeyChunk keys, the largest squared norm of a key. With
  // it a wave can prove after its first tile that no later score exceeds its reference max by
  // more than kBoundTau (Cauchy-Schwarz) and then skips the per-tile row max.
  const float* key_norm2;  // [B * H_kv][key_chunks]
  int32_t key_chunks;      // ceil(n_kv / kKeyChunk)
  uint32_t* tickets;  // the tail's ticket word (read only past static_blocks)
  // Measurement library only (the timeline variant): kTimelineWords uint64 per program,
  // indexed by the program's place in the static order. Null, and never read, in the product's
  // instances.
  uint64_t* timeline;
};

// Words per workgroup of the timeline variant: entry, prologue done (first barrier), tile loop
// done, stores done (s_memrealtime, 100 MHz), the workgroup's K/V tile count, and its hardware
// ids (XCC_ID << 32 | HW_ID).
constexpr int kTimelineWords = 6;

// Arguments of the key-norm pass (attn_key_norm.hip).
struct KeyNormParams {
  const uint16_t* k;
  int64_t skb, skh, skn;
  int32_t h_kv, n_kv, chunks;
  float* out;  // [B * h_kv][chunks]
};

// Arguments of the split-KV combine pass: rows are the [B, H_q, N_q] rows of the output.
struct CombineParams {
  const float* part_o;    // [splits][rows][D]
  const float* part_lse;  // [splits][rows], base 2: merge weights
  const float* part_lse_exact;  // [splits][rows], base 2: the log-sum-exp output (lse != null)
  uint16_t* o;
  float* lse;             // optional natural-log log-sum-exp [rows]
  int64_t sob, soh, son;
  int64_t rows;
  int32_t h_q, n_q, splits;
};

}  // namespace fa2
