// attn_fwd_params.hpp - argument block of the forward kernel, shared by host and device code.
#pragma once

#include <stdint.h>

namespace fa2 {

// The topology the program order is tuned on (MI355X): 8 XCDs, each with its own L2, that the
// hardware deals workgroups to round-robin (block b runs on XCD b % 8), and 256 CUs. With two
// workgroups per CU, the dispatcher's first round places block b and block b + 256 on the same
// CU (measured with the hardware CU id). The host reads the real counts from the device and
// passes them in Params (xcd_shift, cus); other counts get the same order rules with their own
// numbers (attn_fwd_schedule.hpp).
constexpr int kXcds = 8;
constexpr int kCus = 256;
// Largest XCD count the XCD-aware order and the per-XCD tail queues serve; a device that reports
// more, or a count that is not a power of two, is ordered as one XCD.
constexpr int kMaxXcds = 16;

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
  // Topology of the device the launch runs on: log2 of its XCD count (a power of two, at most
  // kMaxXcds) and its CU count. They drive program_of's order only, never a result.
  int32_t xcd_shift;
  int32_t cus;
  // Dynamic tail (causal grids; the host's tail_schedule, attn_fwd_schedule.hpp): the workgroups
  // from static_blocks on are dealt the last programs of the static order at run time through the
  // ticket words at *tickets. Tail workgroup w belongs to queue w % tail_queues (its XCD: block b
  // runs on XCD b % 8). It first takes a ticket from its queue's word; ticket t below
  // tail_private runs its XCD's program static_blocks + t * tail_queues + queue (locality: that
  // XCD's L2 holds the unit's K/V). Otherwise it takes a ticket u from the shared word; u below
  // tail_shared runs program static_blocks + tail_queues * tail_private + u, whichever XCD asks
  // (balance: a fast XCD takes more of them); the rest exit at once. Every word is incremented
  // by a fixed number of workgroups per launch (tail_wgs / tail_queues for a queue, the rest for
  // the shared word) and wraps there, so it is zero again when the launch ends.
  // No tail: static_blocks = INT32_MAX (read beside the grid fields, so that the check costs the
  // prologue no load of its own) and workgroup b runs program b.
  int32_t static_blocks;
  int32_t tail_wgs;
  int32_t tail_queues;
  int32_t tail_private;  // programs per queue
  int32_t tail_shared;   // programs in the shared pool
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
  // The tail's ticket words (read only past static_blocks): the shared word at tickets[0], queue
  // x's at tickets[(1 + x) * kTicketStride].
  uint32_t* tickets;
  // Measurement library only (the timeline variant): kTimelineWords uint64 per program,
  // indexed by the program's place in the static order. Null, and never read, in the product's
  // instances.
  uint64_t* timeline;
};

// uint32 words between two ticket words of a launch: each on its own 64-byte line.
constexpr int kTicketStride = 16;
// Ticket words per launch: the shared word and one per XCD queue.
constexpr int kTicketWordsPerSet = 1 + kMaxXcds;

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
