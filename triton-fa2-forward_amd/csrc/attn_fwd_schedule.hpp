// attn_fwd_schedule.hpp - which program each workgroup of a forward launch runs: the static
// order (program_of), the host's unit chunk and dynamic-tail policy, and the tail's ticket ->
// program rules. Everything the kernel evaluates here is __host__ __device__, so that the
// measurement library can run the very same arithmetic on the CPU (fa2_ablate_program_map) and a
// CPU test can check, over thousands of launch shapes, that every program runs exactly once.
//
// The reference's grid is (q tile, batch x head group) with program (pid0, pid1)
// (fa2/kernel.py:24-26, 126-132); every program is computed alone, so any order of them gives the
// same output bit for bit. The order below only decides which XCD's L2 holds which K/V and when
// the heavy causal programs start.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_fwd_params.hpp"

#define FA2_HD __host__ __device__ __forceinline__

// 1: causal grids of at most two programs per CU in the XCD-aware order reverse the second
// program of every CU, as grids of at most three in the fallback order do (below); 0: only the
// fallback order does.
// Compile-time so that an A/B of two builds can compare them (ab.py).
#ifndef FA2_XCD_REVERSE
#define FA2_XCD_REVERSE 1
#endif
// 1: the fallback order reverses the second program of every CU on causal grids of at most three
// programs per CU (below); 0: it does not. Compile-time, for ab.py.
#ifndef FA2_FALLBACK_REVERSE
#define FA2_FALLBACK_REVERSE 1
#endif

namespace fa2 {

FA2_HD int sched_min(int a, int b) { return a < b ? a : b; }

// The workgroup -> (q tile, batch, first query head) decomposition. Workgroups are dealt to
// the XCDs round-robin; block b runs on XCD b % xcds.
//   * When the (batch, kv head) units split evenly over the XCDs, each XCD owns a fixed set of
//     whole units, so its L2 holds the K/V of the heads it works on (C3: HBM reads fell from
//     635 to 139 MiB per launch). Causal: inside an XCD the order is q tile outermost (heaviest
//     tile first) across all of its units, then unit, then the query-head groups sharing a KV
//     head. Unit after unit instead started the last unit's heaviest tiles late and left the
//     XCD's slots 22% idle on C2 (8 units per XCD): the q-tile-major order runs C2 12% faster,
//     although its L2 now misses more (reads past L2 192 -> ~680 MiB per launch, ~2.6 TB/s).
//     The XCD's units are taken unit_chunk at a time (the host's choice, a divisor of its unit
//     count), q-tile-major inside each chunk: heavy tiles first, and the programs in flight read
//     the K/V of a few units instead of all of the XCD's.
//     Non-causal programs all do the same work, so there the order is unit after unit: the
//     programs in flight on an XCD then share one unit's K/V in its L2 (C4: four units per XCD
//     read K/V 8.3x over in q-tile-major order).
//   * Otherwise a fixed unit set per XCD would hand one XCD more of the heavy causal tiles than
//     another (C5, 12 units over 8 XCDs: 15% more work on XCD 0). Then the order is q tile
//     outermost over all units, heaviest first, and the round-robin dealing balances the XCDs.
//     On causal grids of at most three programs per CU the first round decides the span, and
//     heaviest-first hands each CU two of the heaviest programs. There the second program of
//     every CU (blocks cus .. 2 cus - 1) is taken in reverse, so the heaviest programs share
//     their CU with the lightest of the first round: +2.6% on C5 (672 programs), +6% on its
//     head_dim-64 twin, +3.6% at 384 programs; from 896 programs on it no longer pays (+0.7%,
//     -1.1% at 1344). The hardware fills every CU's first slot before any second one, so the
//     blocks b and b + cus meet on one CU (the timelines show it).
//   * The same holds inside each XCD of the XCD-aware causal order: its programs are dealt to
//     the XCD's CUs a slot at a time (XCD-local slots s and s + CUs per XCD meet on one CU), and
//     q-tile-major order puts tile t beside tile t - (CUs per XCD) / (programs per q tile). On an
//     XCD holding at most two programs per CU its second slots are taken in reverse too. Measured
//     on MI355X against the plain order (same box, interleaved builds): B1 H32/8 N2048 D128 +4.4%
//     (bf16) and +4.3% (fp16), N1536 +3.1%, B2 H16 N2048 +4.3%, B4 H16 N1024 +3.4%, B1 H16
//     N4096 +4.5%, fp16 head_dim 64 B1 H32/8 N2048 +2.9% and H24/8 +1.2%; from 2.5 programs per
//     CU to 3 it did not pay (-1.1% to +0.2%), hence the bound of two.
struct Program {
  int tile, b, hq0, hkv;
};

template <bool CAUSAL>
FA2_HD Program program_of(const Params& p, int block) {
  const int progs_per_kv = p.group / p.pack;  // programs sharing one KV head per q tile
  const int h_kv = p.h_q / p.group;
  const int units = p.n_bh / progs_per_kv;    // batch * h_kv
  const int xcds = 1 << p.xcd_shift;
  int kv_index, t, h_in;
  if ((units & (xcds - 1)) == 0) {
    const int xcd = block & (xcds - 1), slot0 = block >> p.xcd_shift;
    const int upx = units >> p.xcd_shift;      // units per XCD
    if (CAUSAL) {
      const int cu = (p.unit_chunk > 0 && upx % p.unit_chunk == 0) ? p.unit_chunk : upx;
      const int per_chunk = cu * progs_per_kv * p.n_tiles;  // programs of one chunk
      int slot = slot0;
      if (FA2_XCD_REVERSE) {
        const int cpx = p.cus >> p.xcd_shift;  // CUs per XCD
        const int per_xcd = upx * progs_per_kv * p.n_tiles;
        if (per_xcd <= 2 * cpx && slot >= cpx) slot = cpx + (per_xcd - 1 - slot);
      }
      const int ch = slot / per_chunk;
      const int rs = slot - ch * per_chunk;
      const int per_t = cu * progs_per_kv;     // programs per q tile of one chunk
      t = rs / per_t;
      const int r = rs - t * per_t;
      kv_index = xcd * upx + ch * cu + r / progs_per_kv;  // b * h_kv + hkv
      h_in = r % progs_per_kv;
    } else {
      const int per_u = p.n_tiles * progs_per_kv;  // programs of one unit
      const int u = slot0 / per_u;
      const int r = slot0 - u * per_u;
      t = r / progs_per_kv;
      h_in = r - t * progs_per_kv;
      kv_index = xcd * upx + u;
    }
  } else {
    const int grid = p.n_tiles * p.n_bh;
    if (FA2_FALLBACK_REVERSE && CAUSAL && grid <= 3 * p.cus && block >= p.cus) {
      const int end = sched_min(grid, 2 * p.cus);
      if (block < end) block = p.cus + (end - 1 - block);
    }
    t = block / p.n_bh;
    const int r = block - t * p.n_bh;
    kv_index = r / progs_per_kv;
    h_in = r - kv_index * progs_per_kv;
  }
  Program pr;
  pr.tile = CAUSAL ? p.n_tiles - 1 - t : t;
  pr.b = kv_index / h_kv;
  pr.hkv = kv_index - pr.b * h_kv;
  pr.hq0 = pr.hkv * p.group + h_in * p.pack;
  return pr;
}

// ---- the dynamic tail's ticket -> program rules (Params: static_blocks .. tail_shared)

// The queue of tail workgroup `block` (>= static_blocks): its XCD, as static_blocks is a
// multiple of tail_queues.
FA2_HD int tail_queue_of(const Params& p, int block) {
  return (block - p.static_blocks) & (p.tail_queues - 1);
}
// Tail workgroups per queue word, and those that go on to the shared word.
FA2_HD uint32_t tail_queue_wgs(const Params& p) { return (uint32_t)(p.tail_wgs / p.tail_queues); }
FA2_HD uint32_t tail_shared_wgs(const Params& p) {
  return (uint32_t)(p.tail_wgs - p.tail_queues * p.tail_private);
}
// Private ticket t of queue x: the block of that XCD's program, or -1 (go to the shared word).
FA2_HD int tail_private_block(const Params& p, int x, uint32_t t) {
  return t < (uint32_t)p.tail_private ? p.static_blocks + (int)t * p.tail_queues + x : -1;
}
// Shared ticket u: the block of the program, or -1 (nothing left: exit).
FA2_HD int tail_shared_block(const Params& p, uint32_t u) {
  return u < (uint32_t)p.tail_shared ? p.static_blocks + p.tail_queues * p.tail_private + (int)u
                                     : -1;
}

// The program a tail workgroup runs: one ticket from its queue's word and, when that queue has
// none left for it, one from the shared word. inc(word, limit) is the wrapping increment of ticket
// word `word` (0: shared, 1 + x: queue x) that returns the old value: the kernel's agent-scope
// atomic, or the measurement library's CPU emulation of it. Each word is incremented by a fixed
// number of workgroups per launch and wraps there, so it is zero again when the launch ends.
// Returns the block whose program to run, or -1.
template <class Inc>
FA2_HD int tail_pick(const Params& p, int block, Inc&& inc) {
  if (p.tail_private > 0) {
    const int x = tail_queue_of(p, block);
    const uint32_t t = inc(1 + x, tail_queue_wgs(p) - 1u);
    const int b = tail_private_block(p, x, t);
    if (b >= 0) return b;
  }
  const uint32_t u = inc(0, tail_shared_wgs(p) - 1u);
  return tail_shared_block(p, u);
}

}  // namespace fa2

#undef FA2_HD
