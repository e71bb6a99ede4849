// attn_fwd_host.hpp - host side of one forward launch: the argument checks (fa2/kernel.py:218-244
// restated for a C caller), the workspace layout and key-norm policy, the grid, and the launch
// sequence (key-norm pass, attention kernel, split-KV merge). Shared by the library
// (fa2_fwd.hip) and the measurement library (fa2_ablate.hip); everything here has internal
// linkage, so each library compiles its own copy with its own error string.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <utility>

#include "attn_fwd_launch.hpp"
#include "fa2_fwd.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

using fa2::Params;

constexpr int kDims[4] = {16, 32, 64, 128};
// 128 rows x stride x 2 bytes must stay below 2^31.
constexpr int64_t kMaxRowStride = int64_t(1) << 22;
// Longest sequence: key and query positions stay 32-bit in the kernel with two 128-key tiles
// of headroom (INT32_MAX - 256).
constexpr int32_t kMaxSeq = 0x7fffffff - 256;

int dim_index(int d) {
  for (int i = 0; i < 4; ++i)
    if (kDims[i] == d) return i;
  return -1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

using fa2::default_block_n;

// block_n request -> the K/V tile width the kernels are built for (0 = the default)
int tile_n(int block_n, int head_dim) {
  const int req = block_n ? block_n : default_block_n(head_dim);
  return req <= 32 ? 32 : req <= 64 ? 64 : 128;
}

// Split-KV limits: at most 16 splits, and a split of fewer than 4 K/V tiles is not worth a
// workgroup (its fixed cost, Q load and output write, would dominate).
constexpr int kMaxSplits = 16;
constexpr int kMinSplitTiles = 4;

// Workspace of a split-KV launch, each part 256-byte aligned: partial outputs, partial
// log-sum-exps of the rounded P (merge weights), partial exact log-sum-exps (lse output).
struct WorkspaceLayout {
  size_t part_o, part_lse, part_lse_exact, total;
};
WorkspaceLayout workspace_layout(size_t rows, int head_dim, int splits) {
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  WorkspaceLayout w;
  w.part_o = 0;
  w.part_lse = up((size_t)splits * rows * head_dim * sizeof(float));
  w.part_lse_exact = w.part_lse + up((size_t)splits * rows * sizeof(float));
  w.total = w.part_lse_exact + up((size_t)splits * rows * sizeof(float));
  return w;
}

// The key-norm table (attn_key_norm.hip): one fp32 per (batch, kv head, kKeyChunk keys),
// placed after the split-KV partials in the workspace.
size_t key_table_bytes(int64_t batch, int64_t h_kv, int64_t n_kv) {
  const int64_t chunks = (n_kv + fa2::kKeyChunk - 1) / fa2::kKeyChunk;
  return (size_t)((batch * h_kv * chunks * (int64_t)sizeof(float) + 255) & ~(int64_t)255);
}

// Whether the key-norm pass pays for itself: it reads K once (~K bytes at HBM rate, plus a
// launch) and saves the per-tile row max where the bound holds. Measured on MI355X against the
// same launch without the table (N(0,1) inputs unless stated):
//   bf16 D128 causal +1.4% (C3 +1.3-2.2%), bf16 D128 full +0.3%, bf16 D64 full +3.7-4.0%,
//   bf16 D64 causal -0.9%. fp16, whose tau (15, the fp16 range of P) is tighter: D64 full +2.6%
//   at C4's half scale and -0.5% to -0.8% at unit scale with the reference lift (kBoundLift,
//   limited to bounds that keep every P above fp16's smallest subnormal; -1.3% to -3.0% without
//   it), D64 causal -4.0% (-3.5% at half scale), D128 causal -1.6%, D128 full -1.2%.
// Hence: head_dim 128 (bf16) or full attention at 64 (both types), and only where the attention
// does >= 16384 FLOP per byte of K and >= 2^37 FLOP (the pass's cost against the ~2-4% it can
// save).
bool key_table_pays(int64_t batch, int64_t h_q, int64_t h_kv, int64_t n_q, int64_t n_kv,
                    int64_t head_dim, int32_t dtype, bool causal) {
  const bool full64 = head_dim == 64 && !causal;
  if (!(full64 || (dtype == FA2_DTYPE_BF16 && head_dim == 128))) return false;
  const double pairs = causal ? (double)n_q * (n_q + 1) / 2 : (double)n_q * n_kv;
  const double flops = 4.0 * batch * h_q * pairs * head_dim;
  const double kbytes = 2.0 * batch * h_kv * n_kv * head_dim;
  return kbytes > 0 && flops >= 16384.0 * kbytes && flops >= 137438953472.0;  // 2^37
}

// Topology of a device as the program order uses it: log2 of its XCD count and its CU count.
struct Topology {
  int32_t xcd_shift = 3;  // 8 XCDs
  int32_t cus = fa2::kCus;
};

// The topology of a device reporting `cus` CUs on `xcds` XCDs. An XCD count that is not a power
// of two in [1, kMaxXcds], or that does not divide the CUs, is taken as one XCD (one L2): the
// order is then the one-XCD order, correct on any device, only without XCD locality.
Topology make_topology(int cus, int xcds) {
  Topology t;
  t.cus = cus > 0 ? cus : fa2::kCus;
  t.xcd_shift = 0;
  if (xcds > 1 && xcds <= fa2::kMaxXcds && (xcds & (xcds - 1)) == 0 && t.cus % xcds == 0)
    while ((1 << t.xcd_shift) < xcds) ++t.xcd_shift;
  return t;
}

// Causal programs on one XCD (program_of): its (batch, kv head) units are taken a chunk at a
// time, q-tile-major inside the chunk, so that the programs in flight read the K/V of at most
// ~kChunkKvBytes of units. Measured on MI355X against all of the XCD's units at once (causal,
// bf16 unless stated; 2, 3 or 4 units per chunk): B8 H16 N4096 D128 +4.9% (4), B2 H32 N8192
// D128 +2.4% (2), C2 (B4 H16 N4096) +0.5% (4); at head_dim 64 (fp16 B4 H16 N4096) chunks of 4
// and 2 lost 4% and 9%, which the byte budget avoids (1 MiB units: all 8 at once). Budgets of
// 2, 4 and 16 MiB against 8 (FA2_CHUNK_KV_MIB, compile-time so that ab.py can compare builds):
// 8 is the best or tied on every shape measured (C2: 4 MiB +1.1% time, 2 MiB +12%).
#ifndef FA2_CHUNK_KV_MIB
#define FA2_CHUNK_KV_MIB 8
#endif
constexpr int64_t kChunkKvBytes = int64_t(FA2_CHUNK_KV_MIB) << 20;
int32_t unit_chunk(int64_t units, int64_t n_kv, int64_t head_dim, const Topology& topo) {
  const int64_t upx = units >> topo.xcd_shift;
  if (upx < 1) return 1;
  const int64_t unit_kv = 4 * n_kv * head_dim;  // K and V bytes of one unit
  int64_t chunk = unit_kv > 0 ? std::max<int64_t>(1, kChunkKvBytes / unit_kv) : upx;
  if (chunk >= upx) return (int32_t)upx;
  while (upx % chunk) --chunk;
  return (int32_t)chunk;
}

// Tail policy knobs, compile-time so that an A/B of two builds can compare values (ab.py):
//   FA2_TAIL_PRIVATE_PCT  share of each XCD's tail programs that its own workgroups take first
//                         (its queue); the rest form the shared pool that any XCD takes from
//   FA2_TAIL_SHARE_PCT    the tail's share of each XCD's programs (at most)
//   FA2_TAIL_CHUNK_PCT    ... and of one unit chunk's programs (at most)
//   FA2_TAIL_EXTRA_PCT    spare tail workgroups, in percent of the grid
//   FA2_TAIL_EVENT_GUARD  1: each ticket set's launch waits for the event its previous launch
//                         signalled on completion (below); 0: no events, for measuring what
//                         they cost only (unsafe with streams destroyed while their work runs)
#ifndef FA2_TAIL_EVENT_GUARD
#define FA2_TAIL_EVENT_GUARD 1
#endif
#ifndef FA2_TAIL_PRIVATE_PCT
#define FA2_TAIL_PRIVATE_PCT 0
#endif
#ifndef FA2_TAIL_SHARE_PCT
#define FA2_TAIL_SHARE_PCT 25
#endif
#ifndef FA2_TAIL_CHUNK_PCT
#define FA2_TAIL_CHUNK_PCT 50
#endif
#ifndef FA2_TAIL_EXTRA_PCT
#define FA2_TAIL_EXTRA_PCT 6
#endif
// ... and the fewest programs per XCD, in percent of the workgroups the XCD holds at once, for a
// grid to get a tail (200: two rounds)
#ifndef FA2_TAIL_MIN_ROUNDS_PCT
#define FA2_TAIL_MIN_ROUNDS_PCT 200
#endif

// Dynamic tail of causal grids. Each XCD's programs run in a static order (program_of), but the
// XCDs do not run at one speed: their clocks differ by up to ~10% under the chip's power limit,
// and which ones are slow changes between boxes and workloads. The last programs of every XCD's
// order (the lightest, causal programs being taken heaviest first) are therefore dealt at run
// time, and a few extra workgroups (6% of the grid) give the fast XCDs room for more programs
// than their share; the ones that find no program left exit. The tail is the lighter of a quarter
// of each XCD's programs and half of one unit chunk (more would mix the K/V of more units in
// each XCD's L2). Measured on MI355X against the static order with one shared counter for the
// whole tail (back-to-back launches, same box): C3 +1.6-2.9%, C2 +1.0-1.4%, bf16 B2 H32/8 N8192
// D128 causal +2.3-2.7%, fp16 B4 H16 N4096 D64 causal +2.2-2.9%, B8 H16 N4096 D128 +0.7%; grids
// whose units do not split over the XCDs (program_of's fallback order; a quarter of every XCD's
// blocks): B3 H28/4 N4096 +1.2%, N8192 +1.9%, B1 H20/4 N8192 +2.7%. Non-causal grids (every
// program the same work, so no light programs to even out the end) lost 0.3% and keep the static
// order; so do grids of fewer than two rounds per XCD (FA2_TAIL_MIN_ROUNDS_PCT: a tail from one
// or 1.25 rounds cost C5 1.6% and moved the other grids of one to two rounds within noise).
// One shared counter hands a program to whichever XCD asks, so its unit's K/V is fetched into a
// second L2 (C3's reads past L2 rose from 213.6 to 334.1 MB per launch). A build with
// FA2_TAIL_PRIVATE_PCT > 0 gives each XCD of the XCD-aware order a queue of its own: the heavier
// FA2_TAIL_PRIVATE_PCT% of its tail programs stay with its workgroups, and only the lightest go to
// the shared pool. That brings the L2 locality back (C3 337 -> 214 MB per launch at 100%) but
// costs time (C3 -2.2%, fp16 head_dim 64 causal -2.0%, same-box A/B at 50%): only programs that
// any XCD can take even out the XCDs' clocks, and the extra L2 misses cost nothing measurable
// (C3 moves ~0.7 TB/s past L2). So the default is 0: one shared pool. Grids in the fallback
// order have no XCD affinity to keep and use the shared pool alone.
struct TailSchedule {
  int32_t static_blocks = 0, tail_wgs = 0;  // tail_wgs == 0: static order
  int32_t queues = 1, private_per_queue = 0, shared = 0;
  int32_t programs() const { return queues * private_per_queue + shared; }
};
TailSchedule tail_schedule(bool causal, int splits, int waves, int64_t units, int64_t progs_per_kv,
                           int64_t n_tiles, int32_t chunk, int head_dim, int bn,
                           const Topology& topo, int private_pct = FA2_TAIL_PRIVATE_PCT) {
  TailSchedule s;
  if (!causal || splits != 1 || waves != 4) return s;
  const int64_t xcds = int64_t(1) << topo.xcd_shift;
  // workgroups one XCD holds at once: its CUs x (3 at head_dim 64, 64-key tiles; else 2)
  const int64_t slots = std::max<int64_t>(1, topo.cus / xcds) * ((head_dim == 64 && bn <= 64) ? 3 : 2);
  const int64_t grid = units * progs_per_kv * n_tiles;
  const int64_t extra = (grid * FA2_TAIL_EXTRA_PCT / 100 + xcds - 1) / xcds * xcds;
  if (grid + extra > 0x7fffffffLL) return s;
  if (units % xcds) {
    // program_of's fallback order (q tile outermost, heaviest first; the hardware still deals
    // block b to XCD b % xcds): the last quarter of every XCD's blocks, and the remainder
    const int64_t per_xcd = grid / xcds;
    if (per_xcd * 100 < FA2_TAIL_MIN_ROUNDS_PCT * slots) return s;
    const int64_t static_blocks =
        (per_xcd - (per_xcd * FA2_TAIL_SHARE_PCT + 99) / 100) * xcds;
    s.static_blocks = (int32_t)static_blocks;
    s.shared = (int32_t)(grid - static_blocks);
    s.tail_wgs = (int32_t)(grid - static_blocks + extra);
    return s;
  }
  const int64_t upx = units / xcds;
  const int64_t per_xcd = upx * progs_per_kv * n_tiles;
  if (per_xcd * 100 < FA2_TAIL_MIN_ROUNDS_PCT * slots) return s;
  const int64_t cu = (chunk > 0 && upx % chunk == 0) ? chunk : upx;  // program_of's chunk
  const int64_t tail = std::min((per_xcd * FA2_TAIL_SHARE_PCT + 99) / 100,
                                cu * progs_per_kv * n_tiles * FA2_TAIL_CHUNK_PCT / 100);
  if (tail < 1) return s;
  const int64_t priv = tail * private_pct / 100;
  s.static_blocks = (int32_t)((per_xcd - tail) * xcds);
  s.queues = xcds > 1 && priv > 0 ? (int32_t)xcds : 1;
  s.private_per_queue = s.queues > 1 ? (int32_t)priv : 0;
  s.shared = (int32_t)(tail * xcds - (int64_t)s.queues * s.private_per_queue);
  s.tail_wgs = (int32_t)(tail * xcds + extra);
  return s;
}

// ---- device state: topology and the dynamic tail's ticket words, per device
//
// A launch with a dynamic tail uses a set of ticket words (kTicketWordsPerSet words, each on its
// own 64-byte line) in the library's own device memory: a static array, loaded as zeros. Its
// increments bring every word back to zero, so nothing is ever cleared, but two launches that
// share a set must not run at once. Each (device, stream) gets a set of its own, so launches on
// different streams overlap freely, and launches on one stream run one after another. A stream's
// handle can be reused by a stream created after it is destroyed, while the old stream's work
// may still be running (hipStreamDestroy does not promise to wait for it). So every set also has
// an event, which each launch that uses the set signals when it ends (the kernel is launched with
// it as its stop event), and the next launch that uses the set first makes its stream wait for
// that event: a new stream under an old handle then starts its launch only once the old one has
// ended. On one stream the wait costs nothing. Past kTicketSets streams per device, launches run
// the static order.
constexpr int kTicketSets = 256;
constexpr int kTicketDevices = 64;

}  // namespace
static __device__ __align__(256)
    uint32_t g_ticket_words[kTicketSets * fa2::kTicketWordsPerSet * fa2::kTicketStride] = {};
namespace {

struct TicketSet {
  int index = -1;
  hipEvent_t last = nullptr;  // signalled when the last launch that used the set ended
  bool recorded = false;
};

struct DeviceState {
  bool have_topology = false;
  Topology topo;
  uint32_t* ticket_base = nullptr;
  int sets_used = 0;
  std::map<hipStream_t, TicketSet> by_stream;
};

struct DeviceTable {
  std::mutex mu;
  DeviceState dev[kTicketDevices];
};

DeviceTable& device_table() {
  static DeviceTable t;
  return t;
}

// The device a launch on `stream` runs on (the current device for the null stream), or -1.
int stream_device(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  if (stream && stream != hipStreamPerThread) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) {
      (void)hipGetLastError();
      return -1;
    }
    dev = sdev;
  }
  return dev;
}

// The topology of device `dev`, read once (CU count and XCD count); the tuned MI355X topology
// when the device cannot be asked.
Topology device_topology(int dev) {
  if (dev < 0 || dev >= kTicketDevices) return Topology{};
  DeviceTable& t = device_table();
  std::lock_guard<std::mutex> lock(t.mu);
  DeviceState& d = t.dev[dev];
  if (!d.have_topology) {
    int cus = 0, xccs = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) {
      (void)hipGetLastError();
      return Topology{};
    }
    d.topo = make_topology(cus, xccs);
    d.have_topology = true;
  }
  return d.topo;
}

// A ticket set for a launch on `stream` on device `dev`, with the stream already made to wait
// for the set's previous launch; null when the launch should run the static order: a launch
// being recorded under stream capture (a graph can be instantiated twice and both instances run
// at once, which would share the set), one on the per-thread default stream (its handle names
// another stream in every thread), one on a stream of another device than the current one, or
// when no set or event is to be had. With may_create false, only a stream that already has a set
// gets it (making a set creates an event, which a caller that allocates nothing must not do).
// Runtime errors met here are cleared, so that the launch after it does not report them.
// finish_tickets() must follow the launch.
TicketSet* acquire_tickets(hipStream_t stream, int dev, uint32_t** words, bool may_create) {
  *words = nullptr;
  if (stream == hipStreamPerThread || dev < 0 || dev >= kTicketDevices) return nullptr;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != dev) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  DeviceTable& t = device_table();
  std::lock_guard<std::mutex> lock(t.mu);
  DeviceState& d = t.dev[dev];
  const auto it = d.by_stream.find(stream);
  if (it == d.by_stream.end() && !may_create) return nullptr;
  if (!d.ticket_base) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_ticket_words)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    d.ticket_base = static_cast<uint32_t*>(p);
  }
  TicketSet* set;
  if (it != d.by_stream.end()) {
    set = &it->second;
  } else {
    if (d.sets_used >= kTicketSets) return nullptr;
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    set = &d.by_stream[stream];
    set->index = d.sets_used++;
    set->last = ev;
  }
  if (set->index < 0) return nullptr;  // retired (an event record failed)
  if (FA2_TAIL_EVENT_GUARD && set->recorded &&
      hipStreamWaitEvent(stream, set->last, 0) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  *words = d.ticket_base + (size_t)set->index * fa2::kTicketWordsPerSet * fa2::kTicketStride;
  return set;
}

// After the launch that used `set`, which signals the set's event when it ends: the next launch
// on the set waits for it. If the launch failed, the event's state is unknown and the set is
// retired (never handed out again).
void finish_tickets(TicketSet* set, bool launched) {
  if (!FA2_TAIL_EVENT_GUARD) return;
  DeviceTable& t = device_table();
  std::lock_guard<std::mutex> lock(t.mu);
  if (launched)
    set->recorded = true;
  else
    set->index = -1;
}

// Launches the attention kernel of one checked call: the product's instances in the library,
// the timing variants (variant != 0) in the measurement library. Returns a hipError_t value.
using KernelLaunch = int (*)(int dtype, int di, const Params& p, int waves, int block_n,
                             bool causal, unsigned grid, hipStream_t s, int variant,
                             hipEvent_t stop);

// One call's arguments, as the C ABI takes them.
struct LaunchArgs {
  const void *q, *k, *v;
  void* out;
  const int64_t *q_stride, *k_stride, *v_stride, *o_stride;
  int32_t batch, h_q, h_kv, n_q, n_kv, head_dim, dtype, causal, pack, block_m, block_n;
  float qk_scale;
  float* lse;
  int32_t num_splits;
  void* workspace;
  size_t workspace_bytes;
  int32_t variant;
  uint64_t* timeline;
  int64_t timeline_words;
  bool static_order;
  // false: the launch may use its stream's ticket set but not make one (fa2_attn_fwd_noalloc)
  bool new_ticket_set = true;
};

// A checked call, ready to launch: the kernel's arguments (without the key-norm table and the
// ticket words, which need the device), its shape and its grid.
struct LaunchPlan {
  Params p;
  int di = 0, waves = 1, bn = 64, splits = 1;
  int64_t grid = 0;         // workgroups, the dynamic tail's included
  bool empty = false;       // nothing to launch (an empty output)
  bool key_table = false;   // run the key-norm pass into key_table_at
  size_t key_table_at = 0;  // its byte offset in the workspace
  TailSchedule tail;        // tail_wgs == 0: the static order
};

// Every check of a call (fa2/kernel.py:218-244 restated for a C caller) and its plan, on the
// given topology. No device call: the measurement library runs it on the CPU as well.
int plan_launch(const LaunchArgs& a, const Topology& topo, LaunchPlan* out,
                int tail_private_pct = FA2_TAIL_PRIVATE_PCT) {
  g_err[0] = '\0';
  LaunchPlan pl;
  // ---- shape checks (fa2/kernel.py:218-228)
  if (a.batch < 0 || a.h_q <= 0 || a.h_kv <= 0 || a.n_q < 0 || a.n_kv < 0)
    return fail(FA2_EINVAL, "bad sizes: batch=%d h_q=%d h_kv=%d n_q=%d n_kv=%d", a.batch, a.h_q,
                a.h_kv, a.n_q, a.n_kv);
  if (a.h_q % a.h_kv)
    return fail(FA2_EINVAL, "GQA needs H_q divisible by H_kv (%d %% %d)", a.h_q, a.h_kv);
  const int di = dim_index(a.head_dim);
  if (di < 0)
    return fail(FA2_EINVAL, "head_dim must be a power of two in [16, 128], got %d", a.head_dim);
  if (a.dtype != FA2_DTYPE_F16 && a.dtype != FA2_DTYPE_BF16)
    return fail(FA2_EINVAL, "dtype must be FA2_DTYPE_F16 or FA2_DTYPE_BF16, got %d", a.dtype);
  if (a.causal && a.n_q != a.n_kv)
    return fail(FA2_EINVAL, "causal attention here assumes N_q == N_kv (%d != %d)", a.n_q, a.n_kv);
  // ---- program shape (fa2/kernel.py:230-238)
  const int group = a.h_q / a.h_kv;
  if (a.pack != 1 && a.pack != group)
    return fail(FA2_EINVAL, "pack must be 1 or the GQA group %d, got %d", group, a.pack);
  if (a.block_m < 1 || a.block_m > 256)
    return fail(FA2_EINVAL, "BLOCK_M must be in [1, 256], got %d", a.block_m);
  if (a.block_m % a.pack)
    return fail(FA2_EINVAL,
                "pack_gqa needs BLOCK_M (%d) to be a multiple of the GQA group (%d)", a.block_m,
                a.pack);
  if (a.block_n < 0 || a.block_n > 128)
    return fail(FA2_EINVAL, "BLOCK_N must be in [1, 128] (0 = default), got %d", a.block_n);
  if (!(a.qk_scale > 0.f) || !std::isfinite(a.qk_scale))
    return fail(FA2_EINVAL, "qk_scale (sm_scale * log2 e) must be positive and finite, got %g",
                (double)a.qk_scale);
  // ---- split-KV
  if (a.num_splits < 1 || a.num_splits > kMaxSplits)
    return fail(FA2_EINVAL, "num_splits must be in [1, %d], got %d", kMaxSplits, a.num_splits);
  if (a.num_splits > 1 && a.causal)
    return fail(FA2_EINVAL, "split-KV needs causal == 0 (the causal kernel skips tiles instead)");
  // Key positions are 32-bit in the kernel, and its tile loop forms positions up to two K/V
  // tiles (256 keys) past the last one it loads.
  if (a.n_kv > kMaxSeq || a.n_q > kMaxSeq)
    return fail(FA2_EINVAL, "n_q and n_kv must be at most %d (32-bit key positions), got %d and %d",
                kMaxSeq, a.n_q, a.n_kv);
  if (a.batch == 0 || a.n_q == 0) {  // empty output: nothing to launch
    pl.empty = true;
    *out = pl;
    return FA2_OK;
  }
  // ---- the 16-byte load/store rule
  if (!a.q || !a.k || !a.v || !a.out) return fail(FA2_EINVAL, "null tensor pointer");
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || !aligned16(a.out))
    return fail(FA2_EALIGN, "q, k, v and out must be 16-byte aligned");
  const int64_t* strides[4] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride};
  for (int t = 0; t < 4; ++t) {
    if (!strides[t]) return fail(FA2_EINVAL, "null stride array");
    if (strides[t][3] != 1)
      return fail(FA2_EALIGN, "the head_dim stride must be 1 (tensor %d has %lld)", t,
                  (long long)strides[t][3]);
    for (int j = 0; j < 3; ++j)
      if (strides[t][j] % 8 || strides[t][j] < 0)
        return fail(FA2_EALIGN, "strides must be multiples of 8 elements (tensor %d dim %d: %lld)",
                    t, j, (long long)strides[t][j]);
  }
  if (a.lse && (reinterpret_cast<uintptr_t>(a.lse) & 3u))
    return fail(FA2_EALIGN, "lse must be 4-byte aligned");
  // K/V tiles are addressed with 32-bit byte offsets from the tile's first row.
  if (a.k_stride[2] > kMaxRowStride || a.v_stride[2] > kMaxRowStride)
    return fail(FA2_EINVAL, "k/v sequence stride above %lld elements is not supported",
                (long long)kMaxRowStride);

  // block_m rows -> wave64s of 32 rows, rounded up to 1, 2, 4 or 8 (rows past block_m are
  // computed on zeros and dropped); block_n -> the next supported K/V tile width.
  int waves = 1;
  while (waves * 32 < a.block_m) waves *= 2;
  const int bn = tile_n(a.block_n, a.head_dim);

  Params& p = pl.p;
  p = Params{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.o = static_cast<uint16_t*>(a.out);
  p.sqb = a.q_stride[0]; p.sqh = a.q_stride[1]; p.sqn = a.q_stride[2];
  p.skb = a.k_stride[0]; p.skh = a.k_stride[1]; p.skn = a.k_stride[2];
  p.svb = a.v_stride[0]; p.svh = a.v_stride[1]; p.svn = a.v_stride[2];
  p.sob = a.o_stride[0]; p.soh = a.o_stride[1]; p.son = a.o_stride[2];
  p.h_q = a.h_q;
  p.n_q = a.n_q;
  p.n_kv = a.n_kv;
  p.group = group;
  p.pack = a.pack;
  p.block_m = a.block_m;
  const int64_t rows = (int64_t)a.n_q * a.pack;
  const int64_t n_tiles = (rows + a.block_m - 1) / a.block_m;
  const int64_t n_bh = (int64_t)a.batch * (a.h_q / a.pack);
  // checked before any product with it can leave int64 (n_tiles >= 1: n_q > 0 here)
  if (n_bh > 0x7fffffffLL / n_tiles)
    return fail(FA2_EINVAL, "grid of %lld x %lld workgroups is too large", (long long)n_tiles,
                (long long)n_bh);
  // The kernel's packed row index tile * block_m + (row inside the program) is 32-bit; its
  // largest value is (n_tiles - 1) * block_m + 32 * waves - 1 (rows past block_m included).
  if ((n_tiles - 1) * a.block_m + 32 * waves > 0x7fffffffLL)
    return fail(FA2_EINVAL,
                "n_q * pack = %lld rows of block_m %d exceed the kernel's 32-bit row index",
                (long long)rows, a.block_m);
  p.n_tiles = (int32_t)n_tiles;
  p.n_bh = (int32_t)n_bh;
  p.xcd_shift = topo.xcd_shift;
  p.cus = topo.cus;
  p.unit_chunk = unit_chunk(n_bh / (group / a.pack), a.n_kv, a.head_dim, topo);
  p.qk_scale = a.qk_scale;
  p.lse = a.lse;
  p.part_rows = (int64_t)a.batch * a.h_q * a.n_q;
  p.splits = 1;
  p.static_blocks = 0x7fffffff;
  p.tail_queues = 1;

  // Split-KV: cut the key range into whole tiles; drop splits that would be empty.
  const int64_t kv_tiles = ((int64_t)a.n_kv + bn - 1) / bn;
  int splits = a.num_splits;
  if (splits > 1 && kv_tiles > 0) {
    const int64_t per = (kv_tiles + splits - 1) / splits;
    splits = (int)((kv_tiles + per - 1) / per);
    p.split_tiles = (int32_t)per;
  }
  if (splits <= 1 || a.n_kv == 0) splits = 1;
  if (splits > 1) {
    const WorkspaceLayout w = workspace_layout((size_t)p.part_rows, a.head_dim, splits);
    if (!a.workspace || a.workspace_bytes < w.total)
      return fail(FA2_EINVAL, "split-KV with %d splits needs a workspace of %zu bytes, got %zu",
                  splits, w.total, a.workspace ? a.workspace_bytes : (size_t)0);
    if (reinterpret_cast<uintptr_t>(a.workspace) & 255u)
      return fail(FA2_EALIGN, "the workspace must be 256-byte aligned");
    p.part_o = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + w.part_o);
    p.part_lse = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + w.part_lse);
    p.part_lse_exact = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + w.part_lse_exact);
    p.splits = splits;
    // the combine pass runs one thread per 4 dims of every row
    if (p.part_rows * (a.head_dim / 4) / 256 >= 0x7fffffffLL)
      return fail(FA2_EINVAL, "split-KV merge of %lld rows is too large", (long long)p.part_rows);
  } else {
    p.split_tiles = 0;
  }
  int64_t grid = n_tiles * n_bh * splits;
  if (grid > 0x7fffffffLL)
    return fail(FA2_EINVAL, "grid of %lld workgroups is too large", (long long)grid);
  if (a.timeline) {  // the measurement library's timeline variant: kTimelineWords per program
    if (a.timeline_words < grid * fa2::kTimelineWords)
      return fail(FA2_EINVAL, "the timeline needs %lld words for %lld programs, got %lld",
                  (long long)(grid * fa2::kTimelineWords), (long long)grid,
                  (long long)a.timeline_words);
    p.timeline = a.timeline;
  }

  // Key-norm table: used whenever the workspace has room for it beyond the split-KV partials of
  // the REQUESTED split count, fa2_workspace_bytes(..., num_splits), which is where
  // fa2_workspace_bytes_for puts it where it pays. The partials of a clamped (smaller) split
  // count fit inside that size, so the room they leave never turns the table on by itself.
  const size_t split_bytes =
      a.num_splits > 1 ? workspace_layout((size_t)p.part_rows, a.head_dim, a.num_splits).total : 0;
  const size_t table_bytes = key_table_bytes(a.batch, a.h_kv, a.n_kv);
  if (a.workspace && a.n_kv > 0 && a.workspace_bytes >= split_bytes + table_bytes &&
      a.variant == 0 && waves == 4 && bn == default_block_n(a.head_dim)) {
    if (reinterpret_cast<uintptr_t>(a.workspace) & 255u)
      return fail(FA2_EALIGN, "the workspace must be 256-byte aligned");
    const int64_t kgrid = (int64_t)a.batch * a.h_kv * ((a.n_kv + fa2::kKeyChunk - 1) / fa2::kKeyChunk);
    if (kgrid > 0x7fffffffLL)
      return fail(FA2_EINVAL, "key-norm grid of %lld workgroups is too large", (long long)kgrid);
    pl.key_table = true;
    pl.key_table_at = split_bytes;
  }
  if (!a.static_order)
    pl.tail = tail_schedule(a.causal != 0, splits, waves, n_bh / (group / a.pack), group / a.pack,
                            n_tiles, p.unit_chunk, a.head_dim, bn, topo, tail_private_pct);
  if (pl.tail.tail_wgs > 0) grid = (int64_t)pl.tail.static_blocks + pl.tail.tail_wgs;
  pl.di = di;
  pl.waves = waves;
  pl.bn = bn;
  pl.splits = splits;
  pl.grid = grid;
  *out = pl;
  return FA2_OK;
}

// Launches of this library that ran with a dynamic tail (a ticket set), for the measurement
// library's tests: a launch recorded under stream capture must not count.
std::atomic<long long> g_tail_launches{0};

// Puts a plan's dynamic tail into its kernel arguments, with the ticket words at `words`.
void apply_tail(LaunchPlan& pl, uint32_t* words) {
  Params& p = pl.p;
  p.tickets = words;
  p.static_blocks = pl.tail.static_blocks;
  p.tail_wgs = pl.tail.tail_wgs;
  p.tail_queues = pl.tail.queues;
  p.tail_private = pl.tail.private_per_queue;
  p.tail_shared = pl.tail.shared;
}

// One call: plan it on the stream's device, then the key-norm pass, the attention kernel and the
// split-KV merge, asynchronously on `stream`.
int attn_fwd_impl(const LaunchArgs& a, KernelLaunch launch_kernel, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int dev = stream_device(st);
  LaunchPlan pl;
  int rc = plan_launch(a, device_topology(dev), &pl);
  if (rc != FA2_OK || pl.empty) return rc;
  Params& p = pl.p;
  if (pl.key_table) {
    fa2::KeyNormParams kp;
    kp.k = p.k;
    kp.skb = p.skb; kp.skh = p.skh; kp.skn = p.skn;
    kp.h_kv = a.h_kv;
    kp.n_kv = a.n_kv;
    kp.chunks = (a.n_kv + fa2::kKeyChunk - 1) / fa2::kKeyChunk;
    kp.out = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + pl.key_table_at);
    const int64_t kgrid = (int64_t)a.batch * a.h_kv * kp.chunks;
    const int ke = fa2::launch_key_norm(a.dtype, a.head_dim, kp, (unsigned)kgrid, st);
    if (ke != hipSuccess)
      return fail(FA2_ELAUNCH, "key-norm launch failed: %s", hipGetErrorString((hipError_t)ke));
    p.key_norm2 = kp.out;
    p.key_chunks = kp.chunks;
  }
  TicketSet* set = nullptr;
  int64_t grid = pl.grid;
  if (pl.tail.tail_wgs > 0) {
    uint32_t* words = nullptr;
    set = acquire_tickets(st, dev, &words, a.new_ticket_set);
    if (set) {
      apply_tail(pl, words);
    } else {
      grid -= pl.tail.tail_wgs - pl.tail.programs();  // the static order: one workgroup a program
    }
  }
  // the ticket set's event, signalled by the kernel's own completion (hipExtLaunchKernel): a
  // marker of its own behind each launch (hipEventRecord) cost 0.6-1.8% (C3, C2, fp16 head_dim
  // 64), the event on the launch nothing measurable (same-box A/B)
  hipEvent_t stop = (set && FA2_TAIL_EVENT_GUARD) ? set->last : nullptr;
  int e = launch_kernel(a.dtype, pl.di, p, pl.waves, pl.bn, a.causal != 0, (unsigned)grid, st,
                        a.variant, stop);
  if (set) {
    finish_tickets(set, e == hipSuccess);
    if (e == hipSuccess) g_tail_launches.fetch_add(1, std::memory_order_relaxed);
  }
  if (e != hipSuccess)
    return fail(FA2_ELAUNCH, "kernel launch failed: %s", hipGetErrorString((hipError_t)e));
  if (pl.splits > 1) {
    fa2::CombineParams c;
    c.part_o = p.part_o;
    c.part_lse = p.part_lse;
    c.part_lse_exact = p.part_lse_exact;
    c.o = p.o;
    c.lse = a.lse;
    c.sob = p.sob; c.soh = p.soh; c.son = p.son;
    c.rows = p.part_rows;
    c.h_q = a.h_q;
    c.n_q = a.n_q;
    c.splits = pl.splits;
    e = fa2::launch_combine(a.dtype, a.head_dim, c, st);
    if (e != hipSuccess)
      return fail(FA2_ELAUNCH, "combine launch failed: %s", hipGetErrorString((hipError_t)e));
  }
  return FA2_OK;
}

}  // namespace
