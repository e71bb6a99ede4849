// attn_fwd_host.hpp - host side of one forward launch: the argument checks (fa2/kernel.py:218-244
// restated for a C caller), the workspace layout and key-norm policy, the grid, and the launch
// sequence (key-norm pass, attention kernel, split-KV merge). Shared by the library
// (fa2_fwd.hip) and the measurement library (fa2_ablate.hip); everything here has internal
// linkage, so each library compiles its own copy with its own error string.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
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
//   bf16 D128 causal +1.4% (C3 +1.6-2.2%), bf16 D128 full +0.3%, bf16 D64 full +4.0%,
//   bf16 D64 causal -0.9%; fp16 D128 causal -1.8%, fp16 D128 full -2.7%, fp16 D64 full -3.0%
//   (with C4's half-scale inputs +3.9%), fp16 D64 causal -1.3%.
// fp16's tau (15, the fp16 range of P) is too tight for unit-variance scores, so the bound
// fails and the pass is pure cost; bf16's (32) holds. Hence: bf16, head_dim 128 or full
// attention at 64, and only where the attention does >= 16384 FLOP per byte of K and >= 2^37
// FLOP (the pass's cost against the ~2-4% it can save).
bool key_table_pays(int64_t batch, int64_t h_q, int64_t h_kv, int64_t n_q, int64_t n_kv,
                    int64_t head_dim, int32_t dtype, bool causal) {
  if (dtype != FA2_DTYPE_BF16 || !(head_dim == 128 || (head_dim == 64 && !causal))) return false;
  const double pairs = causal ? (double)n_q * (n_q + 1) / 2 : (double)n_q * n_kv;
  const double flops = 4.0 * batch * h_q * pairs * head_dim;
  const double kbytes = 2.0 * batch * h_kv * n_kv * head_dim;
  return kbytes > 0 && flops >= 16384.0 * kbytes && flops >= 137438953472.0;  // 2^37
}

// Causal programs on one XCD (program_of): its (batch, kv head) units are taken a chunk at a
// time, q-tile-major inside the chunk, so that the programs in flight read the K/V of at most
// ~kChunkKvBytes of units. Measured on MI355X against all of the XCD's units at once (causal,
// bf16 unless stated; 2, 3 or 4 units per chunk): B8 H16 N4096 D128 +4.9% (4), B2 H32 N8192
// D128 +2.4% (2), C2 (B4 H16 N4096) +0.5% (4); at head_dim 64 (fp16 B4 H16 N4096) chunks of 4
// and 2 lost 4% and 9%, which the byte budget avoids (1 MiB units: all 8 at once).
constexpr int64_t kChunkKvBytes = int64_t(8) << 20;
int32_t unit_chunk(int64_t units, int64_t n_kv, int64_t head_dim) {
  const int64_t upx = units / fa2::kXcds;
  if (upx < 1) return 1;
  const int64_t unit_kv = 4 * n_kv * head_dim;  // K and V bytes of one unit
  int64_t chunk = unit_kv > 0 ? std::max<int64_t>(1, kChunkKvBytes / unit_kv) : upx;
  if (chunk >= upx) return (int32_t)upx;
  while (upx % chunk) --chunk;
  return (int32_t)chunk;
}

// Dynamic tail of causal grids. Each XCD's programs run in a static order (program_of), but the
// XCDs do not run at one speed: their clocks differ by up to ~10% under the chip's power limit,
// and which ones are slow changes between boxes and workloads. The last programs of every XCD's
// order (the lightest, causal programs being taken heaviest first) are therefore dealt at run
// time: the workgroups past static_blocks take tickets from one counter, so the XCDs that run
// ahead take more of them, heaviest first, and a few extra workgroups (6% of the grid) give the
// fast XCDs room for more programs than their share; the ones that find no program left exit.
// The tail is the lighter of a quarter of each XCD's programs and half of one unit chunk (more
// would mix the K/V of more units in each XCD's L2). Measured on MI355X against the static order
// (back-to-back launches, same box): C3 +1.6-2.9%, C2 +1.0-1.4%, bf16 B2 H32/8 N8192 D128 causal
// +2.3-2.7%, fp16 B4 H16 N4096 D64 causal +2.2-2.9%, B8 H16 N4096 D128 +0.7%; grids whose units
// do not split over the XCDs (program_of's fallback order; a quarter of every XCD's blocks):
// B3 H28/4 N4096 +1.2%, N8192 +1.9%, B1 H20/4 N8192 +2.7%. Non-causal grids (every program the
// same work, so no light programs to even out the end) lost 0.3% and keep the static order; so
// do grids of fewer than two rounds per XCD.
struct TailSchedule {
  int32_t static_blocks = 0, tail_wgs = 0, tail_programs = 0;  // tail_wgs == 0: static order
};
TailSchedule tail_schedule(bool causal, int splits, int waves, int64_t units, int64_t progs_per_kv,
                           int64_t n_tiles, int32_t chunk, int head_dim, int bn) {
  TailSchedule s;
  if (!causal || splits != 1 || waves != 4) return s;
  // workgroups one XCD holds at once: 32 CUs x (3 at head_dim 64, 64-key tiles; else 2)
  const int64_t slots = (fa2::kCus / fa2::kXcds) * ((head_dim == 64 && bn <= 64) ? 3 : 2);
  const int64_t grid = units * progs_per_kv * n_tiles;
  const int64_t extra = (grid * 6 / 100 + 7) / 8 * 8;
  if (grid + extra > 0x7fffffffLL) return s;
  if (units % fa2::kXcds) {
    // program_of's fallback order (q tile outermost, heaviest first; the hardware still deals
    // block b to XCD b % 8): the last quarter of every XCD's blocks, and the remainder
    const int64_t per_xcd = grid / fa2::kXcds;
    if (per_xcd < 2 * slots) return s;
    const int64_t static_blocks = (per_xcd - (per_xcd + 3) / 4) * fa2::kXcds;
    s.static_blocks = (int32_t)static_blocks;
    s.tail_programs = (int32_t)(grid - static_blocks);
    s.tail_wgs = (int32_t)(grid - static_blocks + extra);
    return s;
  }
  const int64_t upx = units / fa2::kXcds;
  const int64_t per_xcd = upx * progs_per_kv * n_tiles;
  if (per_xcd < 2 * slots) return s;
  const int64_t cu = (chunk > 0 && upx % chunk == 0) ? chunk : upx;  // program_of's chunk
  const int64_t tail = std::min((per_xcd + 3) / 4, cu * progs_per_kv * n_tiles / 2);
  if (tail < 1) return s;
  s.static_blocks = (int32_t)((per_xcd - tail) * fa2::kXcds);
  s.tail_programs = (int32_t)(tail * fa2::kXcds);
  s.tail_wgs = (int32_t)(tail * fa2::kXcds + extra);
  return s;
}

// The dynamic tail's ticket words: one per (device, stream) in the library's own device memory.
// A launch's increments bring its word back to zero, the value the array is loaded with, so
// nothing is ever cleared, and the launches on one stream run one after another, so two launches
// that can overlap in time never share a word. A stream's handle is reused by the next stream
// created once it is destroyed, but hipStreamDestroy returns only when the stream's queued work
// has run (measured: 10.6 ms for 20 queued C3 launches), so the new stream's launches cannot meet
// the old one's. Past kTicketWords streams per device, launches run the static order.
constexpr int kTicketWords = 1024;
constexpr int kTicketStride = 16;  // words apart: each word on its own 64-byte line
constexpr int kTicketDevices = 64;

}  // namespace
static __device__ __align__(256) uint32_t g_ticket_words[kTicketWords * kTicketStride] = {};
namespace {

struct TicketPool {
  std::mutex mu;
  uint32_t* base[kTicketDevices] = {};
  int used[kTicketDevices] = {};
  std::map<std::pair<int, hipStream_t>, int> by_stream;
};

TicketPool& ticket_pool() {
  static TicketPool pool;
  return pool;
}

// The ticket word of a launch on `stream`, or null (the launch then runs the static order). None
// for a launch being recorded under stream capture (a graph can be instantiated twice and both
// instances run at once, which would share the word), for the per-thread default stream (its
// handle names another stream in every thread), or when the stream's device is not the current
// one. Runtime errors met here are cleared, so that the launch after it does not report them.
uint32_t* ticket_word(hipStream_t stream) {
  if (stream == hipStreamPerThread) return nullptr;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kTicketDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  TicketPool& pool = ticket_pool();
  std::lock_guard<std::mutex> lock(pool.mu);
  if (!pool.base[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_ticket_words)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    pool.base[dev] = static_cast<uint32_t*>(p);
  }
  int idx;
  const auto it = pool.by_stream.find({dev, stream});
  if (it != pool.by_stream.end()) {
    idx = it->second;
  } else {
    if (pool.used[dev] >= kTicketWords) return nullptr;
    idx = pool.used[dev]++;
    pool.by_stream.emplace(std::make_pair(dev, stream), idx);
  }
  return pool.base[dev] + (size_t)idx * kTicketStride;
}

// Launches the attention kernel of one checked call: the product's instances in the library,
// the timing variants (variant != 0) in the measurement library. Returns a hipError_t value.
using KernelLaunch = int (*)(int dtype, int di, const Params& p, int waves, int block_n,
                             bool causal, unsigned grid, hipStream_t s, int variant);

int attn_fwd_impl(const void* q, const void* k, const void* v, void* out,
                  const int64_t q_stride[4], const int64_t k_stride[4],
                  const int64_t v_stride[4], const int64_t o_stride[4], int32_t batch,
                  int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                  int32_t dtype, int32_t causal, int32_t pack, int32_t block_m, int32_t block_n,
                  float qk_scale, float* lse, int32_t num_splits, void* workspace,
                  size_t workspace_bytes, int32_t variant, KernelLaunch launch_kernel,
                  void* stream, uint64_t* timeline = nullptr, int64_t timeline_words = 0,
                  bool static_order = false) {
  g_err[0] = '\0';
  // ---- shape checks (fa2/kernel.py:218-228)
  if (batch < 0 || h_q <= 0 || h_kv <= 0 || n_q < 0 || n_kv < 0)
    return fail(FA2_EINVAL, "bad sizes: batch=%d h_q=%d h_kv=%d n_q=%d n_kv=%d", batch, h_q,
                h_kv, n_q, n_kv);
  if (h_q % h_kv) return fail(FA2_EINVAL, "GQA needs H_q divisible by H_kv (%d %% %d)", h_q, h_kv);
  const int di = dim_index(head_dim);
  if (di < 0)
    return fail(FA2_EINVAL, "head_dim must be a power of two in [16, 128], got %d", head_dim);
  if (dtype != FA2_DTYPE_F16 && dtype != FA2_DTYPE_BF16)
    return fail(FA2_EINVAL, "dtype must be FA2_DTYPE_F16 or FA2_DTYPE_BF16, got %d", dtype);
  if (causal && n_q != n_kv)
    return fail(FA2_EINVAL, "causal attention here assumes N_q == N_kv (%d != %d)", n_q, n_kv);
  // ---- program shape (fa2/kernel.py:230-238)
  const int group = h_q / h_kv;
  if (pack != 1 && pack != group)
    return fail(FA2_EINVAL, "pack must be 1 or the GQA group %d, got %d", group, pack);
  if (block_m < 1 || block_m > 256)
    return fail(FA2_EINVAL, "BLOCK_M must be in [1, 256], got %d", block_m);
  if (block_m % pack)
    return fail(FA2_EINVAL,
                "pack_gqa needs BLOCK_M (%d) to be a multiple of the GQA group (%d)", block_m,
                pack);
  if (block_n < 0 || block_n > 128)
    return fail(FA2_EINVAL, "BLOCK_N must be in [1, 128] (0 = default), got %d", block_n);
  if (!(qk_scale > 0.f) || !std::isfinite(qk_scale))
    return fail(FA2_EINVAL, "qk_scale (sm_scale * log2 e) must be positive and finite, got %g",
                (double)qk_scale);
  // ---- split-KV
  if (num_splits < 1 || num_splits > kMaxSplits)
    return fail(FA2_EINVAL, "num_splits must be in [1, %d], got %d", kMaxSplits, num_splits);
  if (num_splits > 1 && causal)
    return fail(FA2_EINVAL, "split-KV needs causal == 0 (the causal kernel skips tiles instead)");
  // Key positions are 32-bit in the kernel, and its tile loop forms positions up to two K/V
  // tiles (256 keys) past the last one it loads.
  if (n_kv > kMaxSeq || n_q > kMaxSeq)
    return fail(FA2_EINVAL, "n_q and n_kv must be at most %d (32-bit key positions), got %d and %d",
                kMaxSeq, n_q, n_kv);
  if (batch == 0 || n_q == 0) return FA2_OK;  // empty output: nothing to launch
  // ---- the 16-byte load/store rule
  if (!q || !k || !v || !out) return fail(FA2_EINVAL, "null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(FA2_EALIGN, "q, k, v and out must be 16-byte aligned");
  const int64_t* strides[4] = {q_stride, k_stride, v_stride, o_stride};
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
  if (lse && (reinterpret_cast<uintptr_t>(lse) & 3u))
    return fail(FA2_EALIGN, "lse must be 4-byte aligned");
  // K/V tiles are addressed with 32-bit byte offsets from the tile's first row.
  if (k_stride[2] > kMaxRowStride || v_stride[2] > kMaxRowStride)
    return fail(FA2_EINVAL, "k/v sequence stride above %lld elements is not supported",
                (long long)kMaxRowStride);

  // block_m rows -> wave64s of 32 rows, rounded up to 1, 2, 4 or 8 (rows past block_m are
  // computed on zeros and dropped); block_n -> the next supported K/V tile width.
  int waves = 1;
  while (waves * 32 < block_m) waves *= 2;
  const int bn = tile_n(block_n, head_dim);

  Params p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(out);
  p.sqb = q_stride[0]; p.sqh = q_stride[1]; p.sqn = q_stride[2];
  p.skb = k_stride[0]; p.skh = k_stride[1]; p.skn = k_stride[2];
  p.svb = v_stride[0]; p.svh = v_stride[1]; p.svn = v_stride[2];
  p.sob = o_stride[0]; p.soh = o_stride[1]; p.son = o_stride[2];
  p.h_q = h_q;
  p.n_q = n_q;
  p.n_kv = n_kv;
  p.group = group;
  p.pack = pack;
  p.block_m = block_m;
  const int64_t rows = (int64_t)n_q * pack;
  const int64_t n_tiles = (rows + block_m - 1) / block_m;
  const int64_t n_bh = (int64_t)batch * (h_q / pack);
  // checked before any product with it can leave int64 (n_tiles >= 1: n_q > 0 here)
  if (n_bh > 0x7fffffffLL / n_tiles)
    return fail(FA2_EINVAL, "grid of %lld x %lld workgroups is too large", (long long)n_tiles,
                (long long)n_bh);
  // The kernel's packed row index tile * block_m + (row inside the program) is 32-bit; its
  // largest value is (n_tiles - 1) * block_m + 32 * waves - 1 (rows past block_m included).
  if ((n_tiles - 1) * block_m + 32 * waves > 0x7fffffffLL)
    return fail(FA2_EINVAL,
                "n_q * pack = %lld rows of block_m %d exceed the kernel's 32-bit row index",
                (long long)rows, block_m);
  p.n_tiles = (int32_t)n_tiles;
  p.n_bh = (int32_t)n_bh;
  p.unit_chunk = unit_chunk(n_bh / (group / pack), n_kv, head_dim);
  p.qk_scale = qk_scale;
  p.lse = lse;
  p.part_o = nullptr;
  p.part_lse = nullptr;
  p.part_lse_exact = nullptr;
  p.part_rows = (int64_t)batch * h_q * n_q;
  p.splits = 1;
  p.split_tiles = 0;
  p.key_norm2 = nullptr;
  p.key_chunks = 0;
  p.timeline = nullptr;
  p.tickets = nullptr;
  p.static_blocks = 0x7fffffff;
  p.tail_wgs = 0;
  p.tail_programs = 0;

  // Split-KV: cut the key range into whole tiles; drop splits that would be empty.
  const int64_t kv_tiles = ((int64_t)n_kv + bn - 1) / bn;
  int splits = num_splits;
  if (splits > 1 && kv_tiles > 0) {
    const int64_t per = (kv_tiles + splits - 1) / splits;
    splits = (int)((kv_tiles + per - 1) / per);
    p.split_tiles = (int32_t)per;
  }
  if (splits <= 1 || n_kv == 0) splits = 1;
  if (splits > 1) {
    const WorkspaceLayout w = workspace_layout((size_t)p.part_rows, head_dim, splits);
    if (!workspace || workspace_bytes < w.total)
      return fail(FA2_EINVAL, "split-KV with %d splits needs a workspace of %zu bytes, got %zu",
                  splits, w.total, workspace ? workspace_bytes : (size_t)0);
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      return fail(FA2_EALIGN, "the workspace must be 256-byte aligned");
    p.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.part_o);
    p.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.part_lse);
    p.part_lse_exact = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.part_lse_exact);
    p.splits = splits;
    // the combine pass runs one thread per 4 dims of every row
    if (p.part_rows * (head_dim / 4) / 256 >= 0x7fffffffLL)
      return fail(FA2_EINVAL, "split-KV merge of %lld rows is too large", (long long)p.part_rows);
  }
  int64_t grid = n_tiles * n_bh * splits;
  if (grid > 0x7fffffffLL)
    return fail(FA2_EINVAL, "grid of %lld workgroups is too large", (long long)grid);
  if (timeline) {  // the measurement library's timeline variant: kTimelineWords per program
    if (timeline_words < grid * fa2::kTimelineWords)
      return fail(FA2_EINVAL, "the timeline needs %lld words for %lld programs, got %lld",
                  (long long)(grid * fa2::kTimelineWords), (long long)grid,
                  (long long)timeline_words);
    p.timeline = timeline;
  }

  hipStream_t st = static_cast<hipStream_t>(stream);
  // Key-norm table: used whenever the workspace has room for it beyond the split-KV partials of
  // the REQUESTED split count, fa2_workspace_bytes(..., num_splits), which is where
  // fa2_workspace_bytes_for puts it where it pays. The partials of a clamped (smaller) split
  // count fit inside that size, so the room they leave never turns the table on by itself.
  const size_t split_bytes =
      num_splits > 1 ? workspace_layout((size_t)p.part_rows, head_dim, num_splits).total : 0;
  const size_t table_bytes = key_table_bytes(batch, h_kv, n_kv);
  if (workspace && n_kv > 0 && workspace_bytes >= split_bytes + table_bytes && variant == 0 &&
      waves == 4 && bn == default_block_n(head_dim)) {
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      return fail(FA2_EALIGN, "the workspace must be 256-byte aligned");
    fa2::KeyNormParams kp;
    kp.k = p.k;
    kp.skb = p.skb; kp.skh = p.skh; kp.skn = p.skn;
    kp.h_kv = h_kv;
    kp.n_kv = n_kv;
    kp.chunks = (n_kv + fa2::kKeyChunk - 1) / fa2::kKeyChunk;
    kp.out = reinterpret_cast<float*>(static_cast<char*>(workspace) + split_bytes);
    const int64_t kgrid = (int64_t)batch * h_kv * kp.chunks;
    if (kgrid > 0x7fffffffLL)
      return fail(FA2_EINVAL, "key-norm grid of %lld workgroups is too large", (long long)kgrid);
    const int ke = fa2::launch_key_norm(dtype, head_dim, kp, (unsigned)kgrid, st);
    if (ke != hipSuccess)
      return fail(FA2_ELAUNCH, "key-norm launch failed: %s", hipGetErrorString((hipError_t)ke));
    p.key_norm2 = kp.out;
    p.key_chunks = kp.chunks;
  }
  if (!static_order) {
    const TailSchedule ts = tail_schedule(causal != 0, splits, waves, n_bh / (group / pack),
                                          group / pack, n_tiles, p.unit_chunk, head_dim, bn);
    if (ts.tail_wgs > 0) {
      if (uint32_t* word = ticket_word(st)) {
        p.tickets = word;
        p.static_blocks = ts.static_blocks;
        p.tail_wgs = ts.tail_wgs;
        p.tail_programs = ts.tail_programs;
        grid = (int64_t)ts.static_blocks + ts.tail_wgs;
      }
    }
  }
  int e = launch_kernel(dtype, di, p, waves, bn, causal != 0, (unsigned)grid, st, variant);
  if (e != hipSuccess)
    return fail(FA2_ELAUNCH, "kernel launch failed: %s", hipGetErrorString((hipError_t)e));
  if (splits > 1) {
    fa2::CombineParams c;
    c.part_o = p.part_o;
    c.part_lse = p.part_lse;
    c.part_lse_exact = p.part_lse_exact;
    c.o = p.o;
    c.lse = lse;
    c.sob = p.sob; c.soh = p.soh; c.son = p.son;
    c.rows = p.part_rows;
    c.h_q = h_q;
    c.n_q = n_q;
    c.splits = splits;
    e = fa2::launch_combine(dtype, head_dim, c, st);
    if (e != hipSuccess)
      return fail(FA2_ELAUNCH, "combine launch failed: %s", hipGetErrorString((hipError_t)e));
  }
  return FA2_OK;
}

}  // namespace
