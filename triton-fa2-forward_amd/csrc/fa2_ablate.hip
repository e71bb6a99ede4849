// fa2_ablate.hip - C ABI of the measurement library libfa2_ablate.so (include/fa2_ablate.h):
// the forward kernel's timing variants behind the same argument checks and launch sequence as
// the product (attn_fwd_host.hpp, compiled into this library separately).
#include <hip/hip_runtime.h>

#include <vector>

#include "attn_fwd_ablate.hpp"
#include "attn_fwd_host.hpp"
#include "attn_fwd_schedule.hpp"
#include "fa2_ablate.h"

namespace {

int launch_ablate(int dtype, int di, const Params& p, int waves, int block_n, bool causal,
                  unsigned grid, hipStream_t s, int variant, hipEvent_t stop) {
  // the variants exist at the default configuration only (4 waves of 32 rows, the default tile)
  if (waves != 4 || block_n != default_block_n(kDims[di])) return (int)hipErrorInvalidValue;
  switch (dtype * 4 + di) {
    case 0: return fa2::launch_attn_fwd_ablate<0, 16>(p, variant, causal, grid, s, stop);
    case 1: return fa2::launch_attn_fwd_ablate<0, 32>(p, variant, causal, grid, s, stop);
    case 2: return fa2::launch_attn_fwd_ablate<0, 64>(p, variant, causal, grid, s, stop);
    case 3: return fa2::launch_attn_fwd_ablate<0, 128>(p, variant, causal, grid, s, stop);
    case 4: return fa2::launch_attn_fwd_ablate<1, 16>(p, variant, causal, grid, s, stop);
    case 5: return fa2::launch_attn_fwd_ablate<1, 32>(p, variant, causal, grid, s, stop);
    case 6: return fa2::launch_attn_fwd_ablate<1, 64>(p, variant, causal, grid, s, stop);
    default: return fa2::launch_attn_fwd_ablate<1, 128>(p, variant, causal, grid, s, stop);
  }
}

// The plan of a launch of contiguous [B, H, N, D] tensors at block_m rows and the default
// tile, without a workspace (no split-KV, no key-norm table), on `topo`. No device call.
int plan_default(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t head_dim,
                 int32_t causal, int32_t pack, int32_t block_m, const Topology& topo,
                 bool static_order, LaunchPlan* pl, int private_pct = FA2_TAIL_PRIVATE_PCT) {
  if (batch < 1 || h_q < 1 || h_kv < 1 || n_q < 1 || h_q % h_kv)
    return fail(FA2_EINVAL, "bad sizes: batch=%d h_q=%d h_kv=%d n_q=%d", batch, h_q, h_kv, n_q);
  const int64_t d = head_dim;
  const int64_t sq[4] = {(int64_t)h_q * n_q * d, (int64_t)n_q * d, d, 1};
  const int64_t sk[4] = {(int64_t)h_kv * n_q * d, (int64_t)n_q * d, d, 1};
  // stand-in device addresses: the plan checks their alignment and never dereferences them
  void* const fake = reinterpret_cast<void*>(uintptr_t(1) << 20);
  const LaunchArgs a{fake, fake, fake, fake, sq, sk, sk, sq, batch, h_q, h_kv, n_q, n_q,
                     head_dim, FA2_DTYPE_BF16, causal, pack, block_m, 0, 1.0f, nullptr, 1,
                     nullptr, 0, 0, nullptr, 0, static_order};
  return plan_launch(a, topo, pl, private_pct);
}

}  // namespace

extern "C" {

const char* fa2_ablate_last_error(void) { return g_err; }

int fa2_ablate_attn_fwd(const void* q, const void* k, const void* v, void* out,
                        const int64_t q_stride[4], const int64_t k_stride[4],
                        const int64_t v_stride[4], const int64_t o_stride[4], int32_t batch,
                        int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                        int32_t dtype, int32_t causal, int32_t pack, float qk_scale,
                        int32_t variant, void* stream) {
  // FA2_ABLATE_STATIC_ORDER is the host's: the launch keeps the static order (no dynamic tail);
  // the key split always does (its workgroups hold a whole CU, which the tail's slots do not model)
  const bool static_order =
      (variant & FA2_ABLATE_STATIC_ORDER) != 0 || (variant & fa2::kVariantSplitKeys) != 0;
  variant &= ~FA2_ABLATE_STATIC_ORDER;
  // the timeline instance writes its records: only fa2_ablate_timeline, with a buffer, runs it
  if (!fa2::ablation_variant_built(variant) || (variant & fa2::kVariantTimeline)) {
    g_err[0] = '\0';
    return fail(FA2_EINVAL, "variant 0x%x is not one of the built timing variants",
                (unsigned)variant);
  }
  if ((variant & fa2::kVariantSplitKeys) && head_dim != 128) {
    g_err[0] = '\0';
    return fail(FA2_EINVAL, "the key split is built at head_dim 128 only, got %d", head_dim);
  }
  const LaunchArgs a{q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                     n_q, n_kv, head_dim, dtype, causal, pack, 128, 0, qk_scale, nullptr, 1,
                     nullptr, 0, variant, nullptr, 0, static_order};
  return attn_fwd_impl(a, launch_ablate, stream);
}

int fa2_ablate_timeline(const void* q, const void* k, const void* v, void* out,
                        const int64_t q_stride[4], const int64_t k_stride[4],
                        const int64_t v_stride[4], const int64_t o_stride[4], int32_t batch,
                        int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv, int32_t head_dim,
                        int32_t dtype, int32_t causal, int32_t pack, float qk_scale,
                        uint64_t* records, int64_t record_words, void* stream) {
  g_err[0] = '\0';
  if (!records) return fail(FA2_EINVAL, "null timeline buffer");
  if (reinterpret_cast<uintptr_t>(records) & 7u)
    return fail(FA2_EALIGN, "the timeline buffer must be 8-byte aligned");
  const LaunchArgs a{q, k, v, out, q_stride, k_stride, v_stride, o_stride, batch, h_q, h_kv,
                     n_q, n_kv, head_dim, dtype, causal, pack, 128, 0, qk_scale, nullptr, 1,
                     nullptr, 0, fa2::kVariantTimeline, records, record_words, false};
  return attn_fwd_impl(a, launch_ablate, stream);
}

int fa2_ablate_tail_schedule(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                             int32_t head_dim, int32_t causal, int32_t pack,
                             int32_t* static_blocks, int32_t* tail_programs,
                             int32_t* tail_workgroups) {
  g_err[0] = '\0';
  if (!static_blocks || !tail_programs || !tail_workgroups) return fail(FA2_EINVAL, "null output");
  *static_blocks = *tail_programs = *tail_workgroups = 0;
  LaunchPlan pl;
  const int rc = plan_default(batch, h_q, h_kv, n_q, head_dim, causal, pack, 128, Topology{}, false,
                              &pl);
  if (rc != FA2_OK) return rc;
  *static_blocks = pl.tail.static_blocks;
  *tail_programs = pl.tail.programs();
  *tail_workgroups = pl.tail.tail_wgs;
  return 0;
}

int fa2_ablate_program_map(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                           int32_t head_dim, int32_t causal, int32_t pack, int32_t block_m,
                           int32_t cus, int32_t xcds, int32_t static_order,
                           int32_t tail_private_pct, uint32_t seed, int32_t* programs,
                           int64_t program_words, int32_t* info, int32_t info_words) {
  g_err[0] = '\0';
  if (!programs || !info || info_words < FA2_ABLATE_MAP_INFO_WORDS)
    return fail(FA2_EINVAL, "null output or info shorter than %d words", FA2_ABLATE_MAP_INFO_WORDS);
  if (cus < 1 || xcds < 1) return fail(FA2_EINVAL, "cus and xcds must be positive");
  if (tail_private_pct < -1 || tail_private_pct > 100)
    return fail(FA2_EINVAL, "tail_private_pct must be -1 (the library's) or in [0, 100]");
  LaunchPlan pl;
  const int rc = plan_default(batch, h_q, h_kv, n_q, head_dim, causal, pack, block_m,
                              make_topology(cus, xcds), static_order != 0, &pl,
                              tail_private_pct < 0 ? FA2_TAIL_PRIVATE_PCT : tail_private_pct);
  if (rc != FA2_OK) return rc;
  const int64_t grid = pl.empty ? 0 : pl.grid;
  if (program_words < 3 * grid)
    return fail(FA2_EINVAL, "the map needs %lld words for %lld workgroups, got %lld",
                (long long)(3 * grid), (long long)grid, (long long)program_words);
  Params& p = pl.p;
  if (pl.tail.tail_wgs > 0) apply_tail(pl, nullptr);
  // the kernel's program choice, workgroup by workgroup: the static order, then the tail's
  // tickets in a seeded random order of its workgroups (any order is one the hardware may take)
  uint32_t words[fa2::kTicketWordsPerSet] = {};
  auto inc = [&](int word, uint32_t limit) {
    const uint32_t old = words[word];
    words[word] = old >= limit ? 0u : old + 1u;
    return old;
  };
  const int64_t first_tail = pl.tail.tail_wgs > 0 ? p.static_blocks : grid;
  std::vector<int32_t> order;
  for (int64_t w = first_tail; w < grid; ++w) order.push_back((int32_t)w);
  uint64_t st = 0x9e3779b97f4a7c15ull ^ seed;
  for (size_t i = order.size(); i > 1; --i) {  // Fisher-Yates with a 64-bit LCG
    st = st * 6364136223846793005ull + 1442695040888963407ull;
    std::swap(order[i - 1], order[(size_t)((st >> 33) % i)]);
  }
  auto put = [&](int64_t w, int block) {
    int32_t* o = programs + 3 * w;
    if (block < 0) {
      o[0] = o[1] = o[2] = -1;
      return;
    }
    const fa2::Program pr = causal ? fa2::program_of<true>(p, block) : fa2::program_of<false>(p, block);
    o[0] = pr.tile;
    o[1] = pr.b;
    o[2] = pr.hq0;
  };
  for (int64_t w = 0; w < first_tail; ++w) put(w, (int)w);
  for (int32_t w : order) put(w, fa2::tail_pick(p, w, inc));
  int nonzero = 0;
  for (uint32_t x : words) nonzero += x != 0;
  const int32_t vals[FA2_ABLATE_MAP_INFO_WORDS] = {
      (int32_t)grid, pl.tail.tail_wgs > 0 ? pl.tail.static_blocks : (int32_t)grid,
      pl.tail.tail_wgs, pl.tail.queues, pl.tail.private_per_queue, pl.tail.shared,
      p.unit_chunk, p.xcd_shift, nonzero, p.n_tiles, p.n_bh};
  for (int i = 0; i < FA2_ABLATE_MAP_INFO_WORDS; ++i) info[i] = vals[i];
  return 0;
}

long long fa2_ablate_tail_launches(void) { return g_tail_launches.load(); }

int fa2_ablate_mfma_ceiling(int32_t mode, int32_t workgroups, int32_t iters, float* out,
                            int64_t out_words, void* stream) {
  g_err[0] = '\0';
  if (mode < FA2_ABLATE_CEIL_MFMA || mode > FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE)
    return fail(FA2_EINVAL, "unknown ceiling mode %d", (int)mode);
  if (workgroups < 1 || workgroups > FA2_ABLATE_CEIL_MAX_WORKGROUPS)
    return fail(FA2_EINVAL, "workgroups %d outside [1, %d]", (int)workgroups,
                FA2_ABLATE_CEIL_MAX_WORKGROUPS);
  if (iters < 1 || iters > FA2_ABLATE_CEIL_MAX_ITERS)
    return fail(FA2_EINVAL, "iters %d outside [1, %d]", (int)iters, FA2_ABLATE_CEIL_MAX_ITERS);
  if (!out) return fail(FA2_EINVAL, "null output");
  if (reinterpret_cast<uintptr_t>(out) & 3u)
    return fail(FA2_EALIGN, "the output must be 4-byte aligned");
  if (out_words < (int64_t)workgroups * 256)
    return fail(FA2_EINVAL, "the output holds %lld floats; %d workgroups write %lld",
                (long long)out_words, (int)workgroups, (long long)workgroups * 256);
  const int rc = fa2::launch_mfma_ceiling(mode, out, workgroups, iters,
                                          static_cast<hipStream_t>(stream));
  if (rc != 0)
    return fail(FA2_ELAUNCH, "ceiling launch failed: %s", hipGetErrorString((hipError_t)rc));
  return 0;
}

int fa2_ablate_hbm_read(const void* src, int64_t bytes, uint32_t* out, int64_t out_words,
                        int32_t workgroups, void* stream) {
  g_err[0] = '\0';
  if (!src || !out) return fail(FA2_EINVAL, "null buffer");
  if ((reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(out) & 3u))
    return fail(FA2_EALIGN, "src must be 16-byte and out 4-byte aligned");
  if (bytes < 16 || bytes % 16) return fail(FA2_EINVAL, "bytes (%lld) must be a positive multiple of 16", (long long)bytes);
  if (workgroups < 1 || workgroups > FA2_ABLATE_CEIL_MAX_WORKGROUPS)
    return fail(FA2_EINVAL, "workgroups %d outside [1, %d]", (int)workgroups,
                FA2_ABLATE_CEIL_MAX_WORKGROUPS);
  if (out_words < (int64_t)workgroups * 256)
    return fail(FA2_EINVAL, "the output holds %lld words; %d workgroups write %lld",
                (long long)out_words, (int)workgroups, (long long)workgroups * 256);
  const int rc = fa2::launch_hbm_read(src, bytes / 16, out, workgroups, static_cast<hipStream_t>(stream));
  if (rc != 0)
    return fail(FA2_ELAUNCH, "read launch failed: %s", hipGetErrorString((hipError_t)rc));
  return 0;
}

}  // extern "C"
