// attn_fwd_kernel.hpp - the gfx950 FlashAttention-2 forward kernel.
//
// Computes what `_attn_fwd` / `_attn_fwd_inner` compute (fa2/kernel.py:60-183):
//   O = softmax(Q K^T * sm_scale [+ top-left causal mask]) V
// with the online softmax in base 2 (exp2, qk_scale = sm_scale * log2 e folded into one
// FMA per score, fa2/kernel.py:95-97), two-stage causal skipping (fa2/kernel.py:150-169),
// GQA by index mapping and optional head packing (fa2/kernel.py:126-141).
//
// CDNA4 mapping (one workgroup = one program of the reference):
//   * NW wave64s, each owning 32 consecutive rows of the program's block_m rows; the kernel
//     is register-budgeted for two waves per SIMD so one wave's softmax overlaps another's
//     matrix work.
//   * Each wave computes the TRANSPOSED score block S^T = K Q^T with
//     v_mfma_f32_32x32x16_{bf16,f16}: K (32 keys x 16 dims) is the A operand, read
//     from LDS; Q^T is the B operand and stays in VGPRs for the whole loop.
//     In the 32x32 accumulator, lane l holds column l%32 (= one query row) and 16 of the
//     32 keys; the other 16 keys of that row sit in lane l^32. A row's max and sum are
//     therefore 16-value lane-local reductions plus one v_permlane32_swap.
//   * K rows are fed to the A operand in the order pi(r) (bits 2 and 3 of r swapped),
//     which makes accumulator register i of lane l hold key 16*(i/8) + 8*(l/32) + i%8.
//     Registers 8h..8h+7 are then 8 consecutive keys, i.e. exactly the B operand
//     (P^T, 8 consecutive k) of the second product O^T += V^T P^T: P never leaves VGPRs.
//   * V stays in its HBM layout [key][dim] in LDS and is read as the A operand V^T with
//     ds_read_b64_tr_b16 (gfx950's transposing LDS read): each 16-lane group reads a
//     4-key x 16-dim block and every lane receives 4 consecutive keys of one dim.
//   * O^T accumulates in 32x32 blocks whose lane l holds column l%32 = the lane's own
//     query row, so the per-row rescale by alpha is a lane-local multiply.
//   * K/V tiles go HBM -> LDS directly (buffer_load_dwordx4 ... lds, no VGPR staging) into
//     double buffers, K two tiles and V one tile ahead of their product; one barrier per tile.
//   * LDS layouts are XOR-swizzled at 16-byte granularity so that both the b128 reads
//     of K and the transposing b64 reads of V are free of bank conflicts; the swizzle is
//     applied by choosing which global chunk each lane fetches.
//   * Lazy rescaling: a row's reference max only moves when the new max exceeds it by more
//     than 2^8 (in exp2 units), so the O rescale (D/32 x 16 multiplies per lane) is skipped
//     on most tiles. The result is the same softmax: acc and l share the reference.
//   * Programs are ordered so that each XCD (its own L2) works through whole KV heads,
//     heaviest causal tiles first.
//   * At head_dim 64 the tile loop is software-pipelined inside each wave (S_{j+1}'s MFMAs
//     next to softmax_j, PV_j's next to the row max of S_{j+1}): there a tile's softmax needs
//     more issue time than its MFMAs. At 128 the waves of a SIMD overlap each other instead.
#pragma once

#include "attn_fwd_common.hpp"
#include "attn_fwd_schedule.hpp"

// fp16 below head_dim 128 sums l from P rounded to fp16 with v_dot2 (1) or from the unrounded P
// in fp32 (0); compile-time so that an A/B of two builds can compare them (ab.py).
#ifndef FA2_FP16_ROUNDED_SUM
#define FA2_FP16_ROUNDED_SUM 1
#endif
// Output store of the one-tile loop at head_dim 128 (unpacked rows, no split-KV): 0 writes each
// lane's 16-byte pieces straight from the accumulators (every store instruction touches 32 rows),
// 1 stages the wave's 32 rows through LDS first, so that every store instruction writes 4 whole
// rows. Compile-time so that an A/B of two builds can compare them (ab.py).
#ifndef FA2_STAGED_STORE
#define FA2_STAGED_STORE 0
#endif
// Q, read once per program, and the output, written once: 1 loads / stores them non-temporally
// (bit 0: Q, bit 1: O), so that they take less of L2 from the K/V tiles that programs share.
// Compile-time so that an A/B of two builds can compare them (ab.py).
#ifndef FA2_NT_QO
#define FA2_NT_QO 0
#endif
// 1: 8-wave (256-row) programs at head_dim 128 run the software-pipelined loop (each wave
// interleaves its own softmax with its own MFMAs), whose two waves per SIMD come from one
// workgroup and meet its barrier together; 0: the one-tile loop. Compile-time, for ab.py.
#ifndef FA2_PIPE_WIDE
#define FA2_PIPE_WIDE 0
#endif

namespace fa2 {

// The dynamic tail's program of tail workgroup `block` (tail_pick), with agent-scope atomic
// increments of the launch's ticket words. Returns the block whose program to run, or -1.
__device__ __forceinline__ int take_tail_program(const Params& p, int block) {
  return tail_pick(p, block, [&](int word, uint32_t limit) {
    return __builtin_amdgcn_atomic_inc32(p.tickets + word * kTicketStride, limit,
                                         __ATOMIC_RELAXED, "agent");
  });
}

// ---------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------
// VARIANT is 0 for the product (kVariantKeyBound for its key-norm instance). The measurement
// library instantiates the timing variants of the reference's ablation (bench/ablation.py:1-20):
// kVariantScaleFirst scales every score before the row max and subtracts the max separately
// (two VALU instructions per score instead of one FMA); kVariantMaskEveryTile applies the mask
// on every K/V tile, not only on the tiles that need it (both still compute attention); and the
// knockouts kVariantNoExp, kVariantNoSoftmax, kVariantKvL2 and kVariantNoKvStaging, which skip
// work and compute garbage on purpose (their time is the point). With none of these bits the code is unchanged.
//
// Register budget: two waves per SIMD (256 VGPRs each), except for the software-pipelined loop
// (head_dim 64, 64- or 32-key tiles), which is held to three (168 VGPRs): measured +4.5-5.5% for
// bf16 at head_dim 64, where this costs a few spilled VGPRs; fp16 fits without.
template <int DT, int D, int NW, int BN, bool CAUSAL, int VARIANT = 0>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu((D == 64 && BN <= 64) ? 3 : 2)))
void attn_fwd_kernel(const Params p) {
  using E = Elem<DT>;
  constexpr bool kScaleFirst = (VARIANT & kVariantScaleFirst) != 0;
  constexpr bool kMaskEveryTile = (VARIANT & kVariantMaskEveryTile) != 0;
  constexpr bool KB = (VARIANT & kVariantKeyBound) != 0;  // key-norm table present
  constexpr bool kNoExp = (VARIANT & kVariantNoExp) != 0;
  constexpr bool kNoSoftmax = (VARIANT & kVariantNoSoftmax) != 0;
  constexpr bool kKvL2 = (VARIANT & kVariantKvL2) != 0;
  constexpr bool kNoKvStaging = (VARIANT & kVariantNoKvStaging) != 0;
  constexpr bool kNoQLoad = (VARIANT & kVariantNoQLoad) != 0;
  constexpr bool kNoStore = (VARIANT & kVariantNoStore) != 0;
  constexpr bool kTimeline = (VARIANT & kVariantTimeline) != 0;
  // Measurement library only: the workgroup's waves form two groups of NW / 2 that run the same
  // rows over the two halves of the program's key range, each group with K/V buffers of its own,
  // and merge (m, l, O) through LDS before one store (one workgroup per CU).
  constexpr bool kSplit = (VARIANT & kVariantSplitKeys) != 0;
  constexpr int KG = kSplit ? 2 : 1;       // key groups
  constexpr int GW = NW / KG;              // waves per key group
  static_assert(!kSplit || !(D == 64 && BN <= 64), "the key split runs the one-tile loop");
  static_assert(!kSplit || (VARIANT & (kVariantKeyBound | kVariantTimeline)) == 0,
                "the key split has no key-norm bound and no timeline");
  const uint64_t tl_entry = kTimeline ? __builtin_amdgcn_s_memrealtime() : 0;
  uint64_t tl_prologue = 0, tl_loop = 0;
  // exp2, or (knockout) its argument
  auto ex2 = [](float x) { return kNoExp ? x : __builtin_amdgcn_exp2f(x); };
  constexpr int KS = D / 16;               // 16-dim k-steps of S^T = K Q^T
  constexpr int DB = (D + 31) / 32;        // 32-dim row blocks of O^T
  constexpr int NB = BN / 32;              // 32-key row blocks of S^T
  constexpr int CPR = D / 8;               // 16-byte chunks per K / V row
  constexpr int TCH = BN * CPR;            // chunks per K (or V) tile
  constexpr int NI = TCH / 64;             // 64-lane LDS load instructions per tile
  static_assert(TCH % 64 == 0, "a tile must be whole 1 KiB load instructions");

  __shared__ u32x4 k_lds[KG][2][TCH];
  __shared__ u32x4 v_lds[KG][2][TCH];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS addresses stay scalar
  const int lane = tid & 63;
  const int c = lane & 31;
  const int g = lane >> 5;
  const int grp = kSplit ? wave / GW : 0;  // key group (uniform)
  const int gwave = wave - grp * GW;        // wave inside its group: 32 rows each

  // split-KV: consecutive workgroups are the splits of one program
  const int split = p.splits > 1 ? (int)blockIdx.x % p.splits : 0;
  int block = p.splits > 1 ? (int)blockIdx.x / p.splits : (int)blockIdx.x;
  // dynamic tail: one lane takes the workgroup's tickets (its XCD's queue first, then the shared
  // pool) and passes the program it won to the others through LDS; -1: nothing left to run
  if (block >= p.static_blocks) {
    __shared__ int picked;
    if (tid == 0) picked = take_tail_program(p, block);
    __syncthreads();
    const int b = __builtin_amdgcn_readfirstlane(picked);
    if (b < 0) return;
    block = b;
  }
  const Program pr = program_of<CAUSAL>(p, block);

  // ---- this lane's query row: packed row r -> (position r / pack, head r % pack)
  // (fa2/kernel.py:135-139). Rows past block_m or past n_q compute on zeros and are
  // never stored; they see every key so their softmax stays finite.
  const int lrow = gwave * 32 + c;
  const int r = pr.tile * p.block_m + lrow;
  const int pos = r / p.pack;
  const int head = pr.hq0 + (r - pos * p.pack);
  const bool row_ok = lrow < p.block_m && pos < p.n_q;
  const int pos_vis = row_ok ? pos : 0x3fffffff;

  // ---- Q^T operand, loaded once (fa2/kernel.py:144)
  u32x4 qreg[KS];
  {
    const uint16_t* qrow = p.q + pr.b * p.sqb + head * p.sqh + (int64_t)pos * p.sqn + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (kNoQLoad) {  // knockout: a lane pattern of small values instead of Q
        const uint32_t w = 0x3c003c00u ^ (uint32_t)(lane * 0x00110011u + ks * 0x00050005u);
        qreg[ks] = u32x4{w, w ^ 0x00030003u, w ^ 0x00090009u, w ^ 0x000f000fu};
      } else {
        if constexpr ((FA2_NT_QO & 1) != 0)
          qreg[ks] = row_ok ? __builtin_nontemporal_load((const u32x4*)(qrow + 16 * ks))
                            : u32x4{0u, 0u, 0u, 0u};
        else
          qreg[ks] = row_ok ? *(const u32x4*)(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // ---- key range (fa2/kernel.py:150-175). Tiles below full_end need no mask:
  // causal: every column left of the tile's first position (stage 1, rounded down to
  // a whole tile); full: every whole tile. The rest is masked (stage 2 / the tail).
  const int pos_per_prog = p.block_m / p.pack;
  const int lo_pos = pr.tile * pos_per_prog;
  int kv_begin = 0, kv_end, full_end;
  if (CAUSAL) {
    kv_end = min(lo_pos + pos_per_prog, p.n_kv);
    full_end = (lo_pos / BN) * BN;
  } else {
    kv_end = p.n_kv;
    full_end = (p.n_kv / BN) * BN;
    if (p.splits > 1) {  // this split's tiles (non-causal only; every split is non-empty)
      kv_begin = split * p.split_tiles * BN;
      kv_end = min(kv_begin + p.split_tiles * BN, p.n_kv);
    }
  }
  int n_tiles_kv = (kv_end - kv_begin + BN - 1) / BN;
  // key groups: the first ceil(n / 2) tiles to group 0, the rest to group 1; both groups run
  // n_iter trips of the tile loop, one barrier each (a group with fewer tiles idles through them)
  int n_iter = n_tiles_kv;
  if constexpr (kSplit) {
    const int h = (n_tiles_kv + 1) / 2;
    n_iter = h;
    if (grp == 0) {
      kv_end = min(kv_begin + h * BN, kv_end);
      n_tiles_kv = h;
    } else {
      kv_begin += h * BN;
      n_tiles_kv -= h;
    }
  }

  // ---- score bound from the key-norm table (fa2_attn_fwd_ex with a workspace): a row's scores
  // obey |q . k| <= |q| max|k| over the keys it sees. A causal row sees keys [0, pos]: the chunks
  // before the program's first position (common to its rows: at most four per lane here, the
  // rest folded at once) and its own last one to three; otherwise every row sees the program's
  // key range. Either way the bound depends on the row alone, so packed and unpacked launches
  // decide alike. The table reads are issued here and consumed after the prologue's wait for Q,
  // by bound_from_table(), so their latency hides behind the Q load. The margin in
  // qk_scale_bound covers the fp32 rounding of the norms and of the MFMA sums. Without the
  // table (KB false) the bound is +inf and nothing changes.
  float kt[4] = {0.f, 0.f, 0.f, 0.f};  // this lane's share of the common chunks
  float kr[3] = {0.f, 0.f, 0.f};       // the row's own chunks (causal)
  if (KB) {
    const float* kn = p.key_norm2 + (int64_t)(pr.b * (p.h_q / p.group) + pr.hkv) * p.key_chunks;
    const int c_begin = kv_begin / kKeyChunk;
    const int c_common = CAUSAL ? lo_pos / kKeyChunk : (kv_end + kKeyChunk - 1) / kKeyChunk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c_begin + lane + 64 * i;
      if (c < c_common) kt[i] = kn[c];
    }
    for (int c0 = c_begin + 256 + lane; c0 < c_common; c0 += 256) {  // past 16384 keys
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c0 + 64 * i < c_common) kt[i] = fmaxf(kt[i], kn[c0 + 64 * i]);
    }
    if (CAUSAL) {  // 128 positions span at most three 64-key chunks
      const int c_row = min(pos_vis, kv_end - 1) / kKeyChunk;
#pragma unroll
      for (int t = 0; t < 3; ++t)
        if (c_common + t <= c_row) kr[t] = kn[c_common + t];
    }
  }
  auto bound_from_table = [&]() {
    float km = fmaxf(fmaxf(kt[0], kt[1]), fmaxf(kt[2], kt[3]));
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) km = fmaxf(km, __shfl_xor(km, off, 64));
    km = fmaxf(km, fmaxf(kr[0], fmaxf(kr[1], kr[2])));
    float qn = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int w = 0; w < 4; ++w) qn = E::sumsq2(qreg[ks][w], qn);
    qn = pair_sum(qn);  // the row's other half of the dims sits in lane ^ 32
    return __builtin_sqrtf(qn * km) * qk_scale_bound(p.qk_scale);
  };
  float bound = INFINITY;
  // Set after a row's first tile: no later score of the row can exceed its reference max by
  // more than kBoundTau<DT> (the reference raised by a whole number, to bound - tau or just
  // above, where the bound was within kBoundLift<DT> of that), so its reference never moves
  // again (a NaN bound or reference fails the test). skip_max: every row of the wave is so, and
  // the wave skips the row max.
  bool skip_row = false;
  bool skip_max = false;

  // ---- K/V staging: each wave issues every NW-th 1 KiB load of the tile. Chunk P of a tile
  // (16 bytes, P = 64 * instruction + lane) holds row P / CPR, logical chunk
  // (P % CPR) ^ key(row). The per-lane byte offsets are fixed; each tile moves the base of a
  // buffer resource that ends after row n_kv - 1, so rows past the sequence read as zeros.
  constexpr int JW = (NI + GW - 1) / GW;  // load instructions per wave per tensor
  const char* kbase = (const char*)(p.k + pr.b * p.skb + pr.hkv * p.skh);
  const char* vbase = (const char*)(p.v + pr.b * p.svb + pr.hkv * p.svh);
  uint32_t koff[JW], voff[JW];
#pragma unroll
  for (int jj = 0; jj < JW; ++jj) {
    const int P = (gwave + jj * GW) * 64 + lane;
    const int row = P / CPR, col = P % CPR;
    koff[jj] = (uint32_t)(row * p.skn + (col ^ k_key<D>(pi_row(row & 31) & 15)) * 8) * 2u;
    voff[jj] = (uint32_t)(row * p.svn + (col ^ v_key<D>(row & 15)) * 8) * 2u;
  }
  // The resource of the tile at key n0 covers its rows n0 .. min(n0 + BN, n_kv) - 1 only (the
  // loads touch no other row). The host keeps a row stride at or below 2^22 elements, so its
  // byte stride and (BN - 1) rows of it plus a row's D elements stay below 2^31: 32-bit
  // products, the 64-bit base added once (n0 >= 0, and n0 < n_kv since only tiles of the range
  // are issued).
  auto rsrc_at = [&](const char* base, int64_t stride, int n0) {
    const uint32_t stride2 = (uint32_t)stride * 2u;
    const uint32_t rows = (uint32_t)min(p.n_kv - n0, BN);  // 1 .. BN
    const uint32_t bytes = (rows - 1u) * stride2 + (uint32_t)D * 2u;
    return make_desc(base + (uint64_t)(uint32_t)n0 * stride2, bytes);
  };
  auto issue_k = [&](int n0, int buf) {
    if (kNoKvStaging && n0 >= kv_begin + 2 * BN) return;
    const auto rs = rsrc_at(kbase, p.skn, kKvL2 ? kv_begin : n0);
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
      const int j = gwave + jj * GW;
      if (NI % GW == 0 || j < NI) load_lds16(rs, koff[jj], lds_addr((const FA2_LDS char*)k_lds[grp][buf] + j * 64 * 16));
    }
  };
  auto issue_v = [&](int n0, int buf) {
    if (kNoKvStaging && n0 >= kv_begin + 2 * BN) return;
    const auto rs = rsrc_at(vbase, p.svn, kKvL2 ? kv_begin : n0);
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
      const int j = gwave + jj * GW;
      if (NI % GW == 0 || j < NI) load_lds16(rs, voff[jj], lds_addr((const FA2_LDS char*)v_lds[grp][buf] + j * 64 * 16));
    }
  };

  // ---- LDS operand reads
  const int kk = k_key<D>(c & 15);
  const int vs = lane & 15;          // role inside the 16-lane transpose group
  const int vj = vs >> 2;            // key row within the 4-row block it addresses
  const int vq = vs & 3;
  const int vsig = ((vq & 1) << 1) | ((vq & 2) >> 1);
  const int vdh = (D == 16) ? 0 : ((lane >> 4) & 1);
  // Per-lane byte offsets of the operand reads inside a tile, computed once. The XOR keys make
  // them lane-dependent only through the k-step (K) or the row half and dim block (V); the key
  // block nb (K) and the key step t (V) only add a constant, which the ds_read's immediate
  // offset absorbs, so a tile's reads need one VALU add per offset for the buffer base.
  uint32_t koffs[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    koffs[ks] = (uint32_t)((pi_row(c) * CPR + ((2 * ks + g) ^ kk)) * 16);
  // Kept whole: split into a shared part and a per-k-step part, each read's address would cost
  // two vector instructions per tile (or, add) instead of one (or with the buffer base).
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(koffs[ks]));
  uint32_t voffs[2][DB];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int row = 8 * g + 4 * rr + vj;  // row & 15 of every key step's row 16 t + row
      const int chunk = (4 * db + 2 * vdh + (vsig >> 1)) ^ v_key<D>(row);
      voffs[rr][db] = (uint32_t)(row * (D * 2) + chunk * 16 + (vsig & 1) * 8);
    }
  // A operand of S^T: 32 keys (rows pi(c) of key block nb) x 16 dims (k-step ks)
  auto k_operand = [&](int buf, int ks, int nb) {
    const char FA2_LDS* kt = (const char FA2_LDS*)k_lds[grp][buf] + koffs[ks];
    return *(const u32x4 FA2_LDS*)(kt + nb * 32 * CPR * 16);
  };
  // The same read, volatile: used before the loop so that the compiler cannot merge it with
  // the in-loop prefetch into one load at the top of the loop (which would expose its latency).
  auto k_operand_v = [&](int buf, int ks, int nb) {
    const char FA2_LDS* kt = (const char FA2_LDS*)k_lds[grp][buf] + koffs[ks];
    return *(const volatile u32x4 FA2_LDS*)(kt + nb * 32 * CPR * 16);
  };
  // A operand of O^T: 32 dims (block db) x 16 keys (k-step t), two transposing reads
  auto v_operand = [&](int buf, int t, int db) {
    const char FA2_LDS* vt = (const char FA2_LDS*)v_lds[grp][buf];
    const u32x2 lo = lds_read_tr(vt + voffs[0][db] + t * 16 * D * 2);
    const u32x2 hi = lds_read_tr(vt + voffs[1][db] + t * 16 * D * 2);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  // ---- online-softmax state (fa2/kernel.py:146-148); l is a per-lane partial sum.
  // bf16: l sums P rounded to bf16, the weights the PV product uses, so that O = acc / l is a
  // convex combination of V rows. With the lazy reference max a row's largest P is 2^x, not 1,
  // and its bf16 rounding (2^-9) would otherwise reach a row dominated by one key in full
  // (C5's outlier keys: 1.74x SDPA's error with the fp32 sum, 0.93x with this one). l_exact then
  // sums the unrounded P for the log-sum-exp output. fp16 rounds P 8x finer, but the same holds
  // on peaky rows: a row's largest P is 2^x with x up to tau, not 1, and its fp16 rounding reached
  // the output with the fp32 sum (fp16 head_dim 64 full attention, inputs x2 to x4: 1.5-2.07x
  // SDPA's error; with the rounded sum 1.0-1.2x). So fp16 sums the rounded P too, at every head
  // dim (the fp32 sum, as in the reference, fa2/kernel.py:98, ran 1.6-2.2% faster at head_dim 64
  // and below: the rounded one spills 2-5 VGPRs in the pipelined loop's three waves per SIMD).
  constexpr bool kRoundedSum = DT == 1 || D == 128 || FA2_FP16_ROUNDED_SUM;
  float m_i = -INFINITY;
  float l_i = 0.f;
  float l_exact = 0.f;
  const bool want_exact = kRoundedSum && p.lse != nullptr;
  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  const float qk_scale = p.qk_scale;

  // The main loop: at head_dim 64 software-pipelined across tiles inside each wave, else
  // one tile at a time with two waves per SIMD overlapping each other (measured per D). The
  // pipelined loop holds two S tiles: at 128-key tiles that spills, so those keep the other.
  constexpr bool kPipelined = (D == 64 || (FA2_PIPE_WIDE && D == 128 && NW == 8)) && BN <= 64;
  if constexpr (!kPipelined) {
    // ---- main loop. Per tile j, one barrier, placed between the two products:
    //   S_j = K_j Q^T                      K_j's operands partly read during PV_{j-1}
    //   wait + barrier                     V_j and K_{j+1} have landed; every wave is past S_j
    //   issue K_{j+2} -> K buffer of K_j, V_{j+1} -> V buffer of V_{j-1}
    //   read the first V_j operands, then mask + softmax_j while they arrive
    //   O += V_j P_j, with V_j operands read LA_V MFMAs ahead and K_{j+1}'s first operands
    //   read in between, so every LDS read has MFMA time to land in.
    constexpr int LA_S = KS < 4 ? KS : 4;        // k-steps of K operands read ahead
    constexpr int NPV = (BN / 16) * DB;          // MFMAs of the PV product
    // PV MFMAs whose V operands are read ahead: 2 at head_dim 128 (+0.7% on C2 and C3 over 4;
    // 3, 6 and 8 in between: the transposing reads land in time either way), else 4
    constexpr int kLaV = D == 128 ? 2 : 4;
    constexpr int LA_V = NPV < kLaV ? NPV : kLaV;
    constexpr int NKP = LA_S * NB;               // K operand reads prefetched during PV
    u32x4 kop[LA_S][NB];
    if (n_iter > 0) {
      if (n_tiles_kv > 0) {
        issue_k(kv_begin, 0);
        issue_v(kv_begin, 0);
      }
      if (n_tiles_kv > 1) issue_k(kv_begin + BN, 1);
      // S_0 needs Q and K_0 only: V_0 and K_1 (this wave's last loads; vector loads complete in
      // order) land while S_0 runs, and the loop's first wait covers them. When the waves issue
      // unequal numbers of loads, or more than the 6-bit counter holds, wait for all.
      if constexpr (NI % GW == 0 && 2 * JW < 64) {
        if (n_tiles_kv > 1) wait_vmcnt<2 * JW>();
        else if (!kSplit || n_tiles_kv > 0) wait_vmcnt<JW>();
        else wait_vmcnt<0>();
      } else {
        wait_vmcnt<0>();
      }
      __syncthreads();
      if constexpr (kTimeline) tl_prologue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
      for (int ks = 0; ks < LA_S; ++ks)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand_v(0, ks, nb);
    }
    // Causal: the last tiles of a program can start past every row of a wave (the second masked
    // tile of a 128-row program, for its first 64 rows). The wave skips their products and
    // softmax, which would add exact zeros, and keeps only its share of the loads and barriers
    // (the loop after this one). Measured +0.2% on C3, +0.5% on C2, +1.9% on C5.
    if (KB) bound = bound_from_table();
    int n_active = n_tiles_kv;
    if (CAUSAL) {
      const int wave_last = __builtin_amdgcn_readlane(pos_vis, 31);  // rows grow with the lane
      if (kSplit && wave_last < kv_begin) n_active = 0;  // group 1: every key is past its rows
      else if (wave_last < kv_end) n_active = min(n_tiles_kv, (wave_last - kv_begin) / BN + 1);
    }
    for (int j = 0; j < n_active; ++j) {
      const int n0 = kv_begin + j * BN;
      const int buf = j & 1;

      // S^T = K Q^T  (fa2/kernel.py:75-79). The two products run at raised wave priority and
      // the softmax at the base one, so that when the two waves of a SIMD meet, the one with
      // matrix work issues first and the other's softmax fills the issue slots the MFMAs leave
      // (3% on MI355X over equal priorities; raising it for only one product gains nothing).
      __builtin_amdgcn_s_setprio(1);
      f32x16 s[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[nb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int slot = ks % LA_S;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb] = E::mma(kop[slot][nb], qreg[ks], s[nb]);
        if (ks + LA_S < KS) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) kop[slot][nb] = k_operand(buf, ks + LA_S, nb);
        }
      }
      // keep the K reads LA_S k-steps ahead of the MFMAs that consume them
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, NB, 0);
        if (ks + LA_S < KS) __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);
      }

      __builtin_amdgcn_s_setprio(0);
      wait_vmcnt<0>();  // this wave's loads of V_j and K_{j+1} have landed
      __syncthreads();                // ... every wave's; and every wave is done with K_j
      if (j + 2 < n_tiles_kv) issue_k(n0 + 2 * BN, buf);
      if (j + 1 < n_tiles_kv) issue_v(n0 + BN, buf ^ 1);

      u32x4 va[LA_V];
#pragma unroll
      for (int i = 0; i < LA_V; ++i) va[i] = v_operand(buf, i / DB, i % DB);

      // masks (fa2/kernel.py:81-88): key n is visible iff n < n_kv and (causal) n <= pos. The
      // condition is uniform over the workgroup (a scalar branch), and one copy of the tile code
      // serves masked and unmasked tiles so the accumulators keep one register assignment.
      if (!kNoSoftmax && (kMaskEveryTile || n0 + BN > full_end)) {
        const int lim = (CAUSAL ? min(pos_vis, p.n_kv - 1) : p.n_kv - 1) - n0 - 8 * g;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (nb * 32 + 16 * (i / 8) + (i % 8) > lim) s[nb][i] = -INFINITY;
      }
      // online softmax in base 2 (fa2/kernel.py:95-98), with a lazily moved reference max
      if constexpr (kScaleFirst) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb] *= qk_scale;
      }
      if (!kNoSoftmax && (!KB || !skip_max)) {
        float mx = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[nb][i]);
        mx = kScaleFirst ? pair_max(mx) : pair_max(mx) * qk_scale;
        const bool grow = !skip_row && mx > m_i + kRescaleTau;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float m_new = grow ? mx : m_i;
          const float alpha = ex2(m_i - m_new);
          l_i *= alpha;
          l_exact *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[db] *= alpha;
          m_i = m_new;
        }
        if (KB && j == 0) {
          const float lift = bound <= kBoundLiftMax<DT> ? kBoundLift<DT> : 0.f;
          skip_row = bound <= m_i + (kBoundTau<DT> + lift);
          if (skip_row) m_i += fmaxf(0.f, ceilf(bound - kBoundTau<DT> - m_i));  // O, l still 0
          skip_max = __builtin_amdgcn_ballot_w64(!skip_row) == 0;
        }
      }
      if constexpr (!kNoSoftmax) {
        // group 1 of the key split can meet rows with no visible key yet (reference -inf): their
        // scores are all -inf, and a reference of 0 gives them weight 0 instead of NaN
        const float m_ref = (kSplit && m_i == -INFINITY) ? 0.f : m_i;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            s[nb][i] = ex2(kScaleFirst ? s[nb][i] - m_ref : __builtin_fmaf(s[nb][i], qk_scale, -m_ref));
        if constexpr (!kRoundedSum) {
          l_i += lane_sum(s);
        } else if (want_exact) {
          l_exact += lane_sum(s);
        }
      }

      // O^T += V^T P^T with P rounded to the input type (fa2/kernel.py:100-105)
      u32x4 pb[BN / 16];
#pragma unroll
      for (int t = 0; t < BN / 16; ++t) {
        const int nb = t >> 1, h = t & 1;
        pb[t] = u32x4{E::pack2(s[nb][8 * h + 0], s[nb][8 * h + 1]),
                      E::pack2(s[nb][8 * h + 2], s[nb][8 * h + 3]),
                      E::pack2(s[nb][8 * h + 4], s[nb][8 * h + 5]),
                      E::pack2(s[nb][8 * h + 6], s[nb][8 * h + 7])};
      }
      if constexpr (kRoundedSum && !kNoSoftmax) {
        float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
        for (int t = 0; t < BN / 16; ++t) {
          rs0 = E::sum2(pb[t][0], rs0);
          rs1 = E::sum2(pb[t][1], rs1);
          rs0 = E::sum2(pb[t][2], rs0);
          rs1 = E::sum2(pb[t][3], rs1);
        }
        l_i += rs0 + rs1;
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        acc[i % DB] = E::mma(va[i % LA_V], pb[i / DB], acc[i % DB]);
        if (i + LA_V < NPV) va[i % LA_V] = v_operand(buf, (i + LA_V) / DB, (i + LA_V) % DB);
        // K_{j+1}'s first operands (a harmless stale read after the last tile)
#pragma unroll
        for (int r = i * NKP / NPV; r < (i + 1) * NKP / NPV; ++r)
          kop[r / NB][r % NB] = k_operand(buf ^ 1, r / NB, r % NB);
      }
      // MFMA i, then the reads it makes room for (V operands LA_V ahead, K prefetch)
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        const int nreads = (i + LA_V < NPV ? 2 : 0) + ((i + 1) * NKP / NPV - i * NKP / NPV);
#pragma unroll
        for (int k = 0; k < nreads; ++k) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }

    for (int j = n_active; j < n_iter; ++j) {
      const int n0 = kv_begin + j * BN;
      wait_vmcnt<0>();
      __syncthreads();
      if (j + 2 < n_tiles_kv) issue_k(n0 + 2 * BN, j & 1);
      if (j + 1 < n_tiles_kv) issue_v(n0 + BN, (j & 1) ^ 1);
    }
    __builtin_amdgcn_s_setprio(0);
  } else {
    // ---- main loop, software-pipelined across tiles. At head_dim 64 a tile's softmax takes
    // more issue time than its MFMAs, and two waves per SIMD overlap one's softmax with the
    // other's MFMAs poorly; each wave therefore interleaves its own. Iteration j runs
    //   block A  S_{j+1} = K_{j+1} Q^T (MFMA)   interleaved with  softmax_j -> P_j (VALU)
    //   wait + barrier                           V_j and K_{j+2} have landed; every wave is
    //                                            done with K_{j+1} and V_{j-1}
    //   issue K_{j+3} -> K buffer of K_{j+1}, V_{j+1} -> V buffer of V_{j-1}
    //   block B  O += V_j P_j (MFMA)            interleaved with  the row max of S_{j+1} and
    //                                            K_{j+2}'s first operand reads
    //   lazy rescale for tile j+1 (rare), after the PV product it must follow
    // (C4: +5-7%; at head_dim 128 the same loop is 3% slower, at 32 5% slower). Same two K and
    // two V buffers; K streams three tiles ahead of its product, V one.
    constexpr int LA = KS < 2 ? KS : 2;                 // k-steps of K operands read ahead
    constexpr int NT = BN / 16;                         // 16-key k-steps of O^T
    constexpr int NPV = NT * DB;                        // MFMAs of the PV product
    constexpr int LA_V = NPV < 4 ? NPV : 4;             // PV MFMAs whose V operands are read ahead
    constexpr int KREAD_EVERY = NPV / (LA * NB) > 0 ? NPV / (LA * NB) : 1;
#ifndef FA2_PIPE_VPM
#define FA2_PIPE_VPM 0
#endif
    // VALU / exp instructions per S MFMA: the tile's softmax VALU work over its 8 S MFMAs (per
    // lane 32 FMAs and 16 conversions, plus 32 adds for the fp32 sum or 16 v_dot2 for the rounded
    // one: 80 or 64 instructions). Measured with the rounded sum (same box, interleaved builds;
    // FA2_PIPE_VPM): 7 is best for the key-norm instances (C4 +1.4% over 8, bf16 full +1.2%), 8
    // for the others (fp16 causal +1.0% over 7); 10, the fp32 sum's 80 / 8, spilled and ran 1-2%
    // slower with the rounded sum.
    constexpr int kVpm = FA2_PIPE_VPM ? FA2_PIPE_VPM
                                      : D == 128 ? 4 : (kRoundedSum ? (KB ? 7 : 8) : 10);
    constexpr int kEpm = D == 128 ? 2 : 4;  // 32 exp2 per tile over its KS * NB S MFMAs
    u32x4 kop[LA][NB];
    float m_new = -INFINITY;

    // S^T = K Q^T for the K tile in `buf` (fa2/kernel.py:75-79); kop holds its first LA k-steps
    auto s_product = [&](f32x16 (&sv)[NB], int buf) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) sv[nb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int slot = ks % LA;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) sv[nb] = E::mma(kop[slot][nb], qreg[ks], sv[nb]);
        if (ks + LA < KS) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) kop[slot][nb] = k_operand(buf, ks + LA, nb);
        }
      }
    };
    // masks (fa2/kernel.py:81-88), as in the other loop
    auto mask_s = [&](f32x16 (&sv)[NB], int n0) {
      const int lim = (CAUSAL ? min(pos_vis, p.n_kv - 1) : p.n_kv - 1) - n0 - 8 * g;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (nb * 32 + 16 * (i / 8) + (i % 8) > lim) sv[nb][i] = -INFINITY;
    };
    // the new reference max (fa2/kernel.py:95), lazily moved; returns whether it moved
    auto row_max = [&](f32x16 (&sv)[NB]) {
      if constexpr (kNoSoftmax) {
        m_new = m_i;
        return false;
      }
      if constexpr (kScaleFirst) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) sv[nb] *= qk_scale;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sv[nb][i]);
      mx = kScaleFirst ? pair_max(mx) : pair_max(mx) * qk_scale;
      const bool grow = !skip_row && mx > m_i + kRescaleTau;
      m_new = grow ? mx : m_i;
      return grow;
    };
    // P = exp2(S * scale - m) rounded to the input type, and l (fa2/kernel.py:96-98, 105)
    auto softmax_p = [&](f32x16 (&sv)[NB], u32x4 (&pb)[NT]) {
      if constexpr (!kNoSoftmax) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            sv[nb][i] = ex2(kScaleFirst ? sv[nb][i] - m_i : __builtin_fmaf(sv[nb][i], qk_scale, -m_i));
        if constexpr (!kRoundedSum) {
          l_i += lane_sum(sv);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int nb = t >> 1, h = t & 1;
        pb[t] = u32x4{E::pack2(sv[nb][8 * h + 0], sv[nb][8 * h + 1]),
                      E::pack2(sv[nb][8 * h + 2], sv[nb][8 * h + 3]),
                      E::pack2(sv[nb][8 * h + 4], sv[nb][8 * h + 5]),
                      E::pack2(sv[nb][8 * h + 6], sv[nb][8 * h + 7])};
      }
      if constexpr (kRoundedSum && !kNoSoftmax) {
        float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          rs0 = E::sum2(pb[t][0], rs0);
          rs1 = E::sum2(pb[t][1], rs1);
          rs0 = E::sum2(pb[t][2], rs0);
          rs1 = E::sum2(pb[t][3], rs1);
        }
        l_i += rs0 + rs1;
      }
    };
    // the unrounded P's sum, for the log-sum-exp output only (a uniform branch)
    auto exact_sum = [&](const f32x16 (&sv)[NB]) {
      if (want_exact) {
        l_exact += lane_sum(sv);
      }
    };
    // O^T += V^T P^T for the V tile in `buf` (fa2/kernel.py:100-105)
    auto pv_product = [&](const u32x4 (&pb)[NT], int buf, u32x4 (&va)[LA_V]) {
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        acc[i % DB] = E::mma(va[i % LA_V], pb[i / DB], acc[i % DB]);
        if (i + LA_V < NPV) va[i % LA_V] = v_operand(buf, (i + LA_V) / DB, (i + LA_V) % DB);
      }
    };
    auto rescale = [&]() {
      const float alpha = ex2(m_i - m_new);
      l_i *= alpha;
      l_exact *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
      m_i = m_new;
    };

    // iteration j (tile j + 1 exists): s_cur holds S_j on entry, s_nxt receives S_{j+1}
    auto iteration = [&](f32x16 (&s_cur)[NB], f32x16 (&s_nxt)[NB], int j) {
      const int bufk = (j + 1) & 1;  // K_{j+1}
      const int bufv = j & 1;        // V_j (and K_{j+2})
      const int n1 = kv_begin + (j + 1) * BN;

      // block A: each S MFMA, then kVpm VALU and kEpm exp instructions of the softmax
      u32x4 pb[NT];
      s_product(s_nxt, bufk);
      softmax_p(s_cur, pb);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int m = 0; m < NB; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kVpm, 0);
          __builtin_amdgcn_sched_group_barrier(0x400, kEpm, 0);
        }
        if (ks + LA < KS) __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);
      }
      // P_j and l must be made here, next to the MFMAs, not sunk past the barrier to their use
#pragma unroll
      for (int t = 0; t < NT; ++t) asm volatile("" ::"v"(pb[t]));
      asm volatile("" ::"v"(l_i));
      exact_sum(s_cur);

      wait_vmcnt<0>();  // V_j and K_{j+2} (this wave's part)
      __syncthreads();  // every wave's; every wave is done with K_{j+1} and V_{j-1}
      if (j + 3 < n_tiles_kv) issue_k(kv_begin + (j + 3) * BN, bufk);
      issue_v(n1, bufv ^ 1);
      if (!kNoSoftmax && (kMaskEveryTile || n1 + BN > full_end)) mask_s(s_nxt, n1);

      // block B: PV_j with the row max of S_{j+1} and K_{j+2}'s first operands in between
      u32x4 va[LA_V];
#pragma unroll
      for (int i = 0; i < LA_V; ++i) va[i] = v_operand(bufv, i / DB, i % DB);
      bool grow = false;
      if (!KB || !skip_max) grow = row_max(s_nxt);
      pv_product(pb, bufv, va);
#pragma unroll
      for (int ks = 0; ks < LA; ++ks)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand(bufv, ks, nb);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * LA_V, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i + LA_V < NPV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if (i % KREAD_EVERY == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      if (__builtin_amdgcn_ballot_w64(grow)) rescale();
    };

    f32x16 s_a[NB], s_b[NB];
    if (n_tiles_kv > 0) {
      // prologue: K_0, V_0, K_1 in flight; S_0 and its row max; then K_2 into K_0's buffer
      issue_k(kv_begin, 0);
      issue_v(kv_begin, 0);
      if (n_tiles_kv > 1) issue_k(kv_begin + BN, 1);
      if constexpr (NI % NW == 0 && 2 * JW < 64) {
        if (n_tiles_kv > 1) wait_vmcnt<2 * JW>();
        else wait_vmcnt<JW>();
      } else {
        wait_vmcnt<0>();
      }
      __syncthreads();
      if constexpr (kTimeline) tl_prologue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
      for (int ks = 0; ks < LA; ++ks)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand_v(0, ks, nb);
      s_product(s_a, 0);
      wait_vmcnt<0>();
      __syncthreads();  // V_0 and K_1 have landed; every wave is done with K_0
      if (n_tiles_kv > 2) issue_k(kv_begin + 2 * BN, 0);
      if (!kNoSoftmax && (kMaskEveryTile || kv_begin + BN > full_end)) mask_s(s_a, kv_begin);
      row_max(s_a);
      m_i = m_new;  // O and l are still zero
      if constexpr (KB) {
        bound = bound_from_table();
        const float lift = bound <= kBoundLiftMax<DT> ? kBoundLift<DT> : 0.f;
        skip_row = bound <= m_i + (kBoundTau<DT> + lift);
        if (skip_row) m_i += fmaxf(0.f, ceilf(bound - kBoundTau<DT> - m_i));
        skip_max = __builtin_amdgcn_ballot_w64(!skip_row) == 0;
      }
#pragma unroll
      for (int ks = 0; ks < LA; ++ks)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand_v(1, ks, nb);  // stale if 1 tile
    }
    // two iterations per trip, so S_j and S_{j+1} alternate between s_a and s_b without copies
    int j = 0;
    for (; j + 2 < n_tiles_kv; j += 2) {
      iteration(s_a, s_b, j);
      iteration(s_b, s_a, j + 1);
    }
    if (j + 1 < n_tiles_kv) {
      iteration(s_a, s_b, j);
      ++j;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s_a[nb] = s_b[nb];
    }
    if (n_tiles_kv > 0) {
      // the last tile (j = n_tiles_kv - 1, in s_a): softmax, then its PV product once V landed
      const int bufv = j & 1;
      u32x4 pb[NT];
      softmax_p(s_a, pb);
      exact_sum(s_a);
      wait_vmcnt<0>();
      __syncthreads();
      u32x4 va[LA_V];
#pragma unroll
      for (int i = 0; i < LA_V; ++i) va[i] = v_operand(bufv, i / DB, i % DB);
      pv_product(pb, bufv, va);
    }
  }

  // ---- key split: group 1 hands its (m, l, O) to group 0 through LDS, lane for lane (the two
  // groups' waves hold the same rows in the same lanes); group 0 merges and stores
  if constexpr (kSplit) {
    static_assert(GW * DB * 16 * 64 * sizeof(float) <= sizeof(k_lds), "O fits the K buffers");
    static_assert(GW * 3 * 64 * sizeof(float) <= sizeof(v_lds), "m, l fit the V buffers");
    __syncthreads();  // every wave is done with every K/V buffer
    float FA2_LDS* ob = (float FA2_LDS*)&k_lds[0][0][0];  // [GW][DB][16][64 lanes]
    float FA2_LDS* sb = (float FA2_LDS*)&v_lds[0][0][0];  // [GW][3][64 lanes]
    if (grp == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) ob[((gwave * DB + db) * 16 + i) * 64 + lane] = acc[db][i];
      sb[(gwave * 3 + 0) * 64 + lane] = m_i;
      sb[(gwave * 3 + 1) * 64 + lane] = l_i;
      sb[(gwave * 3 + 2) * 64 + lane] = l_exact;
    }
    __syncthreads();
    if (grp == 1) return;
    const float mb = sb[(gwave * 3 + 0) * 64 + lane];
    const float m_new = fmaxf(m_i, mb);
    if (m_new != -INFINITY) {  // (no key at all: nothing to merge)
      const float a = ex2(m_i - m_new), b = ex2(mb - m_new);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc[db][i] = acc[db][i] * a + ob[((gwave * DB + db) * 16 + i) * 64 + lane] * b;
      l_i = l_i * a + sb[(gwave * 3 + 1) * 64 + lane] * b;
      l_exact = l_exact * a + sb[(gwave * 3 + 2) * 64 + lane] * b;
      m_i = m_new;
    }
  }

  if constexpr (kTimeline) tl_loop = __builtin_amdgcn_s_memrealtime();

  // ---- normalise once, store once (fa2/kernel.py:178-183)
  // (knockout without softmax: l = 1, as the reference's l_i + 1 on a zero sum)
  const float l = kNoSoftmax ? 1.0f : pair_sum(l_i);
  const float lx = want_exact ? pair_sum(l_exact) : l;
  // one division per row, then multiplies: a per-element fp32 division expands to ~11 VALU
  // instructions (64 per lane at head_dim 128, ~1.6 us per wave in every program's epilogue)
  const float inv_l = 1.0f / l;
  // Staged store: after the loop's last barrier no wave reads the last tile's K buffer or the
  // other V buffer (the next tiles' loads into them were never issued), so the 32 KiB they hold
  // give each wave 8 KiB of its own. A wave writes its 32 rows there (row-major, 16-byte chunks
  // XOR-swizzled by row: conflict-free both ways), reads them back four whole rows per
  // instruction and stores those; no other wave is involved, so no barrier.
  constexpr bool kStagedStore = FA2_STAGED_STORE && D == 128 && BN == 64 && NW == 4 && !kPipelined &&
                                !kSplit && !kNoStore;
  if (kStagedStore && p.splits == 1 && p.pack == 1) {
    const int last = (n_iter - 1) & 1;
    u32x4 FA2_LDS* reg = (gwave < 2 ? (u32x4 FA2_LDS*)k_lds[0][last]
                                    : (u32x4 FA2_LDS*)v_lds[0][last ^ 1]) + (gwave & 1) * 512;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int q = 4 * db + 2 * h + g;  // this lane's dims 8 q .. 8 q + 7 of row c
        reg[c * 16 + (q ^ (c & 15))] =
            u32x4{E::pack2(acc[db][8 * h + 0] * inv_l, acc[db][8 * h + 1] * inv_l),
                  E::pack2(acc[db][8 * h + 2] * inv_l, acc[db][8 * h + 3] * inv_l),
                  E::pack2(acc[db][8 * h + 4] * inv_l, acc[db][8 * h + 5] * inv_l),
                  E::pack2(acc[db][8 * h + 6] * inv_l, acc[db][8 * h + 7] * inv_l)};
      }
    const int qq = lane & 15;
    const int wave_row0 = gwave * 32;
    const int pos0 = pr.tile * p.block_m + wave_row0;  // unpacked: a row's index is its position
    char* obase = (char*)(p.o + pr.b * p.sob + pr.hq0 * p.soh) + qq * 16;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r = 4 * k + (lane >> 4);
      const u32x4 v = reg[r * 16 + (qq ^ (r & 15))];
      if (wave_row0 + r < p.block_m && pos0 + r < p.n_q)
        *(u32x4*)(obase + (int64_t)(pos0 + r) * p.son * 2) = v;
    }
    if (p.lse && g == 0 && row_ok) {
      const int64_t row_index = ((int64_t)pr.b * p.h_q + head) * p.n_q + pos;
      p.lse[row_index] = (m_i + log2f(lx)) * kLn2;
    }
  } else if constexpr (kNoStore) {  // knockout: keep the results alive, store nothing
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) asm volatile("" ::"v"(acc[db][i] * inv_l));
    asm volatile("" ::"v"(lx), "v"(m_i));
  } else if (row_ok) {
    const int64_t row_index = ((int64_t)pr.b * p.h_q + head) * p.n_q + pos;  // in [B, H_q, N_q]
    // log2 of this row's sum of the weights O is normalised by (exp2(s * qk_scale) rounded to
    // the input type) and of the exact exp2(s * qk_scale), over the keys seen; m is their
    // reference
    const float lse2 = m_i + log2f(l);
    const float lse2_exact = m_i + log2f(lx);
    if (p.splits > 1) {
      // split-KV: the normalised partial output (fp32) and its base-2 log-sum-exp
      float* po = p.part_o + ((int64_t)split * p.part_rows + row_index) * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int d0 = 32 * db + 16 * h + 8 * g;
          if (d0 < D) {
            f32x4 lo, hi;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              lo[i] = acc[db][8 * h + i] * inv_l;
              hi[i] = acc[db][8 * h + 4 + i] * inv_l;
            }
            *(f32x4*)(po + d0) = lo;
            *(f32x4*)(po + d0 + 4) = hi;
          }
        }
      if (g == 0) {
        p.part_lse[(int64_t)split * p.part_rows + row_index] = lse2;
        if (p.lse) p.part_lse_exact[(int64_t)split * p.part_rows + row_index] = lse2_exact;
      }
    } else {
      uint16_t* orow = p.o + pr.b * p.sob + head * p.soh + (int64_t)pos * p.son;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int d0 = 32 * db + 16 * h + 8 * g;
          if (d0 < D) {
            const u32x4 o = {E::pack2(acc[db][8 * h + 0] * inv_l, acc[db][8 * h + 1] * inv_l),
                             E::pack2(acc[db][8 * h + 2] * inv_l, acc[db][8 * h + 3] * inv_l),
                             E::pack2(acc[db][8 * h + 4] * inv_l, acc[db][8 * h + 5] * inv_l),
                             E::pack2(acc[db][8 * h + 6] * inv_l, acc[db][8 * h + 7] * inv_l)};
            if constexpr ((FA2_NT_QO & 2) != 0)
              __builtin_nontemporal_store(o, (u32x4*)(orow + d0));
            else
              *(u32x4*)(orow + d0) = o;
          }
        }
      if (p.lse && g == 0) p.lse[row_index] = lse2_exact * kLn2;
    }
  }

  // ---- timeline variant (measurement library): the workgroup's stamps, once every wave's
  // stores have completed. Written by one lane with an ordinary vector store.
  if constexpr (kTimeline) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      uint64_t* rec = p.timeline + (int64_t)block * kTimelineWords;
      rec[0] = tl_entry;
      rec[1] = tl_prologue;
      rec[2] = tl_loop;
      rec[3] = __builtin_amdgcn_s_memrealtime();
      rec[4] = (uint64_t)n_tiles_kv;
      rec[5] = ((uint64_t)__builtin_amdgcn_s_getreg(kHwregXccId) << 32) |
               (uint64_t)__builtin_amdgcn_s_getreg(kHwregHwId);
    }
  }
}

}  // namespace fa2
