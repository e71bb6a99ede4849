// attn_fwd_r64.hpp - the gfx950 FlashAttention-2 forward kernel with 64 query rows per wave.
//
// Same computation and the same operand layouts as attn_fwd_kernel.hpp (that file's header
// explains the transposed products S^T = K Q^T and O^T += V^T P^T, the pi row order of K, the
// transposing V reads and the XOR-swizzled LDS tiles). What changes is the work per wave:
//
//   * A wave owns 64 query rows, i.e. two 32-column blocks of every accumulator. Each K or V
//     operand read from LDS feeds two MFMAs, which halves LDS bytes per FLOP (64 FLOP/B). With
//     32 rows per wave the LDS reads plus the K/V staging alone took about half of the kernel
//     time on MI355X (LDS reads near 150 B/clk/CU); at 64 rows they need about a third of that.
//   * One wave per SIMD: Q (KS x 2 x 4 regs) and the O accumulators (2 x D/32 x 16 regs) are
//     large and only MFMAs touch them, so they can live in the AGPR half of the register file.
//   * The latency that a second wave used to hide is hidden inside the wave by software
//     pipelining across tiles. Iteration j runs
//       block A:  S_{j+1} = K_{j+1} Q^T (MFMA)   interleaved with   softmax of S_j -> P_j (VALU)
//       barrier
//       block B:  O += V_j P_j (MFMA)            interleaved with   row max of S_{j+1} (VALU),
//                                                                   V_j operand reads (LDS) and
//                                                                   K_{j+2}'s first operands
//       lazy rescale of O (rare), after the PV product it must follow
//     so the matrix core has independent VALU work next to it in both halves, and every LDS
//     read is issued well before the MFMA that consumes it.
//   * K tiles stream HBM -> LDS three tiles ahead of their product and V tiles one ahead,
//     through two K and two V buffers; one barrier per tile orders every reuse.
//   * Register classes are pinned with empty (non-volatile) inline asm: Q and O in AGPRs (MFMA
//     operands only), S in VGPRs (the softmax reads it); and P_j is "used" by an empty volatile
//     asm before the barrier, otherwise the compiler sinks the softmax below the barrier to
//     where P is consumed and nothing is left to overlap with block A's MFMAs.
//   * 32-key tiles keep the whole working set (two S buffers, P, operands in flight, Q, O)
//     inside one wave's 512 registers without spills; 64-key tiles do not.
#pragma once

#include "attn_fwd_common.hpp"

namespace fa2 {

template <int DT, int D, int NW, int BN, bool CAUSAL, int MB>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(MB == 1 ? 2 : 1, MB == 1 ? 2 : 1)))
void attn_fwd_pipe_kernel(const Params p) {
  using E = Elem<DT>;
  // MB 32-row query blocks per wave: MB = 2 runs one wave per SIMD, MB = 1 two.
  constexpr int KS = D / 16;               // 16-dim k-steps of S^T
  constexpr int DB = D / 32;               // 32-dim row blocks of O^T
  constexpr int NB = BN / 32;              // 32-key row blocks of S^T
  constexpr int NT = BN / 16;              // 16-key k-steps of O^T
  constexpr int CPR = D / 8;               // 16-byte chunks per K / V row
  constexpr int TCH = BN * CPR;            // chunks per K (or V) tile
  constexpr int NI = TCH / 64;             // 64-lane LDS load instructions per tile
  constexpr int JW = (NI + NW - 1) / NW;   // of which this wave issues
  constexpr int LA = KS < 2 ? KS : 2;      // k-steps of K operands read ahead
  constexpr int NPV = NT * DB;             // V operands per tile
  constexpr int LA_V = NPV < 4 ? NPV : 4;  // V operands read ahead
  static_assert(D >= 64 && D % 32 == 0, "64-row waves are built for head_dim 64 and 128");
  static_assert(TCH % 64 == 0, "a tile must be whole 1 KiB load instructions");

  __shared__ u32x4 k_lds[2][TCH];
  __shared__ u32x4 v_lds[2][TCH];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS addresses stay scalar
  const int lane = tid & 63;
  const int c = lane & 31;
  const int g = lane >> 5;

  const Program pr = program_of<CAUSAL>(p, blockIdx.x);

  // ---- this lane's two query rows (fa2/kernel.py:135-139)
  int pos[MB], head[MB], pos_vis[MB];
  bool row_ok[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int lrow = wave * (32 * MB) + mb * 32 + c;
    const int r = pr.tile * p.block_m + lrow;
    pos[mb] = r / p.pack;
    head[mb] = pr.hq0 + (r - pos[mb] * p.pack);
    row_ok[mb] = lrow < p.block_m && pos[mb] < p.n_q;
    pos_vis[mb] = row_ok[mb] ? pos[mb] : 0x3fffffff;
  }

  // ---- Q^T operands, loaded once (fa2/kernel.py:144)
  u32x4 qreg[MB][KS];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const uint16_t* qrow = p.q + pr.b * p.sqb + head[mb] * p.sqh + (int64_t)pos[mb] * p.sqn + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qreg[mb][ks] = row_ok[mb] ? *(const u32x4*)(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
  }
  // Q is only ever an MFMA operand: keep it in AGPRs and leave the VGPRs to S and P.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm("" : "+a"(qreg[mb][ks]));

  // ---- key range (fa2/kernel.py:150-175)
  const int pos_per_prog = p.block_m / p.pack;
  const int lo_pos = pr.tile * pos_per_prog;
  int kv_end, full_end;
  if (CAUSAL) {
    kv_end = min(lo_pos + pos_per_prog, p.n_kv);
    full_end = (lo_pos / BN) * BN;
  } else {
    kv_end = p.n_kv;
    full_end = (p.n_kv / BN) * BN;
  }
  const int n_tiles_kv = (kv_end + BN - 1) / BN;

  // ---- K/V staging HBM -> LDS (see attn_fwd_kernel.hpp)
  const char* kbase = (const char*)(p.k + pr.b * p.skb + pr.hkv * p.skh);
  const char* vbase = (const char*)(p.v + pr.b * p.svb + pr.hkv * p.svh);
  uint32_t koff[JW], voff[JW];
#pragma unroll
  for (int jj = 0; jj < JW; ++jj) {
    const int P = (wave + jj * NW) * 64 + lane;
    const int row = P / CPR, col = P % CPR;
    koff[jj] = (uint32_t)(row * p.skn + (col ^ k_key<D>(pi_row(row & 31) & 15)) * 8) * 2u;
    voff[jj] = (uint32_t)(row * p.svn + (col ^ v_key<D>(row & 15)) * 8) * 2u;
  }
  auto rsrc_at = [&](const char* base, int64_t stride, int n0) {
    const int64_t rows_left = p.n_kv - n0;  // >= 1
    const int64_t bytes = ((rows_left - 1) * stride + D) * 2;
    return make_desc(base + (int64_t)n0 * stride * 2, (uint32_t)min(bytes, (int64_t)0x7fffffff));
  };
  auto issue_k = [&](int n0, int buf) {
    const auto rs = rsrc_at(kbase, p.skn, n0);
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
      const int j = wave + jj * NW;
      if (NI % NW == 0 || j < NI) load_lds16(rs, koff[jj], lds_addr(&k_lds[buf][j * 64]));
    }
  };
  auto issue_v = [&](int n0, int buf) {
    const auto rs = rsrc_at(vbase, p.svn, n0);
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
      const int j = wave + jj * NW;
      if (NI % NW == 0 || j < NI) load_lds16(rs, voff[jj], lds_addr(&v_lds[buf][j * 64]));
    }
  };

  // ---- LDS operand reads
  const int kk = k_key<D>(c & 15);
  const int vs = lane & 15;
  const int vj = vs >> 2;
  const int vq = vs & 3;
  const int vsig = ((vq & 1) << 1) | ((vq & 2) >> 1);
  const int vdh = (lane >> 4) & 1;
  auto k_operand = [&](int buf, int ks, int nb) {
    const u32x4 FA2_LDS* kt = (const u32x4 FA2_LDS*)k_lds[buf];
    return kt[(nb * 32 + pi_row(c)) * CPR + ((2 * ks + g) ^ kk)];
  };
  // The same read, volatile: issued outside the loop, so that the compiler cannot merge it with
  // the in-loop prefetch into one load at the top of the loop.
  auto k_operand_v = [&](int buf, int ks, int nb) {
    const volatile u32x4 FA2_LDS* kt = (const volatile u32x4 FA2_LDS*)k_lds[buf];
    return kt[(nb * 32 + pi_row(c)) * CPR + ((2 * ks + g) ^ kk)];
  };
  auto v_operand = [&](int buf, int t, int db) {
    const char FA2_LDS* vt = (const char FA2_LDS*)v_lds[buf];
    u32x2 part[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int row = 16 * t + 8 * g + 4 * rr + vj;
      const int chunk = (4 * db + 2 * vdh + (vsig >> 1)) ^ v_key<D>(row & 15);
      part[rr] = lds_read_tr(vt + row * (D * 2) + chunk * 16 + (vsig & 1) * 8);
    }
    return u32x4{part[0][0], part[0][1], part[1][0], part[1][1]};
  };

  // ---- online-softmax state (fa2/kernel.py:146-148); l is a per-lane partial sum
  float m_i[MB], l_i[MB], m_new[MB];
  f32x16 acc[MB][DB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    m_i[mb] = -INFINITY;
    l_i[mb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[mb][db] = f32x16{};
  }
  const float qk_scale = p.qk_scale;
  u32x4 kop[LA][NB];  // K operands of the next product's first LA k-steps

  // S^T = K Q^T for the K tile in `buf` (fa2/kernel.py:75-79); kop holds its first LA k-steps
  auto s_product = [&](f32x16 (&s)[MB][NB], int buf) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[mb][nb] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int slot = ks % LA;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) s[mb][nb] = E::mma(kop[slot][nb], qreg[mb][ks], s[mb][nb]);
      if (ks + LA < KS) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) kop[slot][nb] = k_operand(buf, ks + LA, nb);
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) asm("" : "+v"(s[mb][nb]));
  };
  // masks (fa2/kernel.py:81-88): key n is visible iff n < n_kv and (causal) n <= pos
  auto mask_s = [&](f32x16 (&s)[MB][NB], int n0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int lim = (CAUSAL ? min(pos_vis[mb], p.n_kv - 1) : p.n_kv - 1) - n0 - 8 * g;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (nb * 32 + 16 * (i / 8) + (i % 8) > lim) s[mb][nb][i] = -INFINITY;
    }
  };
  // new reference max per row (fa2/kernel.py:95); moves only when it grows by more than tau
  auto row_max = [&](const f32x16 (&s)[MB][NB]) {
    bool grow_any = false;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float mx = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[mb][nb][i]);
      mx = pair_max(mx) * qk_scale;
      const bool grow = mx > m_i[mb] + kRescaleTau;
      m_new[mb] = grow ? mx : m_i[mb];
      grow_any |= grow;
    }
    return grow_any;
  };
  // P = exp2(S * scale - m) (fa2/kernel.py:96-98), rounded to the input type (fa2/kernel.py:105)
  // bf16: l sums P rounded to bf16, the weights the PV product uses; fp16: the fp32 P (as in
  // attn_fwd_kernel.hpp, whose header says why)
  auto softmax_p = [&](f32x16 (&s)[MB][NB], u32x4 (&pb)[MB][NT]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[mb][nb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mb][nb][i], qk_scale, -m_i[mb]));
          if constexpr (DT == 0) rs0 += s[mb][nb][i];
        }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int nb = t >> 1, h = t & 1;
        pb[mb][t] = u32x4{E::pack2(s[mb][nb][8 * h + 0], s[mb][nb][8 * h + 1]),
                          E::pack2(s[mb][nb][8 * h + 2], s[mb][nb][8 * h + 3]),
                          E::pack2(s[mb][nb][8 * h + 4], s[mb][nb][8 * h + 5]),
                          E::pack2(s[mb][nb][8 * h + 6], s[mb][nb][8 * h + 7])};
        if constexpr (DT == 1) {
          rs0 = E::sum2(pb[mb][t][0], rs0);
          rs1 = E::sum2(pb[mb][t][1], rs1);
          rs0 = E::sum2(pb[mb][t][2], rs0);
          rs1 = E::sum2(pb[mb][t][3], rs1);
        }
      }
      l_i[mb] += rs0 + rs1;
    }
  };
  // O^T += V^T P^T for the V tile in `buf` (fa2/kernel.py:100-105)
  auto pv_product = [&](const u32x4 (&pb)[MB][NT], int buf, u32x4 (&va)[LA_V]) {
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
      {
        acc[mb][i % DB] = E::mma(va[i % LA_V], pb[mb][i / DB], acc[mb][i % DB]);
        asm("" : "+a"(acc[mb][i % DB]));
      }
      if (i + LA_V < NPV) va[i % LA_V] = v_operand(buf, (i + LA_V) / DB, (i + LA_V) % DB);
    }
  };
  auto rescale = [&]() {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const float alpha = __builtin_amdgcn_exp2f(m_i[mb] - m_new[mb]);
      l_i[mb] *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[mb][db] *= alpha;
      m_i[mb] = m_new[mb];
    }
  };

  // iteration j: block A (S_{j+1} || softmax_j), barrier, block B (PV_j || row max of S_{j+1}),
  // lazy rescale. s_cur holds S_j on entry; s_nxt receives S_{j+1}.
  auto iteration = [&](f32x16 (&s_cur)[MB][NB], f32x16 (&s_nxt)[MB][NB], int j) {
    const int bufk = (j + 1) & 1;  // holds K_{j+1}
    const int bufv = j & 1;        // holds V_j
    const int n1 = (j + 1) * BN;

    // block A: S_{j+1} on the matrix core while the VALU turns S_j into P_j
    u32x4 pb[MB][NT];
    s_product(s_nxt, bufk);
    softmax_p(s_cur, pb);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int m = 0; m < NB * MB; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);   // exp
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);   // other VALU
      }
      if (ks + LA < KS) __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);  // next K reads
    }

    // P_j and l must be computed here, next to the MFMAs, not sunk to their use after the barrier
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int t = 0; t < NT; ++t) asm volatile("" ::"v"(pb[mb][t]));
      asm volatile("" ::"v"(l_i[mb]));
    }
    wait_vmcnt<0>();  // K_{j+2} and V_j have landed (this wave's part)
    __syncthreads();                // ... every wave's; every wave is done with K_{j+1}
    if (j + 3 < n_tiles_kv) issue_k((j + 3) * BN, bufk);
    issue_v(n1, bufv ^ 1);
    if (n1 + BN > full_end) mask_s(s_nxt, n1);

    // block B: O += V_j P_j on the matrix core; row max of S_{j+1}; K_{j+2}'s first operands
    u32x4 va[LA_V];
#pragma unroll
    for (int i = 0; i < LA_V; ++i) va[i] = v_operand(bufv, i / DB, i % DB);
    const bool grow = row_max(s_nxt);
    pv_product(pb, bufv, va);
#pragma unroll
    for (int ks = 0; ks < LA; ++ks)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand(bufv, ks, nb);  // K_{j+2}: buffer j & 1
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * LA_V, 0);  // first V operands
    __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);         // row max
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);
      if (i + LA_V < NPV) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      if (i % (NPV / (LA * NB)) == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }

    // lazy rescale for tile j+1, after the PV product it must follow
    if (__builtin_amdgcn_ballot_w64(grow)) rescale();
  };

  f32x16 s_a[MB][NB], s_b[MB][NB];
  if (n_tiles_kv > 0) {
    // prologue: K_0, V_0, K_1 in flight; S_0 and its row max; then K_2 into K_0's buffer
    issue_k(0, 0);
    issue_v(0, 0);
    if (n_tiles_kv > 1) issue_k(BN, 1);
    wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < LA; ++ks)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand_v(0, ks, nb);
    s_product(s_a, 0);
    if (BN > full_end) mask_s(s_a, 0);
    row_max(s_a);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) m_i[mb] = m_new[mb];  // O and l are still zero
#pragma unroll
    for (int ks = 0; ks < LA; ++ks)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) kop[ks][nb] = k_operand_v(1, ks, nb);
    __syncthreads();  // every wave is done with K_0
    if (n_tiles_kv > 2) issue_k(2 * BN, 0);
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
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s_a[mb][nb] = s_b[mb][nb];
  }

  if (n_tiles_kv > 0) {
    // the last tile (j = n_tiles_kv - 1, in s_a): softmax, then its PV product once V landed
    const int bufv = j & 1;
    u32x4 pb[MB][NT];
    softmax_p(s_a, pb);
    wait_vmcnt<0>();
    __syncthreads();
    u32x4 va[LA_V];
#pragma unroll
    for (int i = 0; i < LA_V; ++i) va[i] = v_operand(bufv, i / DB, i % DB);
    pv_product(pb, bufv, va);
  }

  // ---- normalise once, store once (fa2/kernel.py:178-183)
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const float l = pair_sum(l_i[mb]);
    if (row_ok[mb]) {
      uint16_t* orow = p.o + pr.b * p.sob + head[mb] * p.soh + (int64_t)pos[mb] * p.son;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int d0 = 32 * db + 16 * h + 8 * g;
          const u32x4 o = {E::pack2(acc[mb][db][8 * h + 0] / l, acc[mb][db][8 * h + 1] / l),
                           E::pack2(acc[mb][db][8 * h + 2] / l, acc[mb][db][8 * h + 3] / l),
                           E::pack2(acc[mb][db][8 * h + 4] / l, acc[mb][db][8 * h + 5] / l),
                           E::pack2(acc[mb][db][8 * h + 6] / l, acc[mb][db][8 * h + 7] / l)};
          *(u32x4*)(orow + d0) = o;
        }
    }
  }
}

}  // namespace fa2
