/*
 * fa2_ablate.h - C ABI of libfa2_ablate.so, the measurement library of the gfx950
 * FlashAttention-2 forward. It is not part of the drop-in: fa2.kernel never loads it, and
 * libfa2_fwd.so exports none of this.
 *
 * The reference attributes its kernel's time with a knockout copy of the kernel whose switches
 * each change or remove one kind of work (bench/ablation.py:1-20, the copy at 56-202,
 * `attention_ablate` at 182-200). Here every variant is the product's kernel template
 * (attn_fwd_kernel) instantiated with VARIANT bits, so a variant differs from the product in the
 * switched work only. Variants that skip work compute wrong outputs on purpose: only their time
 * means anything.
 *
 * Return convention as in fa2_fwd.h: 0 on success, FA2_EINVAL / FA2_EALIGN / FA2_ELAUNCH on a
 * rejected argument or a failed launch, with fa2_ablate_last_error() describing it.
 */
#ifndef FA2_ABLATE_H
#define FA2_ABLATE_H

#include <stddef.h>
#include <stdint.h>

#include "fa2_fwd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Switch bits (bench/ablation.py:6-17). */
#define FA2_ABLATE_SCALE_FIRST 1       /* scale every score, then subtract the row max: two VALU
                                          instructions per score instead of one FMA (:13-14)   */
#define FA2_ABLATE_MASK_EVERY_TILE 2   /* mask every K/V tile, not only those that need it (:15) */
#define FA2_ABLATE_NO_EXP 8            /* exp2 replaced by its argument, alpha too (:6)         */
#define FA2_ABLATE_NO_SOFTMAX 16       /* no mask, max, exp, sum or rescale: O = (Q K^T) V (:7)  */
#define FA2_ABLATE_KV_L2 32            /* every K/V tile load reads the first tile again, so it
                                          hits L2 instead of HBM (:8-9)                          */
/* Not in the reference: K/V tiles from the third on are not loaded (every tile's products read
 * whichever of the first two tiles its LDS buffer holds; output wrong on purpose): what the
 * HBM/L2 -> LDS staging of K/V costs beyond the first tiles. */
#define FA2_ABLATE_NO_KV_STAGING 256
/* Not in the reference: each workgroup runs its program with 8 waves in two groups of 4 on the
 * same 128 rows, group 0 over the first half of the key range and group 1 over the rest, each
 * with K/V buffers of its own (128 KiB of LDS: one workgroup per CU), and merges the two partial
 * softmax states through LDS before one store. Still attention (another summation order, so
 * not the product's bits); head_dim 128 only (FA2_EINVAL otherwise); always the static order.
 * What halving the longest program's key range buys against losing the second workgroup per
 * CU. */
#define FA2_ABLATE_SPLIT_KEYS 512
/* Not in the reference: a program's fixed cost knocked out (outputs wrong on purpose). NO_Q_LOAD:
 * Q is not read (a lane pattern of small values in its registers); NO_STORE: nothing is written
 * (the results are only kept alive). What hiding a program's Q load or its output store behind
 * another program's tiles could gain at most. */
#define FA2_ABLATE_NO_Q_LOAD 1024
#define FA2_ABLATE_NO_STORE 2048
/* Not a kernel switch and not in the reference: the launch keeps the static order of programs
 * (workgroup b runs program b) where fa2_attn_fwd deals a causal grid's last programs at run
 * time (its dynamic tail). Combines with any variant; the output is the same bit for bit. */
#define FA2_ABLATE_STATIC_ORDER 128

/*
 * fa2_ablate_attn_fwd - the forward kernel with the switches in `variant`.
 *
 *   variant  one of the reference's variants (bench/ablation.py:42-53):
 *              0                                          copy (the product kernel, bit for bit
 *                                                         equal to fa2_attn_fwd's launch)
 *              FA2_ABLATE_SCALE_FIRST                     scale_first
 *              FA2_ABLATE_MASK_EVERY_TILE                 mask_every_tile
 *              FA2_ABLATE_SCALE_FIRST | ..._MASK_EVERY_TILE   before_fixes
 *              FA2_ABLATE_NO_EXP                          no_exp
 *              FA2_ABLATE_NO_SOFTMAX                      no_softmax
 *              FA2_ABLATE_KV_L2                           kv_l2
 *              FA2_ABLATE_NO_SOFTMAX | FA2_ABLATE_KV_L2   matmul_only
 *              FA2_ABLATE_NO_KV_STAGING                   no_kv_staging (not in the reference)
 *              FA2_ABLATE_SPLIT_KEYS                      split_keys (not in the reference)
 *            each optionally with FA2_ABLATE_STATIC_ORDER;
 *            other bit sets are rejected (FA2_EINVAL).
 * The other arguments are fa2_attn_fwd's (include/fa2_fwd.h), with the same checks. Runs at the
 * default configuration (block_m 128, fa2_default_config's block_n), without split-KV, the
 * log-sum-exp or the key-norm table: variant 0 is exactly fa2_attn_fwd's kernel.
 */
FA2_API int fa2_ablate_attn_fwd(const void* q, const void* k, const void* v, void* out,
                                const int64_t q_stride[4], const int64_t k_stride[4],
                                const int64_t v_stride[4], const int64_t o_stride[4],
                                int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                                int32_t n_kv, int32_t head_dim, int32_t dtype, int32_t causal,
                                int32_t pack, float qk_scale, int32_t variant, void* stream);

/* Words per workgroup that fa2_ablate_timeline records. */
#define FA2_ABLATE_TIMELINE_WORDS 6

/*
 * fa2_ablate_timeline - the product kernel (variant 0, same output bit for bit) with a timeline,
 * in the product's schedule (its dynamic tail included): the workgroup that runs program b (its
 * place in the static order) writes FA2_ABLATE_TIMELINE_WORDS uint64 at records[6 b ...]:
 *   [0] entry, [1] prologue done (Q and the first K/V tiles in, first barrier passed),
 *   [2] tile loop done, [3] stores done (after a wait for them): s_memrealtime, 100 MHz;
 *   [4] the workgroup's K/V tile count;
 *   [5] XCC_ID << 32 | HW_ID (hardware ids of the wave that wrote: CU, shader array, engine).
 * It waits for its stores before the last stamp, which the product does not do. No counterpart
 * in the reference (its profiling used Nsight); a measurement tool for the schedule of short
 * grids. records: device memory, 8-byte aligned, at least 6 x programs words (record_words),
 * where programs = ceil(n_q * pack / 128) * batch * h_q / pack; else FA2_EINVAL, no launch.
 * (The dynamic tail's spare workgroups, which find no program, write nothing.)
 */
FA2_API int fa2_ablate_timeline(const void* q, const void* k, const void* v, void* out,
                                const int64_t q_stride[4], const int64_t k_stride[4],
                                const int64_t v_stride[4], const int64_t o_stride[4],
                                int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                                int32_t n_kv, int32_t head_dim, int32_t dtype, int32_t causal,
                                int32_t pack, float qk_scale, uint64_t* records,
                                int64_t record_words, void* stream);

/* Modes of fa2_ablate_mfma_ceiling. */
#define FA2_ABLATE_CEIL_MFMA 0              /* random bf16 operands in registers            */
#define FA2_ABLATE_CEIL_MFMA_CONST 1        /* the same with constant operands (1.0)        */
#define FA2_ABLATE_CEIL_MFMA_LDS 2          /* random, one 1 KiB ds_read_b128 per MFMA      */
#define FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX 3  /* that plus the softmax's vector work per MFMA */
#define FA2_ABLATE_CEIL_MFMA_EXP 4          /* random, registers, one exp2 per MFMA          */
#define FA2_ABLATE_CEIL_MFMA_FMA2 5         /* random, registers, two FMAs per MFMA          */
#define FA2_ABLATE_CEIL_MFMA_LDS_SOFTMAX_VACC 6  /* mode 3 with the accumulators in VGPRs    */
#define FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC 7  /* mode 6, one read per two MFMAs, 4 accs  */
#define FA2_ABLATE_CEIL_HALF_LDS_SOFTMAX_VACC_1WAVE 8  /* mode 7, one wave per SIMD           */
#define FA2_ABLATE_CEIL_LDS_SOFTMAX64_VACC_3WAVE 9  /* mode 6 with head_dim 64's softmax per MFMA,
                                                       three waves per SIMD                    */
#define FA2_ABLATE_CEIL_MAX_WORKGROUPS 65536
#define FA2_ABLATE_CEIL_MAX_ITERS 100000

/*
 * fa2_ablate_mfma_ceiling - what the matrix cores sustain on this chip with the attention
 * kernel's launch shape (256-thread workgroups, 64 KiB LDS each: two per CU): every wave issues
 * iters x 16 v_mfma_f32_32x32x16_bf16 (32768 FLOP each) on two independent accumulators, with
 * the per-MFMA extra work of `mode` (FA2_ABLATE_CEIL_*) on independent data. One launch does
 * workgroups x 4 x iters x 16 x 32768 FLOP. The chip lowers its clock to hold its power limit,
 * and an MFMA's energy depends on its operands, so the rate depends on the mode and on how long
 * it runs; time it back to back for a second or more. Modes 7 and 8 price the operand reads of
 * 64-row waves (each K/V operand read feeds two MFMAs); mode 8 launches 128 KiB of LDS per
 * workgroup, so one workgroup (one wave per SIMD) per CU. Mode 9 is the head_dim-64 kernel's mix
 * (two scores, two exp2, one pack and one dot2 per MFMA) at its occupancy: 48 KiB of LDS per
 * workgroup, three workgroups (three waves per SIMD) per CU. No counterpart in the reference: a
 * measurement tool for the roofline's practical ceiling. out: device memory, 4-byte aligned,
 * at least workgroups x 256 floats (out_words); its values mean nothing. FA2_EINVAL for a
 * mode, workgroup or iteration count out of range, before any launch.
 */
FA2_API int fa2_ablate_mfma_ceiling(int32_t mode, int32_t workgroups, int32_t iters, float* out,
                                    int64_t out_words, void* stream);

/*
 * fa2_ablate_hbm_read - the memory-side ceiling: workgroups x 256 threads read `bytes` of src
 * (16 bytes per lane per load, four loads in flight per lane, grid-stride) and each thread writes
 * one word of out (meaningless). Time it back to back over a buffer far larger than the caches
 * (the Infinity Cache holds 256 MiB) for the read rate HBM sustains. No counterpart in the
 * reference: a measurement tool for the few-queries regime's roofline. src: 16-byte aligned,
 * bytes a positive multiple of 16; out: 4-byte aligned, at least workgroups x 256 words.
 */
FA2_API int fa2_ablate_hbm_read(const void* src, int64_t bytes, uint32_t* out, int64_t out_words,
                                int32_t workgroups, void* stream);

/*
 * fa2_ablate_tail_schedule - the dynamic tail fa2_attn_fwd gives a launch at the default
 * configuration (block_m 128, the default block_n, no split-KV) on MI355X's topology (256 CUs,
 * 8 XCDs): of its programs, the first *static_blocks run in the static order and the last
 * *tail_programs are dealt at run time to *tail_workgroups workgroups (the spare ones find no
 * program). All three are 0 when the launch keeps the static order (non-causal, or fewer than
 * two rounds of programs per XCD). Host-side policy only, no GPU call. FA2_EINVAL for sizes
 * attention would reject (h_q % h_kv, head_dim, pack not 1 or the group).
 */
FA2_API int fa2_ablate_tail_schedule(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                                     int32_t head_dim, int32_t causal, int32_t pack,
                                     int32_t* static_blocks, int32_t* tail_programs,
                                     int32_t* tail_workgroups);

/* Words fa2_ablate_program_map writes to info. */
#define FA2_ABLATE_MAP_INFO_WORDS 11

/*
 * fa2_ablate_program_map - which program every workgroup of a launch runs, computed on the CPU
 * with the kernel's own code (program_of and the dynamic tail's ticket rules, which are
 * __host__ __device__) on a device of `cus` CUs and `xcds` XCDs. The launch is fa2_attn_fwd's on
 * contiguous tensors of these sizes (n_kv = n_q) at block_m rows and the default tile, without
 * split-KV; static_order != 0 keeps the static order (FA2_ABLATE_STATIC_ORDER).
 * tail_private_pct is the share of each XCD's tail programs its own queue holds: -1 for the
 * library's (what fa2_attn_fwd launches), or 0..100 to plan another build's policy (the
 * FA2_TAIL_PRIVATE_PCT a variant build is compiled with). The dynamic tail's workgroups take
 * their tickets in a random order seeded by `seed`, with the kernel's wrapping increments
 * emulated on the host.
 *   programs  [grid][3] int32: (q tile, batch, first query head) of the program workgroup w runs,
 *             or (-1, -1, -1) for a spare tail workgroup; program_words >= 3 x grid.
 *   info      [FA2_ABLATE_MAP_INFO_WORDS]: grid (workgroups), static blocks, tail workgroups,
 *             tail queues, private programs per queue, shared programs, unit chunk, log2 of
 *             the XCDs the order uses, ticket words left nonzero after the launch (0: every word
 *             wrapped back), q tiles per head group (n_tiles), head groups (batch x h_q / pack).
 * No counterpart in the reference, and no GPU call: the CPU check that every program runs once.
 */
FA2_API int fa2_ablate_program_map(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                                   int32_t head_dim, int32_t causal, int32_t pack, int32_t block_m,
                                   int32_t cus, int32_t xcds, int32_t static_order,
                                   int32_t tail_private_pct, uint32_t seed, int32_t* programs,
                                   int64_t program_words, int32_t* info, int32_t info_words);

/*
 * fa2_ablate_tail_launches - how many launches of this library (fa2_ablate_attn_fwd,
 * fa2_ablate_timeline) ran with a dynamic tail so far in this process: a launch recorded under
 * stream capture runs the static order and does not count. No counterpart in the reference.
 */
FA2_API long long fa2_ablate_tail_launches(void);

/* Thread-local description of this library's last failure in this thread ("" if none). */
FA2_API const char* fa2_ablate_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FA2_ABLATE_H */
