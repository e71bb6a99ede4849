/*
 * fa2_fwd.h - C ABI of the gfx950 (MI355X) FlashAttention-2 forward.
 *
 * The reference (roy6n23/triton-fa2-forward) reaches its GPU through one Triton launch,
 * `_attn_fwd[grid](q, k, v, out, 16 strides, H_Q, N_Q, N_KV, qk_scale, constexprs...)`
 * at fa2/kernel.py:247-259, and keeps its host policy in Python
 * (`_default_config` fa2/kernel.py:186-195, `should_pack_gqa` fa2/kernel.py:198-207).
 * This header is what a host binds instead: plain pointers, element strides and sizes,
 * no torch types. Device buffers are owned by the caller; the library allocates nothing
 * per call and keeps no per-call state. Launches are asynchronous on the given stream.
 *
 * Causal grids of at least two rounds of programs per XCD deal their last programs at run time
 * (a dynamic tail): their workgroups take tickets from counter words in the library's own device
 * memory (a static array, loaded as zeros; no allocation), which every launch leaves at zero
 * again. Each (device, stream) has its own set of words, made at the stream's first such launch
 * together with one event (hipEventCreateWithFlags; the only object the library creates for a
 * stream), so calls on different streams and threads may overlap freely; a launch that uses a set
 * first makes its stream wait for the event, which the set's previous launch signalled when it
 * ended (its stop event), so a stream created with the handle of a destroyed one never meets the
 * old stream's launches on the words. Launches recorded under stream capture,
 * launches on the per-thread default stream or on a stream of another device than the current
 * one, and launches past 256 streams per device run the static order instead. Either way the
 * output is the same, bit for bit. The order of programs follows the device's CU and XCD counts,
 * read once per device.
 *
 * Return convention: 0 on success, a negative FA2_E* code on a rejected argument or a
 * failed launch; fa2_last_error() then describes the failure (thread-local string).
 */
#ifndef FA2_FWD_H
#define FA2_FWD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of q, k, v and out (all four share it), fa2/kernel.py:222. */
#define FA2_DTYPE_F16 0
#define FA2_DTYPE_BF16 1

/* Every entry point is exported from the shared library; everything else in it is hidden. */
#if defined(__GNUC__)
#define FA2_API __attribute__((visibility("default")))
#else
#define FA2_API
#endif

#define FA2_OK 0
#define FA2_EINVAL (-1)      /* an argument violates the contract below */
#define FA2_EALIGN (-2)      /* a pointer or stride breaks the 16-byte load rule */
#define FA2_ELAUNCH (-3)     /* the HIP launch itself failed */

/*
 * fa2_attn_fwd - out = softmax(q k^T * sm_scale [+ top-left causal mask]) v, fused.
 *
 * Replaces the launch `_attn_fwd[grid](...)` (fa2/kernel.py:247-259), with the kernel
 * `_attn_fwd` (fa2/kernel.py:110-183) and its loop `_attn_fwd_inner` (fa2/kernel.py:60-107).
 *
 *   q, out   [batch, h_q,  n_q,  head_dim]   device pointers
 *   k, v     [batch, h_kv, n_kv, head_dim]
 *   *_stride element strides in [b, h, n, d] order; the d stride must be 1, the others
 *            multiples of 8 elements, and every base pointer 16-byte aligned (FA2_EALIGN).
 *   head_dim in {16, 32, 64, 128};  h_q % h_kv == 0;  causal implies n_q == n_kv
 *            (fa2/kernel.py:218-228).
 *   dtype    FA2_DTYPE_F16 or FA2_DTYPE_BF16.
 *   pack     1, or the GQA group h_q / h_kv: that many query heads share one program
 *            (fa2/kernel.py:233-238); block_m must then be a multiple of pack.
 *   block_m  rows of (position, head) pairs per program, 1..256 (fa2/kernel.py:135-137).
 *   block_n  keys per K/V tile; 0 takes fa2_default_config's (64; 128 at head_dim 16). The
 *            kernel streams K/V in tiles of 32, 64 or 128 keys and rounds block_n up to the
 *            next of these.
 *   qk_scale sm_scale * log2(e) > 0 (fa2/kernel.py:240-244).
 *   stream   a hipStream_t (NULL = the default stream of the current device).
 *   Limits (FA2_EINVAL): at most 2^31 - 1 programs, ceil(n_q * pack / block_m) *
 *            batch * h_q / pack (times the splits of fa2_attn_fwd_ex); k and v sequence
 *            strides of at most 2^22 elements (K/V tiles are addressed with 32-bit offsets).
 */
FA2_API int fa2_attn_fwd(const void* q, const void* k, const void* v, void* out,
                         const int64_t q_stride[4], const int64_t k_stride[4],
                         const int64_t v_stride[4], const int64_t o_stride[4],
                         int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                         int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                         int32_t block_m, int32_t block_n, float qk_scale, void* stream);

/*
 * fa2_attn_fwd_ex - fa2_attn_fwd with two optional extensions the reference does not have
 * (its README.md:308-315 lists both as missing): the log-sum-exp of every row and split-KV,
 * and with a workspace that can also hold a key-norm table. No counterpart in the reference's
 * launch; fa2_attn_fwd(...) is fa2_attn_fwd_ex(..., NULL, 1, NULL, 0, stream).
 *
 *   lse        NULL, or device float[batch * h_q * n_q] (4-byte aligned), row
 *              (b * h_q + h) * n_q + i: log sum_n exp(q_i . k_n * sm_scale) over the keys
 *              row i sees, natural log (the softmax_lse of FlashAttention's backward).
 *   num_splits 1..16. Above 1 (causal == 0 only), every program's key range is cut into
 *              that many pieces of whole K/V tiles (fewer if the key range is shorter), one
 *              workgroup each, and a second kernel merges the pieces. For grids too small
 *              to fill the GPU: few queries against a long K/V. fa2_num_splits() picks it.
 *   workspace  device memory, 256-byte aligned, owned by the caller and untouched until the
 *              launch has run; may be NULL when num_splits == 1. It must hold at least
 *              fa2_workspace_bytes(batch, h_q, n_q, head_dim, num_splits) bytes (the split-KV
 *              partials, 0 without split-KV). fa2_workspace_bytes_for() adds room for a
 *              key-norm table where it pays; whenever the workspace has that room, a first
 *              kernel writes every key chunk's largest norm and the attention kernel uses it to
 *              prove, per row, that later scores cannot pass the row's first-tile max by more
 *              than 15 (fp16) or 32 (bf16) in exp2 units (a weight of at most 2^15 or
 *              2^32), and then skips the per-tile row max.
 *              Only at the default configuration (block_m <= 128 rounds to 4 waves and the
 *              default block_n); otherwise the room is left unused. Same attention either way
 *              (the same 2x-SDPA accuracy); the bits of rows that skip can differ from a launch
 *              without the table.
 */
FA2_API int fa2_attn_fwd_ex(const void* q, const void* k, const void* v, void* out,
                            const int64_t q_stride[4], const int64_t k_stride[4],
                            const int64_t v_stride[4], const int64_t o_stride[4],
                            int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                            int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                            int32_t block_m, int32_t block_n, float qk_scale, float* lse,
                            int32_t num_splits, void* workspace, size_t workspace_bytes, void* stream);

/* Size of the library's own device scratch used by fa2_attn_fwd_noalloc (32 MiB per GPU). */
#define FA2_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * fa2_attn_fwd_noalloc - fa2_attn_fwd_ex without the workspace arguments: it allocates nothing.
 * No counterpart in the reference. It is for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. It creates no
 * event either: it deals a causal grid's tail only on a stream that already has a ticket set
 * (from an earlier fa2_attn_fwd or fa2_attn_fwd_ex call on it) and runs the static order
 * elsewhere, with the same output bit for bit.
 *
 * The split-KV partials and, where it pays, the key-norm table live in a device array owned by
 * the library, FA2_NOALLOC_SCRATCH_BYTES per GPU. The array sits in a device code object of its
 * own, which the first fa2_attn_fwd_noalloc call on a GPU that needs scratch loads (measured on
 * MI355X: 36 MiB less free device memory after that call, 4 MiB after the first other launch),
 * and it stays until the process ends. Its address is looked up on that first call, which must
 * run with the stream's device current. Every call on one GPU shares that array, so calls that
 * overlap on one GPU (two streams or two threads at once) race; serialise them. The caller still
 * passes q, k, v, out and lse.
 *
 *   num_splits 1..16 as in fa2_attn_fwd_ex; fa2_workspace_bytes(batch, h_q, n_q, head_dim,
 *              num_splits) must fit in FA2_NOALLOC_SCRATCH_BYTES, else FA2_EINVAL (no launch).
 *              The key-norm table is used as fa2_attn_fwd_ex with a workspace of
 *              fa2_workspace_bytes_for(...) bytes uses it, and left off if it would not fit.
 * With the same arguments the output is bit for bit that of fa2_attn_fwd_ex given a workspace
 * of fa2_workspace_bytes_for(...) bytes (when that fits in the scratch).
 */
FA2_API int fa2_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* out,
                                 const int64_t q_stride[4], const int64_t k_stride[4],
                                 const int64_t v_stride[4], const int64_t o_stride[4],
                                 int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                                 int32_t head_dim, int32_t dtype, int32_t causal, int32_t pack,
                                 int32_t block_m, int32_t block_n, float qk_scale, float* lse,
                                 int32_t num_splits, void* stream);

/*
 * fa2_workspace_bytes - workspace size of a split-KV launch of fa2_attn_fwd_ex: fp32 partial
 * outputs and log-sum-exps of every split. 0 when num_splits <= 1 or a size is not positive.
 */
FA2_API size_t fa2_workspace_bytes(int32_t batch, int32_t h_q, int32_t n_q, int32_t head_dim,
                                   int32_t num_splits);

/*
 * fa2_workspace_bytes_for - the workspace fa2_attn_fwd_ex can use for this launch:
 * fa2_workspace_bytes(...) plus, where the key-norm pass pays for itself, room for its table
 * (one float per batch, kv head and 64 keys). It pays, as measured on MI355X, for bf16 at
 * head_dim 128 (causal or not) and for fp16 or bf16 at 64 without the causal mask, when the
 * attention does at least 16384 FLOP per byte of K and at least 2^37 FLOP: the pass reads K once
 * and saves the per-tile row max (2-4% of the kernel; fp16 full attention at 64 on
 * unit-variance data loses under 1%). fp16 at head_dim 128 and causal fp16 at 64 are left out:
 * there the pass and the table's instance cost 1-4% more than they save. No counterpart in the
 * reference. Host policy only.
 */
FA2_API size_t fa2_workspace_bytes_for(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q,
                                       int32_t n_kv, int32_t head_dim, int32_t dtype, int32_t causal,
                                       int32_t num_splits);

/*
 * fa2_num_splits - the split count fa2_attn_fwd_ex should use: 1 for causal launches and for
 * grids of at least num_cus workgroups; otherwise the smallest power of two that reaches it,
 * keeping at least 4 K/V tiles per split, at most 16. The grid it sizes is the
 * smaller of the packed and the unpacked GQA layouts, so the answer does not depend on the
 * packing decision and packed and unpacked launches stay equal bit for bit. Host policy only.
 */
FA2_API int32_t fa2_num_splits(int32_t batch, int32_t h_q, int32_t h_kv, int32_t n_q, int32_t n_kv,
                               int32_t head_dim, int32_t causal, int32_t block_m, int32_t block_n,
                               int32_t num_cus);

/*
 * fa2_default_config - the gfx950 tile configuration for a head dim.
 * Replaces `_default_config(head_dim, on_cuda)` (fa2/kernel.py:186-195). Writes
 * block_m (rows per program), block_n (keys per K/V tile), num_waves (wave64s per
 * workgroup, the counterpart of Triton's num_warps) and num_stages (K/V buffers in
 * flight). Returns FA2_EINVAL for an unsupported head_dim.
 */
FA2_API int fa2_default_config(int32_t head_dim, int32_t* block_m, int32_t* block_n,
                               int32_t* num_waves, int32_t* num_stages);

/*
 * fa2_should_pack_gqa - FlashAttention-3's packing rule, as `should_pack_gqa`
 * (fa2/kernel.py:198-207): 1 when group > 1, block_m % group == 0 and the unpacked
 * tiles are less than 90% as full as the packed ones; else 0.
 */
FA2_API int fa2_should_pack_gqa(int32_t n_q, int32_t group, int32_t block_m);

/* Thread-local description of the last failure in this thread ("" if none). */
FA2_API const char* fa2_last_error(void);

/* Library version string, including the gfx target it was built for. */
FA2_API const char* fa2_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA2_FWD_H */
