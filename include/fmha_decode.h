/*
 * fmha_decode.h -- C ABI of the MI355X (gfx950) decode-attention library
 * (libfmha_decode.so).
 *
 * The path: one query token per sequence (seqlen_q == 1) attending to a short
 * KV cache of 0..16 tokens, bf16 Q/K/V, fp32 accumulation, fp16 output:
 *
 *   for every batch b and query head h (kv head hk = h / (Hq / Hkv)):
 *     s_j = sum_d Q[b,h,d] * K[cu[b]+j, hk, d]                  j < S_b
 *     P_j = bf16( exp(s_j*scale - max) / sum_i exp(s_i*scale - max) )
 *     O[b,h,d] = fp16( sum_j P_j * V[cu[b]+j, hk, d] )
 *
 * Numerics.  With at most 2 query heads per KV head (Hq / Hkv <= 2: the
 * reference's own configurations and BASELINE's), fmha_decode_fwd and
 * fmha_decode_fwd_uniform compute this with the arithmetic of the reference
 * CPU loop (fmha_host.cpp:179-244) step for step (see fmha_decode_fwd_exact):
 * their outputs are that loop's, bit for bit.  With larger groups they sum
 * in tree order with the device expf (see fmha_decode_fwd_fast): the same
 * semantics within the comparison gate, not the same bits;
 * fmha_decode_fwd_exact gives the loop's bits for groups of up to 8.
 *
 * Layouts (element counts, row-major, no padding):
 *   Q  [batch, num_heads_q, 1, head_dim]    bf16   (BHSD with S = 1)
 *   O  [batch, num_heads_q, 1, head_dim]    fp16
 *   K  [total_kv, num_heads_kv, head_dim]   bf16   packed over batches
 *   V  [total_kv, num_heads_kv, head_dim]   bf16   packed over batches
 *   cu_seqlens_kv [batch + 1]               int32  batch b owns rows
 *                                                  [cu[b], cu[b+1]) of K/V
 *
 * All pointers are device pointers owned by the caller.  Calls are
 * asynchronous on the given stream (a hipStream_t passed as void*, NULL for
 * the null stream) and may be issued from any number of host threads, with
 * one exception: fmha_decode_fwd_splitkv_noalloc uses one workspace array per
 * GPU, so its calls on one GPU must be ordered (one stream, or synchronised)
 * or they corrupt each other's results.  They allocate no device memory.
 * The one piece of library state: the entry points that read lengths from a
 * device array (fmha_decode_fwd, its _fast, _fp32_weights and _exact forms,
 * fmha_decode_fwd_splitkv up to 16 rows, and the paged entry points up to 16
 * rows) keep pinned host memory per device (64 bytes, allocated by the
 * first such call that is not being captured into a graph, never freed) in
 * which each call's first wave leaves the call's mean length (paged: of a
 * sample of up to 4096 lengths), one word for the cu_seqlens calls and one
 * for the paged ones; the next call sizes its launch (waves per CU) from
 * it.  Results never depend on it.
 *
 * Return value: 0 (hipSuccess) or a hipError_t value.  Arguments are checked
 * before anything touches the GPU; a rejected call launches nothing.
 */
#ifndef FMHA_DECODE_H_
#define FMHA_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest KV length per sequence the kernels accept (the reference hard-codes
 * the same bound: fmha_mfma_4x4x4_kernel.hpp:179, fmha_host.cpp:164). */
#define FMHA_DECODE_MAX_SEQLEN_KV 16

/* hipError_t values returned by this library. */
#define FMHA_DECODE_SUCCESS 0
#define FMHA_DECODE_ERROR_INVALID_VALUE 1    /* hipErrorInvalidValue */
#define FMHA_DECODE_ERROR_NOT_SUPPORTED 801  /* hipErrorNotSupported */

/*
 * Variable-length decode attention.
 *
 * Replaces launch_fmha_mfma_4x4x4 (reference fmha_mfma_4x4x4_kernel.hpp:370-376):
 * the same parameters in the same order and meaning, without the caller-chosen
 * grid/block (the library picks its own launch shape), with the stream passed
 * as void* and with an error code instead of void.
 *
 *   stream          hipStream_t to launch on (NULL = null stream)
 *   Q, K, V, O      device pointers, 16-byte aligned, layouts above
 *   cu_seqlens_kv   device int32 [batch+1], non-decreasing, cu[0] = 0 is not
 *                   required (any base offset works); each S_b = cu[b+1]-cu[b]
 *                   must lie in [0, 16].  A batch with S_b == 0 gets O = 0 (as
 *                   the reference CPU loop does).  A batch with S_b outside
 *                   [0, 16] gets O = NaN: the kernel cannot return an error.
 *   batch           >= 0 (0 launches nothing)
 *   num_heads_q     > 0, a multiple of num_heads_kv
 *   num_heads_kv    > 0; any group size G = num_heads_q / num_heads_kv.
 *                   G <= 2 runs the exact-arithmetic VALU kernel (the
 *                   reference loop's bits), G = 3-8 the tree-order VALU
 *                   kernel (G = 3 on its 4-head and 5-7 on its 8-head
 *                   instantiation, the extra heads reading and writing
 *                   nothing), G > 8 the matrix-core kernel (it needs
 *                   num_heads_kv * head_dim below 2^24, else
 *                   FMHA_DECODE_ERROR_NOT_SUPPORTED).  This entry point,
 *                   fmha_decode_fwd_uniform, their _fast forms and
 *                   fmha_decode_fwd_strided take any G, and so do the
 *                   split-KV entries (through a padded query group beyond
 *                   16 rows); fmha_decode_fwd_exact and
 *                   fmha_decode_fwd_fp32_weights G <= 8 (else
 *                   FMHA_DECODE_ERROR_NOT_SUPPORTED); fmha_decode_fwd_paged
 *                   G > 8 where rows lie in a batch's first page.
 *   seqlen_q        must be 1 (decode)
 *   head_dim_q      64, 128 or 256
 *   head_dim_kv     must equal head_dim_q
 *   softmax_scale   finite; the reference passes 1/sqrt(head_dim)
 *                   (fmha_host.cpp:371)
 *
 * Unlike the reference kernel, which indexes K/V with the query head
 * (fmha_mfma_4x4x4_kernel.hpp:195-196), query head h reads KV head
 * h / (num_heads_q / num_heads_kv) (grouped-query attention).
 */
int fmha_decode_fwd(void* stream,
                    const void* Q, const void* K, const void* V, void* O,
                    const int32_t* cu_seqlens_kv,
                    int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                    int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                    float softmax_scale);

/*
 * fmha_decode_fwd with tree-order numerics for every group size: each score
 * summed over its dims as a tree of packed bf16 dot products, the device
 * expf, the weights rounded to bf16 as in the loop, P.V as packed dot
 * products and the last multiply-add rounded straight to fp16.  A few
 * outputs in ten thousand differ from the reference loop in the last bits
 * (every one within the comparison gate).  At most 1% faster than
 * fmha_decode_fwd with one or two query heads per KV head, 5-6% with short
 * rows at head_dim 256; the same kernels above.  G <= 8 runs the tree-order
 * VALU kernel, G > 8 the matrix-core kernel; the environment variable
 * FMHA_DECODE_GQA_KERNEL=mfma runs the matrix-core kernel for every G here
 * and for G > 2 in fmha_decode_fwd (for comparisons).  Same arguments,
 * layouts, checks and errors as fmha_decode_fwd.  No counterpart in the
 * reference, whose CPU loop and wired-in kernel have these semantics with
 * their own orders of summation.
 */
int fmha_decode_fwd_fast(void* stream,
                         const void* Q, const void* K, const void* V, void* O,
                         const int32_t* cu_seqlens_kv,
                         int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                         int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                         float softmax_scale);

/*
 * fmha_decode_fwd with the softmax weights kept in fp32: P_j is the fp32
 * quotient exp(s_j*scale - max) / sum, not rounded to bf16, and
 * O[b,h,d] = fp16(acc) with acc = fma(P_j, V_j[d], acc) for j = 0, 1, ...
 * in row order.  These are the semantics of the reference's other VALU
 * kernel, fmha_vectorized_fma (fmha_vectorized_fma_kernel.hpp:69-83 for its
 * parameter list, :243-296 for the weights and the accumulation), which has
 * no launch helper in the reference; the wired-in fmha_mfma_4x4x4 and the
 * reference CPU check round the weights to bf16 (fmha_decode_fwd).  Same
 * arguments, layouts, checks and errors as fmha_decode_fwd, with group sizes
 * up to 8 only (the VALU kernel).
 */
int fmha_decode_fwd_fp32_weights(void* stream,
                                 const void* Q, const void* K, const void* V, void* O,
                                 const int32_t* cu_seqlens_kv,
                                 int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                 int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                 float softmax_scale);

/*
 * fmha_decode_fwd with the arithmetic of the reference CPU loop
 * (fmha_host.cpp:179-244) step for step for every call, with the
 * grouped-query head mapping (query head h reads KV head h / G; the loop
 * itself indexes K/V with h, fmha_host.cpp:190-192, which agrees for
 * G = 1): each score a float32 sum over d = 0, 1, ..., D-1 in order (every
 * product exact, every addition rounded), then * softmax_scale; the max;
 * each exponential the float nearest exp(s_j*scale - max) (evaluated in
 * double and rounded once); their float32 sum in row order; the IEEE
 * quotient rounded to bf16; O a float32 sum over rows in order, rounded to
 * fp16.  The outputs equal that loop's bit for bit wherever its expf
 * returns the nearest float (glibc 2.35's expf misses it on about 0.07% of
 * arguments, and an output can differ only where such a miss also flips a
 * bf16 weight: none in ten million random heads).  These are the numerics
 * fmha_decode_fwd takes for G <= 2; this entry point gives them for
 * G <= 8 too (1-45% slower than the tree-order kernels there) and rejects
 * G > 8 (FMHA_DECODE_ERROR_NOT_SUPPORTED).  Same arguments, layouts, checks
 * and errors as fmha_decode_fwd otherwise.  No counterpart in the
 * reference, which has no GPU kernel with these results; for callers that
 * need the CPU loop's outputs whatever the group size.
 */
int fmha_decode_fwd_exact(void* stream,
                          const void* Q, const void* K, const void* V, void* O,
                          const int32_t* cu_seqlens_kv,
                          int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                          int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                          float softmax_scale);

/*
 * Uniform-length decode attention: every batch has seqlen_kv KV rows, K and V
 * are [batch, seqlen_kv, num_heads_kv, head_dim] (the packed layout above with
 * cu[b] = b * seqlen_kv), and no cu_seqlens array is read.  This is the
 * launch contract's seqlen_kv parameter; the reference derives every length
 * from cu_seqlens_kv instead (fmha_mfma_4x4x4_kernel.hpp:94-96).
 * seqlen_kv must lie in [0, 16]; with seqlen_kv == 0 no row is read, every
 * output is 0 and K and V may be NULL.  Other arguments and numerics as
 * fmha_decode_fwd (the reference loop's bits for G <= 2).
 */
int fmha_decode_fwd_uniform(void* stream,
                            const void* Q, const void* K, const void* V, void* O,
                            int32_t seqlen_kv,
                            int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                            int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                            float softmax_scale);

/* fmha_decode_fwd_uniform with the numerics of fmha_decode_fwd_fast.  No
 * counterpart in the reference. */
int fmha_decode_fwd_uniform_fast(void* stream,
                                 const void* Q, const void* K, const void* V, void* O,
                                 int32_t seqlen_kv,
                                 int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                 int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                 float softmax_scale);

/*
 * Decode attention over K/V addressed by strides, for caches that are not
 * packed: element d of head h, row j of batch b is at
 *     K + b*kv_batch_stride + j*kv_row_stride + h*kv_head_stride + d
 * (strides in elements, >= 0, multiples of 8; V uses the same strides).
 * [B, Hkv, S, D] (BHSD, the layout the reference README documents,
 * README.md:166-168) is (Hkv*S*D, D, S*D); a padded [B, S, Hkv, D] cache is
 * (S*Hkv*D, Hkv*D, D).
 *
 *   seqlens_kv   device int32 [batch] lengths, or NULL for a uniform length
 *   seqlen_kv    uniform length (in [0, 16]) when seqlens_kv is NULL; else
 *                the rows each batch has room for: a length above
 *                min(seqlen_kv, 16) gets NaN outputs, rows past a batch's
 *                length are never read (padding may hold anything)
 * One batch's span (rows and heads) must stay below 1 GiB; on the
 * matrix-core kernel (see fmha_decode_fwd) so must the span of the
 * 64/(head_dim/8)/num_heads_kv + 2 batches a wave may touch, else
 * FMHA_DECODE_ERROR_NOT_SUPPORTED.  Other arguments as fmha_decode_fwd.
 */
int fmha_decode_fwd_strided(void* stream,
                            const void* Q, const void* K, const void* V, void* O,
                            const int32_t* seqlens_kv, int32_t seqlen_kv,
                            int64_t kv_batch_stride, int64_t kv_row_stride, int64_t kv_head_stride,
                            int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                            int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                            float softmax_scale);

/*
 * Decode attention over a paged KV cache [num_pages, page_size, Hkv, D]
 * (K_cache and V_cache alike).  Row j of batch b is slot j % page_size of page
 * block_table[b * block_table_stride + j / page_size].
 *
 *   block_table         device int32, ceil(len/page_size) valid entries per
 *                       batch row (the row itself is block_table_stride long)
 *   seqlens_kv          device int32 [batch] lengths in [0, min(16,
 *                       block_table_stride * page_size)]; a length outside
 *                       that range gets NaN outputs
 *   page_size           a power of two in [1, 2^20]
 * Other arguments as fmha_decode_fwd.  Group sizes up to 8 run on the VALU
 * kernel; above 8 on the matrix-core kernel when every length the call
 * accepts (min(16, block_table_stride * page_size)) lies within page_size,
 * else FMHA_DECODE_ERROR_NOT_SUPPORTED (fmha_decode_fwd_splitkv_paged takes
 * those on its split passes).  The reference has no paged layout; this entry
 * point is the KV-cache format of serving engines.
 */
int fmha_decode_fwd_paged(void* stream,
                          const void* Q, const void* K_cache, const void* V_cache, void* O,
                          const int32_t* block_table, int32_t block_table_stride,
                          const int32_t* seqlens_kv, int32_t page_size,
                          int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                          int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                          float softmax_scale);

/*
 * Decode attention for KV lengths beyond 16 (split-KV): the packed layout and
 * cu_seqlens_kv of fmha_decode_fwd, lengths in [0, max_seqlen_kv] (a length
 * outside that range gets NaN outputs).  The weights are still rounded to
 * bf16 after normalisation by the global max and sum, as in the reference's
 * CPU loop (fmha_host.cpp:209-226) extended past its 16-row arrays; the
 * reference itself stops at 16 (fmha_mfma_4x4x4_kernel.hpp:179, README.md:233).
 *
 * The library picks the kernels: the kernel and numerics of fmha_decode_fwd
 * when max_seqlen_kv <= 16; one single-pass launch when there are at least 512
 * (batch, KV-head group) waves and a row's scores fit the wave's LDS; else
 * four split-KV launches (scores, statistics, P.V per chunk, combine).
 *
 * The caller provides a device workspace of at least
 * fmha_decode_splitkv_workspace_size(batch, Hq, Hkv, max_seqlen_kv, head_dim)
 * bytes, 256-byte aligned; its contents on entry do not matter.  Calls that
 * share a workspace must be ordered (same stream or synchronised).
 *
 * Group sizes G = num_heads_q / num_heads_kv: any.  With max_seqlen_kv <= 16
 * as fmha_decode_fwd (the paged entry: as fmha_decode_fwd_paged, and G > 8
 * with rows that may reach a second page as beyond 16).  Beyond 16, G = 3 and 5-7 run on copies of Q and O padded
 * to 4 or 8 query heads per KV head, and G > 8 on copies padded to a
 * multiple of 8 (copies only when G is not one).  G <= 4 runs on the VALU
 * split-KV passes; G = 5-8 and G > 8 on split-KV passes on the matrix cores
 * (all query heads of a KV head per wave; K and V read once), except G = 5-8
 * on pages of fewer than 16 rows with at least half a wave of KV heads,
 * which takes the VALU passes.  Many short rows (>= 512 waves, a row's
 * scores within a wave's LDS) take a single-pass kernel instead, at G <= 8
 * on the rows where it measured faster, and G = 3-4 on pages of fewer than
 * 16 rows with few KV heads, rows of at most 48 and head_dim >= 128 the
 * matrix-core passes.  The workspace size includes the copies (two
 * of [batch, Hkv * padded group, head_dim], ahead of the split-KV data) and
 * covers whichever passes the layout takes.  FMHA_DECODE_GQA_KERNEL=valu
 * keeps every G on the VALU kernels (G > 8 as ceil(G / 8) groups of 8 query
 * heads per KV head, still reading K and V once), =mfma puts every G on the
 * matrix-core passes (G <= 4 measures slower there), for comparisons.
 */
size_t fmha_decode_splitkv_workspace_size(int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                          int32_t max_seqlen_kv, int32_t head_dim);

int fmha_decode_fwd_splitkv(void* stream,
                            const void* Q, const void* K, const void* V, void* O,
                            const int32_t* cu_seqlens_kv, int32_t max_seqlen_kv,
                            int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                            int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                            float softmax_scale, void* workspace, size_t workspace_bytes);

/*
 * fmha_decode_fwd_splitkv without the workspace arguments, for callers that
 * cannot allocate device memory (code under graph capture, serving loops,
 * harnesses that forbid hipMalloc); it has no counterpart in the reference.
 * The workspace is a device array inside the library, one per GPU, of
 * FMHA_DECODE_NOALLOC_SCRATCH_BYTES bytes (held from library load until the
 * process ends); the call allocates nothing, and a call whose
 * fmha_decode_splitkv_workspace_size exceeds the array is rejected
 * (FMHA_DECODE_ERROR_INVALID_VALUE) before anything is launched.  Every call
 * on one GPU uses the same array: calls that overlap on a GPU (different
 * streams, not ordered) race and must be serialised by the caller.  Same
 * kernels, arguments and results as fmha_decode_fwd_splitkv.
 */
#define FMHA_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

int fmha_decode_fwd_splitkv_noalloc(void* stream,
                                    const void* Q, const void* K, const void* V, void* O,
                                    const int32_t* cu_seqlens_kv, int32_t max_seqlen_kv,
                                    int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                    int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                    float softmax_scale);

/*
 * fmha_decode_fwd_splitkv over the strided K/V of fmha_decode_fwd_strided
 * (BHSD, padded BSHD, any batch/row/head strides in elements, multiples of
 * 8): lengths beyond 16 for those caches.
 *
 *   seqlens_kv     device int32 [batch] lengths, or NULL: every batch has
 *                  max_seqlen_kv rows
 *   max_seqlen_kv  rows each batch has room for; a length above it gets NaN
 *                  outputs, rows past a batch's length are never read
 * One batch's span (max_seqlen_kv rows, all heads) must stay below 1 GiB.
 * The workspace is sized by fmha_decode_splitkv_workspace_size(batch, Hq,
 * Hkv, max_seqlen_kv, head_dim) and unused when max_seqlen_kv <= 16 (the
 * call then runs fmha_decode_fwd_strided, any G).  Group sizes as for
 * fmha_decode_fwd_splitkv.  No counterpart in the reference,
 * which has neither layout nor lengths beyond 16 (README.md:166-168,
 * README.md:233).
 */
int fmha_decode_fwd_splitkv_strided(void* stream,
                                    const void* Q, const void* K, const void* V, void* O,
                                    const int32_t* seqlens_kv, int32_t max_seqlen_kv,
                                    int64_t kv_batch_stride, int64_t kv_row_stride, int64_t kv_head_stride,
                                    int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                    int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                    float softmax_scale, void* workspace, size_t workspace_bytes);

/*
 * fmha_decode_fwd_splitkv over the paged cache of fmha_decode_fwd_paged:
 * lengths beyond 16 for a [pages, page_size, Hkv, D] cache.  A length above
 * min(max_seqlen_kv, block_table_stride * page_size) gets NaN outputs (so no
 * batch reads past its row of the block table); rows past a batch's length
 * and pages it does not map are never read.  Workspace as for
 * fmha_decode_fwd_splitkv_strided (when that bound is <= 16 the call runs
 * fmha_decode_fwd_paged's kernel, and the workspace only holds a padded
 * query group).  Any group size, on the passes fmha_decode_fwd_splitkv
 * describes for each G and layout (3 and 5-7 on padded query groups); with
 * that bound <= 16, G > 8 takes the split passes, and needs the workspace,
 * only where the bound exceeds page_size.
 * No counterpart in the reference.
 */
int fmha_decode_fwd_splitkv_paged(void* stream,
                                  const void* Q, const void* K_cache, const void* V_cache, void* O,
                                  const int32_t* block_table, int32_t block_table_stride,
                                  const int32_t* seqlens_kv, int32_t page_size, int32_t max_seqlen_kv,
                                  int32_t batch, int32_t num_heads_q, int32_t num_heads_kv,
                                  int32_t seqlen_q, int32_t head_dim_q, int32_t head_dim_kv,
                                  float softmax_scale, void* workspace, size_t workspace_bytes);

/* Human-readable text for a code returned above (never NULL). */
const char* fmha_decode_error_string(int code);

/* Text describing why the most recent call on this host thread was rejected
 * ("" after a successful call). */
const char* fmha_decode_last_error_detail(void);

/* The kernels the most recent call on this host thread launched, in order,
 * separated by "; " ("" after a rejected or empty call): each a kernel
 * kind with the choices the library made for it, e.g.
 *   "short(numerics=exact D=128 G=1 layout=packed bucket=16 waves_per_cu=4)"
 *   "split(D=128 G=4 layout=packed sub_units=1 blocks=64 chunk_rows=256
 *    chunks=4 passes=4)".
 * Kinds: short, short_multi (several batches per wave), short_matrix_core,
 * onepass, split, split_matrix_core, pad_query_group.  For tests and
 * diagnostics; no counterpart in the reference. */
const char* fmha_decode_last_plan(void);

/* Library version, encoded as major*10000 + minor*100 + patch. */
int fmha_decode_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FMHA_DECODE_H_ */
