/*
 * fast_infer_amd — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Entry points, each a drop-in for one piece of Fast_Infer's attention path or of
 * the operations on either side of it:
 *
 *   fi_flash_attention_fwd   causal prefill attention
 *                            replaces kernels/attention.py:80-113 (flash_attention,
 *                            launching _flash_attn_fwd :8-77); with a non-null
 *                            pool it also performs the prefill K/V write of
 *                            model.py:162-183 (_store_kv_prefill) in the same pass.
 *   fi_paged_attention_fwd   single-query attention over the paged KV pool
 *                            replaces kernels/attention.py:191-233 (paged_attention,
 *                            launching _paged_attention_kernel :116-188).
 *   fi_kv_store              scatter of K/V rows into the paged pool
 *                            replaces model.py:162-183 (_store_kv_prefill copies),
 *                            model.py:185-201 (_store_kv_decode copies) and
 *                            kv_cache.py:69-103 (KVCache.store / store_batch).
 *   fi_rope_store_kv         RoPE on q/k (kernels/rope.py:26-44 at model.py:101), with
 *                            the K/V pool write that follows it in the same pass.
 *   fi_kv_append / fi_kv_release / fi_kv_reset
 *                            the block allocator of kv_cache.py:50-63 / :108-113 as
 *                            model.py drives it, with per-row lengths, on the device.
 *   fi_int4_matmul, fi_int4_quantize, fi_int4_dequantize, fi_rmsnorm,
 *   fi_rmsnorm_int4_matmul   the INT4 projections and RMSNorm around attention
 *                            (kernels/matmul.py:217-231, loader.py:9-41,
 *                            kernels/matmul.py:309-326, kernels/rms_norm.py:29-43).
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; sizes and strides are int64 and counted in
 *     elements (not bytes).  The innermost (head_dim) stride is always 1.
 *   - K/V pools are dense fp16 tensors [num_blocks, block_size, num_kv_heads,
 *     head_dim] (the per-layer slice of kv_cache.py:25-28).
 *   - Block tables are int32 [batch, max_blocks_per_seq] with a row stride;
 *     -1 marks an unallocated entry (kv_cache.py:33-34).  Entries outside
 *     [0, num_blocks) are never dereferenced: rows that map there are skipped.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Every call
 *     is asynchronous: it enqueues work and returns; nothing synchronises.
 *   - Calls are reentrant.  The library's host-side state is the per-thread error
 *     message and, per device, cached on first use: the CU count (an atomic), and,
 *     under a mutex, the result of the workgroup-placement probe and the streams that
 *     were given split-K counter sets (fi_int4_matmul, at most 16 per device).  No
 *     other library is called.
 *   - Return value: FI_OK or an FI_ERR_* code; fi_last_error() then gives a
 *     message for the calling thread.
 *   - fp16 data.  head_dim: a multiple of 8 up to 128 for the attention entry points
 *     (128 for Llama-3.2-3B, config.py:12-15; the kernels load the columns past a
 *     smaller head_dim as zeros and never store them), a multiple of 8 for
 *     fi_kv_store, a multiple of 16 for fi_rope_store_kv.  Other head dims return
 *     FI_ERR_UNSUPPORTED.
 */
#ifndef FAST_INFER_AMD_H
#define FAST_INFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define FI_API __attribute__((visibility("default")))
#else
#define FI_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FI_OK 0
#define FI_ERR_INVALID 1     /* bad shape, stride, alignment or null pointer */
#define FI_ERR_UNSUPPORTED 2 /* valid request outside the implemented shapes */
#define FI_ERR_HIP 3         /* the HIP runtime reported a launch error */
#define FI_ERR_WORKSPACE 4   /* workspace missing or too small */

/* Library ABI version (major * 100 + minor). */
FI_API int fi_version(void);

/* Message describing the last failing call made by this thread ("" if none). */
FI_API const char* fi_last_error(void);

/*
 * Causal prefill attention, GQA-native.
 * Replaces flash_attention(q, k, v, sm_scale) at kernels/attention.py:80-113.
 *
 *   q, o : [batch, num_q_heads,  seq_len, head_dim] with strides (q_sb, q_sh, q_ss)
 *   k, v : [batch, num_kv_heads, seq_len, head_dim] with strides (k_sb, k_sh, k_ss)
 *   num_q_heads % num_kv_heads == 0; query head h reads kv head h / (num_q_heads/num_kv_heads)
 *   (the reference expands K/V with repeat_interleave, model.py:110-111; passing the
 *   expanded K/V with num_kv_heads == num_q_heads gives the identical result).
 *   Query row m attends to key rows n <= m (kernels/attention.py:57-58).
 *   Rows must be 16-byte aligned: every stride a multiple of 8, pointers 16-byte aligned.
 *
 * Optional fused pool write (k_cache != NULL): additionally copies k[b, :, t, :] and
 * v[b, :, t, :] into k_cache/v_cache at block block_table[b, t / block_size], slot
 * t % block_size, for every t < seq_len — the write of model.py:176-183.  Any block_size
 * from 1 to 2^20 (64, the reference's, is the fastest path).  Table entries outside
 * [0, num_pool_blocks), and tokens past the table's max_blocks_per_seq blocks, are skipped.
 */
FI_API int fi_flash_attention_fwd(const void* q, const void* k, const void* v, void* o,
                           int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                           int64_t seq_len, int64_t head_dim,
                           int64_t q_sb, int64_t q_sh, int64_t q_ss,
                           int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           int64_t v_sb, int64_t v_sh, int64_t v_ss,
                           int64_t o_sb, int64_t o_sh, int64_t o_ss,
                           float sm_scale,
                           void* k_cache, void* v_cache, int64_t num_pool_blocks,
                           int64_t block_size, const int32_t* block_table,
                           int64_t bt_stride, int64_t max_blocks_per_seq,
                           void* stream);

/*
 * Bytes of device workspace fi_paged_attention_fwd needs for these sizes
 * (0 when the call is served by a single pass).  `max_num_tokens` is the bound
 * later passed as `num_tokens`.
 */
FI_API size_t fi_paged_attention_workspace_size(int64_t batch, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t max_num_tokens,
                                         int64_t head_dim);

/*
 * Paged-attention decode (one query token per sequence), split-K over the context.
 * Replaces paged_attention(q, k_cache, v_cache, block_table, block_size, num_tokens,
 * sm_scale) at kernels/attention.py:191-233.
 *
 *   q, o        : [batch, num_q_heads, head_dim], strides (q_sb, q_sh) / (o_sb, o_sh)
 *   k/v_cache   : [num_pool_blocks, block_size, num_kv_heads, head_dim], dense
 *   block_table : int32, row b at block_table + b * bt_stride, max_blocks_per_seq entries
 *   context_lens: NULL -> every row attends to its first num_tokens tokens (the
 *                 reference's single shared length, kernels/attention.py:158-160);
 *                 else int32[batch] per-row lengths, each clamped to num_tokens, so
 *                 num_tokens must be >= max(context_lens).
 *   Rows whose length is 0 produce zeros (kernels/attention.py:205-206).
 *   Any block_size >= 1 (a multiple of 16 keeps every 16-token tile inside one block; other
 *   sizes address each tile row through its own block at about the same speed); with
 *   block_size 1 a call takes at most 3520 * 1024 tokens.  workspace must hold
 *   fi_paged_attention_workspace_size(batch, num_q_heads, num_kv_heads, num_tokens, head_dim)
 *   bytes (it may be NULL when that is 0); its contents need no initialisation.
 */
FI_API int fi_paged_attention_fwd(const void* q, int64_t q_sb, int64_t q_sh,
                           const void* k_cache, const void* v_cache,
                           int64_t num_pool_blocks, int64_t block_size, int64_t num_kv_heads,
                           const int32_t* block_table, int64_t bt_stride,
                           int64_t max_blocks_per_seq,
                           const int32_t* context_lens, int64_t num_tokens,
                           void* o, int64_t o_sb, int64_t o_sh,
                           int64_t batch, int64_t num_q_heads, int64_t head_dim,
                           float sm_scale,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * fi_paged_attention_fwd without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, results and errors as
 * fi_paged_attention_fwd; the split-K partials go to a static per-device scratch array of
 * FI_PAGED_NOALLOC_SCRATCH_BYTES bytes inside the library (each GPU the library runs on
 * holds it until the process ends).  Sizes whose
 * fi_paged_attention_workspace_size exceeds that return FI_ERR_UNSUPPORTED.  The call
 * allocates nothing.  Every call on one GPU shares that GPU's scratch: calls that overlap
 * in time on one GPU (concurrent streams, or host threads) race and must not be issued.
 * The stream must belong to the current HIP device.
 */
#define FI_PAGED_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
FI_API int fi_paged_attention_fwd_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                   const void* k_cache, const void* v_cache,
                                   int64_t num_pool_blocks, int64_t block_size,
                                   int64_t num_kv_heads, const int32_t* block_table,
                                   int64_t bt_stride, int64_t max_blocks_per_seq,
                                   const int32_t* context_lens, int64_t num_tokens, void* o,
                                   int64_t o_sb, int64_t o_sh, int64_t batch,
                                   int64_t num_q_heads, int64_t head_dim, float sm_scale,
                                   void* stream);

/*
 * Scatter K/V rows into the paged pool (byte-exact copies).
 * Replaces the slice copies of model.py:176-183 (prefill), model.py:196-201 (decode)
 * and kv_cache.py:69-103.
 *
 *   k, v : [batch, num_tokens, num_kv_heads, head_dim] with strides
 *          (k_sb, k_st, k_sh) / (v_sb, v_st, v_sh)
 *   Token t of row b lands at position p = start + t where start is
 *   start_pos_per_seq[b] if that pointer is non-null, else start_pos; the row goes to
 *   block block_table[b, p / block_size], slot p % block_size.  Positions whose
 *   logical block is >= max_blocks_per_seq or whose table entry is outside
 *   [0, num_pool_blocks) are skipped.
 */
FI_API int fi_kv_store(const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                void* k_cache, void* v_cache, int64_t num_pool_blocks,
                int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                const int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                int64_t batch, int64_t num_tokens,
                int64_t start_pos, const int32_t* start_pos_per_seq,
                void* stream);

/*
 * Rotary position embedding, optionally fused with the paged K/V write.
 * Replaces apply_rope(q, k, cos, sin) at kernels/rope.py:26-44 (call site model.py:101)
 * and, with a pool, the K/V stores after it (model.py:117 -> :162-183, model.py:120 ->
 * :185-201).
 *
 *   q, q_out : [batch, num_tokens, num_q_heads, head_dim], strides (q_sb, q_st, q_sh) /
 *              (qo_sb, qo_st, qo_sh); q_out may be q itself (same strides).
 *   k, v     : [batch, num_tokens, num_kv_heads, head_dim], strides (k_*, v_*).
 *   cos/sin  : fp16 [table_rows, head_dim] dense, the rows of the reference's tables
 *              (kernels/rope.py:9-16, cast to fp16 at model.py:75-76).
 *   Token t of row b uses table row pos = start + t, start = start_pos_per_seq[b] if
 *   that pointer is non-null, else start_pos.  Each element is
 *   fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)) with rotate_half(x)[i] = -x[i+64]
 *   (i < 64) and x[i-64] (i >= 64): bit-exact with the reference's fp16 tensor ops.
 *   A token whose pos is outside [0, table_rows) is skipped entirely (q_out/k_out rows
 *   left unwritten, nothing written to the pool).
 *   k_out (optional, may be NULL): rotated k, strides (ko_sb, ko_st, ko_sh).
 *   k_cache (optional, may be NULL): rotated k and the unrotated v are also written to
 *   k_cache / v_cache [num_pool_blocks, block_size, num_kv_heads, head_dim] at block
 *   block_table[b, pos / block_size], slot pos % block_size; positions whose logical
 *   block is >= max_blocks_per_seq or whose entry is outside [0, num_pool_blocks) are
 *   skipped (as fi_kv_store).
 *   Rows must be 16-byte aligned (pointers 16-byte aligned, strides multiples of 8).
 */
FI_API int fi_rope_store_kv(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                     const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                     const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                     const void* cos_table, const void* sin_table, int64_t table_rows,
                     void* q_out, int64_t qo_sb, int64_t qo_st, int64_t qo_sh,
                     void* k_out, int64_t ko_sb, int64_t ko_st, int64_t ko_sh,
                     void* k_cache, void* v_cache, int64_t num_pool_blocks,
                     int64_t block_size, const int32_t* block_table, int64_t bt_stride,
                     int64_t max_blocks_per_seq,
                     int64_t batch, int64_t num_tokens, int64_t num_q_heads,
                     int64_t num_kv_heads, int64_t head_dim,
                     int64_t start_pos, const int32_t* start_pos_per_seq,
                     void* stream);

/*
 * Device-resident block manager for the paged pool: per-sequence lengths and a FIFO
 * queue of free blocks, served on the stream (no host round trip).  Replaces the host
 * allocator kv_cache.py:50-63 as driven by model.py:172-174 (prefill) and :196-198
 * (decode), and the single shared token count of model.py:169-170 / :193-194.
 *
 * State (int32 device arrays the caller allocates; fi_kv_reset initialises them):
 *   block_table [rows, bt_stride]  logical -> physical block, -1 = unallocated; a row's
 *                                  entries 0 .. num_alloc[b]-1 are valid
 *   num_alloc   [rows]             blocks allocated to each row
 *   seq_lens    [rows]             tokens stored in each row
 *   free_queue  [num_blocks]       ring buffer of free block ids
 *   state       [4]                {head, free count, status, row of the status}
 * status is FI_KV_OK or the first error since the last reset (sticky):
 */
#define FI_KV_OK 0
#define FI_KV_OUT_OF_BLOCKS 1  /* the queue ran out ("KV cache out of memory", :52-53) */
#define FI_KV_TABLE_FULL 2     /* a row needs more than max_blocks_per_seq blocks (:58-59) */
#define FI_KV_NEGATIVE_COUNT 3 /* a negative per-row token count */

/*
 * Add num_new[b] tokens (num_new_all for every row if num_new is NULL) to rows
 * 0..batch-1: each row gets blocks until ceil(seq_lens[b] / block_size) are allocated,
 * rows in order, each row's new blocks taken from the front of the free queue in logical
 * order (the reference's free_blocks.pop(0) order).  The first row that cannot be served
 * and every later row are left unchanged and the status records it.
 *   start_pos_out[b] (optional): the row's length before the call = the position of its
 *   first new token (fi_rope_store_kv's start_pos_per_seq);
 *   context_lens_out[b] (optional): its length after the call (fi_paged_attention_fwd's
 *   context_lens).
 * One workgroup; a call is ordered after earlier work on the stream.
 */
FI_API int fi_kv_append(int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                 int32_t* num_alloc, int32_t* seq_lens, const int32_t* free_queue,
                 int32_t* state, int64_t num_blocks, int64_t block_size,
                 int64_t batch, const int32_t* num_new, int64_t num_new_all,
                 int32_t* start_pos_out, int32_t* context_lens_out, void* stream);

/*
 * Release every row b < batch with release_rows[b] != 0: its blocks go to the back of
 * the free queue in (row, logical block) order, its table entries become -1 and its
 * length 0.  No counterpart in the reference, which only frees everything at once
 * (kv_cache.py:108-113); needed to retire one sequence of a running batch.
 */
FI_API int fi_kv_release(int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                  int32_t* num_alloc, int32_t* seq_lens, int32_t* free_queue,
                  int32_t* state, int64_t num_blocks, int64_t batch,
                  const int32_t* release_rows, void* stream);

/*
 * kv_cache.py:108-113 (reset) for the device state: all max_batch rows' entries -1,
 * lengths 0, free queue 0..num_blocks-1 in order, status FI_KV_OK.
 */
FI_API int fi_kv_reset(int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                int64_t max_batch, int32_t* num_alloc, int32_t* seq_lens,
                int32_t* free_queue, int32_t* state, int64_t num_blocks, void* stream);

/*
 * INT4 group-quantized linear layer, C = X * W^T (kernels/matmul.py:217-231,
 * int4_matmul; the fused kernel :14-132 for packed weights, the fp16 kernel :135-186
 * for dequantized ones).
 *   x      : fp16 [M, K], row stride x_stride elements (16-byte aligned rows).
 *   w      : with scales: int8 bytes [N, K/2] (loader.py:9-41 packing: byte j of a row holds
 *            k = 2j in the low nibble, k = 2j+1 in the high nibble, two's complement),
 *            row stride w_stride bytes (multiple of 16); scales fp16 [N, K/groupsize], row
 *            stride s_stride elements.  Without scales (NULL): fp16 [N, K], row stride
 *            w_stride elements.
 *   out    : fp16 [M, N], row stride out_stride elements.
 *   Each weight is fp16(q * scale) exactly as the reference dequantizes it; products are
 *   accumulated in fp32 and rounded to fp16 once.  Packed weights need groupsize 128 (the
 *   reference's) and K a multiple of 128; for another group size, dequantize with
 *   fi_int4_dequantize and pass the fp16 weight.  Some shapes split K: then a workspace of
 *   fi_int4_matmul_workspace_size(M, N, K) bytes (enough for either weight form) is
 *   required (FI_ERR_WORKSPACE otherwise); calls that overlap in time must not share one.
 *   From 129 rows packed weights are dequantized into that workspace and both forms run
 *   a 256 x 256-tile fp16 GEMM kernel, which needs 256 rows of X (and of an fp16 W) to
 *   span less than 2 GiB (FI_ERR_UNSUPPORTED otherwise).
 */
FI_API size_t fi_int4_matmul_workspace_size(int64_t M, int64_t N, int64_t K);
FI_API int fi_int4_matmul(const void* x, int64_t x_stride, int64_t M, int64_t K,
                   const void* w, int64_t w_stride, const void* scales, int64_t s_stride,
                   int64_t N, int64_t groupsize, void* out, int64_t out_stride,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMSNorm (kernels/rms_norm.py:29-43, rms_norm): out[m] = fp16((x[m] * r) * weight) with
 * r = rsqrt(sum(x[m]^2) / hidden + eps), all in fp32 (rms_norm.py:17-24).
 *   x, out: fp16 [M, hidden] (row strides in elements, 16-byte aligned rows);
 *   weight: fp16 [hidden]; hidden a multiple of 8.
 */
FI_API int fi_rmsnorm(const void* x, int64_t x_stride, int64_t M, int64_t hidden,
               const void* weight, float eps, void* out, int64_t out_stride, void* stream);

/*
 * rms_norm followed by int4_matmul as one call (model.py:82 then :87 / :91-93): out =
 * fi_int4_matmul(fi_rmsnorm(x, norm_weight, eps), w, scales).  Up to a few rows the norm is
 * applied inside the GEMM's X operand (each workgroup computes its rows' r), saving the
 * separate pass and its write and read of the normalized rows; above that a separate norm
 * pass writes them into the workspace first.  Arguments as fi_rmsnorm and
 * fi_int4_matmul; workspace: fi_rmsnorm_int4_matmul_workspace_size(M, N, K) bytes,
 * 256-byte aligned, when non-zero.
 */
FI_API size_t fi_rmsnorm_int4_matmul_workspace_size(int64_t M, int64_t N, int64_t K);
FI_API int fi_rmsnorm_int4_matmul(const void* x, int64_t x_stride, int64_t M, int64_t K,
                           const void* norm_weight, float eps, const void* w,
                           int64_t w_stride, const void* scales, int64_t s_stride,
                           int64_t N, int64_t groupsize, void* out, int64_t out_stride,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * quantize_int4_groupwise (loader.py:9-41) on the device, bit-exact with the reference's
 * fp16 tensor arithmetic on a CUDA device: amax = max |w| over each group of groupsize
 * consecutive k, clamped below at fp16(1e-6); scale = fp16(fp32(amax) * fp32(1/7)); q =
 * round_half_even(fp16(fp32(w) / fp32(scale))) clamped to [-8, 7], packed two per byte.
 * groupsize: a power of two from 8 to 512 (128 in the reference), dividing K.
 *   w fp16 [N, K] (row stride w_stride elements, 16-byte aligned rows);
 *   packed int8 [N, K/2] (row stride p_stride bytes), scales fp16 [N, K/groupsize].
 */
FI_API int fi_int4_quantize(const void* w, int64_t w_stride, int64_t N, int64_t K,
                     int64_t groupsize, void* packed, int64_t p_stride, void* scales,
                     int64_t s_stride, void* stream);

/*
 * _dequant_storage (kernels/matmul.py:309-326): w[n, k] = fp16(q[n, k] *
 * scale[n, k / groupsize]); groupsize as for fi_int4_quantize.
 */
FI_API int fi_int4_dequantize(const void* packed, int64_t p_stride, const void* scales,
                       int64_t s_stride, int64_t N, int64_t K, int64_t groupsize, void* w,
                       int64_t w_stride, void* stream);

/*
 * Self-test of the gfx950 MFMA fragment layout the attention kernels assume
 * (no counterpart in the reference; used by the test suite).  One wave computes
 * C[16x16] = A[16x32] * B[32x16] with v_mfma_f32_16x16x32_f16, where lane l holds
 * A[l % 16][8*(l/16) + s] and B[8*(l/16) + s][l % 16] for s = 0..7 and returns
 * C[4*(l/16) + i][l % 16] for i = 0..3.
 *   a, b: fp16 [64][8] (lane-major), c: fp32 [64][4] (lane-major).
 */
FI_API int fi_selftest_mfma_f16(const void* a, const void* b, void* c, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAST_INFER_AMD_H */
