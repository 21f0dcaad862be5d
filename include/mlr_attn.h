/*
 * mlr_attn.h - C ABI of the MI355X paged-attention library (libmlr_attn.so).
 *
 * The library implements the three kernels of the paged attention path of
 * mini-llm-runtime on gfx950 (MI355X):
 *   1. the KV-cache write: a slot_mapping scatter into one layer's block pool;
 *   2. batched single-token paged decode (split-KV; the splits merge in the
 *      same launch on the bf16 and FP32 matrix-core paths, in a second one
 *      otherwise);
 *   3. paged chunk-prefill attention (causal by absolute token position).
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers, except where a comment says otherwise.
 *   - A KV cache layer is one contiguous array of shape
 *     [num_blocks, block_size, num_kv_heads, head_dim]; slot s addresses the
 *     row [s / block_size, s % block_size]. This is the per-layer view that
 *     PagedKVCache.get_layer_cache hands out (runtime/paged_kv_cache.py:25-35,
 *     251-259 in the reference).
 *   - Strides are in elements, not bytes. Query and output rows are unit-stride
 *     along head_dim; the KV-write sources may have any strides.
 *   - Query head h reads KV head h / (num_q_heads / num_kv_heads) (GQA).
 *   - Calls are asynchronous on `stream` (a hipStream_t); none synchronises the
 *     host and none allocates device memory. Outputs and workspaces are owned
 *     by the caller.
 *   - Return value: MLR_OK (0) or an mlr_status code; mlr_last_error() then
 *     holds a message for the calling thread. Argument errors are detected
 *     before any kernel is launched, so a failed call leaves memory untouched.
 *   - Metadata contents (slot values, block ids, lengths) are validated by the
 *     host layer before the call. Kernels still never access memory outside the
 *     buffers described by the size arguments: an out-of-range slot is skipped
 *     and an out-of-range block id masks its tokens.
 */
#ifndef MLR_ATTN_H
#define MLR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. Values match nothing in torch; the host layer maps them. */
enum mlr_dtype {
  MLR_DTYPE_F32 = 0,
  MLR_DTYPE_F16 = 1,
  MLR_DTYPE_BF16 = 2,
  MLR_DTYPE_F64 = 3
};

/* Index element types for slot_mapping. */
enum mlr_index_dtype { MLR_INDEX_I32 = 0, MLR_INDEX_I64 = 1 };

enum mlr_status {
  MLR_OK = 0,
  MLR_ERR_INVALID = 1,     /* bad argument (shape, stride, pointer, size)  */
  MLR_ERR_UNSUPPORTED = 2, /* valid, but outside what the kernels cover     */
  MLR_ERR_WORKSPACE = 3,   /* workspace missing or too small                */
  MLR_ERR_HIP = 4,         /* the HIP runtime reported an error at launch   */
  MLR_ERR_MERGE = 5        /* a decode workspace's merge-failure flag was set
                              (see mlr_paged_decode_workspace_check)        */
};

/* Message describing the last failed call on this thread ("" if none). */
const char *mlr_last_error(void);

/* Library ABI version (major * 10000 + minor * 100 + patch). */
int mlr_version(void);

/*
 * KV-cache write: k_cache[slot_mapping[t]] = convert(k[t]) and the same for v,
 * for t in [0, num_tokens). Conversion between element types rounds to
 * nearest-even, as Tensor.to does; equal types copy bits.
 *
 * Replaces PagedKVCache.write_slots (runtime/paged_kv_cache.py:194-249), the
 * two index_copy_ calls at :243-249. Slots must be distinct (the host layer
 * rejects duplicates, :238-239); slots outside [0, num_slots) are skipped.
 *   k, v           : [num_tokens, num_kv_heads, head_dim] in src_dtype, any
 *                    strides (the host layer may pass transposed views)
 *   slot_mapping   : [num_tokens], index_dtype
 *   k_cache,v_cache: one layer, [num_slots / block_size, block_size,
 *                    num_kv_heads, head_dim] contiguous, cache_dtype
 */
int mlr_kv_write(const void *k, const void *v, int src_dtype,
                 int64_t num_tokens, int64_t k_stride_t, int64_t k_stride_h,
                 int64_t k_stride_d, int64_t v_stride_t, int64_t v_stride_h,
                 int64_t v_stride_d,
                 const void *slot_mapping, int index_dtype, void *k_cache,
                 void *v_cache, int cache_dtype, int64_t num_slots,
                 int64_t num_kv_heads, int64_t head_dim, void *stream);

/*
 * Bytes of workspace mlr_paged_decode needs for these sizes. `max_context`
 * bounds every context length (the host passes block_table width * block_size).
 * tokens_per_split <= 0 sizes for the library's default splits, whichever
 * kernel the call takes. The defaults: bf16 and FP32 with head_dim 64/128, at
 * most 16 query heads per KV head and block_size a multiple of 16
 * (matrix-core kernel): 320 tokens for bf16 head_dim 64 when max_context <=
 * 5120, else max(256, ceil(max_context / 16)) rounded up to a multiple of
 * 256; other dtypes and shapes an eighth of max_context as a power of two in
 * [32, 256].
 */
size_t mlr_paged_decode_workspace_size(int64_t batch, int64_t num_q_heads,
                                       int64_t head_dim, int64_t max_context,
                                       int64_t tokens_per_split, int dtype);

/*
 * Batched single-token paged decode:
 *   out[b, h] = softmax_t(scale * q[b, h] . K[b, t, h/G]) @ V[b, t, h/G]
 * over t < context_lens[b], where token t of sequence b lives in physical block
 * block_tables[b, t / block_size] at offset t % block_size.
 *
 * Replaces paged_attention_decode_batch_parallel
 * (kernels/reference/paged_attention.py:178-254) and, with batch = 1, the
 * single-request paged_attention_decode (:6-105). Softmax statistics and the
 * split combine are FP32 (FP64 inputs keep FP64 dot products and P@V).
 *   q            : [batch, num_q_heads, head_dim], strides (q_stride_b, q_stride_h)
 *   block_tables : int64 [batch, >= max_blocks_per_seq], row stride
 *                  block_table_stride; entries past ceil(ctx/block_size) unused
 *   context_lens : int64 [batch]; each in [1, max_blocks_per_seq * block_size]
 *   tokens_per_split: split-KV granularity in tokens (<= 0: library default)
 *   workspace    : >= mlr_paged_decode_workspace_size(...) bytes, 256-aligned,
 *                  all-zero before its first use (hipMemset once). It holds
 *                  the splits' partial results; the matrix-core kernel (bf16,
 *                  fp16 and FP32) merges them in the same launch (the workgroup of a
 *                  sequence's last split waits for the words of the others
 *                  to arrive, a zero word meaning "not yet"). Every call
 *                  returns each word it wrote to zero, so the workspace can be
 *                  reused without clearing, by calls of any shape and inside
 *                  captured graphs. Calls that share a workspace must not
 *                  overlap. Should a merge ever wait past its limit (it waits
 *                  only for workgroups launched before its own), it sets the
 *                  workspace's first word and writes NaN, and so does every
 *                  later merge on that workspace until it is cleared:
 *                  mlr_paged_decode_workspace_check reports and clears it.
 *   out          : [batch, num_q_heads, head_dim], strides (out_stride_b, out_stride_h)
 */
int mlr_paged_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k_cache, const void *v_cache,
                     int64_t num_blocks, int64_t block_size,
                     int64_t num_kv_heads, int64_t head_dim,
                     const int64_t *block_tables, int64_t block_table_stride,
                     int64_t max_blocks_per_seq, const int64_t *context_lens,
                     int64_t batch, int64_t num_q_heads, double scale,
                     int dtype, int64_t tokens_per_split, void *workspace,
                     size_t workspace_bytes, void *out, int64_t out_stride_b,
                     int64_t out_stride_h, void *stream);

/*
 * One decode step with the KV write folded in: for every sequence b, the new
 * token's rows new_k[b], new_v[b] ([batch, num_kv_heads, head_dim] in the cache
 * dtype, strides (new_stride_b, new_stride_h), unit stride along head_dim) are
 * written to slot slot_mapping[b] of k_cache/v_cache and attended to as the
 * token at position context_lens[b] - 1. Cache contents and output equal
 * mlr_kv_write(new_k, new_v, slot_mapping) followed by mlr_paged_decode(...)
 * when, as the reference requires of a decode step, slot_mapping[b] is the slot
 * of position context_lens[b] - 1 and the slots are distinct
 * (model/qwen2.py:595-602). The matrix-core kernel (bf16 and FP32, the shapes
 * of mlr_paged_decode's defaults) writes the rows and uses them from LDS,
 * saving the separate write kernel; other dtypes and shapes run the write
 * kernel, then the decode.
 *
 * Replaces the write_slots + paged_attention_decode_batch_parallel pair of
 * Qwen2Attention.forward_decode_batch_with_cache (model/qwen2.py:608-621).
 */
int mlr_paged_decode_append(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, void *k_cache,
    void *v_cache, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
    int64_t head_dim, const int64_t *block_tables, int64_t block_table_stride,
    int64_t max_blocks_per_seq, const int64_t *context_lens, int64_t batch,
    int64_t num_q_heads, double scale, int dtype, int64_t tokens_per_split,
    void *workspace, size_t workspace_bytes, const void *new_k,
    const void *new_v, int64_t new_stride_b, int64_t new_stride_h,
    const int64_t *slot_mapping, void *out, int64_t out_stride_b,
    int64_t out_stride_h, void *stream);

/*
 * The decode step of Qwen2Attention.forward_decode_batch_with_cache after its
 * QKV projection, in one launch: the rotary embedding of q and of the new
 * key, the KV write and the paged decode.
 *
 * Replaces, per layer, Qwen2RotaryEmbedding + apply_rotary_pos_emb at
 * position context_lens[b] - 1 (model/qwen2.py:125-209, called at :605-607),
 * kv_cache.write_slots (:608-613) and paged_attention_decode_batch_parallel
 * (:614-621; kernels/reference/paged_attention.py:178-254). Results equal
 * mlr_qkv_rope_write (positions = context_lens - 1, no bias) followed by
 * mlr_paged_decode bit for bit: the rotation rounds like the reference, each
 * bf16 (fp16) product and sum rounded once, cos and sin of the position
 * rounded to bf16 (fp16).
 *   qkv      : [batch, (num_q_heads + 2 num_kv_heads) * head_dim], row stride
 *              qkv_stride_b, heads in the order q, k, v: the output of the
 *              projection (Qwen2QKVProjection, :211-236) with its bias,
 *              16-byte aligned rows
 *   inv_freq : FP32 [head_dim / 2], the rotary module's inverse frequencies
 *   slot_mapping : int64 [batch], the slot of position context_lens[b] - 1
 * Other arguments as for mlr_paged_decode. bf16 or fp16 with head_dim 64 or 128, at
 * most 16 query heads per KV head and block_size a multiple of 16 only (other
 * shapes: MLR_ERR_INVALID; run mlr_qkv_rope_write, then mlr_paged_decode).
 * No counterpart of its own in the reference: it fuses the calls above.
 */
int mlr_paged_decode_qkv(
    const void *qkv, int64_t qkv_stride_b, const float *inv_freq,
    void *k_cache, void *v_cache, int64_t num_blocks, int64_t block_size,
    int64_t num_kv_heads, int64_t head_dim, const int64_t *block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq, const int64_t *context_lens,
    const int64_t *slot_mapping, int64_t batch, int64_t num_q_heads, double scale,
    int dtype, int64_t tokens_per_split, void *workspace, size_t workspace_bytes, void *out,
    int64_t out_stride_b, int64_t out_stride_h, void *stream);

/*
 * mlr_paged_decode_append without a workspace argument: the decode scratch
 * (split counters and partials) is an 8 MiB array the library keeps on each
 * GPU it runs on, so the call allocates nothing. It has no counterpart in the
 * reference; it is for callers that cannot allocate device memory, such as
 * code under graph capture or a serving loop that forbids allocation.
 *   - Sizes whose scratch would pass 8 MiB are rejected (MLR_ERR_WORKSPACE)
 *     before anything is launched or written; mlr_paged_decode_workspace_size
 *     gives the need (e.g. 64 sequences x 14 query heads x 16 splits of
 *     head_dim 64 take 3.6 MiB; 64 x 28 x 16 of head_dim 128 would take
 *     14.2 MiB and is rejected).
 *   - Every call on one GPU shares that GPU's array: calls that overlap on one
 *     GPU (other streams, other threads) race and must not be issued.
 *   - Arguments, results and cache contents are those of
 *     mlr_paged_decode_append with the same inputs (the same kernels run).
 *   - A merge failure on the array (see mlr_paged_decode_workspace_check) is
 *     reported and cleared by mlr_paged_decode_static_check, outside capture.
 */
int mlr_paged_decode_append_static(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, void *k_cache,
    void *v_cache, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
    int64_t head_dim, const int64_t *block_tables, int64_t block_table_stride,
    int64_t max_blocks_per_seq, const int64_t *context_lens, int64_t batch,
    int64_t num_q_heads, double scale, int dtype, int64_t tokens_per_split,
    const void *new_k, const void *new_v, int64_t new_stride_b,
    int64_t new_stride_h, const int64_t *slot_mapping, void *out,
    int64_t out_stride_b, int64_t out_stride_h, void *stream);

/*
 * Merge-failure check of a decode workspace, and its recovery. The
 * single-launch merge of mlr_paged_decode and its variants waits only for
 * workgroups launched before its own, with a bounded wait; should that wait
 * ever give up, the merge sets the workspace's flag word and writes NaN, and
 * every later multi-split merge on the workspace writes NaN too (partial rows
 * it left behind may be stale). This call waits for `stream`, reads the flag
 * word and returns MLR_OK when it is clear. When it is set, it zeroes the
 * whole workspace (a fill kernel on `stream`, then a wait) and returns
 * MLR_ERR_MERGE: the outputs of the multi-split decodes since the failure
 * are NaN and must be recomputed; the workspace is usable again. It
 * synchronises the host, so it is refused (MLR_ERR_INVALID) while `stream`
 * is being captured into a graph; no other stream may be using the
 * workspace meanwhile.
 *
 * No counterpart in the reference, whose PyTorch decode cannot fail this way;
 * it keeps the reference's contract that failures surface as errors
 * (runtime/paged_kv_cache.py:228-239) rather than as silent values.
 * mlr_paged_decode_static_check does the same for the library's own scratch of
 * mlr_paged_decode_append_static on the current device.
 */
int mlr_paged_decode_workspace_check(void *workspace, size_t workspace_bytes, void *stream);
int mlr_paged_decode_static_check(void *stream);

/*
 * Paged chunk-prefill attention for a packed batch of sequences (varlen):
 * sequence s owns query rows [query_start_loc[s], query_start_loc[s+1]) of q,
 * whose absolute positions are prefix_len_s + i with
 * prefix_len_s = context_lens[s] - query_len_s. Query i of sequence s attends to
 * every cached key at position p <= prefix_len_s + i (the chunk's own keys must
 * already be written to the cache).
 *
 * Replaces paged_attention_prefill_chunk_tiled
 * (kernels/reference/paged_attention.py:346-434): FP32 online softmax and FP32
 * P@V, output rounded once to the input type. kv_tile is the reference's
 * tile_size (the key tile of its online-softmax loop, :398-431), which orders
 * the FP32 accumulation and nothing else; the kernels step by their own key
 * tile (64 keys on the bf16 matrix-core kernel) whatever kv_tile is, so
 * results differ from the reference's only by rounding, as they do between
 * the reference's own tile sizes.
 *   q               : [total_q, num_q_heads, head_dim], strides (q_stride_t, q_stride_h)
 *   block_tables    : int64 [num_seqs, >= max_blocks_per_seq], row stride
 *   query_start_loc : int64 [num_seqs + 1], non-decreasing, starts at 0
 *   context_lens    : int64 [num_seqs]; context >= query_len,
 *                     context <= max_blocks_per_seq * block_size
 *   max_query_len   : upper bound of every query_len (sizes the grid)
 *   out             : [total_q, num_q_heads, head_dim], strides (out_stride_t, out_stride_h)
 */
int mlr_paged_prefill(const void *q, int64_t q_stride_t, int64_t q_stride_h,
                      const void *k_cache, const void *v_cache,
                      int64_t num_blocks, int64_t block_size,
                      int64_t num_kv_heads, int64_t head_dim,
                      const int64_t *block_tables, int64_t block_table_stride,
                      int64_t max_blocks_per_seq,
                      const int64_t *query_start_loc,
                      const int64_t *context_lens, int64_t num_seqs,
                      int64_t max_query_len, int64_t num_q_heads, double scale,
                      int dtype, int64_t kv_tile, void *out,
                      int64_t out_stride_t, int64_t out_stride_h, void *stream);

/*
 * Single-sequence chunk prefill with host-side scalars, the exact argument
 * shape of paged_attention_prefill_chunk_tiled(q, k_cache, v_cache,
 * block_table, prefix_len, context_len, block_size, tile_size)
 * (kernels/reference/paged_attention.py:346-356). block_table is an int64
 * device array of at least ceil(context_len / block_size) entries and
 * context_len == prefix_len + chunk_len.
 */
int mlr_paged_prefill_chunk(const void *q, int64_t q_stride_t,
                            int64_t q_stride_h, const void *k_cache,
                            const void *v_cache, int64_t num_blocks,
                            int64_t block_size, int64_t num_kv_heads,
                            int64_t head_dim, const int64_t *block_table,
                            int64_t block_table_len, int64_t prefix_len,
                            int64_t context_len, int64_t num_q_heads,
                            double scale, int dtype, int64_t kv_tile,
                            void *out, int64_t out_stride_t,
                            int64_t out_stride_h, void *stream);

/*
 * Fused pre-attention step of one layer: optional projection bias, rotary
 * embedding of the q and k heads, and the KV-cache write, in one launch.
 *
 * Replaces, after the QKV projection GEMM, the bias of Qwen2QKVProjection
 * (model/qwen2.py:211-236), Qwen2RotaryEmbedding + apply_rotary_pos_emb
 * (:125-209, called at :605-607 and :737-739) and kv_cache.write_slots
 * (:608-613, :741-746; runtime/paged_kv_cache.py:243-249). Rounding follows
 * the reference operation by operation in the model dtype: f = float(pos) *
 * inv_freq[i] in FP32; c, s = dtype(cos f), dtype(sin f); each product and the
 * sum rounded to dtype (FP32 without fma contraction).
 *   qkv          : [num_tokens, (num_q_heads + 2 num_kv_heads) * head_dim], row
 *                  stride qkv_stride_t, heads in the order q, k, v, unit stride
 *   bias         : [(num_q_heads + 2 num_kv_heads) * head_dim] or NULL; added
 *                  (then rounded to dtype) before the rotation
 *   positions    : int64 [num_tokens]
 *   inv_freq     : FP32 [head_dim / 2], the rotary module's inverse frequencies
 *   slot_mapping : int32/int64 [num_tokens]; a slot outside [0, num_slots) is
 *                  not written (q is)
 *   q_out        : [num_tokens, num_q_heads, head_dim], row stride q_out_stride_t
 *   k_cache, v_cache : one layer, [num_slots / block_size, block_size,
 *                  num_kv_heads, head_dim] contiguous
 * qkv, bias, q_out and the cache share dtype (F32, F16 or BF16).
 */
int mlr_qkv_rope_write(const void *qkv, int64_t qkv_stride_t, const void *bias,
                       const int64_t *positions, const float *inv_freq,
                       const void *slot_mapping, int index_dtype, void *q_out,
                       int64_t q_out_stride_t, void *k_cache, void *v_cache,
                       int64_t num_slots, int64_t num_tokens, int64_t num_q_heads,
                       int64_t num_kv_heads, int64_t head_dim, int dtype, void *stream);

/*
 * Batched weighted row sum in FP32, out[b, d] = sum_n p[b, n] * v[b, n, d],
 * with p [batch, 64], v [batch, 64, 256] and out [batch, 256], all
 * contiguous; v and out 16-byte aligned. Sums run in row order with fma.
 *
 * Replaces forward(p, v) of the reference's only native extension
 * (kernels/cuda/paged_attention_accumulator.cu:83-100; Python wrapper
 * kernels/cuda/accumulator.py:21-37).
 */
int mlr_pa_accumulate(const float *p, const float *v, float *out, int64_t batch, void *stream);

/*
 * ModelBatch metadata of one scheduler step from one row per request:
 * req_info [num_reqs, 2] int64 holds (first position, token count) of
 * request r, block_tables its padded block table (row stride
 * block_table_stride, max_blocks entries used). Writes, for the packed rows,
 *   query_start_loc [num_reqs + 1] = 0, prefix sums of the counts
 *   context_lens    [num_reqs]     = first position + count
 *   positions       [num_tokens]   = first position + i
 *   slot_mapping    [num_tokens]   = block_tables[r, p / block_size] * block_size
 *                                    + p % block_size
 * (slot -1 where p < 0 or p / block_size >= max_blocks). The counts must be
 * >= 0 and sum to num_tokens; num_reqs <= 16384.
 *
 * Replaces the per-token host loops of build_model_batch
 * (runtime/model_runner.py:54-64 append_slots, and the position, offset and
 * context-length lists of :66-143).
 */
int mlr_build_step_metadata(const int64_t *req_info, const int64_t *block_tables,
                            int64_t block_table_stride, int64_t max_blocks, int64_t num_reqs,
                            int64_t num_tokens, int64_t block_size, int64_t *positions,
                            int64_t *slot_mapping, int64_t *query_start_loc,
                            int64_t *context_lens, void *stream);

/*
 * RMSNorm of `rows` rows of `hidden` elements, after a residual add when
 * `residual` is given:
 *   r   = x + residual, rounded to the dtype and written to residual_out
 *         (which may be residual itself); r = x without a residual
 *   out = weight * dtype(r / sqrt(mean(r^2) + eps))
 * Statistics in FP32 for bf16 and fp16; every step rounded as the PyTorch
 * module's separate operations round it (only the order of the row sum
 * differs). dtype bf16, fp16 or FP32; weight [hidden] of the same dtype; row
 * strides in elements. out may be x.
 *
 * Replaces Qwen2RMSNorm.forward (model/qwen2.py:88-123) and the residual add
 * before the post-attention norm of Qwen2DecoderLayer (:794-940).
 */
int mlr_rms_norm(const void *x, int64_t x_stride, const void *residual, int64_t residual_stride,
                 void *residual_out, int64_t residual_out_stride, const void *weight, void *out,
                 int64_t out_stride, int64_t rows, int64_t hidden, double eps, int dtype,
                 void *stream);

/*
 * out[r, j] = dtype(silu(gate_up[r, j])) * gate_up[r, intermediate + j] for
 * j < intermediate: the gate and up projections side by side in one row, as
 * one GEMM with the two weights stacked writes them. silu(g) = g / (1 +
 * expf(-g)) in FP32, rounded to the dtype, then the product rounded to the
 * dtype, as F.silu(gate) * up rounds them. dtype bf16, fp16 or FP32.
 *
 * Replaces the activation and product of Qwen2MLP.forward
 * (model/qwen2.py:768-792).
 */
int mlr_silu_mul(const void *gate_up, int64_t gate_up_stride, void *out, int64_t out_stride,
                 int64_t rows, int64_t intermediate, int dtype, void *stream);

/*
 * Diagnostics. No counterpart in the reference: a read-only pass that
 * measures the memory floor of a decode step on its own block list.
 *
 * mlr_paged_kv_read_floor reads, for every sequence b < batch and every
 * context token t < context_lens[b] (clamped to max_blocks * block_size),
 * the whole slot row (row_bytes = Hkv * D * element size, a multiple of 16)
 * of K and of V through block_tables, and XOR-folds every 32-bit word of
 * those rows into out: one word per (sequence, item of tokens_per_item
 * tokens), out[b * items + i], 0 for items past the context; blocks outside
 * [0, num_blocks) read as zeros. The XOR of all out words is the XOR of all
 * the words read. tokens_per_item is a multiple of block_size, at most 512
 * blocks; block_size is a power of two; out_len >= the count that
 * mlr_paged_kv_read_floor_outputs returns (0 for invalid sizes).
 */
size_t mlr_paged_kv_read_floor_outputs(int64_t batch, int64_t max_blocks, int64_t block_size,
                                       int64_t tokens_per_item);
int mlr_paged_kv_read_floor(const void *k_cache, const void *v_cache, int64_t num_blocks,
                            int64_t block_size, int64_t row_bytes, const int64_t *block_tables,
                            int64_t bt_stride, int64_t max_blocks, const int64_t *context_lens,
                            int64_t batch, int64_t tokens_per_item, uint32_t *out,
                            int64_t out_len, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MLR_ATTN_H */
