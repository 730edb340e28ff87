/*
 * slc_hip.h -- C ABI of the gfx950 (MI355X) KernelIR backend.
 *
 * Every entry point launches hand-written HIP kernels on the stream it is
 * given and returns immediately (no host synchronisation).  Pointers are
 * device pointers; strides are in ELEMENTS; the innermost (head-dim / hidden)
 * axis of every tensor must be contiguous (stride 1), exactly as the
 * reference's Python wrappers require.
 *
 * Return value: SLC_OK (0) on success, SLC_ERR_INVALID_ARGUMENT (-1) when an
 * argument check fails, or a positive hipError_t from the launch.  The text of
 * the last error of the calling thread is available from slc_hip_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * src/stateful_llm_compiler/):
 *   slc_hip_decode_attention   backends/triton_attention.py:134-210
 *                              (triton_decode_attention; semantics of
 *                              execution.py:281-327)
 *   slc_hip_paged_decode_attention, slc_hip_paged_kv_store,
 *   slc_hip_paged_rope_decode_attention: the paged layout
 *                              the reference plans next (docs/kv-bufferization.md:317-323)
 *   slc_hip_kv_store           backends/triton_kv.py:71-129 (triton_kv_store;
 *                              semantics of execution.py:743-781 native_kv_store)
 *   slc_hip_rms_norm           backends/triton_rmsnorm.py:205-443
 *                              (triton_rms_norm; semantics of execution.py:674-692)
 *   slc_hip_rope               backends/triton_rope.py:299-390 (triton_rope;
 *                              semantics of execution.py:741-767)
 *   slc_hip_linear             backends/triton_linear.py:87-148 (triton_linear)
 *                              and triton_executor.py:159-176 (kernel.cublas.linear)
 *   slc_hip_linear_tile        the same, tile chosen by a profile plan
 *                              (cost_model.py:125-245, lowering_selection.py:12-72)
 *   slc_hip_prefill_attention  backends/triton_prefill_attention.py:152-232
 *                              (semantics of execution.py:707-739)
 */
#ifndef SLC_HIP_H_
#define SLC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define SLC_API __attribute__((visibility("default")))
#else
#define SLC_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags used for every tensor argument */
enum slc_dtype {
  SLC_F32 = 0,
  SLC_F16 = 1,
  SLC_BF16 = 2,
  SLC_I32 = 3,
  SLC_I64 = 4
};

/* SLC_ERR_UNSUPPORTED: a fused entry point's kernel does not take these
 * arguments; nothing was launched and the caller runs the unfused ops. */
enum slc_status { SLC_OK = 0, SLC_ERR_INVALID_ARGUMENT = -1, SLC_ERR_UNSUPPORTED = -2 };

/*
 * Softmax order of the attention entry points.
 *   SLC_SOFTMAX_ONLINE : single pass; the running (unnormalised) probabilities
 *                        are rounded to the I/O dtype for the P.V product and
 *                        the sum divides the fp32 result (flash-attention form).
 *   SLC_SOFTMAX_EXACT  : the reference executor's order (execution.py:319-327,
 *                        softmax(...).to(dtype) then matmul): probabilities
 *                        are normalised in fp32, then rounded, then P.V.
 *                        K and V are still read once (decode) / the key tiles
 *                        twice from LDS-staged tiles (prefill).
 */
enum slc_softmax_order { SLC_SOFTMAX_ONLINE = 0, SLC_SOFTMAX_EXACT = 1 };

/*
 * Split-sequence choice of decode attention (the split_tokens argument):
 *   0                  : fixed chunk per (batch, kv head), sized so the grid
 *                        fills the GPU; the chunks past a sequence's length
 *                        exit at once
 *   > 0                : fixed chunk of that many tokens (rounded up to the
 *                        workgroup's 128-token sweep)
 *   SLC_SPLIT_BALANCED : length-balanced split: every workgroup streams one
 *                        contiguous piece of one sequence, the pieces sized
 *                        from the device-side lengths so that all are about
 *                        equal (online order, batch <= 2048; else as 0)
 */
enum slc_split { SLC_SPLIT_BALANCED = -1 };

/* Library version (major*10000 + minor*100 + patch). */
SLC_API int slc_hip_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
SLC_API const char* slc_hip_last_error(void);

/*
 * BENCH-ONLY.  Not for serving code: while armed, the calling thread's
 * entry points change what they launch (see slc_hip_set_timing_repeats).
 *
 * Measurement hook (no counterpart in the reference, which times whole calls
 * with torch events): arm two hipEvent_t handles for the calling thread; each
 * later entry point with a multi-kernel launch sequence records `begin` just
 * before and `end` just after its dominant kernel on the launch stream, so a
 * benchmark can time that kernel alone.  Pass (NULL, NULL) to disarm.
 */
SLC_API void slc_hip_set_timing_events(void* begin, void* end);

/*
 * BENCH-ONLY.  Not for serving code: a repeat count above 1 makes every
 * armed call launch its dominant kernel that many times.
 *
 * Measurement hook (no counterpart in the reference): while timing events are
 * armed, launch the dominant kernel `repeats` times back to back between them
 * (it rewrites the same outputs each time), so the per-launch average excludes
 * the launch latency of a single call.  Default 1.
 */
SLC_API void slc_hip_set_timing_repeats(int repeats);

/*
 * kv_store: scatter the current step's K/V rows into the preallocated
 * B x capacity x H x D buffers.
 *   key_buffer/value_buffer : [batch, capacity, heads, head_dim], contiguous
 *   key/value               : [batch, heads, tokens, head_dim], strides
 *                             (sb, sh, st) in elements, head_dim contiguous
 *   positions               : [batch] int64 (first destination row per batch)
 *   overflow                : optional device int set to 1 when a row falls
 *                             outside [0, capacity) (never cleared here)
 * Row t of batch b lands at buffer row positions[b] + t; rows whose position is
 * outside [0, capacity) are skipped (the reference masks them the same way).
 * The copy is bit-exact for every dtype.
 */
SLC_API int slc_hip_kv_store(void* key_buffer, void* value_buffer, const void* key,
                     const void* value, const int64_t* positions,
                     int* overflow, int dtype,
                     int64_t batch, int64_t heads, int64_t tokens,
                     int64_t head_dim, int64_t capacity, int64_t key_stride_b,
                     int64_t key_stride_h, int64_t key_stride_t,
                     int64_t value_stride_b, int64_t value_stride_h,
                     int64_t value_stride_t, void* stream);

/*
 * decode_attention: single-token GQA attention that reads the physical KV
 * buffers directly.
 *   query        : [batch, q_heads, 1, head_dim], strides (q_sb, q_sh)
 *   key/value    : physical buffers indexed [b, s, h, :] with strides
 *                  (kv_sb, kv_ss, kv_sh) -- contiguous_bshd buffers have
 *                  (capacity*H*D, H*D, D); BHSD views are accepted as well.
 *                  Both buffers must share these strides.
 *   lengths      : [batch] of lengths_dtype (SLC_I64 or SLC_I32) on device
 *   mask         : additive mask [batch, 1, 1, mask_len] with strides
 *                  (mask_sb, mask_ss), dtype mask_dtype; may be NULL (= zeros)
 *   output       : [batch, q_heads, 1, head_dim], strides (out_sb, out_sh),
 *                  same dtype as query
 *   workspace    : device scratch of at least
 *                  slc_hip_decode_attention_workspace_size(...) bytes (split
 *                  partials; may be NULL when that size is 0)
 *   counters     : caller-owned int array of at least
 *                  slc_hip_decode_attention_counter_count(batch, kv_heads)
 *                  elements (cross-workgroup arrival counters): zero-fill it
 *                  once when it is allocated; every call leaves it zero
 *                  again.  Calls that share counters or a workspace must not
 *                  run concurrently (calls on one stream never do); give each
 *                  stream (or each captured graph that may replay
 *                  concurrently) its own.
 * Token s of batch b is attended iff s < min(lengths[b], mask_len, capacity).
 * kv head of query head h is h / (q_heads / kv_heads).
 * split_tokens selects the split (slc_split above; ignored by the exact
 * order, which runs one chunk per (batch, kv head)).
 * softmax_order: SLC_SOFTMAX_ONLINE or SLC_SOFTMAX_EXACT; the exact order
 * takes min(mask_len, capacity) up to
 * slc_hip_decode_attention_exact_max_tokens(head_dim, dtype) tokens.
 */
SLC_API int64_t slc_hip_decode_attention_workspace_size(int64_t batch, int64_t q_heads,
                                                int64_t head_dim,
                                                int64_t mask_len,
                                                int64_t kv_heads, int dtype,
                                                int64_t split_tokens);

SLC_API int64_t slc_hip_decode_attention_counter_count(int64_t batch, int64_t kv_heads);

SLC_API int slc_hip_decode_attention(
    const void* query, const void* key_buffer, const void* value_buffer,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype,
    void* output, void* workspace, int64_t workspace_bytes, int* counters,
    int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t capacity, int64_t mask_len, int64_t q_stride_b, int64_t q_stride_h,
    int64_t kv_stride_b, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int64_t split_tokens, int softmax_order,
    void* stream);

/*
 * slc_hip_decode_attention without allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 * Same arguments and result as slc_hip_decode_attention minus the workspace
 * and counters: the split partials (at most 8 MiB) and arrival counters (at
 * most 131072) live in one device array of the library that each GPU holds
 * until the process ends.  A call needing more returns
 * SLC_ERR_INVALID_ARGUMENT before any device work.  The first call on a GPU
 * launches one small kernel on `stream` to zero the counters; no call
 * allocates.  All calls on one GPU share its array: calls that overlap in
 * time on one GPU (other streams, other threads) race; calls on one stream
 * do not.
 */
SLC_API int slc_hip_decode_attention_noalloc(
    const void* query, const void* key_buffer, const void* value_buffer,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype,
    void* output, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
    int64_t head_dim, int64_t capacity, int64_t mask_len, int64_t q_stride_b,
    int64_t q_stride_h, int64_t kv_stride_b, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int64_t split_tokens, int softmax_order,
    void* stream);

/*
 * Paged KV (reference: the paged layout and block table that
 * docs/kv-bufferization.md:317-323 names as the next step after the
 * contiguous buffers; KVStateType.layout, ir.py:87).  Per layer, K and V rows
 * live in page pools [num_pages, page_tokens, kv_heads, head_dim] with row
 * stride kv_stride_s, head stride kv_stride_h and page stride page_stride
 * (elements); block_table is int32 [batch, >= pages_per_seq] with batch
 * stride table_stride_b, entry j of sequence b naming the pool page of its
 * tokens [j * page_tokens, (j + 1) * page_tokens).  page_tokens is a power of
 * two >= 16; capacity = pages_per_seq * page_tokens.
 *
 * slc_hip_paged_decode_attention: slc_hip_decode_attention over the paged
 * layout, same arguments otherwise (bf16/fp16, head_dim 64 or 128, at most 16
 * query heads per kv head; workspace and counters sized by
 * slc_hip_decode_attention_workspace_size / _counter_count).  A call equals
 * the contiguous call over the same tokens bit for bit.
 */
SLC_API int slc_hip_paged_decode_attention(
    const void* query, const void* key_pool, const void* value_pool, const int* block_table,
    int64_t table_stride_b, int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t mask_len,
    int64_t q_stride_b, int64_t q_stride_h, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b, int64_t out_stride_h,
    float scale, int64_t split_tokens, int softmax_order, void* stream);

/*
 * slc_hip_paged_kv_store: slc_hip_kv_store over the paged layout: row t of
 * (b, h) goes to position positions[b] + t of sequence b (its page from the
 * block table); positions outside [0, capacity) are dropped and set
 * *overflow (if not NULL).  Rows, strides and pointers 16-byte aligned.
 */
SLC_API int slc_hip_paged_kv_store(
    void* key_pool, void* value_pool, const int* block_table, int64_t table_stride_b,
    int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride, int64_t kv_stride_s,
    int64_t kv_stride_h, const void* key, const void* value, const int64_t* positions,
    int* overflow, int dtype, int64_t batch, int64_t heads, int64_t tokens, int64_t head_dim,
    int64_t key_stride_b, int64_t key_stride_h, int64_t key_stride_t, int64_t value_stride_b,
    int64_t value_stride_h, int64_t value_stride_t, void* stream);

/*
 * slc_hip_paged_rope_decode_attention: slc_hip_rope_decode_attention over the
 * paged layout (the paged attention's pool, block-table and page arguments,
 * the RoPE variant's key/value/cosine/sine, lengths_out and overflow): RoPE of
 * the query and the new key, the new key and value row written at position
 * lengths[b] of sequence b (its page from the block table), the length
 * advance and the attention, in one kernel; equal bit for bit to RoPE, the
 * paged KV store and the paged attention run in turn.  Returns
 * SLC_ERR_UNSUPPORTED (nothing launched) for the cases its kernel does not
 * take, as slc_hip_rope_decode_attention does.  Workspace and counters as for
 * slc_hip_decode_attention_workspace_size(..., 0) / _counter_count.
 */
SLC_API int slc_hip_paged_rope_decode_attention(
    const void* query, const void* key, const void* value, const void* cosine, const void* sine,
    void* key_pool, void* value_pool, const int* block_table, int64_t table_stride_b,
    int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride, const int64_t* lengths,
    int64_t* lengths_out, int* overflow, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t mask_len,
    int64_t q_stride_b, int64_t q_stride_h, int64_t k_stride_b, int64_t k_stride_h,
    int64_t v_stride_b, int64_t v_stride_h, int64_t cos_stride_b, int64_t sin_stride_b,
    int64_t kv_stride_s, int64_t kv_stride_h, int64_t mask_stride_b, int64_t mask_stride_s,
    int64_t out_stride_b, int64_t out_stride_h, float scale, int softmax_order, void* stream);

/* Longest mask the SLC_SOFTMAX_EXACT order takes (INT64_MAX: no limit). */
SLC_API int64_t slc_hip_decode_attention_exact_max_tokens(int64_t head_dim, int dtype);

/*
 * rms_norm over the last axis:
 *   normalized = x * rsqrt(mean(x^2) + epsilon)            (fp32)
 *   round_before_weight=1 : out = weight * round(normalized, norm_dtype)
 *   round_before_weight=0 : out = round(normalized * weight, out_dtype)
 * input rows are [rows, hidden] with row stride in_stride_row; output rows
 * have stride out_stride_row.  norm_dtype is the dtype the normalized value
 * is materialised in before the weight multiply (the reference's
 * output_dtype or the input dtype).
 * waves_per_row picks the kernel variant -- the gfx950 counterpart of the
 * reference plan's num_warps: 1 = one wavefront per row, the row held in
 * registers (one HBM read and write; same dtype throughout, 16-byte aligned
 * rows of at most 512 vectors); 4 = a 256-thread workgroup per row (any
 * dtypes; the second pass re-reads the row from L2); 0 = the first when it
 * applies, else the second.  A variant that does not apply falls back to 4.
 */
SLC_API int slc_hip_rms_norm(const void* input, const void* weight, void* output,
                     int in_dtype, int weight_dtype, int out_dtype,
                     int norm_dtype, int64_t rows, int64_t hidden,
                     int64_t in_stride_row, int64_t out_stride_row,
                     float epsilon, int round_before_weight, int waves_per_row,
                     void* stream);

/*
 * rope (dual output, Qwen2 half rotation):
 *   q' = round(q*cos) + round(rotate_half(q)*sin), same for k,
 *   rotate_half(x) = cat(-x[D/2:], x[:D/2]);
 * query [B, QH, T, D], key [B, KVH, T, D], cos/sin [B, T, D]; every tensor
 * passes (sb, sh, st) or (sb, st) strides in elements; all share one dtype.
 */
SLC_API int slc_hip_rope(const void* query, const void* key, const void* cosine,
                 const void* sine, void* query_out, void* key_out, int dtype,
                 int64_t batch, int64_t q_heads, int64_t kv_heads,
                 int64_t tokens, int64_t head_dim, int64_t q_sb, int64_t q_sh,
                 int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st,
                 int64_t cos_sb, int64_t cos_st, int64_t sin_sb,
                 int64_t sin_st, int64_t qo_sb, int64_t qo_sh, int64_t qo_st,
                 int64_t ko_sb, int64_t ko_sh, int64_t ko_st, void* stream);

/*
 * linear: output[m, n] = sum_k input[m, k] * weight[n, k] (+ bias[n]),
 * fp32 accumulation, one rounding to dtype on store.
 *   input  : rows x in_features, row stride in_stride_row (elements)
 *   weight : out_features x in_features, contiguous (PyTorch Linear layout)
 *   bias   : out_features or NULL
 *   output : rows x out_features, row stride out_stride_row
 */
SLC_API int slc_hip_linear(const void* input, const void* weight,
                           const void* bias, void* output, int dtype,
                           int64_t rows, int64_t out_features,
                           int64_t in_features, int64_t in_stride_row,
                           int64_t out_stride_row, void* stream);

/*
 * linear_tile: slc_hip_linear with the workgroup tile of the prefill-sized
 * (rows > 64, bf16/fp16) MFMA path chosen by the caller: the variant a
 * profile plan selects, as the reference's planner selects an RMSNorm backend
 * from measured latencies (cost_model.py:125-245,
 * passes/lowering_selection.py:12-72).  Every tile gives bit-identical
 * results (each output's k range accumulates in the same order); only the
 * launch shape differs.  SLC_TILE_AUTO is slc_hip_linear's choice (128 x 128);
 * decode-sized rows and the fp32 path ignore the tile.
 */
#define SLC_TILE_AUTO 0
#define SLC_TILE_128X128 1
#define SLC_TILE_128X64 2
#define SLC_TILE_64X128 3
#define SLC_TILE_64X64 4
#define SLC_TILE_32X64 5
/* Deep-pipelined forms (producer waves stream k-tiles into a multi-stage LDS
 * ring); shapes they cannot take (K not a multiple of 64, outputs not
 * 16-byte aligned) run SLC_TILE_128X128. */
#define SLC_TILE_R128X128 6
#define SLC_TILE_R256X128 7
#define SLC_TILE_R128X64 8
#define SLC_TILE_R64X64 9
/* Persistent 256 x 128 ring (one workgroup per CU walks the output tiles;
 * the next tile's k-tiles stream in while the current one is written out);
 * calls with a residual run SLC_TILE_R256X128. */
#define SLC_TILE_S256X128 10
SLC_API int slc_hip_linear_tile(const void* input, const void* weight,
                                const void* bias, void* output, int dtype,
                                int64_t rows, int64_t out_features,
                                int64_t in_features, int64_t in_stride_row,
                                int64_t out_stride_row, int tile, void* stream);

/*
 * prefill_attention: multi-token GQA attention.
 *   query [B, QH, T, D], key/value [B, KVH, T, D] with (sb, sh, st) strides,
 *   mask  : additive [B, 1, T, T] with (m_sb, m_sq, m_sk) strides, dtype
 *           mask_dtype, or NULL (= zeros)
 *   causal: nonzero removes keys after each query (the op's causal=True)
 *   output [B, QH, T, D] with (o_sb, o_sh, o_st) strides, dtype of query
 *   softmax_order: SLC_SOFTMAX_ONLINE or SLC_SOFTMAX_EXACT (any length)
 * kv head of query head h is h / (QH / KVH).
 */
SLC_API int slc_hip_prefill_attention(
    const void* query, const void* key, const void* value, const void* mask,
    int mask_dtype, void* output, int dtype, int64_t batch, int64_t q_heads,
    int64_t kv_heads, int64_t tokens, int64_t head_dim, int causal, int64_t q_sb,
    int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st,
    int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq,
    int64_t m_sk, int64_t o_sb, int64_t o_sh, int64_t o_st, float scale,
    int softmax_order, void* stream);

/*
 * prefill_attention_classes: slc_hip_prefill_attention with the mask's tile
 * classes from slc_hip_prefill_mask_tiles (or NULL: every tile loads its
 * mask).  Tiles of class 0 are not visited (no K/V or mask traffic), class 1
 * applies the causal pattern from the indices, class 2 loads and adds the
 * mask tile; the result equals adding the whole mask.  The reference loops
 * over every key tile and reads the whole mask
 * (backends/triton_prefill_attention.py:69); this is the same operation.
 */
SLC_API int slc_hip_prefill_attention_classes(
    const void* query, const void* key, const void* value, const void* mask,
    int mask_dtype, const unsigned char* mask_tile_classes, void* output, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t head_dim,
    int causal, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq,
    int64_t m_sk, int64_t o_sb, int64_t o_sh, int64_t o_st, float scale,
    int softmax_order, void* stream);

/*
 * prefill_mask_tiles: classify an additive [B, 1, T, T] mask (strides m_sb,
 * m_sq, m_sk in elements) per (batch, 64-query block, 64-key tile) into
 * classes[B][ceil(T/64)][ceil(T/64)]: 0 = every entry -inf, 1 = +0 where
 * key <= query and -inf above (the causal pattern), 2 = anything else.
 * prefill_mask_tile_count gives the number of class bytes.  (Supports
 * serve.prefill_attention, execution.py:707-739; no reference counterpart.)
 */
SLC_API int64_t slc_hip_prefill_mask_tile_count(int64_t batch, int64_t tokens);
SLC_API int slc_hip_prefill_mask_tiles(const void* mask, int mask_dtype, int64_t batch,
                                       int64_t tokens, int64_t m_sb, int64_t m_sq,
                                       int64_t m_sk, unsigned char* classes, void* stream);

/*
 * Ops that complete a Qwen2 step without eager PyTorch kernels.  None has a
 * separate reference kernel: the reference runs them as PyTorch ops
 * (execution.py:500-528 handler table; qwen2.py model code cited per op).
 *   embedding  : output[r, :] = table[ids[r], :]; ids outside [0, vocab) set
 *                *bad_index (optional) and read row 0      (qwen2.py:427-430)
 *   add        : output = a + b, elementwise, contiguous    (qwen2.py:288-294)
 *   swiglu     : output = round(silu(gate)) * up             (qwen2.py:253-256)
 *   rope_table : cos/sin[b, t, :] of cat(f, f), f = positions[b, t] * inv_freq
 *                (fp32 math, rounded to dtype), outputs [B, T, D] contiguous
 *                                                           (qwen2.py:136-149)
 *   kv_advance : lengths_out = lengths_in + delta (may alias); sets *overflow
 *                when a length leaves [0, capacity]          (execution.py:421-443)
 *   argmax     : output[r] = index of the first maximum of row r (NaN counts
 *                as the maximum, as in torch.argmax).  With a scratch
 *                workspace of slc_hip_argmax_workspace_size(rows) bytes and
 *                `rows` counters (caller-owned, zero-filled once, left zeroed
 *                by every call; neither shared by concurrent calls) wide rows
 *                are split over several workgroups; with NULL each row is one
 *                workgroup.  Same result.
 */
SLC_API int slc_hip_embedding(const int64_t* ids, const void* table, void* output,
                              int dtype, int64_t rows, int64_t hidden, int64_t vocab,
                              int* bad_index, void* stream);
SLC_API int slc_hip_add(const void* a, const void* b, void* output, int dtype,
                        int64_t numel, void* stream);
SLC_API int slc_hip_swiglu(const void* gate, const void* up, void* output, int dtype,
                           int64_t numel, void* stream);
SLC_API int slc_hip_rope_table(const int64_t* positions, const float* inv_freq,
                               void* cosine, void* sine, int dtype, int64_t batch,
                               int64_t tokens, int64_t pos_stride_b, int64_t head_dim,
                               void* stream);
SLC_API int slc_hip_kv_advance(const int64_t* lengths_in, int64_t* lengths_out,
                               int64_t batch, int64_t delta, int64_t capacity,
                               int* overflow, void* stream);
SLC_API int64_t slc_hip_argmax_workspace_size(int64_t rows);
SLC_API int slc_hip_argmax(const void* logits, int64_t* output, int dtype, int64_t rows,
                           int64_t cols, int64_t row_stride, void* workspace,
                           int64_t workspace_bytes, int* counters, int64_t num_counters,
                           void* stream);

/*
 * Fused decode-step ops (no single counterpart in the reference: each one
 * replaces a short sequence of the reference's KernelIR ops, and produces
 * bit-identically what that sequence of this library's kernels produces).
 * rows <= 32 (decode-sized), dtype bf16 or fp16, 16-byte aligned rows; larger
 * or other inputs are rejected with SLC_ERR_INVALID_ARGUMENT and the caller
 * runs the unfused sequence.
 *
 *   norm_linear_group : y_j = linear(rms_norm(x, norm_weight), w_j, b_j) for
 *                       count = 1..3 matrices [n_j, hidden] (Q/K/V); no norm
 *                       when norm_weight is NULL.  Replaces
 *                       kernel.triton.rms_norm (round_before_weight=1) plus
 *                       one kernel.triton.linear per matrix
 *                       (triton_rmsnorm.py:205-443, triton_linear.py:87-148).
 *                       One matrix of >= 16384 rows with a norm (the LM head
 *                       and the final norm): one launch for rows <= 16;
 *                       SLC_ERR_UNSUPPORTED (nothing launched) above, where
 *                       the caller runs the norm and the linear.
 *   norm_linear_swiglu: y = round(silu(round(x_n . w_gate^T))) *
 *                       round(x_n . w_up^T), x_n = rms_norm(x, norm_weight)
 *                       (the Qwen2 MLP front, qwen2.py:253-256).
 *   linear_residual   : y = residual + round(x . w^T + bias) (O / down
 *                       projection and the residual add, qwen2.py:288-294).
 *   rope_kv_store     : q_out = rope(q); key_buffer[b, positions[b] + t] =
 *                       rope(k)[b, :, t]; value_buffer[...] = v[b, :, t]; rows
 *                       at or past the capacity are skipped and set *overflow
 *                       (triton_rope.py:299-390 then triton_kv.py:71-129).
 *                       Buffers are contiguous [B, capacity, kv_heads, D].
 *                       With lengths_out set it also advances the lengths:
 *                       lengths_out[b] = positions[b] + advance (in place
 *                       allowed), flagging *overflow past the capacity, as
 *                       slc_hip_kv_advance does after the store (the
 *                       runtime.kv.advance that follows the store in the
 *                       decode graph, execution.py:741-767).  The advance
 *                       rides on the store kernel when `counters` (>= 1 int,
 *                       caller-owned, zero-filled once, left zeroed, not
 *                       shared by concurrent calls) is given, else it is a
 *                       second launch.
 */
SLC_API int slc_hip_norm_linear_group(
    const void* x, int64_t x_rs, const void* norm_weight, float epsilon, int64_t rows,
    int64_t hidden, int count, const void* w0, const void* b0, void* y0, int64_t n0,
    int64_t y0_rs, const void* w1, const void* b1, void* y1, int64_t n1, int64_t y1_rs,
    const void* w2, const void* b2, void* y2, int64_t n2, int64_t y2_rs, int dtype,
    void* stream);
SLC_API int slc_hip_norm_linear_swiglu(const void* x, int64_t x_rs, const void* norm_weight,
                                       float epsilon, int64_t rows, int64_t hidden,
                                       int64_t features, const void* w_gate, const void* w_up,
                                       void* y, int64_t y_rs, int dtype, void* stream);
SLC_API int slc_hip_linear_residual(const void* x, int64_t x_rs, int64_t rows,
                                    int64_t in_features, int64_t out_features,
                                    const void* weight, const void* bias,
                                    const void* residual, int64_t residual_rs, void* y,
                                    int64_t y_rs, int dtype, void* stream);
SLC_API int slc_hip_rope_kv_store(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, void* query_out, void* key_buffer, void* value_buffer,
    const int64_t* positions, int* overflow, int64_t* lengths_out, int64_t advance, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t head_dim,
    int64_t capacity, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t cos_sb, int64_t cos_st,
    int64_t sin_sb, int64_t sin_st, int64_t qo_sb, int64_t qo_sh, int64_t qo_st, int* counters,
    int64_t num_counters, void* stream);

/*
 * linear_group: y_j = linear(x, w_j, b_j) for count = 1..3 matrices [n_j,
 * in_features] (the Q/K/V projections of one input) at prefill-sized rows
 * (> 64), in one launch; each output bit for bit that of slc_hip_linear
 * (kernel.triton.linear, triton_linear.py:87-148).  bf16 or fp16.  Returns
 * SLC_ERR_UNSUPPORTED (nothing launched) for rows <= 64, in_features not a
 * multiple of 64, n_j or strides not multiples of 8, or unaligned rows.
 */
SLC_API int slc_hip_linear_group(const void* input, int64_t in_stride_row, int64_t rows,
                                 int64_t in_features, int count, const void* w0,
                                 const void* b0, void* y0, int64_t n0, int64_t y0_rs,
                                 const void* w1, const void* b1, void* y1, int64_t n1,
                                 int64_t y1_rs, const void* w2, const void* b2, void* y2,
                                 int64_t n2, int64_t y2_rs, int dtype, void* stream);

/*
 * linear_swiglu: y = swiglu(round(x . w_gate^T), round(x . w_up^T)) for
 * prefill-sized rows (> 64), in one kernel: the Qwen2 MLP front after its
 * norm (qwen2.py:253-256), replacing two kernel.triton.linear calls and the
 * elementwise SwiGLU (triton_linear.py:87-148) with bit-identical results.
 * x [rows, in_features] (row stride in_stride_row), w_gate/w_up [features,
 * in_features] contiguous, y [rows, features] (row stride out_stride_row);
 * bf16 or fp16.  Returns SLC_ERR_UNSUPPORTED (nothing launched) for rows <= 64,
 * in_features not a multiple of 64, features or strides not multiples of 8,
 * or rows not 16-byte aligned.
 */
SLC_API int slc_hip_linear_swiglu(const void* input, int64_t in_stride_row, int64_t rows,
                                  int64_t in_features, int64_t features, const void* w_gate,
                                  const void* w_up, void* output, int64_t out_stride_row,
                                  int dtype, void* stream);

/*
 * rope_decode_attention: one decode token's RoPE, KV store, length advance and
 * GQA attention in one kernel.  Replaces rope_kv_store (with advance = 1)
 * followed by slc_hip_decode_attention of the rotated query over the advanced
 * state -- the reference's triton_rope, triton_kv_store, kv.advance and
 * triton_decode_attention sequence (triton_rope.py:299-390,
 * triton_kv.py:71-129, execution.py:741-767, triton_attention.py:134-210) --
 * with bit-identical results:
 *   pos = lengths[b]; key_buffer[b, pos] = rope(key[b]); value_buffer[b, pos]
 *   = value[b] (skipped, *overflow set, when pos is outside [0, capacity));
 *   out[b, h] = decode attention of rope(query[b, h]) over the tokens
 *   s < min(pos + 1, mask_len, capacity); lengths_out[b] = pos + 1 (in place
 *   allowed; *overflow set past the capacity).
 * query [B, q_heads, D], key/value [B, kv_heads, D] (one token), cosine/sine
 * [B, D] (the token's rows); buffers [B, capacity, kv_heads, D] with strides
 * as in slc_hip_decode_attention; lengths int64; the workspace is
 * slc_hip_decode_attention_workspace_size(batch, q_heads, head_dim, mask_len,
 * kv_heads, dtype, 0) bytes and the counters are
 * slc_hip_decode_attention_counter_count(batch, kv_heads) ints, owned as
 * described there (the counters also carry the length advance).  softmax_order as in slc_hip_decode_attention.
 * Returns SLC_ERR_UNSUPPORTED (nothing launched) for shapes, dtypes,
 * alignments or (exact order) mask lengths its kernel does not take.
 */
SLC_API int slc_hip_rope_decode_attention(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, void* key_buffer, void* value_buffer, const int64_t* lengths,
    int64_t* lengths_out, int* overflow, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads,
    int64_t kv_heads, int64_t head_dim, int64_t capacity, int64_t mask_len, int64_t q_stride_b,
    int64_t q_stride_h, int64_t k_stride_b, int64_t k_stride_h, int64_t v_stride_b,
    int64_t v_stride_h, int64_t cos_stride_b, int64_t sin_stride_b, int64_t kv_stride_b,
    int64_t kv_stride_s, int64_t kv_stride_h, int64_t mask_stride_b, int64_t mask_stride_s,
    int64_t out_stride_b, int64_t out_stride_h, float scale, int softmax_order, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SLC_HIP_H_ */
