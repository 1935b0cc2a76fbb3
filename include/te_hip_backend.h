/*
 * HIP (gfx950 / MI355X) backend slot for TinyEngine's attention step.
 *
 * This header takes the place of the reference GPU backend contract
 * c/src/metal_backend.h for the attention step only, with the same
 * conventions (metal_backend.h:13-347, metal_backend_layers.mm.inc:529-556,
 * :670-720):
 *   - every entry point is extern "C" and returns te_status;
 *   - NULL / zero / inconsistent arguments  -> TE_STATUS_INVALID_ARGUMENT;
 *   - a shape, cap or device the kernels do not handle -> TE_STATUS_UNSUPPORTED
 *     (callers read it as "take another path");
 *   - a failed HIP call or launch -> TE_STATUS_RUNTIME_ERROR;
 *   - a failed device allocation -> TE_STATUS_OUT_OF_MEMORY.
 *
 * Two kinds of entry points:
 *   - te_hip_* taking DEVICE pointers and a stream (`void *stream`, a
 *     hipStream_t; NULL = the null stream).  They only enqueue work and return;
 *     they are the fast path the benchmark measures.
 *   - te_hip_attention_*_mma_f32 taking HOST pointers: synchronous twins of the
 *     reference's MMA attention test entry points (metal_backend.h:104-142),
 *     serialized by the library's process-wide mutex.
 *
 * Data layout in HBM (all row-major, innermost dimension last):
 *   query/out  fp32  [seqs][layers][tokens][heads][head_dim]
 *   k, v (new) fp32  [seqs][layers][tokens][kv_heads][head_dim]
 *   q_bias     fp32  [layers][heads*head_dim]      (NULL = no bias)
 *   k/v_bias   fp32  [layers][kv_heads*head_dim]   (NULL = no bias)
 *   rope_cos/sin fp32 [context_tokens][head_dim/2] (row = absolute position)
 *   key/value_cache fp16 (IEEE binary16 bits, uint16_t)
 *                    [seqs][layers][context_tokens][kv_heads][head_dim]
 * The cache slot of (seq, layer, position, kv_head, i) is
 *   (((seq*layers + layer)*context_tokens + position)*kv_heads + kv_head)*head_dim + i,
 * i.e. the reference slot formula (layer*context_tokens + position)*kv_dim
 * (qwen.c:805, :1034) with a leading sequence index.
 */
#ifndef TE_HIP_BACKEND_H
#define TE_HIP_BACKEND_H

#include "tinyengine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest number of independent sequences one call accepts (positions are
 * passed by value to the kernels). */
#define TE_HIP_MAX_SEQS 64u

/* 1 when a gfx950 device is visible and the kernels in this library can run
 * on it, else 0.  Never aborts. */
TE_API int te_hip_available(void);

/* Writes the device name (e.g. "AMD Instinct MI355X (gfx950)") and compute-unit
 * count.  TE_STATUS_UNSUPPORTED without a usable device. */
TE_API te_status te_hip_device_info(char *name, size_t name_capacity, uint32_t *compute_units);

/*
 * RoPE cos/sin tables.  Replaces the table build of te_qwen_state_init
 * (reference qwen.c:531-539): row p, column i holds cosf/sinf of
 * (float)p * powf(theta, -(2.0f*i)/(float)head_dim), computed with the host
 * libm exactly as the reference does, then copied to the device tables
 * `cos_table` / `sin_table` ([context_tokens][head_dim/2] fp32, device).
 * Synchronous.
 */
TE_API te_status te_hip_rope_table_f32(float *cos_table, float *sin_table, size_t context_tokens,
                                       size_t head_dim, float theta);

/*
 * Bias + RoPE + fp16 KV append, for `tokens` tokens of each (seq, layer).
 * Replaces te_qkv_bias_rope_cache_batch_f32 / _h_f32
 * (metal_kernels.metal.inc:2172-2252, :2344-2429) and the CPU sequence
 * bias-add -> te_qwen_rope_cached(q), (k) -> memcpy append
 * (qwen.c:774-808, :998-1036).
 *
 * Token b of sequence s sits at position base_positions[s] + b (or
 * base_position + b when base_positions is NULL); every position must be
 * < context_tokens.  In place: q and k become bias-added and rotated, v becomes
 * bias-added.  The rotated k and the biased v are rounded to fp16 (IEEE
 * round-to-nearest-even) into the cache slot above.  When q_half is non-NULL the
 * rotated q is also written there as fp16 (layout of `query`), the operand of
 * te_hip_attention_prefill_f16.
 * head_dim must be even and <= 256.  base_positions is a HOST array of `seqs`
 * entries (seqs <= TE_HIP_MAX_SEQS).
 */
TE_API te_status te_hip_rope_kv_append_f16(
    float *q, float *k, float *v,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *q_half,
    size_t seqs, size_t layers, size_t tokens,
    const size_t *base_positions, size_t base_position,
    size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
    void *stream);

/*
 * GQA decode attention over the fp16 cache, one query token per (seq, layer).
 * Replaces te_attention_decode_f32_kernel (metal_kernels.metal.inc:2431-2500)
 * and, numerically, te_attention_decode_f32 (ops.c:323-395) fed the fp16 cache
 * upcast to fp32.  Query token of sequence s attends cache positions
 * 0..positions[s] inclusive (positions NULL -> `position` for all sequences;
 * positions is a HOST array, seqs <= TE_HIP_MAX_SEQS, every position
 * < context_tokens).
 *
 * Split-K ("flash-decoding"): the positions are cut into chunks, each chunk of
 * each (seq, layer, kv_head) is one workgroup that produces an unnormalized
 * partial (running max m, sum l, accumulator o[heads/kv_heads][head_dim]), and
 * a combine kernel merges the partials.  Softmax and all accumulation are fp32.
 * head_dim in {64, 128}; heads/kv_heads <= 16.
 *
 * workspace: device scratch of at least te_hip_attention_decode_workspace_bytes
 * bytes for the same positions, or NULL to use a buffer the library owns (grown
 * on demand, guarded by the library mutex; calls using it must all go to one
 * stream).  Calls sharing one workspace must be stream-ordered.  The chunking
 * depends on all positions, not only the longest (the chunk length balances
 * the total work over the GPU's wave slots); the workspace size depends only
 * on the largest position and never decreases with it.
 */
TE_API size_t te_hip_attention_decode_workspace_bytes(const size_t *positions, size_t position, size_t seqs,
                                                      size_t layers, size_t heads, size_t kv_heads,
                                                      size_t head_dim);

/*
 * The chunking behind the decode entry points: *chunk = cache positions per
 * split-K workgroup, *chunks = chunks of the longest sequence.  fp32_cache != 0
 * gives the chunking of te_attention_decode_f32 (seqs == layers == 1; a
 * power-of-two multiple of 512 positions, at most 4096 chunks for any
 * position).  A host computation from the sizes and the device's compute-unit
 * count (256 assumed without a device).  The workspace query above sizes for
 * an upper bound of `chunks` that never decreases with the position, so a
 * workspace sized at the largest position a caller reaches serves every
 * smaller one.  INVALID_ARGUMENT for null outputs, zero sizes or
 * seqs > TE_HIP_MAX_SEQS.
 */
TE_API te_status te_hip_attention_decode_chunking(const size_t *positions, size_t position, size_t seqs,
                                                  size_t layers, size_t kv_heads, int fp32_cache, size_t *chunk,
                                                  size_t *chunks);

TE_API te_status te_hip_attention_decode_f16(
    const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream);

/* The two stages of te_hip_attention_decode_f16 as separate launches, so a
 * caller (the benchmark) can time the split-K kernel on its own.  Same
 * arguments; the workspace must be supplied and be the same for both calls. */
TE_API te_status te_hip_attention_decode_splitk_f16(
    const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    void *workspace, size_t workspace_bytes, void *stream);
TE_API te_status te_hip_attention_decode_combine(
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t heads, size_t kv_heads, size_t head_dim,
    float *out, const void *workspace, size_t workspace_bytes, void *stream);

/*
 * Fused decode step: te_hip_rope_kv_append_f16 (tokens = 1) followed by
 * te_hip_attention_decode_f16, as one split-K launch plus the combine launch.
 * Same semantics as that pair for the cache and the output, with one
 * difference: `query`, `k_new` and `v_new` are inputs only (not rotated or
 * bias-added in place) -- the rotated q lives in registers, and the rotated k /
 * biased v go straight to the fp16 cache slot of each sequence's position.
 * The append happens inside the workgroup that owns that position, before it
 * reads it.  Layouts: query [seqs][layers][heads][head_dim], k_new / v_new
 * [seqs][layers][kv_heads][head_dim]; other arguments as above.  The
 * workspace (required, no NULL form) is sized by
 * te_hip_attention_decode_workspace_bytes.
 */
TE_API te_status te_hip_attention_decode_step_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream);

/* The split-K launch of te_hip_attention_decode_step_f16 alone (append +
 * partials into the workspace), for timing; te_hip_attention_decode_combine with
 * the same workspace completes the step.  Repeating it is idempotent: the
 * appended slot is rewritten with the same values. */
TE_API te_status te_hip_attention_decode_step_splitk_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    void *workspace, size_t workspace_bytes, void *stream);

/*
 * No counterpart in the reference: the fused decode step for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc).  Same arguments and results as
 * te_hip_attention_decode_step_f16 without the workspace: the split-K partials
 * go to a device array inside the library, TE_HIP_DECODE_NOALLOC_SCRATCH_BYTES
 * (16 MiB) per GPU, held from first use until the process ends.  The call
 * allocates nothing.  A call whose partials
 * (seqs*layers*heads*chunks*(head_dim+2)*4 bytes, chunks as reported by
 * te_hip_attention_decode_chunking) exceed the array returns
 * TE_STATUS_UNSUPPORTED before any work is queued.  Every call on one GPU
 * shares the array: calls that overlap in time on one GPU (different streams,
 * different threads) race and must be ordered by the caller.
 */
#define TE_HIP_DECODE_NOALLOC_SCRATCH_BYTES (16u << 20)
TE_API te_status te_hip_attention_decode_step_noalloc_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *stream);

/*
 * Batched-prefill causal attention over the fp16 cache.  Replaces the CPU
 * per-token loop (qwen.c:810-824: row t = decode at position t) and the MMA
 * prefill kernel te_attention_flash_mma_t_f32_kernel
 * (metal_kernels.metal.inc:2693-2836), whose mask
 * `past <= base_position + row` defines chunked prefill.  Row t of (seq, layer)
 * attends cache positions 0..base_position+t inclusive; the cache must already
 * hold those positions (te_hip_rope_kv_append_f16 writes them).
 *
 * The kernel reads the K cache and a transposed copy of the V cache, V^T:
 *   value_t fp16 [seqs][layers][kv_heads][head_dim][ctx_pad],
 *   ctx_pad = context_tokens rounded up to a multiple of 64,
 * element (s, l, h, i, p) = value_cache (s, l, p, h, i) -- one row of positions
 * per (kv head, dim), the layout the PV product reads with 16-byte loads
 * (as the reference's Metal path keeps transposed copies,
 * te_qkv_bias_rope_cache_batch_t_f32, metal_kernels.metal.inc:2254-2342).
 * The *_vt entry points take V^T from the caller (te_hip_value_transpose_f16 or
 * te_hip_attention_prefill_step_vt_f16 keep it current); the others build it
 * for positions 0 .. base_position+tokens on every call.  V^T positions from
 * base_position+tokens up to the next multiple of 8 must be finite (the V^T
 * writers set them to 0): the kernel loads 8 positions at a time and weights
 * the ones past a row's position by exactly 0.
 *
 * q_half: fp16 rotated queries [seqs][layers][tokens][heads][head_dim];
 * out: fp32, same layout.  QK^T and PV run on fp16 MFMA with fp32 accumulation;
 * softmax is fp32.  head_dim in {64, 128}; heads % kv_heads == 0;
 * base_position + tokens <= context_tokens.
 */

/* Bytes of a V^T buffer (0 for zero sizes). */
TE_API size_t te_hip_value_t_bytes(size_t seqs, size_t layers, size_t context_tokens, size_t kv_heads,
                                   size_t head_dim);

/* V^T of positions [first_position, first_position + count) of every
 * (seq, layer, kv head), and 0 at the positions after them up to the next
 * multiple of 8.  Other positions are not written.  Bit-exact copy. */
TE_API te_status te_hip_value_transpose_f16(const uint16_t *value_cache, uint16_t *value_cache_t, size_t seqs,
                                            size_t layers, size_t first_position, size_t count,
                                            size_t context_tokens, size_t kv_heads, size_t head_dim,
                                            void *stream);

/*
 * Prefill attention over the K cache and V^T.  With a workspace of at least
 * te_hip_attention_prefill_vt_workspace_bytes bytes (the same shape), a launch
 * whose tile pairs alone would leave compute units idle (short prompts, few
 * heads, a chunk after a long cache) splits each (tile pair, head) over S key
 * ranges: every split writes unnormalised partial rows to the workspace, and a
 * second launch merges them into `out`.  S comes from the shape and the
 * device's compute-unit count; the query returns S*seqs*layers*tokens*heads*
 * (head_dim+2)*4 bytes, or 0 when S == 1.  workspace NULL runs one split.
 * INVALID_ARGUMENT when a given workspace is too small.
 */
TE_API size_t te_hip_attention_prefill_vt_workspace_bytes(size_t seqs, size_t layers, size_t tokens,
                                                          size_t base_position, size_t context_tokens, size_t heads,
                                                          size_t kv_heads, size_t head_dim);
TE_API te_status te_hip_attention_prefill_vt_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache_t,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Fused prefill step keeping V^T: bias + RoPE + fp16 append of the chunk's
 * k / v into key_cache and value_cache (te_hip_rope_kv_append_f16's slots and
 * bits), the chunk's V^T positions into value_cache_t, then the causal
 * attention, whose prologue applies bias + RoPE to each query row in registers
 * and rounds it to the fp16 operand (the bits te_hip_rope_kv_append_f16 writes
 * to q_half).  `query`, `k_new` and `v_new` are inputs only.  Layouts: query
 * [seqs][layers][tokens][heads][head_dim], k_new / v_new
 * [seqs][layers][tokens][kv_heads][head_dim], out like query.  Every sequence
 * starts at base_position; value_cache_t must hold V^T of positions
 * 0 .. base_position-1.  workspace as te_hip_attention_prefill_vt_f16.  Four
 * launches: append, V^T, attention, and the merge when the launch splits.
 */
TE_API te_status te_hip_attention_prefill_step_vt_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *value_cache_t,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Prefill over the plain caches: V^T of positions 0 .. base_position+tokens-1
 * goes to a buffer the library owns (grown on demand under the library mutex;
 * calls must share one stream), then the attention runs as one split.
 */
TE_API te_status te_hip_attention_prefill_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *stream);

/*
 * Key-split prefill over the plain caches: the workspace holds the key-split
 * partials (when the launch splits, as te_hip_attention_prefill_vt_f16) followed
 * by V^T of the cache; te_hip_attention_prefill_workspace_bytes returns both
 * (0 only for invalid arguments).  INVALID_ARGUMENT when the workspace is
 * missing or too small.
 */
TE_API size_t te_hip_attention_prefill_workspace_bytes(size_t seqs, size_t layers, size_t tokens,
                                                       size_t base_position, size_t context_tokens, size_t heads,
                                                       size_t kv_heads, size_t head_dim);
TE_API te_status te_hip_attention_prefill_split_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Fused prefill step over the plain caches: te_hip_attention_prefill_step_vt_f16
 * with V^T of positions 0 .. base_position+tokens-1 built in the library-owned
 * buffer (as te_hip_attention_prefill_f16) and one split.
 */
TE_API te_status te_hip_attention_prefill_step_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *stream);

/*
 * Host-pointer twins of the reference MMA attention entry points
 * (metal_backend.h:104-142, metal_backend.mm:30-373), same signatures and the
 * same shape guards (q_rows == 8, head_dim == 64; k_cols == 8 for qk/tile,
 * k_cols % 8 == 0 for stream/causal, q_base <= k_cols for causal).
 * key_t is [head_dim][k_cols], value is [k_cols][head_dim], all fp32.  They run
 * fp32 MFMA (v_mfma_f32_16x16x4_f32) on the GPU.
 *   qk:     out[q][k]  = sum_d query[q][d]*key_t[d][k]
 *   tile:   out[q][:]  = softmax_k(scale*scores) @ value, k_cols == 8
 *   stream: same, k_cols any multiple of 8
 *   causal: same, keys k > q_base + q masked
 */
TE_API te_status te_hip_attention_qk_mma_f32(const float *query, const float *key_t, size_t q_rows,
                                             size_t k_cols, size_t head_dim, float *out);
TE_API te_status te_hip_attention_tile_mma_f32(const float *query, const float *key_t, const float *value,
                                               size_t q_rows, size_t k_cols, size_t head_dim, float *out);
TE_API te_status te_hip_attention_stream_mma_f32(const float *query, const float *key_t, const float *value,
                                                 size_t q_rows, size_t k_cols, size_t head_dim, float *out);
TE_API te_status te_hip_attention_causal_mma_f32(const float *query, const float *key_t, const float *value,
                                                 size_t q_rows, size_t k_cols, size_t head_dim, size_t q_base,
                                                 float *out);

/*
 * Decode-layer vector operations around attention (device pointers, async on
 * `stream`).  te_hip_matvec_f32 replaces te_metal_matvec_f32
 * (metal_backend.h:13-22) for weights already in HBM: `weights` points at the
 * tensor data (the GGUF mapping + tensor offset of the reference, uploaded),
 * out[r] = sum_c W[r][c] * input[c] for a [rows][cols] tensor of GGUF type
 * ggml_type: 0 = F32 (cols % 4 == 0), 2 = Q4_0 and 8 = Q8_0 (cols % 32 == 0;
 * rows of cols/32 blocks of 18 / 34 bytes, ops.c:15-21); other types ->
 * UNSUPPORTED; `weights` must be 4-byte aligned (16 for F32) and `input`
 * 16-byte aligned, else UNSUPPORTED (16-byte aligned quantized weights take
 * the fastest kernel).  F32 results equal the reference's te_model_matvec_f32
 * within fp32 rounding of the row's terms (the summation order differs).  For
 * Q4_0 / Q8_0 rows with an even block count, each 32-value block of `input`
 * is rounded to 22-bit integers relative to its largest magnitude and the
 * products are summed exactly: error <= 2^-22 max|block| per value plus fp32
 * rounding of the block sums; a NaN or inf input value gives NaN rows.
 * The others are the reference ops.c functions (te_rmsnorm_f32 :272-293,
 * te_swiglu_f32 :397-406, te_add_f32 :408-416, te_argmax_f32 :418-433) on
 * device arrays, with the same argument checks; te_hip_rmsnorm_f32 normalises
 * `rows` rows of `len` each; te_hip_argmax_f32 writes the index to DEVICE
 * memory.  The argmax is exact (first maximum, NaN never taken); add is exact;
 * RMSNorm sums squares in fp64 like the reference; SwiGLU uses the device expf.
 */
TE_API te_status te_hip_matvec_f32(const void *weights, uint32_t ggml_type, const float *input, size_t cols,
                                   size_t rows, float *out, void *stream);
TE_API te_status te_hip_rmsnorm_f32(const float *input, const float *weight, size_t rows, size_t len,
                                    float epsilon, float *out, void *stream);
TE_API te_status te_hip_swiglu_f32(const float *gate, const float *up, size_t len, float *out, void *stream);
TE_API te_status te_hip_add_f32(const float *lhs, const float *rhs, size_t len, float *out, void *stream);
TE_API te_status te_hip_argmax_f32(const float *values, size_t len, uint32_t *out_index, void *stream);

/*
 * Top-k temperature sampling of the next token from device logits: the
 * reference sampler (c/src/qwen.c:1182-1250; candidate scan :1198-1225,
 * xorshift64* :1170-1178), which te_qwen_generate_text runs on host logits.
 * It has no Metal counterpart: the reference copies the logits back.  Here
 * the device keeps the logits that can enter the candidate list (above a
 * lower bound of the k-th largest logit before them) and the host runs the
 * reference's scan and draw over those, so the token and the next *rng_state
 * equal the reference's for the same logits (any NaN logit: the host scans
 * them all).  top_k 0 means 1; k is capped at 1024 and at vocab.  Blocks the
 * caller (the read-back is synchronous).  workspace: device memory of
 * te_hip_sample_workspace_bytes(vocab) bytes.
 */
TE_API size_t te_hip_sample_workspace_bytes(size_t vocab);
TE_API te_status te_hip_sample_top_k_f32(const float *logits, size_t vocab, uint32_t top_k, float temperature,
                                         uint64_t *rng_state, uint32_t *out_token, void *workspace,
                                         size_t workspace_bytes, void *stream);

/*
 * Quantized GEMM of batched prompt prefill: out[m][n] = sum_k pre(x)[m][k] *
 * W[n][k] (+ resid[m][n]) for `rows` activation rows at once -- the per-row
 * meaning of te_model_matvec_f32 (ops.c:177-269) for the projections of
 * te_qwen_prefill_prompt_batch (qwen.c:630-905), whose Metal matmuls it
 * replaces.  pre: 0 none, 1 RMSNorm (norm_w, epsilon, as te_rmsnorm_f32),
 * 2 SwiGLU (x is gate, x2 is up, as te_swiglu_f32).  W is a GGUF Q4_0 (2) or
 * Q8_0 (8) tensor [n][k] in device memory at a 2-byte aligned address,
 * k % 32 == 0.  The activations are rounded per 32-value block to 15 bits of
 * the block's largest magnitude (error <= 2^-14 of it per value); products
 * are exact int8 MFMA sums, accumulated per block in fp32.  `act` is device
 * scratch of te_hip_gemm_act_bytes(rows, k) bytes.  `partials` (may be NULL)
 * is device scratch of partial_bytes bytes: with it, an output grid too small
 * to fill the GPU splits K into up to partial_bytes / (rows * n * 4) parts,
 * summed afterwards in a fixed order.  Device pointers, asynchronous on
 * `stream`; UNSUPPORTED for other types or shapes.
 */
TE_API size_t te_hip_gemm_act_bytes(size_t rows, size_t k);
TE_API te_status te_hip_gemm_q_f32(const void *weights, uint32_t ggml_type, const float *x, const float *x2,
                                   const float *norm_w, float epsilon, int pre, size_t rows, size_t n, size_t k,
                                   float *out, const float *resid, void *act, float *partials,
                                   size_t partial_bytes, void *stream);

/*
 * One decode token through every layer (and, with out_token_id, the final
 * norm, lm_head and argmax): replaces te_metal_decode_all_layers_f32
 * (metal_backend.h:239-276, called by te_qwen_decode_all_layers_exact,
 * qwen.c:1464-1640), with the same arguments and per-layer order as the CPU
 * loop of te_qwen_forward_token (qwen.c:907-1087).  Differences from the Metal
 * slot, all device-resident:
 *   - `mapping` is the model file's bytes (or its tensor data) in HBM,
 *     mapping_len bytes; the *_offsets arrays (host, `layers` entries each) and
 *     head_offset are byte offsets into it, as the reference's absolute tensor
 *     offsets.  Weights are [rows][cols] GGUF tensors of ggml_type (F32, Q4_0
 *     or Q8_0; the head may have its own type); 16-byte aligned quantized
 *     tensors take the fused kernels, 4-byte aligned ones a slower path.
 *   - key_cache / value_cache are the HIP path's fp16 caches [layers]
 *     [context_tokens][kv]; the new token's k / v are appended at `position`.
 *   - rope_cos / rope_sin are the full tables [context_tokens][head_dim / 2]
 *     (te_hip_rope_table_f32), not the position's row.
 *   - hidden_in / out are device [hidden] (out may equal hidden_in: the
 *     reference passes hidden_buf for both); out_token_id is a device uint32.
 *   - workspace: device scratch of te_hip_decode_all_layers_workspace_bytes
 *     (same position, sizes, and vocab or 0 without a head), 256-byte aligned.
 * Asynchronous on `stream`; per layer six launches (RMSNorm + QKV, the fused
 * decode step's two, Wo + residual, RMSNorm + gate/up, SwiGLU + down +
 * residual).  Checks: null pointers, layers == 0, position >=
 * context_tokens, epsilon <= 0, a tensor past mapping_len, a short workspace ->
 * INVALID_ARGUMENT; hidden != heads * head_dim, kv != kv_heads * head_dim,
 * head_dim not 64 / 128, other GGUF types, misaligned tensors or vectors ->
 * UNSUPPORTED.  Numerics: each projection as te_hip_matvec_f32, RMSNorm as
 * te_hip_rmsnorm_f32, SwiGLU as te_hip_swiglu_f32, attention as
 * te_hip_attention_decode_step_f16.
 */
TE_API size_t te_hip_decode_all_layers_workspace_bytes(size_t position, size_t hidden, size_t kv, size_t heads,
                                                       size_t kv_heads, size_t head_dim, size_t ffn, size_t vocab);
TE_API te_status te_hip_decode_all_layers_f16(
    const void *mapping, size_t mapping_len,
    const uint64_t *q_offsets, const uint64_t *k_offsets, const uint64_t *v_offsets,
    const uint64_t *output_offsets, const uint64_t *gate_offsets, const uint64_t *up_offsets,
    const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights,
    const float *q_biases, const float *k_biases, const float *v_biases,
    const float *rope_cos, const float *rope_sin, uint16_t *key_cache, uint16_t *value_cache,
    size_t position, size_t context_tokens, size_t hidden, size_t kv, size_t heads, size_t kv_heads,
    size_t head_dim, size_t ffn, float epsilon, float *out,
    uint64_t head_offset, uint32_t head_ggml_type, const float *output_norm_weight, size_t vocab,
    uint32_t *out_token_id, void *workspace, size_t workspace_bytes, void *stream);

/*
 * One decode token through one layer: te_hip_decode_all_layers_f16 with
 * layers == 1 and the layer's offsets, norms, biases and cache slice passed
 * directly -- the twin of te_metal_decode_layer_f32 (metal_backend.h:206-237,
 * called per layer by qwen.c:1392-1462), without the head.  The workspace is
 * sized by te_hip_decode_all_layers_workspace_bytes(position, ..., vocab 0).
 */
TE_API te_status te_hip_decode_layer_f16(
    const void *mapping, size_t mapping_len,
    uint64_t q_offset, uint64_t k_offset, uint64_t v_offset, uint64_t output_offset,
    uint64_t gate_offset, uint64_t up_offset, uint64_t down_offset, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weight, const float *ffn_norm_weight,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin, uint16_t *key_cache, uint16_t *value_cache,
    size_t position, size_t context_tokens, size_t hidden, size_t kv, size_t heads, size_t kv_heads,
    size_t head_dim, size_t ffn, float epsilon, float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * A chunk of `batch` prompt tokens at positions base_position .. base_position
 * + batch - 1 through every layer: replaces te_metal_prefill_all_layers_f32
 * (metal_backend.h:311-343, called by te_qwen_prefill_all_layers_exact,
 * qwen.c:1640-1797), with the same arguments and per-layer order, and the
 * result of the per-token CPU loop for each row (qwen.c:774-824: row t is
 * decode at position base_position + t).  Differences from the Metal slot,
 * all device-resident:
 *   - hidden_in / out are [batch][hidden] (out may equal hidden_in); out gets
 *     every row's final hidden state;
 *   - key_cache / value_cache are the fp16 caches [layers][context_tokens][kv],
 *     and value_cache_t their transposed value copy [layers][kv_heads]
 *     [head_dim][ctx_pad] (te_hip_value_t_bytes(1, layers, ...)), which must
 *     hold positions 0 .. base_position - 1 (te_hip_value_transpose_f16 builds
 *     it from value_cache); the chunk's k / v go to all three;
 *   - base_position (the reference always starts at 0) allows chunked
 *     prefill after a cached prefix;
 *   - mapping, offsets, rope tables as te_hip_decode_all_layers_f16;
 *   - workspace: te_hip_prefill_all_layers_workspace_bytes(batch, hidden, kv,
 *     ffn) bytes, 256-byte aligned.
 * The projections are the batched-prefill GEMM (te_hip_gemm_q_f32: each
 * activation row rounded per 32-value block to 15 bits of its largest
 * magnitude, exact int8 MFMA products); the attention is
 * te_hip_attention_prefill_step_vt_f16.  Asynchronous on `stream`.  Checks as
 * te_hip_decode_all_layers_f16; Q4_0 / Q8_0 layer weights at 2-byte aligned
 * addresses only (other types or alignments -> UNSUPPORTED, the reference's
 * cue to take the per-token path); batch <= 65535.
 */
TE_API size_t te_hip_prefill_all_layers_workspace_bytes(size_t batch, size_t hidden, size_t kv, size_t ffn);
TE_API te_status te_hip_prefill_all_layers_f16(
    const void *mapping, size_t mapping_len,
    const uint64_t *q_offsets, const uint64_t *k_offsets, const uint64_t *v_offsets,
    const uint64_t *output_offsets, const uint64_t *gate_offsets, const uint64_t *up_offsets,
    const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights,
    const float *q_biases, const float *k_biases, const float *v_biases,
    const float *rope_cos, const float *rope_sin, uint16_t *key_cache, uint16_t *value_cache,
    uint16_t *value_cache_t, size_t base_position, size_t batch, size_t context_tokens, size_t hidden, size_t kv,
    size_t heads, size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out,
    void *workspace, size_t workspace_bytes, void *stream);

/* One layer of the chunk: te_hip_prefill_all_layers_f16 with layers == 1 and
 * the layer's arguments passed directly -- the twin of
 * te_metal_prefill_layer_f32 (metal_backend.h:278-309, called per layer by
 * qwen.c:1799-1870). */
TE_API te_status te_hip_prefill_layer_f16(
    const void *mapping, size_t mapping_len,
    uint64_t q_offset, uint64_t k_offset, uint64_t v_offset, uint64_t output_offset,
    uint64_t gate_offset, uint64_t up_offset, uint64_t down_offset, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weight, const float *ffn_norm_weight,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin, uint16_t *key_cache, uint16_t *value_cache,
    uint16_t *value_cache_t, size_t base_position, size_t batch, size_t context_tokens, size_t hidden, size_t kv,
    size_t heads, size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out,
    void *workspace, size_t workspace_bytes, void *stream);

/*
 * Measurement only, no counterpart in the reference: `blocks` workgroups of 8
 * waves each run `iters` rounds of 8 independent fp16 16x16x32 MFMAs on
 * register operands (blocks*8*iters*8*16384 FLOP), so a benchmark can report
 * the MFMA rate the device sustains next to the data-sheet peak.  `out` holds
 * blocks*512 floats.  blocks in [1, 65535], iters in [1, 2^20].  Asynchronous.
 */
TE_API te_status te_hip_calibrate_mfma_f16(size_t blocks, size_t iters, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TE_HIP_BACKEND_H */
