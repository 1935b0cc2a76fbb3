/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference TinyEngine
 * attention step, used as the parity checker for the HIP path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (libtinyengine.so) never links or calls it.
 *
 * Every function cites the reference source it restates.  Loop order and
 * floating-point operation order follow the reference so that, compiled like
 * the reference (-std=c11 -O3, no FP contraction), results are bit-identical
 * to the reference C functions on the same host libm.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   orc_f16_to_f32        exhaustive 65536-pattern check against numpy float16
 *   orc_f32_to_f16_rne    exhaustive f16->f32->f16 round trip, tie/overflow/
 *                         subnormal cases, 2^24 random floats vs numpy
 *   orc_rope_f32          reference KAT (kernel_ops.c:330-339), compiled
 *                         reference ops.c (oracle/_ref), golden fixtures,
 *                         closed forms (position 0 identity, pair norms)
 *   orc_rope_table        row p == orc_rope_f32 applied to unit vectors, and
 *                         golden rows from the compiled reference te_rope_f32
 *   orc_rope_cached       equals orc_rope_f32 with table rows (bit-exact)
 *   orc_attention_decode_f32  reference KAT (kernel_ops.c:341-356), compiled
 *                         reference ops.c, golden fixtures, fp64 brute force,
 *                         invariants (one key -> V[0], constant V -> V)
 *   orc_rope_kv_append_f16  slot formula by position-tagged values; rotation
 *                         bit-exact vs orc_rope_cached
 *   orc_attention_decode_f16kv / orc_attention_prefill  compositions of the
 *                         pinned functions above (row t == decode at base+t)
 *   orc_rmsnorm_f32, orc_swiglu_f32, orc_add_f32, orc_argmax_f32
 *                         compiled reference ops.c (bit-exact), closed forms
 *   orc_dequantize_row_f32  closed forms: every 4-bit / 8-bit code times the
 *                         block scale, exhaustively per code
 *   orc_matvec_f32        fp64 brute force over the dequantized rows, and
 *                         equality with dequantize + te_f32 dot for F32
 */
#ifndef TE_ORACLE_H
#define TE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status values mirror te_status (reference tinyengine.h:28-35). */
#define ORC_OK 0
#define ORC_INVALID_ARGUMENT 1
#define ORC_UNSUPPORTED 3
#define ORC_OUT_OF_MEMORY 4

float orc_f16_to_f32(uint16_t bits);
uint16_t orc_f32_to_f16_rne(float value);
void orc_f16_to_f32_array(const uint16_t *in, float *out, size_t n);
void orc_f32_to_f16_array(const float *in, uint16_t *out, size_t n);

int orc_rope_f32(float *values, size_t heads, size_t head_dim, size_t position, float theta);
int orc_rope_table(float *cos_table, float *sin_table, size_t context_tokens, size_t head_dim, float theta);
int orc_rope_cached(float *values, size_t heads, size_t head_dim, const float *cos_table,
                    const float *sin_table, size_t position);
int orc_attention_decode_f32(const float *query, const float *key_cache, const float *value_cache,
                             size_t position, size_t heads, size_t kv_heads, size_t head_dim, float *out);

int orc_rope_kv_append_f16(float *q, float *k, float *v, const float *q_bias, const float *k_bias,
                           const float *v_bias, const float *cos_table, const float *sin_table,
                           uint16_t *key_cache, uint16_t *value_cache, size_t seqs, size_t layers,
                           size_t tokens, const size_t *base_positions, size_t base_position,
                           size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim);

int orc_attention_decode_f16kv(const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
                               const size_t *positions, size_t position, size_t seqs, size_t layers,
                               size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
                               float *out);

int orc_attention_prefill(const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
                          size_t tokens, size_t base_position, size_t context_tokens, size_t heads,
                          size_t kv_heads, size_t head_dim, size_t row_begin, size_t row_end,
                          size_t row_step, float *out);

/* Decode-layer vector operations (reference c/src/ops.c:272-433). */
int orc_rmsnorm_f32(const float *input, const float *weight, size_t len, float epsilon, float *out);
int orc_swiglu_f32(const float *gate, const float *up, size_t len, float *out);
int orc_add_f32(const float *lhs, const float *rhs, size_t len, float *out);
int orc_argmax_f32(const float *values, size_t len, uint32_t *out_index);

/* GGUF tensor types of the reference matvec (ops.c:15-21): F32 = 0, Q4_0 = 2
 * (18-byte blocks of 32: f16 scale + 16 bytes of 4-bit codes, low nibbles are
 * elements 0-15, high nibbles 16-31, value (code - 8) * scale), Q8_0 = 8
 * (34-byte blocks: f16 scale + 32 int8 codes).  Rows are `cols` elements,
 * stored back to back. */
#define ORC_GGML_F32 0u
#define ORC_GGML_Q4_0 2u
#define ORC_GGML_Q8_0 8u
size_t orc_ggml_row_bytes(uint32_t ggml_type, size_t cols);
int orc_dequantize_row_f32(const uint8_t *data, uint32_t ggml_type, size_t cols, size_t row, float *out);
int orc_matvec_f32(const uint8_t *data, uint32_t ggml_type, const float *input, size_t cols, size_t rows,
                   float *out);

#ifdef __cplusplus
}
#endif

#endif
