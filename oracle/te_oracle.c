/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference attention step
 * (parity checker; never linked into libtinyengine.so).  See te_oracle.h for
 * what pins each function.  Compiled with -std=c11 -O3 like the reference
 * (reference c/Makefile:17), which keeps FP contraction off.
 */
#include "te_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_STACK_SCORES 1024u

/* Exact binary16 -> binary32, including subnormals, inf and NaN.
 * Restates te_f16_to_f32 (reference c/src/ops.c:435-462). */
float orc_f16_to_f32(uint16_t bits) {
    const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)bits >> 10) & 0x1fu;
    uint32_t man = (uint32_t)bits & 0x3ffu;
    uint32_t word;
    if (exp == 0u) {
        if (man == 0u) {
            word = sign;
        } else {
            /* subnormal: normalise the mantissa */
            int32_t e = -14;
            while ((man & 0x400u) == 0u) {
                man <<= 1;
                e -= 1;
            }
            man &= 0x3ffu;
            word = sign | ((uint32_t)(e + 127) << 23) | (man << 13);
        }
    } else if (exp == 31u) {
        word = sign | 0x7f800000u | (man << 13);
    } else {
        word = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &word, sizeof(out));
    return out;
}

/* binary32 -> binary16, IEEE 754 round-to-nearest-even, overflow to inf,
 * gradual underflow to subnormals, NaN stays NaN (quiet, sign kept).  The
 * reference has no CPU f32->f16; its GPU path uses Metal half()
 * (metal_kernels.metal.inc:2418-2427), which is IEEE RNE. */
uint16_t orc_f32_to_f16_rne(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof(x));
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t abs = x & 0x7fffffffu;
    if (abs >= 0x7f800000u) {
        if (abs > 0x7f800000u) {
            return (uint16_t)(sign | 0x7e00u | ((abs >> 13) & 0x3ffu));
        }
        return (uint16_t)(sign | 0x7c00u);
    }
    if (abs >= 0x477ff000u) {
        /* >= 65520 rounds to inf (65504 + half an ulp) */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (abs < 0x38800000u) {
        /* result is subnormal or zero: value = man * 2^-24 after rounding */
        if (abs < 0x33000000u) {
            /* < 2^-25: rounds to zero (2^-25 exactly is a tie -> even -> 0) */
            return sign;
        }
        const uint32_t e = abs >> 23;               /* biased exponent, 102..112 */
        const uint32_t m = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;            /* so that result = m >> shift */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) {
            h += 1u;
        }
        return (uint16_t)(sign | h);
    }
    /* normal range */
    uint32_t h = ((abs >> 13) - (112u << 10));
    const uint32_t rem = abs & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h += 1u; /* may carry into the exponent, which is still correct */
    }
    return (uint16_t)(sign | h);
}

void orc_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = orc_f16_to_f32(in[i]);
    }
}

void orc_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = orc_f32_to_f16_rne(in[i]);
    }
}

/* Half-split RoPE with libm powf/sinf/cosf per element pair.
 * Restates te_rope_f32 (reference c/src/ops.c:295-321). */
int orc_rope_f32(float *values, size_t heads, size_t head_dim, size_t position, float theta) {
    if (values == NULL || heads == 0u || head_dim == 0u || (head_dim % 2u) != 0u || theta <= 0.0f) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t half = head_dim / 2u;
    for (size_t h = 0; h < heads; ++h) {
        float *row = values + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            const float freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
            const float angle = (float)position * freq;
            const float s = sinf(angle);
            const float c = cosf(angle);
            const float a = row[i];
            const float b = row[i + half];
            row[i] = a * c - b * s;
            row[i + half] = b * c + a * s;
        }
    }
    return ORC_OK;
}

/* cos/sin tables [context_tokens][head_dim/2], same formula as orc_rope_f32.
 * Restates the table build in te_qwen_state_init (reference qwen.c:531-539). */
int orc_rope_table(float *cos_table, float *sin_table, size_t context_tokens, size_t head_dim, float theta) {
    if (cos_table == NULL || sin_table == NULL || head_dim == 0u || (head_dim % 2u) != 0u || theta <= 0.0f) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t half = head_dim / 2u;
    for (size_t p = 0; p < context_tokens; ++p) {
        for (size_t i = 0; i < half; ++i) {
            const float freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
            const float angle = (float)p * freq;
            cos_table[p * half + i] = cosf(angle);
            sin_table[p * half + i] = sinf(angle);
        }
    }
    return ORC_OK;
}

/* RoPE from precomputed table row `position`.
 * Restates te_qwen_rope_cached (reference qwen.c:2133-2160). */
int orc_rope_cached(float *values, size_t heads, size_t head_dim, const float *cos_table,
                    const float *sin_table, size_t position) {
    if (values == NULL || cos_table == NULL || sin_table == NULL || heads == 0u || head_dim == 0u ||
        (head_dim % 2u) != 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t half = head_dim / 2u;
    const float *crow = cos_table + position * half;
    const float *srow = sin_table + position * half;
    for (size_t h = 0; h < heads; ++h) {
        float *row = values + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            const float a = row[i];
            const float b = row[i + half];
            const float c = crow[i];
            const float s = srow[i];
            row[i] = a * c - b * s;
            row[i + half] = b * c + a * s;
        }
    }
    return ORC_OK;
}

/* Single-query GQA attention over positions 0..position inclusive with a
 * two-pass softmax (max, exp-sum, divide) and dim-outer PV loop.
 * Restates te_attention_decode_f32 (reference c/src/ops.c:323-395). */
int orc_attention_decode_f32(const float *query, const float *key_cache, const float *value_cache,
                             size_t position, size_t heads, size_t kv_heads, size_t head_dim, float *out) {
    if (query == NULL || key_cache == NULL || value_cache == NULL || out == NULL || heads == 0u ||
        kv_heads == 0u || head_dim == 0u || (heads % kv_heads) != 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    if (position == SIZE_MAX) {
        return ORC_UNSUPPORTED;
    }
    const size_t group = heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t n = position + 1u;
    float stack_scores[ORC_STACK_SCORES];
    float *scores = n <= ORC_STACK_SCORES ? stack_scores : (float *)malloc(n * sizeof(float));
    if (scores == NULL) {
        return ORC_OUT_OF_MEMORY;
    }
    for (size_t h = 0; h < heads; ++h) {
        const size_t kvh = h / group;
        const float *q = query + h * head_dim;
        for (size_t p = 0; p < n; ++p) {
            const float *krow = key_cache + (p * kv_heads + kvh) * head_dim;
            float acc = 0.0f;
            for (size_t i = 0; i < head_dim; ++i) {
                acc += q[i] * krow[i];
            }
            scores[p] = acc * scale;
        }
        float mx = -FLT_MAX;
        for (size_t p = 0; p < n; ++p) {
            if (scores[p] > mx) {
                mx = scores[p];
            }
        }
        float sum = 0.0f;
        for (size_t p = 0; p < n; ++p) {
            scores[p] = expf(scores[p] - mx);
            sum += scores[p];
        }
        if (sum > 0.0f) {
            for (size_t p = 0; p < n; ++p) {
                scores[p] /= sum;
            }
        }
        float *o = out + h * head_dim;
        for (size_t i = 0; i < head_dim; ++i) {
            float acc = 0.0f;
            for (size_t p = 0; p < n; ++p) {
                acc += scores[p] * value_cache[(p * kv_heads + kvh) * head_dim + i];
            }
            o[i] = acc;
        }
    }
    if (scores != stack_scores) {
        free(scores);
    }
    return ORC_OK;
}

/* Bias add, RoPE of q and k from table rows, fp16 append of k and v, for
 * `tokens` tokens per (seq, layer) at positions base + b.  Restates the CPU
 * per-token sequence of reference qwen.c:774-808 (prefill) / :998-1036 (decode)
 * with the position rule of te_qkv_bias_rope_cache_batch_f32
 * (metal_kernels.metal.inc:2206) and the fp16 copy of
 * te_qkv_bias_rope_cache_batch_h_f32 (:2418-2427).  Layouts as in
 * include/te_hip_backend.h. */
int orc_rope_kv_append_f16(float *q, float *k, float *v, const float *q_bias, const float *k_bias,
                           const float *v_bias, const float *cos_table, const float *sin_table,
                           uint16_t *key_cache, uint16_t *value_cache, size_t seqs, size_t layers,
                           size_t tokens, const size_t *base_positions, size_t base_position,
                           size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim) {
    if (q == NULL || k == NULL || v == NULL || cos_table == NULL || sin_table == NULL ||
        key_cache == NULL || value_cache == NULL || seqs == 0u || layers == 0u || tokens == 0u ||
        heads == 0u || kv_heads == 0u || head_dim == 0u || (head_dim % 2u) != 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t hidden = heads * head_dim;
    const size_t kv_dim = kv_heads * head_dim;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t base = base_positions != NULL ? base_positions[s] : base_position;
        if (base + tokens > context_tokens) {
            return ORC_INVALID_ARGUMENT;
        }
        for (size_t layer = 0; layer < layers; ++layer) {
            const size_t sl = s * layers + layer;
            for (size_t b = 0; b < tokens; ++b) {
                const size_t pos = base + b;
                float *tq = q + (sl * tokens + b) * hidden;
                float *tk = k + (sl * tokens + b) * kv_dim;
                float *tv = v + (sl * tokens + b) * kv_dim;
                if (q_bias != NULL) {
                    for (size_t i = 0; i < hidden; ++i) {
                        tq[i] += q_bias[layer * hidden + i];
                    }
                }
                for (size_t i = 0; i < kv_dim; ++i) {
                    if (k_bias != NULL) {
                        tk[i] += k_bias[layer * kv_dim + i];
                    }
                    if (v_bias != NULL) {
                        tv[i] += v_bias[layer * kv_dim + i];
                    }
                }
                orc_rope_cached(tq, heads, head_dim, cos_table, sin_table, pos);
                orc_rope_cached(tk, kv_heads, head_dim, cos_table, sin_table, pos);
                const size_t slot = (sl * context_tokens + pos) * kv_dim;
                orc_f32_to_f16_array(tk, key_cache + slot, kv_dim);
                orc_f32_to_f16_array(tv, value_cache + slot, kv_dim);
            }
        }
    }
    return ORC_OK;
}

/* Decode attention for every (seq, layer) over the fp16 cache, upcast exactly
 * to fp32, then orc_attention_decode_f32 -- the reference decode call site
 * (qwen.c:1037-1049) on the fp16-rounded cache. */
int orc_attention_decode_f16kv(const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
                               const size_t *positions, size_t position, size_t seqs, size_t layers,
                               size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
                               float *out) {
    if (query == NULL || key_cache == NULL || value_cache == NULL || out == NULL || seqs == 0u ||
        layers == 0u || heads == 0u || kv_heads == 0u || head_dim == 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t kv_dim = kv_heads * head_dim;
    size_t max_n = 0;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t pos = positions != NULL ? positions[s] : position;
        if (pos >= context_tokens) {
            return ORC_INVALID_ARGUMENT;
        }
        if (pos + 1u > max_n) {
            max_n = pos + 1u;
        }
    }
    float *kf = (float *)malloc(max_n * kv_dim * sizeof(float));
    float *vf = (float *)malloc(max_n * kv_dim * sizeof(float));
    if (kf == NULL || vf == NULL) {
        free(kf);
        free(vf);
        return ORC_OUT_OF_MEMORY;
    }
    int status = ORC_OK;
    for (size_t s = 0; s < seqs && status == ORC_OK; ++s) {
        const size_t pos = positions != NULL ? positions[s] : position;
        for (size_t layer = 0; layer < layers && status == ORC_OK; ++layer) {
            const size_t sl = s * layers + layer;
            const size_t base = sl * context_tokens * kv_dim;
            orc_f16_to_f32_array(key_cache + base, kf, (pos + 1u) * kv_dim);
            orc_f16_to_f32_array(value_cache + base, vf, (pos + 1u) * kv_dim);
            status = orc_attention_decode_f32(query + sl * heads * head_dim, kf, vf, pos, heads, kv_heads,
                                              head_dim, out + sl * heads * head_dim);
        }
    }
    free(kf);
    free(vf);
    return status;
}

/* Causal prefill for one (seq, layer): row t attends positions 0..base+t.
 * Restates the per-token loop of reference qwen.c:810-824 (row t == decode at
 * position t) generalised with the base_position of
 * te_attention_flash_mma_t_f32_kernel (metal_kernels.metal.inc:2767-2775).
 * Only rows row_begin, row_begin+row_step, ... < row_end are computed (the
 * others are left untouched), so large cases can be checked on a strided
 * sample.  query fp32 [tokens][heads][head_dim]; caches fp16 [ctx][kv][d]. */
int orc_attention_prefill(const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
                          size_t tokens, size_t base_position, size_t context_tokens, size_t heads,
                          size_t kv_heads, size_t head_dim, size_t row_begin, size_t row_end,
                          size_t row_step, float *out) {
    if (query == NULL || key_cache == NULL || value_cache == NULL || out == NULL || tokens == 0u ||
        heads == 0u || kv_heads == 0u || head_dim == 0u || row_step == 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    if (base_position + tokens > context_tokens) {
        return ORC_INVALID_ARGUMENT;
    }
    const size_t kv_dim = kv_heads * head_dim;
    const size_t n_all = base_position + tokens;
    float *kf = (float *)malloc(n_all * kv_dim * sizeof(float));
    float *vf = (float *)malloc(n_all * kv_dim * sizeof(float));
    if (kf == NULL || vf == NULL) {
        free(kf);
        free(vf);
        return ORC_OUT_OF_MEMORY;
    }
    orc_f16_to_f32_array(key_cache, kf, n_all * kv_dim);
    orc_f16_to_f32_array(value_cache, vf, n_all * kv_dim);
    int status = ORC_OK;
    if (row_end > tokens) {
        row_end = tokens;
    }
    for (size_t t = row_begin; t < row_end && status == ORC_OK; t += row_step) {
        status = orc_attention_decode_f32(query + t * heads * head_dim, kf, vf, base_position + t, heads,
                                          kv_heads, head_dim, out + t * heads * head_dim);
    }
    free(kf);
    free(vf);
    return status;
}

/* ---- decode-layer vector operations ---- */

/* Restates te_rmsnorm_f32 (reference c/src/ops.c:272-293): sum of squares in
 * double, one float scale 1/sqrtf(mean + eps), then input * scale * weight. */
int orc_rmsnorm_f32(const float *input, const float *weight, size_t len, float epsilon, float *out) {
    if (input == NULL || weight == NULL || out == NULL || len == 0u || epsilon <= 0.0f) {
        return ORC_INVALID_ARGUMENT;
    }
    double sum_squares = 0.0;
    for (size_t i = 0; i < len; ++i) {
        const double value = (double)input[i];
        sum_squares += value * value;
    }
    const float scale = 1.0f / sqrtf((float)(sum_squares / (double)len) + epsilon);
    for (size_t i = 0; i < len; ++i) {
        out[i] = input[i] * scale * weight[i];
    }
    return ORC_OK;
}

/* Restates te_swiglu_f32 (ops.c:397-406): silu(gate) * up with
 * silu(g) = g / (1 + expf(-g)). */
int orc_swiglu_f32(const float *gate, const float *up, size_t len, float *out) {
    if (gate == NULL || up == NULL || out == NULL || len == 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    for (size_t i = 0; i < len; ++i) {
        const float silu = gate[i] / (1.0f + expf(-gate[i]));
        out[i] = silu * up[i];
    }
    return ORC_OK;
}

/* Restates te_add_f32 (ops.c:408-416). */
int orc_add_f32(const float *lhs, const float *rhs, size_t len, float *out) {
    if (lhs == NULL || rhs == NULL || out == NULL || len == 0u) {
        return ORC_INVALID_ARGUMENT;
    }
    for (size_t i = 0; i < len; ++i) {
        out[i] = lhs[i] + rhs[i];
    }
    return ORC_OK;
}

/* Restates te_argmax_f32 (ops.c:418-433): the first index whose value is
 * greater than every earlier one, starting from -FLT_MAX; NaN is never taken,
 * and an all -inf / NaN vector gives index 0. */
int orc_argmax_f32(const float *values, size_t len, uint32_t *out_index) {
    if (values == NULL || out_index == NULL || len == 0u || len > UINT32_MAX) {
        return ORC_INVALID_ARGUMENT;
    }
    float best = -FLT_MAX;
    uint32_t best_index = 0;
    for (size_t i = 0; i < len; ++i) {
        if (values[i] > best) {
            best = values[i];
            best_index = (uint32_t)i;
        }
    }
    *out_index = best_index;
    return ORC_OK;
}

static uint16_t orc_read_u16_le(const uint8_t *b) { return (uint16_t)(b[0] | (b[1] << 8)); }

static float orc_read_f32_le(const uint8_t *b) {
    const uint32_t bits = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
    float v;
    memcpy(&v, &bits, sizeof(v));
    return v;
}

/* Bytes of one row (ops.c:217-264: blocks_per_row * block bytes, or cols * 4). */
size_t orc_ggml_row_bytes(uint32_t ggml_type, size_t cols) {
    switch (ggml_type) {
        case ORC_GGML_Q4_0:
            return cols % 32u == 0u ? cols / 32u * 18u : 0u;
        case ORC_GGML_Q8_0:
            return cols % 32u == 0u ? cols / 32u * 34u : 0u;
        case ORC_GGML_F32:
            return cols * sizeof(float);
        default:
            return 0u;
    }
}

/* Restates te_dequantize_q4_0_row / _q8_0_row / _f32_row (ops.c:505-582). */
int orc_dequantize_row_f32(const uint8_t *data, uint32_t ggml_type, size_t cols, size_t row, float *out) {
    const size_t row_bytes = orc_ggml_row_bytes(ggml_type, cols);
    if (data == NULL || out == NULL || row_bytes == 0u) {
        return ORC_UNSUPPORTED;
    }
    const uint8_t *r = data + row * row_bytes;
    if (ggml_type == ORC_GGML_F32) {
        for (size_t col = 0; col < cols; ++col) {
            out[col] = orc_read_f32_le(r + col * sizeof(float));
        }
        return ORC_OK;
    }
    for (size_t block = 0; block < cols / 32u; ++block) {
        if (ggml_type == ORC_GGML_Q4_0) {
            const uint8_t *src = r + block * 18u;
            const float scale = orc_f16_to_f32(orc_read_u16_le(src));
            const uint8_t *qs = src + 2u;
            for (size_t j = 0; j < 16u; ++j) {
                out[block * 32u + j] = ((float)(qs[j] & 0x0fu) - 8.0f) * scale;
                out[block * 32u + j + 16u] = ((float)(qs[j] >> 4u) - 8.0f) * scale;
            }
        } else {
            const uint8_t *src = r + block * 34u;
            const float scale = orc_f16_to_f32(orc_read_u16_le(src));
            const int8_t *qs = (const int8_t *)(src + 2u);
            for (size_t j = 0; j < 32u; ++j) {
                out[block * 32u + j] = (float)qs[j] * scale;
            }
        }
    }
    return ORC_OK;
}

/* Restates te_model_matvec_f32's row loop (ops.c:177-269, te_matvec_worker
 * :828-845) with the portable dot products te_q4_0_dot_row / te_q8_0_dot_row /
 * te_f32_dot_row (ops.c:584-629, the non-NEON branches): one fp32 sum per row,
 * element by element in column order, each term (code * scale) * x. */
int orc_matvec_f32(const uint8_t *data, uint32_t ggml_type, const float *input, size_t cols, size_t rows,
                   float *out) {
    const size_t row_bytes = orc_ggml_row_bytes(ggml_type, cols);
    if (data == NULL || input == NULL || out == NULL || row_bytes == 0u) {
        return ORC_UNSUPPORTED;
    }
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *r = data + row * row_bytes;
        float sum = 0.0f;
        if (ggml_type == ORC_GGML_F32) {
            for (size_t col = 0; col < cols; ++col) {
                sum += orc_read_f32_le(r + col * sizeof(float)) * input[col];
            }
        } else if (ggml_type == ORC_GGML_Q4_0) {
            for (size_t block = 0; block < cols / 32u; ++block) {
                const uint8_t *src = r + block * 18u;
                const float scale = orc_f16_to_f32(orc_read_u16_le(src));
                const uint8_t *qs = src + 2u;
                const float *x = input + block * 32u;
                for (size_t j = 0; j < 16u; ++j) {
                    sum += (((float)(qs[j] & 0x0fu) - 8.0f) * scale) * x[j];
                    sum += (((float)(qs[j] >> 4u) - 8.0f) * scale) * x[j + 16u];
                }
            }
        } else {
            for (size_t block = 0; block < cols / 32u; ++block) {
                const uint8_t *src = r + block * 34u;
                const float scale = orc_f16_to_f32(orc_read_u16_le(src));
                const int8_t *qs = (const int8_t *)(src + 2u);
                const float *x = input + block * 32u;
                for (size_t j = 0; j < 32u; ++j) {
                    sum += ((float)qs[j] * scale) * x[j];
                }
            }
        }
        out[row] = sum;
    }
    return ORC_OK;
}
