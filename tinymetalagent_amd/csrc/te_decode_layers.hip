// The decode step of every layer of a Qwen2 model on the GPU: the HIP twin of
// the reference's te_metal_decode_all_layers_f32 (c/src/metal_backend.h:239-276),
// which qwen.c calls per generated token (te_qwen_decode_all_layers_exact,
// qwen.c:1464-1640) and which replaces the CPU layer loop of
// te_qwen_forward_token (qwen.c:907-1087).  Per layer, in the reference's order:
//
//   norm = rmsnorm(hidden, attn_norm[l])                           (te_rmsnorm_f32)
//   q, k, v = Wq norm + bq, Wk norm + bk, Wv norm + bv; RoPE q, k; append k, v
//   attn = decode attention over positions 0..position           (te_attention_decode_f32)
//   hidden += Wo attn
//   norm = rmsnorm(hidden, ffn_norm[l])
//   hidden += Wd (silu(Wg norm) * Wu norm)                         (te_swiglu_f32)
//
// and, when a token is asked for, token = argmax(W_head rmsnorm(hidden, out_norm)).
//
// Launches per layer (one stream, no host synchronisation): the fused GEMVs of
// te_vecops.hip take the RMSNorm / SwiGLU into their input staging and the
// residual add into their epilogue, and the attention is the fused decode step
// (bias + RoPE of q in registers, bias + RoPE + fp16 append of k / v, split-K)
// plus its merge:
//   1. RMSNorm + [Wq; Wk; Wv]            (three matrices, one launch)
//   2. decode step split-K, 3. merge
//   4. Wo + residual
//   5. RMSNorm + [Wg; Wu]                (two matrices, one launch)
//   6. SwiGLU + Wd + residual
// The KV cache is the HIP path's fp16 cache [layers][context][kv]; the weights
// are the model file's tensor data in HBM (`mapping` is its device copy, the
// offsets are the reference's absolute tensor offsets).
#include "te_hip_common.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct LayerBuffers {
    float *q, *k, *v, *attn, *gate, *up, *xtmp, *proj, *logits;
    void *step_ws;
    size_t step_ws_bytes;
};

// Byte sizes of the workspace pieces, in carve-up order.
size_t carve(size_t position, size_t hidden, size_t kv, size_t heads, size_t kv_heads, size_t head_dim, size_t ffn,
             size_t vocab, unsigned char *base, LayerBuffers *b) {
    const size_t step = te_hip_attention_decode_workspace_bytes(nullptr, position, 1, 1, heads, kv_heads, head_dim);
    const size_t sizes[9] = {hidden, kv, kv, hidden, ffn, ffn, std::max(hidden, ffn), hidden, vocab};
    size_t off = 0;
    float **slots[9] = {&b->q, &b->k, &b->v, &b->attn, &b->gate, &b->up, &b->xtmp, &b->proj, &b->logits};
    for (int i = 0; i < 9; ++i) {
        if (base != nullptr) {
            *slots[i] = reinterpret_cast<float *>(base + off);
        }
        off += align_up(sizes[i] * sizeof(float));
    }
    if (base != nullptr) {
        b->step_ws = base + off;
        b->step_ws_bytes = step;
    }
    return off + align_up(step);
}

bool tensor_fits(uint64_t offset, size_t rows, size_t row_bytes, size_t mapping_len) {
    return row_bytes != 0 && rows <= mapping_len / row_bytes && offset <= mapping_len - rows * row_bytes;
}

bool supported_type(uint32_t t) { return t == 0 || t == 2 || t == 8; }

// Quantized tensors need dword-aligned rows; F32 ones float4-aligned.
bool aligned_for(uint32_t t, const void *p) { return ((size_t)p & (t == 0 ? 15u : 3u)) == 0; }

}  // namespace

extern "C" size_t te_hip_decode_all_layers_workspace_bytes(size_t position, size_t hidden, size_t kv, size_t heads,
                                                           size_t kv_heads, size_t head_dim, size_t ffn,
                                                           size_t vocab) {
    if (heads == 0 || kv_heads == 0 || head_dim == 0) {
        return 0;
    }
    return carve(position, hidden, kv, heads, kv_heads, head_dim, ffn, vocab, nullptr, nullptr);
}

static te_status decode_all_layers_impl(
    const void *mapping, size_t mapping_len, const uint64_t *q_offsets, const uint64_t *k_offsets,
    const uint64_t *v_offsets, const uint64_t *output_offsets, const uint64_t *gate_offsets,
    const uint64_t *up_offsets, const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights, const float *q_biases,
    const float *k_biases, const float *v_biases, const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, size_t position, size_t context_tokens, size_t hidden, size_t kv,
    size_t heads, size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out, uint64_t head_offset,
    uint32_t head_ggml_type, const float *output_norm_weight, size_t vocab, uint32_t *out_token_id,
    void *workspace, size_t workspace_bytes, void *stream) {
    // the reference's argument checks (metal_backend.mm, qwen.c:1478-1488)
    if (mapping == nullptr || q_offsets == nullptr || k_offsets == nullptr || v_offsets == nullptr ||
        output_offsets == nullptr || gate_offsets == nullptr || up_offsets == nullptr || down_offsets == nullptr ||
        hidden_in == nullptr || attn_norm_weights == nullptr || ffn_norm_weights == nullptr || q_biases == nullptr ||
        k_biases == nullptr || v_biases == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || out == nullptr || layers == 0 || hidden == 0 ||
        kv == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || ffn == 0 || position >= context_tokens ||
        epsilon <= 0.0f || workspace == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (out_token_id != nullptr && (output_norm_weight == nullptr || vocab == 0)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (hidden != heads * head_dim || kv != kv_heads * head_dim || heads % kv_heads != 0 ||
        (head_dim != 64 && head_dim != 128) || heads / kv_heads > 16 || hidden % 64 != 0 ||
        ffn % 64 != 0 || !supported_type(ggml_type) ||
        (out_token_id != nullptr && !supported_type(head_ggml_type)) || context_tokens > (1u << 30) ||
        vocab > 0xffffffffu) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t rb_hidden = te_hip::ggml_row_bytes(ggml_type, hidden);
    const size_t rb_ffn = te_hip::ggml_row_bytes(ggml_type, ffn);
    const unsigned char *m = static_cast<const unsigned char *>(mapping);
    for (size_t l = 0; l < layers; ++l) {
        const struct {
            uint64_t off;
            size_t rows, row_bytes;
        } t[7] = {{q_offsets[l], hidden, rb_hidden},     {k_offsets[l], kv, rb_hidden},
                  {v_offsets[l], kv, rb_hidden},         {output_offsets[l], hidden, rb_hidden},
                  {gate_offsets[l], ffn, rb_hidden},     {up_offsets[l], ffn, rb_hidden},
                  {down_offsets[l], hidden, rb_ffn}};
        for (const auto &e : t) {
            if (!tensor_fits(e.off, e.rows, e.row_bytes, mapping_len)) {
                return TE_STATUS_INVALID_ARGUMENT;
            }
            if (!aligned_for(ggml_type, m + e.off)) {
                return TE_STATUS_UNSUPPORTED;
            }
        }
    }
    if (out_token_id != nullptr) {
        const size_t rb_head = te_hip::ggml_row_bytes(head_ggml_type, hidden);
        if (!tensor_fits(head_offset, vocab, rb_head, mapping_len)) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
        if (!aligned_for(head_ggml_type, m + head_offset)) {
            return TE_STATUS_UNSUPPORTED;
        }
    }
    if (((size_t)workspace & (kAlign - 1)) != 0 || ((size_t)hidden_in & 15u) != 0 || ((size_t)out & 15u) != 0 ||
        ((size_t)attn_norm_weights & 15u) != 0 || ((size_t)ffn_norm_weights & 15u) != 0 ||
        (output_norm_weight != nullptr && ((size_t)output_norm_weight & 15u) != 0)) {
        return TE_STATUS_UNSUPPORTED;
    }
    LayerBuffers b = {};
    const size_t need = carve(position, hidden, kv, heads, kv_heads, head_dim, ffn,
                              out_token_id != nullptr ? vocab : 0, static_cast<unsigned char *>(workspace), &b);
    if (workspace_bytes < need) {
        return TE_STATUS_INVALID_ARGUMENT;
    }

    const hipStream_t st = te_hip::as_stream(stream);
    te_hip::prof_begin(st);
    if (out != hidden_in && hipMemcpyAsync(out, hidden_in, hidden * sizeof(float), hipMemcpyDeviceToDevice, st) !=
                                hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    using te_hip::prof_mark;
    const te_hip::ProfShare qkv_share[3] = {
        {te_hip::kProfQ, (double)hidden}, {te_hip::kProfK, (double)kv}, {te_hip::kProfV, (double)kv}};
    const te_hip::ProfShare gu_share[2] = {{te_hip::kProfGate, 1.0}, {te_hip::kProfUp, 1.0}};
    // The attention step's merge folds into the Wo projection's input staging
    // (launch_gemv_merge) where the one-layer split is short: its partials,
    // heads x chunks x (head_dim + 2) floats, are then read by every workgroup
    // of the projection instead of by a merge launch.  TE_HIP_DECODE_MERGE_WO=0
    // keeps the merge launch.  The workspace holds the partials as the split-K
    // launch lays them out for one (seq, layer): o, then (m, l).
    size_t dchunk = 0, dchunks = 0;
    const char *merge_env = getenv("TE_HIP_DECODE_MERGE_WO");
    const bool merge_wo = !(merge_env != nullptr && strcmp(merge_env, "0") == 0) &&
                          te_hip_attention_decode_chunking(nullptr, position, 1, 1, kv_heads, 0, &dchunk, &dchunks) ==
                              TE_STATUS_OK &&
                          dchunks <= (size_t)te_hip::kGemvMergeMaxChunks;
    const float *part_o = static_cast<const float *>(b.step_ws);
    const float *part_ml = part_o + heads * dchunks * head_dim;
    te_status s = TE_STATUS_OK;
    for (size_t l = 0; l < layers && s == TE_STATUS_OK; ++l) {
        const te_hip::GemvSeg qkv[3] = {{m + q_offsets[l], b.q, nullptr, hidden},
                                        {m + k_offsets[l], b.k, nullptr, kv},
                                        {m + v_offsets[l], b.v, nullptr, kv}};
        s = te_hip::launch_gemv(ggml_type, te_hip::kGemvRmsNorm, qkv, 3, hidden, out, nullptr,
                                attn_norm_weights + l * hidden, epsilon, b.xtmp, b.proj, st);
        if (s != TE_STATUS_OK) {
            break;
        }
        prof_mark(st, qkv_share, 3);
        const size_t cache_off = l * context_tokens * kv;
        const te_hip::GemvSeg o = {m + output_offsets[l], out, out, hidden};
        bool merged_in_wo = false;
        if (merge_wo) {
            s = te_hip_attention_decode_step_splitk_f16(b.q, b.k, b.v, q_biases + l * hidden, k_biases + l * kv,
                                                        v_biases + l * kv, rope_cos, rope_sin, key_cache + cache_off,
                                                        value_cache + cache_off, nullptr, position, 1, 1,
                                                        context_tokens, heads, kv_heads, head_dim, b.step_ws,
                                                        b.step_ws_bytes, stream);
            if (s != TE_STATUS_OK) {
                break;
            }
            prof_mark(st, te_hip::kProfAttention);
            s = te_hip::launch_gemv_merge(ggml_type, o, hidden, part_o, part_ml, dchunks, dchunks, head_dim, st,
                                          &merged_in_wo);
            if (s == TE_STATUS_OK && !merged_in_wo) {
                s = te_hip_attention_decode_combine(nullptr, position, 1, 1, heads, kv_heads, head_dim, b.attn,
                                                    b.step_ws, b.step_ws_bytes, stream);
                prof_mark(st, te_hip::kProfAttention);
            }
        } else {
            s = te_hip_attention_decode_step_f16(b.q, b.k, b.v, q_biases + l * hidden, k_biases + l * kv,
                                                 v_biases + l * kv, rope_cos, rope_sin, key_cache + cache_off,
                                                 value_cache + cache_off, nullptr, position, 1, 1, context_tokens,
                                                 heads, kv_heads, head_dim, b.attn, b.step_ws, b.step_ws_bytes,
                                                 stream);
            prof_mark(st, te_hip::kProfAttention);
        }
        if (s != TE_STATUS_OK) {
            break;
        }
        if (!merged_in_wo) {
            s = te_hip::launch_gemv(ggml_type, te_hip::kGemvPlain, &o, 1, hidden, b.attn, nullptr, nullptr, 0.0f,
                                    b.xtmp, b.proj, st);
            if (s != TE_STATUS_OK) {
                break;
            }
        }
        prof_mark(st, te_hip::kProfO);
        // gate / up with the SwiGLU in their epilogue (h into b.gate) where the
        // shapes allow it, else both projections and the SwiGLU staged by down
        bool glu = false;
        s = te_hip::launch_gemv_glu(ggml_type, m + gate_offsets[l], m + up_offsets[l], ffn, hidden, out,
                                    ffn_norm_weights + l * hidden, epsilon, b.gate, st, &glu);
        if (s == TE_STATUS_OK && !glu) {
            const te_hip::GemvSeg gu[2] = {{m + gate_offsets[l], b.gate, nullptr, ffn},
                                           {m + up_offsets[l], b.up, nullptr, ffn}};
            s = te_hip::launch_gemv(ggml_type, te_hip::kGemvRmsNorm, gu, 2, hidden, out, nullptr,
                                    ffn_norm_weights + l * hidden, epsilon, b.xtmp, b.proj, st);
        }
        if (s != TE_STATUS_OK) {
            break;
        }
        prof_mark(st, gu_share, 2);
        const te_hip::GemvSeg d = {m + down_offsets[l], out, out, hidden};
        s = te_hip::launch_gemv(ggml_type, glu ? te_hip::kGemvPlain : te_hip::kGemvSwiGLU, &d, 1, ffn, b.gate,
                                b.up, nullptr, 0.0f, b.xtmp, b.proj, st);
        prof_mark(st, te_hip::kProfDown);
    }
    if (s == TE_STATUS_OK && out_token_id != nullptr) {
        const te_hip::GemvSeg h = {m + head_offset, b.logits, nullptr, vocab};
        s = te_hip::launch_gemv(head_ggml_type, te_hip::kGemvRmsNorm, &h, 1, hidden, out, nullptr,
                                output_norm_weight, epsilon, b.xtmp, b.proj, st);
        prof_mark(st, te_hip::kProfLmHead);
        if (s == TE_STATUS_OK) {
            s = te_hip::launch_argmax(b.logits, vocab, out_token_id, st);
            prof_mark(st, te_hip::kProfElementwise);
        }
    }
    return s;
}

extern "C" te_status te_hip_decode_all_layers_f16(
    const void *mapping, size_t mapping_len, const uint64_t *q_offsets, const uint64_t *k_offsets,
    const uint64_t *v_offsets, const uint64_t *output_offsets, const uint64_t *gate_offsets,
    const uint64_t *up_offsets, const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights, const float *q_biases,
    const float *k_biases, const float *v_biases, const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, size_t position, size_t context_tokens, size_t hidden, size_t kv,
    size_t heads, size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out, uint64_t head_offset,
    uint32_t head_ggml_type, const float *output_norm_weight, size_t vocab, uint32_t *out_token_id,
    void *workspace, size_t workspace_bytes, void *stream) {
    const te_hip::BackendBucket bucket =
        out_token_id != nullptr ? te_hip::kBucketDecodeProject : te_hip::kBucketDecodeAllLayers;
    te_hip::BackendTimer timer(bucket, te_hip::as_stream(stream));
    return timer.finish(decode_all_layers_impl(mapping, mapping_len, q_offsets, k_offsets, v_offsets, output_offsets,
                                               gate_offsets, up_offsets, down_offsets, layers, ggml_type, hidden_in,
                                               attn_norm_weights, ffn_norm_weights, q_biases, k_biases, v_biases,
                                               rope_cos, rope_sin, key_cache, value_cache, position, context_tokens,
                                               hidden, kv, heads, kv_heads, head_dim, ffn, epsilon, out, head_offset,
                                               head_ggml_type, output_norm_weight, vocab, out_token_id, workspace,
                                               workspace_bytes, stream));
}
