// A chunk of prompt tokens through every layer of a Qwen2 model on the GPU:
// the HIP twin of the reference's te_metal_prefill_all_layers_f32
// (c/src/metal_backend.h:311-343), which te_qwen_prefill_all_layers_exact
// calls for a whole prompt (qwen.c:1640-1797).  Row t of the chunk is the
// token at position base_position + t; per layer, for all rows at once:
//
//   norm = rmsnorm(x, attn_norm[l])                               (te_rmsnorm_f32)
//   q, k, v = norm Wq^T + bq, norm Wk^T + bk, norm Wv^T + bv; RoPE q, k; append k, v
//   attn = causal attention: row t over positions 0 .. base + t  (qwen.c:810-824)
//   x += attn Wo^T
//   norm = rmsnorm(x, ffn_norm[l])
//   x += (silu(norm Wg^T) * (norm Wu^T)) Wd^T                     (te_swiglu_f32)
//
// Launches per layer (one stream, no host synchronisation): the GEMM's
// activation digits with RMSNorm folded in, then the Q, K and V GEMMs as one
// segmented launch (te_gemm.hip); the fused prefill step keeping V^T (bias + RoPE + fp16
// append into the K / V caches and V^T, then the MFMA causal attention,
// te_prefill.hip); the digits of the attention output and the Wo GEMM with
// the residual (and the next RMSNorm's digits in its split-K sums); gate and
// up as one launch
// whose epilogue writes the SwiGLU digits (else two GEMMs and the SwiGLU
// digits); the down GEMM with the residual and the next layer's attention
// RMSNorm digits.
//
// Differences from the Metal slot, all device-resident: the K / V caches are
// the HIP path's fp16 caches [layers][context_tokens][kv] plus the transposed
// value copy V^T [layers][kv_heads][head_dim][ctx_pad] the prefill kernel
// reads; the chunk starts at base_position (the reference always starts at 0,
// metal_backend_layers.mm.inc:2205-2222); the weights are the model file's
// bytes in HBM at the reference's absolute tensor offsets.
#include "te_hip_common.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>

namespace {

// Per-stage timing of the prompt-layer flow, the reference's
// TINYENGINE_METAL_PREFILL_STAGE_PROFILE (metal_backend_layers.mm.inc:2295-2340,
// the switch metal_backend_runtime.mm.inc:183-186: set and not "0"): after each
// stage the stream is synchronised and one line goes to stderr in the
// reference's format, `tinyengine_metal_stage_profile: scope=prefill_all_layers
// layer=L stage=S cpu_ms=C gpu_ms=G` -- G the stage's GPU time between two
// events, C the host wait for it.  The synchronisation serialises the stages,
// as the reference's per-stage command buffers do.
class StageProfile {
  public:
    explicit StageProfile(hipStream_t st) : st_(st) {
        const char *v = getenv("TINYENGINE_METAL_PREFILL_STAGE_PROFILE");
        on_ = v != nullptr && strcmp(v, "0") != 0;
        if (on_ && (hipEventCreate(&e0_) != hipSuccess || hipEventCreate(&e1_) != hipSuccess ||
                    hipEventRecord(e0_, st_) != hipSuccess)) {
            (void)hipGetLastError();
            on_ = false;
            failed_ = true;
        }
    }
    ~StageProfile() {
        if (e0_ != nullptr) {
            (void)hipEventDestroy(e0_);
        }
        if (e1_ != nullptr) {
            (void)hipEventDestroy(e1_);
        }
    }
    StageProfile(const StageProfile &) = delete;
    StageProfile &operator=(const StageProfile &) = delete;
    bool failed() const { return failed_; }
    // the stage that was just enqueued (no-op when off); false on a runtime error
    bool stage(const char *name, size_t layer) {
        if (!on_) {
            return true;
        }
        using clock = std::chrono::steady_clock;
        if (hipEventRecord(e1_, st_) != hipSuccess) {
            return false;
        }
        const auto t0 = clock::now();
        if (hipEventSynchronize(e1_) != hipSuccess) {
            return false;
        }
        const double cpu_ms = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
        float gpu_ms = 0.0f;
        if (hipEventElapsedTime(&gpu_ms, e0_, e1_) != hipSuccess) {
            return false;
        }
        fprintf(stderr,
                "tinyengine_metal_stage_profile: scope=prefill_all_layers layer=%zu stage=%s cpu_ms=%.3f "
                "gpu_ms=%.3f\n",
                layer, name, cpu_ms, (double)gpu_ms);
        std::swap(e0_, e1_);  // this stage's end is the next one's start
        return true;
    }

  private:
    hipStream_t st_;
    hipEvent_t e0_ = nullptr, e1_ = nullptr;
    bool on_ = false;
    bool failed_ = false;
};

constexpr size_t kAlign = 256;

size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct ChunkBuffers {
    float *q, *k, *v, *attn, *gate, *up, *part;
    void *act, *act_ffn;  // digits of the hidden-wide inputs; of the SwiGLU output (down's input)
    size_t part_bytes;
};

// Byte layout of the workspace, in carve-up order: the GEMM outputs, the
// split-K partial sums (up to 8 splits of a hidden-wide output), the
// activation digits of the hidden-wide GEMM inputs, then of down's input.
size_t carve(size_t batch, size_t hidden, size_t kv, size_t ffn, unsigned char *base, ChunkBuffers *b) {
    const size_t floats[7] = {batch * hidden, batch * kv, batch * kv, batch * hidden, batch * ffn, batch * ffn,
                              8 * batch * hidden};
    float **slots[7] = {&b->q, &b->k, &b->v, &b->attn, &b->gate, &b->up, &b->part};
    size_t off = 0;
    for (int i = 0; i < 7; ++i) {
        if (base != nullptr) {
            *slots[i] = reinterpret_cast<float *>(base + off);
        }
        off += align_up(floats[i] * sizeof(float));
    }
    const size_t act_hidden = align_up(te_hip::act_buffer_bytes(batch, hidden));
    if (base != nullptr) {
        b->act = base + off;
        b->act_ffn = base + off + act_hidden;
        b->part_bytes = floats[6] * sizeof(float);
    }
    return off + act_hidden + align_up(te_hip::act_buffer_bytes(batch, ffn));
}

bool tensor_fits(uint64_t offset, size_t rows, size_t row_bytes, size_t mapping_len) {
    return row_bytes != 0 && rows <= mapping_len / row_bytes && offset <= mapping_len - rows * row_bytes;
}

}  // namespace

extern "C" size_t te_hip_prefill_all_layers_workspace_bytes(size_t batch, size_t hidden, size_t kv, size_t ffn) {
    if (batch == 0 || hidden == 0 || kv == 0 || ffn == 0) {
        return 0;
    }
    return carve(batch, hidden, kv, ffn, nullptr, nullptr);
}

static te_status prefill_all_layers_impl(
    const void *mapping, size_t mapping_len, const uint64_t *q_offsets, const uint64_t *k_offsets,
    const uint64_t *v_offsets, const uint64_t *output_offsets, const uint64_t *gate_offsets,
    const uint64_t *up_offsets, const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights, const float *q_biases,
    const float *k_biases, const float *v_biases, const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *value_cache_t, size_t base_position, size_t batch,
    size_t context_tokens, size_t hidden, size_t kv, size_t heads, size_t kv_heads, size_t head_dim, size_t ffn,
    float epsilon, float *out, void *workspace, size_t workspace_bytes, void *stream) {
    // the reference's argument checks (qwen.c:1650-1652, metal_backend.mm)
    if (mapping == nullptr || q_offsets == nullptr || k_offsets == nullptr || v_offsets == nullptr ||
        output_offsets == nullptr || gate_offsets == nullptr || up_offsets == nullptr || down_offsets == nullptr ||
        hidden_in == nullptr || attn_norm_weights == nullptr || ffn_norm_weights == nullptr || q_biases == nullptr ||
        k_biases == nullptr || v_biases == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || value_cache_t == nullptr || out == nullptr ||
        workspace == nullptr || layers == 0 || batch == 0 || hidden == 0 || kv == 0 || heads == 0 ||
        kv_heads == 0 || head_dim == 0 || ffn == 0 || context_tokens == 0 || base_position > context_tokens ||
        batch > context_tokens - base_position || epsilon <= 0.0f) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (hidden != heads * head_dim || kv != kv_heads * head_dim || heads % kv_heads != 0 ||
        (head_dim != 64 && head_dim != 128) || (ggml_type != 2 && ggml_type != 8) || hidden % 32 != 0 ||
        ffn % 32 != 0 || batch > 65535 || context_tokens > (1u << 30)) {
        return TE_STATUS_UNSUPPORTED;  // the GEMM takes Q4_0 / Q8_0 rows of whole blocks
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
            if (((size_t)(m + e.off) & 1u) != 0) {
                return TE_STATUS_UNSUPPORTED;  // the GEMM reads 16-bit words of the blocks
            }
        }
    }
    if (((size_t)workspace & (kAlign - 1)) != 0) {
        return TE_STATUS_UNSUPPORTED;
    }
    ChunkBuffers b = {};
    if (workspace_bytes < carve(batch, hidden, kv, ffn, static_cast<unsigned char *>(workspace), &b)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const hipStream_t st = te_hip::as_stream(stream);
    const char *digits_env = getenv("TE_HIP_PREFILL_DIGITS");
    const bool attn_digits = !(digits_env != nullptr && digits_env[0] == '0');
    if (out != hidden_in &&
        hipMemcpyAsync(out, hidden_in, batch * hidden * sizeof(float), hipMemcpyDeviceToDevice, st) != hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    const size_t ctx_kv = context_tokens * kv;
    const size_t vt_layer = te_hip_value_t_bytes(1, 1, context_tokens, kv_heads, head_dim) / sizeof(uint16_t);
    te_hip::prof_begin(st);
    StageProfile stages(st);
    if (stages.failed()) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    te_status s = TE_STATUS_OK;
    for (size_t l = 0; l < layers && s == TE_STATUS_OK; ++l) {
        // each piece of the layer, then its profile mark (no-op unless profiling)
        // and its stage line (no-op unless the stage profile is on)
        const char *stage_name = "";
        auto staged = [&](te_status r) {
            if (r == TE_STATUS_OK && !stages.stage(stage_name, l)) {
                s = TE_STATUS_RUNTIME_ERROR;
                return false;
            }
            return r == TE_STATUS_OK;
        };
        auto done = [&](te_status r, te_hip::ProfPhase p) {
            te_hip::prof_mark(st, p);
            return staged(r);
        };
        auto gemm = [&](const uint64_t *offs, size_t n, size_t k, float *y, const float *resid) {
            return te_hip::launch_gemm_q(m + offs[l], ggml_type, b.act, batch, n, k, y, resid, b.part, b.part_bytes,
                                         st);
        };
        const te_hip::ProfPhase ew = te_hip::kProfElementwise;
        // Q, K and V in one launch (one split-K reduction), profiled by rows
        const te_hip::GemmSeg qkv[3] = {{m + q_offsets[l], b.q, nullptr, hidden},
                                        {m + k_offsets[l], b.k, nullptr, kv},
                                        {m + v_offsets[l], b.v, nullptr, kv}};
        // gate and up with the SwiGLU digits in their epilogue where the
        // shapes allow it, else both GEMMs and the SwiGLU digits
        bool glu = false;
        auto glu_done = [&](te_status r) {
            if (glu) {
                const te_hip::ProfShare share[2] = {{te_hip::kProfGate, 1.0}, {te_hip::kProfUp, 1.0}};
                te_hip::prof_mark(st, share, 2);
                stage_name = "gate_up_swiglu_pair_digits";
                return staged(r);
            }
            return r == TE_STATUS_OK;
        };
        auto qkv_done = [&](te_status r) {
            const te_hip::ProfShare share[3] = {
                {te_hip::kProfQ, (double)hidden}, {te_hip::kProfK, (double)kv}, {te_hip::kProfV, (double)kv}};
            te_hip::prof_mark(st, share, 3);
            return staged(r);
        };
        // the attention RMSNorm digits of layer l > 0 came with the previous
        // layer's down projection
        if ((l == 0 && !done((stage_name = "attn_norm_digits",
                              s = te_hip::launch_quant_act(1, out, nullptr, attn_norm_weights, epsilon, batch, hidden,
                                                           b.act, st)),
                             ew)) ||
            !qkv_done((stage_name = "qkv_proj",
                       s = te_hip::launch_gemm_q_segs(ggml_type, qkv, 3, b.act, batch, hidden, b.part, b.part_bytes,
                                                      st))) ||
            // the attention output leaves the attention kernel as the output
            // projection's digits (TE_HIP_PREFILL_DIGITS=0: fp32 rows and a
            // digits launch, the same bits)
            !done((stage_name = "qkv_bias_rope_flash_attention_mma_vt",
                   s = te_hip::launch_prefill_step_vt(
                       b.q, b.k, b.v, q_biases + l * hidden, k_biases + l * kv, v_biases + l * kv, rope_cos, rope_sin,
                       key_cache + l * ctx_kv, value_cache + l * ctx_kv, value_cache_t + l * vt_layer, 1, 1, batch,
                       base_position, context_tokens, heads, kv_heads, head_dim, b.attn, attn_digits ? b.act : nullptr,
                       nullptr, 0, st)),
                  te_hip::kProfAttention) ||
            (!attn_digits &&
             !done((stage_name = "attn_out_digits",
                    s = te_hip::launch_quant_act(0, b.attn, nullptr, nullptr, 0.0f, batch, hidden, b.act, st)),
                   ew)) ||
            !done((stage_name = "output_proj_add_ffn_norm_digits",
                   s = te_hip::launch_gemm_q_rms(m + output_offsets[l], ggml_type, b.act, batch, hidden, hidden, out,
                                                 out, b.part, b.part_bytes, ffn_norm_weights + l * hidden, epsilon,
                                                 b.act, st)),
                  te_hip::kProfO) ||
            !glu_done(s = te_hip::launch_gemm_glu_q(ggml_type, m + gate_offsets[l], m + up_offsets[l], b.act, batch,
                                                    ffn, hidden, b.act_ffn, st, &glu))) {
            break;
        }
        if (!glu && (!done((stage_name = "gate_proj", s = gemm(gate_offsets, ffn, hidden, b.gate, nullptr)),
                           te_hip::kProfGate) ||
                     !done((stage_name = "up_proj", s = gemm(up_offsets, ffn, hidden, b.up, nullptr)),
                           te_hip::kProfUp) ||
                     !done((stage_name = "swiglu_digits",
                            s = te_hip::launch_quant_act(2, b.gate, b.up, nullptr, 0.0f, batch, ffn, b.act_ffn, st)),
                           ew))) {
            break;
        }
        // down + residual, with the next layer's attention RMSNorm digits
        s = l + 1 < layers
                ? te_hip::launch_gemm_q_rms(m + down_offsets[l], ggml_type, b.act_ffn, batch, hidden, ffn, out, out,
                                            b.part, b.part_bytes, attn_norm_weights + (l + 1) * hidden, epsilon,
                                            b.act, st)
                : te_hip::launch_gemm_q(m + down_offsets[l], ggml_type, b.act_ffn, batch, hidden, ffn, out, out,
                                        b.part, b.part_bytes, st);
        stage_name = l + 1 < layers ? "down_proj_add_attn_norm_digits" : "down_proj_add";
        if (!done(s, te_hip::kProfDown)) {
            break;
        }
    }
    return s;
}

extern "C" te_status te_hip_prefill_all_layers_f16(
    const void *mapping, size_t mapping_len, const uint64_t *q_offsets, const uint64_t *k_offsets,
    const uint64_t *v_offsets, const uint64_t *output_offsets, const uint64_t *gate_offsets,
    const uint64_t *up_offsets, const uint64_t *down_offsets, size_t layers, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weights, const float *ffn_norm_weights, const float *q_biases,
    const float *k_biases, const float *v_biases, const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *value_cache_t, size_t base_position, size_t batch,
    size_t context_tokens, size_t hidden, size_t kv, size_t heads, size_t kv_heads, size_t head_dim, size_t ffn,
    float epsilon, float *out, void *workspace, size_t workspace_bytes, void *stream) {
    te_hip::BackendTimer timer(te_hip::kBucketPrefillAllLayers, te_hip::as_stream(stream));
    return timer.finish(prefill_all_layers_impl(mapping, mapping_len, q_offsets, k_offsets, v_offsets, output_offsets,
                                                gate_offsets, up_offsets, down_offsets, layers, ggml_type, hidden_in,
                                                attn_norm_weights, ffn_norm_weights, q_biases, k_biases, v_biases,
                                                rope_cos, rope_sin, key_cache, value_cache, value_cache_t,
                                                base_position, batch, context_tokens, hidden, kv, heads, kv_heads,
                                                head_dim, ffn, epsilon, out, workspace, workspace_bytes, stream));
}

// ---- single-layer twins ------------------------------------------------------

extern "C" te_status te_hip_prefill_layer_f16(
    const void *mapping, size_t mapping_len, uint64_t q_offset, uint64_t k_offset, uint64_t v_offset,
    uint64_t output_offset, uint64_t gate_offset, uint64_t up_offset, uint64_t down_offset, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weight, const float *ffn_norm_weight, const float *q_bias,
    const float *k_bias, const float *v_bias, const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
    uint16_t *value_cache, uint16_t *value_cache_t, size_t base_position, size_t batch, size_t context_tokens,
    size_t hidden, size_t kv, size_t heads, size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out,
    void *workspace, size_t workspace_bytes, void *stream) {
    // one prefill_layer call in the backend profile (the inner flow's timer is nested)
    te_hip::BackendTimer timer(te_hip::kBucketPrefillLayer, te_hip::as_stream(stream));
    return timer.finish(te_hip_prefill_all_layers_f16(mapping, mapping_len, &q_offset, &k_offset, &v_offset,
                                                      &output_offset, &gate_offset, &up_offset, &down_offset, 1,
                                                      ggml_type, hidden_in, attn_norm_weight, ffn_norm_weight, q_bias,
                                                      k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache,
                                                      value_cache_t, base_position, batch, context_tokens, hidden, kv,
                                                      heads, kv_heads, head_dim, ffn, epsilon, out, workspace,
                                                      workspace_bytes, stream));
}

extern "C" te_status te_hip_decode_layer_f16(
    const void *mapping, size_t mapping_len, uint64_t q_offset, uint64_t k_offset, uint64_t v_offset,
    uint64_t output_offset, uint64_t gate_offset, uint64_t up_offset, uint64_t down_offset, uint32_t ggml_type,
    const float *hidden_in, const float *attn_norm_weight, const float *ffn_norm_weight, const float *q_bias,
    const float *k_bias, const float *v_bias, const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
    uint16_t *value_cache, size_t position, size_t context_tokens, size_t hidden, size_t kv, size_t heads,
    size_t kv_heads, size_t head_dim, size_t ffn, float epsilon, float *out, void *workspace,
    size_t workspace_bytes, void *stream) {
    // one decode_layer call in the backend profile (the inner flow's timer is nested)
    te_hip::BackendTimer timer(te_hip::kBucketDecodeLayer, te_hip::as_stream(stream));
    return timer.finish(te_hip_decode_all_layers_f16(mapping, mapping_len, &q_offset, &k_offset, &v_offset,
                                                     &output_offset, &gate_offset, &up_offset, &down_offset, 1,
                                                     ggml_type, hidden_in, attn_norm_weight, ffn_norm_weight, q_bias,
                                                     k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache,
                                                     position, context_tokens, hidden, kv, heads, kv_heads, head_dim,
                                                     ffn, epsilon, out, 0, 0, nullptr, 0, nullptr, workspace,
                                                     workspace_bytes, stream));
}
