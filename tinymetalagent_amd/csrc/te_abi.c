/*
 * ABI plumbing of libtinyengine.so (reference c/src/tinyengine.c:13-268):
 * version and status strings, option defaults, capability and kernel-plan
 * reports.
 *
 * The status strings are part of the contract (reference tinyengine.c:17-34):
 * the agent layer matches the exact text "unsupported"
 * (python/tinyagent/engine.py:46, :62).
 *
 * GGUF models, the tokenizer, contexts and generation are in te_model.hip;
 * the element-wise ops (te_rmsnorm_f32, te_swiglu_f32, te_add_f32,
 * te_argmax_f32) run on the GPU in te_hip_runtime.hip.
 */
#include "tinyengine.h"
#include "te_hip_backend.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static const char *const TE_VERSION_STRING = "0.1.0-c-abi-hip-gfx950";

const char *te_version(void) {
    return TE_VERSION_STRING;
}

const char *te_strerror(te_status status) {
    switch (status) {
        case TE_STATUS_OK:
            return "ok";
        case TE_STATUS_INVALID_ARGUMENT:
            return "invalid argument";
        case TE_STATUS_IO_ERROR:
            return "I/O error";
        case TE_STATUS_UNSUPPORTED:
            return "unsupported";
        case TE_STATUS_OUT_OF_MEMORY:
            return "out of memory";
        case TE_STATUS_RUNTIME_ERROR:
            return "runtime error";
        default:
            return "unknown error";
    }
}

/* Names as the reference prints them (tinyengine.c:36-83): the GGUF block
 * formats carry their "GGUF_" prefix, anything else is "UNKNOWN". */
const char *te_quant_name(te_quant_kind quant) {
    static const char *const names[TE_QUANT_COUNT] = {
        "UNKNOWN", "F32", "F16", "BF16", "GGUF_Q4_0", "GGUF_Q4_1", "GGUF_Q5_0", "GGUF_Q5_1", "GGUF_Q8_0",
        "GGUF_Q2_K", "GGUF_Q3_K", "GGUF_Q4_K", "GGUF_Q5_K", "GGUF_Q6_K", "GGUF_Q8_K", "GGUF_IQ2_XXS",
        "GGUF_IQ2_XS", "GGUF_IQ3_XXS", "GGUF_IQ3_S", "GGUF_IQ4_NL", "GGUF_IQ4_XS", "MXFP4"};
    if ((int)quant < 0 || quant >= TE_QUANT_COUNT) {
        return "UNKNOWN";
    }
    return names[quant];
}

/* Names as the reference prints them (tinyengine.c:85-118). */
const char *te_vector_op_name(te_vector_op op) {
    static const char *const names[TE_OP_COUNT] = {
        "matvec", "matmul", "batched-prefill", "decode-token", "rmsnorm", "rope", "causal-attention",
        "swiglu", "residual-add", "argmax", "sampling", "kv-cache", "tokenize"};
    if ((int)op < 0 || op >= TE_OP_COUNT) {
        return "unknown";
    }
    return names[op];
}

/* Defaults: reference tinyengine.c:121-132 (context 512, batch 128). */
te_runtime_options te_default_options(void) {
    te_runtime_options options;
    memset(&options, 0, sizeof(options));
    options.abi_version = TE_ABI_VERSION;
    options.target_arch = TE_ARCH_AUTO;
    options.context_tokens = 512u;
    options.batch_tokens = 128u;
    return options;
}

/* The operations this build implements: the attention step, the decode-layer
 * vector operations around it (matvec, RMSNorm, SwiGLU, residual add, argmax),
 * whole decode tokens, top-k sampling and the tokenizer. */
static uint64_t te_hip_op_mask(void) {
    return (1ull << TE_OP_ROPE) | (1ull << TE_OP_CAUSAL_ATTENTION) | (1ull << TE_OP_KV_CACHE) |
           (1ull << TE_OP_BATCHED_PREFILL) | (1ull << TE_OP_MATVEC) | (1ull << TE_OP_RMSNORM) |
           (1ull << TE_OP_SWIGLU) | (1ull << TE_OP_RESIDUAL_ADD) | (1ull << TE_OP_ARGMAX) |
           (1ull << TE_OP_DECODE_TOKEN) | (1ull << TE_OP_SAMPLING) | (1ull << TE_OP_TOKENIZE);
}

/* Weight / cache formats: fp32 and fp16 data, GGUF Q4_0 and Q8_0 matvec. */
static uint64_t te_hip_quant_mask(void) {
    return (1ull << TE_QUANT_F32) | (1ull << TE_QUANT_F16) | (1ull << TE_QUANT_GGUF_Q4_0) |
           (1ull << TE_QUANT_GGUF_Q8_0);
}

te_status te_detect_arch(te_arch_info *out_info) {
    if (out_info == NULL) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    memset(out_info, 0, sizeof(*out_info));
    long cores = sysconf(_SC_NPROCESSORS_ONLN);
    out_info->cpu_cores = cores > 0 ? (uint32_t)cores : 0u;
    uint32_t cus = 0;
    if (te_hip_device_info(out_info->name, sizeof(out_info->name), &cus) == TE_STATUS_OK) {
        out_info->kind = TE_ARCH_AMD_GFX950;
        out_info->gpu_cores = cus;
        out_info->recommended_max_context = 131072u;
    } else {
        out_info->kind = TE_ARCH_AUTO;
        snprintf(out_info->name, sizeof(out_info->name), "%s", "no gfx950 device");
    }
    return TE_STATUS_OK;
}

te_status te_get_capabilities(te_capabilities *out_capabilities) {
    if (out_capabilities == NULL) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    memset(out_capabilities, 0, sizeof(*out_capabilities));
    out_capabilities->abi_version = TE_ABI_VERSION;
    out_capabilities->known_quant_mask[0] = te_hip_quant_mask();
    out_capabilities->optimized_quant_mask[0] = te_hip_quant_mask();
    out_capabilities->vector_op_mask = te_hip_op_mask();
    out_capabilities->optimization_flags = TE_OPT_ARCH_SPECIALIZED | TE_OPT_GPU_RESIDENT_KV | TE_OPT_BATCHED_PREFILL;
    out_capabilities->preferred_alignment_bytes = 256u;
    snprintf(out_capabilities->backend_name, sizeof(out_capabilities->backend_name), "%s", "hip-gfx950");
    snprintf(out_capabilities->notes, sizeof(out_capabilities->notes), "%s",
             "MI355X: RoPE, fp16 KV append, split-K GQA decode, MFMA causal prefill; Q4_0/Q8_0/F32 matvec, "
             "RMSNorm, SwiGLU, add, argmax");
    return TE_STATUS_OK;
}

/* Reference tinyengine.c:201-235: NULL options mean te_default_options(),
 * ABI version 0 is accepted as "current", TE_ARCH_AUTO resolves through
 * te_detect_arch.  The masks and sizes describe this library's kernels. */
te_status te_make_kernel_plan(const te_runtime_options *options, te_kernel_plan *out_plan) {
    const te_runtime_options effective = options != NULL ? *options : te_default_options();
    if (out_plan == NULL) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (effective.abi_version != 0u && effective.abi_version != TE_ABI_VERSION) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_arch_kind arch = effective.target_arch;
    if (arch == TE_ARCH_AUTO) {
        te_arch_info info;
        const te_status status = te_detect_arch(&info);
        if (status != TE_STATUS_OK) {
            return status;
        }
        arch = info.kind;
    }
    memset(out_plan, 0, sizeof(*out_plan));
    out_plan->abi_version = TE_ABI_VERSION;
    out_plan->target_arch = arch;
    out_plan->quant_mask[0] = te_hip_quant_mask();
    out_plan->optimized_quant_mask[0] = te_hip_quant_mask();
    out_plan->vector_op_mask = te_hip_op_mask();
    out_plan->optimization_flags = TE_OPT_ARCH_SPECIALIZED | TE_OPT_GPU_RESIDENT_KV | TE_OPT_BATCHED_PREFILL;
    out_plan->dot_threads = 64u; /* wavefront width */
    out_plan->preferred_alignment_bytes = 256u;
    out_plan->max_context_tokens = effective.context_tokens != 0u ? effective.context_tokens : 512u;
    out_plan->memory_budget_bytes = effective.memory_limit_bytes;
    snprintf(out_plan->metal_function_suffix, sizeof(out_plan->metal_function_suffix), "%s", "_gfx950");
    return TE_STATUS_OK;
}

/* Reference tinyengine.c:237-246: the plan is required, the options are not. */
te_status te_compile_kernels(const te_runtime_options *options, const te_kernel_plan *plan) {
    (void)options;
    if (plan == NULL) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (plan->abi_version != TE_ABI_VERSION) {
        return TE_STATUS_UNSUPPORTED;
    }
    /* Kernels are compiled ahead of time for gfx950. */
    return te_hip_available() ? TE_STATUS_OK : TE_STATUS_UNSUPPORTED;
}

static int te_mask_has(const uint64_t *mask, unsigned bit) {
    return (mask[bit / 64u] >> (bit % 64u)) & 1u;
}

int te_kernel_plan_supports_quant(const te_kernel_plan *plan, te_quant_kind quant) {
    if (plan == NULL || (int)quant < 0 || quant >= TE_QUANT_COUNT) {
        return 0;
    }
    return te_mask_has(plan->quant_mask, (unsigned)quant);
}

int te_kernel_plan_optimizes_quant(const te_kernel_plan *plan, te_quant_kind quant) {
    if (plan == NULL || (int)quant < 0 || quant >= TE_QUANT_COUNT) {
        return 0;
    }
    return te_mask_has(plan->optimized_quant_mask, (unsigned)quant);
}

int te_kernel_plan_supports_op(const te_kernel_plan *plan, te_vector_op op) {
    if (plan == NULL || (int)op < 0 || op >= TE_OP_COUNT) {
        return 0;
    }
    return (int)((plan->vector_op_mask >> (unsigned)op) & 1u);
}
