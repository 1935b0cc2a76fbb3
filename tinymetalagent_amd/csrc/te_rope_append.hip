// Bias + RoPE + fp16 KV-cache append (decode: 1 token per (seq, layer);
// prefill: `tokens` tokens per (seq, layer)), and the plain row rotation used
// by te_rope_f32.
//
// Semantics follow te_qkv_bias_rope_cache_batch_f32 / _h_f32
// (reference metal_kernels.metal.inc:2172-2252, :2344-2429) and the CPU order
// bias-add -> te_qwen_rope_cached -> append (qwen.c:774-808, :998-1036):
//   a = x[i] + bias[i], b = x[i+half] + bias[i+half]
//   x[i] = a*cos - b*sin,  x[i+half] = b*cos + a*sin
// FP contraction is off in this file so the rotated values are bit-identical
// to the CPU reference given the same cos/sin table rows; the bias add is
// skipped (not "+0") when no bias is given, again matching the CPU path.
//
// HBM traffic per token-layer: read q,k,v fp32 + table row, write q,k,v fp32
// and k,v fp16 -- a few KB; the kernel is launch/latency-bound at decode and
// HBM-bound at prefill.
#include "te_hip_common.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace {

struct RopeAppendArgs {
    float *q;
    float *k;
    float *v;
    const float *q_bias;
    const float *k_bias;
    const float *v_bias;
    const float *cos_t;
    const float *sin_t;
    f16 *key_cache;
    f16 *value_cache;
    f16 *q_half;
    int write_back;  // 0: k and v are inputs only (fused prefill step)
    int layers;
    int tokens;
    int ctx;
    int heads;
    int kv_heads;
    int head_dim;
    int base[TE_HIP_MAX_SEQS];
};

// VEC consecutive values of a row: one 16-byte access for VEC = 4.
template <int VEC>
__device__ __forceinline__ void load_vec(const float *p, float (&x)[VEC]) {
    if constexpr (VEC == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p);
        x[0] = t.x;
        x[1] = t.y;
        x[2] = t.z;
        x[3] = t.w;
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            x[j] = p[j];
        }
    }
}

template <int VEC>
__device__ __forceinline__ void store_vec(float *p, const float (&x)[VEC]) {
    if constexpr (VEC == 4) {
        *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            p[j] = x[j];
        }
    }
}

template <int VEC>
__device__ __forceinline__ void store_vec_f16(f16 *p, const float (&x)[VEC]) {
    if constexpr (VEC == 4) {
        *reinterpret_cast<f16x4 *>(p) = f16x4{(f16)x[0], (f16)x[1], (f16)x[2], (f16)x[3]};
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            p[j] = (f16)x[j];
        }
    }
}

// Item = VEC consecutive rotation pairs (q, k) or VEC consecutive values (v)
// of one token; the operations per element are the same for every VEC.
template <int VEC>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(RopeAppendArgs a) {
    const int item = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    const int sl = blockIdx.z;
    const int s = sl / a.layers;
    const int layer = sl - s * a.layers;
    const int half = a.head_dim >> 1;
    const int hq = half / VEC;  // items per head
    const int pos = a.base[s] + b;
    const int hidden = a.heads * a.head_dim;
    const int kv_dim = a.kv_heads * a.head_dim;
    const float *cos_row = a.cos_t + (size_t)pos * half;
    const float *sin_row = a.sin_t + (size_t)pos * half;
    const size_t tok = (size_t)sl * a.tokens + b;

    // one rotation of VEC pairs (x0 + bias, x1 + bias) at dims i .. and i + half ..
    auto rotate = [&](const float *row, const float *bias, int off, int i, float (&lo)[VEC], float (&hi)[VEC]) {
        float x0[VEC], x1[VEC], cs[VEC], sn[VEC];
        load_vec<VEC>(row + off, x0);
        load_vec<VEC>(row + off + half, x1);
        if (bias != nullptr) {
            float b0[VEC], b1[VEC];
            load_vec<VEC>(bias + off, b0);
            load_vec<VEC>(bias + off + half, b1);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                x0[j] = x0[j] + b0[j];
                x1[j] = x1[j] + b1[j];
            }
        }
        load_vec<VEC>(cos_row + i, cs);
        load_vec<VEC>(sin_row + i, sn);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            lo[j] = x0[j] * cs[j] - x1[j] * sn[j];
            hi[j] = x1[j] * cs[j] + x0[j] * sn[j];
        }
    };

    if (a.q != nullptr && item < a.heads * hq) {
        const int head = item / hq;
        const int i = VEC * (item - head * hq);
        const int off = head * a.head_dim + i;
        float *qrow = a.q + tok * hidden;
        float lo[VEC], hi[VEC];
        rotate(qrow, a.q_bias != nullptr ? a.q_bias + (size_t)layer * hidden : nullptr, off, i, lo, hi);
        store_vec<VEC>(qrow + off, lo);
        store_vec<VEC>(qrow + off + half, hi);
        if (a.q_half != nullptr) {
            store_vec_f16<VEC>(a.q_half + tok * hidden + off, lo);
            store_vec_f16<VEC>(a.q_half + tok * hidden + off + half, hi);
        }
    }

    const size_t slot = ((size_t)sl * a.ctx + pos) * kv_dim;
    if (item < a.kv_heads * hq) {
        const int head = item / hq;
        const int i = VEC * (item - head * hq);
        const int off = head * a.head_dim + i;
        float *krow = a.k + tok * kv_dim;
        float lo[VEC], hi[VEC];
        rotate(krow, a.k_bias != nullptr ? a.k_bias + (size_t)layer * kv_dim : nullptr, off, i, lo, hi);
        if (a.write_back) {
            store_vec<VEC>(krow + off, lo);
            store_vec<VEC>(krow + off + half, hi);
        }
        store_vec_f16<VEC>(a.key_cache + slot + off, lo);
        store_vec_f16<VEC>(a.key_cache + slot + off + half, hi);
    }

    if (item < kv_dim / VEC) {
        const int off = VEC * item;
        float *vrow = a.v + tok * kv_dim;
        float x[VEC];
        load_vec<VEC>(vrow + off, x);
        if (a.v_bias != nullptr) {
            float bv[VEC];
            load_vec<VEC>(a.v_bias + (size_t)layer * kv_dim + off, bv);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                x[j] = x[j] + bv[j];
            }
            if (a.write_back) {
                store_vec<VEC>(vrow + off, x);
            }
        }
        store_vec_f16<VEC>(a.value_cache + slot + off, x);
    }
}

// The kernel's vector width: 4 when every row piece it touches is 16-byte
// aligned (fp32) / 8-byte aligned (fp16), else 1.
int rope_append_vec(const RopeAppendArgs &a) {
    auto al = [](const void *p, uintptr_t n) { return p == nullptr || ((uintptr_t)p % n) == 0; };
    const bool ok = a.head_dim % 8 == 0 && al(a.q, 16) && al(a.k, 16) && al(a.v, 16) && al(a.q_bias, 16) &&
                    al(a.k_bias, 16) && al(a.v_bias, 16) && al(a.cos_t, 16) && al(a.sin_t, 16) &&
                    al(a.key_cache, 8) && al(a.value_cache, 8) && al(a.q_half, 8);
    return ok ? 4 : 1;
}

te_status launch_rope_append(const RopeAppendArgs &a, size_t seqs, size_t layers, size_t tokens, hipStream_t st) {
    const int vec = rope_append_vec(a);
    const size_t half = (size_t)a.head_dim / 2;
    size_t items = (a.q != nullptr ? (size_t)a.heads : 0) * half;
    items = std::max(items, (size_t)a.kv_heads * a.head_dim) / (size_t)vec;
    const dim3 grid((unsigned)((items + 255) / 256), (unsigned)tokens, (unsigned)(seqs * layers));
    if (vec == 4) {
        rope_kv_append_kernel<4><<<grid, 256, 0, st>>>(a);
    } else {
        rope_kv_append_kernel<1><<<grid, 256, 0, st>>>(a);
    }
    return te_hip::launch_status();
}

// Fused prefill step's append and V^T in one launch: for the chunk's
// positions [base, base + tokens) of every (seq*layer), bias + RoPE of k and
// bias of v with rope_kv_append_kernel's operations (so the fp16 cache rows
// are the same bits), and the V^T rows of those positions as
// value_transpose_kernel writes them (zeros at [end, end8), end8 = end
// rounded up to 8 within the row pitch).  One workgroup per 32 aligned
// positions, KV head and seq*layer; the tile's v rows meet in LDS and leave
// as 16-byte chunks of 8 positions per dim row.
struct KvAppendVtArgs {
    const float *k;  // [sl][tokens][kv_heads][D]
    const float *v;
    const float *k_bias;  // [layers][kv_heads*D] or null
    const float *v_bias;
    const float *cos_t;
    const float *sin_t;
    f16 *key_cache;    // [sl][ctx][kv_heads][D]
    f16 *value_cache;
    f16 *value_t;      // [sl][kv_heads][D][ctx_pad]
    int layers;
    int tokens;
    int base;
    int end8;
    int ctx;
    int ctx_pad;
    int kv_heads;
};

template <int D>
__global__ __launch_bounds__(256) void kv_append_vt_kernel(KvAppendVtArgs a) {
    constexpr int P = 32;  // positions per workgroup (64 measured 5 % slower at 512 tokens)
    constexpr int HALF = D / 2;
    __shared__ __attribute__((aligned(16))) f16 tile[P][D + 8];
    const int first = a.base;
    const int end = a.base + a.tokens;
    const int p0 = (first & ~(P - 1)) + P * (int)blockIdx.x;
    const int h = blockIdx.y;
    const int sl = blockIdx.z;
    const int layer = sl % a.layers;
    const int kv_dim = a.kv_heads * D;
    const float *kb = a.k_bias != nullptr ? a.k_bias + (size_t)layer * kv_dim + h * D : nullptr;
    const float *vb = a.v_bias != nullptr ? a.v_bias + (size_t)layer * kv_dim + h * D : nullptr;
    // Every load of the workgroup is issued before the first store (the
    // stores could alias the loads as far as the compiler knows, so loads
    // placed after a store would wait for it): one round of memory latency.
    // k items: pairs (i, i + D/2), four per item; v items: 8 values.  A
    // position outside the chunk loads the chunk's first row and stores
    // nothing (its V^T tile entry is zero).
    constexpr int KI = P * (HALF / 4) / 256;  // k items per thread
    constexpr int VI = P * (D / 8) / 256;     // v items per thread
    static_assert(KI * 256 == P * (HALF / 4) && VI * 256 == P * (D / 8), "items tile the workgroup");
    float4 k0[KI], k1[KI], c4[KI], s4[KI], kb0[KI], kb1[KI];
    float4 v0[VI], v1[VI], vb0[VI], vb1[VI];
#pragma unroll
    for (int u = 0; u < KI; ++u) {
        const int idx = threadIdx.x + 256 * u;
        const int r = idx / (HALF / 4);
        const int i = 4 * (idx % (HALF / 4));
        const int p = p0 + r;
        const int pl = p >= first && p < end ? p : first;
        const float *krow = a.k + ((size_t)sl * a.tokens + (pl - first)) * kv_dim + h * D;
        k0[u] = *reinterpret_cast<const float4 *>(krow + i);
        k1[u] = *reinterpret_cast<const float4 *>(krow + i + HALF);
        c4[u] = *reinterpret_cast<const float4 *>(a.cos_t + (size_t)pl * HALF + i);
        s4[u] = *reinterpret_cast<const float4 *>(a.sin_t + (size_t)pl * HALF + i);
        if (kb != nullptr) {
            kb0[u] = *reinterpret_cast<const float4 *>(kb + i);
            kb1[u] = *reinterpret_cast<const float4 *>(kb + i + HALF);
        }
    }
#pragma unroll
    for (int u = 0; u < VI; ++u) {
        const int idx = threadIdx.x + 256 * u;
        const int r = idx / (D / 8);
        const int cq = idx % (D / 8);
        const int p = p0 + r;
        const int pl = p >= first && p < end ? p : first;
        const float *vrow = a.v + ((size_t)sl * a.tokens + (pl - first)) * kv_dim + h * D + 8 * cq;
        v0[u] = *reinterpret_cast<const float4 *>(vrow);
        v1[u] = *reinterpret_cast<const float4 *>(vrow + 4);
        if (vb != nullptr) {
            vb0[u] = *reinterpret_cast<const float4 *>(vb + 8 * cq);
            vb1[u] = *reinterpret_cast<const float4 *>(vb + 8 * cq + 4);
        }
    }
    // k: bias, rotation, fp16 (rope_kv_append_kernel's operation order)
#pragma unroll
    for (int u = 0; u < KI; ++u) {
        const int idx = threadIdx.x + 256 * u;
        const int r = idx / (HALF / 4);
        const int i = 4 * (idx % (HALF / 4));
        const int p = p0 + r;
        if (p < first || p >= end) {
            continue;
        }
        float x0[4] = {k0[u].x, k0[u].y, k0[u].z, k0[u].w};
        float x1[4] = {k1[u].x, k1[u].y, k1[u].z, k1[u].w};
        if (kb != nullptr) {
            const float b0[4] = {kb0[u].x, kb0[u].y, kb0[u].z, kb0[u].w};
            const float b1[4] = {kb1[u].x, kb1[u].y, kb1[u].z, kb1[u].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x0[j] = x0[j] + b0[j];
                x1[j] = x1[j] + b1[j];
            }
        }
        const float cs[4] = {c4[u].x, c4[u].y, c4[u].z, c4[u].w};
        const float sn[4] = {s4[u].x, s4[u].y, s4[u].z, s4[u].w};
        f16x4 lo, hi;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo[j] = (f16)(x0[j] * cs[j] - x1[j] * sn[j]);
            hi[j] = (f16)(x1[j] * cs[j] + x0[j] * sn[j]);
        }
        f16 *dst = a.key_cache + ((size_t)sl * a.ctx + p) * kv_dim + h * D;
        *reinterpret_cast<f16x4 *>(dst + i) = lo;
        *reinterpret_cast<f16x4 *>(dst + i + HALF) = hi;
    }
    // v: bias, fp16, into the cache and the LDS tile (zeros outside the chunk)
#pragma unroll
    for (int u = 0; u < VI; ++u) {
        const int idx = threadIdx.x + 256 * u;
        const int r = idx / (D / 8);
        const int cq = idx % (D / 8);
        const int p = p0 + r;
        f16x8 val = {0, 0, 0, 0, 0, 0, 0, 0};
        if (p >= first && p < end) {
            float x[8] = {v0[u].x, v0[u].y, v0[u].z, v0[u].w, v1[u].x, v1[u].y, v1[u].z, v1[u].w};
            if (vb != nullptr) {
                const float b[8] = {vb0[u].x, vb0[u].y, vb0[u].z, vb0[u].w, vb1[u].x, vb1[u].y, vb1[u].z, vb1[u].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    x[j] = x[j] + b[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                val[j] = (f16)x[j];
            }
            *reinterpret_cast<f16x8 *>(a.value_cache + ((size_t)sl * a.ctx + p) * kv_dim + h * D + 8 * cq) = val;
        }
        *reinterpret_cast<f16x8 *>(&tile[r][8 * cq]) = val;
    }
    __syncthreads();
    f16 *dst = a.value_t + ((size_t)sl * a.kv_heads + h) * (size_t)D * a.ctx_pad;
    for (int idx = threadIdx.x; idx < D * (P / 8); idx += 256) {
        const int i = idx / (P / 8);
        const int pc = idx % (P / 8);
        const int pa = p0 + 8 * pc;
        if (pa >= a.end8 || pa + 8 <= first) {
            continue;
        }
        f16x8 val;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            val[j] = tile[8 * pc + j][i];
        }
        f16 *row = dst + (size_t)i * a.ctx_pad + pa;
        if (pa >= first && pa + 8 <= a.end8) {
            *reinterpret_cast<f16x8 *>(row) = val;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (pa + j >= first && pa + j < a.end8) {
                    row[j] = val[j];
                }
            }
        }
    }
}

// In-place rotation of `heads` rows with one cos/sin row (te_rope_f32).
__global__ __launch_bounds__(256) void rope_rows_kernel(float *values, int heads, int head_dim,
                                                        const float *cos_row, const float *sin_row) {
    const int item = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = head_dim >> 1;
    if (item >= heads * half) {
        return;
    }
    const int head = item / half;
    const int i = item - head * half;
    float *row = values + (size_t)head * head_dim;
    const float x0 = row[i];
    const float x1 = row[i + half];
    const float c = cos_row[i];
    const float sn = sin_row[i];
    row[i] = x0 * c - x1 * sn;
    row[i + half] = x1 * c + x0 * sn;
}

}  // namespace

namespace te_hip {

te_status launch_kv_append(const float *k, const float *v, const float *k_bias, const float *v_bias,
                           const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
                           uint16_t *value_cache, size_t seqs, size_t layers, size_t tokens, size_t base_position,
                           size_t context_tokens, size_t kv_heads, size_t head_dim, hipStream_t stream) {
    RopeAppendArgs a = {};
    a.q = nullptr;
    a.k = const_cast<float *>(k);  // read only: write_back = 0
    a.v = const_cast<float *>(v);
    a.k_bias = k_bias;
    a.v_bias = v_bias;
    a.cos_t = rope_cos;
    a.sin_t = rope_sin;
    a.key_cache = reinterpret_cast<f16 *>(key_cache);
    a.value_cache = reinterpret_cast<f16 *>(value_cache);
    a.write_back = 0;
    a.layers = (int)layers;
    a.tokens = (int)tokens;
    a.ctx = (int)context_tokens;
    a.heads = 0;
    a.kv_heads = (int)kv_heads;
    a.head_dim = (int)head_dim;
    for (size_t s = 0; s < seqs; ++s) {
        a.base[s] = (int)base_position;
    }
    return launch_rope_append(a, seqs, layers, tokens, stream);
}

te_status launch_kv_append_vt(const float *k, const float *v, const float *k_bias, const float *v_bias,
                              const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
                              uint16_t *value_cache, uint16_t *value_t, size_t sl_count, size_t layers,
                              size_t tokens, size_t base_position, size_t context_tokens, size_t ctx_pad,
                              size_t kv_heads, size_t head_dim, hipStream_t stream) {
    if ((head_dim != 64 && head_dim != 128) || tokens == 0 || ctx_pad < base_position + tokens ||
        ctx_pad % 64 != 0 || sl_count > 65535 || kv_heads > 65535) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    KvAppendVtArgs a = {};
    a.k = k;
    a.v = v;
    a.k_bias = k_bias;
    a.v_bias = v_bias;
    a.cos_t = rope_cos;
    a.sin_t = rope_sin;
    a.key_cache = reinterpret_cast<f16 *>(key_cache);
    a.value_cache = reinterpret_cast<f16 *>(value_cache);
    a.value_t = reinterpret_cast<f16 *>(value_t);
    a.layers = (int)layers;
    a.tokens = (int)tokens;
    a.base = (int)base_position;
    const size_t end = base_position + tokens;
    a.end8 = (int)std::min((end + 7) / 8 * 8, ctx_pad);
    a.ctx = (int)context_tokens;
    a.ctx_pad = (int)ctx_pad;
    a.kv_heads = (int)kv_heads;
    const size_t tiles = ((size_t)a.end8 - (base_position & ~(size_t)31) + 31) / 32;
    const dim3 grid((unsigned)tiles, (unsigned)kv_heads, (unsigned)sl_count);
    if (head_dim == 128) {
        kv_append_vt_kernel<128><<<grid, 256, 0, stream>>>(a);
    } else {
        kv_append_vt_kernel<64><<<grid, 256, 0, stream>>>(a);
    }
    return launch_status();
}

te_status launch_rope_rows(float *values, size_t heads, size_t head_dim, const float *cos_row,
                           const float *sin_row, hipStream_t stream) {
    const size_t items = heads * (head_dim / 2);
    const unsigned blocks = (unsigned)((items + 255) / 256);
    rope_rows_kernel<<<blocks, 256, 0, stream>>>(values, (int)heads, (int)head_dim, cos_row, sin_row);
    return launch_status();
}

}  // namespace te_hip

extern "C" te_status te_hip_rope_kv_append_f16(
    float *q, float *k, float *v,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *q_half,
    size_t seqs, size_t layers, size_t tokens,
    const size_t *base_positions, size_t base_position,
    size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
    void *stream) {
    if (q == nullptr || k == nullptr || v == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || seqs == 0 || layers == 0 || tokens == 0 ||
        context_tokens == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || (head_dim % 2) != 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (seqs > TE_HIP_MAX_SEQS || head_dim > 256 || heads * head_dim > (1u << 20) ||
        context_tokens > (1u << 30) || tokens > 65535 || seqs * layers > 65535) {
        return TE_STATUS_UNSUPPORTED;
    }
    RopeAppendArgs a;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t base = base_positions != nullptr ? base_positions[s] : base_position;
        if (base > context_tokens || tokens > context_tokens - base) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
        a.base[s] = (int)base;
    }
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_bias = q_bias;
    a.k_bias = k_bias;
    a.v_bias = v_bias;
    a.cos_t = rope_cos;
    a.sin_t = rope_sin;
    a.key_cache = reinterpret_cast<f16 *>(key_cache);
    a.value_cache = reinterpret_cast<f16 *>(value_cache);
    a.q_half = reinterpret_cast<f16 *>(q_half);
    a.write_back = 1;
    a.layers = (int)layers;
    a.tokens = (int)tokens;
    a.ctx = (int)context_tokens;
    a.heads = (int)heads;
    a.kv_heads = (int)kv_heads;
    a.head_dim = (int)head_dim;
    return launch_rope_append(a, seqs, layers, tokens, te_hip::as_stream(stream));
}
