// GQA decode attention over the fp16 KV cache: split-K ("flash-decoding")
// kernel + combine kernel, and the fp32-cache variant behind te_attention_decode_f32.
//
// Numerical contract: the reference te_attention_decode_f32 (ops.c:323-395)
// -- scores q.k/sqrt(d) over positions 0..pos, softmax, PV -- in fp32.  Here
// the softmax is online (base-2, exp2 of log2e-prescaled scores) per chunk and
// merged exactly by the combine kernel; every accumulation is fp32.
//
// Split-K kernel, one single-wave workgroup per (chunk of positions, kv_head,
// seq*layer).  The wave streams its chunk 32 positions at a time for all
// `group` (= heads/kv_heads <= 16) query heads of its KV head at once, so every
// K/V element is read from HBM exactly once per query token (the GQA sharing of
// te_attention_flash_gqa_f32_kernel, metal_kernels.metal.inc:3209-3372):
//
//   S^T[32 pos x 16 heads] = K[32 x D] . Q^T[D x 16]          (fp16 MFMA 16x16x32)
//   O^T[D x 16 heads]     += V^T[D x 32 pos] . P^T[32 x 16]    (fp16 MFMA 16x16x32)
//
// q and P are fp32 values split into hi+lo fp16 pairs (two MFMAs each), so the
// only rounding relative to an fp32 computation is the fp16 cache itself.
// Lane mapping (l = lane, g = l/16, c = l%16):
//   K, V loads: each instruction reads 4 whole cache rows (16 lanes x 16 B =
//               one 256-byte row for D = 128), non-temporal:
//               K rows p0 + 4j + g, V rows p0 + kmap(g,j),
//               kmap(g,j) = 16(j/4)+4g+(j%4), dims NT*c .. NT*c+NT-1.
//   K operand : the K tile is written row-major to a padded LDS stage and read
//               back as A-operand rows 16h + c, dims 8g + 32kk.
//   V operand : an in-register 8 x NT transpose of the V rows gives the A
//               operand of output tile t = dims {NT*m + t}.
//   S^T result: lane holds head c at positions 4g+r (+16h) -- exactly the
//               P^T B-operand layout of the PV MFMA for kmap, so P never moves.
//   O^T result: lane holds head c, dims 4NT*g .. 4NT*g + 4NT - 1, written
//               straight to the partial with 16-byte stores.
// The next tile's loads are issued before the current tile is consumed (two
// register tiles, 32 KB in flight per wave).  The chunk length is chosen from
// the total tile count (about 3.5 single-wave workgroups per CU, chunks evened
// out per stream), which also balances ragged sequence lengths.
//
// HBM bytes per (seq, layer), the roofline unit: 2*(pos+1)*kv_heads*D*2 B of
// K/V + heads*D*4 B of q; partials add (chunks*heads*(D+2)*4 B) x2.
#include "te_hip_common.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>

namespace {

constexpr int kTile = 32;               // positions per MFMA step
constexpr int kTargetWaves2PerCU = 7;    // split-K waves per CU the chunking aims at, x2 (3.5)
constexpr int kMaxCombineChunks = 4096;

struct DecodeArgs {
    const float *query;
    const f16 *key_cache;
    const f16 *value_cache;
    float *part_o;   // [SL][heads][max_chunks][D]
    float *part_ml;  // [SL][heads][max_chunks][2]  (m in log2 units, l)
    // Fused decode step only (bias + RoPE of q and of the new k, fp16 append of
    // the new k/v at `positions[s]`); unused by the plain split-K kernel.
    const float *k_new;   // [SL][kv_heads][D]
    const float *v_new;   // [SL][kv_heads][D]
    const float *q_bias;  // [layers][heads*D] or null
    const float *k_bias;  // [layers][kv_heads*D] or null
    const float *v_bias;  // [layers][kv_heads*D] or null
    const float *rope_cos;
    const float *rope_sin;
    f16 *key_cache_w;
    f16 *value_cache_w;
    int layers;
    int ctx;
    int heads;
    int kv_heads;
    int group;
    int chunk;
    int max_chunks;
    float qscale;    // log2(e)/sqrt(D)
    int positions[TE_HIP_MAX_SEQS];
};

template <int D>
struct VRow;
template <>
struct VRow<128> {
    typedef f16x8 type;
};
template <>
struct VRow<64> {
    typedef f16x4 type;
};

// A 32-position tile of one KV head as loaded from HBM.  Both K and V are read
// the same way: each load instruction covers 4 cache rows, 16 lanes x NT
// halves per row (a whole D*2-byte head row, contiguous), non-temporal since
// the stream is read once.
//   k[j]: row 4j + g,           dims NT*c .. NT*c + NT-1  (row-major staging)
//   v[j]: row kmap(g, j),       dims NT*c .. NT*c + NT-1  (PV A-operand order)
template <int D>
struct DecodeTile {
    typename VRow<D>::type k[8];
    typename VRow<D>::type v[8];
};

// LDS staging of the K tile, transposed into the QK^T A-operand layout:
// 32 rows of D halves padded by 8 halves (16 bytes), which makes the
// 16-row x 16-byte operand reads bank-conflict free.
template <int D>
struct KStage {
    static constexpr int kPitch = D + 8;
    f16 rows[32 * kPitch];
};

template <int D>
__device__ __forceinline__ void decode_load_tile(DecodeTile<D> &t, const f16 *kbase, const f16 *vbase,
                                                 int row_stride, int p0, int last, int g, int c) {
    constexpr int NT = D / 16;
    typedef typename VRow<D>::type vrow_t;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int kr = min(p0 + 4 * j + g, last);
        t.k[j] = __builtin_nontemporal_load(reinterpret_cast<const vrow_t *>(kbase + kr * row_stride + NT * c));
        const int vr = min(p0 + 16 * (j >> 2) + 4 * g + (j & 3), last);
        t.v[j] = __builtin_nontemporal_load(reinterpret_cast<const vrow_t *>(vbase + vr * row_stride + NT * c));
    }
}

// One 32-position step of the online softmax + both MFMA products.
template <int D>
__device__ __forceinline__ void decode_consume_tile(const DecodeTile<D> &t, KStage<D> &ks,
                                                    const f16x8 (&qh)[D / 32], const f16x8 (&ql)[D / 32], int p0,
                                                    int pos, int g, int c, float &m, float &l,
                                                    f32x4 (&acc)[D / 16]) {
    constexpr int NT = D / 16;
    constexpr int KK = D / 32;
    constexpr int P = KStage<D>::kPitch;
    typedef typename VRow<D>::type vrow_t;
    // K tile -> LDS (row-major) -> A operand rows 16h + c, dims 8g + 32kk.
    // One wave per workgroup: the LDS unit serves this wave's writes before its
    // later reads; the barrier only orders the compiler.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        *reinterpret_cast<vrow_t *>(&ks.rows[(4 * j + g) * P + NT * c]) = t.k[j];
    }
    __syncthreads();
    f32x4 sacc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        sacc[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const f16x8 ka = *reinterpret_cast<const f16x8 *>(&ks.rows[(16 * h + c) * P + 8 * g + 32 * kk]);
            sacc[h] = mfma16x16x32(ka, qh[kk], sacc[h]);
            sacc[h] = mfma16x16x32(ka, ql[kk], sacc[h]);
        }
    }
    __syncthreads();  // the next tile's staging writes come after these reads
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int p = p0 + 16 * (j >> 2) + 4 * g + (j & 3);
        const float x = sacc[j >> 2][j & 3];
        sv[j] = p <= pos ? x : -INFINITY;
        mx = fmaxf(mx, sv[j]);
    }
    mx = wave_xor_max16_32(mx);
    const float m_new = fmaxf(m, mx);
    const float alpha = fast_exp2(m - m_new);
    m = m_new;
    f16x8 ph, pl;
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float p = fast_exp2(sv[j] - m_new);
        psum += p;
        f16 hi, lo;
        split_f16(p, hi, lo);
        ph[j] = hi;
        pl[j] = lo;
    }
    l = l * alpha + psum;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        f16x8 va;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            va[j] = t.v[j][tt];
        }
        acc[tt] = acc[tt] * alpha;
        acc[tt] = mfma16x16x32(va, ph, acc[tt]);
        acc[tt] = mfma16x16x32(va, pl, acc[tt]);
    }
}

// Fused decode step, in the workgroup whose chunk holds the query position:
// bias + RoPE of the new token's k and bias of its v for this KV head, rounded
// to fp16 into the cache slot, with the same operation order as
// rope_kv_append_kernel (FP contraction off), then fenced so the tile loads
// that follow see it.  Only this workgroup reads that position.
template <int D>
__device__ __forceinline__ void decode_append_new_token(const DecodeArgs &a, int sl, int layer, int kvh, int pos,
                                                        int lane) {
#pragma clang fp contract(off)
    constexpr int HALF = D / 2;
    const int kv_dim = a.kv_heads * D;
    const float *kn = a.k_new + ((size_t)sl * a.kv_heads + kvh) * D;
    const float *vn = a.v_new + ((size_t)sl * a.kv_heads + kvh) * D;
    const size_t slot = ((size_t)sl * a.ctx + pos) * kv_dim + (size_t)kvh * D;
    const float *cos_row = a.rope_cos + (size_t)pos * HALF;
    const float *sin_row = a.rope_sin + (size_t)pos * HALF;
    for (int i = lane; i < HALF; i += 64) {
        float x0 = kn[i];
        float x1 = kn[i + HALF];
        if (a.k_bias != nullptr) {
            x0 = x0 + a.k_bias[(size_t)layer * kv_dim + kvh * D + i];
            x1 = x1 + a.k_bias[(size_t)layer * kv_dim + kvh * D + i + HALF];
        }
        const float cs = cos_row[i];
        const float sn = sin_row[i];
        a.key_cache_w[slot + i] = (f16)(x0 * cs - x1 * sn);
        a.key_cache_w[slot + i + HALF] = (f16)(x1 * cs + x0 * sn);
    }
    for (int i = lane; i < D; i += 64) {
        float x = vn[i];
        if (a.v_bias != nullptr) {
            x = x + a.v_bias[(size_t)layer * kv_dim + kvh * D + i];
        }
        a.value_cache_w[slot + i] = (f16)x;
    }
    // The workgroup is this one wave and the only reader of the slot, so a
    // workgroup-scope release/acquire orders the stores before the tile loads;
    // an agent-scope fence would also write back and invalidate the XCD's L2.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Bias + RoPE of this lane's q values in registers (fused step).  Lane (g, c)
// holds dims 8g + 32kk + j of head c; the rotation partner of dim d < D/2 is
// d + D/2, held by the same lane at kk + KK/2.
template <int D>
__device__ __forceinline__ void decode_rope_q(const DecodeArgs &a, float (&xs)[D / 32][8], int layer, int head,
                                              int pos, int g) {
#pragma clang fp contract(off)
    constexpr int KK = D / 32;
    constexpr int HALF = D / 2;
    if (a.q_bias != nullptr) {
        const float *qb = a.q_bias + ((size_t)layer * a.heads + head) * D;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xs[kk][j] = xs[kk][j] + qb[8 * g + 32 * kk + j];
            }
        }
    }
    const float *cos_row = a.rope_cos + (size_t)pos * HALF;
    const float *sin_row = a.rope_sin + (size_t)pos * HALF;
#pragma unroll
    for (int kk = 0; kk < KK / 2; ++kk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = 8 * g + 32 * kk + j;
            const float cs = cos_row[i];
            const float sn = sin_row[i];
            const float x0 = xs[kk][j];
            const float x1 = xs[kk + KK / 2][j];
            xs[kk][j] = x0 * cs - x1 * sn;
            xs[kk + KK / 2][j] = x1 * cs + x0 * sn;
        }
    }
}

template <int D, bool FUSED>
__global__ __launch_bounds__(64, 2) void decode_splitk_f16_kernel(DecodeArgs a) {
    constexpr int NT = D / 16;  // output tiles over head_dim; also dims per lane in V loads
    constexpr int KK = D / 32;  // MFMA K-steps over head_dim for QK^T

    const int chunk_id = blockIdx.x;
    const int kvh = blockIdx.y;
    const int sl = blockIdx.z;
    const int s = sl / a.layers;
    const int pos = a.positions[s];
    const int c0 = chunk_id * a.chunk;
    if (c0 > pos) {
        return;  // this sequence has fewer chunks than the longest one
    }
    const int c1 = min(c0 + a.chunk, pos + 1);
    const int last = c1 - 1;  // loads are clamped to the chunk; positions > pos are masked
    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const int c = lane & 15;

    const int row_stride = a.kv_heads * D;
    const size_t sl_base = (size_t)sl * a.ctx * row_stride + (size_t)kvh * D;
    const f16 *kbase = a.key_cache + sl_base;
    const f16 *vbase = a.value_cache + sl_base;

    if (FUSED && c1 == pos + 1) {
        decode_append_new_token<D>(a, sl, sl - s * a.layers, kvh, pos, lane);
    }

    DecodeTile<D> ta, tb;
    decode_load_tile<D>(ta, kbase, vbase, row_stride, c0, last, g, c);

    // Q^T operand, hi/lo split, pre-scaled into the log2 domain (loads overlap tile 0).
    f16x8 qh[KK], ql[KK];
    {
        const bool head_ok = c < a.group;
        const int head = kvh * a.group + (head_ok ? c : 0);
        const float *qrow = a.query + ((size_t)sl * a.heads + head) * D;
        float xs[KK][8];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const float4 x0 = *reinterpret_cast<const float4 *>(qrow + 8 * g + 32 * kk);
            const float4 x1 = *reinterpret_cast<const float4 *>(qrow + 8 * g + 32 * kk + 4);
            xs[kk][0] = x0.x;
            xs[kk][1] = x0.y;
            xs[kk][2] = x0.z;
            xs[kk][3] = x0.w;
            xs[kk][4] = x1.x;
            xs[kk][5] = x1.y;
            xs[kk][6] = x1.z;
            xs[kk][7] = x1.w;
        }
        if (FUSED) {
            decode_rope_q<D>(a, xs, sl - s * a.layers, head, pos, g);
        }
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = head_ok ? xs[kk][j] * a.qscale : 0.0f;
                f16 hi, lo;
                split_f16(x, hi, lo);
                qh[kk][j] = hi;
                ql[kk][j] = lo;
            }
        }
    }

    float m = -INFINITY;
    float l = 0.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // Two register tiles, ping-pong: the loads of step n+1 are in flight while
    // step n is consumed.  Every branch below is wave-uniform.
    __shared__ KStage<D> kstage;
    int p0 = c0;
    for (;;) {
        if (p0 + 32 < c1) {
            decode_load_tile<D>(tb, kbase, vbase, row_stride, p0 + 32, last, g, c);
        }
        decode_consume_tile<D>(ta, kstage, qh, ql, p0, pos, g, c, m, l, acc);
        p0 += 32;
        if (p0 >= c1) {
            break;
        }
        if (p0 + 32 < c1) {
            decode_load_tile<D>(ta, kbase, vbase, row_stride, p0 + 32, last, g, c);
        }
        decode_consume_tile<D>(tb, kstage, qh, ql, p0, pos, g, c, m, l, acc);
        p0 += 32;
        if (p0 >= c1) {
            break;
        }
    }

    l = wave_xor_sum16_32(l);
    if (c < a.group) {
        const size_t pidx = ((size_t)sl * a.heads + (size_t)kvh * a.group + c) * a.max_chunks + chunk_id;
        float *po = a.part_o + pidx * D + 4 * NT * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int t = 0; t < NT; t += 4) {
                float4 v;
                v.x = acc[t][r];
                v.y = acc[t + 1][r];
                v.z = acc[t + 2][r];
                v.w = acc[t + 3][r];
                *reinterpret_cast<float4 *>(po + NT * r + t) = v;
            }
        }
        if (g == 0) {
            a.part_ml[pidx * 2] = m;
            a.part_ml[pidx * 2 + 1] = l;
        }
    }
}

struct CombineArgs {
    const float *part_o;
    const float *part_ml;
    float *out;  // [SL][heads][D]
    int layers;
    int heads;
    int head_dim;
    int chunk;
    int max_chunks;
    int positions[TE_HIP_MAX_SEQS];
};

// Merge of two softmax partials (m, l, o) in the log2 domain; a side whose max
// equals the merged max keeps weight 1, so -inf maxima never form -inf - -inf.
__device__ __forceinline__ void merge_partial(float &m, float &l, float4 &o, float mi, float li, float4 oi) {
    const float mn = fmaxf(m, mi);
    const float sa = m == mn ? 1.0f : fast_exp2(m - mn);
    const float sb = mi == mn ? 1.0f : fast_exp2(mi - mn);
    m = mn;
    l = l * sa + li * sb;
    o.x = o.x * sa + oi.x * sb;
    o.y = o.y * sa + oi.y * sb;
    o.z = o.z * sa + oi.z * sb;
    o.w = o.w * sa + oi.w * sb;
}

// Combine for the split-K f16 path (head_dim D in {64, 128}), one 256-thread
// workgroup per (head, seq*layer): thread (grp, col) owns the float4 column col
// of the head and the chunks grp, grp + G, ...; it merges them online, so all of
// its partial loads are independent and in flight together.  The G group
// results are then merged through LDS.  Same result as decode_combine_kernel
// up to fp32 rounding of the rescale factors.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(CombineArgs a) {
    constexpr int COLS = D / 4;
    constexpr int G = 256 / COLS;
    const int h = blockIdx.x;
    const int sl = blockIdx.y;
    const int s = sl / a.layers;
    const int n_chunks = (a.positions[s] + a.chunk) / a.chunk;  // ceil((pos+1)/chunk)
    const size_t base = ((size_t)sl * a.heads + h) * a.max_chunks;
    const int tid = threadIdx.x;
    const int col = tid % COLS;
    const int grp = tid / COLS;
    const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml) + base;
    const float4 *po = reinterpret_cast<const float4 *>(a.part_o + base * D) + col;

    float m = -INFINITY;
    float l = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (int i = grp; i < n_chunks; i += G) {
        const float2 mli = ml[i];
        const float4 oi = po[(size_t)i * COLS];
        merge_partial(m, l, o, mli.x, mli.y, oi);
    }

    __shared__ float4 o_s[G][COLS];
    __shared__ float m_s[G];
    __shared__ float l_s[G];
    o_s[grp][col] = o;
    if (col == 0) {
        m_s[grp] = m;
        l_s[grp] = l;
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
        for (int k = 1; k < G; ++k) {
            merge_partial(m, l, o, m_s[k], l_s[k], o_s[k][col]);
        }
        const float inv = l > 0.0f ? 1.0f / l : 1.0f;
        o.x *= inv;
        o.y *= inv;
        o.z *= inv;
        o.w *= inv;
        reinterpret_cast<float4 *>(a.out + ((size_t)sl * a.heads + h) * D)[col] = o;
    }
}

// One workgroup per (head, seq*layer): out = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c.
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgs a) {
    const int h = blockIdx.x;
    const int sl = blockIdx.y;
    const int s = sl / a.layers;
    const int n_chunks = (a.positions[s] + a.chunk) / a.chunk;  // ceil((pos+1)/chunk)
    const size_t base = ((size_t)sl * a.heads + h) * a.max_chunks;
    const float *ml = a.part_ml + base * 2;
    const int tid = threadIdx.x;

    __shared__ float red[256];
    __shared__ float wts[kMaxCombineChunks];

    float mx = -INFINITY;
    for (int i = tid; i < n_chunks; i += 256) {
        mx = fmaxf(mx, ml[2 * i]);
    }
    red[tid] = mx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) {
            red[tid] = fmaxf(red[tid], red[tid + w]);
        }
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float ls = 0.0f;
    for (int i = tid; i < n_chunks; i += 256) {
        const float w = fast_exp2(ml[2 * i] - M);
        wts[i] = w;
        ls += w * ml[2 * i + 1];
    }
    red[tid] = ls;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) {
            red[tid] += red[tid + w];
        }
        __syncthreads();
    }
    const float L = red[0];
    const float inv = L > 0.0f ? 1.0f / L : 1.0f;
    const float *po = a.part_o + base * a.head_dim;
    float *o = a.out + ((size_t)sl * a.heads + h) * a.head_dim;
    for (int d = tid; d < a.head_dim; d += 256) {
        float acc = 0.0f;
        for (int i = 0; i < n_chunks; ++i) {
            acc += wts[i] * po[(size_t)i * a.head_dim + d];
        }
        o[d] = acc * inv;
    }
}

// fp32-cache decode for te_attention_decode_f32 (host-pointer API, any head_dim):
// one wave per (chunk of positions, head).  The chunk is walked in blocks of
// kF32Block positions whose scores sit in LDS; each block is a two-pass
// softmax merged online into the partial (m, l, o), where o lives in the
// partial itself (each lane owns dims lane, lane + 64, ...).  The partial is
// then merged by decode_combine_kernel.
constexpr int kF32Block = 512;

__global__ __launch_bounds__(64) void decode_f32_chunk_kernel(const float *query, const float *key_cache,
                                                              const float *value_cache, int pos, int heads,
                                                              int kv_heads, int head_dim, float qscale, int chunk,
                                                              int max_chunks, float *part_o, float *part_ml) {
    const int chunk_id = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    const int c0 = chunk_id * chunk;
    const int c1 = min(c0 + chunk, pos + 1);
    const int kvh = h / (heads / kv_heads);
    const float *q = query + (size_t)h * head_dim;
    const size_t pidx = (size_t)h * max_chunks + chunk_id;
    float *po = part_o + pidx * head_dim;
    __shared__ float sc[kF32Block];

    float m = -INFINITY;
    float l = 0.0f;
    for (int b0 = c0; b0 < c1; b0 += kF32Block) {
        const int b1 = min(b0 + kF32Block, c1);
        float mx = -INFINITY;
        for (int p = b0 + lane; p < b1; p += 64) {
            const float *kr = key_cache + ((size_t)p * kv_heads + kvh) * head_dim;
            float dot = 0.0f;
            for (int i = 0; i < head_dim; ++i) {
                dot = fmaf(q[i], kr[i], dot);
            }
            const float x = dot * qscale;
            sc[p - b0] = x;
            mx = fmaxf(mx, x);
        }
        for (int off = 32; off > 0; off >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        }
        const float mn = fmaxf(m, mx);
        const float alpha = m == mn ? 1.0f : fast_exp2(m - mn);  // first block: o and l are still 0
        float ls = 0.0f;
        for (int p = b0 + lane; p < b1; p += 64) {
            const float e = fast_exp2(sc[p - b0] - mn);
            sc[p - b0] = e;
            ls += e;
        }
        for (int off = 32; off > 0; off >>= 1) {
            ls += __shfl_xor(ls, off, 64);
        }
        l = l * alpha + ls;
        m = mn;
        __syncthreads();
        for (int d = lane; d < head_dim; d += 64) {
            float acc = b0 == c0 ? 0.0f : po[d] * alpha;
            for (int p = b0; p < b1; ++p) {
                acc = fmaf(sc[p - b0], value_cache[((size_t)p * kv_heads + kvh) * head_dim + d], acc);
            }
            po[d] = acc;
        }
        __syncthreads();  // the next block's scores overwrite sc
    }
    if (lane == 0) {
        part_ml[pidx * 2] = m;
        part_ml[pidx * 2 + 1] = l;
    }
}

bool valid_positions(const size_t *positions, size_t position, size_t seqs, size_t context_tokens,
                     size_t *max_position) {
    size_t mx = 0;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t p = positions != nullptr ? positions[s] : position;
        if (p >= context_tokens) {
            return false;
        }
        if (p > mx) {
            mx = p;
        }
    }
    *max_position = mx;
    return true;
}

te_status check_decode_args(const size_t *positions, size_t position, size_t seqs, size_t layers,
                            size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
                            size_t *max_position) {
    if (seqs == 0 || layers == 0 || context_tokens == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 ||
        (heads % kv_heads) != 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (seqs > TE_HIP_MAX_SEQS || (head_dim != 64 && head_dim != 128) || heads / kv_heads > 16 ||
        seqs * layers > 65535 || kv_heads > 65535 || context_tokens * kv_heads * head_dim >= ((size_t)1 << 31)) {
        return TE_STATUS_UNSUPPORTED;  // per-(seq, layer) cache offsets are 32-bit in the kernel
    }
    if (!valid_positions(positions, position, seqs, context_tokens, max_position)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return TE_STATUS_OK;
}

}  // namespace

namespace te_hip {

int device_compute_units() {
    static const int cus = [] {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
            prop.multiProcessorCount > 0) {
            return prop.multiProcessorCount;
        }
        (void)hipGetLastError();
        return 256;  // MI355X
    }();
    return cus;
}

DecodeGeometry decode_geometry(const size_t *positions, size_t position, size_t seqs, size_t layers,
                               size_t kv_heads) {
    // The chunk is the total number of 32-position tiles over all (seq,
    // layer, kv_head) streams divided by a target of 3.5 single-wave
    // workgroups per CU (at least two tiles, so the prefetch pipeline has
    // work), then evened out so the longest stream's chunks are equal.
    // Measured on MI355X (3B at 2K/8K/32K, 1.5B at 128K, 7B ragged x8): HBM
    // efficiency is highest with about that many concurrent streams -- the
    // 8 resident waves per CU the registers allow run 4-8 % slower -- and a
    // short last chunk per stream costs a partly idle tail.  Balancing on the
    // total rather than the longest sequence keeps ragged batches even.
    // A launch too small to fill the GPU (one layer's decode step) takes
    // one-tile chunks instead where those stay within 3/4 of a workgroup per
    // CU and two-tile chunks would exceed the kGemvMergeMaxChunks partials the
    // decode-layer flow merges in its Wo projection (so that flow runs the
    // merge launch either way): 3B Q4_0 decode token at 1K / 2K / 3K 1,309 ->
    // 1,279 / ~1,318 -> ~1,293 / 1,332 -> 1,316 us; at 4K (one workgroup per
    // CU) 1,327 against 1,344, so it stops below.
    // TE_HIP_DECODE_CHUNK (a multiple of 32) overrides the choice.
    DecodeGeometry g;
    size_t max_n = 0, total_tiles = 0;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t n = (positions != nullptr ? positions[s] : position) + 1;
        max_n = n > max_n ? n : max_n;
        total_tiles += layers * kv_heads * ((n + kTile - 1) / kTile);
    }
    const size_t target = (size_t)device_compute_units() * kTargetWaves2PerCU / 2;
    const size_t max_tiles = (max_n + kTile - 1) / kTile;
    const bool one_tile = total_tiles * 4 <= (size_t)device_compute_units() * 3 &&
                          (max_tiles + 1) / 2 > (size_t)kGemvMergeMaxChunks;
    const size_t min_tiles = one_tile ? 1 : 2;
    size_t tiles = (total_tiles + target - 1) / target;
    if (tiles < min_tiles) {
        tiles = min_tiles;
    }
    const size_t n_longest = (max_tiles + tiles - 1) / tiles;  // chunks of the longest stream
    tiles = (max_tiles + n_longest - 1) / n_longest;           // equal chunks for it
    if (tiles < min_tiles) {
        tiles = min_tiles;
    }
    size_t chunk = tiles * kTile;
    const char *env = getenv("TE_HIP_DECODE_CHUNK");
    if (env != nullptr) {
        const long v = strtol(env, nullptr, 10);
        if (v >= kTile && v % kTile == 0 && v <= (1 << 24)) {
            chunk = (size_t)v;
        }
    }
    while ((max_n + chunk - 1) / chunk > (size_t)kMaxCombineChunks) {
        chunk *= 2;
    }
    g.chunk = (int)chunk;
    g.max_chunks = (int)((max_n + chunk - 1) / chunk);
    return g;
}

size_t decode_workspace_bytes(const DecodeGeometry &g, size_t seqs, size_t layers, size_t heads,
                              size_t head_dim) {
    const size_t parts = seqs * layers * heads * (size_t)g.max_chunks;
    return parts * head_dim * sizeof(float) + parts * 2 * sizeof(float);
}

size_t decode_chunks_bound(size_t max_position, size_t layers, size_t kv_heads) {
    // decode_geometry gives the longest stream n_longest = ceil(M / t0) chunks,
    // M = its 32-position tiles, t0 = max(2, ceil(T / target)) and T >= layers *
    // kv_heads * M the total tiles; the later steps only lengthen the chunk.  So
    // n_longest <= ceil(M / 2) and n_longest <= ceil(target / (layers * kv_heads)),
    // both non-decreasing in M.  One-tile chunks give n_longest = M where
    // layers * kv_heads * M <= T <= 3/4 of the CUs: at most
    // min(M, 3/4 CUs / (layers * kv_heads)), also non-decreasing in M.  With
    // TE_HIP_DECODE_CHUNK the count is ceil(n / chunk) before the doubling
    // that keeps it <= kMaxCombineChunks.
    const size_t max_n = max_position + 1;
    const size_t m_tiles = (max_n + kTile - 1) / kTile;
    const char *env = getenv("TE_HIP_DECODE_CHUNK");
    if (env != nullptr) {
        const long v = strtol(env, nullptr, 10);
        if (v >= kTile && v % kTile == 0 && v <= (1 << 24)) {
            return std::min((max_n + (size_t)v - 1) / (size_t)v, (size_t)kMaxCombineChunks);
        }
    }
    const size_t target = (size_t)device_compute_units() * kTargetWaves2PerCU / 2;
    const size_t streams = layers * kv_heads;
    const size_t b = std::max(std::min((m_tiles + 1) / 2, (target + streams - 1) / streams),
                              std::min(m_tiles, (size_t)device_compute_units() * 3 / 4 / streams));
    return std::min(std::max(b, (size_t)1), (size_t)kMaxCombineChunks);
}

int f32_decode_chunk(size_t position) {
    // Positions per workgroup of te_attention_decode_f32: kF32Block, doubled
    // until the chunks fit the combine kernel's weight cache.
    const size_t n = position + 1;
    size_t chunk = kF32Block;
    while ((n + chunk - 1) / chunk > (size_t)kMaxCombineChunks) {
        chunk *= 2;
    }
    return (int)chunk;
}

te_status launch_decode_f32(const float *query, const float *key_cache, const float *value_cache,
                            size_t position, size_t heads, size_t kv_heads, size_t head_dim, float *out,
                            float *part_o, float *part_ml, hipStream_t stream) {
    const int chunk = f32_decode_chunk(position);
    const int max_chunks = (int)((position + (size_t)chunk) / (size_t)chunk);
    const float qscale = TE_LOG2E / sqrtf((float)head_dim);
    decode_f32_chunk_kernel<<<dim3(max_chunks, (unsigned)heads), 64, 0, stream>>>(
        query, key_cache, value_cache, (int)position, (int)heads, (int)kv_heads, (int)head_dim, qscale, chunk,
        max_chunks, part_o, part_ml);
    te_status st = launch_status();
    if (st != TE_STATUS_OK) {
        return st;
    }
    CombineArgs c;
    c.part_o = part_o;
    c.part_ml = part_ml;
    c.out = out;
    c.layers = 1;
    c.heads = (int)heads;
    c.head_dim = (int)head_dim;
    c.chunk = chunk;
    c.max_chunks = max_chunks;
    c.positions[0] = (int)position;
    decode_combine_kernel<<<dim3((unsigned)heads, 1), 256, 0, stream>>>(c);
    return launch_status();
}

}  // namespace te_hip

extern "C" size_t te_hip_attention_decode_workspace_bytes(const size_t *positions, size_t position, size_t seqs,
                                                          size_t layers, size_t heads, size_t kv_heads,
                                                          size_t head_dim) {
    if (seqs == 0 || seqs > TE_HIP_MAX_SEQS || layers == 0 || heads == 0 || kv_heads == 0 || head_dim == 0) {
        return 0;
    }
    // Sized by the chunk bound of the largest position, not by the chunking
    // of these exact positions: the bound never decreases with the position,
    // so a workspace sized for one position serves every smaller one.
    size_t max_position = 0;
    for (size_t s = 0; s < seqs; ++s) {
        const size_t p = positions != nullptr ? positions[s] : position;
        max_position = p > max_position ? p : max_position;
    }
    te_hip::DecodeGeometry g;
    g.chunk = 0;
    g.max_chunks = (int)te_hip::decode_chunks_bound(max_position, layers, kv_heads);
    return te_hip::decode_workspace_bytes(g, seqs, layers, heads, head_dim);
}

extern "C" te_status te_hip_attention_decode_chunking(const size_t *positions, size_t position, size_t seqs,
                                                      size_t layers, size_t kv_heads, int fp32_cache,
                                                      size_t *chunk, size_t *chunks) {
    if (chunk == nullptr || chunks == nullptr || seqs == 0 || layers == 0 || kv_heads == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (fp32_cache != 0) {
        if (seqs != 1 || layers != 1 || position == SIZE_MAX) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
        *chunk = (size_t)te_hip::f32_decode_chunk(position);
        *chunks = (position + *chunk) / *chunk;
        return TE_STATUS_OK;
    }
    if (seqs > TE_HIP_MAX_SEQS) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const te_hip::DecodeGeometry g = te_hip::decode_geometry(positions, position, seqs, layers, kv_heads);
    *chunk = (size_t)g.chunk;
    *chunks = (size_t)g.max_chunks;
    return TE_STATUS_OK;
}

namespace {

// Shared by the plain split-K entry point and the fused decode step; `fused`
// carries the new token (k_new/v_new non-null) and the RoPE tables.
te_status launch_splitk(const DecodeArgs &fused, bool is_fused, const float *query, const uint16_t *key_cache,
                        const uint16_t *value_cache, const size_t *positions, size_t position, size_t seqs,
                        size_t layers, size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
                        void *workspace, size_t workspace_bytes, void *stream) {
    if (query == nullptr || key_cache == nullptr || value_cache == nullptr || workspace == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t max_position = 0;
    te_status st = check_decode_args(positions, position, seqs, layers, context_tokens, heads, kv_heads,
                                     head_dim, &max_position);
    if (st != TE_STATUS_OK) {
        return st;
    }
    const te_hip::DecodeGeometry geo = te_hip::decode_geometry(positions, position, seqs, layers, kv_heads);
    if (workspace_bytes < te_hip::decode_workspace_bytes(geo, seqs, layers, heads, head_dim)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    DecodeArgs a = fused;
    a.query = query;
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_cache = reinterpret_cast<const f16 *>(value_cache);
    const size_t parts = seqs * layers * heads * (size_t)geo.max_chunks;
    a.part_o = static_cast<float *>(workspace);
    a.part_ml = a.part_o + parts * head_dim;
    a.layers = (int)layers;
    a.ctx = (int)context_tokens;
    a.heads = (int)heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)(heads / kv_heads);
    a.chunk = geo.chunk;
    a.max_chunks = geo.max_chunks;
    a.qscale = TE_LOG2E / sqrtf((float)head_dim);
    for (size_t s = 0; s < seqs; ++s) {
        a.positions[s] = (int)(positions != nullptr ? positions[s] : position);
    }
    const dim3 grid((unsigned)geo.max_chunks, (unsigned)kv_heads, (unsigned)(seqs * layers));
    hipStream_t strm = te_hip::as_stream(stream);
    if (head_dim == 128) {
        if (is_fused) {
            decode_splitk_f16_kernel<128, true><<<grid, 64, 0, strm>>>(a);
        } else {
            decode_splitk_f16_kernel<128, false><<<grid, 64, 0, strm>>>(a);
        }
    } else {
        if (is_fused) {
            decode_splitk_f16_kernel<64, true><<<grid, 64, 0, strm>>>(a);
        } else {
            decode_splitk_f16_kernel<64, false><<<grid, 64, 0, strm>>>(a);
        }
    }
    return te_hip::launch_status();
}

}  // namespace

extern "C" te_status te_hip_attention_decode_splitk_f16(
    const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    void *workspace, size_t workspace_bytes, void *stream) {
    DecodeArgs none = {};
    return launch_splitk(none, false, query, key_cache, value_cache, positions, position, seqs, layers,
                         context_tokens, heads, kv_heads, head_dim, workspace, workspace_bytes, stream);
}

extern "C" te_status te_hip_attention_decode_step_splitk_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    void *workspace, size_t workspace_bytes, void *stream) {
    if (k_new == nullptr || v_new == nullptr || rope_cos == nullptr || rope_sin == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    DecodeArgs f = {};
    f.k_new = k_new;
    f.v_new = v_new;
    f.q_bias = q_bias;
    f.k_bias = k_bias;
    f.v_bias = v_bias;
    f.rope_cos = rope_cos;
    f.rope_sin = rope_sin;
    f.key_cache_w = reinterpret_cast<f16 *>(key_cache);
    f.value_cache_w = reinterpret_cast<f16 *>(value_cache);
    return launch_splitk(f, true, query, key_cache, value_cache, positions, position, seqs, layers,
                         context_tokens, heads, kv_heads, head_dim, workspace, workspace_bytes, stream);
}

extern "C" te_status te_hip_attention_decode_step_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream) {
    if (out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = te_hip_attention_decode_step_splitk_f16(
        query, k_new, v_new, q_bias, k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache, positions,
        position, seqs, layers, context_tokens, heads, kv_heads, head_dim, workspace, workspace_bytes, stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return te_hip_attention_decode_combine(positions, position, seqs, layers, heads, kv_heads, head_dim, out,
                                           workspace, workspace_bytes, stream);
}

extern "C" te_status te_hip_attention_decode_combine(
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t heads, size_t kv_heads, size_t head_dim,
    float *out, const void *workspace, size_t workspace_bytes, void *stream) {
    if (out == nullptr || workspace == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    // The combine reads no cache: validate against the smallest cache the
    // positions could belong to.
    size_t max_position = 0;
    for (size_t s = 0; s < seqs && s < TE_HIP_MAX_SEQS; ++s) {
        const size_t p = positions != nullptr ? positions[s] : position;
        max_position = p > max_position ? p : max_position;
    }
    te_status st = check_decode_args(positions, position, seqs, layers, max_position + 1, heads, kv_heads,
                                     head_dim, &max_position);
    if (st != TE_STATUS_OK) {
        return st;
    }
    const te_hip::DecodeGeometry geo = te_hip::decode_geometry(positions, position, seqs, layers, kv_heads);
    if (workspace_bytes < te_hip::decode_workspace_bytes(geo, seqs, layers, heads, head_dim)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    CombineArgs c;
    const size_t parts = seqs * layers * heads * (size_t)geo.max_chunks;
    c.part_o = static_cast<const float *>(workspace);
    c.part_ml = c.part_o + parts * head_dim;
    c.out = out;
    c.layers = (int)layers;
    c.heads = (int)heads;
    c.head_dim = (int)head_dim;
    c.chunk = geo.chunk;
    c.max_chunks = geo.max_chunks;
    for (size_t s = 0; s < seqs; ++s) {
        c.positions[s] = (int)(positions != nullptr ? positions[s] : position);
    }
    const dim3 grid((unsigned)heads, (unsigned)(seqs * layers));
    if (head_dim == 128) {
        decode_merge_kernel<128><<<grid, 256, 0, te_hip::as_stream(stream)>>>(c);
    } else {
        decode_merge_kernel<64><<<grid, 256, 0, te_hip::as_stream(stream)>>>(c);
    }
    return te_hip::launch_status();
}

// ---- te_hip_attention_decode_step_noalloc_f16 -------------------------------
//
// The fused decode step for callers that cannot allocate (code under graph
// capture, serving loops that forbid hipMalloc): its split-K partials go to a
// file-scope device array instead of a caller workspace.  Every GPU the library
// runs on holds its own copy of `scratch` until the process ends; host code
// reaches it only through the address hipGetSymbolAddress returns for the
// current device (the array's name is a host-side stand-in, not a device
// address).  All calls on one GPU share the array, so calls that overlap on
// one GPU race; stream-ordered calls are safe (each call's merge reads only
// partials its own split-K launch wrote, so nothing needs clearing).
namespace {

static __device__ __align__(256) unsigned char scratch[TE_HIP_DECODE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxScratchDevices] = {};

// Address of `scratch` on the current device, looked up once per device.
te_status scratch_address(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return TE_STATUS_RUNTIME_ERROR;
    }
    if (dev < 0 || dev >= kMaxScratchDevices) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return TE_STATUS_RUNTIME_ERROR;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TE_STATUS_OK;
}

}  // namespace

extern "C" te_status te_hip_attention_decode_step_noalloc_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *stream) {
    if (query == nullptr || k_new == nullptr || v_new == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t max_position = 0;
    te_status st = check_decode_args(positions, position, seqs, layers, context_tokens, heads, kv_heads, head_dim,
                                     &max_position);
    if (st != TE_STATUS_OK) {
        return st;
    }
    // The partials this exact call writes (not the position-monotone bound
    // the workspace query reports) must fit the array.
    const te_hip::DecodeGeometry geo = te_hip::decode_geometry(positions, position, seqs, layers, kv_heads);
    const size_t need = te_hip::decode_workspace_bytes(geo, seqs, layers, heads, head_dim);
    if (need > (size_t)TE_HIP_DECODE_NOALLOC_SCRATCH_BYTES) {
        return TE_STATUS_UNSUPPORTED;
    }
    void *ws = nullptr;
    if ((st = scratch_address(&ws)) != TE_STATUS_OK) {
        return st;
    }
    return te_hip_attention_decode_step_f16(query, k_new, v_new, q_bias, k_bias, v_bias, rope_cos, rope_sin,
                                            key_cache, value_cache, positions, position, seqs, layers,
                                            context_tokens, heads, kv_heads, head_dim, out, ws,
                                            (size_t)TE_HIP_DECODE_NOALLOC_SCRATCH_BYTES, stream);
}
