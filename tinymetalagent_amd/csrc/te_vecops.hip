// Decode-layer vector operations around attention: the quantized matrix-vector
// product of the projections (GGUF F32 / Q4_0 / Q8_0 weights resident in HBM),
// RMSNorm, SwiGLU, residual add and argmax.  HIP twins of te_metal_matvec_f32
// (reference c/src/metal_backend.h:13-22) and of the CPU functions
// te_model_matvec_f32 / te_rmsnorm_f32 / te_swiglu_f32 / te_add_f32 /
// te_argmax_f32 (c/src/ops.c:177-269, :272-293, :397-433).
//
// Matvec.  Row r of a [rows][cols] tensor is cols/32 blocks stored back to back
// (ops.c:15-21): Q4_0 = f16 scale d + 16 bytes whose low nibbles are elements
// 0-15 and high nibbles 16-31, value (code - 8) * d; Q8_0 = f16 d + 32 int8
// codes, value code * d; F32 rows are plain floats.  Quantized rows with an even
// block count (every Qwen2.5 shape) take the pair kernels below: the input is
// rounded per 32-value block to 22-bit integers and the products are summed
// exactly with integer dot instructions.  F32 rows and odd block counts take
// matvec_kernel: one wave owns R rows, lane l takes blocks l, l + 64, ... and
// converts each code to float (one v_cvt_f32_ubyteN + one FMA per element,
// with the offset factored out: d * (sum_j u_j x_j - off sum_j x_j)).
// Summation order differs from the reference's sequential loop: the results
// agree within the rounding bounds stated with each kernel, not bit for bit.
//
// HBM bytes per launch (the roofline unit): rows * row_bytes + cols * 4 + rows * 4.
#include "te_hip_common.h"

#include <float.h>
#include <math.h>
#include <string.h>

namespace {

constexpr uint32_t kGgmlF32 = 0;
constexpr uint32_t kGgmlQ4_0 = 2;
constexpr uint32_t kGgmlQ8_0 = 8;
constexpr int kMatvecWaves = 4;
constexpr int kPairWaves = 12;                     // pair kernel: one 12-wave workgroup per CU (3 per SIMD)
constexpr int kPairThreads = 64 * kPairWaves;
constexpr int kStageBatch = 4;                      // input float4 loads in flight per thread while staging
constexpr int kMergeChunks = te_hip::kGemvMergeMaxChunks;  // split-K partials a merge staging takes per head
constexpr size_t kMaxPairLdsBytes = 160 * 1024;     // staged digit planes (gfx950 LDS per CU)
constexpr size_t kPairLdsBytes = 13 * 16;           // LDS per block pair: 12 uint4 of digit planes + scales
constexpr int kStreamChunks = 10;                   // streamed kernel: 16-byte chunk loads per lane per tile
constexpr size_t kStreamTileBytes = kStreamChunks * 1024;  // its LDS tile buffer per wave
constexpr int kWideStreamChunks = 12;
constexpr int kShortStreamChunks = 4;               // one-row-per-group tiles of at most 4 KB                // Q8_0 rows of 10-12 KB, one row per tile
template <uint32_t TYPE>
constexpr int kDigitPlanes = TYPE == kGgmlQ4_0 ? 6 : 3;  // balanced base-16 / base-256 digits of 22-bit X

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        v += __shfl_xor(v, o, 64);
    }
    return v;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(f16, (uint16_t)bits);
}

// dwords w[0..N] starting at the 4-byte boundary at or below `p` (p even):
// returns the block's bytes as N dwords after its 2-byte scale, plus the scale.
template <int N>
__device__ __forceinline__ uint32_t load_block(const unsigned char *p, uint32_t (&q)[N]) {
    const size_t addr = (size_t)p;
    const uint32_t *w = reinterpret_cast<const uint32_t *>(addr & ~(size_t)3);
    uint32_t d;
    if ((addr & 2u) == 0) {
        // scale = low half of w[0]; data bytes start at +2: q[k] = w[k] >> 16 | w[k+1] << 16;
        // the last data pair sits in the low half of w[N], read as 16 bits
        uint32_t v[N + 1];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            v[k] = w[k];
        }
        v[N] = *reinterpret_cast<const uint16_t *>(w + N);
        d = v[0] & 0xffffu;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            q[k] = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2);
        }
    } else {
        // scale = high half of w[0]; data bytes are w[1..N]
        d = w[0] >> 16;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            q[k] = w[k + 1];
        }
    }
    return d;
}

// acc + sum_k byte_k(u) * x[k]; each byte -> float is one v_cvt_f32_ubyteN
__device__ __forceinline__ float dot_u8x4(uint32_t u, const float *x, float acc) {
    acc = fmaf((float)(u & 0xffu), x[0], acc);
    acc = fmaf((float)((u >> 8) & 0xffu), x[1], acc);
    acc = fmaf((float)((u >> 16) & 0xffu), x[2], acc);
    acc = fmaf((float)(u >> 24), x[3], acc);
    return acc;
}

template <uint32_t TYPE, int R>
__global__ __launch_bounds__(64 * kMatvecWaves) void matvec_kernel(const unsigned char *weights, const float *input,
                                                                 int cols, int rows, size_t row_bytes, float *out) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * kMatvecWaves + (int)(threadIdx.x >> 6)) * R;
    if (row0 >= rows) {
        return;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        acc[r] = 0.0f;
    }
    if (TYPE == kGgmlF32) {
        // lane takes float4 columns lane, lane + 64, ...; cols % 4 == 0 (host check)
        const int c4 = cols / 4;
        for (int j = lane; j < c4; j += 64) {
            const float4 x = reinterpret_cast<const float4 *>(input)[j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (row0 + r < rows) {
                    const float4 w = reinterpret_cast<const float4 *>(weights + (size_t)(row0 + r) * row_bytes)[j];
                    acc[r] = fmaf(w.x, x.x, acc[r]);
                    acc[r] = fmaf(w.y, x.y, acc[r]);
                    acc[r] = fmaf(w.z, x.z, acc[r]);
                    acc[r] = fmaf(w.w, x.w, acc[r]);
                }
            }
        }
    } else {
        constexpr int BLOCK_BYTES = TYPE == kGgmlQ4_0 ? 18 : 34;
        constexpr int QW = TYPE == kGgmlQ4_0 ? 4 : 8;  // data dwords per block
        const int blocks = cols / 32;
        for (int b = lane; b < blocks; b += 64) {
            float x[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float4 v = reinterpret_cast<const float4 *>(input + 32 * b)[k];
                x[4 * k] = v.x;
                x[4 * k + 1] = v.y;
                x[4 * k + 2] = v.z;
                x[4 * k + 3] = v.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                xs += x[j];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (row0 + r < rows) {
                    uint32_t q[QW];
                    const uint32_t dbits =
                        load_block<QW>(weights + (size_t)(row0 + r) * row_bytes + (size_t)b * BLOCK_BYTES, q);
                    float s = 0.0f;
                    float off;
                    if (TYPE == kGgmlQ4_0) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            s = dot_u8x4(q[k] & 0x0f0f0f0fu, x + 4 * k, s);         // elements 4k .. 4k+3
                            s = dot_u8x4((q[k] >> 4) & 0x0f0f0f0fu, x + 16 + 4 * k, s);  // 16+4k ..
                        }
                        off = 8.0f;
                    } else {
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            s = dot_u8x4(q[k] ^ 0x80808080u, x + 4 * k, s);
                        }
                        off = 128.0f;
                    }
                    acc[r] = fmaf(f16_bits_to_f32(dbits), fmaf(-off, xs, s), acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < rows) {
            out[row0 + r] = v;
        }
    }
}

// Quantized rows with an even block count (every Qwen2.5 shape), as exact
// integer dot products.
//
// Input staging.  The workgroup scales each 32-value block of the input by a
// power of two, 2^e with e = 22 - ceil(log2 max|x|), so the block's largest
// magnitude lies in [2^21, 2^22), and rounds it to integers X (error <= 2^-22 of
// the block max; the block's own 2^-e is kept).  X is written in balanced
// digits: six base-16 digits in [-8, 7] (Q4_0) or three base-256 digits in
// [-128, 127] (Q8_0), X = sum_t D_t 16^t (256^t).  Digit plane t of a block is
// packed like the weights: for Q4_0 dword k holds elements 4k..4k+3 in its even
// nibbles and 16+4k..19+4k in its odd ones (the Q4_0 byte layout); for Q8_0 dword
// k holds elements 4k..4k+3, one per byte.  A block's planes are 24 dwords; a
// pair is 13 float4 in LDS (12 of planes, then the two 2^-e), and 13 is odd, so
// 16 lanes reading 16 consecutive pairs hit 16 distinct bank groups.
//
// Product.  Q4_0 codes n become signed nibbles n - 8 = n ^ 8; Q8_0 codes are
// signed bytes already.  v_dot8c_i32_i4 / v_dot4c_i32_i8 of a weight dword and a
// digit dword accumulate S_t = sum_j w_j D_tj exactly; per block |S_t| <= 2^11
// (Q4_0) / 2^19 (Q8_0), so the planes combine in int32 into two parts below
// 2^24 (Q4_0: S0 + 16 S1 + 256 S2 and S3 + 16 S4 + 256 S5; Q8_0: S0 + 256 S1
// and S2), which convert to float exactly (Q4_0) or with one rounding (Q8_0)
// and meet in one FMA.  The block adds d * 2^-e * that sum to the row.  Every
// element costs 6 / 8 (Q4_0) or 3 / 4 (Q8_0) integer dot instructions.

// Input pre-operations applied while staging (the decode layer fuses them
// into its projections): kPreNone stages x; kPreRmsNorm is the reference
// te_rmsnorm_f32 (ops.c:272-293), x * scale * w with scale = 1 / sqrtf(mean(x^2)
// + eps), squares summed in fp64 (here per workgroup over the whole vector):
// it stages x * w and multiplies each row's sum by the scale, which is then
// known, at the end (the scale is common to every element, and the staging
// does not wait for the workgroup's reduction); kPreSwiGLU stages silu(x) * x2
// as te_swiglu_f32 (ops.c:397-406); kPreMerge stages the attention output
// merged from its split-K partials (the decode layer's Wo projection; the sum
// decode_merge_kernel forms, see merged_slice).
enum : int { kPreNone = 0, kPreRmsNorm = 1, kPreSwiGLU = 2, kPreMerge = 3 };

struct StageInput {
    const float *x;
    const float *x2;      // kPreSwiGLU: the up projection
    const float *norm_w;  // kPreRmsNorm: the norm weight
    float eps;            // kPreRmsNorm
    // kPreMerge: the split-K partials of one (seq, layer), o [heads][max_chunks][head_dim]
    // and (m, l) [heads][max_chunks][2], chunks [0, n_chunks) of each head
    const float *part_o;
    const float *part_ml;
    int n_chunks;
    int max_chunks;
    int head_dim;
};

// The first kStageBatch float4 slices of a thread's input, loaded before the
// kernel issues its weight loads: loads complete in issue order, so slices
// loaded after a tile's weights would wait for all of them.  Slice u is float4
// u * blockDim.x + threadIdx.x of x and of the operand its pre-operation needs
// (the norm weight or the up projection); zero past the input.
struct StagePrefetch {
    float4 x[kStageBatch];
    float4 y[kStageBatch];
    // kPreMerge: the partials of the thread's one slice, chunk c of its head
    // (m = -inf, l = 0, o = 0 past n_chunks)
    float4 mo[kMergeChunks];
    float2 mml[kMergeChunks];
};

template <int PRE>
__device__ __forceinline__ void stage_prefetch(const StageInput &in, int n4, StagePrefetch &pf) {
    if constexpr (PRE == kPreMerge) {
        // one slice per thread (the launch checks n4 <= threads): float4 i of
        // the attention output is dims 4 (i % (D / 4)) .. of head i / (D / 4)
        const int i = (int)threadIdx.x;
        const int q4 = in.head_dim / 4;
        const int base = (i < n4 ? i / q4 : 0) * in.max_chunks;
        const float4 *o4 = reinterpret_cast<const float4 *>(in.part_o);
        const float2 *ml2 = reinterpret_cast<const float2 *>(in.part_ml);
#pragma unroll
        for (int c = 0; c < kMergeChunks; ++c) {
            const bool live = i < n4 && c < in.n_chunks;
            pf.mml[c] = live ? ml2[base + c] : make_float2(-__builtin_inff(), 0.0f);
            pf.mo[c] = live ? o4[(size_t)(base + c) * q4 + i % q4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            pf.x[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            pf.y[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        return;
    }
    const float4 *y4 = reinterpret_cast<const float4 *>(PRE == kPreRmsNorm ? in.norm_w : in.x2);
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
        const int i = u * (int)blockDim.x + (int)threadIdx.x;
        const bool in_range = i < n4;
        pf.x[u] = in_range ? reinterpret_cast<const float4 *>(in.x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        pf.y[u] = PRE != kPreNone && in_range ? y4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// One lane's value DPP-moved (a 64-bit value as its two halves).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}

// The wave's sum of v, in every lane: within each 16-lane row by quad
// exchanges 1 and 2, the half-row mirror and the row mirror, then the four row
// sums in row order.
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x141>(v);
    v += dpp_f64<0x140>(v);
    auto row = [&](int lane) {
        return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                                __builtin_amdgcn_readlane(__double2loint(v), lane));
    };
    return ((row(0) + row(16)) + row(32)) + row(48);
}

// RMSNorm's scale 1 / sqrtf(mean(x^2) + eps) of in.x[0, n) (n % 4 == 0), in
// two halves around the workgroup barrier that ends the staging, so that the
// staging itself does not wait for it: rms_partial sums the squares of each
// thread's slices i = threadIdx.x + k * blockDim.x in fp64 (the first
// kStageBatch from the prefetched registers) and stores each wave's sum to
// LDS; rms_scale, after the barrier, adds the waves' sums in wave order.
__shared__ double rms_part[kPairWaves];

__device__ __forceinline__ void rms_partial(const StageInput &in, int n, const StagePrefetch &pf) {
    double ss = 0.0;
    auto add = [&](const float4 v) {
        ss += (double)v.x * v.x;
        ss += (double)v.y * v.y;
        ss += (double)v.z * v.z;
        ss += (double)v.w * v.w;
    };
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
        add(pf.x[u]);  // zero past the input
    }
    for (int i = kStageBatch * (int)blockDim.x + (int)threadIdx.x; i < n / 4; i += blockDim.x) {
        add(reinterpret_cast<const float4 *>(in.x)[i]);
    }
    ss = wave_sum_f64(ss);
    if ((threadIdx.x & 63) == 0) {
        rms_part[threadIdx.x >> 6] = ss;
    }
}

__device__ __forceinline__ float rms_scale(const StageInput &in, int n) {
    double total = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
        total += rms_part[w];
    }
    return 1.0f / sqrtf((float)(total / (double)n) + in.eps);
}

// Cross-lane moves of the staging below as DPP operand modifiers (VALU, no LDS
// round trip).  octet_max: the max over the aligned 8-lane group (quad
// exchanges 1 and 2, then the half-row mirror, lane i <-> 7 - i).
__device__ __forceinline__ float octet_max(float m) {
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    return fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
}

// Lane i + 4's value in lanes i with i % 16 < 12 (row shift left by 4).
__device__ __forceinline__ uint32_t from_lane_plus4(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);
}

// The thread's slice of the attention output from its head's split-K
// partials: M = max_c m_c, then sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c
// over the chunks in order (chunk 0 always holds position 0, so M is finite);
// the quotient as decode_merge_kernel forms it (1 / l, 1 for l = 0).  Its
// rounding differs from that kernel's pairwise merges by a few ulps.
__device__ __forceinline__ float4 merged_slice(const StagePrefetch &pf) {
    float mx = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < kMergeChunks; ++c) {
        mx = fmaxf(mx, pf.mml[c].x);
    }
    float l = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int c = 0; c < kMergeChunks; ++c) {
        const float w = pf.mml[c].x == -__builtin_inff() ? 0.0f : fast_exp2(pf.mml[c].x - mx);
        l += w * pf.mml[c].y;
        o.x += w * pf.mo[c].x;
        o.y += w * pf.mo[c].y;
        o.z += w * pf.mo[c].z;
        o.w += w * pf.mo[c].w;
    }
    const float inv = l > 0.0f ? 1.0f / l : 1.0f;
    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// Stage the (pre-operated) input's digit planes and block scales (layout above)
// into LDS for the whole workgroup; the caller synchronises.  Coalesced float4
// reads, kStageBatch per thread issued before any is used.  Float4 i is block
// i / 8 (of pair i / 16), slice i % 8; a block's 8 slices sit in 8 consecutive
// lanes, which share its max and its digit dwords (pairs * 16 is a multiple of
// 8, so those lanes agree on the bound).
template <uint32_t TYPE, int PRE>
__device__ __forceinline__ void stage_digit_planes(const StageInput &in, int pairs, uint32_t *xs_lds,
                                                   const StagePrefetch &pf) {
    const int nthreads = (int)blockDim.x;
    const int n4 = pairs * 16;
    if (PRE == kPreRmsNorm) {
        rms_partial(in, n4 * 4, pf);
    }
    auto pre_op = [&](float4 x, const float4 y) {
        if (PRE == kPreRmsNorm) {
            // x * w: the launch's epilogue multiplies each row's sum by the scale
            x = make_float4(x.x * y.x, x.y * y.y, x.z * y.z, x.w * y.w);
        } else if (PRE == kPreSwiGLU) {
            x = make_float4(x.x / (1.0f + expf(-x.x)) * y.x, x.y / (1.0f + expf(-x.y)) * y.y,
                            x.z / (1.0f + expf(-x.z)) * y.z, x.w / (1.0f + expf(-x.w)) * y.w);
        }
        return x;
    };
    // digit planes of one batch of slices v[u] = float4 base + u * nthreads + threadIdx.x
    auto digitize = [&](const int base, const float4 (&v)[kStageBatch]) {
        // waves whose slice of a batch row starts past the input skip it (uniform branch)
        const int wave_first = base + (int)(threadIdx.x & ~63u);
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            if (wave_first + u * nthreads >= n4) {
                break;
            }
            const int i = base + u * nthreads + (int)threadIdx.x;
            const float xv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            // the block's max |x| over its lane octet, +inf when any value is not finite
            float m = fmaxf(fmaxf(fabsf(xv[0]), fabsf(xv[1])), fmaxf(fabsf(xv[2]), fabsf(xv[3])));
            if (!(isfinite(xv[0]) && isfinite(xv[1]) && isfinite(xv[2]) && isfinite(xv[3]))) {
                m = __builtin_inff();
            }
            m = octet_max(m);
            const bool bad = m == __builtin_inff();
            int ex = 0;
            frexpf(m, &ex);  // m < 2^ex <= 2 m
            // blocks whose max is below 2^-104 keep an absolute error of 2^-127
            const int e = bad || m == 0.0f ? 0 : min(22 - ex, 126);
            const int f = i & 7;
            // Balanced digits from plain ones: with B = sum_t 8 * 16^t (Q4_0) or
            // sum_t 128 * 256^t (Q8_0), Y = X + B lies in [0, 2^24), and digit t of X is
            // (digit t of Y) - 8 (or - 128), whose 4- (8-) bit two's complement is
            // digit t of Y with its top bit flipped, the flips done on whole dwords.
            uint32_t y[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int xq = bad ? 0 : (int)rintf(ldexpf(xv[j], e));  // |xq| <= 2^22
                y[j] = (uint32_t)(xq + (TYPE == kGgmlQ4_0 ? 0x888888 : 0x808080));
            }
            // Byte k of the four values into byte planes yb[k] (byte j = byte k of
            // y[j]) by v_perm_b32: bytes 0 and 1, then byte 2, of value pairs, then
            // the pairs' halves (selector byte 0x0c is a zero byte).
            const uint32_t p01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
            const uint32_t p23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
            const uint32_t q01 = __builtin_amdgcn_perm(y[1], y[0], 0x0C0C0602u);
            const uint32_t q23 = __builtin_amdgcn_perm(y[3], y[2], 0x0C0C0602u);
            const uint32_t yb[3] = {__builtin_amdgcn_perm(p23, p01, 0x05040100u),
                                    __builtin_amdgcn_perm(p23, p01, 0x07060302u),
                                    __builtin_amdgcn_perm(q23, q01, 0x05040100u)};
            uint32_t planes[kDigitPlanes<TYPE>];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                if (TYPE == kGgmlQ4_0) {
                    // nibble planes 2k and 2k + 1: slice f's nibbles low, slice f + 4's high
                    const uint32_t lo = yb[k] ^ 0x88888888u;
                    const uint32_t hi = from_lane_plus4(lo);
                    planes[2 * k] = (lo & 0x0F0F0F0Fu) | ((hi << 4) & 0xF0F0F0F0u);
                    planes[2 * k + 1] = ((lo >> 4) & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
                } else {
                    planes[k] = yb[k] ^ 0x80808080u;
                }
            }
            if (i < n4) {
                const int p = i >> 4, c = (i >> 3) & 1;
                uint32_t *slot = xs_lds + p * 52 + c * 24;
                if (TYPE == kGgmlQ4_0) {
                    if (f < 4) {
#pragma unroll
                        for (int t = 0; t < 6; ++t) {
                            slot[4 * t + f] = planes[t];
                        }
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 3; ++t) {
                        slot[8 * t + f] = planes[t];
                    }
                }
                if (f == 0) {
                    // a non-finite input makes the block's rows NaN
                    xs_lds[p * 52 + 48 + c] = __float_as_uint(bad ? __builtin_nanf("") : ldexpf(1.0f, -e));
                }
            }
        }
    };
    // The first batch from the prefetched slices, outside the loop below: the
    // wait for them then leaves the weight loads issued after them in flight.
    {
        float4 v[kStageBatch];
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            if constexpr (PRE == kPreMerge) {
                v[u] = u == 0 && (int)threadIdx.x < n4 ? merged_slice(pf) : pf.x[u];
            } else {
                v[u] = u * nthreads + (int)threadIdx.x < n4 ? pre_op(pf.x[u], pf.y[u]) : pf.x[u];
            }
        }
        digitize(0, v);
    }
    if constexpr (PRE == kPreMerge) {
        return;  // one slice per thread
    }
    for (int base = kStageBatch * nthreads; base < n4; base += kStageBatch * nthreads) {
        float4 v[kStageBatch];
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            const int i = base + u * nthreads + (int)threadIdx.x;
            v[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < n4) {
                const float4 y = PRE == kPreNone
                                     ? v[u]
                                     : reinterpret_cast<const float4 *>(PRE == kPreRmsNorm ? in.norm_w : in.x2)[i];
                v[u] = pre_op(reinterpret_cast<const float4 *>(in.x)[i], y);
            }
        }
        digitize(base, v);
    }
}

// acc + the row's block pair (PW dwords w) against the lane's digit planes xq
// (48 dwords) and the two block scales sc0, sc1 (2^-e).
template <uint32_t TYPE>
__device__ __forceinline__ float pair_dot(const uint32_t *w, const uint32_t (&xq)[48], float sc0, float sc1,
                                          float acc) {
    float d0, d1, dot0, dot1;
    if (TYPE == kGgmlQ4_0) {
        // block 0: scale = w0 low half, codes = bytes 2..17; block 1: scale = w4 high half, codes = w5..w8
        d0 = f16_bits_to_f32(w[0] & 0xffffu);
        d1 = f16_bits_to_f32(w[4] >> 16);
        int s0[6] = {}, s1[6] = {};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q0 = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2) ^ 0x88888888u;
            const uint32_t q1 = w[5 + k] ^ 0x88888888u;
#pragma unroll
            for (int t = 0; t < 6; ++t) {
                s0[t] = __builtin_amdgcn_sdot8((int)q0, (int)xq[4 * t + k], s0[t], false);
                s1[t] = __builtin_amdgcn_sdot8((int)q1, (int)xq[24 + 4 * t + k], s1[t], false);
            }
        }
        dot0 = fmaf((float)(s0[3] + s0[4] * 16 + s0[5] * 256), 4096.0f, (float)(s0[0] + s0[1] * 16 + s0[2] * 256));
        dot1 = fmaf((float)(s1[3] + s1[4] * 16 + s1[5] * 256), 4096.0f, (float)(s1[0] + s1[1] * 16 + s1[2] * 256));
    } else {
        // block 0: scale = w0 low half, codes = bytes 2..33; block 1: scale = w8 high half, codes = w9..w16
        d0 = f16_bits_to_f32(w[0] & 0xffffu);
        d1 = f16_bits_to_f32(w[8] >> 16);
        int s0[3] = {}, s1[3] = {};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t q0 = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
            const uint32_t q1 = w[9 + k];
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                s0[t] = __builtin_amdgcn_sdot4((int)q0, (int)xq[8 * t + k], s0[t], false);
                s1[t] = __builtin_amdgcn_sdot4((int)q1, (int)xq[24 + 8 * t + k], s1[t], false);
            }
        }
        dot0 = fmaf((float)s0[2], 65536.0f, (float)(s0[0] + s0[1] * 256));
        dot1 = fmaf((float)s1[2], 65536.0f, (float)(s1[0] + s1[1] * 256));
    }
    acc = fmaf(d0 * sc0, dot0, acc);
    return fmaf(d1 * sc1, dot1, acc);
}

// Both pair kernels cut the rows into tiles of 64 / LPR row groups x NR rows;
// each wave walks tiles gwave, gwave + waves, ..., and lane li of a group takes
// block PAIRS li, li + LPR, ... of its NR rows.  A pair is 36 (Q4_0) or 68 (Q8_0)
// bytes on a dword boundary.
//
// Strided pair kernel (weights not 16-byte aligned, or row groups longer than
// the streamed kernel's LDS tile): each lane reads its pairs straight from HBM
// as whole dwords, and the next (tile, pair step)'s weights are loaded into a
// second register set before the current one is computed.
template <uint32_t TYPE, int LPR, int NR>
__global__ __launch_bounds__(kPairThreads) void matvec_pairs_kernel(const unsigned char *weights,
                                                                       const float *input, int cols, int rows,
                                                                       size_t row_bytes, float *out, int tiles) {
    constexpr int PW = TYPE == kGgmlQ4_0 ? 9 : 17;  // dwords per block pair
    constexpr int G = 64 / LPR;                      // row groups per wave
    extern __shared__ uint4 xs_lds4[];  // [pairs][13] uint4: block 0 planes, block 1 planes, scales
    uint32_t *const xs_lds = reinterpret_cast<uint32_t *>(xs_lds4);
    const int lane = threadIdx.x & 63;
    const int grp = lane / LPR;
    const int li = lane % LPR;
    // tile t goes to wave t mod waves; consecutive tiles land on different CUs
    const int gwave = (int)(threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int nwaves = gridDim.x * kPairWaves;
    const int pairs = cols / 64;
    const int steps = (pairs + LPR - 1) / LPR;  // pair steps per tile

    uint32_t wa[NR][PW], wb[NR][PW];
    // Loads are never skipped: past the last tile a wave re-reads the last one
    // (unused), so the loop below has no branch around a load and the compiler
    // keeps the next step's loads outstanding while the current one is summed.
    auto load = [&](uint32_t(&w)[NR][PW], int tile, int step) {
        tile = min(tile, tiles - 1);
        const int p = min(li + step * LPR, pairs - 1);  // lanes past the last pair re-read it, unused
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int row = min((tile * G + grp) * NR + r, rows - 1);  // rows past the end: never stored
            // plain loads: the three loads of a lane's pair share cache lines with the
            // neighbouring lanes' pairs (nontemporal loads re-fetched them: 1.3-2x slower)
            const uint32_t *src =
                reinterpret_cast<const uint32_t *>(weights + (size_t)row * row_bytes + (size_t)p * 4 * PW);
#pragma unroll
            for (int k = 0; k < PW; ++k) {
                w[r][k] = src[k];
            }
        }
    };
    const StageInput in{input, nullptr, nullptr, 0.0f};
    StagePrefetch pf;
    stage_prefetch<kPreNone>(in, pairs * 16, pf);
    if (gwave < tiles) {
        load(wa, gwave, 0);
    }

    stage_digit_planes<TYPE, kPreNone>(in, pairs, xs_lds, pf);
    __syncthreads();
    if (gwave >= tiles) {
        return;
    }

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        acc[r] = 0.0f;
    }
    uint32_t xq[48];  // digit planes of the lane's pair: block c, plane t, dword k at 24c + (4|8)t + k
    float sc0 = 0.0f, sc1 = 0.0f;
    int x_step = -1;
    // sum of one pair step of NR rows into acc; the digit planes are re-read from
    // LDS only when the step changes (never when a tile is one step)
    auto compute = [&](const uint32_t(&w)[NR][PW], int step) {
        const int p = li + step * LPR;
        if (step != x_step) {
            x_step = step;
            const int pp = min(p, pairs - 1);
#pragma unroll
            for (int k = 0; k < 12; ++k) {
                const uint4 v = xs_lds4[pp * 13 + k];
                xq[4 * k] = v.x;
                xq[4 * k + 1] = v.y;
                xq[4 * k + 2] = v.z;
                xq[4 * k + 3] = v.w;
            }
            const uint4 s = xs_lds4[pp * 13 + 12];
            sc0 = __uint_as_float(s.x);
            sc1 = __uint_as_float(s.y);
        }
        if (p >= pairs) {
            return;
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            acc[r] = pair_dot<TYPE>(w[r], xq, sc0, sc1, acc[r]);
        }
    };
    auto finish_tile = [&](int tile) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            float v = acc[r];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) {
                v += __shfl_xor(v, o, 64);
            }
            const int row = (tile * G + grp) * NR + r;
            if (li == 0 && row < rows) {
                out[row] = v;
            }
            acc[r] = 0.0f;
        }
    };
    // (tile, step) walk; wave-uniform, so every branch below is scalar
    int tile = gwave, step = 0;
    auto advance = [&](int &t, int &s) {
        if (++s == steps) {
            s = 0;
            t += nwaves;
        }
    };
    for (;;) {
        int tn = tile, sn = step;
        advance(tn, sn);
        load(wb, tn, sn);
        compute(wa, step);
        if (sn == 0) {
            finish_tile(tile);
        }
        if (tn >= tiles) {
            break;
        }
        tile = tn;
        step = sn;
        advance(tn, sn);
        load(wa, tn, sn);
        compute(wb, step);
        if (sn == 0) {
            finish_tile(tile);
        }
        if (tn >= tiles) {
            break;
        }
        tile = tn;
        step = sn;
    }
}

// Streamed pair kernel.  A tile's rows are one contiguous byte range.  The wave
// reads it as 16-byte chunks, lane l taking chunks l, l + 64, ... (every load
// instruction covers 1 KB contiguous; nontemporal, the weights are read once
// per token), writes them to its own LDS buffer, and each lane reads its pairs
// from there.  The next tile's chunks load into registers while the current
// tile is summed from LDS; a wave's LDS operations complete in order, so the
// next tile is stored over the buffer after the current one's reads with no
// barrier.  CH chunk loads per lane: CH KB >= the tile plus 15 bytes of
// misalignment (tiles start on dword, not 16-byte, boundaries).
// One weight matrix of a streamed launch: out[r] = W[r] . x' (+ resid[r] when
// resid is set; resid may be out) for r < rows.  A launch takes up to three
// matrices of the same type and width, one input; their row tiles are numbered
// one after another.
struct StreamSeg {
    const unsigned char *w;
    float *out;
    const float *resid;
    size_t total_chunks;  // rows * row_bytes / 16
    int rows;
    int tiles;
};

struct StreamArgs {
    StreamSeg seg[3];
    int nseg;
    int tiles;  // all segments
    int cols;
    size_t row_bytes;
    StageInput in;
};

//
// GLU launches (the decode layer's gate and up projections, seg[0] = gate
// with the output, seg[1] = up): a tile holds the same NR * G / 2 rows of
// both matrices, gate rows in the first G / 2 row groups (their chunks in the
// first CH / 2 KB of the tile buffer), up rows in the rest, and the epilogue
// writes silu(gate) * up as te_swiglu_f32 (ops.c:397-406) instead of either.
template <uint32_t TYPE, int LPR, int NR, int CH, int PRE, bool GLU>
__global__ __launch_bounds__(kPairThreads) void matvec_stream_kernel(const StreamArgs a) {
    constexpr int PW = TYPE == kGgmlQ4_0 ? 9 : 17;  // dwords per block pair
    constexpr int G = 64 / LPR;                      // row groups per wave
    constexpr int HG = GLU ? G / 2 : G;              // row groups per matrix of a tile
    static_assert(!GLU || (G >= 2 && CH % 2 == 0), "GLU tiles split the row groups and chunks in two");
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    extern __shared__ uint4 lds4[];  // [pairs][13] digit planes + scales, then one CH KB tile buffer per wave
    uint32_t *const xs_lds = reinterpret_cast<uint32_t *>(lds4);
    const int lane = threadIdx.x & 63;
    const int grp = lane / LPR;
    const int li = lane % LPR;
    // the wave index through readfirstlane: the compiler then keeps every
    // tile-derived value (segment fields included) in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // tile t goes to wave t mod waves; consecutive tiles land on different CUs
    const int gwave = wave * gridDim.x + blockIdx.x;
    const int nwaves = gridDim.x * (int)(blockDim.x >> 6);
    const int pairs = a.cols / 64;
    const int steps = (pairs + LPR - 1) / LPR;  // pair steps per tile
    const size_t tile_bytes = (size_t)HG * NR * a.row_bytes;  // one matrix's rows of a tile
    uint4 *const buf = lds4 + pairs * 13 + wave * CH * 64;

    // Segment of global tile t, as values chosen by scalar selects: indexing the
    // kernel-argument array (or taking a reference into it) with a run-time index
    // makes the compiler read it with vector loads and wait on them in the loop.
    auto seg_of = [&](int t, int &local) {
        const int t0 = a.seg[0].tiles, t1 = a.seg[1].tiles;
        const int s = t < t0 ? 0 : (a.nseg > 2 && t >= t0 + t1) ? 2 : 1;
        local = s == 0 ? t : s == 1 ? t - t0 : t - t0 - t1;
        StreamSeg g;
        g.w = s == 0 ? a.seg[0].w : s == 1 ? a.seg[1].w : a.seg[2].w;
        g.out = s == 0 ? a.seg[0].out : s == 1 ? a.seg[1].out : a.seg[2].out;
        g.resid = s == 0 ? a.seg[0].resid : s == 1 ? a.seg[1].resid : a.seg[2].resid;
        g.total_chunks = s == 0 ? a.seg[0].total_chunks : s == 1 ? a.seg[1].total_chunks : a.seg[2].total_chunks;
        g.rows = s == 0 ? a.seg[0].rows : s == 1 ? a.seg[1].rows : a.seg[2].rows;
        return g;
    };

    // A tile's loads: its weight chunks and (residual launches) the residuals of
    // its rows, issued together one tile ahead, so the wait for them at the next
    // tile's start never waits for loads issued later.  Every lane issues every
    // load (lanes past the tile re-read its last chunk, a wave with no tile
    // reads one chunk) and
    // nothing uses them until the tile's start: no branch or select waits on
    // them, so the staging below never waits for the weight loads.
    u32x4 ck[CH] = {};
    float res[NR] = {};
    auto load = [&](int tile, bool live) {
        int local;
        const StreamSeg sg = seg_of(tile, local);
        const size_t b = (size_t)local * tile_bytes;
        const size_t c0 = b >> 4;
        const size_t c1 = min((b + tile_bytes + 15) >> 4, sg.total_chunks);
        const size_t c_last = live ? c1 - 1 : c0;
        const u32x4 *w16 = reinterpret_cast<const u32x4 *>(sg.w);
        if (GLU) {
            // the same byte range of the up matrix (equal shapes) into the second half
            const u32x4 *u16 = reinterpret_cast<const u32x4 *>(a.seg[1].w);
#pragma unroll
            for (int i = 0; i < CH / 2; ++i) {
                ck[i] = __builtin_nontemporal_load(w16 + min(c0 + lane + 64 * i, c_last));
                ck[CH / 2 + i] = __builtin_nontemporal_load(u16 + min(c0 + lane + 64 * i, c_last));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            ck[i] = __builtin_nontemporal_load(w16 + min(c0 + lane + 64 * i, c_last));
        }
        // (the tile's epilogue adds res only for residual launches, in lane 0 of
        // a group, to rows < rows; other launches read the first 4 * rows bytes
        // of their weights, a valid range with one address per row)
        const float *rp = sg.resid != nullptr ? sg.resid : reinterpret_cast<const float *>(sg.w);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int row = (local * G + grp) * NR + r;
            res[r] = rp[min(row, sg.rows - 1)];
        }
    };
    // The input slices, then the tile's weight loads: the staging waits for
    // the input only.
    StagePrefetch pf;
    stage_prefetch<PRE>(a.in, pairs * 16, pf);
    load(min(gwave, a.tiles - 1), gwave < a.tiles);
    stage_digit_planes<TYPE, PRE>(a.in, pairs, xs_lds, pf);
    __syncthreads();
    const float rms = PRE == kPreRmsNorm ? rms_scale(a.in, pairs * 64) : 1.0f;
    if (gwave >= a.tiles) {
        return;
    }

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        acc[r] = 0.0f;
    }
    uint32_t xq[48];
    float sc0 = 0.0f, sc1 = 0.0f;
    auto read_planes = [&](int p) {
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const uint4 v = lds4[p * 13 + k];
            xq[4 * k] = v.x;
            xq[4 * k + 1] = v.y;
            xq[4 * k + 2] = v.z;
            xq[4 * k + 3] = v.w;
        }
        const uint4 s = lds4[p * 13 + 12];
        sc0 = __uint_as_float(s.x);
        sc1 = __uint_as_float(s.y);
    };
    if (steps == 1) {
        read_planes(min(li, pairs - 1));
    }
    for (int tile = gwave;;) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            buf[lane + 64 * i] = make_uint4(ck[i].x, ck[i].y, ck[i].z, ck[i].w);
        }
        float res_cur[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            res_cur[r] = res[r];
        }
        int local;
        const StreamSeg sg = seg_of(tile, local);
        const int tn = tile + nwaves;
        if (tn < a.tiles) {
            load(tn, true);
        }
        const unsigned char *tb =
            reinterpret_cast<const unsigned char *>(buf) + (((size_t)local * tile_bytes) & 15);
        for (int step = 0; step < steps; ++step) {
            const int p = li + step * LPR;
            if (steps > 1) {
                read_planes(min(p, pairs - 1));
            }
            if (p < pairs) {
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const uint32_t *src = reinterpret_cast<const uint32_t *>(
                        tb + (GLU && grp >= HG ? (size_t)(CH / 2) * 1024 : 0) +
                        (size_t)((grp % HG) * NR + r) * a.row_bytes + (size_t)p * 4 * PW);
                    uint32_t w[PW];
#pragma unroll
                    for (int k = 0; k < PW; ++k) {
                        w[k] = src[k];
                    }
                    acc[r] = pair_dot<TYPE>(w, xq, sc0, sc1, acc[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            float v = acc[r];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) {
                v += __shfl_xor(v, o, 64);
            }
            if (GLU) {
                // lanes 32 apart hold the gate and up sums of the same row
                const float g = v * rms;
                const float u = __shfl_xor(g, 32, 64);
                const int row = (local * HG + grp) * NR + r;
                if (li == 0 && grp < HG && row < sg.rows) {
                    sg.out[row] = g / (1.0f + expf(-g)) * u;
                }
                acc[r] = 0.0f;
                continue;
            }
            const int row = (local * G + grp) * NR + r;
            if (li == 0 && row < sg.rows) {
                // the residual add of the reference's te_add_f32(hidden, proj)
                if (PRE == kPreRmsNorm) {
                    v *= rms;
                }
                sg.out[row] = sg.resid != nullptr ? res_cur[r] + v : v;
            }
            acc[r] = 0.0f;
        }
        if (tn >= a.tiles) {
            break;
        }
        tile = tn;
    }
}

// One workgroup per row: sum of squares in fp64 (as the reference), the scale
// 1/sqrtf(mean + eps) in fp32, then x * scale * w.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *input, const float *weight, int len, float eps,
                                                      float *out) {
    const float *x = input + (size_t)blockIdx.x * len;
    float *y = out + (size_t)blockIdx.x * len;
    double ss = 0.0;
    for (int i = threadIdx.x; i < len; i += 256) {
        const double v = (double)x[i];
        ss += v * v;
    }
    __shared__ double part[4];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        ss += __shfl_xor(ss, o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    const double total = part[0] + part[1] + part[2] + part[3];
    const float scale = 1.0f / sqrtf((float)(total / (double)len) + eps);
    for (int i = threadIdx.x; i < len; i += 256) {
        y[i] = x[i] * scale * weight[i];
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float *gate, const float *up, size_t len, float *out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (size_t)gridDim.x * 256) {
        const float g = gate[i];
        const float silu = g / (1.0f + expf(-g));
        out[i] = silu * up[i];
    }
}

__global__ __launch_bounds__(256) void add_kernel(const float *lhs, const float *rhs, size_t len, float *out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (size_t)gridDim.x * 256) {
        out[i] = lhs[i] + rhs[i];
    }
}

// First index of the maximum, as the reference's sequential scan: a value
// counts only when it is > -FLT_MAX's running best (NaN never does), ties keep
// the lower index, and an all -inf / NaN vector gives 0.  One workgroup;
// (value, index) pairs reduce with that order.
__device__ __forceinline__ void argmax_take(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float *values, uint32_t len, uint32_t *out_index) {
    float bv = -FLT_MAX;
    uint32_t bi = 0xffffffffu;
    // strictly greater: the first maximum of this thread's indices, which it
    // visits in increasing order (float4 slices t, t + 1024, ..., then the tail)
    auto take = [&](float v, uint32_t i) {
        if (v > bv) {
            bv = v;
            bi = i;
        }
    };
    const uint32_t n4 = ((size_t)values & 15u) == 0 ? len / 4 : 0;
    const float4 *v4 = reinterpret_cast<const float4 *>(values);
    for (uint32_t base = 0; base < n4; base += 4 * 1024) {
        float4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {  // all loads issued before the compares
            const uint32_t j = base + u * 1024 + threadIdx.x;
            q[u] = j < n4 ? v4[j] : make_float4(-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t i = 4 * (base + u * 1024 + threadIdx.x);
            take(q[u].x, i);
            take(q[u].y, i + 1);
            take(q[u].z, i + 2);
            take(q[u].w, i + 3);
        }
    }
    for (uint32_t i = 4 * n4 + threadIdx.x; i < len; i += 1024) {
        take(values[i], i);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        argmax_take(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    }
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w) {
            argmax_take(bv, bi, sv[w], si[w]);
        }
        *out_index = bi == 0xffffffffu ? 0u : bi;  // nothing above -FLT_MAX: index 0
    }
}

// Row `row` of a [rows][cols] GGUF tensor as fp32 (te_model_dequantize_row_f32,
// ops.c:127-175; block formats ops.c:15-21): Q4_0 (code - 8) * d with low
// nibbles first, Q8_0 code * d, F32 as stored.  One thread per value.
// Row rows[blockIdx.y] (or `row` without a list) into out + blockIdx.y * cols.
__global__ __launch_bounds__(256) void dequant_row_kernel(const unsigned char *weights, uint32_t ggml_type,
                                                          int cols, size_t row_bytes, size_t row,
                                                          const uint32_t *rows, float *out) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) {
        return;
    }
    const unsigned char *r = weights + (rows != nullptr ? (size_t)rows[blockIdx.y] : row) * row_bytes;
    out += (size_t)blockIdx.y * cols;
    float v;
    if (ggml_type == kGgmlF32) {
        __builtin_memcpy(&v, r + (size_t)c * 4, 4);  // any byte alignment
    } else if (ggml_type == kGgmlQ4_0) {
        const unsigned char *b = r + (size_t)(c / 32) * 18;
        const int j = c % 32;
        const float d = f16_bits_to_f32((uint32_t)b[0] | (uint32_t)b[1] << 8);
        const int q = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
        v = (float)(q - 8) * d;
    } else {
        const unsigned char *b = r + (size_t)(c / 32) * 34;
        const float d = f16_bits_to_f32((uint32_t)b[0] | (uint32_t)b[1] << 8);
        v = (float)(signed char)b[2 + c % 32] * d;
    }
    out[c] = v;
}

}  // namespace

namespace te_hip {

size_t ggml_row_bytes(uint32_t ggml_type, size_t cols) {
    switch (ggml_type) {
        case kGgmlQ4_0:
            return cols % 32 == 0 ? cols / 32 * 18 : 0;
        case kGgmlQ8_0:
            return cols % 32 == 0 ? cols / 32 * 34 : 0;
        case kGgmlF32:
            return cols % 4 == 0 ? cols * 4 : 0;
        default:
            return 0;
    }
}

// Streamed GEMV launch over a.seg[0, a.nseg) with input pre-operation `pre`
// (a.cols, a.in and each segment's w / out / resid / rows set by the caller;
// the tile shape, tile counts and chunk bounds are filled in here).  *launched
// stays false, with OK, when the shapes do not suit the streamed kernel: a
// weight tensor not 16-byte aligned or not a multiple of 16 bytes long, a row
// group longer than the 10 KB tile, or staged input leaving LDS for fewer than
// 4 waves.
te_status launch_stream(uint32_t ggml_type, int pre, StreamArgs a, hipStream_t stream, bool *launched,
                        bool glu = false) {
    *launched = false;
    const size_t cols = (size_t)a.cols;
    if ((ggml_type != kGgmlQ4_0 && ggml_type != kGgmlQ8_0) || cols % 64 != 0 || a.nseg < 1 || a.nseg > 3 ||
        (glu && (a.nseg != 2 || pre != kPreRmsNorm || a.seg[0].rows != a.seg[1].rows))) {
        return TE_STATUS_OK;
    }
    const size_t row_bytes = ggml_row_bytes(ggml_type, cols);
    const size_t pairs = cols / 64;
    const size_t plane_bytes = pairs * kPairLdsBytes;
    size_t rows_total = 0;
    for (int s = 0; s < a.nseg; ++s) {
        const size_t rows = (size_t)a.seg[s].rows;
        if (((size_t)a.seg[s].w & 15u) != 0 || rows * row_bytes % 16 != 0) {
            return TE_STATUS_OK;
        }
        rows_total += rows;
    }
    const int lpr = pairs >= 64 ? 64 : pairs >= 32 ? 32 : 16;
    const size_t groups = 64 / lpr;
    if (glu && groups < 2) {
        return TE_STATUS_OK;  // a GLU tile needs a row group of each matrix
    }
    // a GLU tile's rows of one matrix fill half its buffer
    const size_t hgroups = glu ? groups / 2 : groups;
    const size_t cus = (size_t)device_compute_units();
    // tiles of at most 10 KB (larger tiles measured faster at lm_head, 4 / 8 / 12 KB: more bytes
    // in flight per wave), as many rows as keep 16 tiles per CU for Q4_0 and 24 for Q8_0 (3B
    // decode token against 8 per CU, same box: Q4_0 1,396 -> 1,371 us, mostly the 11008-row
    // projections at one row per lane group instead of two and the paired gate / up at two
    // instead of four; Q8_0 1,633 -> 1,611 us, its paired gate / up at one row instead of two;
    // the lm_head keeps its rows per group)
    const size_t want = cus * (ggml_type == kGgmlQ8_0 ? 24 : 16);
    size_t tile_cap = kStreamTileBytes;
    if (const char *env = getenv("TE_HIP_GEMV_TILE")) {  // tuning override: bytes per row-group tile
        tile_cap = (size_t)atoi(env) >= 1024 && (size_t)atoi(env) <= kStreamTileBytes ? (size_t)atoi(env) : tile_cap;
    }
    int nr = 1;
    for (int cand = 2; cand <= (ggml_type == kGgmlQ4_0 ? 4 : 2); cand *= 2) {
        if (hgroups * cand * row_bytes + 15 <= (glu ? tile_cap / 2 : tile_cap) &&
            rows_total >= cand * groups * want) {
            nr = cand;
        }
    }
    // Q8_0 rows of 10-12 KB (ffn_down at 11008 columns: 11696 bytes) take
    // 12-chunk tiles, one row per tile
    const bool wide = !glu && ggml_type == kGgmlQ8_0 && groups == 1 && row_bytes + 15 > kStreamTileBytes &&
                      row_bytes + 15 <= (size_t)kWideStreamChunks * 1024;
    // Small tiles take 4-chunk loads: every lane issues every chunk load of a
    // tile (lanes past it re-read its last chunk), so the load count follows
    // the tile, not the largest one.
    const bool short_tile = !glu && !wide && nr == 1 && groups * row_bytes + 15 <= (size_t)kShortStreamChunks * 1024;
    const size_t tile_lds = wide ? (size_t)kWideStreamChunks * 1024
                                 : short_tile ? (size_t)kShortStreamChunks * 1024 : kStreamTileBytes;
    const size_t waves_fit = hgroups * row_bytes + 15 <= (glu ? tile_lds / 2 : tile_lds) &&
                                     plane_bytes < kMaxPairLdsBytes
                                 ? (kMaxPairLdsBytes - plane_bytes) / tile_lds
                                 : 0;
    if (waves_fit < 4) {
        return TE_STATUS_OK;
    }
    const int wpg = waves_fit < (size_t)kPairWaves ? (int)waves_fit : kPairWaves;
    // a merge staging takes one slice of the input per thread, with one row per tile
    if (pre == kPreMerge && (glu || wide || nr != 1 || pairs * 16 > (size_t)(64 * wpg))) {
        return TE_STATUS_OK;
    }
    const size_t lds = plane_bytes + (size_t)wpg * tile_lds;
    a.row_bytes = row_bytes;
    a.tiles = 0;
    for (int s = 0; s < a.nseg; ++s) {
        const size_t rows = (size_t)a.seg[s].rows;
        a.seg[s].tiles = (int)((rows + hgroups * nr - 1) / (hgroups * nr));
        a.seg[s].total_chunks = rows * row_bytes / 16;
        a.tiles += a.seg[s].tiles;
    }
    if (glu) {
        // every tile is the gate matrix's (segment 0); the up rows ride along
        a.tiles = a.seg[0].tiles;
        a.seg[1].tiles = 0;
    }
    const dim3 grid((unsigned)((size_t)a.tiles < cus ? (size_t)a.tiles : cus));
#define TE_STREAM(T, L, N, C, P, GL)                                                                      \
    do {                                                                                                  \
        if (lds > 65536 &&                                                                                \
            hipFuncSetAttribute(reinterpret_cast<const void *>(&matvec_stream_kernel<T, L, N, C, P, GL>), \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {    \
            return TE_STATUS_RUNTIME_ERROR;                                                               \
        }                                                                                                 \
        matvec_stream_kernel<T, L, N, C, P, GL><<<grid, dim3(64 * wpg), lds, stream>>>(a);                \
    } while (0)
#define TE_STREAM_PRE(T, L, N, C)                          \
    do {                                                   \
        if (glu) {                                         \
            if constexpr (L <= 32 && C == kStreamChunks) { \
                TE_STREAM(T, L, N, C, kPreRmsNorm, true);  \
            }                                              \
        } else if (pre == kPreRmsNorm) {                   \
            TE_STREAM(T, L, N, C, kPreRmsNorm, false);     \
        } else if (pre == kPreSwiGLU) {                    \
            TE_STREAM(T, L, N, C, kPreSwiGLU, false);      \
        } else if (pre == kPreMerge) {                     \
            if constexpr (N == 1) {                        \
                TE_STREAM(T, L, N, C, kPreMerge, false);   \
            }                                              \
        } else {                                           \
            TE_STREAM(T, L, N, C, kPreNone, false);        \
        }                                                  \
    } while (0)
#define TE_STREAM_NR(T, L)                                                \
    do {                                                                  \
        if (nr == 4) {                                                    \
            TE_STREAM_PRE(T, L, (T == kGgmlQ4_0 ? 4 : 2), kStreamChunks); \
        } else if (nr == 2) {                                             \
            TE_STREAM_PRE(T, L, 2, kStreamChunks);                        \
        } else if (short_tile) {                                          \
            TE_STREAM_PRE(T, L, 1, kShortStreamChunks);                   \
        } else {                                                          \
            TE_STREAM_PRE(T, L, 1, kStreamChunks);                        \
        }                                                                 \
    } while (0)
#define TE_STREAM_LPR(T)          \
    do {                          \
        if (lpr == 64) {          \
            TE_STREAM_NR(T, 64);  \
        } else if (lpr == 32) {   \
            TE_STREAM_NR(T, 32);  \
        } else {                  \
            TE_STREAM_NR(T, 16);  \
        }                         \
    } while (0)
    if (wide) {
#define TE_STREAM_WIDE(P)                                                                                           \
    do {                                                                                                            \
        if (lds > 65536 &&                                                                                          \
            hipFuncSetAttribute(                                                                                    \
                reinterpret_cast<const void *>(&matvec_stream_kernel<kGgmlQ8_0, 64, 1, kWideStreamChunks, P, false>), \
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {                              \
            return TE_STATUS_RUNTIME_ERROR;                                                                         \
        }                                                                                                           \
        matvec_stream_kernel<kGgmlQ8_0, 64, 1, kWideStreamChunks, P, false><<<grid, dim3(64 * wpg), lds, stream>>>(a); \
    } while (0)
        if (pre == kPreRmsNorm) {
            TE_STREAM_WIDE(kPreRmsNorm);
        } else if (pre == kPreSwiGLU) {
            TE_STREAM_WIDE(kPreSwiGLU);
        } else {
            TE_STREAM_WIDE(kPreNone);
        }
#undef TE_STREAM_WIDE
    } else if (ggml_type == kGgmlQ4_0) {
        TE_STREAM_LPR(kGgmlQ4_0);
    } else {
        TE_STREAM_LPR(kGgmlQ8_0);
    }
#undef TE_STREAM_LPR
#undef TE_STREAM_NR
#undef TE_STREAM_PRE
#undef TE_STREAM
    *launched = true;
    return launch_status();
}

te_status launch_matvec(const void *weights, uint32_t ggml_type, const float *input, size_t cols, size_t rows,
                        float *out, hipStream_t stream) {
    const size_t row_bytes = ggml_row_bytes(ggml_type, cols);
    const unsigned char *w = static_cast<const unsigned char *>(weights);
    const size_t waves_wanted = (size_t)device_compute_units() * 16;
    const size_t pair_lds_bytes = cols / 64 * kPairLdsBytes;
    if (ggml_type != kGgmlF32 && cols % 64 == 0 && pair_lds_bytes <= kMaxPairLdsBytes) {
        // block pairs: lanes per row from the pair count; rows per group so that the
        // tiles give every CU at least 8 waves where the rows allow (Q8_0 stays at two
        // rows: four double-buffered 68-byte pairs do not fit 3 waves per SIMD)
        const size_t pairs = cols / 64;
        const int lpr = pairs >= 64 ? 64 : pairs >= 32 ? 32 : 16;
        const size_t groups = 64 / lpr;
        const size_t cus = (size_t)device_compute_units();
        const size_t want = cus * 8;
        if (getenv("TE_HIP_GEMV_STRIDED") == nullptr) {
            StreamArgs a = {};
            a.seg[0] = StreamSeg{w, out, nullptr, 0, (int)rows, 0};
            a.nseg = 1;
            a.cols = (int)cols;
            a.in = StageInput{input, nullptr, nullptr, 0.0f};
            bool launched = false;
            const te_status st = launch_stream(ggml_type, kPreNone, a, stream, &launched);
            if (launched || st != TE_STATUS_OK) {
                return st;
            }
        }
        int nr = rows >= 4 * groups * want && ggml_type == kGgmlQ4_0 ? 4 : rows >= 2 * groups * want ? 2 : 1;
        if (const char *env = getenv("TE_HIP_GEMV_NR")) {  // tuning override: rows per lane group
            const int v = atoi(env);
            nr = v == 1 || v == 2 || (v == 4 && ggml_type == kGgmlQ4_0) ? v : nr;
        }
        const size_t tiles = (rows + groups * nr - 1) / (groups * nr);
        const dim3 grid((unsigned)(tiles < cus ? tiles : cus));
        const dim3 block(kPairThreads);
#define TE_PAIRS(T, L, N)                                                                                         \
    do {                                                                                                          \
        if (pair_lds_bytes > 65536 &&                                                                             \
            hipFuncSetAttribute(reinterpret_cast<const void *>(&matvec_pairs_kernel<T, L, N>),                    \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)pair_lds_bytes) != hipSuccess) { \
            return TE_STATUS_RUNTIME_ERROR;                                                                       \
        }                                                                                                         \
        matvec_pairs_kernel<T, L, N><<<grid, block, pair_lds_bytes, stream>>>(w, input, (int)cols, (int)rows,     \
                                                                             row_bytes, out, (int)tiles);         \
    } while (0)
#define TE_PAIRS_NR(T, L)                                    \
    do {                                                     \
        if (nr == 4) {                                       \
            TE_PAIRS(T, L, (T == kGgmlQ4_0 ? 4 : 2));        \
        } else if (nr == 2) {                                \
            TE_PAIRS(T, L, 2);                               \
        } else {                                             \
            TE_PAIRS(T, L, 1);                               \
        }                                                    \
    } while (0)
#define TE_PAIRS_LPR(T)          \
    do {                         \
        if (lpr == 64) {         \
            TE_PAIRS_NR(T, 64);  \
        } else if (lpr == 32) {  \
            TE_PAIRS_NR(T, 32);  \
        } else {                 \
            TE_PAIRS_NR(T, 16);  \
        }                        \
    } while (0)
        if (ggml_type == kGgmlQ4_0) {
            TE_PAIRS_LPR(kGgmlQ4_0);
        } else {
            TE_PAIRS_LPR(kGgmlQ8_0);
        }
#undef TE_PAIRS_LPR
#undef TE_PAIRS_NR
#undef TE_PAIRS
        return launch_status();
    }
    // F32, and quantized rows with an odd block count: one block (or float4) per lane step
    const int R = rows >= 4 * waves_wanted ? 4 : rows >= 2 * waves_wanted ? 2 : 1;
    const size_t rows_per_wg = (size_t)R * kMatvecWaves;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
#define TE_MATVEC_LAUNCH(T)                                                                                   \
    do {                                                                                                      \
        if (R == 4) {                                                                                         \
            matvec_kernel<T, 4><<<grid, 64 * kMatvecWaves, 0, stream>>>(w, input, (int)cols, (int)rows,      \
                                                                         row_bytes, out);                     \
        } else if (R == 2) {                                                                                  \
            matvec_kernel<T, 2><<<grid, 64 * kMatvecWaves, 0, stream>>>(w, input, (int)cols, (int)rows,      \
                                                                         row_bytes, out);                     \
        } else {                                                                                              \
            matvec_kernel<T, 1><<<grid, 64 * kMatvecWaves, 0, stream>>>(w, input, (int)cols, (int)rows,      \
                                                                         row_bytes, out);                     \
        }                                                                                                     \
    } while (0)
    if (ggml_type == kGgmlQ4_0) {
        TE_MATVEC_LAUNCH(kGgmlQ4_0);
    } else if (ggml_type == kGgmlQ8_0) {
        TE_MATVEC_LAUNCH(kGgmlQ8_0);
    } else {
        TE_MATVEC_LAUNCH(kGgmlF32);
    }
#undef TE_MATVEC_LAUNCH
    return launch_status();
}

te_status launch_gemv(uint32_t ggml_type, GemvPre pre, const GemvSeg *segs, int nseg, size_t cols, const float *x,
                      const float *x2, const float *norm_w, float eps, float *xtmp, float *ytmp,
                      hipStream_t stream) {
    if (getenv("TE_HIP_GEMV_STRIDED") == nullptr && nseg >= 1 && nseg <= 3) {
        StreamArgs a = {};
        for (int s = 0; s < nseg; ++s) {
            a.seg[s] = StreamSeg{static_cast<const unsigned char *>(segs[s].w), segs[s].out, segs[s].resid, 0,
                                 (int)segs[s].rows, 0};
        }
        a.nseg = nseg;
        a.cols = (int)cols;
        a.in = StageInput{x, x2, norm_w, eps};
        const int kpre = pre == kGemvRmsNorm ? kPreRmsNorm : pre == kGemvSwiGLU ? kPreSwiGLU : kPreNone;
        bool launched = false;
        const te_status st = launch_stream(ggml_type, kpre, a, stream, &launched);
        if (launched || st != TE_STATUS_OK) {
            return st;
        }
    }
    const float *input = x;
    te_status st = TE_STATUS_OK;
    if (pre == kGemvRmsNorm) {
        st = launch_rmsnorm(x, norm_w, 1, cols, eps, xtmp, stream);
        input = xtmp;
    } else if (pre == kGemvSwiGLU) {
        st = launch_swiglu(x, x2, cols, xtmp, stream);
        input = xtmp;
    }
    for (int s = 0; s < nseg && st == TE_STATUS_OK; ++s) {
        if (segs[s].resid == nullptr) {
            st = launch_matvec(segs[s].w, ggml_type, input, cols, segs[s].rows, segs[s].out, stream);
        } else {
            st = launch_matvec(segs[s].w, ggml_type, input, cols, segs[s].rows, ytmp, stream);
            if (st == TE_STATUS_OK) {
                st = launch_add(segs[s].resid, ytmp, segs[s].rows, segs[s].out, stream);
            }
        }
    }
    return st;
}

te_status launch_gemv_glu(uint32_t ggml_type, const void *gate_w, const void *up_w, size_t rows, size_t cols,
                          const float *x, const float *norm_w, float eps, float *h, hipStream_t stream,
                          bool *launched) {
    *launched = false;
    const char *glu_env = getenv("TE_HIP_GEMV_GLU");
    if (getenv("TE_HIP_GEMV_STRIDED") != nullptr || (glu_env != nullptr && strcmp(glu_env, "0") == 0)) {
        return TE_STATUS_OK;  // the switches that take the separate launches
    }
    StreamArgs a = {};
    a.seg[0] = StreamSeg{static_cast<const unsigned char *>(gate_w), h, nullptr, 0, (int)rows, 0};
    a.seg[1] = StreamSeg{static_cast<const unsigned char *>(up_w), nullptr, nullptr, 0, (int)rows, 0};
    a.nseg = 2;
    a.cols = (int)cols;
    a.in = StageInput{x, nullptr, norm_w, eps};
    return launch_stream(ggml_type, kPreRmsNorm, a, stream, launched, true);
}

te_status launch_gemv_merge(uint32_t ggml_type, const GemvSeg &seg, size_t cols, const float *part_o,
                            const float *part_ml, size_t chunks, size_t max_chunks, size_t head_dim,
                            hipStream_t stream, bool *launched) {
    *launched = false;
    if (getenv("TE_HIP_GEMV_STRIDED") != nullptr || chunks == 0 || chunks > (size_t)kMergeChunks ||
        chunks > max_chunks || head_dim % 4 != 0 || cols % head_dim != 0 || ((size_t)part_o & 15u) != 0 ||
        ((size_t)part_ml & 7u) != 0 || max_chunks > 65535) {
        return TE_STATUS_OK;
    }
    StreamArgs a = {};
    a.seg[0] = StreamSeg{static_cast<const unsigned char *>(seg.w), seg.out, seg.resid, 0, (int)seg.rows, 0};
    a.nseg = 1;
    a.cols = (int)cols;
    a.in = StageInput{nullptr, nullptr, nullptr, 0.0f, part_o, part_ml, (int)chunks, (int)max_chunks, (int)head_dim};
    return launch_stream(ggml_type, kPreMerge, a, stream, launched);
}

te_status launch_dequant_row(const void *weights, uint32_t ggml_type, size_t cols, size_t row, float *out,
                             hipStream_t stream) {
    const size_t row_bytes = ggml_type == kGgmlF32 ? cols * 4 : ggml_row_bytes(ggml_type, cols);
    dequant_row_kernel<<<dim3((unsigned)((cols + 255) / 256)), 256, 0, stream>>>(
        static_cast<const unsigned char *>(weights), ggml_type, (int)cols, row_bytes, row, nullptr, out);
    return launch_status();
}

te_status launch_dequant_rows(const void *weights, uint32_t ggml_type, size_t cols, const uint32_t *rows, size_t n,
                              float *out, hipStream_t stream) {
    const size_t row_bytes = ggml_type == kGgmlF32 ? cols * 4 : ggml_row_bytes(ggml_type, cols);
    dequant_row_kernel<<<dim3((unsigned)((cols + 255) / 256), (unsigned)n), 256, 0, stream>>>(
        static_cast<const unsigned char *>(weights), ggml_type, (int)cols, row_bytes, 0, rows, out);
    return launch_status();
}

te_status launch_rmsnorm(const float *input, const float *weight, size_t rows, size_t len, float epsilon, float *out,
                         hipStream_t stream) {
    rmsnorm_kernel<<<dim3((unsigned)rows), 256, 0, stream>>>(input, weight, (int)len, epsilon, out);
    return launch_status();
}

static unsigned elementwise_grid(size_t len) {
    const size_t wgs = (len + 255) / 256;
    const size_t cap = (size_t)device_compute_units() * 16;
    return (unsigned)(wgs < cap ? wgs : cap);
}

te_status launch_swiglu(const float *gate, const float *up, size_t len, float *out, hipStream_t stream) {
    swiglu_kernel<<<elementwise_grid(len), 256, 0, stream>>>(gate, up, len, out);
    return launch_status();
}

te_status launch_add(const float *lhs, const float *rhs, size_t len, float *out, hipStream_t stream) {
    add_kernel<<<elementwise_grid(len), 256, 0, stream>>>(lhs, rhs, len, out);
    return launch_status();
}

te_status launch_argmax(const float *values, size_t len, uint32_t *out_index, hipStream_t stream) {
    argmax_kernel<<<1, 1024, 0, stream>>>(values, (uint32_t)len, out_index);
    return launch_status();
}

}  // namespace te_hip

extern "C" te_status te_hip_matvec_f32(const void *weights, uint32_t ggml_type, const float *input, size_t cols,
                                       size_t rows, float *out, void *stream) {
    if (weights == nullptr || input == nullptr || out == nullptr || cols == 0 || rows == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (te_hip::ggml_row_bytes(ggml_type, cols) == 0 || cols > (1u << 24) || rows > (1u << 30)) {
        return TE_STATUS_UNSUPPORTED;  // other GGUF types, cols not a multiple of the block
    }
    // dword (quantized) / float4 (F32) weight reads and float4 input reads
    if (((size_t)weights & (ggml_type == 0 ? 15u : 3u)) != 0 || ((size_t)input & 15u) != 0) {
        return TE_STATUS_UNSUPPORTED;
    }
    return te_hip::launch_matvec(weights, ggml_type, input, cols, rows, out, te_hip::as_stream(stream));
}

extern "C" te_status te_hip_rmsnorm_f32(const float *input, const float *weight, size_t rows, size_t len,
                                        float epsilon, float *out, void *stream) {
    if (input == nullptr || weight == nullptr || out == nullptr || rows == 0 || len == 0 || epsilon <= 0.0f) {
        return TE_STATUS_INVALID_ARGUMENT;  // the reference check (ops.c:279)
    }
    if (rows > 0x7fffffffu || len > 0x7fffffffu) {
        return TE_STATUS_UNSUPPORTED;
    }
    return te_hip::launch_rmsnorm(input, weight, rows, len, epsilon, out, te_hip::as_stream(stream));
}

extern "C" te_status te_hip_swiglu_f32(const float *gate, const float *up, size_t len, float *out, void *stream) {
    if (gate == nullptr || up == nullptr || out == nullptr || len == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return te_hip::launch_swiglu(gate, up, len, out, te_hip::as_stream(stream));
}

extern "C" te_status te_hip_add_f32(const float *lhs, const float *rhs, size_t len, float *out, void *stream) {
    if (lhs == nullptr || rhs == nullptr || out == nullptr || len == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return te_hip::launch_add(lhs, rhs, len, out, te_hip::as_stream(stream));
}

extern "C" te_status te_hip_argmax_f32(const float *values, size_t len, uint32_t *out_index, void *stream) {
    if (values == nullptr || out_index == nullptr || len == 0 || len > 0xffffffffu) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return te_hip::launch_argmax(values, len, out_index, te_hip::as_stream(stream));
}
