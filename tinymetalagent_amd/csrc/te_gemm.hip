// Quantized GEMM for batched prompt prefill: Y[m][n] = sum_k X[m][k] * W[n][k]
// (+ R[m][n]) for M prompt rows at once against a GGUF Q4_0 / Q8_0 weight
// matrix W [N][K] -- the projections of te_qwen_prefill_prompt_batch
// (reference c/src/qwen.c:630-905), whose per-row meaning is te_model_matvec_f32
// (ops.c:177-269) applied to every row.
//
// Activations (quant_act_kernel): each row, after an optional RMSNorm or
// SwiGLU pre-op, is cut into 32-value blocks.  A block of largest magnitude
// m = f * 2^E (f in [0.5, 1)) is scaled by 2^(14-E) and rounded to integers v,
// |v| <= 2^14, stored as two balanced int8 digits v = 256*hi + lo
// (lo in [-128, 127]) plus the block scale 2^(E-14).  Rounding moves each value
// by at most 2^-14 of its block's largest magnitude.
//
// Products (gemm_q_kernel): one 32-value block of a row against one GGUF
// block of a weight row is a K = 32 step of v_mfma_i32_32x32x32_i8 -- the
// integer sum of hi * q, shifted by 8, then the lo * q sum accumulated onto it
// by a second MFMA: exact, |C| <= 32 * 2^14 * 128 < 2^31.  Each block's integer
// result is scaled by (activation scale * weight block scale) and accumulated
// in fp32.  Weight codes enter the MFMA as int8: Q8_0 as stored, Q4_0 nibbles
// n as n - 8 (the reference's (q - 8) * d, ops.c:15-21).
//
// Layout: the digit planes are stored in 32 x 32 tiles ([M/32][K/32][32 rows]
// [32 k] int8), so one wave's operand for one block is 1 KiB contiguous.
//
// Tiles: a 256-thread workgroup computes a 64 x 64 block of Y as four 32 x 32
// wave tiles; the K loop takes two blocks per step (two independent MFMA
// chains) and stages the activation scales of the workgroup's 64 rows in
// LDS, 8 blocks at a time.  Where the output tiles alone would not fill the GPU,
// the K range is split over grid.z and a second kernel adds the partial sums
// in a fixed order (deterministic).
#include "te_hip_common.h"

#include <float.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr uint32_t kQ4_0 = 2, kQ8_0 = 8;
constexpr int kActThreads = 256;
constexpr int kChunkBlocks = 8;

__device__ __forceinline__ float half_bits(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

enum ActPre { kActPlain = 0, kActRmsNorm = 1, kActSwiGLU = 2 };

// One 32-value block of digits: lane j of a half wave holds value j (every
// lane of the half takes part; only `store` lanes write).
__device__ __forceinline__ void quant_block(float v, size_t row, int K, int b, int lane, int8_t *__restrict__ hi,
                                            int8_t *__restrict__ lo, float *__restrict__ scales, bool store = true) {
    float m = fabsf(v);
    for (int off = 16; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off, 32));
    }
    int q = 0;
    float s;
    if (!(m <= FLT_MAX)) {  // inf or NaN in the block: its products are NaN
        s = __builtin_nanf("");
    } else if (m == 0.0f) {
        s = 0.0f;
    } else {
        int E;
        (void)frexpf(m, &E);
        const int e = min(14 - E, 126);  // blocks below 2^-112 round towards 0
        q = (int)rintf(ldexpf(v, e));
        s = ldexpf(1.0f, -e);
    }
    if (store) {
        const int l8 = ((q + 128) & 255) - 128;
        const size_t t = (((row >> 5) * (size_t)(K >> 5) + b) << 10) + ((row & 31) << 5) + lane;
        hi[t] = (int8_t)((q - l8) >> 8);
        lo[t] = (int8_t)l8;
        if (lane == 0) {
            scales[row * (size_t)(K / 32) + b] = s;
        }
    }
}

// One 32-value block of digits held as eight consecutive values by each of
// four adjacent lanes (g = lane & 3 holds values 8g .. 8g + 7): the same
// digits and scale as quant_block (the block maximum does not depend on the
// order it is taken in), stored as 8-byte pieces where `vec`.
__device__ __forceinline__ void quant_block8(const float (&v)[8], size_t row, int K, int b, int g,
                                             int8_t *__restrict__ hi, int8_t *__restrict__ lo,
                                             float *__restrict__ scales, bool vec) {
    float m = fabsf(v[0]);
#pragma unroll
    for (int j = 1; j < 8; ++j) {
        m = fmaxf(m, fabsf(v[j]));
    }
    // the quad's maximum by DPP moves (lanes xor 1, then xor 2)
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    int q[8] = {};
    float s;
    if (!(m <= FLT_MAX)) {  // inf or NaN in the block: its products are NaN
        s = __builtin_nanf("");
    } else if (m == 0.0f) {
        s = 0.0f;
    } else {
        int E;
        (void)frexpf(m, &E);
        const int e = min(14 - E, 126);  // blocks below 2^-112 round towards 0
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            q[j] = (int)rintf(ldexpf(v[j], e));
        }
        s = ldexpf(1.0f, -e);
    }
    uint32_t h[2] = {0, 0}, l[2] = {0, 0};
    // q = 256 * hi + lo with lo in [-128, 127]: hi = (q + 128) >> 8, and lo's
    // byte is q's low byte
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        h[j >> 2] |= (uint32_t)(((q[j] + 128) >> 8) & 255) << (8 * (j & 3));
        l[j >> 2] |= (uint32_t)(q[j] & 255) << (8 * (j & 3));
    }
    const size_t t = (((row >> 5) * (size_t)(K >> 5) + b) << 10) + ((row & 31) << 5) + 8 * g;
    if (vec) {
        *reinterpret_cast<uint2 *>(hi + t) = make_uint2(h[0], h[1]);
        *reinterpret_cast<uint2 *>(lo + t) = make_uint2(l[0], l[1]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            hi[t + j] = (int8_t)(h[j >> 2] >> (8 * (j & 3)));
            lo[t + j] = (int8_t)(l[j >> 2] >> (8 * (j & 3)));
        }
    }
    if (g == 0) {
        scales[row * (size_t)(K / 32) + b] = s;
    }
}

// Eight consecutive floats: two 16-byte loads where `vec`.
__device__ __forceinline__ void load8(const float *p, bool vec, float (&v)[8]) {
    if (vec) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        const float4 c = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = c.x, v[5] = c.y, v[6] = c.z, v[7] = c.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = p[j];
        }
    }
}

__device__ __forceinline__ void store8(float *p, bool vec, const float (&v)[8]) {
    if (vec) {
        *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[j] = v[j];
        }
    }
}

// The fp64 sum of squares of a row whose thread t holds columns
// 8t + 2048i .. +7 (i = 0, 1, ...): each thread adds its values in column
// order, the wave's lanes are added by an xor butterfly and the workgroup's
// four waves in wave order.  quant_act_kernel<kActRmsNorm> and
// gemm_reduce_rms_kernel both sum this way, so their RMSNorm factors agree
// bit for bit.  (te_rmsnorm_f32, ops.c:272-293, sums in fp64 in index order.)
__device__ __forceinline__ double row_sum_squares(double ss) {
    __shared__ double part[kActThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        ss += __shfl_xor(ss, off);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kActThreads / 64; ++w) {
        t += part[w];
    }
    return t;
}

// x' = pre(x), then digits and block scales.  Thread t of a workgroup holds
// eight consecutive values of block t / 4 of a pass of 64 blocks; without a
// row-wide norm the gridDim.y workgroups of a row take every gridDim.y-th
// pass, else one workgroup takes the row (the norm's sum first, then the
// digits from a second read of the row).
// planes: hi and lo, int8 in 32 x 32 tiles [M/32][K/32][32][32]; scales [M][K/32] fp32.
// `vec`: every pointer 16-byte aligned (16-byte loads, 8-byte digit stores).
constexpr int kActPass = kActThreads * 8;
template <int PRE>
__global__ __launch_bounds__(kActThreads) void quant_act_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ x2,
                                                                const float *__restrict__ norm_w, float eps,
                                                                int K, int8_t *__restrict__ hi,
                                                                int8_t *__restrict__ lo,
                                                                float *__restrict__ scales, bool vec) {
    const size_t row = blockIdx.x;
    const float *xr = x + row * (size_t)K;
    const int c0 = 8 * (int)threadIdx.x;
    float rms = 1.0f;
    if (PRE == kActRmsNorm) {
        double ss = 0.0;
        for (int c = c0; c < K; c += kActPass) {
            float v[8];
            load8(xr + c, vec, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const double d = (double)v[j];
                ss += d * d;
            }
        }
        rms = 1.0f / sqrtf((float)(row_sum_squares(ss) / (double)K) + eps);
    }
    for (int c = c0 + blockIdx.y * kActPass; c < K; c += kActPass * gridDim.y) {
        float v[8], w2[8];
        load8(xr + c, vec, v);
        if (PRE == kActRmsNorm) {
            load8(norm_w + c, vec, w2);
        } else if (PRE == kActSwiGLU) {
            load8(x2 + row * (size_t)K + c, vec, w2);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (PRE == kActRmsNorm) {
                v[j] = v[j] * rms * w2[j];
            } else if (PRE == kActSwiGLU) {
                v[j] = v[j] / (1.0f + expf(-v[j])) * w2[j];  // te_swiglu_f32 (ops.c:397-405)
            }
        }
        quant_block8(v, row, K, c >> 5, threadIdx.x & 3, hi, lo, scales, vec);
    }
}

// 16 weight codes of one GGUF block as int8: for Q4_0 the low (k < 16) or
// high (k >= 16) nibbles of the 16 code bytes, n - 8; for Q8_0 the bytes
// 16 * half .. +15.  `blk` is 2-byte aligned.
template <uint32_t TYPE>
__device__ __forceinline__ v4i weight_codes(const unsigned char *blk, int half, float &d) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(blk);
    d = half_bits(h[0]);
    uint32_t w[4];
    const int base = TYPE == kQ4_0 ? 1 : 1 + 8 * half;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = (uint32_t)h[base + 2 * k] | (uint32_t)h[base + 2 * k + 1] << 16;
    }
    v4i out;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (TYPE == kQ4_0) {
            // n ^ 8 is n - 8 as a 4-bit two's complement value; sign-extend per byte
            const uint32_t x = ((half ? w[k] >> 4 : w[k]) & 0x0f0f0f0fu) ^ 0x08080808u;
            out[k] = (int)(x | ((x & 0x08080808u) * 0x1eu));
        } else {
            out[k] = (int)w[k];
        }
    }
    return out;
}

// grid (N/64, M/64, splits): split z covers blocks [z * per, (z + 1) * per).
// With one split the result (+ resid) goes to `out`; otherwise the split's
// partial sums go to part[z][M][N].
template <uint32_t TYPE, bool RESID>
__global__ __launch_bounds__(256) void gemm_q_kernel(const unsigned char *__restrict__ w, size_t row_bytes,
                                                     const int8_t *__restrict__ hi, const int8_t *__restrict__ lo,
                                                     const float *__restrict__ scales, int M, int N, int K, int per,
                                                     float *out, const float *resid, float *part) {
    constexpr int kBlockBytes = TYPE == kQ4_0 ? 18 : 34;
    __shared__ __align__(16) float s_lds[kChunkBlocks][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane & 31, kh = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;
    const int m_wg = blockIdx.y * 64;
    const int m0 = m_wg + wm * 32, n0 = blockIdx.x * 64 + wn * 32;
    const int b_col = min(n0 + lr, N - 1);
    const int nb = K / 32;
    const int kb0 = blockIdx.z * per, kb1 = min(nb, kb0 + per);
    // rows of a partial 32-row tile read padding; their results are not stored
    const size_t a_tile = (size_t)(min(m0, (M - 1) & ~31) >> 5) * nb;
    const int a_lane = lr * 32 + kh * 16;
    const unsigned char *b_row = w + (size_t)b_col * row_bytes;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = 0.0f;
    }
    auto load = [&](int b, v4i &ah, v4i &al, v4i &bq, float &d) {
        const size_t o = ((a_tile + b) << 10) + a_lane;
        ah = *reinterpret_cast<const v4i *>(hi + o);
        al = *reinterpret_cast<const v4i *>(lo + o);
        bq = weight_codes<TYPE>(b_row + (size_t)b * kBlockBytes, kh, d);
    };
    // two blocks per step: two independent MFMA chains in flight
    auto step = [&](int bb, const v4i &ah, const v4i &al, const v4i &bq, float d, v16i &c) {
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bq, v16i{}, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            c[r] <<= 8;
        }
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bq, c, 0, 0, 0);
        (void)bb;
        (void)d;
    };
    auto scale_add = [&](int bb, const v16i &c, float d) {
        // lane holds column lr of rows 8 * (r / 4) + 4 * kh + r % 4
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 s4 = *reinterpret_cast<const float4 *>(&s_lds[bb][wm * 32 + 8 * g + 4 * kh]);
            acc[4 * g + 0] = fmaf((float)c[4 * g + 0], s4.x * d, acc[4 * g + 0]);
            acc[4 * g + 1] = fmaf((float)c[4 * g + 1], s4.y * d, acc[4 * g + 1]);
            acc[4 * g + 2] = fmaf((float)c[4 * g + 2], s4.z * d, acc[4 * g + 2]);
            acc[4 * g + 3] = fmaf((float)c[4 * g + 3], s4.w * d, acc[4 * g + 3]);
        }
    };
    for (int b = kb0; b < kb1; b += 2) {
        const int bb = (b - kb0) & (kChunkBlocks - 1);
        if (bb == 0) {
            __syncthreads();
            for (int t = threadIdx.x; t < kChunkBlocks * 64; t += 256) {
                const int rr = t & 63, cb = b + (t >> 6);
                const int row = min(m_wg + rr, M - 1);
                s_lds[t >> 6][rr] = cb < kb1 ? scales[(size_t)row * nb + cb] : 0.0f;
            }
            __syncthreads();
        }
        v4i ah0, al0, bq0, ah1, al1, bq1;
        float d0, d1;
        load(b, ah0, al0, bq0, d0);
        const bool two = b + 1 < kb1;
        if (two) {
            load(b + 1, ah1, al1, bq1, d1);
        }
        v16i c0, c1;
        step(bb, ah0, al0, bq0, d0, c0);
        if (two) {
            step(bb + 1, ah1, al1, bq1, d1, c1);
        }
        scale_add(bb, c0, d0);
        if (two) {
            scale_add(bb + 1, c1, d1);
        }
    }
    const int col = n0 + lr;
    if (col < N) {
        float *dst = gridDim.z > 1 ? part + (size_t)blockIdx.z * M * N : out;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (row < M) {
                const size_t o = (size_t)row * N + col;
                dst[o] = RESID && gridDim.z == 1 ? resid[o] + acc[r] : acc[r];
            }
        }
    }
}

// The same products with the weights staged through LDS: each K step takes a
// chunk of kWChunk GGUF blocks of the workgroup's 64 weight rows, read as
// 16-byte coalesced loads (a row's chunk is contiguous: 144 B for Q4_0, 272 B
// for Q8_0, 16-byte aligned when the tensor and its row length are), one
// chunk ahead of its use and double-buffered in LDS with a row pitch of an odd
// dword count, so the wave's 32 rows read a block without bank conflicts.  A
// lane's block (fp16 scale + codes) is a 5-dword LDS window whose byte
// alignment is the same for every lane (the block index's parity), unpacked by
// byte alignment and nibble masks.  Activation digits are prefetched one
// block ahead.  Needs row_bytes % 16 == 0 and a 16-byte aligned tensor;
// split boundaries fall on whole chunks.
constexpr int kWChunk = 8;

// Weight matrices of one launch (same K and type), whose 64-column tiles are
// numbered one after another along grid.x: segment i holds tiles
// tile_end[i-1] .. tile_end[i]-1.  Split-K partial sums are laid out
// [split][segment][M][n] (n_off: columns before segment i).
constexpr int kMaxGemmSegs = 3;
struct GemmSegsArg {
    const unsigned char *w[kMaxGemmSegs];
    float *out[kMaxGemmSegs];
    const float *resid[kMaxGemmSegs];
    int n[kMaxGemmSegs];
    int tile_end[kMaxGemmSegs];
    int n_off[kMaxGemmSegs + 1];
    int nseg;
};

// GLU form's output: the SwiGLU of the paired gate / up products as the next
// GEMM's activation digits (quant_act_kernel's planes and scales, K = n).
struct GluDigits {
    int8_t *hi;
    int8_t *lo;
    float *scales;
};

// GLU = true: sg.w[0] / sg.w[1] are the gate / up matrices (n rows each) and
// a workgroup's 64 weight rows pair the same 32 rows of both (wave wn = 0 the
// gate products, wn = 1 the up products of the same 32 columns); the epilogue
// forms silu(gate) * up with te_swiglu_f32's operations and writes its digits
// (one 32-value block per row and workgroup), exactly as quant_act_kernel
// would from the two products.  One K split.
template <uint32_t TYPE, bool RESID, bool GLU>
__global__ __launch_bounds__(256) void gemm_q2_kernel(GemmSegsArg sg, size_t row_bytes,
                                                      const int8_t *__restrict__ hi, const int8_t *__restrict__ lo,
                                                      const float *__restrict__ scales, int M, int K, int per,
                                                      float *part, GluDigits glu) {
    // this workgroup's segment (uniform)
    int seg = 0;
#pragma unroll
    for (int i = 1; i < kMaxGemmSegs; ++i) {
        seg += (i < sg.nseg && (int)blockIdx.x >= sg.tile_end[i - 1]) ? 1 : 0;
    }
    const unsigned char *__restrict__ w = sg.w[seg];
    const int N = sg.n[seg];
    float *out = sg.out[seg];
    const float *resid = sg.resid[seg];
    const int n_tile = (int)blockIdx.x - (seg > 0 ? sg.tile_end[seg - 1] : 0);
    const uintptr_t up_delta = GLU ? (uintptr_t)sg.w[1] - (uintptr_t)sg.w[0] : 0;  // modulo 2^64
    constexpr int BB = TYPE == kQ4_0 ? 18 : 34;     // bytes per GGUF block
    constexpr int CB = kWChunk * BB;                // bytes of one row's chunk
    constexpr int PITCH = CB + 4;                   // LDS row pitch (CB is a multiple of 16)
    constexpr int RC = CB / 16;                     // 16-byte pieces per row chunk
    constexpr int PIECES = 64 * RC;
    constexpr int PPT = (PIECES + 255) / 256;       // pieces per thread
    static_assert(CB % 16 == 0 && (PITCH / 4) % 2 == 1, "chunk layout");
    __shared__ __align__(16) unsigned char w_lds[2][64 * PITCH];
    __shared__ __align__(16) float s_lds[2][kWChunk][64];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, kh = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;
    const int m_wg = blockIdx.y * 64, n_wg = n_tile * (GLU ? 32 : 64);
    const int m0 = m_wg + wm * 32, n0 = GLU ? n_wg : n_wg + wn * 32;
    const int nb = K / 32;
    const int kb0 = blockIdx.z * per, kb1 = min(nb, kb0 + per);
    const size_t a_tile = (size_t)(min(m0, (M - 1) & ~31) >> 5) * nb;
    const int a_lane = lr * 32 + kh * 16;
    const int n_chunks = (kb1 - kb0 + kWChunk - 1) / kWChunk;

    // chunk c's pieces and activation scales: global -> registers (a chunk
    // ahead), then registers -> LDS buffer. Q8_0 stages its 5 pieces per
    // thread in two halves (the first stored and the second loaded at the
    // chunk's midpoint): only 3 pieces are held in registers, which keeps the
    // kernel at <= 128 VGPRs (4 waves per SIMD instead of 3). Q4_0 (3 pieces)
    // stages the chunk at once: halves measured slower there.
    constexpr int SPT = kWChunk * 64 / 256;  // scales per thread
    constexpr bool HALVES = TYPE == kQ8_0;
    constexpr int PA = HALVES ? (PPT + 1) / 2 : PPT;  // pieces of the first half
    using P0 = std::integral_constant<int, 0>;
    using PMid = std::integral_constant<int, PA>;
    using PEnd = std::integral_constant<int, PPT>;
    using PLast = std::integral_constant<int, HALVES ? PA : 0>;  // first piece stored at the chunk's end
    uint4 wreg[PA];
    float sreg[SPT];
    auto load_scales = [&](int c) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int t = tid + 256 * i;
            const int rr = t & 63, cb = kb0 + c * kWChunk + (t >> 6);
            const int row = min(m_wg + rr, M - 1);
            sreg[i] = cb < kb1 ? scales[(size_t)row * nb + cb] : 0.0f;
        }
    };
    // pieces I0 .. I1 - 1 of chunk c into wreg[0 ..]
    auto load_pieces = [&](int c, auto i0, auto i1) {
        constexpr int I0 = decltype(i0)::value, I1 = decltype(i1)::value;
        const size_t cbyte = (size_t)(kb0 + c * kWChunk) * BB;
#pragma unroll
        for (int i = I0; i < I1; ++i) {
            const int item = tid + 256 * i;
            const int r = item / RC, j = item % RC;
            const size_t off = cbyte + 16 * (size_t)j;
            wreg[i - I0] = make_uint4(0u, 0u, 0u, 0u);
            if (item < PIECES && off < row_bytes) {  // a piece is wholly in its row or wholly past it
                // GLU: rows 0..31 of the tile from the gate matrix, 32..63 from
                // up (a byte offset from gate: a per-piece pointer select
                // costs registers that lower occupancy)
                const int row = min(n_wg + (GLU ? (r & 31) : r), N - 1);
                const uintptr_t base = (uintptr_t)w + (GLU ? (uintptr_t)(r >> 5) * up_delta : 0);
                wreg[i - I0] = *reinterpret_cast<const uint4 *>(base + (size_t)row * row_bytes + off);
            }
        }
    };
    auto store_pieces = [&](int buf, auto i0, auto i1) {
        constexpr int I0 = decltype(i0)::value, I1 = decltype(i1)::value;
#pragma unroll
        for (int i = I0; i < I1; ++i) {
            const int item = tid + 256 * i;
            if (item < PIECES) {
                uint32_t *dst = reinterpret_cast<uint32_t *>(&w_lds[buf][(item / RC) * PITCH + 16 * (item % RC)]);
                dst[0] = wreg[i - I0].x;
                dst[1] = wreg[i - I0].y;
                dst[2] = wreg[i - I0].z;
                dst[3] = wreg[i - I0].w;
            }
        }
    };
    auto store_scales = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int t = tid + 256 * i;
            s_lds[buf][t >> 6][t & 63] = sreg[i];
        }
    };
    // activation digits of block b, one block ahead of use (two ahead took 8
    // more VGPRs and measured 3-4 % slower)
    v4i ah[2], al[2];
    auto load_a = [&](int b, int slot) {
        if (b < kb1) {
            const size_t o = ((a_tile + b) << 10) + a_lane;
            ah[slot] = *reinterpret_cast<const v4i *>(hi + o);
            al[slot] = *reinterpret_cast<const v4i *>(lo + o);
        }
    };
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = 0.0f;
    }
    if (n_chunks > 0) {
        load_scales(0);
        load_pieces(0, P0{}, PMid{});
        store_pieces(0, P0{}, PMid{});
        load_pieces(0, PMid{}, PEnd{});
        store_pieces(0, PMid{}, PEnd{});
        store_scales(0);
        load_a(kb0, 0);
    }
    __syncthreads();
    for (int c = 0; c < n_chunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < n_chunks) {
            load_scales(c + 1);
            load_pieces(c + 1, P0{}, PMid{});
        }
        const unsigned char *wrow = &w_lds[buf][(wn * 32 + lr) * PITCH];
#pragma unroll
        for (int bb = 0; bb < kWChunk; ++bb) {
            const int b = kb0 + c * kWChunk + bb;
            load_a(b + 1, (bb + 1) & 1);
            if (HALVES && bb == kWChunk / 2 && c + 1 < n_chunks) {
                // buffer buf ^ 1 was last read before the previous chunk's barrier
                store_pieces(buf ^ 1, P0{}, PMid{});
                load_pieces(c + 1, PMid{}, PEnd{});
            }
            if (b < kb1) {
                // the block's fp16 scale and 16 codes of this lane's k half: a
                // 5-dword window starting at the block's dword (Q8_0: the half's)
                const int blk = bb * BB;                                  // compile-time per bb
                const int start = TYPE == kQ4_0 ? blk : blk + 16 * kh;   // the lane's codes are at start + 2
                const uint32_t *win = reinterpret_cast<const uint32_t *>(wrow + (start & ~3));
                uint32_t dw[5];
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    dw[i] = win[i];
                }
                // fp16 scale: bytes blk, blk + 1 (the same dword as the window's
                // first for Q4_0)
                const uint32_t dwin =
                    TYPE == kQ4_0 ? dw[0] : *reinterpret_cast<const uint32_t *>(wrow + (blk & ~3));
                const float d = half_bits((blk & 2) ? dwin >> 16 : dwin & 0xffffu);
                // codes: bytes start + 2 + 4k .. +3 for k = 0..3, at byte 2 or 4
                // of the window (blk is 0 or 2 mod 4, as start is)
                const int sh = (blk & 3) + 2;
                uint32_t code[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    code[k] = sh == 4 ? dw[k + 1] : __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
                }
                v4i bq;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (TYPE == kQ4_0) {
                        // per byte n in 0..15: (n + 0x78) ^ 0x80 is n - 8 as int8
                        // (no byte carries: n + 0x78 <= 0x87)
                        const uint32_t n4 = (kh ? code[k] >> 4 : code[k]) & 0x0f0f0f0fu;
                        bq[k] = (int)((n4 + 0x78787878u) ^ 0x80808080u);
                    } else {
                        bq[k] = (int)code[k];
                    }
                }
                const int slot = bb & 1;
                v16i cc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah[slot], bq, v16i{}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    cc[r] <<= 8;
                }
                cc = __builtin_amdgcn_mfma_i32_32x32x32_i8(al[slot], bq, cc, 0, 0, 0);
                // lane holds column lr of rows 8 * (r / 4) + 4 * kh + r % 4
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 s4 = *reinterpret_cast<const float4 *>(&s_lds[buf][bb][wm * 32 + 8 * g + 4 * kh]);
                    acc[4 * g + 0] = fmaf((float)cc[4 * g + 0], s4.x * d, acc[4 * g + 0]);
                    acc[4 * g + 1] = fmaf((float)cc[4 * g + 1], s4.y * d, acc[4 * g + 1]);
                    acc[4 * g + 2] = fmaf((float)cc[4 * g + 2], s4.z * d, acc[4 * g + 2]);
                    acc[4 * g + 3] = fmaf((float)cc[4 * g + 3], s4.w * d, acc[4 * g + 3]);
                }
            }
        }
        if (c + 1 < n_chunks) {
            store_pieces(buf ^ 1, PLast{}, PEnd{});
            store_scales(buf ^ 1);
        }
        __syncthreads();
    }
    const int col = n0 + lr;
    if constexpr (GLU) {
        // up products -> LDS (the weight stages are free after the last
        // barrier); the gate wave forms h and its digits
        float *xch = reinterpret_cast<float *>(&w_lds[0][0]);
        static_assert(sizeof(w_lds) >= 2 * 16 * 64 * sizeof(float), "exchange fits the weight stages");
        if (wn == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                xch[(wm * 16 + r) * 64 + lane] = acc[r];
            }
        }
        __syncthreads();
        if (wn == 0) {
            const int b = n_wg >> 5;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + 8 * (r >> 2) + 4 * kh + (r & 3);
                const float g = acc[r];
                const float u = xch[(wm * 16 + r) * 64 + lane];
                const float v = g / (1.0f + expf(-g)) * u;  // te_swiglu_f32 (ops.c:397-405)
                quant_block(v, (size_t)row, N, b, lr, glu.hi, glu.lo, glu.scales, row < M);
            }
        }
        return;
    }
    if (col < N) {
        float *dst = gridDim.z > 1 ? part + ((size_t)blockIdx.z * sg.n_off[sg.nseg] + sg.n_off[seg]) * M : out;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (row < M) {
                const size_t o = (size_t)row * N + col;
                dst[o] = RESID && gridDim.z == 1 ? resid[o] + acc[r] : acc[r];
            }
        }
    }
}

// part[0][i] + part[1][i] + ... + part[splits-1][i], added in split order,
// for W consecutive elements at i (W = 4: 16-byte loads); the splits' loads
// are issued eight at a time.
template <int W>
struct Vals {
    float v[W];
};
template <int W>
__device__ __forceinline__ Vals<W> load_vals(const float *p) {
    Vals<W> r;
    if constexpr (W == 4) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        r.v[0] = a.x, r.v[1] = a.y, r.v[2] = a.z, r.v[3] = a.w;
    } else {
        r.v[0] = *p;
    }
    return r;
}
template <int W>
__device__ __forceinline__ void store_vals(float *p, const Vals<W> &r) {
    if constexpr (W == 4) {
        *reinterpret_cast<float4 *>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
    } else {
        *p = r.v[0];
    }
}
template <int W>
__device__ __forceinline__ Vals<W> sum_splits(const float *__restrict__ part, int splits, size_t count, size_t i) {
    Vals<W> a = load_vals<W>(part + i);
    for (int z0 = 1; z0 < splits; z0 += 8) {
        Vals<W> b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (z0 + u < splits) {
                b[u] = load_vals<W>(part + (size_t)(z0 + u) * count + i);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (z0 + u < splits) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    a.v[j] += b[u].v[j];
                }
            }
        }
    }
    return a;
}

// out = (resid +) the splits' partial sums, added in split order, for every
// segment of a segmented launch (element i of the [segment][M][n] order),
// W elements per thread (W = 4: every pointer 16-byte aligned and every
// segment boundary M * n_off a multiple of 4, so four elements never straddle
// one).
template <int W>
__global__ __launch_bounds__(256) void gemm_reduce_segs_kernel(const float *__restrict__ part, int splits, int M,
                                                               GemmSegsArg sg) {
    const size_t count = (size_t)M * sg.n_off[sg.nseg];
    for (size_t i = (blockIdx.x * (size_t)256 + threadIdx.x) * W; i < count; i += (size_t)gridDim.x * 256 * W) {
        int seg = 0;
#pragma unroll
        for (int t = 1; t < kMaxGemmSegs; ++t) {
            seg += (t < sg.nseg && i >= (size_t)M * sg.n_off[t]) ? 1 : 0;
        }
        Vals<W> a = sum_splits<W>(part, splits, count, i);
        const size_t j = i - (size_t)M * sg.n_off[seg];
        if (sg.resid[seg] != nullptr) {
            const Vals<W> r = load_vals<W>(sg.resid[seg] + j);
#pragma unroll
            for (int k = 0; k < W; ++k) {
                a.v[k] = r.v[k] + a.v[k];
            }
        }
        store_vals<W>(sg.out[seg] + j, a);
    }
}

// gemm_reduce_kernel's sums for one row (resid + the splits' partial sums in
// split order -> out), then that row's RMSNorm digits into hi / lo / scales,
// exactly as quant_act_kernel<kActRmsNorm> computes them from out: thread t
// holds columns 8t .. 8t + 7, summed into the fp64 sum of squares in
// row_sum_squares's order, and quantizes them as quant_act_kernel's thread t
// does.  One workgroup per row, N <= kActPass, N % 32 == 0,
// splits <= kRmsSplits.  Every load, the norm weights' included, is issued
// before the first store (out may be resid), so all of a thread's loads are
// in flight together.
constexpr int kRmsSplits = 8;
__global__ __launch_bounds__(kActThreads) void gemm_reduce_rms_kernel(const float *__restrict__ part, int splits,
                                                                      size_t count, const float *resid, float *out,
                                                                      int N, const float *__restrict__ norm_w,
                                                                      float eps, int8_t *__restrict__ hi,
                                                                      int8_t *__restrict__ lo,
                                                                      float *__restrict__ scales, bool vec) {
    const size_t row = blockIdx.x;
    const int c = 8 * (int)threadIdx.x;
    const bool mine = c < N;
    const int cl = mine ? c : 0;  // threads past the row load column 0 and store nothing
    const size_t o = row * (size_t)N + cl;
    float pv[kRmsSplits][8], rv[8] = {}, wv[8];
#pragma unroll
    for (int z = 0; z < kRmsSplits; ++z) {
        if (z < splits) {
            load8(part + (size_t)z * count + o, vec, pv[z]);
        }
    }
    if (resid != nullptr) {
        load8(resid + o, vec, rv);
    }
    load8(norm_w + cl, vec, wv);
    float xv[8];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float a = pv[0][j];
#pragma unroll
        for (int z = 1; z < kRmsSplits; ++z) {
            if (z < splits) {
                a += pv[z][j];
            }
        }
        xv[j] = resid != nullptr ? rv[j] + a : a;
        const double d = (double)xv[j];
        ss += mine ? d * d : 0.0;
    }
    if (mine) {
        store8(out + o, vec, xv);
    }
    const float rms = 1.0f / sqrtf((float)(row_sum_squares(ss) / (double)N) + eps);
    if (mine) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xv[j] = xv[j] * rms * wv[j];
        }
        quant_block8(xv, row, N, c >> 5, threadIdx.x & 3, hi, lo, scales, vec);
    }
}

// out = (resid +) the splits' partial sums, added in split order, W
// elements per thread (W = 4: count % 4 == 0 and every pointer 16-byte
// aligned).
template <int W>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float *__restrict__ part, int splits, size_t count,
                                                          const float *resid, float *out) {
    for (size_t i = (blockIdx.x * (size_t)256 + threadIdx.x) * W; i < count; i += (size_t)gridDim.x * 256 * W) {
        Vals<W> a = sum_splits<W>(part, splits, count, i);
        if (resid != nullptr) {
            const Vals<W> r = load_vals<W>(resid + i);
#pragma unroll
            for (int k = 0; k < W; ++k) {
                a.v[k] = r.v[k] + a.v[k];
            }
        }
        store_vals<W>(out + i, a);
    }
}

}  // namespace

namespace te_hip {

static bool aligned16(const void *p) {
    return ((uintptr_t)p & 15u) == 0;
}

// digit planes padded to whole 32-row tiles
static size_t plane_bytes(size_t rows, size_t cols) {
    return (rows + 31) / 32 * 32 * cols;
}

size_t act_plane_bytes(size_t rows, size_t cols) {
    return plane_bytes(rows, cols);
}

size_t act_buffer_bytes(size_t rows, size_t cols) {
    return 2 * plane_bytes(rows, cols) + rows * (cols / 32) * sizeof(float);
}

te_status launch_quant_act(int pre, const float *x, const float *x2, const float *norm_w, float eps, size_t rows,
                           size_t cols, void *act, hipStream_t stream) {
    if (rows == 0 || cols == 0 || cols % 32 != 0 || rows > 0x7fffffffu || cols > (1u << 24)) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t planes = plane_bytes(rows, cols);
    int8_t *hi = static_cast<int8_t *>(act);
    int8_t *lo = hi + planes;
    float *scales = reinterpret_cast<float *>(lo + planes);
    const bool vec = aligned16(x) && aligned16(act) && (pre != kActSwiGLU || aligned16(x2)) &&
                     (pre != kActRmsNorm || aligned16(norm_w));
    // without a row-wide norm, the row's passes of kActPass values are spread over workgroups
    const dim3 grid((unsigned)rows, pre == kActRmsNorm ? 1u : (unsigned)std::max<size_t>(1, cols / kActPass));
    if (pre == kActRmsNorm) {
        quant_act_kernel<kActRmsNorm>
            <<<grid, kActThreads, 0, stream>>>(x, x2, norm_w, eps, (int)cols, hi, lo, scales, vec);
    } else if (pre == kActSwiGLU) {
        quant_act_kernel<kActSwiGLU><<<grid, kActThreads, 0, stream>>>(x, x2, norm_w, eps, (int)cols, hi, lo, scales, vec);
    } else {
        quant_act_kernel<kActPlain><<<grid, kActThreads, 0, stream>>>(x, x2, norm_w, eps, (int)cols, hi, lo, scales, vec);
    }
    return launch_status();
}

te_status launch_gemm_q_segs(uint32_t ggml_type, const GemmSeg *segs, int nseg, const void *act, size_t rows,
                             size_t k, float *partials, size_t partial_bytes, hipStream_t stream,
                             const GemmRmsDigits *post) {
    if ((ggml_type != kQ4_0 && ggml_type != kQ8_0) || k % 32 != 0 || rows == 0 || rows > 0x7fffffffu ||
        k > (1u << 24) || nseg < 1 || nseg > kMaxGemmSegs) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (post != nullptr && nseg != 1) {
        return TE_STATUS_INVALID_ARGUMENT;  // the digits are of one output
    }
    const size_t row_bytes = k / 32 * (ggml_type == kQ4_0 ? 18 : 34);
    // the LDS-staged kernel where a row's chunks are 16-byte aligned (its
    // split boundaries fall on whole chunks), else one gemm_q_kernel launch
    // per matrix
    bool staged = row_bytes % 16 == 0 && getenv("TE_HIP_GEMM_V1") == nullptr;
    size_t n_total = 0, tiles_n = 0;
    for (int i = 0; i < nseg; ++i) {
        if (segs[i].n == 0 || segs[i].n > 0x7fffffffu || ((size_t)segs[i].w & 1u) != 0 ||
            (segs[i].resid != nullptr) != (segs[0].resid != nullptr)) {
            return TE_STATUS_UNSUPPORTED;
        }
        staged = staged && ((size_t)segs[i].w & 15u) == 0;
        n_total += segs[i].n;
        tiles_n += (segs[i].n + 63) / 64;
    }
    if (n_total > 0x7fffffffu) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t planes = plane_bytes(rows, k);
    const int8_t *hi = static_cast<const int8_t *>(act);
    const int8_t *lo = hi + planes;
    const float *scales = reinterpret_cast<const float *>(lo + planes);
    if (!staged && nseg > 1) {
        for (int i = 0; i < nseg; ++i) {
            const te_status st = launch_gemm_q_segs(ggml_type, &segs[i], 1, act, rows, k, partials, partial_bytes,
                                                    stream, nullptr);
            if (st != TE_STATUS_OK) {
                return st;
            }
        }
        return TE_STATUS_OK;
    }
    const size_t tiles = tiles_n * ((rows + 63) / 64);
    const size_t nb = k / 32;
    // split K until the grid covers four workgroups per CU (measured: down at 512 rows 175 -> 159 us
    // against two; eight gains nothing more), keeping >= 8 blocks per split
    size_t splits = 1;
    size_t per_cu = 4;
    if (const char *env = getenv("TE_HIP_GEMM_SPLIT_TARGET")) {  // tuning override: workgroups per CU
        const long v = strtol(env, nullptr, 10);
        per_cu = v >= 1 && v <= 16 ? (size_t)v : per_cu;
    }
    const size_t want = per_cu * (size_t)device_compute_units();
    while (partials != nullptr && tiles * splits < want && nb / (splits * 2) >= 8 &&
           splits * 2 * rows * n_total * sizeof(float) <= partial_bytes) {
        splits *= 2;
    }
    int per = (int)((nb + splits - 1) / splits);
    if (staged) {
        per = (per + kWChunk - 1) / kWChunk * kWChunk;
        splits = (nb + (size_t)per - 1) / (size_t)per;
    }
    const dim3 grid((unsigned)tiles_n, (unsigned)((rows + 63) / 64), (unsigned)splits);
    const bool resid = segs[0].resid != nullptr;
    GemmSegsArg sg = {};
    sg.nseg = nseg;
    int tile_end = 0;
    for (int i = 0; i < nseg; ++i) {
        sg.w[i] = static_cast<const unsigned char *>(segs[i].w);
        sg.out[i] = segs[i].out;
        sg.resid[i] = segs[i].resid;
        sg.n[i] = (int)segs[i].n;
        tile_end += (int)((segs[i].n + 63) / 64);
        sg.tile_end[i] = tile_end;
        sg.n_off[i + 1] = sg.n_off[i] + (int)segs[i].n;
    }
    const unsigned char *w = sg.w[0];
    const size_t n = segs[0].n;
    float *out = segs[0].out;
    const float *res = segs[0].resid;
#define TE_GEMM(T, R)                                                                                              \
    do {                                                                                                           \
        if (staged) {                                                                                              \
            gemm_q2_kernel<T, R, false><<<grid, 256, 0, stream>>>(sg, row_bytes, hi, lo, scales, (int)rows,       \
                                                                  (int)k, per, partials, GluDigits{});             \
        } else {                                                                                                   \
            gemm_q_kernel<T, R><<<grid, 256, 0, stream>>>(w, row_bytes, hi, lo, scales, (int)rows, (int)n, (int)k, \
                                                          per, out, res, partials);                                \
        }                                                                                                          \
    } while (0)
    if (ggml_type == kQ4_0) {
        if (resid) {
            TE_GEMM(kQ4_0, true);
        } else {
            TE_GEMM(kQ4_0, false);
        }
    } else {
        if (resid) {
            TE_GEMM(kQ8_0, true);
        } else {
            TE_GEMM(kQ8_0, false);
        }
    }
#undef TE_GEMM
    // the RMSNorm digits of a single output: fused into the split-K sums
    // where the row fits the fused kernel, else from out afterwards
    const bool rms = post != nullptr && nseg == 1 && n % 32 == 0;
    bool digits_done = false;
    if (splits > 1) {
        const size_t count = rows * n_total;
        bool vec = aligned16(partials) && count % 4 == 0;
        for (int i = 0; i < nseg; ++i) {
            vec = vec && aligned16(sg.out[i]) && aligned16(sg.resid[i]) && (rows * (size_t)sg.n_off[i + 1]) % 4 == 0;
        }
        const int width = vec ? 4 : 1;
        const unsigned blocks = (unsigned)std::min<size_t>((count / width + 255) / 256, 4096);
        const char *env = getenv("TE_HIP_GEMM_REDUCE_RMS");
        if (rms && n <= (size_t)kActPass && splits <= (size_t)kRmsSplits && !(env != nullptr && env[0] == '0')) {
            const size_t planes_out = plane_bytes(rows, n);
            int8_t *ohi = static_cast<int8_t *>(post->act_out);
            int8_t *olo = ohi + planes_out;
            float *osc = reinterpret_cast<float *>(olo + planes_out);
            gemm_reduce_rms_kernel<<<(unsigned)rows, kActThreads, 0, stream>>>(
                partials, (int)splits, count, res, out, (int)n, post->norm_w, post->eps, ohi, olo, osc,
                vec && aligned16(post->norm_w) && aligned16(post->act_out));
            digits_done = true;
        } else if (nseg == 1) {
            if (vec) {
                gemm_reduce_kernel<4><<<blocks, 256, 0, stream>>>(partials, (int)splits, count, res, out);
            } else {
                gemm_reduce_kernel<1><<<blocks, 256, 0, stream>>>(partials, (int)splits, count, res, out);
            }
        } else if (vec) {
            gemm_reduce_segs_kernel<4><<<blocks, 256, 0, stream>>>(partials, (int)splits, (int)rows, sg);
        } else {
            gemm_reduce_segs_kernel<1><<<blocks, 256, 0, stream>>>(partials, (int)splits, (int)rows, sg);
        }
    }
    te_status st = launch_status();
    if (st == TE_STATUS_OK && post != nullptr && !digits_done) {
        st = launch_quant_act(kActRmsNorm, out, nullptr, post->norm_w, post->eps, rows, n, post->act_out, stream);
    }
    return st;
}

te_status launch_gemm_q(const void *weights, uint32_t ggml_type, const void *act, size_t rows, size_t n, size_t k,
                        float *out, const float *resid, float *partials, size_t partial_bytes, hipStream_t stream) {
    const GemmSeg seg = {weights, out, resid, n};
    return launch_gemm_q_segs(ggml_type, &seg, 1, act, rows, k, partials, partial_bytes, stream, nullptr);
}

te_status launch_gemm_q_rms(const void *weights, uint32_t ggml_type, const void *act, size_t rows, size_t n,
                            size_t k, float *out, const float *resid, float *partials, size_t partial_bytes,
                            const float *norm_w, float eps, void *act_out, hipStream_t stream) {
    const GemmSeg seg = {weights, out, resid, n};
    const GemmRmsDigits post = {norm_w, eps, act_out};
    return launch_gemm_q_segs(ggml_type, &seg, 1, act, rows, k, partials, partial_bytes, stream, &post);
}

te_status launch_gemm_glu_q(uint32_t ggml_type, const void *gate_w, const void *up_w, const void *act, size_t rows,
                            size_t n, size_t k, void *act_out, hipStream_t stream, bool *launched) {
    *launched = false;
    const size_t row_bytes = k / 32 * (ggml_type == kQ4_0 ? 18 : 34);
    const size_t tiles = n / 32 * ((rows + 63) / 64);
    const char *env = getenv("TE_HIP_GEMM_GLU");
    if ((ggml_type != kQ4_0 && ggml_type != kQ8_0) || k % 32 != 0 || n % 32 != 0 || rows == 0 ||
        rows > 0x7fffffffu || n > 0x7fffffffu || k > (1u << 24) || row_bytes % 16 != 0 ||
        ((size_t)gate_w & 15u) != 0 || ((size_t)up_w & 15u) != 0 || getenv("TE_HIP_GEMM_V1") != nullptr ||
        (env != nullptr && env[0] == '0') ||
        (tiles < (size_t)device_compute_units() && !(env != nullptr && env[0] == '1'))) {
        return TE_STATUS_OK;  // not launched: the caller runs the two GEMMs and the SwiGLU digits
    }
    const size_t planes = plane_bytes(rows, k);
    const int8_t *hi = static_cast<const int8_t *>(act);
    const int8_t *lo = hi + planes;
    const float *scales = reinterpret_cast<const float *>(lo + planes);
    const size_t out_planes = plane_bytes(rows, n);
    GluDigits d;
    d.hi = static_cast<int8_t *>(act_out);
    d.lo = d.hi + out_planes;
    d.scales = reinterpret_cast<float *>(d.lo + out_planes);
    GemmSegsArg sg = {};
    sg.nseg = 1;
    sg.w[0] = static_cast<const unsigned char *>(gate_w);
    sg.w[1] = static_cast<const unsigned char *>(up_w);
    sg.n[0] = (int)n;
    sg.tile_end[0] = (int)(n / 32);
    sg.n_off[1] = (int)n;
    const dim3 grid((unsigned)(n / 32), (unsigned)((rows + 63) / 64), 1);
    const int per = (int)(k / 32);
    if (ggml_type == kQ4_0) {
        gemm_q2_kernel<kQ4_0, false, true><<<grid, 256, 0, stream>>>(sg, row_bytes, hi, lo, scales, (int)rows, (int)k,
                                                                     per, nullptr, d);
    } else {
        gemm_q2_kernel<kQ8_0, false, true><<<grid, 256, 0, stream>>>(sg, row_bytes, hi, lo, scales, (int)rows, (int)k,
                                                                     per, nullptr, d);
    }
    *launched = true;
    return launch_status();
}

}  // namespace te_hip

// Test entry point: Y = pre(X) * W^T (+ R) through the two launches above, on
// device pointers; `act` is scratch of te_hip_gemm_act_bytes(rows, k) bytes.
extern "C" size_t te_hip_gemm_act_bytes(size_t rows, size_t k) {
    return te_hip::act_buffer_bytes(rows, k);
}

extern "C" te_status te_hip_gemm_q_f32(const void *weights, uint32_t ggml_type, const float *x, const float *x2,
                                       const float *norm_w, float epsilon, int pre, size_t rows, size_t n, size_t k,
                                       float *out, const float *resid, void *act, float *partials,
                                       size_t partial_bytes, void *stream) {
    if (weights == nullptr || x == nullptr || out == nullptr || act == nullptr || pre < 0 || pre > 2 ||
        (pre == kActRmsNorm && (norm_w == nullptr || !(epsilon > 0.0f))) || (pre == kActSwiGLU && x2 == nullptr)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = te_hip::as_stream(stream);
    te_status st = te_hip::launch_quant_act(pre, x, x2, norm_w, epsilon, rows, k, act, s);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return te_hip::launch_gemm_q(weights, ggml_type, act, rows, n, k, out, resid, partials, partial_bytes, s);
}
