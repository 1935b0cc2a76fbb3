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
// codes, value code * d; F32 rows are plain floats.  One wave owns R rows; lane
// l takes blocks l, l + 64, ... of every row, so the wave reads each row as one
// contiguous stream, and the lane's 32 input values (and their sum) serve all R
// rows.  Per block, with u = the code read as an unsigned byte or nibble:
//   Q4_0: d * (sum_j u_j x_j - 8 sum_j x_j)
//   Q8_0: d * (sum_j u_j x_j - 128 sum_j x_j),  u = code ^ 0x80 (code + 128)
// so each element costs one byte -> float conversion and one FMA.  Blocks are
// 18 / 34 bytes, so a block starts 0 or 2 bytes past a 4-byte boundary: the
// lane reads the covering dwords (never a byte past the block's last
// dword-pair) and funnel-shifts.  The lane sums are reduced across the wave.
// Summation order differs from the reference's sequential loop: results agree
// within fp32 rounding of the row's terms, not bit for bit.
//
// HBM bytes per launch (the roofline unit): rows * row_bytes + cols * 4 + rows * 4.
#include "te_hip_common.h"

#include <float.h>
#include <math.h>

namespace {

constexpr uint32_t kGgmlF32 = 0;
constexpr uint32_t kGgmlQ4_0 = 2;
constexpr uint32_t kGgmlQ8_0 = 8;
constexpr int kMatvecWaves = 4;

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
    for (uint32_t i = threadIdx.x; i < len; i += 1024) {
        const float v = values[i];
        if (v > bv) {  // strictly greater: the first maximum of this thread's stride
            bv = v;
            bi = i;
        }
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

te_status launch_matvec(const void *weights, uint32_t ggml_type, const float *input, size_t cols, size_t rows,
                        float *out, hipStream_t stream) {
    const size_t row_bytes = ggml_row_bytes(ggml_type, cols);
    // Each row takes R = 1, 2 or 4 waves' worth of rows so large tensors
    // amortise the input loads while small ones still fill the device.
    const size_t waves_wanted = (size_t)device_compute_units() * 16;
    const int R = rows >= 4 * waves_wanted ? 4 : rows >= 2 * waves_wanted ? 2 : 1;
    const size_t rows_per_wg = (size_t)R * kMatvecWaves;
    const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg));
    const unsigned char *w = static_cast<const unsigned char *>(weights);
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
