// fp32 MFMA attention tiles behind the te_hip_attention_{qk,tile,stream,causal}_mma_f32
// entry points -- the HIP twins of the reference MMA test kernels
// te_attention_{qk,tile,stream}_mma_f32_kernel and the 8-row causal use of
// te_attention_flash_mma_t_f32_kernel (metal_kernels.metal.inc:2502-2836,
// host side metal_backend.mm:30-373).
//
// One wave computes S = Q K^T (v_mfma_f32_16x16x4_f32, 8 query rows padded to
// 16), stores S in LDS, applies scale + (causal) mask + softmax per row in
// fp32, then O = P V with the same fp32 MFMA.  head_dim is 64 (host guard).
#include "te_hip_common.h"

#include <math.h>

namespace {

constexpr int kKatMaxKeys = 1024;
constexpr int kKatDim = 64;

__global__ __launch_bounds__(64) void mma_kat_kernel(int mode, const float *query, const float *key_t,
                                                     const float *value, int k_cols, int q_base, float *out) {
    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const int c = lane & 15;
    __shared__ float S[8][kKatMaxKeys];

    const int n_kt = (k_cols + 15) / 16;
    for (int kt = 0; kt < n_kt; ++kt) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        const int key = 16 * kt + c;
#pragma unroll
        for (int kk = 0; kk < kKatDim / 4; ++kk) {
            const int d = 4 * kk + g;
            const float a = c < 8 ? query[c * kKatDim + d] : 0.0f;
            const float b = key < k_cols ? key_t[d * k_cols + key] : 0.0f;
            acc = mfma16x16x4f32(a, b, acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r;
            if (row < 8 && key < k_cols) {
                S[row][key] = acc[r];
            }
        }
    }
    __syncthreads();

    if (mode == 0) {
        for (int i = lane; i < 8 * k_cols; i += 64) {
            out[i] = S[i / k_cols][i % k_cols];
        }
        return;
    }

    const float scale = 1.0f / sqrtf((float)kKatDim);
    for (int row = 0; row < 8; ++row) {
        float mx = -INFINITY;
        for (int k = lane; k < k_cols; k += 64) {
            float x = S[row][k] * scale;
            if (mode == 2 && k > q_base + row) {
                x = -INFINITY;
            }
            S[row][k] = x;
            mx = fmaxf(mx, x);
        }
        for (int off = 32; off > 0; off >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        }
        float sum = 0.0f;
        for (int k = lane; k < k_cols; k += 64) {
            const float e = expf(S[row][k] - mx);
            S[row][k] = e;
            sum += e;
        }
        for (int off = 32; off > 0; off >>= 1) {
            sum += __shfl_xor(sum, off, 64);
        }
        for (int k = lane; k < k_cols; k += 64) {
            S[row][k] = S[row][k] / sum;
        }
    }
    __syncthreads();

    // O = P V: A = P[16 rows][4 keys], B = V[4 keys][16 dims].
    for (int dt = 0; dt < kKatDim / 16; ++dt) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int ks = 0; ks < k_cols / 4; ++ks) {
            const int k = 4 * ks + g;
            const float a = c < 8 ? S[c][k] : 0.0f;
            const float b = value[k * kKatDim + 16 * dt + c];
            acc = mfma16x16x4f32(a, b, acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r;
            if (row < 8) {
                out[row * kKatDim + 16 * dt + c] = acc[r];
            }
        }
    }
}

}  // namespace

namespace te_hip {

// mode 0: QK^T scores; 1: softmax attention; 2: causal attention with q_base.
te_status launch_mma_kat(int mode, const float *query, const float *key_t, const float *value, int k_cols,
                         int q_base, float *out, hipStream_t stream) {
    if (k_cols <= 0 || k_cols > kKatMaxKeys || (mode != 0 && (k_cols % 4) != 0)) {
        return TE_STATUS_UNSUPPORTED;
    }
    mma_kat_kernel<<<1, 64, 0, stream>>>(mode, query, key_t, value, k_cols, q_base, out);
    return launch_status();
}

}  // namespace te_hip
