// Measurement only: the fp16 MFMA rate this device sustains with operands in
// registers, so prefill throughput can be read against an achievable ceiling
// as well as the 2.5 PFLOP/s data-sheet figure.  No counterpart in the
// reference; nothing on the attention path calls it.
//
// Each wave runs `iters` rounds of 8 independent v_mfma_f32_16x16x32_f16
// (16*16*32*2 FLOP each) on register operands, 8 waves per workgroup, and
// stores one float per thread so the work is not dead.
#include "te_hip_common.h"

namespace {

constexpr int kCalThreads = 512;

__global__ __launch_bounds__(kCalThreads, 1) void mfma_rate_kernel(float *out, int iters, float seed) {
    f16x8 a;
    f16x8 b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (f16)(seed * (float)((threadIdx.x + i) & 7));
        b[i] = (f16)(seed * (float)(8 - i));
    }
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[j] = mfma16x16x32(a, b, acc[j]);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    }
    out[(size_t)blockIdx.x * kCalThreads + threadIdx.x] = s;
}

}  // namespace

extern "C" TE_API te_status te_hip_calibrate_mfma_f16(size_t blocks, size_t iters, float *out, void *stream) {
    if (out == nullptr || blocks == 0 || blocks > 65535 || iters == 0 || iters > (1u << 20)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    mfma_rate_kernel<<<dim3((unsigned)blocks), dim3(kCalThreads), 0, te_hip::as_stream(stream)>>>(out, (int)iters,
                                                                                                  1.0e-3f);
    return te_hip::launch_status();
}
