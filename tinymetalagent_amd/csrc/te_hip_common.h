// Shared device types, MFMA wrappers and launch helpers for the gfx950
// attention kernels.  CDNA4 only: wave64, v_mfma_f32_16x16x32_f16 (gfx950),
// v_mfma_f32_16x16x4_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>

#include "te_hip_backend.h"

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// log2(e): softmax runs in the base-2 domain, exp(x) == exp2(x * log2(e)).
#define TE_LOG2E 1.4426950408889634f

// D = A(16 x 32) * B(32 x 16) + C, fp16 operands, fp32 accumulation.
// Lane l holds A row (l % 16) and B column (l % 16), eight K-elements each
// (the same K-subset for A and B, selected by l / 16); D lane l holds column
// (l % 16), rows 4*(l / 16) + {0,1,2,3}.
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// fp32 MFMA: A(16 x 4) * B(4 x 16); lane l holds A[l%16][l/16], B[l/16][l%16].
__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16 (gfx950): every lane passes an LDS address of 4 halves;
// within each 16-lane group, lane i receives element i%4 of the 4 halves read
// by source lanes 4j + i/4, j = 0..3 (checked on the device: a 16 x 4 block of
// halves comes back transposed).
__device__ __forceinline__ f16x4 lds_read_tr16(const f16 *p) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s16x4 __attribute__((address_space(3))) *)(const_cast<f16 *>(p)));
    return __builtin_bit_cast(f16x4, v);
}

__device__ __forceinline__ float wave_xor_max16_32(float v) {
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

__device__ __forceinline__ float wave_xor_sum16_32(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Split x into hi + lo fp16 parts (hi = RNE(x), lo = RNE(x - hi)) so that a
// pair of fp16 MFMAs reproduces an fp32 operand to ~2^-22 relative.
__device__ __forceinline__ void split_f16(float x, f16 &hi, f16 &lo) {
    hi = (f16)x;
    lo = (f16)(x - (float)hi);
}

// Host-side helpers shared by the launchers.
namespace te_hip {

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline te_status launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TE_STATUS_OK : TE_STATUS_RUNTIME_ERROR;
}

// Decode split-K geometry, shared by the split-K and combine launches and the
// workspace-size query so all three agree.
struct DecodeGeometry {
    int chunk;       // cache positions per workgroup (multiple of 32)
    int max_chunks;  // chunks of the longest sequence
};

// Compute units of the current device (256 when the query fails).
int device_compute_units();

// The library's process-wide mutex: held by the host-pointer entry points, and
// by device entry points called without a workspace while they enqueue work
// that uses a library-owned buffer.
std::mutex &library_mutex();

// Library-owned device buffers for entry points called without a workspace,
// one per purpose, grown on demand (a growth frees the old buffer, which
// waits for the device) and kept.  The caller holds library_mutex() from the
// request until its last use of the buffer is enqueued; calls sharing a
// buffer must go to one stream.
enum LibraryBuffer { kLibBufDecode = 0, kLibBufPrefillVt = 1, kLibBufCount = 2 };
te_status library_buffer(LibraryBuffer which, size_t bytes, void **ptr);

// Decode-layer vector operations (te_vecops.hip); arguments already checked.
size_t ggml_row_bytes(uint32_t ggml_type, size_t cols);  // 0 = type / cols not supported
te_status launch_matvec(const void *weights, uint32_t ggml_type, const float *input, size_t cols, size_t rows,
                        float *out, hipStream_t stream);
te_status launch_rmsnorm(const float *input, const float *weight, size_t rows, size_t len, float epsilon, float *out,
                         hipStream_t stream);
te_status launch_swiglu(const float *gate, const float *up, size_t len, float *out, hipStream_t stream);
te_status launch_add(const float *lhs, const float *rhs, size_t len, float *out, hipStream_t stream);
te_status launch_argmax(const float *values, size_t len, uint32_t *out_index, hipStream_t stream);
// Row `row` of a [rows][cols] F32 / Q4_0 / Q8_0 tensor as fp32 (Q4_0 / Q8_0: cols % 32 == 0);
// the tensor may start at any byte address.
te_status launch_dequant_row(const void *weights, uint32_t ggml_type, size_t cols, size_t row, float *out,
                             hipStream_t stream);
// Rows rows[0 .. n) (a device array of valid row indices) into out [n][cols].
te_status launch_dequant_rows(const void *weights, uint32_t ggml_type, size_t cols, const uint32_t *rows, size_t n,
                              float *out, hipStream_t stream);

// Batched-prefill GEMM (te_gemm.hip).  launch_quant_act turns rows x cols fp32
// activations (after pre-op 0 none, 1 RMSNorm with norm_w / eps, 2 SwiGLU
// with x2 as `up`) into the digit planes + block scales held in `act`
// (act_buffer_bytes(rows, cols) bytes); launch_gemm_q then writes
// out[m][n] = sum_k act[m][k] W[n][k] (+ resid[m][n]) for a Q4_0 / Q8_0
// weight tensor W [n][k] at a 2-byte aligned address.
size_t act_buffer_bytes(size_t rows, size_t cols);
// The layout inside `act`: the hi plane at act, the lo plane at
// act + act_plane_bytes(rows, cols), the fp32 block scales after the lo plane.
size_t act_plane_bytes(size_t rows, size_t cols);
te_status launch_quant_act(int pre, const float *x, const float *x2, const float *norm_w, float eps, size_t rows,
                           size_t cols, void *act, hipStream_t stream);
// `partials` (partial_bytes, may be NULL) lets small output grids split K.
te_status launch_gemm_q(const void *weights, uint32_t ggml_type, const void *act, size_t rows, size_t n, size_t k,
                        float *out, const float *resid, float *partials, size_t partial_bytes, hipStream_t stream);
// Up to three weight matrices of the same K against the same activations in
// one launch (their column tiles numbered one after another, one split-K
// reduction for all): segs[i].out[m][r] = sum_k act[m][k] W_i[r][k]
// (+ segs[i].resid[m][r]), r < segs[i].n.  Either every segment has a
// residual or none.  partial_bytes bounds the splits by rows * sum(n).
struct GemmSeg {
    const void *w;
    float *out;
    const float *resid;
    size_t n;
};
// With `post` (one segment): afterwards also the RMSNorm digits of out
// (launch_quant_act(1, out, nullptr, norm_w, eps) into act_out, the same
// bits), fused into the split-K sums where they run (TE_HIP_GEMM_REDUCE_RMS=0:
// separate launches).  act_out may be act.
struct GemmRmsDigits {
    const float *norm_w;
    float eps;
    void *act_out;
};
te_status launch_gemm_q_segs(uint32_t ggml_type, const GemmSeg *segs, int nseg, const void *act, size_t rows,
                             size_t k, float *partials, size_t partial_bytes, hipStream_t stream,
                             const GemmRmsDigits *post = nullptr);
// launch_gemm_q, then the RMSNorm digits of out (see GemmRmsDigits).
te_status launch_gemm_q_rms(const void *weights, uint32_t ggml_type, const void *act, size_t rows, size_t n,
                            size_t k, float *out, const float *resid, float *partials, size_t partial_bytes,
                            const float *norm_w, float eps, void *act_out, hipStream_t stream);
// Gate and up [n][k] against the same activation digits in one launch whose
// tiles pair the same rows of both, writing silu(gate) * up as the down
// projection's digits into act_out (act_buffer_bytes(rows, n) bytes, the same
// digits launch_quant_act(2, gate, up) gives).  *launched = false (and
// nothing queued) where the shapes or alignment do not allow it, n % 32 != 0,
// or the grid would not cover the GPU: the caller then runs the two GEMMs and
// launch_quant_act.  TE_HIP_GEMM_GLU=0 turns it off, =1 takes it for grids of
// any size.
te_status launch_gemm_glu_q(uint32_t ggml_type, const void *gate_w, const void *up_w, const void *act, size_t rows,
                            size_t n, size_t k, void *act_out, hipStream_t stream, bool *launched);

// te_hip_attention_prefill_step_vt_f16 (te_prefill.hip; arguments as there)
// with the attention output as the next GEMM's digits: with act_out set, the
// launch_quant_act(0) digits of the output rows [seqs*layers*tokens][heads *
// head_dim] go to act_out (act_buffer_bytes of that shape), formed by the
// attention kernel from the rows it holds, and `out` is not written.  Only
// without a key split (workspace NULL or one split): else UNSUPPORTED.
te_status launch_prefill_step_vt(const float *query, const float *k_new, const float *v_new, const float *q_bias,
                                 const float *k_bias, const float *v_bias, const float *rope_cos,
                                 const float *rope_sin, uint16_t *key_cache, uint16_t *value_cache,
                                 uint16_t *value_cache_t, size_t seqs, size_t layers, size_t tokens,
                                 size_t base_position, size_t context_tokens, size_t heads, size_t kv_heads,
                                 size_t head_dim, float *out, void *act_out, void *workspace, size_t workspace_bytes,
                                 hipStream_t stream);

// One weight matrix of a fused GEMV launch: out[r] = W[r] . x' (+ resid[r] when
// resid is set; resid may equal out), r < rows.
struct GemvSeg {
    const void *w;
    float *out;
    const float *resid;
    size_t rows;
};
enum GemvPre { kGemvPlain = 0, kGemvRmsNorm = 1, kGemvSwiGLU = 2 };
// Up to three matrices of one type and width `cols` against one input x' =
// x (plain), RMSNorm(x) * norm_w (as te_rmsnorm_f32) or silu(x) * x2 (as
// te_swiglu_f32).  One streamed launch when the weights allow it; otherwise the
// pre-operation into `xtmp` (cols floats), then te_hip_matvec_f32 per matrix
// (into `ytmp`, rows floats, when it has a residual) and the residual add.
te_status launch_gemv(uint32_t ggml_type, GemvPre pre, const GemvSeg *segs, int nseg, size_t cols, const float *x,
                      const float *x2, const float *norm_w, float eps, float *xtmp, float *ytmp,
                      hipStream_t stream);
// The gate and up projections of one RMSNorm input in one streamed launch
// whose tiles hold the same rows of both, writing h[r] = silu(gate[r]) * up[r]
// (as te_swiglu_f32) and neither projection.  *launched stays false, with OK,
// when the shapes do not suit it (then launch_gemv and a SwiGLU pre-operation
// on the down projection do the same work).
te_status launch_gemv_glu(uint32_t ggml_type, const void *gate_w, const void *up_w, size_t rows, size_t cols,
                          const float *x, const float *norm_w, float eps, float *h, hipStream_t stream,
                          bool *launched);
// One matrix against the attention output merged from one (seq, layer)'s
// split-K partials (te_hip_attention_decode_step_splitk_f16's workspace:
// o [heads][max_chunks][head_dim], then (m, l) [heads][max_chunks][2]) while
// the launch stages its input: the decode step's merge launch folded into the
// Wo projection.  *launched stays false, with OK and nothing queued, when it
// does not apply: more than kGemvMergeMaxChunks chunks, shapes the streamed
// kernel does not take, or an input wider than one float4 per thread; the
// caller then runs the merge and launch_gemv.
constexpr int kGemvMergeMaxChunks = 12;
te_status launch_gemv_merge(uint32_t ggml_type, const GemvSeg &seg, size_t cols, const float *part_o,
                            const float *part_ml, size_t chunks, size_t max_chunks, size_t head_dim,
                            hipStream_t stream, bool *launched);

DecodeGeometry decode_geometry(const size_t *positions, size_t position, size_t seqs, size_t layers,
                               size_t kv_heads);

size_t decode_workspace_bytes(const DecodeGeometry &g, size_t seqs, size_t layers, size_t heads, size_t head_dim);

// Upper bound on decode_geometry(...).max_chunks over every set of positions
// whose largest is <= max_position; non-decreasing in max_position.
size_t decode_chunks_bound(size_t max_position, size_t layers, size_t kv_heads);

// Chunk length of the fp32-cache decode (te_attention_decode_f32): a power-of-two
// multiple of 512 positions giving at most 4096 chunks.
int f32_decode_chunk(size_t position);

// Internal launchers used by the host-pointer wrappers (te_hip_runtime.hip).
te_status launch_decode_f32(const float *query, const float *key_cache, const float *value_cache,
                            size_t position, size_t heads, size_t kv_heads, size_t head_dim, float *out,
                            float *part_o, float *part_ml, hipStream_t stream);
te_status launch_kv_append(const float *k, const float *v, const float *k_bias, const float *v_bias,
                           const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
                           uint16_t *value_cache, size_t seqs, size_t layers, size_t tokens, size_t base_position,
                           size_t context_tokens, size_t kv_heads, size_t head_dim, hipStream_t stream);
// The fused prefill step's k / v append (launch_kv_append's arithmetic) and
// the V^T rows of the chunk's positions (launch_value_transpose's layout,
// row pitch ctx_pad) in one launch; head_dim 64 or 128.
te_status launch_kv_append_vt(const float *k, const float *v, const float *k_bias, const float *v_bias,
                              const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
                              uint16_t *value_cache, uint16_t *value_t, size_t sl_count, size_t layers,
                              size_t tokens, size_t base_position, size_t context_tokens, size_t ctx_pad,
                              size_t kv_heads, size_t head_dim, hipStream_t stream);
te_status launch_rope_rows(float *values, size_t heads, size_t head_dim, const float *cos_row,
                           const float *sin_row, hipStream_t stream);
te_status launch_mma_kat(int mode, const float *query, const float *key_t, const float *value, int k_cols,
                         int q_base, float *out, hipStream_t stream);

// In-library profiling of te_generate (TINYENGINE_PROFILE set and not "0",
// the reference's switch, qwen.c:2216-2219).  While a thread's profile is
// active, the layer flows record a HIP event on their stream after each piece
// of work (prof_mark); prof_flush waits for the last one and adds the time
// from the previous event to each piece's phases, split by the given shares
// (the weight rows of a launch that covers several matrices).  The phases are
// the reference's matvec buckets plus the embedding rows, the attention and
// the other elementwise work (normalisation, activation quantisation, argmax).  Thread-local: contexts on other threads keep their own.
enum ProfPhase {
    kProfQ, kProfK, kProfV, kProfO, kProfGate, kProfUp, kProfDown, kProfLmHead, kProfOther,
    kProfEmbed, kProfAttention, kProfElementwise, kProfCount
};
struct ProfShare {
    ProfPhase phase;
    double weight;
};
bool prof_active();
void prof_start();                   // reset and activate this thread's profile
void prof_stop();
void prof_begin(hipStream_t stream);  // the reference point of the next mark
void prof_mark(hipStream_t stream, const ProfShare *shares, int n);
inline void prof_mark(hipStream_t stream, ProfPhase phase) {
    const ProfShare one = {phase, 1.0};
    prof_mark(stream, &one, 1);
}
te_status prof_flush();              // synchronise and account the recorded marks
double prof_ms(ProfPhase phase);
unsigned long long prof_calls(ProfPhase phase);

// Backend call profile (TINYENGINE_METAL_PROFILE set and not "0", the
// reference's switch and buckets, metal_backend_runtime.mm.inc:132-244).
// A layer-flow entry point holds a BackendTimer over its whole call: when the
// switch is on it records a HIP event pair around the call's launches on its
// stream and, in finish(), waits for the second event and adds one call, the
// host wall time and the GPU time to its bucket.  Only the outermost timer
// of a thread records (a single-layer twin that calls the all-layers flow
// counts as one decode_layer / prefill_layer call).  Buckets with calls are
// printed at process exit, one line each in the reference's format.
enum BackendBucket {
    kBucketMatvecBatch, kBucketMatvecArgmax, kBucketQkv, kBucketQkvBatch, kBucketMlp, kBucketMlpBatch,
    kBucketPostAttnMlp, kBucketPostAttnMlpBatch, kBucketMatvec2, kBucketMatvec, kBucketDecodeLayer,
    kBucketDecodeAllLayers, kBucketDecodeProject, kBucketPrefillLayer, kBucketPrefillAllLayers, kBucketCount
};
class BackendTimer {
  public:
    BackendTimer(BackendBucket bucket, hipStream_t stream);
    ~BackendTimer();
    BackendTimer(const BackendTimer &) = delete;
    BackendTimer &operator=(const BackendTimer &) = delete;
    // Records the call when the switch is on and st is OK; returns st, or a
    // runtime error when waiting for the call's launches fails.
    te_status finish(te_status st);

  private:
    void release();
    BackendBucket bucket_;
    hipStream_t stream_;
    hipEvent_t e0_ = nullptr;
    hipEvent_t e1_ = nullptr;
    double t0_ms_ = 0.0;
    bool nested_ = false;
    bool on_ = false;
    bool done_ = false;
};

}  // namespace te_hip
