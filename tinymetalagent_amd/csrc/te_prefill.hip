// Batched-prefill causal attention (flash-attention forward) on fp16 MFMA.
//
// Semantics: row t of (seq, layer) is the reference decode at position
// base + t over the cache (qwen.c:810-824), i.e. the causal mask
// `key <= base + row` of te_attention_flash_mma_t_f32_kernel
// (metal_kernels.metal.inc:2767-2775), which also defines chunked prefill.
//
// Inputs: the fp16 K cache in the slot layout [sl][ctx][kv][D], and a
// transposed copy of the V cache, V^T [sl][kv][D][ctx_pad] (ctx_pad =
// context_tokens rounded up to 64): one row of keys per (kv head, dim), the
// layout the PV product reads (the reference Metal path keeps transposed
// copies the same way, te_qkv_bias_rope_cache_batch_t_f32).
//
// Work decomposition.  Query rows are cut into tiles of BM (128) rows.  One
// workgroup = 8 waves (two per SIMD) = the PAIR of tiles (n-1-i, i) of one
// head, processed one after the other, so every workgroup does the same causal
// work ((n+1) tiles' worth of key blocks).  Within a tile, wave w owns 32 rows
// (32*(w&3), two 16-row MFMA column blocks) and key half w>>2: a step of 128
// keys is two BN (64) key blocks, block 2*step + half for each wave, and the
// two halves' softmax states merge through LDS at the end of the tile.  The
// K and V^T of each step reach LDS by global_load_lds DMA, double-buffered:
// the DMA of step s+1 is in flight while step s is consumed, one barrier per
// step.  A key split (te_hip_attention_prefill_vt_f16 with a workspace) gives
// each workgroup a range of the steps and writes unnormalised partial rows.
//
//   S^T[64 keys x 32 rows] = K[64 x D] . Q^T[D x 32]            fp16 MFMA 16x16x32
//   O^T[D x 32 rows]      += V^T[D x 64] . P^T[64 x 32]         fp16 MFMA 16x16x32
//
// Key order.  The A operand of QK^T tile i (16 rows) takes, for row m, key
// sigma(i, m) = 32(i/2) + 8(m/4) + 4(i%2) + m%4 of the block.  The S^T result
// of lane (c, g) (query row c, result rows 4g + r) then holds keys
// 32(i/2) + 8g + 4(i%2) + r, so for the PV k-step ks (tiles 2ks, 2ks+1) each
// lane holds the eight consecutive keys 32ks + 8g .. +7: its P^T B operand,
// kept in registers, and its V^T A operand is one 16-byte LDS read (dim
// 16t + c, keys 32ks + 8g ..).
//
// LDS layouts (every operand read is a conflict-free ds_read_b128; the rates
// were measured on MI355X against a linear read):
//   K half block:  64 rows of 2D bytes; row 16i + c holds key sigma(i, c);
//                  16-byte chunk q of a row sits at slot q ^ (c & (D/8 - 1)).
//   V^T half block: D rows (dims) of 128 bytes (64 keys); chunk q (keys
//                  8q .. 8q+7) at slot q ^ (dim & 7).
// The DMA writes 1 KB per wave instruction with lane l at +16 l; each lane's
// global source is the chunk its slot holds.
//
// Softmax: fp32, base 2, per 32-key half of a block.  The weights are
// p = exp2(fma(s, qscale, -m_ref)) with qscale = log2(e)/sqrt(D) applied in
// fp32 to the raw score (the fp16 query is the operand as given, rounded
// once), against a per-row reference m_ref that is only raised (and O, l
// rescaled) when a row's maximum exceeds it by more than kLazyLog2 (log2
// units).  No row maximum is taken in the common case: a lane's fp16 weights
// are summed for l anyway, and while that sum stays <= 2^kLazyLog2 no weight
// exceeds 2^kLazyLog2, so m_ref is within kLazyLog2 of the maximum and O/l is
// exact.  A larger (or non-finite: the row's first keys, m_ref = -inf) sum
// sends the wave through the exact path: the half's row maxima, the new
// reference, the rescale and the weights again.  Q and P are single fp16
// operands.
//
// Work per (seq, layer): 2*heads*D*sum_t(base+t+1) MACs (QK^T + PV); the
// roofline unit is that count x2 FLOP.
#include "te_hip_common.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace {

constexpr int BM = 128;   // query rows per tile: 4 row groups of 32
constexpr int BN = 64;    // keys per block
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr float kLazyLog2 = 8.0f;
constexpr float kLazyMax = 256.0f;  // 2^kLazyLog2: the largest lane sum of one half's weights taken as is
constexpr int kMaxPrefillSplits = 32;
constexpr int kVtAlign = 64;  // V^T rows are padded to a multiple of this many positions
constexpr int kXcds = 8;      // MI355X: 8 XCDs, workgroups dispatched to them round-robin
constexpr int kQkAhead = 2;   // K operand read-ahead, in batches of two reads (four MFMAs)
constexpr int kPvAhead = 4;   // V^T operand read-ahead, in reads (two MFMAs each)

struct PrefillArgs {
    const f16 *q;            // fp16 rotated queries, or null when q32 is given
    const float *q32;        // fused step: fp32 queries, bias + RoPE applied on load
    const float *q_bias;     // fused step: [layers][heads*D] or null
    const float *rope_cos;   // fused step: [ctx][D/2]
    const float *rope_sin;
    const f16 *key_cache;
    const f16 *value_t;      // V^T [sl][kv][D][ctx_pad]
    float *out;
    int layers;
    int tokens;
    int base;
    int ctx;
    int ctx_pad;
    int heads;
    int kv_heads;
    int group;
    int n_qtiles;
    int paired;      // 1: unit = tile pair (n-1-i, i); 0: unit = one tile (a launch that fits one round)
    float qscale;  // log2(e)/sqrt(D), applied to the fp32 scores
    int splits;      // key splits: blockIdx.z = (seq*layers + layer) * splits + split
    float *part_o;   // splits > 1: unnormalised O per (split, seq*layer, row, head), else null
    float *part_ml;  // splits > 1: (m, l) per (split, seq*layer, row, head)
    // one split only: the output rows as the next GEMM's digits (hi / lo
    // planes in 32 x 32 tiles, fp32 block scales; te_gemm.hip's layout)
    // instead of fp32 rows; null: fp32 rows to `out`
    int8_t *dhi;
    int8_t *dlo;
    float *dscales;
#ifdef TE_PREFILL_PHASES
    unsigned *phase_log;  // [workgroup][wave][kPhases]: shader-clock cycles per phase, summed
#endif
};

// Four consecutive output values (columns col .. col + 3 of `row`, col % 4
// == 0) as digits: the eight lanes holding one 32-value block (lanes 8j ..
// 8j + 7, every lane of the wave taking part) share its largest magnitude,
// then each value becomes v = 256 * hi + lo at the block's scale -- the
// arithmetic of te_gemm.hip's quant_act_kernel<kActPlain>, so the digits are
// the ones that kernel makes from the fp32 rows.  K = the row length (heads *
// D); only `store` lanes write.
__device__ __forceinline__ void store_digits4(const f32x4 &v, size_t row, int K, int col, int8_t *__restrict__ hi,
                                              int8_t *__restrict__ lo, float *__restrict__ scales, bool store) {
    // the eight lanes' maximum by DPP moves (no LDS round trip): lanes xor 1
    // and xor 2 within each quad, then the half-row mirror (lane i <-> 7 - i)
    // joins the two quads
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    if (!store) {
        return;
    }
    int q[4] = {0, 0, 0, 0};
    float s;
    if (!(m <= __FLT_MAX__)) {  // inf or NaN in the block: its products are NaN
        s = __builtin_nanf("");
    } else if (m == 0.0f) {
        s = 0.0f;
    } else {
        int E;
        (void)frexpf(m, &E);
        const int e = min(14 - E, 126);  // blocks below 2^-112 round towards 0
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[j] = (int)rintf(ldexpf(v[j], e));
        }
        s = ldexpf(1.0f, -e);
    }
    // q = 256 * hi + lo with lo in [-128, 127]: hi = (q + 128) >> 8, and lo's
    // byte is q's low byte
    uint32_t h = 0, l = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h |= (uint32_t)(((q[j] + 128) >> 8) & 255) << (8 * j);
        l |= (uint32_t)(q[j] & 255) << (8 * j);
    }
    const int b = col >> 5;
    const size_t t = (((row >> 5) * (size_t)(K >> 5) + b) << 10) + ((row & 31) << 5) + (col & 31);
    *reinterpret_cast<uint32_t *>(hi + t) = h;
    *reinterpret_cast<uint32_t *>(lo + t) = l;
    if ((col & 31) == 0) {
        scales[row * (size_t)(K >> 5) + b] = s;
    }
}

// Phase instrumentation (a build with -DTE_PREFILL_PHASES only, see
// build.py --phases and bench.py --phases): each wave sums s_memtime deltas
// per phase of the step loop and writes them when it ends.
#ifdef TE_PREFILL_PHASES
constexpr int kPhases = 10;  // step start, QK^T + weights, merge put, checks + PV, merge finish, DMA wait, barrier, merge end, steps, prologue
#define TE_PHASE(i)                                                 \
    do {                                                            \
        const unsigned t_ = (unsigned)__builtin_amdgcn_s_memtime(); \
        ph[i] += t_ - t_last;                                       \
        t_last = t_;                                                \
    } while (0)
#else
#define TE_PHASE(i) \
    do {            \
    } while (0)
#endif

// Fused prefill step: query row `row` of (sl, layer) for head h, bias + RoPE at
// its position, rounded to the fp16 Q^T operand -- the operation order of
// rope_kv_append_kernel (FP contraction off), so the operand bits equal the
// fp16 queries the unfused path stores.  Lane (g, c) holds dims 8g + 32kk + j;
// the rotation partner of dim d < D/2 is d + D/2, at kk + KK/2 in the same lane.
template <int D>
__device__ __forceinline__ void load_q_rope(const PrefillArgs &a, int sl, int layer, int h, int row, int g,
                                            f16x8 (&qop)[D / 32]) {
#pragma clang fp contract(off)
    constexpr int KK = D / 32;
    constexpr int HALF = D / 2;
    const float *qrow = a.q32 + (((size_t)sl * a.tokens + row) * a.heads + h) * D;
    float x[KK][8];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const float4 v0 = *reinterpret_cast<const float4 *>(qrow + 8 * g + 32 * kk);
        const float4 v1 = *reinterpret_cast<const float4 *>(qrow + 8 * g + 32 * kk + 4);
        x[kk][0] = v0.x;
        x[kk][1] = v0.y;
        x[kk][2] = v0.z;
        x[kk][3] = v0.w;
        x[kk][4] = v1.x;
        x[kk][5] = v1.y;
        x[kk][6] = v1.z;
        x[kk][7] = v1.w;
    }
    if (a.q_bias != nullptr) {
        const float *qb = a.q_bias + ((size_t)layer * a.heads + h) * D;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const float4 b0 = *reinterpret_cast<const float4 *>(qb + 8 * g + 32 * kk);
            const float4 b1 = *reinterpret_cast<const float4 *>(qb + 8 * g + 32 * kk + 4);
            const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                x[kk][j] = x[kk][j] + bv[j];
            }
        }
    }
    const int pos = a.base + row;
    const float *cos_row = a.rope_cos + (size_t)pos * HALF;
    const float *sin_row = a.rope_sin + (size_t)pos * HALF;
#pragma unroll
    for (int kk = 0; kk < KK / 2; ++kk) {
        const float4 c0 = *reinterpret_cast<const float4 *>(cos_row + 8 * g + 32 * kk);
        const float4 c1 = *reinterpret_cast<const float4 *>(cos_row + 8 * g + 32 * kk + 4);
        const float4 s0 = *reinterpret_cast<const float4 *>(sin_row + 8 * g + 32 * kk);
        const float4 s1 = *reinterpret_cast<const float4 *>(sin_row + 8 * g + 32 * kk + 4);
        const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x0 = x[kk][j];
            const float x1 = x[kk + KK / 2][j];
            qop[kk][j] = (f16)(x0 * cv[j] - x1 * sv[j]);
            qop[kk + KK / 2][j] = (f16)(x1 * cv[j] + x0 * sv[j]);
        }
    }
}

__device__ __forceinline__ float xor_max_16_32(float v) {
    // lanes l, l^16, l^32, l^48 hold one row's values: two permlane swaps (VALU, no LDS)
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float xor_sum_16_32(float v) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Key of row m of QK^T tile i within a 64-key block (see "Key order").
__device__ __forceinline__ int sigma(int i, int m) { return 32 * (i >> 1) + 8 * (m >> 2) + 4 * (i & 1) + (m & 3); }

template <int D>
struct KHalf {
    static constexpr int ROWB = 2 * D;              // bytes per key row
    static constexpr int CPR = D / 8;               // 16-byte chunks per row
    static constexpr int BYTES = BN * ROWB;         // 16 KB (D = 128)
    static constexpr int LOADS = BYTES / 1024;      // DMA instructions per half block
};

template <int D>
struct VtHalf {
    static constexpr int ROWB = 2 * BN;             // 64 keys per dim row
    static constexpr int BYTES = D * ROWB;          // 16 KB (D = 128)
    static constexpr int LOADS = BYTES / 1024;
};

// Where a step issues the next step's DMA pieces (see dma_piece in the kernel).
struct DmaPlan {
    unsigned char *stage;  // the next step's staging buffer
    bool live;             // false: every piece goes to the sink
    int ksoff;             // scalar source offsets of the K and V^T pieces
    int vsoff;
};

// Q32: the fused step's fp32 queries (bias + RoPE on load), else fp16
// queries; one instantiation per query kind keeps each kind's registers to
// its own path.
template <int D, bool Q32>
__global__ __launch_bounds__(kThreads, 1) void prefill_causal_f16_kernel(PrefillArgs a) {
    typedef KHalf<D> KH;
    typedef VtHalf<D> VH;
    constexpr int KK = D / 32;                      // QK^T K-steps
    constexpr int NT = D / 16;                      // O^T output tiles
    constexpr int KB = KH::BYTES;
    constexpr int VB = VH::BYTES;
    constexpr int XFER = (4 * NT + 2) * 64;         // floats per wave in the merge exchange
    constexpr int STAGE = std::max(2 * KB + 2 * VB, kWaves * XFER * 4);
    static_assert(kWaves * KK * 64 * 16 <= STAGE, "the fused step's query exchange fits st1");
    constexpr int GROUPS = 2 * KH::LOADS + 2 * VH::LOADS;  // 1 KB loads per step
    constexpr int LOADS = GROUPS / kWaves;          // per wave per step
    static_assert(LOADS * kWaves == GROUPS, "staging loads must tile the step");

    // Two staging buffers as separate LDS variables: the compiler can then
    // tell the DMA into one from the operand reads of the other and does not
    // make those reads wait for the DMA (vmcnt).
    __shared__ __attribute__((aligned(1024))) unsigned char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) unsigned char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) unsigned char dma_sink[1024];  // target of idle DMA slots

    // Work unit of this workgroup.  Units are ordered pair-fastest, then the
    // heads of one KV group, then KV head, then (seq*layer, split); the
    // hardware hands workgroup ids to the 8 XCDs round-robin, so XCD x gets
    // units [x W/8, (x+1) W/8): the heads sharing one KV group's K/V run on
    // one XCD and its L2 holds that group's keys and values only.
    int unit = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
    const int n_units = (int)(gridDim.x * gridDim.y * gridDim.z);
    if (n_units % kXcds == 0) {
        unit = (unit % kXcds) * (n_units / kXcds) + unit / kXcds;
    }
    // (Heads are numbered kv head * group + head in group, so the head is
    // just hg mod heads.)  32-bit unsigned divisions, and none for the split
    // when there is one: every wave of the CU runs this on one scalar unit.
    const unsigned pair_u = (unsigned)unit % gridDim.x;
    const unsigned hg = (unsigned)unit / gridDim.x;  // (z, head)
    const int pair = (int)pair_u;
    const int h = (int)(hg % (unsigned)a.heads);
    const int zz = (int)(hg / (unsigned)a.heads);
    const int kvh = h / a.group;
    const int sl = a.splits == 1 ? zz : (int)((unsigned)zz / (unsigned)a.splits);
    const int split = a.splits == 1 ? 0 : zz - sl * a.splits;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = wave >> 2;  // key half: blocks 2*step + half
    const int g = lane >> 4;
    const int c = lane & 15;
#ifdef TE_PREFILL_PHASES
    unsigned ph[kPhases] = {};
    unsigned t_last = (unsigned)__builtin_amdgcn_s_memtime();
#endif
    const int long_tile = a.paired ? a.n_qtiles - 1 - pair : pair;
    // odd tile count: the middle tile has no partner; unpaired units are one tile
    const int n_tiles_wg = !a.paired || pair == long_tile ? 1 : 2;

    const size_t row_stride = (size_t)a.kv_heads * D;
    const f16 *kbase = a.key_cache + (size_t)sl * a.ctx * row_stride + (size_t)kvh * D;
    const f16 *vtbase = a.value_t + ((size_t)sl * a.kv_heads + kvh) * D * (size_t)a.ctx_pad;
    const float qs = a.qscale;

    auto tile_kmax = [&](int qt) { return a.base + min(qt * BM + BM, a.tokens) - 1; };  // last key of a tile

    // Direct global -> LDS staging of step `step` (keys step*128 ..) into
    // buffer `stage`: wave w issues loads w, w + 8, ...; loads 0 .. 2 KL-1 are
    // the K half blocks, the rest the V^T half blocks (a wave-uniform choice).
    // The loads are buffer loads: a descriptor per operand (base = this unit's
    // K slice / V^T rows, bounded by their extent, so any address past them
    // reads 0 instead of faulting), a per-lane byte offset fixed for the
    // kernel (ld_off) and a scalar per-step offset, so a step's loads cost no
    // vector address arithmetic.  On a step that reaches past kmax (the last
    // step of a partial tile), K keys past kmax are clamped to it and a V^T
    // chunk past kmax becomes the chunk holding kmax (its extra keys are
    // masked, and finite: the V^T writers zero the positions up to the next
    // multiple of 8 after a sequence).
    const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16 *>(kbase), (short)0, (int)(((size_t)a.ctx * row_stride - (size_t)kvh * D) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16 *>(vtbase), (short)0, (int)((size_t)D * a.ctx_pad * 2), 0x00020000);
    // Load i of a wave is a K load for i < KH::LOADS / 4 (the first half of
    // the wave's loads), else a V^T load; its half block and 1 KB slot follow
    // from i at compile time plus the wave index.
    static_assert(KH::LOADS == VH::LOADS && KH::LOADS % kWaves == 0, "load split");
    constexpr int NKL = KH::LOADS / 4;  // K loads per wave per step
    const int wave_slot = __builtin_amdgcn_readfirstlane(wave) * 1024;
    auto stage_dst = [&](unsigned char *stage, int i) __attribute__((always_inline)) {
        const int w = i < NKL ? i : i - NKL;          // index among this wave's K (or V^T) loads
        const int hh = (kWaves * w) / KH::LOADS;      // half block
        const int slot = (kWaves * w) % KH::LOADS;    // + wave: 1 KB slot in the half block
        return stage + (i < NKL ? hh * KB : 2 * KB + hh * VB) + 1024 * slot + wave_slot;
    };
    unsigned ld_off[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int w = i < NKL ? i : i - NKL;
        const int hh = (kWaves * w) / KH::LOADS;
        const int j = (kWaves * w) % KH::LOADS + wave;
        if (i < NKL) {
            const int byte = 1024 * j + 16 * lane;
            const int row = byte / KH::ROWB;
            const int q = ((byte % KH::ROWB) >> 4) ^ (row & 15 & (KH::CPR - 1));
            ld_off[i] = (unsigned)(((hh * BN + sigma(row >> 4, row & 15)) * (int)row_stride + 8 * q) * 2);
        } else {
            const int dim = 8 * j + (lane >> 3);
            const int q = (lane & 7) ^ (dim & 7);
            ld_off[i] = (unsigned)((dim * a.ctx_pad + hh * BN + 8 * q) * 2);
        }
    }
    auto stage_load = [&](int step, int kmax, unsigned char *stage) {
        const int key0 = step * 2 * BN;
        if (key0 + 2 * BN - 1 <= kmax) {
            const int k_soff = key0 * (int)row_stride * 2;
            const int v_soff = key0 * 2;
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    i < NKL ? krsrc : vrsrc, (__attribute__((address_space(3))) void *)stage_dst(stage, i), 16,
                    (int)ld_off[i], i < NKL ? k_soff : v_soff, 0, 0);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int w = i < NKL ? i : i - NKL;
            const int hh = (kWaves * w) / KH::LOADS;
            const int j = (kWaves * w) % KH::LOADS + wave;
            int off;
            if (i < NKL) {
                const int byte = 1024 * j + 16 * lane;
                const int row = byte / KH::ROWB;
                const int q = ((byte % KH::ROWB) >> 4) ^ (row & 15 & (KH::CPR - 1));
                const int key = min(key0 + hh * BN + sigma(row >> 4, row & 15), kmax);
                off = (key * (int)row_stride + 8 * q) * 2;
            } else {
                const int dim = 8 * j + (lane >> 3);
                const int q = (lane & 7) ^ (dim & 7);
                const int kc = min(key0 + hh * BN + 8 * q, kmax & ~7);
                off = (dim * a.ctx_pad + kc) * 2;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(i < NKL ? krsrc : vrsrc,
                                                     (__attribute__((address_space(3))) void *)stage_dst(stage, i),
                                                     16, off, 0, 0, 0);
        }
    };
    // The fast-path DMA of the next step, one piece per QK^T batch of the
    // current one: the CU's vector memory path takes ~16 cycles per 1 KB
    // piece, and the 64 pieces of a step issued back to back at its start
    // held every wave until the last was accepted.  A plan that is not
    // `live` (no next step, or one staged by the clamping path) sends every
    // slot to dma_sink with zero offsets, so the instruction stream is the
    // same for every step.
    auto dma_piece = [&](const DmaPlan &d, int i) __attribute__((always_inline)) {
        unsigned char *dst = d.live ? stage_dst(d.stage, i) : dma_sink;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(i < NKL ? krsrc : vrsrc, (__attribute__((address_space(3))) void *)dst,
                                                 16, (int)ld_off[i], i < NKL ? d.ksoff : d.vsoff, 0, 0);
    };
    auto stage_wait = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0): this wave's loads are in LDS

    // Lane-dependent parts of the operand addresses (tiles add immediates).
    int k_off[KK];  // K row c of tile 0, chunk 4kk + g
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        k_off[kk] = c * KH::ROWB + 16 * ((4 * kk + g) ^ (c & (KH::CPR - 1)));
    }
    int v_off[2];   // V^T row c (dim c of tile 0), keys 32 ks + 8 g ..
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        v_off[ks] = c * VH::ROWB + 16 * ((4 * ks + g) ^ (c & 7));
    }

    // Key split `split` of a tile takes its steps [lo, lo + cnt) (of 128 keys);
    // with one split that is every step.  A tile's first step is staged in st0.
    auto tile_steps = [&](int qt) __attribute__((always_inline)) { return (tile_kmax(qt) / BN + 2) / 2; };
    // (split * n < 2^22: at most 32 splits of fewer than 2^24 / 128 steps.)
    auto split_lo = [&](int n) __attribute__((always_inline)) {
        return a.splits == 1 ? 0 : (int)((unsigned)(split * n) / (unsigned)a.splits);
    };
    auto split_cnt = [&](int n) __attribute__((always_inline)) {
        return a.splits == 1 ? n : (int)((unsigned)((split + 1) * n) / (unsigned)a.splits) - split_lo(n);
    };
    // Q^T operand for the wave's two 16-row blocks.  fp16 queries are loaded
    // raw (load_q16) before they are needed: the first tile's with its first
    // K/V step, the second tile's right after the first tile's last step, so
    // that load overlaps the merge; prep_q then zeroes rows past the end (and
    // the fused step loads and rotates its fp32 queries there).
    f16x8 qop[2][KK];
    auto load_q16 = [&](int qt) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int row = qt * BM + 32 * (wave & 3) + 16 * nb + c;
            const f16 *qrow = a.q + (((size_t)sl * a.tokens + (row < a.tokens ? row : 0)) * a.heads + h) * D;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                qop[nb][kk] = *reinterpret_cast<const f16x8 *>(qrow + 8 * g + 32 * kk);
            }
        }
    };
    // Barrier over LDS traffic only: the waves' LDS reads and writes are done
    // and visible, while global loads and stores (the next tile's queries, the
    // output rows) stay in flight.  A workgroup-scope fence would also wait
    // for those (vmcnt), since the counter it must drain for the LDS DMA is
    // the one the global accesses use; no DMA is in flight at these barriers
    // (each step's is waited for before its step barrier).  The memory clobber
    // keeps the compiler's LDS accesses on their side of the barrier.
    auto lds_barrier = []() __attribute__((always_inline)) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // The fused step's queries: waves w and w ^ 4 hold the same 32 rows, so
    // each loads, biases and rotates one 16-row block (half h: block h) and
    // they hand each other their blocks through st1, which is free at a
    // tile's start (the tile's first step is staged in st0): half the fp32
    // query and rotation-table loads, which arrive with nothing to hide them.
    // Two LDS barriers: the blocks are written before they are read, and read
    // before the first step stages into st1.
    auto prep_q = [&](int qt) __attribute__((always_inline)) {
        if constexpr (Q32) {
            const int row = qt * BM + 32 * (wave & 3) + 16 * half + c;
            f16x8 mine[KK];
            if (row < a.tokens) {
                load_q_rope<D>(a, sl, sl % a.layers, h, row, g, mine);
            } else {
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    mine[kk] = f16x8{};  // rows past the end: zero operands (finite scores, never stored)
                }
            }
            f16x8 *xq = reinterpret_cast<f16x8 *>(st1);
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                xq[(wave * KK + kk) * 64 + lane] = mine[kk];
            }
            lds_barrier();
            f16x8 other[KK];
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                other[kk] = xq[((wave ^ 4) * KK + kk) * 64 + lane];
            }
            lds_barrier();
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                qop[0][kk] = half == 0 ? mine[kk] : other[kk];
                qop[1][kk] = half == 0 ? other[kk] : mine[kk];
            }
            return;
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            // rows past the end: zero operands (finite scores, never stored)
            if (qt * BM + 32 * (wave & 3) + 16 * nb + c >= a.tokens) {
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    qop[nb][kk] = f16x8{};
                }
            }
        }
    };

    if (split_cnt(tile_steps(long_tile)) > 0) {
        stage_load(split_lo(tile_steps(long_tile)), tile_kmax(long_tile), st0);
    }
    if constexpr (!Q32) {
        load_q16(long_tile);
    }
    bool first_staged = true;  // the tile's first step is in LDS (waited for) when it starts
    for (int ti = 0; ti < n_tiles_wg; ++ti) {
        const int qt = ti == 0 ? long_tile : pair;
        const int wr0 = qt * BM + 32 * (wave & 3);  // first row of this wave
        const int kmax = tile_kmax(qt);
        const int n_all = tile_steps(qt);            // ceil(blocks / 2)
        const int lo = split_lo(n_all);
        const int cnt = split_cnt(n_all);
        const int n_next = ti + 1 < n_tiles_wg ? tile_steps(pair) : 0;
        const int lo_next = split_lo(n_next);
        const int cnt_next = split_cnt(n_next);
        prep_q(qt);

        float mref[2] = {-INFINITY, -INFINITY};  // exp reference per row, log2 units
        float l[2] = {0.0f, 0.0f};               // per-lane partial row sums
        f32x4 o[2][NT];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                o[nb][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        const int wave_last_row = min(wr0 + 31, a.tokens - 1);
        const bool wave_active = wr0 < a.tokens;
        const int wave_max_pos = a.base + wave_last_row;
        const int wave_min_pos = a.base + wr0;

        // One 64-key block (keys kb0 .. kb0+63) staged at lk (K) / lv (V^T).
        // MASK: a diagonal block (some key beyond some row's position); the
        // interior variant carries no mask code, so nothing splits the QK^T
        // MFMAs from the softmax into separate scheduling regions.
        auto compute = [&](auto mask_tag, int kb0, const unsigned char *lk, const unsigned char *lv,
                           const DmaPlan &dma) __attribute__((always_inline)) {
            constexpr bool MASK = decltype(mask_tag)::value;
            // ---- S^T = K Q^T, tiles 0-1 (keys 0-31) then 2-3 (keys 32-63):
            // batch b = (key half b / KK, k-step b % KK) is two K operand reads
            // (tiles 2hk, 2hk+1) and four MFMAs; the reads run kQkAhead batches
            // ahead of their MFMAs so LDS latency hides under the MFMAs, and
            // the first half's weights are computed while the second half's
            // MFMAs run ----
            constexpr int QB = 2 * KK;
            f32x4 s[4][2];
            f16x8 pb[2][2];     // [key half = PV k-step][row block]: keys 32 hk + 8 g + j
            float psum[2][2];   // [key half][row block]: the lane's sum of those weights
            f16x8 kbuf[QB][2];
            auto kread = [&](int b) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    kbuf[b][i] = *reinterpret_cast<const f16x8 *>(lk + k_off[b % KK] +
                                                                  (2 * (b / KK) + i) * 16 * KH::ROWB);
                }
            };
            // fp16 weights of key half hk, row block nb, against the current
            // reference (0 for every key while a row has none: m_ref = -inf
            // only reaches here from the exact path), and their lane sum
            auto weights = [&](int hk, int nb) __attribute__((always_inline)) {
                const float nm = -mref[nb];
                const bool none = mref[nb] == -INFINITY;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = fast_exp2(fmaf(s[2 * hk + (e >> 2)][nb][e & 3], qs, nm));
                    pb[hk][nb][e] = none ? (f16)0.0f : (f16)x;
                }
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const f16x2 pr = {pb[hk][nb][j], pb[hk][nb][j + 1]};
                    sum = __builtin_amdgcn_fdot2(pr, f16x2{(f16)1.0f, (f16)1.0f}, sum, false);
                }
                psum[hk][nb] = sum;
            };
            // the common case: no reference test, m_ref = -inf gives inf / NaN
            // weights and so a failing sum
            auto weights_fast = [&](int hk, int nb) __attribute__((always_inline)) {
                const float nm = -mref[nb];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    pb[hk][nb][e] = (f16)fast_exp2(fmaf(s[2 * hk + (e >> 2)][nb][e & 3], qs, nm));
                }
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const f16x2 pr = {pb[hk][nb][j], pb[hk][nb][j + 1]};
                    sum = __builtin_amdgcn_fdot2(pr, f16x2{(f16)1.0f, (f16)1.0f}, sum, false);
                }
                psum[hk][nb] = sum;
            };
#pragma unroll
            for (int b = 0; b < kQkAhead; ++b) {
                kread(b);
            }
            static_assert(QB == LOADS, "one DMA piece per QK^T batch");
#pragma unroll
            for (int b = 0; b < QB; ++b) {
                const int hk = b / KK;
                const int kk = b % KK;
                dma_piece(dma, b);
                if (b + kQkAhead < QB) {
                    kread(b + kQkAhead);
                }
                if (kk == 0) {
#pragma unroll
                    for (int i = 2 * hk; i < 2 * hk + 2; ++i) {
                        s[i][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        s[i][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    }
                }
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    s[2 * hk + i][0] = mfma16x16x32(kbuf[b][i], qop[0][kk], s[2 * hk + i][0]);
                    s[2 * hk + i][1] = mfma16x16x32(kbuf[b][i], qop[1][kk], s[2 * hk + i][1]);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // this batch's reads ahead ...
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // ... of its MFMAs
                if (kk != KK - 1) {
                    continue;
                }
                if (MASK) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        // key of s[i][nb][r] is kb0 + 32(i/2) + 8g + 4(i%2) + r; masked past the row's position
                        const int lim = a.base + wr0 + 16 * nb + c - kb0 - 8 * g;
#pragma unroll
                        for (int i = 2 * hk; i < 2 * hk + 2; ++i) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if (32 * (i >> 1) + 4 * (i & 1) + r > lim) {
                                    s[i][nb][r] = -INFINITY;
                                }
                            }
                        }
                    }
                }
                if (hk == 0) {
                    weights_fast(0, 0);
                    weights_fast(0, 1);
                }
            }
            TE_PHASE(1);
            f16x8 vbuf[2 * NT];
            auto vread = [&](int b) __attribute__((always_inline)) {
                vbuf[b] = *reinterpret_cast<const f16x8 *>(lv + v_off[b / NT] + (b % NT) * 16 * VH::ROWB);
            };
#pragma unroll
            for (int b = 0; b < kPvAhead; ++b) {
                vread(b);
            }
#pragma unroll
            for (int hk = 0; hk < 2; ++hk) {
                // ---- the exact path, when a lane's weights of this half sum
                // past 2^kLazyLog2 (or are not finite) ----
                if (__any(!(psum[hk][0] <= kLazyMax) || !(psum[hk][1] <= kLazyMax))) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        float m = -INFINITY;
#pragma unroll
                        for (int i = 2 * hk; i < 2 * hk + 2; ++i) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                m = fmaxf(m, s[i][nb][r]);
                            }
                        }
                        // the half's row maximum in log2 units (-inf: no unmasked key)
                        const float mx = xor_max_16_32(m) * qs;
                        const bool first = mref[nb] == -INFINITY;
                        const bool move = first ? mx > -INFINITY : mx - mref[nb] > kLazyLog2;
                        const float alpha = !move ? 1.0f : first ? 0.0f : fast_exp2(mref[nb] - mx);
                        mref[nb] = move ? mx : mref[nb];
                        l[nb] *= alpha;
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            o[nb][t] = o[nb][t] * alpha;
                        }
                        weights(hk, nb);
                    }
                }
                l[0] += psum[hk][0];
                l[1] += psum[hk][1];
                // ---- O^T += V^T P^T, k-step hk: tile t (dims 16t .. 16t+15):
                // lane (c, g) reads dim 16t + c, keys 32 hk + 8g .. +7; the
                // first kPvAhead reads are issued before the check above and
                // each later one kPvAhead MFMA pairs ahead.  The second half's
                // weights are computed under the first half's MFMAs. ----
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int b = hk * NT + t;
                    if (b + kPvAhead < 2 * NT) {
                        vread(b + kPvAhead);
                    }
                    o[0][t] = mfma16x16x32(vbuf[b], pb[hk][0], o[0][t]);
                    o[1][t] = mfma16x16x32(vbuf[b], pb[hk][1], o[1][t]);
                }
                if (hk == 0) {
                    weights_fast(1, 0);
                    weights_fast(1, 1);
                }
            }
        };

        // Steps alternate st0 / st1 (the loop is unrolled by two so every
        // buffer reference is static); an odd step count gets one empty step,
        // so a tile always ends on st1, whose last step is done before the
        // next tile's first DMA (into st0) is issued.  j counts this split's
        // steps; the step index is lo + j.
        auto body = [&](auto tag, int j) {
            constexpr int B = decltype(tag)::value;
            const unsigned char *cur = B == 0 ? st0 : st1;
            unsigned char *nxt = B == 0 ? st1 : st0;
            // The step staged during this one: the tile's next step, or (on
            // st1's last step) the next tile's first, in flight across the
            // merge.  One that reaches past its tile's last key goes through
            // the clamping path here; a full one is issued piece by piece
            // inside compute (or here, when this wave has nothing to compute).
            int next = -1, next_kmax = 0;
            if (j + 1 < cnt) {
                next = lo + j + 1;
                next_kmax = kmax;
            } else if (B == 1 && cnt_next > 0) {
                next = lo_next;
                next_kmax = tile_kmax(pair);
            }
            const bool next_fast = next >= 0 && next * 2 * BN + 2 * BN - 1 <= next_kmax;
            if (next >= 0 && !next_fast) {
                stage_load(next, next_kmax, nxt);
            }
            DmaPlan dma;
            dma.stage = nxt;
            dma.live = next_fast;
            dma.ksoff = next_fast ? next * 2 * BN * (int)row_stride * 2 : 0;
            dma.vsoff = next_fast ? next * 2 * BN * 2 : 0;
            TE_PHASE(0);
            const int kb0 = (2 * (lo + j) + half) * BN;
            if (j < cnt && wave_active && kb0 <= wave_max_pos) {
                if (kb0 + BN - 1 > wave_min_pos) {
                    compute(std::true_type(), kb0, cur + half * KB, cur + 2 * KB + half * VB, dma);  // diagonal block
                } else {
                    compute(std::false_type(), kb0, cur + half * KB, cur + 2 * KB + half * VB, dma);
                }
            } else if (next_fast) {
                stage_load(next, next_kmax, nxt);
            }
            TE_PHASE(3);
            stage_wait();
            TE_PHASE(5);
            __syncthreads();
            TE_PHASE(6);
#ifdef TE_PREFILL_PHASES
            ph[8] += 1;
#endif
        };
        if (ti == 0 || !first_staged) {
            // The kernel's first step (and a step staged after an empty key
            // range below) is waited for here; every other tile's first step
            // landed during the previous tile's last step, whose wait and
            // barrier cover it, so the output stores of that tile's merge
            // stay in flight.
            stage_wait();
            __syncthreads();
        }
        if (ti == 0) {
            TE_PHASE(9);
        }
        for (int j = 0; j < cnt; j += 2) {
            body(std::integral_constant<int, 0>(), j);
            body(std::integral_constant<int, 1>(), j + 1);
        }
        first_staged = cnt > 0;
        if (!Q32 && ti + 1 < n_tiles_wg) {
            load_q16(pair);  // qop is dead after the last step: the next tile's queries load across the merge
        }

        // ---- merge the two key halves through LDS, normalise, store ----
        // Wave w and wave w^4 hold the same 32 rows.  Each hands the partner
        // one 16-row block (half 0 keeps block 0, half 1 keeps block 1).  The
        // exchange uses st1, free after the last step's barrier.
        // Per wave: the NT float4 of each lane (lane-contiguous, so one
        // ds_write_b128 / ds_read_b128 per tile), then (m, l) per lane.
        float *xf = reinterpret_cast<float *>(st1);
        auto put = [&](const f32x4 (&ob)[NT], float m, float lsum) {
            f32x4 *dst = reinterpret_cast<f32x4 *>(xf + wave * XFER) + lane;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                dst[t * 64] = ob[t];
            }
            reinterpret_cast<float2 *>(xf + wave * XFER + 4 * NT * 64)[lane] = make_float2(m, lsum);
        };
        // The normalised rows leave through LDS: a wave writes its 16 rows
        // row-major into the partner's slot, which only it reads and which it
        // has just read (LDS operations of one wave stay in order), with rows
        // padded to D + 4 floats (the 16 rows' 16-byte pieces of one write
        // land on distinct banks), and stores them back as whole 512-byte
        // rows, two per instruction, where the MFMA layout would give 16
        // pieces of 64 bytes.
        constexpr int OPITCH = D + 4;  // floats per staged output row
        static_assert(16 * OPITCH <= XFER, "staged rows fit the exchange slot");
        // rows = ob * w1 + po * w2 (po: the partner's block, already read)
        auto store_rows = [&](const f32x4 (&ob)[NT], const f32x4 (&po)[NT], float w1, float w2, int nb) {
            float *stg = xf + (wave ^ 4) * XFER;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                // dims 16t + 4g + r of the lane's row
                *reinterpret_cast<f32x4 *>(stg + c * OPITCH + 16 * t + 4 * g) = ob[t] * w1 + po[t] * w2;
            }
            constexpr int LPR = D / 4;          // lanes per row: 16 bytes each
            constexpr int NS = 16 * LPR / 64;   // rows per lane
            // (the lane index is opaque here, so the row addresses are formed
            // here rather than kept live across the step loop)
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int r0 = (int)((unsigned)ln / LPR);
            const int q = (int)((unsigned)ln % LPR);
            // every staged piece is read before the first store, so the stores
            // wait for the LDS once
            f32x4 v[NS];
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                v[i] = *reinterpret_cast<const f32x4 *>(stg + (i * (64 / LPR) + r0) * OPITCH + 4 * q);
            }
            // rows row0 + r, r = i * (64 / LPR) + r0, of this (seq*layer, head):
            // a 32-bit float offset from the block's first row (16 rows of
            // heads * D floats)
            const int row0 = wr0 + 16 * nb;
            if constexpr (Q32) {
                if (a.dhi != nullptr) {  // the fused step's rows as digits (uniform)
#pragma unroll
                    for (int i = 0; i < NS; ++i) {
                        const int r = i * (64 / LPR) + r0;
                        store_digits4(v[i], (size_t)sl * a.tokens + row0 + r, a.heads * D, h * D + 4 * q, a.dhi,
                                      a.dlo, a.dscales, row0 + r < a.tokens);
                    }
                    return;
                }
            }
            float *orow = a.out + (((size_t)sl * a.tokens + row0) * a.heads + h) * D;
            const unsigned rstride = (unsigned)a.heads * D;
            // non-temporal: the output is not read back by this launch
            if (row0 + 15 < a.tokens) {
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const unsigned off = (unsigned)(i * (64 / LPR) + r0) * rstride + 4u * (unsigned)q;
                    __builtin_nontemporal_store(v[i], reinterpret_cast<f32x4 *>(orow + off));
                }
            } else {
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const int r = i * (64 / LPR) + r0;
                    if (row0 + r < a.tokens) {
                        const unsigned off = (unsigned)r * rstride + 4u * (unsigned)q;
                        __builtin_nontemporal_store(v[i], reinterpret_cast<f32x4 *>(orow + off));
                    }
                }
            }
        };
        auto finish = [&](const f32x4 (&ob)[NT], float m, float lsum, int nb) {
            const f32x4 *src = reinterpret_cast<const f32x4 *>(xf + (wave ^ 4) * XFER) + lane;
            const float2 ml2 = reinterpret_cast<const float2 *>(xf + (wave ^ 4) * XFER + 4 * NT * 64)[lane];
            f32x4 po[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                po[t] = src[t * 64];
            }
            const float m2 = ml2.x;
            const float l2 = ml2.y;
            const float mn = fmaxf(m, m2);
            const float s1 = m == mn ? 1.0f : fast_exp2(m - mn);
            const float s2 = m2 == mn ? 1.0f : fast_exp2(m2 - mn);
            const float ltot = xor_sum_16_32(lsum * s1 + l2 * s2);
            const int row = wr0 + 16 * nb + c;
            if (row < a.tokens && a.part_o != nullptr) {
                // key split: O relative to the row maximum mn, unnormalised, with (mn, l)
                const size_t pi = ((size_t)zz * a.tokens + row) * a.heads + h;
                float *prow = a.part_o + pi * D;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    float4 v;
                    v.x = ob[t][0] * s1 + po[t][0] * s2;
                    v.y = ob[t][1] * s1 + po[t][1] * s2;
                    v.z = ob[t][2] * s1 + po[t][2] * s2;
                    v.w = ob[t][3] * s1 + po[t][3] * s2;
                    *reinterpret_cast<float4 *>(prow + 16 * t + 4 * g) = v;
                }
                if (g == 0) {
                    *reinterpret_cast<float2 *>(a.part_ml + 2 * pi) = make_float2(mn, ltot);
                }
            } else if (a.part_o == nullptr) {
                // (v_rcp_f32: within 1 ulp; ltot >= 2^-kLazyLog2 when a key was seen)
                const float inv = ltot > 0.0f ? __builtin_amdgcn_rcpf(ltot) : 0.0f;
                const float w1 = s1 * inv;
                const float w2 = s2 * inv;
                store_rows(ob, po, w1, w2, nb);
            }
        };
        if (half == 0) {
            put(o[1], mref[1], l[1]);
        } else {
            put(o[0], mref[0], l[0]);
        }
        lds_barrier();
        TE_PHASE(2);
        if (half == 0) {
            finish(o[0], mref[0], l[0], 0);
        } else {
            finish(o[1], mref[1], l[1], 1);
        }
        TE_PHASE(4);
        lds_barrier();  // exchange and staged rows are read before st1 is staged again
        TE_PHASE(7);
        if (cnt == 0 && cnt_next > 0) {
            // Nothing of this tile was staged (an empty key range of the
            // split), so st0 is free; staged after the merge, so no LDS DMA
            // is in flight across the merge barriers.
            stage_load(lo_next, tile_kmax(pair), st0);
        }
    }
#ifdef TE_PREFILL_PHASES
    if (a.phase_log != nullptr && lane == 0) {
        const unsigned wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        for (int i = 0; i < kPhases; ++i) {
            a.phase_log[(wg * kWaves + wave) * kPhases + i] = ph[i];
        }
    }
#endif
}

// Short launches: the rows kernel.  One workgroup per RM (32) query rows of
// one head; its 8 waves take the row group's 64-key blocks round-robin (wave
// w: blocks w, w + 8, ...), each over all 32 rows, so a row group of at most
// 8 blocks is one block per wave: no step loop, no per-step barrier, no K /
// V^T staging.  The group's queries go to LDS once; the K and V^T operands
// load from global memory straight into registers in the MFMA layouts of the
// tile kernel (K rows in the sigma key order, V^T rows of 8 consecutive
// keys), and only waves that have a block load anything.  The softmax is the
// tile kernel's (fp32, base 2, lazy reference, fp16 P), with each block's row
// maximum taken exactly.  At the end the waves' states merge
// once through LDS: every wave writes its rows scaled by 2^(m_w - M) / L
// (M, L: the row's maximum and weight sum over the waves), and wave w sums
// rows 4w .. 4w + 3 over the waves and stores them as whole rows.
constexpr int RM = 32;

template <int D>
__global__ __launch_bounds__(kThreads, 1) void prefill_rows_f16_kernel(PrefillArgs a) {
    constexpr int KK = D / 32;     // QK^T K-steps
    constexpr int NT = D / 16;     // O^T output tiles
    constexpr int OPITCH = D + 4;  // floats per staged row (16 rows of one write on distinct banks)
    __shared__ __attribute__((aligned(16))) float part[kWaves][RM * OPITCH];
    __shared__ float2 mls[kWaves][RM];
    __shared__ __attribute__((aligned(16))) f16 qlds[RM][D + 8];  // rows padded: conflict-free operand reads

    // Units: row group fastest, then head, then seq*layer; remapped so that
    // XCD x runs units [x W/8, (x+1) W/8) (the heads of one KV group share
    // an L2), as in the tile kernel.
    int unit = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
    const int n_units = (int)(gridDim.x * gridDim.y * gridDim.z);
    if (n_units % kXcds == 0) {
        unit = (unit % kXcds) * (n_units / kXcds) + unit / kXcds;
    }
    const int rg = (int)((unsigned)unit % gridDim.x);
    const unsigned hg = (unsigned)unit / gridDim.x;
    const int h = (int)(hg % (unsigned)a.heads);
    const int sl = (int)(hg / (unsigned)a.heads);
    const int kvh = h / a.group;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int r0 = rg * RM;
    const int kmax = a.base + min(r0 + RM, a.tokens) - 1;  // the row group's last key
    const int nblk = kmax / BN + 1;
    const float qs = a.qscale;
    const size_t row_stride = (size_t)a.kv_heads * D;
    const f16 *kbase = a.key_cache + (size_t)sl * a.ctx * row_stride + (size_t)kvh * D;
    const f16 *vtbase = a.value_t + ((size_t)sl * a.kv_heads + kvh) * D * (size_t)a.ctx_pad;
#ifdef TE_PREFILL_PHASES
    // wall-clock marks (s_memrealtime, 100 MHz): start, first block's weights,
    // block loop done, (m, l) exchanged, rows staged, rows stored; shader cycles
    unsigned tr[kPhases] = {};
    tr[0] = (unsigned)__builtin_amdgcn_s_memrealtime();
    const unsigned cyc0 = (unsigned)__builtin_amdgcn_s_memtime();
#endif

    // The group's fp16 queries, loaded once into LDS by the whole workgroup
    // (the loads into one CU bound this kernel): thread t takes row t / (D/8),
    // dims 8 (t % (D/8)) ..; rows past the end are zero (finite scores, never
    // stored).  The fused step adds the bias and rotates here, with the
    // operation order of rope_kv_append_kernel (FP contraction off), so the
    // bits equal the fp16 queries the unfused path stores.
    {
#pragma clang fp contract(off)
        constexpr int CPR = D / 8;     // 16-byte chunks per row
        constexpr int HCH = CPR / 2;   // chunks per rotation half
        const int t = threadIdx.x;
        if (t < RM * CPR) {
            const int rr = t / CPR;
            const int ch = t % CPR;
            const int row = r0 + rr;
            f16x8 v = f16x8{};
            if (row < a.tokens && a.q32 == nullptr) {
                v = *reinterpret_cast<const f16x8 *>(a.q + (((size_t)sl * a.tokens + row) * a.heads + h) * D + 8 * ch);
            } else if (row < a.tokens) {
                // own chunk and its rotation partner (dims +-D/2), bias first
                const float *qrow = a.q32 + (((size_t)sl * a.tokens + row) * a.heads + h) * D;
                const int pc = ch ^ HCH;
                float x[8], y[8];
                *reinterpret_cast<float4 *>(x) = *reinterpret_cast<const float4 *>(qrow + 8 * ch);
                *reinterpret_cast<float4 *>(x + 4) = *reinterpret_cast<const float4 *>(qrow + 8 * ch + 4);
                *reinterpret_cast<float4 *>(y) = *reinterpret_cast<const float4 *>(qrow + 8 * pc);
                *reinterpret_cast<float4 *>(y + 4) = *reinterpret_cast<const float4 *>(qrow + 8 * pc + 4);
                if (a.q_bias != nullptr) {
                    const float *qb = a.q_bias + ((size_t)(sl % a.layers) * a.heads + h) * D;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        x[j] = x[j] + qb[8 * ch + j];
                        y[j] = y[j] + qb[8 * pc + j];
                    }
                }
                const int pos = a.base + row;
                const float *cr = a.rope_cos + (size_t)pos * (D / 2) + 8 * (ch % HCH);
                const float *sr = a.rope_sin + (size_t)pos * (D / 2) + 8 * (ch % HCH);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // first half: x0 c - x1 s; second half: x1 c + x0 s (x0 = dim d, x1 = dim d + D/2)
                    v[j] = ch < HCH ? (f16)(x[j] * cr[j] - y[j] * sr[j]) : (f16)(x[j] * cr[j] + y[j] * sr[j]);
                }
            }
            *reinterpret_cast<f16x8 *>(&qlds[rr][8 * ch]) = v;
        }
    }
    __syncthreads();
    // Q^T operand: lane (c, g) holds row 16 nb + c of the group, dims 32 kk + 8 g ..
    f16x8 qop[2][KK];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            qop[nb][kk] = *reinterpret_cast<const f16x8 *>(&qlds[16 * nb + c][32 * kk + 8 * g]);
        }
    }

    float mref[2] = {-INFINITY, -INFINITY};  // exp reference per row, log2 units
    float l[2] = {0.0f, 0.0f};               // per-lane partial row sums
    f32x4 o[2][NT];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            o[nb][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    for (int j = wave; j < nblk; j += kWaves) {
        const int kb0 = j * BN;
        // a block reaching past kmax clamps its K keys to kmax and its V^T
        // chunks to the chunk holding kmax (those keys are masked; the V^T
        // writers keep that chunk's positions finite)
        const bool tail = kb0 + BN - 1 > kmax;
        // ---- S^T = K Q^T: tile i holds keys kb0 + sigma(i, m) ----
        f16x8 kop[4][KK];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = tail ? min(kb0 + sigma(i, c), kmax) : kb0 + sigma(i, c);
            const f16 *kr = kbase + (size_t)key * row_stride + 8 * g;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                kop[i][kk] = *reinterpret_cast<const f16x8 *>(kr + 32 * kk);
            }
        }
        f32x4 s[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                s[i][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    s[i][nb] = mfma16x16x32(kop[i][kk], qop[nb][kk], s[i][nb]);
                }
            }
        }
        // ---- V^T operand: tile t, k-step ks: dim 16 t + c, keys kb0 + 32 ks + 8 g .. ----
        f16x8 vop[2][NT];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int kc = tail ? min(kb0 + 32 * ks + 8 * g, kmax & ~7) : kb0 + 32 * ks + 8 * g;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                vop[ks][t] = *reinterpret_cast<const f16x8 *>(vtbase + (size_t)(16 * t + c) * a.ctx_pad + kc);
            }
        }
        // causal mask: the key of s[i][nb][r] is kb0 + 32(i/2) + 8g + 4(i%2) + r
        if (kb0 + BN - 1 > a.base + r0) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int lim = a.base + r0 + 16 * nb + c - kb0 - 8 * g;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (32 * (i >> 1) + 4 * (i & 1) + r > lim) {
                            s[i][nb][r] = -INFINITY;
                        }
                    }
                }
            }
        }
        // ---- softmax: the block's row maxima, the lazy reference, fp16 weights ----
        f16x8 pb[2][2];  // [PV k-step][row block]: keys 32 ks + 8 g + e
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    m = fmaxf(m, s[i][nb][r]);
                }
            }
            const float mx = xor_max_16_32(m) * qs;  // -inf: no unmasked key in the block
            const bool first = mref[nb] == -INFINITY;
            const bool move = first ? mx > -INFINITY : mx - mref[nb] > kLazyLog2;
            if (__any(move && !first)) {
                const float alpha = move && !first ? fast_exp2(mref[nb] - mx) : 1.0f;
                l[nb] *= alpha;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    o[nb][t] = o[nb][t] * alpha;
                }
            }
            mref[nb] = move ? mx : mref[nb];
            const float nm = -mref[nb];
            const bool none = mref[nb] == -INFINITY;
            float sum = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = fast_exp2(fmaf(s[2 * ks + (e >> 2)][nb][e & 3], qs, nm));
                    pb[ks][nb][e] = none ? (f16)0.0f : (f16)x;
                }
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const f16x2 pr = {pb[ks][nb][e], pb[ks][nb][e + 1]};
                    sum = __builtin_amdgcn_fdot2(pr, f16x2{(f16)1.0f, (f16)1.0f}, sum, false);
                }
            }
            l[nb] += sum;
        }
#ifdef TE_PREFILL_PHASES
        if (j == wave) {
            tr[1] = (unsigned)__builtin_amdgcn_s_memrealtime();
        }
#endif
        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                o[0][t] = mfma16x16x32(vop[ks][t], pb[ks][0], o[0][t]);
                o[1][t] = mfma16x16x32(vop[ks][t], pb[ks][1], o[1][t]);
            }
        }
    }

#ifdef TE_PREFILL_PHASES
    tr[2] = (unsigned)__builtin_amdgcn_s_memrealtime();
#endif
    // ---- merge the waves' states: (m, l) per row, then the scaled rows ----
    const int nact = min(nblk, kWaves);  // waves that took a block
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        l[nb] = xor_sum_16_32(l[nb]);
        if (g == 0 && wave < nact) {
            mls[wave][16 * nb + c] = make_float2(mref[nb], l[nb]);
        }
    }
    __syncthreads();
#ifdef TE_PREFILL_PHASES
    tr[3] = (unsigned)__builtin_amdgcn_s_memrealtime();
#endif
    if (wave < nact) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            float mm = -INFINITY;
            for (int p = 0; p < nact; ++p) {
                mm = fmaxf(mm, mls[p][16 * nb + c].x);
            }
            float lt = 0.0f;
            for (int p = 0; p < nact; ++p) {
                const float2 ml = mls[p][16 * nb + c];
                lt += ml.x == -INFINITY ? 0.0f : fast_exp2(ml.x - mm) * ml.y;
            }
            // (v_rcp_f32: within 1 ulp; lt >= 1 for a row that saw a key)
            const float w = mref[nb] == -INFINITY || !(lt > 0.0f) ? 0.0f
                                                                  : fast_exp2(mref[nb] - mm) * __builtin_amdgcn_rcpf(lt);
            float *dst = &part[wave][(16 * nb + c) * OPITCH + 4 * g];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                *reinterpret_cast<f32x4 *>(dst + 16 * t) = o[nb][t] * w;
            }
        }
    }
    __syncthreads();
#ifdef TE_PREFILL_PHASES
    tr[4] = (unsigned)__builtin_amdgcn_s_memrealtime();
#endif
    // wave w: rows 4w .. 4w + 3 of the group, LPR lanes of 16 bytes per row
    constexpr int LPR = D / 4;
    constexpr int RPP = 64 / LPR;  // rows per pass
    const int q = lane % LPR;
#pragma unroll
    for (int i = 0; i < 4 / RPP; ++i) {
        const int r = 4 * wave + i * RPP + lane / LPR;
        f32x4 acc = *reinterpret_cast<const f32x4 *>(&part[0][r * OPITCH + 4 * q]);
        for (int p = 1; p < nact; ++p) {
            acc += *reinterpret_cast<const f32x4 *>(&part[p][r * OPITCH + 4 * q]);
        }
        if (a.dhi != nullptr) {  // uniform
            store_digits4(acc, (size_t)sl * a.tokens + r0 + r, a.heads * D, h * D + 4 * q, a.dhi, a.dlo, a.dscales,
                          r0 + r < a.tokens);
        } else if (r0 + r < a.tokens) {
            float *orow = a.out + (((size_t)sl * a.tokens + r0 + r) * a.heads + h) * D;
            __builtin_nontemporal_store(acc, reinterpret_cast<f32x4 *>(orow + 4 * q));
        }
    }
#ifdef TE_PREFILL_PHASES
    __builtin_amdgcn_s_waitcnt(0);
    tr[5] = (unsigned)__builtin_amdgcn_s_memrealtime();
    tr[6] = (unsigned)__builtin_amdgcn_s_memtime() - cyc0;
    if (a.phase_log != nullptr && lane == 0) {
        const unsigned wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        for (int i = 0; i < kPhases; ++i) {
            a.phase_log[(wg * kWaves + wave) * kPhases + i] = tr[i];
        }
    }
#endif
}

// Key-split merge: out[row][h] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s
// over the splits of one (seq*layer); M = max_s m_s.  A split that saw no
// unmasked key of the row has m_s = -inf and weight 0 (split 0 always holds
// key 0).  Thread (item, col) handles 4 dims of one (row, head).
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float *part_o, const float *part_ml, int splits,
                                                           int items, float *out) {
    constexpr int COLS = D / 4;
    constexpr int ITEMS = 256 / COLS;
    const int item = blockIdx.x * ITEMS + (int)threadIdx.x / COLS;
    const int col = threadIdx.x % COLS;
    if (item >= items) {
        return;
    }
    const size_t sl = blockIdx.y;
    float m = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) {
        m = fmaxf(m, part_ml[2 * ((sl * splits + sp) * items + item)]);
    }
    float den = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int sp = 0; sp < splits; ++sp) {
        const size_t pi = (sl * splits + sp) * items + item;
        const float2 ml = *reinterpret_cast<const float2 *>(part_ml + 2 * pi);
        const float w = ml.x == -INFINITY ? 0.0f : fast_exp2(ml.x - m);
        const float4 o = reinterpret_cast<const float4 *>(part_o + pi * D)[col];
        den += w * ml.y;
        acc.x += w * o.x;
        acc.y += w * o.y;
        acc.z += w * o.z;
        acc.w += w * o.w;
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    reinterpret_cast<float4 *>(out + (sl * items + item) * D)[col] =
        make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// V^T of positions [first, end) of every (seq*layer, kv head):
//   vt[((sl*kv + h)*D + i)*ctx_pad + p] = v[((sl*ctx + p)*kv + h)*D + i],
// and zeros at [end, end8) (end8 = end rounded up to 8, at most ctx_pad), so
// the 8-key chunks the attention kernel reads past a sequence's end are
// finite.  One workgroup per 32 aligned positions, kv head and seq*layer:
// the rows come in as whole 16-byte chunks into LDS, the dim rows go out as
// 16-byte chunks of 8 positions (single halves at the range's edges).
template <int D>
__global__ __launch_bounds__(256) void value_transpose_kernel(const f16 *v, f16 *vt, int first, int end, int end8,
                                                              int ctx, int ctx_pad, int kv_heads) {
    constexpr int P = 32;
    constexpr int CPR = D / 8;
    __shared__ __attribute__((aligned(16))) f16 tile[P][D + 8];
    const int p0 = (first & ~(P - 1)) + P * (int)blockIdx.x;
    const int h = blockIdx.y;
    const size_t sl = blockIdx.z;
    const f16 *src = v + sl * (size_t)ctx * kv_heads * D + (size_t)h * D;
    for (int idx = threadIdx.x; idx < P * CPR; idx += 256) {
        const int r = idx / CPR;
        const int cq = idx % CPR;
        const int p = p0 + r;
        f16x8 val = {0, 0, 0, 0, 0, 0, 0, 0};
        if (p >= first && p < end) {
            val = *reinterpret_cast<const f16x8 *>(src + (size_t)p * kv_heads * D + 8 * cq);
        }
        *reinterpret_cast<f16x8 *>(&tile[r][8 * cq]) = val;
    }
    __syncthreads();
    f16 *dst = vt + (sl * kv_heads + h) * (size_t)D * ctx_pad;
    for (int idx = threadIdx.x; idx < D * (P / 8); idx += 256) {
        const int i = idx / (P / 8);
        const int pc = idx % (P / 8);
        const int pa = p0 + 8 * pc;
        if (pa >= end8 || pa + 8 <= first) {
            continue;
        }
        f16x8 val;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            val[j] = tile[8 * pc + j][i];
        }
        f16 *row = dst + (size_t)i * ctx_pad + pa;
        if (pa >= first && pa + 8 <= end8) {
            *reinterpret_cast<f16x8 *>(row) = val;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (pa + j >= first && pa + j < end8) {
                    row[j] = val[j];
                }
            }
        }
    }
}

}  // namespace

namespace {

size_t vt_pitch(size_t context_tokens) { return (context_tokens + kVtAlign - 1) / kVtAlign * kVtAlign; }

size_t vt_bytes(size_t seqs, size_t layers, size_t context_tokens, size_t kv_heads, size_t head_dim) {
    return seqs * layers * kv_heads * head_dim * vt_pitch(context_tokens) * sizeof(uint16_t);
}

// 16-byte alignment (null passes): the attention kernel's operand loads and
// output stores and the V^T kernels' 16-byte chunks assume it of every base
// pointer; the entry points return UNSUPPORTED for a base that lacks it.
bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

te_status launch_value_transpose(const f16 *v, f16 *vt, size_t sl_count, size_t first, size_t count,
                                 size_t context_tokens, size_t kv_heads, size_t head_dim, hipStream_t stream) {
    const size_t pad = vt_pitch(context_tokens);
    const size_t end = first + count;
    const size_t end8 = std::min((end + 7) / 8 * 8, pad);
    if (end8 <= first) {
        return TE_STATUS_OK;
    }
    const size_t tiles = (end8 - (first & ~(size_t)31) + 31) / 32;
    const dim3 grid((unsigned)tiles, (unsigned)kv_heads, (unsigned)sl_count);
    if (head_dim == 128) {
        value_transpose_kernel<128><<<grid, 256, 0, stream>>>(v, vt, (int)first, (int)end, (int)end8,
                                                             (int)context_tokens, (int)pad, (int)kv_heads);
    } else {
        value_transpose_kernel<64><<<grid, 256, 0, stream>>>(v, vt, (int)first, (int)end, (int)end8,
                                                            (int)context_tokens, (int)pad, (int)kv_heads);
    }
    return te_hip::launch_status();
}

// Tile pairs (n-1-i, i) give every workgroup the same causal work, which
// balances launches of several rounds; a launch whose single tiles fit one
// round (one workgroup per CU) takes them unpaired instead: its time is the
// longest tile's, not a pair's (3B at L = 2048: 256 single tiles; a 2K chunk
// after a long prefix, whose tiles all have nearly the same length).
bool prefill_paired(size_t seqs, size_t layers, size_t tokens, size_t heads, int splits) {
    const size_t n_qtiles = (tokens + BM - 1) / BM;
    return n_qtiles * heads * seqs * layers * (size_t)splits > (size_t)te_hip::device_compute_units();
}

// The rows kernel (one 32-row group per workgroup, its keys split over the
// 8 waves) for a launch with one split over at most kRowsMaxKeys keys.  Its
// last row group reads every key's K and V^T through one CU, in the MFMA
// operand order (16 rows x 64 bytes per load instruction), with no compute
// to hide it.  Measured on MI355X (3B shapes, graph-replayed) against the
// tile kernel: L = 128 6.00 against 8.55 us, 256 8.53 against 9.99, 384
// 11.24 against 11.73, 512 12.92 against 13.17, 1,024 about twice as long.
// At 512 keys its 256 workgroups of 146 KB LDS need every CU at once (one
// measured launch started a workgroup 6.6 us late, in a second round), so
// for fp16 queries the choice stops at 256.  With fp32 queries (the fused
// step: bias and RoPE on load) the tile kernel's query preparation costs
// more than the rows kernel's (which loads a group's queries once, into
// LDS), so the fused step takes the rows kernel up to kRowsMaxKeysQ32:
// its attention at 3B L = 512 15.3 against 23.5 us, the 3B Q4_0 512-token
// prompt 12.81 -> 12.43-12.67 ms.  TE_HIP_PREFILL_ROWS=1 takes it for every
// launch with one split, =0 never.
constexpr size_t kRowsMaxKeys = 256;
constexpr size_t kRowsMaxKeysQ32 = 512;

bool prefill_rows(size_t tokens, size_t base_position, int splits, bool q32) {
    if (splits != 1) {
        return false;
    }
    const char *env = getenv("TE_HIP_PREFILL_ROWS");
    if (env != nullptr && (env[0] == '0' || env[0] == '1') && env[1] == '\0') {
        return env[0] == '1';
    }
    return base_position + tokens <= (q32 ? kRowsMaxKeysQ32 : kRowsMaxKeys);
}

#ifdef TE_PREFILL_PHASES
unsigned *g_phase_log = nullptr;
#endif

te_status launch_prefill(PrefillArgs a, size_t seqs, size_t layers, size_t tokens, size_t base_position,
                         size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim, hipStream_t strm) {
    a.layers = (int)layers;
    a.tokens = (int)tokens;
    a.base = (int)base_position;
    a.ctx = (int)context_tokens;
    a.ctx_pad = (int)vt_pitch(context_tokens);
    a.heads = (int)heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)(heads / kv_heads);
    a.n_qtiles = (int)((tokens + BM - 1) / BM);
    a.qscale = TE_LOG2E / sqrtf((float)head_dim);
    if (a.splits < 1) {
        a.splits = 1;
    }
#ifdef TE_PREFILL_PHASES
    a.phase_log = g_phase_log;
#endif
    if (prefill_rows(tokens, base_position, a.splits, a.q32 != nullptr)) {
        const dim3 grid((unsigned)((tokens + RM - 1) / RM), (unsigned)heads, (unsigned)(seqs * layers));
        if (head_dim == 128) {
            prefill_rows_f16_kernel<128><<<grid, kThreads, 0, strm>>>(a);
        } else {
            prefill_rows_f16_kernel<64><<<grid, kThreads, 0, strm>>>(a);
        }
        return te_hip::launch_status();
    }
    a.paired = prefill_paired(seqs, layers, tokens, heads, a.splits) ? 1 : 0;
#ifdef TE_PREFILL_PHASES
    a.phase_log = g_phase_log;
#endif
    const int n_units_x = a.paired ? (a.n_qtiles + 1) / 2 : a.n_qtiles;
    const dim3 grid((unsigned)n_units_x, (unsigned)heads, (unsigned)(seqs * layers * a.splits));
    if (head_dim == 128) {
        if (a.q32 != nullptr) {
            prefill_causal_f16_kernel<128, true><<<grid, kThreads, 0, strm>>>(a);
        } else {
            prefill_causal_f16_kernel<128, false><<<grid, kThreads, 0, strm>>>(a);
        }
    } else if (a.q32 != nullptr) {
        prefill_causal_f16_kernel<64, true><<<grid, kThreads, 0, strm>>>(a);
    } else {
        prefill_causal_f16_kernel<64, false><<<grid, kThreads, 0, strm>>>(a);
    }
    return te_hip::launch_status();
}

// Key splits for a launch whose tile pairs alone leave CUs idle.  One
// workgroup fills a CU (its LDS), every pair carries the same causal work
// (~ the steps of tiles n-1-i and i), and a launch of W workgroups runs in
// ceil(W / CUs) rounds, so S splits take ceil(S*W0 / CUs) * ceil(steps / S)
// step times (a step, 128 keys for 256 rows, is ~2.5 us).  The merge costs a
// launch (~2 steps) plus writing and reading every split's partial rows,
// priced at 8 TB/s (fitted on MI355X over 3B L = 512..4096 and 1.5B 2K chunks
// at bases 0..131072: it picks the fastest measured S or one within 4 %).
// The smallest S with the least time wins; S = 1 whenever the pairs fill the
// device.  TE_HIP_PREFILL_SPLITS (1..32) overrides the choice.
int prefill_splits(size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t heads,
                   size_t head_dim) {
    const size_t n_qtiles = (tokens + BM - 1) / BM;
    const size_t cus = (size_t)te_hip::device_compute_units();
    auto tile_steps = [&](size_t qt) {
        const size_t kmax = base_position + std::min(qt * BM + BM, tokens) - 1;
        return (kmax / BN + 2) / 2;
    };
    const char *env = getenv("TE_HIP_PREFILL_SPLITS");
    if (env != nullptr) {
        const long v = strtol(env, nullptr, 10);
        if (v >= 1 && v <= kMaxPrefillSplits && (size_t)v * seqs * layers <= 65535) {
            return (int)v;
        }
    }
    // A unit's time in step times: its steps split S ways, plus ~2.5 steps of
    // prologue and merge per tile it holds; units run in ceil(S*W / CUs) rounds.
    auto launch_steps = [&](int sp) {
        const bool paired = prefill_paired(seqs, layers, tokens, heads, sp);
        const size_t units = (paired ? (n_qtiles + 1) / 2 : n_qtiles) * heads * seqs * layers;
        const size_t tiles = paired && n_qtiles > 1 ? 2 : 1;
        const size_t steps = tile_steps(n_qtiles - 1) + (tiles > 1 ? tile_steps(0) : 0);
        return (double)((sp * units + cus - 1) / cus) * ((double)((steps + sp - 1) / sp) + 2.5 * (double)tiles);
    };
    // partial bytes of one split, written then read, in step times
    const double split_steps = (double)(seqs * layers * tokens * heads * (head_dim + 2) * sizeof(float)) * 2.0 /
                               (8.0e12 * 2.5e-6);
    const size_t max_steps = tile_steps(n_qtiles - 1) + (n_qtiles > 1 ? tile_steps(0) : 0);
    int best = 1;
    double best_t = launch_steps(1);
    for (int sp = 2; sp <= kMaxPrefillSplits && (size_t)sp <= max_steps; ++sp) {
        const double t = launch_steps(sp) + 2.0 + split_steps * (double)sp;
        if (t < best_t && (size_t)sp * seqs * layers <= 65535) {
            best_t = t;
            best = sp;
        }
    }
    return best;
}

size_t prefill_workspace(int splits, size_t seqs, size_t layers, size_t tokens, size_t heads, size_t head_dim) {
    return splits <= 1 ? 0 : (size_t)splits * seqs * layers * tokens * heads * (head_dim + 2) * sizeof(float);
}

te_status check_prefill_args(size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
                             size_t heads, size_t kv_heads, size_t head_dim) {
    if (seqs == 0 || layers == 0 || tokens == 0 || context_tokens == 0 || heads == 0 || kv_heads == 0 ||
        head_dim == 0 || (heads % kv_heads) != 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    // Cache offsets of one (seq, layer) are 32-bit buffer offsets in the kernel.
    if ((head_dim != 64 && head_dim != 128) || context_tokens * kv_heads * head_dim * 2 >= ((size_t)1 << 31) ||
        heads > 65535 || seqs * layers > 65535) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (base_position > context_tokens || tokens > context_tokens - base_position) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return TE_STATUS_OK;
}

// The attention over V^T with `splits` key splits (workspace = the partials),
// then the merge launch when splits > 1.  With act_out (the fused step, one
// split only): the output rows as digits, formed in the attention kernel.
te_status run_prefill(PrefillArgs a, int splits, void *partials, size_t seqs, size_t layers, size_t tokens,
                      size_t base_position, size_t context_tokens, size_t heads, size_t kv_heads, size_t head_dim,
                      float *out, hipStream_t strm, void *act_out = nullptr) {
    a.out = out;
    a.splits = splits;
    if (splits > 1) {
        const size_t parts = (size_t)splits * seqs * layers * tokens * heads;
        a.part_o = static_cast<float *>(partials);
        a.part_ml = a.part_o + parts * head_dim;
    } else if (act_out != nullptr) {
        const size_t planes = te_hip::act_plane_bytes(seqs * layers * tokens, heads * head_dim);
        a.dhi = static_cast<int8_t *>(act_out);
        a.dlo = a.dhi + planes;
        a.dscales = reinterpret_cast<float *>(a.dlo + planes);
    }
    te_status st = launch_prefill(a, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim,
                                  strm);
    if (st != TE_STATUS_OK || splits == 1) {
        return st;
    }
    const int items = (int)(tokens * heads);
    const int per_block = 256 / (int)(head_dim / 4);
    const dim3 grid((unsigned)((items + per_block - 1) / per_block), (unsigned)(seqs * layers));
    if (head_dim == 128) {
        prefill_merge_kernel<128><<<grid, 256, 0, strm>>>(a.part_o, a.part_ml, splits, items, out);
    } else {
        prefill_merge_kernel<64><<<grid, 256, 0, strm>>>(a.part_o, a.part_ml, splits, items, out);
    }
    return te_hip::launch_status();
}

// The split count a call with this workspace runs with: the cost model's
// choice when the workspace holds its partials, else one split.
int splits_for(void *workspace, size_t workspace_bytes, size_t seqs, size_t layers, size_t tokens,
               size_t base_position, size_t heads, size_t head_dim, te_status *st) {
    *st = TE_STATUS_OK;
    if (workspace == nullptr) {
        return 1;
    }
    const int splits = prefill_splits(seqs, layers, tokens, base_position, heads, head_dim);
    if (workspace_bytes < prefill_workspace(splits, seqs, layers, tokens, heads, head_dim)) {
        *st = TE_STATUS_INVALID_ARGUMENT;
    }
    return splits;
}

}  // namespace

#ifdef TE_PREFILL_PHASES
// Phase log of the next prefill launches ([workgroup][wave][10] unsigned, see
// kPhases); a build with -DTE_PREFILL_PHASES only.
extern "C" void te_hip_prefill_phase_log_set(unsigned *device_log) { g_phase_log = device_log; }
#endif

extern "C" size_t te_hip_value_t_bytes(size_t seqs, size_t layers, size_t context_tokens, size_t kv_heads,
                                       size_t head_dim) {
    if (seqs == 0 || layers == 0 || context_tokens == 0 || kv_heads == 0 || head_dim == 0) {
        return 0;
    }
    return vt_bytes(seqs, layers, context_tokens, kv_heads, head_dim);
}

extern "C" te_status te_hip_value_transpose_f16(const uint16_t *value_cache, uint16_t *value_cache_t, size_t seqs,
                                                size_t layers, size_t first_position, size_t count,
                                                size_t context_tokens, size_t kv_heads, size_t head_dim,
                                                void *stream) {
    if (value_cache == nullptr || value_cache_t == nullptr || seqs == 0 || layers == 0 || context_tokens == 0 ||
        kv_heads == 0 || head_dim == 0 || first_position > context_tokens ||
        count > context_tokens - first_position) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if ((head_dim != 64 && head_dim != 128) || context_tokens * kv_heads * head_dim * 2 >= ((size_t)1 << 31) ||
        seqs * layers > 65535 || kv_heads > 65535 || !al16(value_cache) || !al16(value_cache_t)) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (count == 0) {
        return TE_STATUS_OK;
    }
    return launch_value_transpose(reinterpret_cast<const f16 *>(value_cache), reinterpret_cast<f16 *>(value_cache_t),
                                  seqs * layers, first_position, count, context_tokens, kv_heads, head_dim,
                                  te_hip::as_stream(stream));
}

extern "C" size_t te_hip_attention_prefill_vt_workspace_bytes(size_t seqs, size_t layers, size_t tokens,
                                                             size_t base_position, size_t context_tokens,
                                                             size_t heads, size_t kv_heads, size_t head_dim) {
    if (check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim) !=
        TE_STATUS_OK) {
        return 0;
    }
    const int splits = prefill_splits(seqs, layers, tokens, base_position, heads, head_dim);
    return prefill_workspace(splits, seqs, layers, tokens, heads, head_dim);
}

extern "C" te_status te_hip_attention_prefill_vt_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache_t,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream) {
    if (q_half == nullptr || key_cache == nullptr || value_cache_t == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (!al16(q_half) || !al16(key_cache) || !al16(value_cache_t) || !al16(out) || !al16(workspace)) {
        return TE_STATUS_UNSUPPORTED;
    }
    const int splits = splits_for(workspace, workspace_bytes, seqs, layers, tokens, base_position, heads, head_dim,
                                  &st);
    if (st != TE_STATUS_OK) {
        return st;
    }
    PrefillArgs a = {};
    a.q = reinterpret_cast<const f16 *>(q_half);
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_t = reinterpret_cast<const f16 *>(value_cache_t);
    return run_prefill(a, splits, workspace, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads,
                       head_dim, out, te_hip::as_stream(stream));
}

te_status te_hip::launch_prefill_step_vt(const float *query, const float *k_new, const float *v_new,
                                         const float *q_bias, const float *k_bias, const float *v_bias,
                                         const float *rope_cos, const float *rope_sin, uint16_t *key_cache,
                                         uint16_t *value_cache, uint16_t *value_cache_t, size_t seqs, size_t layers,
                                         size_t tokens, size_t base_position, size_t context_tokens, size_t heads,
                                         size_t kv_heads, size_t head_dim, float *out, void *act_out,
                                         void *workspace, size_t workspace_bytes, hipStream_t strm) {
    if (query == nullptr || k_new == nullptr || v_new == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || value_cache_t == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (seqs > TE_HIP_MAX_SEQS || tokens > 65535) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (!al16(query) || !al16(q_bias) || !al16(rope_cos) || !al16(rope_sin) || !al16(key_cache) ||
        !al16(value_cache) || !al16(value_cache_t) || !al16(out) || !al16(workspace) || !al16(act_out)) {
        return TE_STATUS_UNSUPPORTED;
    }
    const int splits = splits_for(workspace, workspace_bytes, seqs, layers, tokens, base_position, heads, head_dim,
                                  &st);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (act_out != nullptr && splits != 1) {
        return TE_STATUS_UNSUPPORTED;  // the digits come from the one-split kernels only
    }
    if (al16(k_new) && al16(v_new)) {
        // bias + RoPE + fp16 append of k / v and the chunk's V^T rows: one launch
        st = te_hip::launch_kv_append_vt(k_new, v_new, k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache,
                                         value_cache_t, seqs * layers, layers, tokens, base_position, context_tokens,
                                         vt_pitch(context_tokens), kv_heads, head_dim, strm);
    } else {
        // k / v rows off 16-byte alignment: the append's element-wise form
        // (the same bits), then the chunk's V^T rows from the value cache
        st = te_hip::launch_kv_append(k_new, v_new, k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache, seqs,
                                      layers, tokens, base_position, context_tokens, kv_heads, head_dim, strm);
        if (st == TE_STATUS_OK) {
            st = launch_value_transpose(reinterpret_cast<const f16 *>(value_cache),
                                        reinterpret_cast<f16 *>(value_cache_t), seqs * layers, base_position, tokens,
                                        context_tokens, kv_heads, head_dim, strm);
        }
    }
    if (st != TE_STATUS_OK) {
        return st;
    }
    PrefillArgs a = {};
    a.q32 = query;
    a.q_bias = q_bias;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_t = reinterpret_cast<const f16 *>(value_cache_t);
    return run_prefill(a, splits, workspace, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads,
                       head_dim, out, strm, act_out);
}

extern "C" te_status te_hip_attention_prefill_step_vt_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache, uint16_t *value_cache_t,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream) {
    return te_hip::launch_prefill_step_vt(query, k_new, v_new, q_bias, k_bias, v_bias, rope_cos, rope_sin, key_cache,
                                          value_cache, value_cache_t, seqs, layers, tokens, base_position,
                                          context_tokens, heads, kv_heads, head_dim, out, nullptr, workspace,
                                          workspace_bytes, te_hip::as_stream(stream));
}

// ---- entry points over the plain value cache: V^T is built per call --------

extern "C" te_status te_hip_attention_prefill_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *stream) {
    if (q_half == nullptr || key_cache == nullptr || value_cache == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (!al16(q_half) || !al16(key_cache) || !al16(value_cache) || !al16(out)) {
        return TE_STATUS_UNSUPPORTED;
    }
    // V^T of positions 0 .. base + tokens in a library-owned buffer: whole
    // calls are serialized on it (calls must share one stream).
    std::lock_guard<std::mutex> lock(te_hip::library_mutex());
    void *vt = nullptr;
    st = te_hip::library_buffer(te_hip::kLibBufPrefillVt, vt_bytes(seqs, layers, context_tokens, kv_heads, head_dim),
                                &vt);
    if (st != TE_STATUS_OK) {
        return st;
    }
    hipStream_t strm = te_hip::as_stream(stream);
    st = launch_value_transpose(reinterpret_cast<const f16 *>(value_cache), static_cast<f16 *>(vt), seqs * layers, 0,
                                base_position + tokens, context_tokens, kv_heads, head_dim, strm);
    if (st != TE_STATUS_OK) {
        return st;
    }
    PrefillArgs a = {};
    a.q = reinterpret_cast<const f16 *>(q_half);
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_t = static_cast<const f16 *>(vt);
    return run_prefill(a, 1, nullptr, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim,
                       out, strm);
}

extern "C" size_t te_hip_attention_prefill_workspace_bytes(size_t seqs, size_t layers, size_t tokens,
                                                          size_t base_position, size_t context_tokens, size_t heads,
                                                          size_t kv_heads, size_t head_dim) {
    if (check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim) !=
        TE_STATUS_OK) {
        return 0;
    }
    const int splits = prefill_splits(seqs, layers, tokens, base_position, heads, head_dim);
    return prefill_workspace(splits, seqs, layers, tokens, heads, head_dim) +
           vt_bytes(seqs, layers, context_tokens, kv_heads, head_dim);
}

extern "C" te_status te_hip_attention_prefill_split_f16(
    const uint16_t *q_half, const uint16_t *key_cache, const uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream) {
    if (q_half == nullptr || key_cache == nullptr || value_cache == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (workspace == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (!al16(q_half) || !al16(key_cache) || !al16(value_cache) || !al16(out) || !al16(workspace)) {
        return TE_STATUS_UNSUPPORTED;
    }
    const int splits = prefill_splits(seqs, layers, tokens, base_position, heads, head_dim);
    const size_t part = prefill_workspace(splits, seqs, layers, tokens, heads, head_dim);
    if (workspace_bytes < part + vt_bytes(seqs, layers, context_tokens, kv_heads, head_dim)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    f16 *vt = reinterpret_cast<f16 *>(static_cast<unsigned char *>(workspace) + part);
    hipStream_t strm = te_hip::as_stream(stream);
    st = launch_value_transpose(reinterpret_cast<const f16 *>(value_cache), vt, seqs * layers, 0,
                                base_position + tokens, context_tokens, kv_heads, head_dim, strm);
    if (st != TE_STATUS_OK) {
        return st;
    }
    PrefillArgs a = {};
    a.q = reinterpret_cast<const f16 *>(q_half);
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_t = vt;
    return run_prefill(a, splits, workspace, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads,
                       head_dim, out, strm);
}

extern "C" te_status te_hip_attention_prefill_step_f16(
    const float *query, const float *k_new, const float *v_new,
    const float *q_bias, const float *k_bias, const float *v_bias,
    const float *rope_cos, const float *rope_sin,
    uint16_t *key_cache, uint16_t *value_cache,
    size_t seqs, size_t layers, size_t tokens, size_t base_position, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim, float *out, void *stream) {
    if (query == nullptr || k_new == nullptr || v_new == nullptr || rope_cos == nullptr || rope_sin == nullptr ||
        key_cache == nullptr || value_cache == nullptr || out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    te_status st = check_prefill_args(seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim);
    if (st != TE_STATUS_OK) {
        return st;
    }
    if (seqs > TE_HIP_MAX_SEQS || tokens > 65535) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (!al16(query) || !al16(q_bias) || !al16(rope_cos) || !al16(rope_sin) || !al16(key_cache) ||
        !al16(value_cache) || !al16(out)) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(te_hip::library_mutex());
    void *vt = nullptr;
    st = te_hip::library_buffer(te_hip::kLibBufPrefillVt, vt_bytes(seqs, layers, context_tokens, kv_heads, head_dim),
                                &vt);
    if (st != TE_STATUS_OK) {
        return st;
    }
    hipStream_t strm = te_hip::as_stream(stream);
    st = te_hip::launch_kv_append(k_new, v_new, k_bias, v_bias, rope_cos, rope_sin, key_cache, value_cache, seqs,
                                  layers, tokens, base_position, context_tokens, kv_heads, head_dim, strm);
    if (st == TE_STATUS_OK) {
        st = launch_value_transpose(reinterpret_cast<const f16 *>(value_cache), static_cast<f16 *>(vt), seqs * layers,
                                    0, base_position + tokens, context_tokens, kv_heads, head_dim, strm);
    }
    if (st != TE_STATUS_OK) {
        return st;
    }
    PrefillArgs a = {};
    a.q32 = query;
    a.q_bias = q_bias;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.key_cache = reinterpret_cast<const f16 *>(key_cache);
    a.value_t = static_cast<const f16 *>(vt);
    return run_prefill(a, 1, nullptr, seqs, layers, tokens, base_position, context_tokens, heads, kv_heads, head_dim,
                       out, strm);
}
