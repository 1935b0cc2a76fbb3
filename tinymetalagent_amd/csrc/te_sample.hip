// Top-k temperature sampling of a generated token (the reference's sampler,
// c/src/qwen.c:1182-1250) with the candidate search on the device.
//
// The reference scans the logits once, in index order, keeping k candidates:
// the first k logits, then each logit strictly greater than the current
// minimum replaces that minimum (the first one on a tie).  The candidates'
// ORDER matters -- the draw walks their cumulative probabilities in slot
// order -- so the scan itself runs on the host, exactly as the reference
// runs it, but only over the logits that can enter the list: after the fill,
// a logit enters only if it is above the k-th largest value of everything
// before it.  Any subset of the prefix bounds that from below, so the device
// computes, for each 1024-logit block c, t_c = the largest k-th largest value
// over the 1024-blocks and the 8192-blocks lying wholly before c, and keeps
// the logits above t_c (all of block 0, which holds the fill).  A logit at or
// below t_c is at or below the list's minimum when the scan reaches it, so it
// never enters, and the host scan over the kept logits builds the same list
// in the same slot order.  For 151,936 logits and k = 40 that is a few
// hundred to a few thousand (index, value) pairs instead of 600 KB.
//
// A NaN logit makes the reference's minimum search order-dependent; the
// device flags it and the host then scans every logit.

#include "te_hip_common.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

namespace {

constexpr int kBlock = 1024;       // scan block: one workgroup of the candidate pass
constexpr int kBigBlock = 8192;    // second, coarser set of bounding blocks
constexpr int kThreads = 256;
constexpr uint32_t kMaxTopK = 1024;  // the reference's cap on k
constexpr size_t kFirstCopy = 4096;  // candidates read back with the header

// Order-preserving key of a float: larger float, larger key.
__device__ __forceinline__ uint32_t float_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SampleLayout {
    size_t hdr, entries, kth, kth_big, bytes;
    int blocks, big_blocks;
};

// Device workspace: [0] candidate count, [1] NaN flag, then per block
// (base, count) of its candidates, the (index, value bits) pairs, and the
// two k-th-largest arrays.  Capacity: every logit.
SampleLayout sample_layout(size_t n) {
    SampleLayout l;
    l.blocks = (int)((n + kBlock - 1) / kBlock);
    l.big_blocks = (int)(n / kBigBlock);  // whole 8192-blocks only
    l.hdr = 8;
    l.entries = l.hdr + (size_t)l.blocks * 8;
    l.kth = l.entries + n * 8;
    l.kth_big = l.kth + (size_t)l.blocks * 4;
    l.bytes = (l.kth_big + (size_t)l.big_blocks * 4 + 255) / 256 * 256;
    return l;
}

// The k-th largest of the `cnt` keys held PER per thread (thread t, slot j:
// key j * 256 + t), by a 4-pass radix select (8 bits a pass) over LDS
// histograms; exact.
template <int PER>
__device__ __forceinline__ uint32_t kth_key(const uint32_t (&key)[PER], uint32_t cnt, uint32_t k) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel[2];  // chosen digit, the rank left within it
    uint32_t prefix = 0, mask = 0, rank = k;  // the rank-th largest among keys matching prefix under mask
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[threadIdx.x] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if ((uint32_t)j * kThreads + threadIdx.x < cnt && (key[j] & mask) == prefix) {
                atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
            }
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            // lane l sums digits 255-4l .. 252-4l; the first lane whose running
            // total from the top reaches the rank holds the digit
            const int lane = threadIdx.x;
            uint32_t c[4], s = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c[q] = hist[255 - 4 * lane - q];
                s += c[q];
            }
            uint32_t incl = s;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o, 64);
                if (lane >= o) {
                    incl += t;
                }
            }
            const unsigned long long hit = __ballot(incl >= rank);
            const int first = __ffsll((long long)hit) - 1;
            if (lane == first) {
                uint32_t above = incl - s;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (above + c[q] >= rank) {
                        sel[0] = 255u - 4u * (uint32_t)lane - (uint32_t)q;
                        sel[1] = rank - above;
                        break;
                    }
                    above += c[q];
                }
            }
        }
        __syncthreads();
        prefix |= sel[0] << shift;
        mask |= 255u << shift;
        rank = sel[1];
        __syncthreads();
    }
    return prefix;
}

template <int LEN>
__device__ __forceinline__ void kth_block(const float *x, uint32_t n, uint32_t k, uint32_t start, float *out) {
    constexpr int PER = LEN / kThreads;
    const uint32_t cnt = min((uint32_t)LEN, n - start);
    if (cnt < k) {  // uniform
        if (threadIdx.x == 0) {
            *out = -INFINITY;
        }
        return;
    }
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t i = (uint32_t)j * kThreads + threadIdx.x;
        key[j] = i < cnt ? float_key(x[start + i]) : 0u;
    }
    const uint32_t kk = kth_key<PER>(key, cnt, k);
    if (threadIdx.x == 0) {
        *out = key_float(kk);
    }
}

// Workgroup w < blocks: the k-th largest of 1024-block w; w >= blocks: of
// 8192-block w - blocks; -inf for a block shorter than k.  Workgroup 0 also
// clears the header (candidate counter, NaN flag) for the candidate pass,
// which runs after this launch.
__global__ __launch_bounds__(kThreads) void kth_largest_kernel(const float *x, uint32_t n, uint32_t k, int blocks,
                                                               unsigned char *ws, SampleLayout l) {
    const int w = blockIdx.x;
    if (w == 0 && threadIdx.x < 2) {
        reinterpret_cast<uint32_t *>(ws)[threadIdx.x] = 0u;
    }
    if (w < blocks) {
        kth_block<kBlock>(x, n, k, (uint32_t)w * kBlock, reinterpret_cast<float *>(ws + l.kth) + w);
    } else {
        kth_block<kBigBlock>(x, n, k, (uint32_t)(w - blocks) * kBigBlock,
                             reinterpret_cast<float *>(ws + l.kth_big) + (w - blocks));
    }
}

// Workgroup c: the logits of 1024-block c above t_c (every logit of block 0),
// in index order, at a base taken from the shared counter; (base, count) to
// the block's header slot.
__global__ __launch_bounds__(kThreads) void candidates_kernel(const float *x, uint32_t n, unsigned char *ws,
                                                              SampleLayout l) {
    const int c = blockIdx.x;
    const uint32_t start = (uint32_t)c * kBlock;
    const float *kth = reinterpret_cast<const float *>(ws + l.kth);
    const float *kth_big = reinterpret_cast<const float *>(ws + l.kth_big);
    __shared__ float red[kThreads];
    __shared__ uint32_t scan[kThreads];
    __shared__ uint32_t base_s;
    float t = -INFINITY;
    for (int b = threadIdx.x; b < c; b += kThreads) {
        t = fmaxf(t, kth[b]);
    }
    for (int b = threadIdx.x; b < c / (kBigBlock / kBlock) && b < l.big_blocks; b += kThreads) {
        t = fmaxf(t, kth_big[b]);
    }
    red[threadIdx.x] = t;
    __syncthreads();
    for (int o = kThreads / 2; o >= 1; o >>= 1) {
        if ((int)threadIdx.x < o) {
            red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        }
        __syncthreads();
    }
    t = red[0];
    float v[4];
    uint32_t take = 0;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = start + 4 * threadIdx.x + j;
        v[j] = i < n ? x[i] : -INFINITY;
        nan |= v[j] != v[j];
        if (i < n && (c == 0 || v[j] > t)) {
            take |= 1u << j;
        }
    }
    if (nan) {
        reinterpret_cast<uint32_t *>(ws)[1] = 1u;  // the host then scans every logit
    }
    // exclusive scan of the per-thread counts (Hillis-Steele)
    const uint32_t mine = __popc(take);
    scan[threadIdx.x] = mine;
    __syncthreads();
    for (int o = 1; o < kThreads; o <<= 1) {
        const uint32_t add = (int)threadIdx.x >= o ? scan[threadIdx.x - o] : 0u;
        __syncthreads();
        scan[threadIdx.x] += add;
        __syncthreads();
    }
    const uint32_t total = scan[kThreads - 1];
    uint32_t *hdr = reinterpret_cast<uint32_t *>(ws);
    if (threadIdx.x == 0) {
        const uint32_t base = total > 0 ? atomicAdd(&hdr[0], total) : 0u;
        base_s = base;
        uint32_t *slot = reinterpret_cast<uint32_t *>(ws + l.hdr) + 2 * c;
        slot[0] = base;
        slot[1] = total;
    }
    __syncthreads();
    uint32_t pos = base_s + scan[threadIdx.x] - mine;
    uint2 *entries = reinterpret_cast<uint2 *>(ws + l.entries);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (take & (1u << j)) {
            entries[pos++] = make_uint2(start + 4 * threadIdx.x + j, __float_as_uint(v[j]));
        }
    }
}

// The reference's scan and draw over a stream of (index, value) in index
// order; next(j) gives element j of `count`.  The reference's list: slots
// filled in order, then each value strictly above the list's minimum replaces
// it, the minimum being the first (lowest) slot holding the smallest value.
// Without NaN the slots sit in a binary heap ordered by (value, slot), whose
// top is exactly that slot, so a replacement costs O(log k) instead of a pass
// over the k slots; with a NaN (`reference_min`) the minimum is searched the
// reference's way, whose comparisons then decide the list.
template <typename Next>
uint32_t scan_and_draw(size_t count, uint32_t k, float temperature, uint64_t *rng, Next next,
                       bool reference_min = false) {
    thread_local std::vector<float> v;
    thread_local std::vector<uint32_t> idx;
    thread_local std::vector<uint32_t> heap;  // slots
    v.clear();
    idx.clear();
    heap.clear();
    auto below = [&](uint32_t a, uint32_t b) { return v[a] < v[b] || (!(v[b] < v[a]) && a < b); };
    auto sift_down = [&](size_t i) {
        const size_t n = heap.size();
        for (;;) {
            const size_t l = 2 * i + 1, r = l + 1;
            size_t m = i;
            if (l < n && below(heap[l], heap[m])) {
                m = l;
            }
            if (r < n && below(heap[r], heap[m])) {
                m = r;
            }
            if (m == i) {
                return;
            }
            std::swap(heap[i], heap[m]);
            i = m;
        }
    };
    size_t min_pos = 0;
    auto find_min = [&] {
        min_pos = 0;
        for (size_t j = 1; j < v.size(); ++j) {
            if (v[j] < v[min_pos]) {
                min_pos = j;
            }
        }
    };
    for (size_t j = 0; j < count; ++j) {
        uint32_t i;
        float x;
        next(j, i, x);
        if (reference_min) {
            if (v.size() < k) {
                v.push_back(x);
                idx.push_back(i);
                if (v.size() == k) {
                    find_min();
                }
            } else if (x > v[min_pos]) {
                v[min_pos] = x;
                idx[min_pos] = i;
                find_min();
            }
            continue;
        }
        if (v.size() < k) {
            v.push_back(x);
            idx.push_back(i);
            if (v.size() == k) {
                heap.resize(k);
                for (uint32_t t = 0; t < k; ++t) {
                    heap[t] = t;
                }
                for (size_t t = k / 2; t-- > 0;) {
                    sift_down(t);
                }
            }
        } else if (x > v[heap[0]]) {
            v[heap[0]] = x;
            idx[heap[0]] = i;
            sift_down(0);
        }
    }
    float mx = v[0];
    for (size_t j = 1; j < v.size(); ++j) {
        mx = v[j] > mx ? v[j] : mx;
    }
    const double t = temperature > 1e-6f ? (double)temperature : 1e-6;
    thread_local std::vector<double> p;
    p.resize(v.size());
    double sum = 0.0;
    for (size_t j = 0; j < v.size(); ++j) {
        p[j] = exp(((double)v[j] - (double)mx) / t);
        sum += p[j];
    }
    // xorshift64* to a double in [0, 1) (qwen.c:1170-1178)
    uint64_t s = *rng;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *rng = s;
    const double r = (double)((s * 0x2545F4914F6CDD1DULL) >> 11) / 9007199254740992.0 * sum;
    size_t choice = v.size() - 1;
    double acc = 0.0;
    for (size_t j = 0; j < v.size(); ++j) {
        acc += p[j];
        if (r <= acc) {
            choice = j;
            break;
        }
    }
    return idx[choice];
}

// Pinned host staging for the read-back, grown on demand, one per thread and
// released when the thread ends (a thread's thread_local objects are
// destroyed before the process's static objects, so the runtime is still up).
struct HostStage {
    void *p = nullptr;
    size_t bytes = 0;
    HostStage() = default;
    HostStage(const HostStage &) = delete;
    HostStage &operator=(const HostStage &) = delete;
    ~HostStage() {
        if (p != nullptr) {
            (void)hipHostFree(p);
        }
    }
    unsigned char *get(size_t need) {
        if (need > bytes) {
            if (p != nullptr) {
                (void)hipHostFree(p);
                p = nullptr;
                bytes = 0;
            }
            if (hipHostMalloc(&p, need, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                return nullptr;
            }
            bytes = need;
        }
        return static_cast<unsigned char *>(p);
    }
};
thread_local HostStage g_stage;

}  // namespace

extern "C" size_t te_hip_sample_workspace_bytes(size_t vocab) { return vocab == 0 ? 0 : sample_layout(vocab).bytes; }

extern "C" te_status te_hip_sample_top_k_f32(const float *logits, size_t vocab, uint32_t top_k, float temperature,
                                             uint64_t *rng_state, uint32_t *out_token, void *workspace,
                                             size_t workspace_bytes, void *stream) {
    if (logits == nullptr || vocab == 0 || rng_state == nullptr || out_token == nullptr || workspace == nullptr ||
        vocab > 0x7fffffffu) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const SampleLayout l = sample_layout(vocab);
    if (workspace_bytes < l.bytes) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const uint32_t k = (uint32_t)std::min<size_t>(top_k == 0 ? 1 : std::min(top_k, kMaxTopK), vocab);
    const hipStream_t st = te_hip::as_stream(stream);
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    kth_largest_kernel<<<l.blocks + l.big_blocks, kThreads, 0, st>>>(logits, (uint32_t)vocab, k, l.blocks, ws, l);
    candidates_kernel<<<l.blocks, kThreads, 0, st>>>(logits, (uint32_t)vocab, ws, l);
    te_status s = te_hip::launch_status();
    if (s != TE_STATUS_OK) {
        return s;
    }
    // header and the first candidates in one copy, the rest only if needed
    const size_t first = l.entries + std::min<size_t>(vocab, kFirstCopy) * 8;
    unsigned char *h = g_stage.get(l.entries + vocab * 8);
    if (h == nullptr) {
        return TE_STATUS_OUT_OF_MEMORY;
    }
    if (hipMemcpyAsync(h, ws, first, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    uint32_t hdr[2];
    memcpy(hdr, h, sizeof hdr);
    if (hdr[1] != 0) {
        // a NaN logit: the reference's scan over every logit
        std::vector<float> all(vocab);
        if (hipMemcpy(all.data(), logits, vocab * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
            return TE_STATUS_RUNTIME_ERROR;
        }
        *out_token = scan_and_draw(
            vocab, k, temperature, rng_state,
            [&](size_t j, uint32_t &i, float &x) {
                i = (uint32_t)j;
                x = all[j];
            },
            true);
        return TE_STATUS_OK;
    }
    const size_t total = hdr[0];
    if (total > kFirstCopy && hipMemcpy(h + first, ws + first, (total - kFirstCopy) * 8, hipMemcpyDeviceToHost) !=
                                  hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    // the candidates in block order (blocks took their bases in any order)
    thread_local std::vector<size_t> order;
    order.clear();
    order.reserve(total);
    const uint32_t *slots = reinterpret_cast<const uint32_t *>(h + l.hdr);
    for (int c = 0; c < l.blocks; ++c) {
        for (uint32_t j = 0; j < slots[2 * c + 1]; ++j) {
            order.push_back((size_t)slots[2 * c] + j);
        }
    }
    if (order.size() != total) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    const uint32_t *e = reinterpret_cast<const uint32_t *>(h + l.entries);
    *out_token = scan_and_draw(total, k, temperature, rng_state, [&](size_t j, uint32_t &i, float &x) {
        i = e[2 * order[j]];
        memcpy(&x, &e[2 * order[j] + 1], sizeof x);
    });
    return TE_STATUS_OK;
}
