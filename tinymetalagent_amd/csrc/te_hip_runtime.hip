// Host side of the HIP backend: device discovery, the process-wide mutex and
// lazily grown device buffers used by the host-pointer entry points, and the
// GPU implementations of the public attention-step functions te_rope_f32 and
// te_attention_decode_f32.
//
// Mirrors the reference backend runtime's ownership model
// (metal_backend_runtime.mm.inc:68-130): one process-global runtime, buffers
// grown on demand and kept, every host-pointer call serialized by one mutex and
// synchronous (upload, launch, download, wait).
#include "te_hip_common.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <mutex>
#include <vector>

namespace {

std::mutex g_mutex;

struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;

    te_status ensure(size_t need) {
        if (need <= bytes) {
            return TE_STATUS_OK;
        }
        if (ptr != nullptr) {
            (void)hipFree(ptr);
            ptr = nullptr;
            bytes = 0;
        }
        if (hipMalloc(&ptr, need) != hipSuccess) {
            ptr = nullptr;
            (void)hipGetLastError();
            return TE_STATUS_OUT_OF_MEMORY;
        }
        bytes = need;
        return TE_STATUS_OK;
    }
    template <typename T>
    T *as() const {
        return static_cast<T *>(ptr);
    }
};

struct Runtime {
    int probed = 0;      // 0 = not yet, 1 = done
    int available = 0;   // gfx950 device present
    int device = 0;
    char name[128] = {0};
    uint32_t cus = 0;
    hipStream_t stream = nullptr;
    DeviceBuffer buf[6];
};

Runtime g_rt;
DeviceBuffer g_library_buffers[te_hip::kLibBufCount];

// Caller holds g_mutex.
int probe_locked() {
    if (g_rt.probed) {
        return g_rt.available;
    }
    g_rt.probed = 1;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return 0;
    }
    if (hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    g_rt.device = dev;
    snprintf(g_rt.name, sizeof(g_rt.name), "%s (%s)", prop.name, "gfx950");
    g_rt.cus = (uint32_t)prop.multiProcessorCount;
    g_rt.available = 1;
    return 1;
}

te_status sync_status() {
    return hipStreamSynchronize(g_rt.stream) == hipSuccess ? TE_STATUS_OK : TE_STATUS_RUNTIME_ERROR;
}

te_status h2d(void *dst, const void *src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_rt.stream) == hipSuccess
               ? TE_STATUS_OK
               : TE_STATUS_RUNTIME_ERROR;
}

te_status d2h(void *dst, const void *src, size_t bytes) {
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_rt.stream) != hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    return sync_status();
}

bool mul_ok(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) {
        return false;
    }
    *out = a * b;
    return true;
}

// Shared body of the four MMA twins.
te_status mma_twin(int mode, const float *query, const float *key_t, const float *value, size_t k_cols,
                   size_t q_base, float *out) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t qb = 8 * 64 * sizeof(float);
    const size_t kb = 64 * k_cols * sizeof(float);
    const size_t ob = (mode == 0 ? 8 * k_cols : 8 * 64) * sizeof(float);
    te_status st;
    if ((st = g_rt.buf[0].ensure(qb)) != TE_STATUS_OK || (st = g_rt.buf[1].ensure(kb)) != TE_STATUS_OK ||
        (st = g_rt.buf[2].ensure(kb)) != TE_STATUS_OK || (st = g_rt.buf[3].ensure(ob)) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, query, qb)) != TE_STATUS_OK ||
        (st = h2d(g_rt.buf[1].ptr, key_t, kb)) != TE_STATUS_OK) {
        return st;
    }
    if (value != nullptr && (st = h2d(g_rt.buf[2].ptr, value, kb)) != TE_STATUS_OK) {
        return st;
    }
    st = te_hip::launch_mma_kat(mode, g_rt.buf[0].as<float>(), g_rt.buf[1].as<float>(), g_rt.buf[2].as<float>(),
                                (int)k_cols, (int)q_base, g_rt.buf[3].as<float>(), g_rt.stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return d2h(out, g_rt.buf[3].ptr, ob);
}

}  // namespace

namespace te_hip {

namespace {

struct ProfMark {
    hipEvent_t ev;
    double share[kProfCount];
};

// One thread's profile: a pool of events reused across flushes, the marks
// recorded since the last flush, and the accumulated phase times.
struct Profile {
    bool active = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    hipEvent_t begin = nullptr;
    std::vector<ProfMark> marks;
    double ms[kProfCount] = {};
    unsigned long long calls[kProfCount] = {};
    // (the pool's events are not destroyed at thread exit: the runtime may
    // already be gone then)
    hipEvent_t next_event() {
        if (used == pool.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) {
                return nullptr;
            }
            pool.push_back(e);
        }
        return pool[used++];
    }
};

thread_local Profile t_prof;

}  // namespace

bool prof_active() { return t_prof.active; }

void prof_start() {
    t_prof.active = true;
    t_prof.used = 0;
    t_prof.begin = nullptr;
    t_prof.marks.clear();
    for (int i = 0; i < kProfCount; ++i) {
        t_prof.ms[i] = 0.0;
        t_prof.calls[i] = 0;
    }
}

void prof_stop() { t_prof.active = false; }

void prof_begin(hipStream_t stream) {
    if (!t_prof.active || t_prof.begin != nullptr) {
        return;
    }
    hipEvent_t e = t_prof.next_event();
    if (e != nullptr && hipEventRecord(e, stream) == hipSuccess) {
        t_prof.begin = e;
    }
}

void prof_mark(hipStream_t stream, const ProfShare *shares, int n) {
    if (!t_prof.active) {
        return;
    }
    prof_begin(stream);
    hipEvent_t e = t_prof.next_event();
    if (e == nullptr || hipEventRecord(e, stream) != hipSuccess) {
        return;
    }
    ProfMark m = {};
    m.ev = e;
    double total = 0.0;
    for (int i = 0; i < n; ++i) {
        total += shares[i].weight;
    }
    for (int i = 0; i < n && total > 0.0; ++i) {
        m.share[shares[i].phase] += shares[i].weight / total;
    }
    t_prof.marks.push_back(m);
}

te_status prof_flush() {
    if (!t_prof.active || t_prof.marks.empty()) {
        t_prof.begin = nullptr;
        t_prof.used = 0;
        return TE_STATUS_OK;
    }
    if (hipEventSynchronize(t_prof.marks.back().ev) != hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    hipEvent_t prev = t_prof.begin;
    for (const ProfMark &m : t_prof.marks) {
        float dt = 0.0f;
        if (prev != nullptr && hipEventElapsedTime(&dt, prev, m.ev) == hipSuccess) {
            for (int i = 0; i < kProfCount; ++i) {
                if (m.share[i] > 0.0) {
                    t_prof.ms[i] += dt * m.share[i];
                    t_prof.calls[i] += 1;
                }
            }
        }
        prev = m.ev;
    }
    t_prof.marks.clear();
    t_prof.begin = nullptr;
    t_prof.used = 0;
    return TE_STATUS_OK;
}

double prof_ms(ProfPhase phase) { return t_prof.ms[phase]; }

unsigned long long prof_calls(ProfPhase phase) { return t_prof.calls[phase]; }

namespace {

struct BackendBucketTotals {
    const char *name;
    unsigned long long calls;
    double cpu_ms;
    double gpu_ms;
};

// The reference's bucket names, in its order (metal_backend_runtime.mm.inc:
// 134-175); this backend records the layer-flow ones.
BackendBucketTotals g_backend_buckets[kBucketCount] = {
    {"matvec_batch", 0, 0.0, 0.0},        {"matvec_argmax", 0, 0.0, 0.0},
    {"qkv", 0, 0.0, 0.0},                 {"qkv_batch", 0, 0.0, 0.0},
    {"mlp", 0, 0.0, 0.0},                 {"mlp_batch", 0, 0.0, 0.0},
    {"post_attn_mlp", 0, 0.0, 0.0},       {"post_attn_mlp_batch", 0, 0.0, 0.0},
    {"matvec2", 0, 0.0, 0.0},             {"matvec", 0, 0.0, 0.0},
    {"decode_layer", 0, 0.0, 0.0},        {"decode_all_layers", 0, 0.0, 0.0},
    {"decode_project", 0, 0.0, 0.0},      {"prefill_layer", 0, 0.0, 0.0},
    {"prefill_all_layers", 0, 0.0, 0.0},
};
std::mutex g_backend_mutex;
bool g_backend_registered = false;
thread_local int t_backend_depth = 0;

bool backend_profile_enabled() {
    const char *v = getenv("TINYENGINE_METAL_PROFILE");
    return v != nullptr && strcmp(v, "0") != 0;
}

double now_ms() {
    using clock = std::chrono::steady_clock;
    return std::chrono::duration<double, std::milli>(clock::now().time_since_epoch()).count();
}

// At exit: one line per bucket with calls, the reference's format
// (metal_backend_runtime.mm.inc:199-217), while the switch is still set.
void backend_profile_print() {
    if (!backend_profile_enabled()) {
        return;
    }
    std::lock_guard<std::mutex> lock(g_backend_mutex);
    for (const BackendBucketTotals &b : g_backend_buckets) {
        if (b.calls == 0) {
            continue;
        }
        fprintf(stderr,
                "tinyengine_metal_profile: name=%s calls=%llu cpu_ms=%.3f gpu_ms=%.3f avg_cpu_ms=%.3f "
                "avg_gpu_ms=%.3f\n",
                b.name, b.calls, b.cpu_ms, b.gpu_ms, b.cpu_ms / (double)b.calls, b.gpu_ms / (double)b.calls);
    }
}

}  // namespace

BackendTimer::BackendTimer(BackendBucket bucket, hipStream_t stream) : bucket_(bucket), stream_(stream) {
    nested_ = t_backend_depth++ > 0;
    if (nested_ || !backend_profile_enabled()) {
        return;
    }
    {
        std::lock_guard<std::mutex> lock(g_backend_mutex);
        if (!g_backend_registered) {
            atexit(backend_profile_print);
            g_backend_registered = true;
        }
    }
    // (the host clock starts first, so the call's GPU interval lies inside its wall time)
    t0_ms_ = now_ms();
    if (hipEventCreate(&e0_) != hipSuccess || hipEventCreate(&e1_) != hipSuccess ||
        hipEventRecord(e0_, stream_) != hipSuccess) {
        (void)hipGetLastError();  // no profile for this call; the call itself goes on
        return;
    }
    on_ = true;
}

void BackendTimer::release() {
    if (done_) {
        return;
    }
    done_ = true;
    --t_backend_depth;
    if (e0_ != nullptr) {
        (void)hipEventDestroy(e0_);
    }
    if (e1_ != nullptr) {
        (void)hipEventDestroy(e1_);
    }
    e0_ = e1_ = nullptr;
}

BackendTimer::~BackendTimer() { release(); }

te_status BackendTimer::finish(te_status st) {
    if (on_ && !done_) {
        if (hipEventRecord(e1_, stream_) != hipSuccess || hipEventSynchronize(e1_) != hipSuccess) {
            release();
            return st == TE_STATUS_OK ? TE_STATUS_RUNTIME_ERROR : st;
        }
        const double cpu_ms = now_ms() - t0_ms_;
        float gpu_ms = 0.0f;
        if (hipEventElapsedTime(&gpu_ms, e0_, e1_) != hipSuccess) {
            gpu_ms = 0.0f;
        }
        if (st == TE_STATUS_OK) {
            std::lock_guard<std::mutex> lock(g_backend_mutex);
            BackendBucketTotals &b = g_backend_buckets[bucket_];
            b.calls += 1;
            b.cpu_ms += cpu_ms;
            b.gpu_ms += (double)gpu_ms;
        }
    }
    release();
    return st;
}

std::mutex &library_mutex() { return g_mutex; }

te_status library_buffer(LibraryBuffer which, size_t bytes, void **ptr) {
    DeviceBuffer &b = g_library_buffers[which];
    const te_status st = b.ensure(bytes);
    *ptr = st == TE_STATUS_OK ? b.ptr : nullptr;
    return st;
}

}  // namespace te_hip

extern "C" int te_hip_available(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    return probe_locked();
}

extern "C" te_status te_hip_device_info(char *name, size_t name_capacity, uint32_t *compute_units) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (name != nullptr && name_capacity > 0) {
        snprintf(name, name_capacity, "%s", g_rt.name);
    }
    if (compute_units != nullptr) {
        *compute_units = g_rt.cus;
    }
    return TE_STATUS_OK;
}

extern "C" te_status te_hip_rope_table_f32(float *cos_table, float *sin_table, size_t context_tokens,
                                           size_t head_dim, float theta) {
    if (cos_table == nullptr || sin_table == nullptr || context_tokens == 0 || head_dim == 0 ||
        (head_dim % 2) != 0 || !(theta > 0.0f)) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    const size_t half = head_dim / 2;
    size_t n = 0;
    if (!mul_ok(context_tokens, half, &n) || n > ((size_t)1 << 32)) {
        return TE_STATUS_UNSUPPORTED;
    }
    // Same expression order as the reference table build (qwen.c:531-539).
    std::vector<float> c(n), s(n);
    std::vector<float> freq(half);
    for (size_t i = 0; i < half; ++i) {
        freq[i] = powf(theta, -(2.0f * (float)i) / (float)head_dim);
    }
    for (size_t p = 0; p < context_tokens; ++p) {
        for (size_t i = 0; i < half; ++i) {
            const float angle = (float)p * freq[i];
            c[p * half + i] = cosf(angle);
            s[p * half + i] = sinf(angle);
        }
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    if (hipMemcpy(cos_table, c.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(sin_table, s.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
        return TE_STATUS_RUNTIME_ERROR;
    }
    return TE_STATUS_OK;
}

// Public te_rope_f32 (reference ops.c:295-321): the cos/sin row is computed on
// the host with the reference expression (powf/sinf/cosf in fp32, as the
// reference GPU path receives host table rows, qwen.c:1448-1449); the rotation
// itself runs on the GPU.
extern "C" te_status te_rope_f32(float *values, size_t heads, size_t head_dim, size_t position, float theta) {
    if (values == nullptr || heads == 0 || head_dim == 0 || (head_dim % 2) != 0 || theta <= 0.0f) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t n = 0;
    if (!mul_ok(heads, head_dim, &n) || n > ((size_t)1 << 31)) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t half = head_dim / 2;
    std::vector<float> row(2 * half);
    for (size_t i = 0; i < half; ++i) {
        const float freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
        const float angle = (float)position * freq;
        row[i] = cosf(angle);
        row[half + i] = sinf(angle);
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_status st;
    if ((st = g_rt.buf[0].ensure(n * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[1].ensure(2 * half * sizeof(float))) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, values, n * sizeof(float))) != TE_STATUS_OK ||
        (st = h2d(g_rt.buf[1].ptr, row.data(), 2 * half * sizeof(float))) != TE_STATUS_OK) {
        return st;
    }
    float *dcos = g_rt.buf[1].as<float>();
    st = te_hip::launch_rope_rows(g_rt.buf[0].as<float>(), heads, head_dim, dcos, dcos + half, g_rt.stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return d2h(values, g_rt.buf[0].ptr, n * sizeof(float));
}

// Public decode-layer vector operations (reference ops.c:272-293, :397-433) on
// the GPU: host arrays are copied in, the te_hip_* kernel runs, the result is
// copied back; synchronous, serialized by the library mutex like te_rope_f32.
namespace {

te_status host_vector_op(const float *a, const float *b, size_t len, float *out,
                         te_status (*launch)(const float *, const float *, size_t, float *, hipStream_t)) {
    size_t bytes = 0;
    if (!mul_ok(len, sizeof(float), &bytes) || len > ((size_t)1 << 31)) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_status st;
    if ((st = g_rt.buf[0].ensure(bytes)) != TE_STATUS_OK || (st = g_rt.buf[1].ensure(bytes)) != TE_STATUS_OK ||
        (st = g_rt.buf[2].ensure(bytes)) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, a, bytes)) != TE_STATUS_OK || (st = h2d(g_rt.buf[1].ptr, b, bytes)) != TE_STATUS_OK) {
        return st;
    }
    if ((st = launch(g_rt.buf[0].as<float>(), g_rt.buf[1].as<float>(), len, g_rt.buf[2].as<float>(), g_rt.stream)) !=
        TE_STATUS_OK) {
        return st;
    }
    return d2h(out, g_rt.buf[2].ptr, bytes);
}

}  // namespace

extern "C" te_status te_rmsnorm_f32(const float *input, const float *weight, size_t len, float epsilon, float *out) {
    if (input == nullptr || weight == nullptr || out == nullptr || len == 0 || epsilon <= 0.0f) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t bytes = 0;
    if (!mul_ok(len, sizeof(float), &bytes) || len > 0x7fffffffu) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_status st;
    if ((st = g_rt.buf[0].ensure(bytes)) != TE_STATUS_OK || (st = g_rt.buf[1].ensure(bytes)) != TE_STATUS_OK ||
        (st = g_rt.buf[2].ensure(bytes)) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, input, bytes)) != TE_STATUS_OK ||
        (st = h2d(g_rt.buf[1].ptr, weight, bytes)) != TE_STATUS_OK) {
        return st;
    }
    st = te_hip::launch_rmsnorm(g_rt.buf[0].as<float>(), g_rt.buf[1].as<float>(), 1, len, epsilon,
                                g_rt.buf[2].as<float>(), g_rt.stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return d2h(out, g_rt.buf[2].ptr, bytes);
}

extern "C" te_status te_swiglu_f32(const float *gate, const float *up, size_t len, float *out) {
    if (gate == nullptr || up == nullptr || out == nullptr || len == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return host_vector_op(gate, up, len, out, te_hip::launch_swiglu);
}

extern "C" te_status te_add_f32(const float *lhs, const float *rhs, size_t len, float *out) {
    if (lhs == nullptr || rhs == nullptr || out == nullptr || len == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    return host_vector_op(lhs, rhs, len, out, te_hip::launch_add);
}

extern "C" te_status te_argmax_f32(const float *values, size_t len, uint32_t *out_index) {
    if (values == nullptr || out_index == nullptr || len == 0 || len > 0xffffffffu) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    size_t bytes = 0;
    if (!mul_ok(len, sizeof(float), &bytes)) {
        return TE_STATUS_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_status st;
    if ((st = g_rt.buf[0].ensure(bytes)) != TE_STATUS_OK || (st = g_rt.buf[1].ensure(sizeof(uint32_t))) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, values, bytes)) != TE_STATUS_OK) {
        return st;
    }
    if ((st = te_hip::launch_argmax(g_rt.buf[0].as<float>(), len, g_rt.buf[1].as<uint32_t>(), g_rt.stream)) !=
        TE_STATUS_OK) {
        return st;
    }
    return d2h(out_index, g_rt.buf[1].ptr, sizeof(uint32_t));
}

// Public te_attention_decode_f32 (reference ops.c:323-395) on the GPU: the fp32
// cache prefix 0..position is uploaded and attended by a chunked fp32 kernel
// plus the split-K combine kernel.
extern "C" te_status te_attention_decode_f32(const float *query, const float *key_cache,
                                             const float *value_cache, size_t position, size_t heads,
                                             size_t kv_heads, size_t head_dim, float *out) {
    if (query == nullptr || key_cache == nullptr || value_cache == nullptr || out == nullptr || heads == 0 ||
        kv_heads == 0 || head_dim == 0 || (heads % kv_heads) != 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (position == SIZE_MAX) {
        return TE_STATUS_UNSUPPORTED;
    }
    size_t n = position + 1, kv_elems = 0, q_elems = 0;
    if (!mul_ok(kv_heads, head_dim, &kv_elems) || !mul_ok(n, kv_elems, &kv_elems) ||
        !mul_ok(heads, head_dim, &q_elems) || kv_elems > ((size_t)1 << 34) || n > ((size_t)1 << 30) ||
        heads > 65535 || head_dim > 65535) {
        return TE_STATUS_UNSUPPORTED;
    }
    const size_t chunk = (size_t)te_hip::f32_decode_chunk(position);
    const size_t chunks = (n + chunk - 1) / chunk;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!probe_locked()) {
        return TE_STATUS_UNSUPPORTED;
    }
    te_status st;
    if ((st = g_rt.buf[0].ensure(q_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[1].ensure(kv_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[2].ensure(kv_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[3].ensure(q_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[4].ensure(heads * chunks * head_dim * sizeof(float))) != TE_STATUS_OK ||
        (st = g_rt.buf[5].ensure(heads * chunks * 2 * sizeof(float))) != TE_STATUS_OK) {
        return st;
    }
    if ((st = h2d(g_rt.buf[0].ptr, query, q_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = h2d(g_rt.buf[1].ptr, key_cache, kv_elems * sizeof(float))) != TE_STATUS_OK ||
        (st = h2d(g_rt.buf[2].ptr, value_cache, kv_elems * sizeof(float))) != TE_STATUS_OK) {
        return st;
    }
    st = te_hip::launch_decode_f32(g_rt.buf[0].as<float>(), g_rt.buf[1].as<float>(), g_rt.buf[2].as<float>(),
                                   position, heads, kv_heads, head_dim, g_rt.buf[3].as<float>(),
                                   g_rt.buf[4].as<float>(), g_rt.buf[5].as<float>(), g_rt.stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return d2h(out, g_rt.buf[3].ptr, q_elems * sizeof(float));
}

// Convenience form of the two decode stages with an optional library-owned
// workspace.
extern "C" te_status te_hip_attention_decode_f16(
    const float *query, const uint16_t *key_cache, const uint16_t *value_cache,
    const size_t *positions, size_t position,
    size_t seqs, size_t layers, size_t context_tokens,
    size_t heads, size_t kv_heads, size_t head_dim,
    float *out, void *workspace, size_t workspace_bytes, void *stream) {
    if (out == nullptr) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (workspace == nullptr) {
        const size_t need =
            te_hip_attention_decode_workspace_bytes(positions, position, seqs, layers, heads, kv_heads, head_dim);
        if (need == 0) {
            return TE_STATUS_INVALID_ARGUMENT;
        }
        // The library-owned workspace is shared: serialize whole calls on it.
        std::lock_guard<std::mutex> lock(g_mutex);
        void *ws = nullptr;
        te_status st = te_hip::library_buffer(te_hip::kLibBufDecode, need, &ws);
        if (st != TE_STATUS_OK) {
            return st;
        }
        st = te_hip_attention_decode_splitk_f16(query, key_cache, value_cache, positions, position, seqs, layers,
                                                context_tokens, heads, kv_heads, head_dim, ws, need, stream);
        if (st != TE_STATUS_OK) {
            return st;
        }
        return te_hip_attention_decode_combine(positions, position, seqs, layers, heads, kv_heads, head_dim, out,
                                               ws, need, stream);
    }
    te_status st = te_hip_attention_decode_splitk_f16(query, key_cache, value_cache, positions, position, seqs,
                                                      layers, context_tokens, heads, kv_heads, head_dim,
                                                      workspace, workspace_bytes, stream);
    if (st != TE_STATUS_OK) {
        return st;
    }
    return te_hip_attention_decode_combine(positions, position, seqs, layers, heads, kv_heads, head_dim, out,
                                           workspace, workspace_bytes, stream);
}

extern "C" te_status te_hip_attention_qk_mma_f32(const float *query, const float *key_t, size_t q_rows,
                                                 size_t k_cols, size_t head_dim, float *out) {
    if (query == nullptr || key_t == nullptr || out == nullptr || q_rows == 0 || k_cols == 0 || head_dim == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (q_rows != 8 || k_cols != 8 || head_dim != 64) {
        return TE_STATUS_UNSUPPORTED;
    }
    return mma_twin(0, query, key_t, nullptr, k_cols, 0, out);
}

extern "C" te_status te_hip_attention_tile_mma_f32(const float *query, const float *key_t, const float *value,
                                                   size_t q_rows, size_t k_cols, size_t head_dim, float *out) {
    if (query == nullptr || key_t == nullptr || value == nullptr || out == nullptr || q_rows == 0 ||
        k_cols == 0 || head_dim == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (q_rows != 8 || k_cols != 8 || head_dim != 64) {
        return TE_STATUS_UNSUPPORTED;
    }
    return mma_twin(1, query, key_t, value, k_cols, 0, out);
}

extern "C" te_status te_hip_attention_stream_mma_f32(const float *query, const float *key_t,
                                                     const float *value, size_t q_rows, size_t k_cols,
                                                     size_t head_dim, float *out) {
    if (query == nullptr || key_t == nullptr || value == nullptr || out == nullptr || q_rows == 0 ||
        k_cols == 0 || head_dim == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (q_rows != 8 || (k_cols % 8) != 0 || head_dim != 64 || k_cols > 1024) {
        return TE_STATUS_UNSUPPORTED;
    }
    return mma_twin(1, query, key_t, value, k_cols, 0, out);
}

extern "C" te_status te_hip_attention_causal_mma_f32(const float *query, const float *key_t,
                                                     const float *value, size_t q_rows, size_t k_cols,
                                                     size_t head_dim, size_t q_base, float *out) {
    if (query == nullptr || key_t == nullptr || value == nullptr || out == nullptr || q_rows == 0 ||
        k_cols == 0 || head_dim == 0) {
        return TE_STATUS_INVALID_ARGUMENT;
    }
    if (q_rows != 8 || (k_cols % 8) != 0 || head_dim != 64 || q_base > k_cols || k_cols > 1024) {
        return TE_STATUS_UNSUPPORTED;
    }
    return mma_twin(2, query, key_t, value, k_cols, q_base, out);
}
