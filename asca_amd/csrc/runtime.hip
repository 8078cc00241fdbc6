// Device runtime of libasca_hip: initialisation, a size-class device memory
// pool, copies, traffic counters, error reporting and launch fault injection.
//
// It replaces the CUDA driver FFI of the reference crate
// (rust/src/cuda/sys.rs:33-65) and the DevBuf pool / counters of
// rust/src/cuda/mod.rs:25-33,100-174 with one C ABI over HIP.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "runtime.h"

namespace asca {

static std::mutex g_mu;
static thread_local std::string t_err;
static int g_device = -1;
static int g_cus = 0;
static char g_name[256] = {0};
static thread_local int t_device_set = -1;

static std::atomic<uint64_t> g_h2d{0}, g_d2h{0}, g_launches{0};
static std::atomic<int64_t> g_fail_after{-1};

// Size-class pool (rust/src/cuda/mod.rs:100-174): sizes are rounded up to a
// power of two and freed blocks are kept for reuse instead of returned to HIP.
static std::unordered_map<size_t, std::vector<void*>> g_pool;
static std::unordered_map<void*, size_t> g_live;

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

int cu_count() { return g_cus; }

int ensure_device() {
    if (g_device < 0) return fail(ASCA_ERR_NOT_INIT, "asca_init has not been called");
    if (t_device_set != g_device) {
        hipError_t e = hipSetDevice(g_device);
        if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipSetDevice(%d): %s", g_device, hipGetErrorString(e));
        t_device_set = g_device;
    }
    return ASCA_OK;
}

int pre_launch(const char* kernel) {
    int rc = ensure_device();
    if (rc) return rc;
    int64_t f = g_fail_after.load();
    if (f >= 0) {
        if (f == 0) {
            g_fail_after.store(-1);
            return fail(ASCA_ERR_INJECTED, "injected launch failure at %s", kernel);
        }
        g_fail_after.store(f - 1);
    }
    g_launches.fetch_add(1);
    return ASCA_OK;
}

static std::mutex g_attr_mu;
static std::unordered_map<const void*, std::vector<size_t>> g_attr;  // per kernel: bytes set, by device

int allow_lds(const void* fn, size_t bytes) {
    int rc = ensure_device();
    if (rc) return rc;
    const int dev = g_device;
    std::lock_guard<std::mutex> lk(g_attr_mu);
    std::vector<size_t>& set = g_attr[fn];
    if ((int)set.size() <= dev) set.resize(dev + 1, 0);
    if (set[dev] >= bytes) return ASCA_OK;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess)
        return fail(ASCA_ERR_HIP, "hipFuncSetAttribute(LDS %zu) on device %d: %s", bytes, dev, hipGetErrorString(e));
    set[dev] = bytes;
    return ASCA_OK;
}

// The stream-ordered pool behind StreamScratch: the library's own (created at
// asca_init), so that its release threshold (keep what is freed for reuse
// instead of returning it to the driver at every synchronisation) does not
// change the device's default pool that other code in the process may use.
static hipMemPool_t g_scratch_pool = nullptr;

// One cached buffer per stream (a stream-ordered allocation and free per call
// costs several microseconds of stream time).
struct ScratchEntry {
    float* p = nullptr;
    size_t floats = 0;
};
static std::mutex g_scratch_mu;
static std::unordered_map<hipStream_t, ScratchEntry> g_scratch;

int StreamScratch::get(size_t floats, hipStream_t st) {
    ws = Ws{nullptr, 0};
    if (floats == 0) return ASCA_OK;
    if (!g_scratch_pool) return fail(ASCA_ERR_NOT_INIT, "asca_init has not been called");
    g_scratch_mu.lock();
    held_ = true;
    ScratchEntry& en = g_scratch[st];
    if (en.floats < floats) {
        if (en.p) (void)hipFreeAsync(en.p, st);   // behind the queued work that still uses it
        en = ScratchEntry{};
        const size_t want = floats + floats / 4;  // headroom for slightly larger calls
        void* p = nullptr;
        hipError_t e = hipMallocFromPoolAsync(&p, want * sizeof(float), g_scratch_pool, st);
        if (e != hipSuccess) {
            held_ = false;
            g_scratch_mu.unlock();
            return fail(ASCA_ERR_OOM, "hipMallocFromPoolAsync(%zu): %s", want * sizeof(float), hipGetErrorString(e));
        }
        en = ScratchEntry{reinterpret_cast<float*>(p), want};
    }
    ws = Ws{en.p, floats};
    return ASCA_OK;
}

int StreamScratch::release(hipStream_t) {
    ws = Ws{nullptr, 0};
    if (held_) {
        held_ = false;
        g_scratch_mu.unlock();
    }
    return ASCA_OK;
}

StreamScratch::~StreamScratch() { (void)release(nullptr); }

void stream_scratch_forget(hipStream_t st) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch.find(st);
    if (it == g_scratch.end()) return;
    if (it->second.p) (void)hipFreeAsync(it->second.p, st);
    g_scratch.erase(it);
}

int post_launch(const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "launch of %s failed: %s", kernel, hipGetErrorString(e));
    return ASCA_OK;
}

}  // namespace asca

using namespace asca;

extern "C" {

const char* asca_last_error(void) { return t_err.c_str(); }

int asca_device_count(int* n) {
    if (!n) return fail(ASCA_ERR_INVALID, "null output pointer");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) { *n = 0; return fail(ASCA_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e)); }
    *n = c;
    return ASCA_OK;
}

int asca_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (const char* f = getenv("ASCA_FAIL_LAUNCH")) g_fail_after.store(atoll(f));
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(ASCA_ERR_NO_DEVICE, "no HIP device (%s)", e == hipSuccess ? "count 0" : hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(ASCA_ERR_INVALID, "device %d out of range [0,%d)", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(ASCA_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only", device,
                    prop.gcnArchName);
    if (!g_scratch_pool || g_device != device) {
        hipMemPoolProps props;
        memset(&props, 0, sizeof props);
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = device;
        hipMemPool_t pool = nullptr;
        e = hipMemPoolCreate(&pool, &props);
        if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipMemPoolCreate: %s", hipGetErrorString(e));
        uint64_t keep = UINT64_MAX;
        e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) {
            (void)hipMemPoolDestroy(pool);
            return fail(ASCA_ERR_HIP, "hipMemPoolSetAttribute: %s", hipGetErrorString(e));
        }
        g_scratch_pool = pool;   // a pool of an earlier device stays until the process ends
    }
    if (int rc = noalloc_scratch_init(device)) return rc;
    g_device = device;
    g_cus = prop.multiProcessorCount;
    snprintf(g_name, sizeof g_name, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, g_cus);
    t_device_set = device;
    return ASCA_OK;
}

int asca_describe(char* buf, int len) {
    if (!buf || len <= 0) return fail(ASCA_ERR_INVALID, "bad buffer");
    if (g_device < 0) return fail(ASCA_ERR_NOT_INIT, "asca_init has not been called");
    snprintf(buf, (size_t)len, "%s", g_name);
    return ASCA_OK;
}

int asca_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(ASCA_ERR_INVALID, "null output pointer");
    *ptr = nullptr;
    int rc = ensure_device();
    if (rc) return rc;
    size_t sz = 4;
    while (sz < bytes) sz <<= 1;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_pool.find(sz);
    if (it != g_pool.end() && !it->second.empty()) {
        *ptr = it->second.back();
        it->second.pop_back();
        g_live[*ptr] = sz;
        return ASCA_OK;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ASCA_ERR_OOM, "hipMalloc(%zu): %s", sz, hipGetErrorString(e));
    }
    g_live[p] = sz;
    *ptr = p;
    return ASCA_OK;
}

int asca_free(void* ptr) {
    if (!ptr) return ASCA_OK;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) return fail(ASCA_ERR_INVALID, "asca_free: %p was not allocated by asca_alloc", ptr);
    g_pool[it->second].push_back(ptr);
    g_live.erase(it);
    return ASCA_OK;
}

int asca_pool_release(void) {
    int rc = ensure_device();
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    hipDeviceSynchronize();
    for (auto& kv : g_pool)
        for (void* p : kv.second) hipFree(p);
    g_pool.clear();
    {
        std::lock_guard<std::mutex> lk2(g_scratch_mu);   // the streams' cached scratch too (the device is idle)
        for (auto& kv : g_scratch)
            if (kv.second.p) (void)hipFreeAsync(kv.second.p, kv.first);
        g_scratch.clear();
    }
    hipDeviceSynchronize();
    if (g_scratch_pool) (void)hipMemPoolTrimTo(g_scratch_pool, 0);
    return ASCA_OK;
}

int asca_h2d(void* dst, const void* src, size_t bytes) {
    int rc = ensure_device();
    if (rc) return rc;
    if (bytes == 0) return ASCA_OK;
    if (!dst || !src) return fail(ASCA_ERR_INVALID, "null pointer in asca_h2d");
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipMemcpy H2D: %s", hipGetErrorString(e));
    g_h2d.fetch_add(bytes);
    return ASCA_OK;
}

int asca_d2h(void* dst, const void* src, size_t bytes) {
    int rc = ensure_device();
    if (rc) return rc;
    if (bytes == 0) return ASCA_OK;
    if (!dst || !src) return fail(ASCA_ERR_INVALID, "null pointer in asca_d2h");
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipMemcpy D2H: %s", hipGetErrorString(e));
    g_d2h.fetch_add(bytes);
    return ASCA_OK;
}

int asca_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (bytes == 0) return ASCA_OK;
    if (!dst || !src) return fail(ASCA_ERR_INVALID, "null pointer in asca_d2d");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipMemcpyAsync D2D: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_memset32(void* dst, uint32_t value, size_t count, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (count == 0) return ASCA_OK;
    if (!dst) return fail(ASCA_ERR_INVALID, "null pointer in asca_memset32");
    hipError_t e = hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(dst), (int)value, count, as_stream(stream));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipMemsetD32Async: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_sync(void) {
    int rc = ensure_device();
    if (rc) return rc;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipDeviceSynchronize: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_stream_sync(void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(as_stream(stream));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_stats(uint64_t* h2d, uint64_t* d2h, uint64_t* launches) {
    if (h2d) *h2d = g_h2d.load();
    if (d2h) *d2h = g_d2h.load();
    if (launches) *launches = g_launches.load();
    return ASCA_OK;
}

int asca_reset_stats(void) {
    g_h2d.store(0);
    g_d2h.store(0);
    g_launches.store(0);
    return ASCA_OK;
}

int asca_fail_after(int64_t n) {
    g_fail_after.store(n < 0 ? -1 : n);
    return ASCA_OK;
}

}  // extern "C"

// ------------------------------------------------------------ streams/events
extern "C" {

int asca_stream_create(void** stream) {
    if (!stream) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = ensure_device();
    if (rc) return rc;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
    *stream = s;
    return ASCA_OK;
}

int asca_stream_destroy(void* stream) {
    if (!stream) return ASCA_OK;
    stream_scratch_forget(as_stream(stream));
    hipError_t e = hipStreamDestroy(as_stream(stream));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipStreamDestroy: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_event_create(void** ev) {
    if (!ev) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = ensure_device();
    if (rc) return rc;
    hipEvent_t e0 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    *ev = e0;
    return ASCA_OK;
}

int asca_event_destroy(void* ev) {
    if (!ev) return ASCA_OK;
    hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(ev));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventDestroy: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_event_record(void* ev, void* stream) {
    hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(ev), as_stream(stream));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord: %s", hipGetErrorString(e));
    return ASCA_OK;
}

int asca_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms) return fail(ASCA_ERR_INVALID, "null output pointer");
    hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventSynchronize: %s", hipGetErrorString(e));
    e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop));
    if (e != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventElapsedTime: %s", hipGetErrorString(e));
    return ASCA_OK;
}

// ------------------------------------------------------------------- rng
// Input generator of the reference, rust/src/tensor.rs:299-337: xorshift128+
// with Box-Muller normals in f32.  state[2] = {s0, s1}; calls continue the stream.

void asca_rng_seed(uint64_t seed, uint64_t* state) {
    state[0] = (seed * 0x9E3779B97F4A7C15ULL) | 1ULL;
    state[1] = ((seed ^ 0xDEADBEEFCAFEF00DULL) * 0xBF58476D1CE4E5B9ULL) | 1ULL;
}

static inline uint64_t rng_next(uint64_t* st) {
    uint64_t x = st[0];
    const uint64_t y = st[1];
    st[0] = y;
    x ^= x << 23;
    st[1] = x ^ y ^ (x >> 17) ^ (y >> 26);
    return st[1] + y;
}

static inline float rng_uniform(uint64_t* st) { return (float)(rng_next(st) >> 40) / (float)(1u << 24); }

void asca_rng_u64(uint64_t* state, uint64_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = rng_next(state);
}

// out[i] = offset + scale * normal()
void asca_rng_normal(uint64_t* state, float* out, size_t n, float scale, float offset) {
    const float two_pi = 2.0f * 3.14159265358979323846f;
    for (size_t i = 0; i < n; ++i) {
        float u1 = rng_uniform(state);
        if (!(u1 >= 1e-7f)) u1 = 1e-7f;
        const float u2 = rng_uniform(state);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(two_pi * u2);
        out[i] = offset + z * scale;
    }
}

}  // extern "C"
