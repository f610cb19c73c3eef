// Implementation of the thin HIP runtime (see runtime.hpp) and the library-wide C entry
// points that are not kernels: nacho_free, error strings, version, kernel timing.
#include "runtime.hpp"

#include <atomic>
#include <cstdint>
#include <cstring>
#include <mutex>

namespace nacho {
namespace {

// Devices whose default memory pool has been told to keep freed memory cached.  Without it
// the pool returns memory to the driver at every synchronisation and each call pays for
// fresh mappings.
std::mutex g_pool_mutex;
uint64_t g_pool_ready_mask = 0;
int g_pool_supported[64];

int prepare_pool(int device, bool *supported) {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (device < 0 || device >= 64) {
        *supported = false;
        return NACHO_OK;
    }
    if (!(g_pool_ready_mask & (1ull << device))) {
        int has_pools = 0;
        NACHO_TRY_HIP(hipDeviceGetAttribute(&has_pools, hipDeviceAttributeMemoryPoolsSupported,
                                            device));
        if (has_pools) {
            hipMemPool_t pool;
            NACHO_TRY_HIP(hipDeviceGetDefaultMemPool(&pool, device));
            uint64_t keep = UINT64_MAX;
            NACHO_TRY_HIP(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
        }
        g_pool_supported[device] = has_pools;
        g_pool_ready_mask |= (1ull << device);
    }
    *supported = g_pool_supported[device] != 0;
    return NACHO_OK;
}

void *default_allocate(size_t bytes, hipStream_t stream) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    bool pools = false;
    if (prepare_pool(device, &pools) != NACHO_OK) return nullptr;
    void *ptr = nullptr;
    hipError_t err = pools ? hipMallocAsync(&ptr, bytes, stream) : hipMalloc(&ptr, bytes);
    if (err != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky-free error so later calls are unaffected
        return nullptr;
    }
    return ptr;
}

void default_release(void *ptr, hipStream_t stream) {
    if (!ptr) return;
    int device = 0;
    bool pools = false;
    if (hipGetDevice(&device) == hipSuccess && prepare_pool(device, &pools) == NACHO_OK && pools) {
        (void)hipFreeAsync(ptr, stream);
    } else {
        (void)hipStreamSynchronize(stream);
        (void)hipFree(ptr);
    }
}

// Kernel timing state (per host thread).
std::atomic<int> g_timing_enabled{0};
thread_local hipEvent_t t_ev_start = nullptr;
thread_local hipEvent_t t_ev_stop = nullptr;
thread_local bool t_timer_armed = false;
thread_local float t_last_ms = 0.0f;
thread_local const char *t_last_name = "";

// Pinned host word for length readbacks, one per host thread.
thread_local void *t_pinned = nullptr;

}  // namespace

Call::Call(void *stream, const nacho_allocator *alloc)
    : stream_(static_cast<hipStream_t>(stream)),
      alloc_(alloc && alloc->allocate ? alloc : nullptr),
      timing_(g_timing_enabled.load(std::memory_order_relaxed) != 0) {}

Call::~Call() {
    for (void *p : scratch_) release(p);
    if (!committed_) {
        for (void *p : results_) release(p);
    }
}

void *Call::allocate(size_t bytes) {
    if (alloc_) return alloc_->allocate(alloc_->ctx, bytes, stream_);
    return default_allocate(bytes, stream_);
}

void Call::release(void *ptr) {
    if (!ptr) return;
    if (alloc_) {
        if (alloc_->release) alloc_->release(alloc_->ctx, ptr, stream_);
        return;
    }
    default_release(ptr, stream_);
}

int Call::scratch(size_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0) return NACHO_OK;
    void *p = allocate(bytes);
    if (!p) return NACHO_ERR_OUT_OF_MEMORY;
    scratch_.push_back(p);
    *out = p;
    return NACHO_OK;
}

int Call::result(size_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0) return NACHO_OK;
    void *p = allocate(bytes);
    if (!p) return NACHO_ERR_OUT_OF_MEMORY;
    results_.push_back(p);
    *out = p;
    return NACHO_OK;
}

void Call::drop_result(void *ptr) {
    if (!ptr) return;
    for (size_t i = 0; i < results_.size(); ++i) {
        if (results_[i] == ptr) {
            release(ptr);
            results_.erase(results_.begin() + static_cast<std::ptrdiff_t>(i));
            return;
        }
    }
}

int Call::read_back(void *host, const void *device, size_t bytes) {
    if (bytes > 64) return NACHO_ERR_INVALID_ARGUMENT;
    if (!t_pinned) NACHO_TRY_HIP(hipHostMalloc(&t_pinned, 64, hipHostMallocDefault));
    NACHO_TRY_HIP(hipMemcpyAsync(t_pinned, device, bytes, hipMemcpyDeviceToHost, stream_));
    NACHO_TRY_HIP(hipStreamSynchronize(stream_));
    std::memcpy(host, t_pinned, bytes);
    if (t_timer_armed) {
        t_timer_armed = false;
        float ms = 0.0f;
        NACHO_TRY_HIP(hipEventElapsedTime(&ms, t_ev_start, t_ev_stop));
        t_last_ms = ms;
    }
    return NACHO_OK;
}

int Call::timer_start(const char *name) {
    if (!timing_) return NACHO_OK;
    if (!t_ev_start) NACHO_TRY_HIP(hipEventCreate(&t_ev_start));
    if (!t_ev_stop) NACHO_TRY_HIP(hipEventCreate(&t_ev_stop));
    t_last_name = name;
    NACHO_TRY_HIP(hipEventRecord(t_ev_start, stream_));
    return NACHO_OK;
}

int Call::timer_stop() {
    if (!timing_) return NACHO_OK;
    NACHO_TRY_HIP(hipEventRecord(t_ev_stop, stream_));
    t_timer_armed = true;
    return NACHO_OK;
}

}  // namespace nacho

extern "C" {

int nacho_free(void *ptr, void *stream) {
    nacho::default_release(ptr, static_cast<hipStream_t>(stream));
    return NACHO_OK;
}

const char *nacho_error_string(int code) {
    switch (code) {
        case NACHO_OK: return "success";
        case NACHO_ERR_INVALID_ARGUMENT: return "nacho: invalid argument";
        case NACHO_ERR_INDEX_OVERFLOW: return "nacho: index or work count exceeds int32";
        case NACHO_ERR_OUT_OF_MEMORY: return "nacho: device allocation failed";
        case NACHO_ERR_MALFORMED_INPUT: return "nacho: malformed sparse operand";
        case NACHO_ERR_NO_DEVICE: return "nacho: no HIP device";
        case NACHO_ERR_INTERNAL: return "nacho: internal error (kernel wait bound expired)";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "nacho: unknown error";
}

const char *nacho_version(void) { return "nacho-mi355x 0.1 (gfx950)"; }

void nacho_set_kernel_timing(int enable) {
    nacho::g_timing_enabled.store(enable ? 1 : 0, std::memory_order_relaxed);
}

float nacho_last_kernel_ms(void) { return nacho::t_last_ms; }

const char *nacho_last_kernel_name(void) { return nacho::t_last_name; }

}  // extern "C"
