// Implementation of the thin HIP runtime (see runtime.hpp) and the library-wide C entry
// points that are not kernels: nacho_free, error strings, version, kernel timing.
#include "runtime.hpp"

#include <atomic>
#include <chrono>
#include <climits>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace nacho {
namespace {

// ---- caching device allocator --------------------------------------------------------
// Result and scratch buffers are recycled instead of going back to the driver: every call
// of an entry point allocates a handful of buffers, and driver allocation (or the
// stream-ordered pool) costs tens of microseconds each.  Blocks are binned by size class
// (powers of two split into 4 sub-classes, minimum 512 B).
//
// Ordering.  A block freed on stream S is reused only by later allocations on S, which
// stream order puts after every use of the block on S; an allocation on another stream
// takes a fresh block.  Work on other streams that used the block is announced with
// nacho_record_stream: the release then records an event on each such stream, and the
// allocation that takes the block makes S wait for those events (hipStreamWaitEvent,
// outside the cache lock).  The host never blocks on a stream for reuse, and the common case
// (one stream) records no event at all.  When the driver runs out of memory the cache is
// emptied (after a device synchronise) and the allocation retried.
//
// Size.  By default every released block stays cached (a C4 SpGEMM leaves about 100 GB
// there, which other allocators in the process cannot use until nacho_release_cached_memory).
// nacho_set_cache_limit caps the cached bytes: a release that takes them past the cap
// synchronises the device and returns the oldest blocks of the largest size classes to the
// driver until they fit.

// A pooled event, possibly shared by several blocks.
struct SharedEvent {
    hipEvent_t event;
    hipStream_t stream;  // where it was recorded
    int refs;
};

struct Block {
    void *ptr;
    size_t size;  // rounded size class
    int device;
    hipStream_t stream;                  // the stream that allocated / released it
    std::vector<hipStream_t> used_on;    // other streams named by nacho_record_stream
    std::vector<SharedEvent *> pending;  // their events, waited for at reuse (free blocks)
};

std::mutex g_cache_mutex;
std::unordered_map<void *, Block> g_live;              // allocated blocks by pointer
std::map<std::pair<int, size_t>, std::vector<Block>> g_free;  // (device, size) -> free
std::vector<hipEvent_t> g_event_pool;  // idle events (created with timing disabled)
size_t g_free_bytes = 0;               // bytes in g_free
std::atomic<size_t> g_cache_limit{SIZE_MAX};

// An idle event, or a new one (nullptr if creation fails).  Caller holds g_cache_mutex.
hipEvent_t take_event_locked() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

// Event recorded on `stream` now, shared with refcount `refs` (nullptr if recording fails:
// the caller then falls back to host synchronisation).  Caller holds g_cache_mutex.
SharedEvent *record_shared_locked(hipStream_t stream, int refs) {
    hipEvent_t e = take_event_locked();
    if (!e) return nullptr;
    if (hipEventRecord(e, stream) != hipSuccess) {
        (void)hipGetLastError();
        g_event_pool.push_back(e);
        return nullptr;
    }
    return new SharedEvent{e, stream, refs};
}

void drop_shared_locked(SharedEvent *s) {
    if (--s->refs == 0) {
        g_event_pool.push_back(s->event);
        delete s;
    }
}

size_t size_class(size_t bytes) {
    if (bytes <= 512) return 512;
    size_t p = 1;
    while (p < bytes) p <<= 1;
    const size_t quarter = p >> 3;  // p/2 .. p in 4 steps of p/8
    size_t c = p >> 1;
    while (c < bytes) c += quarter;
    return c;
}

void release_cached_blocks_locked() {
    (void)hipDeviceSynchronize();
    for (auto &bin : g_free) {
        for (Block &b : bin.second) {
            for (SharedEvent *e : b.pending) drop_shared_locked(e);
            (void)hipFree(b.ptr);
        }
    }
    g_free.clear();
    g_free_bytes = 0;
    for (hipEvent_t e : g_event_pool) (void)hipEventDestroy(e);
    g_event_pool.clear();
}

// Return cached blocks to the driver until at most `limit` bytes stay cached: the largest
// size classes first, the oldest block of a class first.  The device is synchronised first
// (a cached block's last use may still be queued).  Caller holds g_cache_mutex.
void trim_cache_locked(size_t limit) {
    if (g_free_bytes <= limit) return;
    (void)hipDeviceSynchronize();
    for (auto it = g_free.rbegin(); it != g_free.rend() && g_free_bytes > limit; ++it) {
        std::vector<Block> &bin = it->second;
        size_t drop = 0;
        while (drop < bin.size() && g_free_bytes > limit) {
            Block &b = bin[drop++];
            for (SharedEvent *e : b.pending) drop_shared_locked(e);
            b.pending.clear();
            (void)hipFree(b.ptr);
            g_free_bytes -= b.size;
        }
        bin.erase(bin.begin(), bin.begin() + static_cast<std::ptrdiff_t>(drop));
    }
}

// Make `stream` wait for the events a reused block carries (outside the cache lock), then
// return the events.  If the runtime refuses a device-side wait, the host waits for the
// event instead.
void wait_pending(std::vector<SharedEvent *> &pending, hipStream_t stream) {
    for (SharedEvent *e : pending) {
        if (e->stream == stream) continue;
        if (hipStreamWaitEvent(stream, e->event, 0) != hipSuccess) {
            (void)hipGetLastError();
            if (hipEventSynchronize(e->event) != hipSuccess) {
                (void)hipGetLastError();
                (void)hipDeviceSynchronize();
            }
        }
    }
    if (pending.empty()) return;
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    for (SharedEvent *e : pending) drop_shared_locked(e);
    pending.clear();
}

void *default_allocate(size_t bytes, hipStream_t stream) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    const size_t size = size_class(bytes);
    std::vector<SharedEvent *> pending;
    void *reused = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_cache_mutex);
        auto it = g_free.find({device, size});
        if (it != g_free.end()) {
            std::vector<Block> &bin = it->second;
            for (size_t i = bin.size(); i-- > 0;) {  // most recently freed first
                if (bin[i].stream != stream) continue;
                Block b = std::move(bin[i]);
                bin.erase(bin.begin() + static_cast<std::ptrdiff_t>(i));
                g_free_bytes -= b.size;
                pending.swap(b.pending);
                b.used_on.clear();
                reused = b.ptr;
                g_live[b.ptr] = std::move(b);
                break;
            }
        }
    }
    if (reused) {
        wait_pending(pending, stream);
        return reused;
    }
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    void *ptr = nullptr;
    hipError_t err = hipMalloc(&ptr, size);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        release_cached_blocks_locked();
        err = hipMalloc(&ptr, size);
        if (err != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    g_live[ptr] = Block{ptr, size, device, stream, {}, {}};
    return ptr;
}

// Return blocks to the cache of `stream` (the stream their last use is ordered on; a
// block released on another stream than the one that allocated it moves to that stream's
// cache).  For every other stream named by nacho_record_stream an event is recorded now; if
// one cannot be recorded, the host synchronises that stream instead (rare fallback).
// Pointers the cache does not own are ignored.
void release_batch(void *const *ptrs, size_t n, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    for (size_t i = 0; i < n; ++i) {
        if (!ptrs[i]) continue;
        auto it = g_live.find(ptrs[i]);
        if (it == g_live.end()) continue;
        Block b = std::move(it->second);
        g_live.erase(it);
        if (b.stream != stream) b.used_on.push_back(b.stream);
        b.stream = stream;
        for (hipStream_t u : b.used_on) {
            if (u == stream) continue;
            SharedEvent *e = record_shared_locked(u, 1);
            if (e) {
                b.pending.push_back(e);
            } else {
                (void)hipStreamSynchronize(u);
            }
        }
        b.used_on.clear();
        g_free_bytes += b.size;
        g_free[{b.device, b.size}].push_back(std::move(b));
    }
    trim_cache_locked(g_cache_limit.load(std::memory_order_relaxed));
}

void default_release(void *ptr, hipStream_t stream) { release_batch(&ptr, 1, stream); }

// Note that `stream` also uses a live block (the block's own stream is implied).
int record_stream(void *ptr, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) return NACHO_ERR_INVALID_ARGUMENT;
    Block &b = it->second;
    if (stream == b.stream) return NACHO_OK;
    for (hipStream_t u : b.used_on) {
        if (u == stream) return NACHO_OK;
    }
    b.used_on.push_back(stream);
    return NACHO_OK;
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

// Coherent pinned words that kernels store a length and a side count into (early readback)
// and their device address; one pair per host thread.
thread_local volatile int64_t *t_len_host = nullptr;
thread_local int64_t *t_len_dev = nullptr;

}  // namespace

Call::Call(void *stream, const nacho_allocator *alloc)
    : stream_(static_cast<hipStream_t>(stream)),
      alloc_(alloc && alloc->allocate ? alloc : nullptr),
      timing_(g_timing_enabled.load(std::memory_order_relaxed) != 0) {}

Call::Call(void *stream, void *arena, size_t arena_bytes)
    : stream_(static_cast<hipStream_t>(stream)),
      alloc_(nullptr),
      timing_(false),
      arena_(static_cast<unsigned char *>(arena)),
      arena_size_(arena_bytes) {}

Call::~Call() {
    if (arena_) return;  // nothing was allocated
    if (timed_) t_last_ms = timed_ms_;
    if (!committed_) scratch_.insert(scratch_.end(), results_.begin(), results_.end());
    if (alloc_) {
        for (void *p : scratch_) release(p);
    } else if (!scratch_.empty()) {
        release_batch(scratch_.data(), scratch_.size(), stream_);
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
    if (arena_) {
        const size_t at = (arena_used_ + 255) & ~static_cast<size_t>(255);
        if (at > arena_size_ || bytes > arena_size_ - at) return NACHO_ERR_SCRATCH_TOO_SMALL;
        arena_used_ = at + bytes;
        *out = arena_ + at;
        return NACHO_OK;
    }
    void *p = allocate(bytes);
    if (!p) return NACHO_ERR_OUT_OF_MEMORY;
    scratch_.push_back(p);
    *out = p;
    return NACHO_OK;
}

int Call::result(size_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0) return NACHO_OK;
    if (arena_) return NACHO_ERR_INVALID_ARGUMENT;  // the caller passes result buffers
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
    if (arena_) {  // no pinned staging word: copy straight into the caller's variable
        NACHO_TRY_HIP(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, stream_));
        NACHO_TRY_HIP(hipStreamSynchronize(stream_));
        return NACHO_OK;
    }
    if (!t_pinned) NACHO_TRY_HIP(hipHostMalloc(&t_pinned, 64, hipHostMallocDefault));
    NACHO_TRY_HIP(hipMemcpyAsync(t_pinned, device, bytes, hipMemcpyDeviceToHost, stream_));
    NACHO_TRY_HIP(hipStreamSynchronize(stream_));
    std::memcpy(host, t_pinned, bytes);
    return collect_timer();
}

namespace {
int ensure_len_words() {
    if (!t_len_host) {
        void *h = nullptr;
        NACHO_TRY_HIP(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent |
                                                hipHostMallocPortable));
        void *d = nullptr;
        const hipError_t e = hipHostGetDevicePointer(&d, h, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(h);
            return static_cast<int>(e);
        }
        t_len_host = static_cast<volatile int64_t *>(h);
        t_len_dev = static_cast<int64_t *>(d);
    }
    return NACHO_OK;
}
}  // namespace

int Call::length_word(int64_t **dev) {
    if (arena_) {  // the kernel that totals the length stores it in the arena
        NACHO_TRY(scratch_n(1, &arena_len_));
        *dev = arena_len_;
        return NACHO_OK;
    }
    NACHO_TRY(ensure_len_words());
    *t_len_host = -1;  // a kernel that did not store would show as an impossible length
    *dev = t_len_dev;
    return NACHO_OK;
}

int Call::side_word(int64_t **dev) {
    if (arena_) {
        NACHO_TRY(scratch_n(1, &arena_side_));
        *dev = arena_side_;
        return NACHO_OK;
    }
    NACHO_TRY(ensure_len_words());
    t_len_host[1] = -1;
    *dev = t_len_dev + 1;
    return NACHO_OK;
}

namespace {
// Waits until the device has stored a value >= 0 into the pinned word `w` (set to -1 before
// the launch; kernels store it with a system-scope release).  Nothing is enqueued on the
// stream for the wait: an event recorded after the kernel that stores the word, or a
// stream query while the pipeline runs, each held the next dispatch back by about 6 us on
// MI355X.  Only after kStreamCheckAfter of waiting is the stream checked now and then, so
// that a stream that failed, or that finished without storing the word, ends the wait.
constexpr auto kStreamCheckAfter = std::chrono::milliseconds(20);

int spin_for_word(volatile int64_t *w, hipStream_t stream, int64_t *out) {
    const auto begin = std::chrono::steady_clock::now();
    bool check = false;
    for (unsigned i = 1;; ++i) {
        const int64_t v = *w;
        if (v >= 0) {
            std::atomic_thread_fence(std::memory_order_acquire);
            *out = v;
            return NACHO_OK;
        }
        if ((i & 4095u) != 0) continue;
        if (!check) {
            check = std::chrono::steady_clock::now() - begin >= kStreamCheckAfter;
        } else {
            const hipError_t e = hipStreamQuery(stream);
            if (e == hipSuccess) {  // every kernel of the stream ended: the word is final
                const int64_t last = *w;
                if (last < 0) return NACHO_ERR_INTERNAL;
                *out = last;
                return NACHO_OK;
            }
            if (e != hipErrorNotReady) return static_cast<int>(e);
        }
    }
}
}  // namespace

int Call::side_value(int64_t *v) {
    if (arena_) {
        if (!arena_side_) return NACHO_ERR_INTERNAL;
        NACHO_TRY(read_back(v, arena_side_, sizeof(*v)));
    } else {
        // The side word is stored (system scope) by a kernel of this call before the one
        // that stores the length; it is waited for in the same way.
        if (!len_marked_) return NACHO_ERR_INTERNAL;
        NACHO_TRY(spin_for_word(t_len_host + 1, stream_, v));
    }
    return *v < 0 ? NACHO_ERR_INTERNAL : NACHO_OK;
}

int Call::mark_length() {
    len_marked_ = true;  // wait_length spins on the pinned word (or synchronises, arena)
    return NACHO_OK;
}

int Call::wait_length(int64_t *len) {
    if (arena_) {
        if (!arena_len_) return NACHO_ERR_INTERNAL;
        int64_t v = -1;
        NACHO_TRY(read_back(&v, arena_len_, sizeof(v)));
        if (v < 0) return NACHO_ERR_INTERNAL;
        *len = v;
        return NACHO_OK;
    }
    if (!len_marked_) return NACHO_ERR_INTERNAL;
    NACHO_TRY(spin_for_word(t_len_host, stream_, len));
    return collect_timer();
}

int Call::collect_timer() {
    if (!t_timer_armed) return NACHO_OK;
    t_timer_armed = false;
    NACHO_TRY_HIP(hipEventSynchronize(t_ev_stop));
    float ms = 0.0f;
    NACHO_TRY_HIP(hipEventElapsedTime(&ms, t_ev_start, t_ev_stop));
    timed_ms_ += ms;
    timed_ = true;
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

int resident_grid(const void *kernel, int block, int *grid) {
    static std::mutex mutex;
    static std::map<std::pair<const void *, int>, int> cache;
    int device = 0;
    NACHO_TRY_HIP(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(mutex);
    auto it = cache.find({kernel, device});
    if (it != cache.end()) {
        *grid = it->second;
        return NACHO_OK;
    }
    int per_cu = 0, cus = 0;
    NACHO_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0));
    NACHO_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    const int g = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    cache[{kernel, device}] = g;
    *grid = g;
    return NACHO_OK;
}

}  // namespace nacho

extern "C" {

int nacho_free(void *ptr, void *stream) {
    nacho::default_release(ptr, static_cast<hipStream_t>(stream));
    return NACHO_OK;
}

int nacho_record_stream(void *ptr, void *stream) {
    if (!ptr) return NACHO_ERR_INVALID_ARGUMENT;
    return nacho::record_stream(ptr, static_cast<hipStream_t>(stream));
}

int nacho_release_cached_memory(void) {
    std::lock_guard<std::mutex> lock(nacho::g_cache_mutex);
    nacho::release_cached_blocks_locked();
    return NACHO_OK;
}

int nacho_set_cache_limit(size_t bytes) {
    std::lock_guard<std::mutex> lock(nacho::g_cache_mutex);
    nacho::g_cache_limit.store(bytes, std::memory_order_relaxed);
    nacho::trim_cache_locked(bytes);
    return NACHO_OK;
}

size_t nacho_cached_bytes(void) {
    std::lock_guard<std::mutex> lock(nacho::g_cache_mutex);
    return nacho::g_free_bytes;
}

const char *nacho_error_string(int code) {
    switch (code) {
        case NACHO_OK: return "success";
        case NACHO_ERR_INVALID_ARGUMENT: return "nacho: invalid argument";
        case NACHO_ERR_INDEX_OVERFLOW: return "nacho: index or work count exceeds int32";
        case NACHO_ERR_OUT_OF_MEMORY: return "nacho: device allocation failed";
        case NACHO_ERR_MALFORMED_INPUT: return "nacho: malformed sparse operand";
        case NACHO_ERR_NO_DEVICE: return "nacho: no HIP device";
        case NACHO_ERR_INTERNAL: return "nacho: internal error (a kernel did not publish its result length)";
        case NACHO_ERR_IO: return "nacho: file could not be opened or read";
        case NACHO_ERR_UNSUPPORTED: return "nacho: unsupported file format variant";
        case NACHO_ERR_SCRATCH_TOO_SMALL:
            return "nacho: input too large for the allocation-free entry point's static scratch";
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
