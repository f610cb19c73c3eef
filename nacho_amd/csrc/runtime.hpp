// Thin HIP runtime shared by every entry point of the gfx950 backend: error plumbing,
// stream-ordered allocation through the caller's allocator (or the library's caching
// allocator over hipMalloc, with event-ordered reuse across streams), scratch that is
// released on every exit path, the pinned host word used to read result lengths back, and
// the optional kernel timing hook.
//
// It stands where the reference's generated entry points use cudaMallocAsync /
// cudaFreeAsync / cudaMemsetAsync / cudaMemcpyAsync on stream 0
// (src/backend/stitch_and_generate_gpu.cpp:187-196, 368-377, 663-671, 742-763) and
// runtime/cuda_utils (cudaFreeWrapper, CHECK_CUDA).  Unlike the generated code, every HIP
// call is checked and the length readback is explicitly synchronised.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/nacho_hip.h"

namespace nacho {

// Return the first failing HIP call's code from the enclosing int-returning function.
#define NACHO_TRY_HIP(expr)                                                                  \
    do {                                                                                     \
        hipError_t nacho_err_ = (expr);                                                      \
        if (nacho_err_ != hipSuccess) return static_cast<int>(nacho_err_);                   \
    } while (0)

#define NACHO_TRY(expr)                                                                      \
    do {                                                                                     \
        int nacho_rc_ = (expr);                                                              \
        if (nacho_rc_ != NACHO_OK) return nacho_rc_;                                         \
    } while (0)

// One call's execution context: its stream and allocator, and every buffer it allocated.
// Scratch buffers are released when the call ends; result buffers are released only if the
// call fails (commit() hands them to the caller).
class Call {
  public:
    Call(void *stream, const nacho_allocator *alloc);
    // Arena mode, for the allocation-free entry points: scratch is carved from the device
    // region [arena, arena + arena_bytes) (256-byte aligned pieces), results cannot be
    // allocated, the length word lives in the region and is read back with a copy and a
    // stream synchronise, and kernel timing is off.  Nothing is allocated or released.
    Call(void *stream, void *arena, size_t arena_bytes);
    ~Call();
    Call(const Call &) = delete;
    Call &operator=(const Call &) = delete;

    hipStream_t stream() const { return stream_; }

    // Device buffer of `bytes` (NULL when bytes == 0).  Returns NACHO_ERR_OUT_OF_MEMORY or
    // a HIP error code on failure.
    int scratch(size_t bytes, void **out);
    int result(size_t bytes, void **out);

    template <typename T>
    int scratch_n(size_t count, T **out) {
        return scratch(count * sizeof(T), reinterpret_cast<void **>(out));
    }
    template <typename T>
    int result_n(size_t count, T **out) {
        return result(count * sizeof(T), reinterpret_cast<void **>(out));
    }

    // Release one result buffer early (e.g. an over-allocated array that turned out empty).
    void drop_result(void *ptr);

    // The call succeeded: result buffers now belong to the caller.
    void commit() { committed_ = true; }

    // Copy `bytes` from device to a host variable and wait for the stream.
    int read_back(void *host, const void *device, size_t bytes);

    // Early length readback.  A kernel stores a result length (system scope) straight into
    // this host thread's pinned, device-visible word (`*dev` receives its device address;
    // the word reads -1 until then); the host marks that the kernel is launched
    // (mark_length), keeps launching the rest of the pipeline, and wait_length waits only
    // for the word, so the call returns while the remaining kernels still run,
    // stream-ordered, like the reference's generated entry point, which returns after
    // launching its write pass.
    int length_word(int64_t **dev);
    int mark_length();
    int wait_length(int64_t *len);
    // A second word beside the length, for a count whose kernel runs before the one that
    // stores the length: side_value waits for it in the same way, after mark_length;
    // without mark_length it returns NACHO_ERR_INTERNAL.
    int side_word(int64_t **dev);
    int side_value(int64_t *v);

    // Kernel timing hook (see nacho_set_kernel_timing): intervals between timer_start and
    // timer_stop are summed over the call and reported when the call ends.  An interval is
    // collected at the next read_back (which synchronises the stream).
    int timer_start(const char *name);
    int timer_stop();
    // Wait for the stopped interval (if any) and add it to the call's total, for calls whose
    // last step is not a read_back.
    int collect_timer();

  private:
    void *allocate(size_t bytes);
    void release(void *ptr);

    hipStream_t stream_;
    const nacho_allocator *alloc_;
    std::vector<void *> scratch_;
    std::vector<void *> results_;
    bool committed_ = false;
    bool timing_ = false;
    unsigned char *arena_ = nullptr;  // arena mode when non-null
    size_t arena_size_ = 0;
    size_t arena_used_ = 0;
    int64_t *arena_len_ = nullptr;
    int64_t *arena_side_ = nullptr;
    bool timed_ = false;
    bool len_marked_ = false;  // mark_length: this call launched the kernel storing its length
    float timed_ms_ = 0.0f;  // sum of this call's bracketed intervals
};

// Validate launch-geometry hints the reference passes (generate_bindings.cpp:292-325).
inline int check_launch_hints(int32_t num_blocks, int32_t threads_per_block) {
    return (num_blocks > 0 && threads_per_block > 0) ? NACHO_OK : NACHO_ERR_INVALID_ARGUMENT;
}

inline unsigned ceil_div(size_t a, size_t b) { return static_cast<unsigned>((a + b - 1) / b); }

// Number of workgroups of `kernel` (block size `block`, static LDS only) that the current
// device holds resident at once: the grid of a persistent kernel.  Cached per kernel/device.
int resident_grid(const void *kernel, int block, int *grid);

}  // namespace nacho
