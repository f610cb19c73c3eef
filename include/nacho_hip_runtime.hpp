// nacho_hip_runtime.hpp — C++ helpers shared by nacho_hip.hpp and by the <k>_gpu.h headers
// that the HIP code generator (nacho_amd/codegen) writes: the per-thread stream the entry
// points run on, the check that turns an error code into an exception, and the byte copy
// between a generated tensor struct and its C descriptor (the two have the same fields in
// the same order).
#ifndef NACHO_HIP_RUNTIME_HPP
#define NACHO_HIP_RUNTIME_HPP

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "nacho_hip.h"

namespace nacho_hip {

namespace detail {
inline void *&stream_slot() {
    thread_local void *s = nullptr;
    return s;
}
}  // namespace detail

// The hipStream_t the entry points run on, per calling thread (default: null stream, the
// generated code's `stream = 0`).
inline void *stream() { return detail::stream_slot(); }
inline void set_stream(void *s) { detail::stream_slot() = s; }

namespace detail {

// A format instantiated at <int32_t, float> and its C descriptor are the same sequence of
// fields, so values convert by copying bytes.
template <typename C, typename F>
inline C to_c(const F &f) {
    static_assert(sizeof(C) == sizeof(F) && std::is_trivially_copyable<F>::value,
                  "format and C descriptor differ");
    C c;
    std::memcpy(&c, &f, sizeof(C));
    return c;
}

template <typename F, typename C>
inline F from_c(const C &c) {
    static_assert(sizeof(C) == sizeof(F) && std::is_trivially_copyable<F>::value,
                  "format and C descriptor differ");
    F f;
    std::memcpy(&f, &c, sizeof(F));
    return f;
}

inline void check(int rc, const char *kernel) {
    if (rc != NACHO_OK) {
        throw std::runtime_error(std::string(kernel) + ": " + nacho_error_string(rc));
    }
}

}  // namespace detail
}  // namespace nacho_hip

#endif  // NACHO_HIP_RUNTIME_HPP
