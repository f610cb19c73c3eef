// The device-copy bandwidth reference of the roofline measurement: a hand-written copy in
// 16-byte granules.
//
// A grid-stride loop over 16-byte granules, consecutive lanes on consecutive granules, with
// non-temporal loads and stores (streamed data, not kept in the caches) and a large grid
// (kBlocksPerCu workgroups per compute unit, spread by the dispatcher over every XCD), so
// that many waves keep coalesced reads in flight.  Measured on MI355X against variants of
// 1-8 granules per lane per pass, 8-512 workgroups per CU and cached accesses, this shape
// moved 1 GiB in + 1 GiB out fastest (5.5-5.7 TB/s, where torch's copy_ reached 4.8 TB/s).
// It bounds what one streaming pass (read once, write once) reaches on the machine, which
// the merge pipelines' achieved rates are compared with.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "nacho_hip.h"
#include "runtime.hpp"

namespace nacho {
namespace bandwidth {

constexpr int kBlock = 256;
constexpr int kBlocksPerCu = 128;

typedef unsigned grain_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void copy_kernel(const grain_t *__restrict__ src,
                                                      grain_t *__restrict__ dst, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(&src[i]), &dst[i]);
    }
}

int device_copy(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return NACHO_OK;
    if (!dst || !src || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    int device = 0, cus = 0;
    NACHO_TRY_HIP(hipGetDevice(&device));
    NACHO_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    const size_t n = bytes / 16;
    const size_t want = (n + kBlock - 1) / kBlock;
    const size_t cap = static_cast<size_t>(cus > 0 ? cus : 1) * kBlocksPerCu;
    const unsigned grid = static_cast<unsigned>(want < cap ? want : cap);
    copy_kernel<<<grid, kBlock, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const grain_t *>(src), static_cast<grain_t *>(dst), n);
    NACHO_TRY_HIP(hipGetLastError());
    return NACHO_OK;
}

}  // namespace bandwidth
}  // namespace nacho

extern "C" int nacho_device_copy(void *dst, const void *src, size_t bytes, void *stream) {
    return nacho::bandwidth::device_copy(dst, src, bytes, stream);
}
