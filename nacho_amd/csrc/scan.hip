// Device-wide exclusive prefix sum of int64 counts (reduce, scan of block sums, scan) — the
// 64-bit replacement for the CUB DeviceScan::InclusiveSum calls of the reference's generated
// code (stitch_and_generate_gpu.cpp:412-446, 717-740), whose int32 counters overflow on the
// SpGEMM configuration (6.0e9 products).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_utils.hpp"
#include "scan.hpp"

namespace nacho {
namespace scan {

constexpr int kBlock = 256;
constexpr int kPerThread = 16;
constexpr int kChunk = kBlock * kPerThread;
constexpr int64_t kSmall = 8 * kChunk;  // scanned by one workgroup in one launch

__global__ __launch_bounds__(kBlock) void block_sums_kernel(const int64_t *__restrict__ in,
                                                            int64_t n,
                                                            int64_t *__restrict__ sums) {
    __shared__ int64_t s_wave[kBlock / dev::kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
    int64_t v = 0;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int64_t i = base + threadIdx.x + static_cast<int64_t>(j) * kBlock;
        if (i < n) v += in[i];
    }
    int64_t total = 0;
    (void)dev::block_exclusive_sum<kBlock>(v, s_wave, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One workgroup: exclusive scan of in[0, n) into out (in == out allowed), chunk by chunk with
// a running carry; the total goes to *grand.
template <int BLOCK>
__device__ __forceinline__ void scan_one_workgroup(const int64_t *in, int64_t n, int64_t *out,
                                                   int64_t *grand) {
    constexpr int kStep = BLOCK * kPerThread;
    __shared__ int64_t s_wave[BLOCK / dev::kWave];
    int64_t carry = 0;
    for (int64_t start = 0; start < n; start += kStep) {
        int64_t v[kPerThread];
        int64_t mine = 0;
#pragma unroll
        for (int j = 0; j < kPerThread; ++j) {
            const int64_t i = start + static_cast<int64_t>(threadIdx.x) * kPerThread + j;
            v[j] = i < n ? in[i] : 0;
            mine += v[j];
        }
        int64_t total = 0;
        int64_t run = carry + dev::block_exclusive_sum<BLOCK>(mine, s_wave, total);
#pragma unroll
        for (int j = 0; j < kPerThread; ++j) {
            const int64_t i = start + static_cast<int64_t>(threadIdx.x) * kPerThread + j;
            if (i < n) out[i] = run;
            run += v[j];
        }
        carry += total;
    }
    if (threadIdx.x == 0) *grand = carry;
}

// Exclusive scan of the block sums in place; total to *grand.
__global__ __launch_bounds__(kBlock) void scan_sums_kernel(int64_t *sums, int64_t nb,
                                                           int64_t *__restrict__ grand) {
    scan_one_workgroup<kBlock>(sums, nb, sums, grand);
}

// Short inputs in one launch of one wide workgroup: out[0, n) and out[n] = total.
constexpr int kSmallBlock = 1024;
__global__ __launch_bounds__(kSmallBlock) void scan_small_kernel(const int64_t *in, int64_t n,
                                                                 int64_t *out) {
    scan_one_workgroup<kSmallBlock>(in, n, out, out + n);
}

__global__ __launch_bounds__(kBlock) void scan_blocks_kernel(const int64_t *__restrict__ in,
                                                             int64_t n,
                                                             const int64_t *__restrict__ sums,
                                                             int64_t *__restrict__ out) {
    __shared__ int64_t s_wave[kBlock / dev::kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
    // blocked arrangement: thread t owns elements [t*kPerThread, (t+1)*kPerThread)
    int64_t v[kPerThread];
    int64_t mine = 0;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int64_t i = base + static_cast<int64_t>(threadIdx.x) * kPerThread + j;
        v[j] = i < n ? in[i] : 0;
        mine += v[j];
    }
    int64_t total = 0;
    int64_t run = sums[blockIdx.x] + dev::block_exclusive_sum<kBlock>(mine, s_wave, total);
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int64_t i = base + static_cast<int64_t>(threadIdx.x) * kPerThread + j;
        if (i < n) out[i] = run;
        run += v[j];
    }
}

__global__ void copy_total_kernel(const int64_t *__restrict__ grand, int64_t *__restrict__ dst) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *dst = *grand;
}

int exclusive_scan_i64(Call &call, const int64_t *in, int64_t n, int64_t *out) {
    const hipStream_t s = call.stream();
    if (n <= kSmall) {  // one workgroup, one launch: launch latency dominates short scans
        scan_small_kernel<<<1, kSmallBlock, 0, s>>>(in, n, out);
        NACHO_TRY_HIP(hipGetLastError());
        return NACHO_OK;
    }
    const int64_t nb = n > 0 ? (n + kChunk - 1) / kChunk : 0;
    int64_t *sums = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nb) + 2, &sums));
    int64_t *grand = sums + nb;
    if (nb > 0) {
        block_sums_kernel<<<static_cast<unsigned>(nb), kBlock, 0, s>>>(in, n, sums);
        NACHO_TRY_HIP(hipGetLastError());
    }
    scan_sums_kernel<<<1, kBlock, 0, s>>>(sums, nb, grand);
    NACHO_TRY_HIP(hipGetLastError());
    if (nb > 0) {
        scan_blocks_kernel<<<static_cast<unsigned>(nb), kBlock, 0, s>>>(in, n, sums, out);
        NACHO_TRY_HIP(hipGetLastError());
    }
    copy_total_kernel<<<1, 64, 0, s>>>(grand, out + n);
    NACHO_TRY_HIP(hipGetLastError());
    return NACHO_OK;
}

}  // namespace scan
}  // namespace nacho
