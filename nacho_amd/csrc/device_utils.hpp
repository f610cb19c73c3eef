// Wave64 / workgroup building blocks shared by the gfx950 kernels: prefix sums over a
// wavefront and a workgroup, and a device-wide total taken by the last workgroup of a grid.
//
// These replace the reference's CUB DeviceScan::InclusiveSum calls between its count and
// write kernels (src/backend/stitch_and_generate_gpu.cpp:641-715) and its warp-32 shuffles
// (stitch_and_generate_gpu.cpp:337-363): on CDNA4 a wavefront is 64 lanes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nacho {
namespace dev {

constexpr int kWave = 64;

__device__ __forceinline__ int lane() { return static_cast<int>(__lane_id()); }

// Inclusive prefix sum of a 32-bit integer over the 64 lanes, on DPP: four row shifts
// (1, 2, 4, 8) scan each row of 16 lanes, then row broadcasts of lane 15 into rows 1 and 3
// and of lane 31 into rows 2 and 3 carry the row totals.  Lanes whose DPP source lies
// outside their row keep `old` = 0 (bound_ctrl off, so such lanes are not written).  Every
// lane must be active.
__device__ __forceinline__ int wave_inclusive_sum_dpp(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// The same for a running maximum of values >= 0 (0 is the identity).
__device__ __forceinline__ int wave_inclusive_max_dpp(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wavefront (DPP for 32-bit integers, lane
// shuffles otherwise).
template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T v) {
    if constexpr (sizeof(T) == 4 && !__is_same(T, float)) {
        return static_cast<T>(wave_inclusive_sum_dpp(static_cast<int>(v)));
    } else {
        const int l = lane();
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            T n = __shfl_up(v, off, kWave);
            if (l >= off) v += n;
        }
        return v;
    }
}

// Orders one wavefront's LDS accesses across its lanes.  The LDS processes a wavefront's
// instructions in order, so only the compiler must not move accesses across this point; a
// workgroup-scope fence would also wait for the wavefront's outstanding global stores.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Sum over the 64 lanes, result in every lane.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Exclusive prefix sum over a workgroup of BLOCK threads; `total` receives the sum of all.
// `s_wave` holds BLOCK/64 entries.  Ends with the workgroup synchronised and `s_wave` free,
// unless SYNC_END is false: then `s_wave` must not be written again before the caller's next
// barrier.
template <int BLOCK, typename T, bool SYNC_END = true>
__device__ __forceinline__ T block_exclusive_sum(T v, T *s_wave, T &total) {
    static_assert(BLOCK % kWave == 0, "workgroup must be whole wavefronts");
    constexpr int kWaves = BLOCK / kWave;
    const T incl = wave_inclusive_sum(v);
    const int w = threadIdx.x / kWave;
    if (lane() == kWave - 1) s_wave[w] = incl;
    __syncthreads();
    T before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        const T x = s_wave[i];
        before += (i < w) ? x : T(0);
        all += x;
    }
    if (SYNC_END) __syncthreads();
    total = all;
    return before + incl - v;
}

// Last index x in [lo, hi] with a[x] <= q (a non-decreasing, a[lo] <= q).
template <typename T>
__device__ __forceinline__ int64_t last_le(const T *__restrict__ a, int64_t lo, int64_t hi,
                                           int64_t q) {
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (static_cast<int64_t>(a[mid]) <= q) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    return lo;
}

// Largest x in [lo, hi] with pred(x) true, for a predicate that holds up to some point and
// fails after it; pred(lo) is taken to hold and is not evaluated.  G consecutive lanes (an
// aligned group of a wave, G a power of two up to 64; G = 1 is a binary search) call it together with the same lo,
// hi and pred, and all receive the result; other groups of the wave may search at the same
// time.  Each round splits the interval into G + 1 parts of at most `step` points and every
// lane of the group evaluates pred at the start of one of the last G parts, so n points take ceil(log_{G+1} n) rounds (one dependent
// load each) instead of log2 n.  Points evaluated lie in (lo, hi].  On a predicate that is
// not monotone the rounds still end, with some x in [lo, hi].
template <int G, typename Pred>
__device__ __forceinline__ int group_last_true(int lo, int hi, Pred pred) {
    static_assert(G >= 1 && G <= kWave && (G & (G - 1)) == 0, "G: a power of two in [1, 64]");
    if constexpr (G == 1) {  // one lane: a plain binary search
        while (lo < hi) {
            const int mid = static_cast<int>((static_cast<long long>(lo) + hi + 1) >> 1);
            if (pred(mid)) {
                lo = mid;
            } else {
                hi = mid - 1;
            }
        }
        return lo;
    }
    const int l = lane() % G;
    const int first = lane() - l;  // the group's first lane
    while (lo < hi) {  // uniform within the group
        const int step = static_cast<int>((static_cast<long long>(hi) - lo + 1 + G) / (G + 1));
        const long long x = lo + static_cast<long long>(l + 1) * step;
        const bool t = x <= hi && pred(static_cast<int>(x));
        const unsigned long long bits = __ballot(t) >> first;
        // the points that hold: lanes 0 .. c-1 of the group
        const int c = __popcll(G == kWave ? bits : bits & ((1ull << (G % kWave)) - 1));
        lo += c * step;
        hi = static_cast<int>(min(static_cast<long long>(hi), static_cast<long long>(lo) + step - 1));
    }
    return lo;
}

// Exclusive max over the workgroup (values >= 0, identity 0).  Ends synchronised, unless
// SYNC_END is false: then `s_wave` must not be written again before the caller's next
// barrier.
template <bool SYNC_END = true>
__device__ __forceinline__ int block_exclusive_max(int v, int *s_wave) {
    const int l = lane();
    const int w = threadIdx.x / kWave;
    const int incl = wave_inclusive_max_dpp(v);
    if (l == kWave - 1) s_wave[w] = incl;
    int excl = __shfl_up(incl, 1, kWave);
    if (l == 0) excl = 0;
    __syncthreads();
    for (int i = 0; i < w; ++i) excl = max(excl, s_wave[i]);
    if (SYNC_END) __syncthreads();
    return excl;
}

// ---- XCD-aware workgroup order -------------------------------------------------------
// The dispatcher sends workgroup b to XCD b % kXcds, and each XCD has its own L2.  Kernels
// whose neighbouring work items share data (a row's units reading adjacent ranges of the
// same B rows, a mask row's probes into one table) take logical index xcd_block<G>()
// instead of blockIdx.x: in every run of kXcds * G workgroups, those of one XCD take G
// consecutive items, so the lines those items share are fetched into one L2, while each
// XCD still draws its items from every part of the launch.  A bijection on
// [0, gridDim.x) (a last partial run keeps its order).
constexpr unsigned kXcds = 8;

template <unsigned G>
__device__ __forceinline__ unsigned xcd_block() {
    constexpr unsigned kRun = kXcds * G;
    const unsigned b = blockIdx.x;
    const unsigned run = b / kRun, w = b % kRun;
    if (run >= gridDim.x / kRun) return b;
    return run * kRun + (w % kXcds) * G + w / kXcds;
}

// ---- device-wide total without a second kernel -------------------------------------
// Called by thread 0 of every workgroup of a grid with the workgroup's own part (< 2^32).
// A 64-bit atomic add puts a ticket in the high half of a counter and the part in the low
// half; the workgroup whose ticket is the last one on a counter sees every other part on it
// already added (one address, so the adds are totally ordered).  Atomics on one address are
// serialised where they are executed (about 13 ns each measured on MI355X: 13.5 us for a
// launch of 1000 workgroups that only add their part), so the workgroups first add into one
// of kTotalGroups group counters (workgroup b into group b % kTotalGroups), each in its own
// 256-byte line, and the last of each group adds the group's sum into the top counter,
// whose last adder stores the total to `*out`.  Nothing waits and no fence is needed.  The
// caller guarantees that the total stays below 2^32 (it is a result length < 2^31).
//
// The accumulator holds kTotalWords 64-bit words, zeroed by zero_total in an earlier kernel
// on the stream.
constexpr int kTotalGroups = 32;
constexpr int kTotalStride = 32;  // 64-bit words between counters: 256 bytes
constexpr int kTotalWords = (kTotalGroups + 1) * kTotalStride;

// Zeroes the counters of a total's accumulator (one thread).
__device__ __forceinline__ void zero_total(unsigned long long *acc) {
#pragma unroll
    for (int g = 0; g <= kTotalGroups; ++g) acc[g * kTotalStride] = 0ull;
}

// The grid's total of `part`, or -1 in every workgroup but the last to add.
__device__ __forceinline__ int64_t two_level_total(uint32_t part, unsigned long long *acc) {
    const unsigned groups = gridDim.x < kTotalGroups ? gridDim.x : kTotalGroups;
    const unsigned g = blockIdx.x % kTotalGroups;
    const unsigned members = (gridDim.x - g + kTotalGroups - 1) / kTotalGroups;
    const unsigned long long prev = atomicAdd(&acc[(g + 1) * kTotalStride], (1ull << 32) | part);
    if ((prev >> 32) != members - 1) return -1;
    const uint32_t group_sum = static_cast<uint32_t>((prev + part) & 0xffffffffull);
    const unsigned long long top = atomicAdd(&acc[0], (1ull << 32) | group_sum);
    if ((top >> 32) != groups - 1) return -1;
    return static_cast<int64_t>((top + group_sum) & 0xffffffffull);
}

// Stores a result length with a system-scope release: the host reads it from pinned memory
// while later kernels of the stream still run.
__device__ __forceinline__ void store_system(int64_t *out, int64_t v) {
    __hip_atomic_store(out, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void add_to_total(uint32_t part, unsigned long long *acc,
                                             int64_t *out) {
    const int64_t total = two_level_total(part, acc);
    if (total >= 0) store_system(out, total);
}

// The same, storing `from` minus the total (a result length counted as the operands'
// entries less the pairs that merge).
__device__ __forceinline__ void subtract_total(uint32_t part, unsigned long long *acc,
                                               int64_t from, int64_t *out) {
    const int64_t total = two_level_total(part, acc);
    if (total >= 0) store_system(out, from - total);
}

}  // namespace dev
}  // namespace nacho
