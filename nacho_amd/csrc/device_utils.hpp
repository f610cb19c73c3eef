// Wave64 / workgroup building blocks shared by the gfx950 kernels: prefix sums over a
// wavefront and a workgroup, and the single-pass decoupled look-back that turns per-tile
// output counts into device-wide exclusive offsets without a second pass over the data.
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

// Inclusive prefix sum over the 64 lanes of a wavefront.
template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T v) {
    const int l = lane();
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        T n = __shfl_up(v, off, kWave);
        if (l >= off) v += n;
    }
    return v;
}

// Sum over the 64 lanes, result in every lane.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Exclusive prefix sum over a workgroup of BLOCK threads; `total` receives the sum of all.
// `s_wave` holds BLOCK/64 entries.  Ends with the workgroup synchronised and `s_wave` free.
template <int BLOCK, typename T>
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
    __syncthreads();
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

// Exclusive max over the workgroup (values >= 0, identity 0).  Ends synchronised.
__device__ __forceinline__ int block_exclusive_max(int v, int *s_wave) {
    const int l = lane();
    const int w = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int n = __shfl_up(incl, o, kWave);
        if (l >= o) incl = max(incl, n);
    }
    if (l == kWave - 1) s_wave[w] = incl;
    int excl = __shfl_up(incl, 1, kWave);
    if (l == 0) excl = 0;
    __syncthreads();
    for (int i = 0; i < w; ++i) excl = max(excl, s_wave[i]);
    __syncthreads();
    return excl;
}

// ---- decoupled look-back ------------------------------------------------------------
// One 64-bit status word per tile: state in the high half (0 = not yet published,
// 1 = tile aggregate, 2 = inclusive prefix), 32-bit value in the low half.  Word and state
// are published together by one 64-bit atomic store, so no fence orders them.
constexpr uint32_t kStateEmpty = 0, kStateAggregate = 1, kStateInclusive = 2;

__device__ __forceinline__ unsigned long long pack_status(uint32_t state, uint32_t value) {
    return (static_cast<unsigned long long>(state) << 32) | value;
}

__device__ __forceinline__ void publish(unsigned long long *slot, unsigned long long word) {
    __hip_atomic_store(slot, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long peek(const unsigned long long *slot) {
    return __hip_atomic_load(const_cast<unsigned long long *>(slot), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Upper bound on polls of one look-back window.  Tiles are numbered in launch-ticket order,
// so every predecessor is resident or finished and the wait ends long before this; the bound
// only guarantees that no wave can spin forever if that invariant were ever broken.  On
// expiry the tile records an error in `*error` (the host turns it into a failed call) and
// carries on with whatever prefix it has.
constexpr uint32_t kMaxPolls = 1u << 24;

// Executed by every lane of ONE wavefront of the tile's workgroup.  Publishes `aggregate`
// for `tile`, walks back over predecessors until an inclusive prefix is found, publishes
// this tile's inclusive prefix, and returns the exclusive prefix (uniform across the wave).
// One poll covers kLookbackWindow predecessors (kPerLane status words per lane, nearest
// first), because with hundreds of tiles in flight the nearest inclusive prefix is usually
// further back than one word per lane reaches, and every extra round is a device-coherent
// memory round trip.
constexpr int kPerLane = 4;
constexpr int kLookbackWindow = kWave * kPerLane;

__device__ __forceinline__ uint32_t lookback_exclusive(unsigned long long *status, int tile,
                                                       uint32_t aggregate, uint32_t *error) {
    const int l = lane();
    if (tile == 0) {
        if (l == 0) publish(&status[0], pack_status(kStateInclusive, aggregate));
        return 0;
    }
    if (l == 0) publish(&status[tile], pack_status(kStateAggregate, aggregate));
    uint32_t exclusive = 0;
    int nearest = tile - 1;  // lane l inspects nearest - (kPerLane*l + q), q = 0..kPerLane-1
    uint32_t polls = 0;
    while (true) {
        uint32_t state[kPerLane], value[kPerLane];
#pragma unroll
        for (int q = 0; q < kPerLane; ++q) {
            const int idx = nearest - (kPerLane * l + q);
            const unsigned long long word =
                idx >= 0 ? peek(&status[idx]) : pack_status(kStateInclusive, 0);
            state[q] = static_cast<uint32_t>(word >> 32);
            value[q] = static_cast<uint32_t>(word);
        }
        // First inclusive word in this lane (kPerLane = none), and whether an unpublished
        // word precedes it.
        int first = kPerLane;
#pragma unroll
        for (int q = kPerLane - 1; q >= 0; --q) {
            if (state[q] == kStateInclusive) first = q;
        }
        bool empty_before = false;
#pragma unroll
        for (int q = 0; q < kPerLane; ++q) {
            if (q <= first && q < kPerLane && state[q] == kStateEmpty) empty_before = true;
        }
        const unsigned long long inclusive_lanes = __ballot(first < kPerLane);
        const int stop = inclusive_lanes ? (__ffsll(static_cast<long long>(inclusive_lanes)) - 1)
                                         : kWave;  // lanes before `stop` contribute fully
        const bool lane_needed = l <= stop;
        if (__ballot(lane_needed && empty_before) != 0ull) {
            if (++polls < kMaxPolls) {
                __builtin_amdgcn_s_sleep(1);
                continue;
            }
            if (l == 0) atomicOr(error, 1u);
            break;
        }
        uint32_t mine = 0;
#pragma unroll
        for (int q = 0; q < kPerLane; ++q) {
            if (l < stop || (l == stop && q <= first)) mine += value[q];
        }
        exclusive += wave_sum(mine);
        if (stop < kWave) break;
        nearest -= kLookbackWindow;
    }
    if (l == 0) publish(&status[tile], pack_status(kStateInclusive, exclusive + aggregate));
    return exclusive;
}

}  // namespace dev
}  // namespace nacho
