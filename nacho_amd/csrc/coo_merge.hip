// COO / COO3 elementwise add (union) and multiply (intersection) for gfx950.
//
// Reference path replaced: coo_add, coo_mul and coo3d_add (compiler.cpp:118, 120, 138).  The
// reference lowers a COO operand's levels to one merged level whose coordinates are tuples
// compared lexicographically (Compile.cpp:66-154, tensor.cpp:447-577) and runs the same
// partition / count / scan / write pipeline as CSR over it, re-reading 2-3 coordinate arrays
// per comparison.  Here each tuple becomes one sortable key:
//   COO  (i, j)    -> (uint64)i << 32 | j
//   COO3 (i, j, k) -> i << (bj+bk) | j << bk | k  when the three extents fit 64 bits
//                     (bj, bk = bits of the j and k extents), else a (i<<32|j, k) pair.
// Coordinates are non-negative int32 below their extents, so key order is tuple order.
// The work is the merged sequence of both key lists (nnzA + nnzB items), cut into tiles.  A
// partition kernel finds every tile's merge-path split (equal keys never split, as the
// reference's balancing step, partition.cpp:964-983).  As for CSR (csr_merge.hip), each
// workgroup then owns a fixed chunk of tiles: a count kernel stores each chunk's output count
// and a write kernel starts from the preceding chunks' total.  Inside a tile the keys and
// values are staged in LDS from registers loaded one tile ahead, lanes split the tile by a
// merge-path search in LDS and walk their items (equal keys combined at the A step, the B
// step skipped), and results go through LDS to coalesced stores of the unpacked coordinates.
// Values are one IEEE binary32 add / multiply or a copy, as the reference's lattice
// (compute.cpp:476-491), so results are bit-exact.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "device_utils.hpp"
#include "csr_merge.hpp"
#include "runtime.hpp"

namespace nacho {
namespace coo {

enum class Op { Union, Intersect };

constexpr int kBlock = 256;
constexpr int kItemsPerLane = 8;
constexpr int kTile = kBlock * kItemsPerLane;

struct WideKey {
    unsigned long long hi;
    unsigned lo;
};
__device__ __forceinline__ bool operator<(const WideKey &x, const WideKey &y) {
    return x.hi < y.hi || (x.hi == y.hi && x.lo < y.lo);
}
__device__ __forceinline__ bool operator<=(const WideKey &x, const WideKey &y) {
    return !(y < x);
}
__device__ __forceinline__ bool operator==(const WideKey &x, const WideKey &y) {
    return x.hi == y.hi && x.lo == y.lo;
}

// Key encoding of one operand's coordinate arrays.
struct Coords {
    const int *c0, *c1, *c2;  // i, j, k (c2 unused for COO)
};

struct PackedCodec {  // COO, and COO3 whose extents fit 64 bits
    using Key = unsigned long long;
    int arity;
    int shift_i, shift_j;  // key = i << shift_i | j << shift_j | k
    unsigned long long mask_j, mask_k;
    __device__ __forceinline__ Key load(const Coords &c, int x) const {
        Key key = static_cast<Key>(static_cast<unsigned>(c.c0[x])) << shift_i;
        key |= static_cast<Key>(static_cast<unsigned>(c.c1[x])) << shift_j;
        if (arity == 3) key |= static_cast<unsigned>(c.c2[x]);
        return key;
    }
    __device__ __forceinline__ void unpack(Key key, int &i, int &j, int &k) const {
        i = static_cast<int>(key >> shift_i);
        j = static_cast<int>((key >> shift_j) & mask_j);
        k = static_cast<int>(key & mask_k);
    }
};

struct WideCodec {  // COO3 whose extents need more than 64 bits
    using Key = WideKey;
    int arity;
    __device__ __forceinline__ Key load(const Coords &c, int x) const {
        Key key;
        key.hi = (static_cast<unsigned long long>(static_cast<unsigned>(c.c0[x])) << 32) |
                 static_cast<unsigned>(c.c1[x]);
        key.lo = static_cast<unsigned>(c.c2[x]);
        return key;
    }
    __device__ __forceinline__ void unpack(Key key, int &i, int &j, int &k) const {
        i = static_cast<int>(key.hi >> 32);
        j = static_cast<int>(key.hi & 0xffffffffull);
        k = static_cast<int>(key.lo);
    }
};

template <typename ReadA, typename ReadB>
__device__ __forceinline__ void merge_split(ReadA A, ReadB B, int aS, int aE, int bS, int bE,
                                            int D, int &a, int &b) {
    int lo = max(aS, D - bE);
    int hi = min(aE, D - bS);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (A(mid) <= B(D - 1 - mid)) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    a = lo;
    b = D - lo;
    if (a > aS && b < bE && A(a - 1) == B(b)) ++b;
}

constexpr int kPartBlock = 64;

template <typename Codec>
__global__ __launch_bounds__(kPartBlock) void coo_partition_kernel(Codec codec, Coords ca, int nnz_a,
                                                            Coords cb, int nnz_b, int num_tiles,
                                                            int *__restrict__ split_a,
                                                            int *__restrict__ split_b,
                                                            unsigned long long *__restrict__ done) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t > num_tiles) return;
    if (t == 0) dev::zero_total(done);  // accumulator of the kernel that totals the length
    const int total = nnz_a + nnz_b;
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);
    int a, b;
    merge_split([&](int x) { return codec.load(ca, x); }, [&](int y) { return codec.load(cb, y); },
                0, nnz_a, 0, nnz_b, diag, a, b);
    split_a[t] = a;
    split_b[t] = b;
}

constexpr int kMaxChunk = 64;

// Stage the chunk's splits (2 ints per boundary) in LDS once per workgroup.
__device__ __forceinline__ void stage_splits(int *s_split, const int *__restrict__ split_a,
                                             const int *__restrict__ split_b, int t0, int t1) {
    for (int i = threadIdx.x; i <= t1 - t0; i += kBlock) {
        s_split[2 * i] = split_a[t0 + i];
        s_split[2 * i + 1] = split_b[t0 + i];
    }
}

// One lane's keys/values of a tile, loaded one tile ahead (unconditional, clamped loads).
template <typename Key, int LOADS>
struct StagedKeys {
    Key key[LOADS];
    int val[LOADS];
};

template <bool VALUES, typename Codec, int LOADS>
__device__ __forceinline__ void fetch_keys(StagedKeys<typename Codec::Key, LOADS> &st,
                                           const Codec &codec, const int *s_split, int i,
                                           Coords ca, const float *__restrict__ va, Coords cb,
                                           const float *__restrict__ vb, int tid) {
    const int a0 = s_split[2 * i], b0 = s_split[2 * i + 1];
    const int na = s_split[2 * i + 2] - a0, nab = na + s_split[2 * i + 3] - b0;
    if (nab <= 0) return;
    const int *vai = reinterpret_cast<const int *>(va);
    const int *vbi = reinterpret_cast<const int *>(vb);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int k = min(tid + j * kBlock, nab - 1);
        const bool in_a = k < na;
        const int off = in_a ? a0 + k : b0 + (k - na);
        st.key[j] = codec.load(in_a ? ca : cb, off);
        if (VALUES) st.val[j] = (in_a ? vai : vbi)[off];
    }
}

template <bool VALUES, typename Key, int LOADS>
__device__ __forceinline__ void stage_keys(const StagedKeys<Key, LOADS> &st, const int *s_split,
                                           int i, Key *s_key, float *s_val, int tid) {
    const int nab = s_split[2 * i + 2] - s_split[2 * i] + s_split[2 * i + 3] - s_split[2 * i + 1];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int k = tid + j * kBlock;
        if (k < nab) {
            s_key[k] = st.key[j];
            if (VALUES) s_val[k] = __int_as_float(st.val[j]);
        }
    }
}

// Lane walk over a tile of keys (no rows): lane t owns items [t*IPT, (t+1)*IPT) of the
// tile's merged order; equal keys are combined at the A step and the B step is skipped.
template <Op OP, bool VALUES, typename Key, int STEPS>
struct KeyLaneOut {
    Key key[STEPS];
    float val[STEPS];
    unsigned valid;
};

template <Op OP, bool VALUES, typename Key>
__device__ __forceinline__ void walk_keys(KeyLaneOut<OP, VALUES, Key, kItemsPerLane + 1> &out,
                                          const int *s_split, int i, int tile, const Key *s_key,
                                          const float *s_val, int tid) {
    constexpr int kSteps = kItemsPerLane + 1;
    const int a0 = s_split[2 * i], b0 = s_split[2 * i + 1];
    const int a1 = s_split[2 * i + 2], b1 = s_split[2 * i + 3];
    const int na = a1 - a0;
    auto A = [&](int x) { return s_key[x - a0]; };
    auto B = [&](int y) { return s_key[na + y - b0]; };
    const int tile_lo = tile * kTile;
    const int tile_start = a0 + b0, tile_end = a1 + b1;
    const int g_lo = tid == 0 ? tile_start : tile_lo + tid * kItemsPerLane;
    const int steps = tid == kBlock - 1 ? tile_end - g_lo
                                        : min(tile_lo + (tid + 1) * kItemsPerLane, tile_end) - g_lo;
    int a = a0, b = b0;
    if (tid > 0 && g_lo < tile_end) {
        int slo = max(a0, g_lo - b1), shi = min(a1, g_lo - b0);
        while (slo < shi) {
            const int mid = (slo + shi) >> 1;
            if (A(mid) <= B(g_lo - 1 - mid)) {
                slo = mid + 1;
            } else {
                shi = mid;
            }
        }
        a = slo;
        b = g_lo - slo;
    }
    bool has_last = a > a0;
    Key last_a = has_last ? A(a - 1) : Key{};
    unsigned valid = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        out.val[s] = 0.0f;
        if (s < steps) {
            const bool a_in = a < a1, b_in = b < b1;
            // out-of-range heads read a harmless in-bounds slot and are masked by a_in / b_in
            const Key xa = A(a_in ? a : a0);
            const Key xb = B(b_in ? b : b0);
            const bool take_a = a_in && (!b_in || xa <= xb);
            const bool pair = take_a && b_in && xa == xb;
            out.key[s] = take_a ? xa : xb;
            if (VALUES) {
                const float own = s_val[take_a ? a - a0 : na + b - b0];
                if (OP == Op::Union) {
                    out.val[s] = pair ? own + s_val[na + b - b0] : own;
                } else {
                    out.val[s] = own * s_val[na + b - b0];
                }
            }
            const bool skip = !take_a && has_last && last_a == xb;
            const bool emit = (OP == Op::Union) ? !skip : pair;
            valid |= static_cast<unsigned>(emit) << s;
            if (take_a) {
                last_a = xa;
                has_last = true;
            }
            a += take_a;
            b += !take_a;
        }
    }
    out.valid = valid;
}

template <Op OP, typename Codec>
__global__ __launch_bounds__(kBlock) void coo_count_kernel(Codec codec, Coords ca, Coords cb,
                                                          int num_tiles, int chunk,
                                                          const int *__restrict__ split_a,
                                                          const int *__restrict__ split_b,
                                                          unsigned *__restrict__ chunk_count,
                                                          unsigned long long *__restrict__ done,
                                                          int64_t *__restrict__ length_out) {
    using Key = typename Codec::Key;
    constexpr int kCap = kTile + 2;
    constexpr int kLoads = (kCap + kBlock - 1) / kBlock;
    __shared__ Key s_key[kCap];
    __shared__ unsigned s_wave[kBlock / dev::kWave];
    __shared__ int s_split[2 * (kMaxChunk + 1)];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) {
        if (tid == 0) {
            chunk_count[blockIdx.x] = 0u;
            dev::add_to_total(0u, done, length_out);
        }
        return;
    }
    stage_splits(s_split, split_a, split_b, t0, t1);
    __syncthreads();
    StagedKeys<Key, kLoads> st;
    fetch_keys<false>(st, codec, s_split, 0, ca, nullptr, cb, nullptr, tid);
    stage_keys<false>(st, s_split, 0, s_key, nullptr, tid);
    __syncthreads();
    unsigned total = 0;
    for (int t = t0; t < t1; ++t) {
        const int i = t - t0;
        if (t + 1 < t1) fetch_keys<false>(st, codec, s_split, i + 1, ca, nullptr, cb, nullptr, tid);
        KeyLaneOut<OP, false, Key, kItemsPerLane + 1> lo;
        walk_keys<OP, false, Key>(lo, s_split, i, t, s_key, nullptr, tid);
        unsigned c = dev::wave_sum(static_cast<unsigned>(__popc(lo.valid)));
        if (dev::lane() == 0) s_wave[tid / dev::kWave] = c;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kBlock / dev::kWave; ++w) total += s_wave[w];
        __syncthreads();
        if (t + 1 < t1) {
            stage_keys<false>(st, s_split, i + 1, s_key, nullptr, tid);
            __syncthreads();
        }
    }
    if (tid == 0) {
        chunk_count[blockIdx.x] = total;
        // The last workgroup to finish stores the result length (the sum of every chunk).
        dev::add_to_total(total, done, length_out);
    }
}

// SPREAD (intersection only, no count pass): a tile's outputs go to zi/zj/zk/zv at the
// tile's own start position in A (spread_by_a) or B, whose range holds every pair the tile
// can emit; tile_count[t] receives the tile's length, chunk_total[w] the sum over
// workgroup w's chunk, and the last workgroup to finish stores the sum of all chunks, the
// result length, to `length_out`.  coo_compact_kernel then moves each tile to its final
// offset.
template <Op OP, typename Codec, bool SPREAD>
__global__ __launch_bounds__(kBlock) void coo_write_kernel(
    Codec codec, Coords ca, const float *__restrict__ va, Coords cb, const float *__restrict__ vb,
    int num_tiles, int chunk, const int *__restrict__ split_a, const int *__restrict__ split_b,
    const unsigned *__restrict__ chunk_count, int *__restrict__ zi, int *__restrict__ zj,
    int *__restrict__ zk, float *__restrict__ zv, unsigned *__restrict__ length,
    int spread_by_a, int64_t *__restrict__ tile_count, int64_t *__restrict__ chunk_total,
    unsigned long long *__restrict__ done, int64_t *__restrict__ length_out) {
    static_assert(!SPREAD || OP == Op::Intersect, "spread output: intersection");
    using Key = typename Codec::Key;
    constexpr int kCap = kTile + 2;
    constexpr int kLoads = (kCap + kBlock - 1) / kBlock;
    constexpr int kSteps = kItemsPerLane + 1;
    __shared__ Key s_key[kCap];
    __shared__ float s_val[kCap];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_split[2 * (kMaxChunk + 1)];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) {
        if (SPREAD) {
            if (tid == 0) {
                chunk_total[blockIdx.x] = 0;
                dev::add_to_total(0u, done, length_out);
            }
        }
        return;
    }
    stage_splits(s_split, split_a, split_b, t0, t1);
    int base = 0;
    if (!SPREAD) {
        int before = 0;
        for (int i = tid; i < static_cast<int>(blockIdx.x); i += kBlock) before += chunk_count[i];
        (void)dev::block_exclusive_sum<kBlock>(before, s_wave, base);
    } else {
        __syncthreads();  // the staged splits
    }

    StagedKeys<Key, kLoads> st;
    fetch_keys<true>(st, codec, s_split, 0, ca, va, cb, vb, tid);
    stage_keys<true>(st, s_split, 0, s_key, s_val, tid);
    __syncthreads();
    int64_t spread_sum = 0;
    for (int t = t0; t < t1; ++t) {
        const int i = t - t0;
        if (t + 1 < t1) fetch_keys<true>(st, codec, s_split, i + 1, ca, va, cb, vb, tid);
        KeyLaneOut<OP, true, Key, kSteps> lo;
        walk_keys<OP, true, Key>(lo, s_split, i, t, s_key, s_val, tid);
        if (SPREAD) base = spread_by_a ? s_split[2 * i] : s_split[2 * i + 1];
        int tile_total = 0;
        const int offset =
            dev::block_exclusive_sum<kBlock>(static_cast<int>(__popc(lo.valid)), s_wave, tile_total);
        int o = offset;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (lo.valid & (1u << s)) {
                s_key[o] = lo.key[s];
                s_val[o] = lo.val[s];
                ++o;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int q = tid + j * kBlock;
            if (q < tile_total) {
                int ci, cj, ck;
                codec.unpack(s_key[q], ci, cj, ck);
                zi[base + q] = ci;
                zj[base + q] = cj;
                if (codec.arity == 3) zk[base + q] = ck;
                zv[base + q] = s_val[q];
            }
        }
        if (SPREAD && tid == 0) {
            tile_count[t] = tile_total;
            spread_sum += tile_total;
            if (t + 1 == t1) chunk_total[blockIdx.x] = spread_sum;
        }
        base += tile_total;
        if (!SPREAD && t == num_tiles - 1 && tid == 0) *length = static_cast<unsigned>(base);
        __syncthreads();
        if (t + 1 < t1) {
            stage_keys<true>(st, s_split, i + 1, s_key, s_val, tid);
            __syncthreads();
        }
    }
    // Spread output: the last workgroup to finish stores the result length.
    if (SPREAD && tid == 0) dev::add_to_total(static_cast<uint32_t>(spread_sum), done, length_out);
}

// Moves each tile's outputs from its spread position (coo_write_kernel<SPREAD>) to its final
// offset: the sum of the earlier chunks' totals and of the earlier tiles of its own chunk
// (`chunk` tiles per chunk).  One workgroup per tile; the last one stores the length.
__global__ __launch_bounds__(kBlock) void coo_compact_kernel(
    const int *__restrict__ split_a, const int *__restrict__ split_b, int num_tiles, int chunk,
    int spread_by_a, int arity, const int64_t *__restrict__ tile_count,
    const int64_t *__restrict__ chunk_total, const int *__restrict__ ti,
    const int *__restrict__ tj, const int *__restrict__ tk, const float *__restrict__ tv,
    int *__restrict__ zi, int *__restrict__ zj, int *__restrict__ zk, float *__restrict__ zv,
    int64_t *__restrict__ length) {
    __shared__ int64_t s_wave[kBlock / dev::kWave];
    const int t = blockIdx.x;
    const int c = t / chunk;
    int64_t before = 0;
    for (int i = threadIdx.x; i < c; i += kBlock) before += chunk_total[i];
    for (int i = c * chunk + static_cast<int>(threadIdx.x); i < t; i += kBlock) before += tile_count[i];
    int64_t to64 = 0;
    (void)dev::block_exclusive_sum<kBlock>(before, s_wave, to64);
    const int from = spread_by_a ? split_a[t] : split_b[t];
    const int to = static_cast<int>(to64);
    const int n = static_cast<int>(tile_count[t]);
    if (t == num_tiles - 1 && threadIdx.x == 0) *length = to64 + n;
    for (int q = threadIdx.x; q < n; q += kBlock) {
        zi[to + q] = ti[from + q];
        zj[to + q] = tj[from + q];
        if (arity == 3) zk[to + q] = tk[from + q];
        zv[to + q] = tv[from + q];
    }
}

int bits_for_extent(int extent) {
    unsigned m = extent > 1 ? static_cast<unsigned>(extent - 1) : 0u;
    int bits = 0;
    while (m) {
        ++bits;
        m >>= 1;
    }
    return bits;
}

// Shared host orchestration.  `arity` 2 (COO) or 3 (COO3); `extents` are the dimension
// sizes; coordinate arrays and values per operand; outputs allocated here.
template <Op OP>
int coo_binary(int arity, const int32_t extents[3], Coords ca, const float *va, int nnz_a,
               Coords cb, const float *vb, int nnz_b, int32_t num_blocks,
               int32_t threads_per_block, void *stream, const nacho_allocator *alloc,
               const char *kernel_name, int32_t *out_coords[3], float **out_val,
               int32_t *out_nnz) {
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    const long long total = static_cast<long long>(nnz_a) + nnz_b;
    if (total > static_cast<long long>(INT_MAX) - 2 * kTile) return NACHO_ERR_INDEX_OVERFLOW;
    const long long cap = (OP == Op::Union) ? total : (nnz_a < nnz_b ? nnz_a : nnz_b);
    const int num_tiles = total > 0 ? static_cast<int>((total + kTile - 1) / kTile) : 1;

    Call call(stream, alloc);
    int *splits = nullptr;
    NACHO_TRY(call.scratch_n(2 * (static_cast<size_t>(num_tiles) + 1), &splits));
    int *split_a = splits, *split_b = splits + num_tiles + 1;

    int32_t *z[3] = {nullptr, nullptr, nullptr};
    float *zv = nullptr;
    for (int d = 0; d < arity; ++d) NACHO_TRY(call.result_n(static_cast<size_t>(cap), &z[d]));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zv));

    const hipStream_t s = call.stream();
    // one thread per boundary in 64-thread workgroups, so the dependent searches spread
    // over every CU
    const unsigned part_grid = ceil_div(static_cast<size_t>(num_tiles) + 1, kPartBlock);
    const int bi = bits_for_extent(extents[0]), bj = bits_for_extent(extents[1]);
    const int bk = arity == 3 ? bits_for_extent(extents[2]) : 0;
    unsigned *counts = nullptr;
    auto launch = [&](auto codec) -> int {
        using Codec = decltype(codec);
        constexpr bool kSpread = OP == Op::Intersect;
        int resident = 0;
        NACHO_TRY(resident_grid(
            reinterpret_cast<const void *>(coo_write_kernel<OP, Codec, kSpread>), kBlock,
            &resident));
        int chunk = (num_tiles + resident - 1) / resident;
        if (chunk > kMaxChunk) chunk = kMaxChunk;
        const int grid = (num_tiles + chunk - 1) / chunk;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 4 + 2 * dev::kTotalWords, &counts));
        // 64-bit accumulator of the length total (an 8-byte aligned slot after the counts).
    unsigned long long *done =
        reinterpret_cast<unsigned long long *>(counts + ((grid + 2) & ~1));
        // The result length goes straight to a pinned host word as soon as the kernel that
        // totals it ends; the host waits for that kernel only, not for the writes after it.
        int64_t *length_out = nullptr;
        NACHO_TRY(call.length_word(&length_out));
        if (kSpread) {
            // One walk: each tile writes its pairs at its own position in the smaller
            // operand's range of scratch arrays, then one compaction moves them into place.
            const int by_a = nnz_a <= nnz_b ? 1 : 0;
            int32_t *t[3] = {nullptr, nullptr, nullptr};
            float *tv = nullptr;
            int64_t *tile_count = nullptr, *chunk_total = nullptr;
            for (int d = 0; d < arity; ++d) NACHO_TRY(call.scratch_n(static_cast<size_t>(cap), &t[d]));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(cap), &tv));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles), &tile_count));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 1, &chunk_total));
            int64_t *len_dev = chunk_total + grid;
            NACHO_TRY(call.timer_start(kernel_name));
            coo_partition_kernel<Codec><<<part_grid, kPartBlock, 0, s>>>(codec, ca, nnz_a, cb, nnz_b,
                                                                  num_tiles, split_a, split_b,
                                                                  done);
            NACHO_TRY_HIP(hipGetLastError());
            coo_write_kernel<OP, Codec, kSpread><<<grid, kBlock, 0, s>>>(
                codec, ca, va, cb, vb, num_tiles, chunk, split_a, split_b, nullptr, t[0], t[1],
                t[2], tv, nullptr, by_a, tile_count, chunk_total, done, length_out);
            NACHO_TRY_HIP(hipGetLastError());
            NACHO_TRY(call.mark_length());
            coo_compact_kernel<<<num_tiles, kBlock, 0, s>>>(
                split_a, split_b, num_tiles, chunk, by_a, arity, tile_count, chunk_total, t[0],
                t[1], t[2], tv, z[0], z[1], z[2], zv, len_dev);
            NACHO_TRY_HIP(hipGetLastError());
            NACHO_TRY(call.timer_stop());
            int64_t len = 0;
            NACHO_TRY(call.wait_length(&len));
            if (len > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;
            *out_nnz = static_cast<int32_t>(len);
            return NACHO_OK;
        }
        NACHO_TRY(call.timer_start(kernel_name));
        coo_partition_kernel<Codec><<<part_grid, kPartBlock, 0, s>>>(codec, ca, nnz_a, cb, nnz_b, num_tiles,
                                                              split_a, split_b, done);
        NACHO_TRY_HIP(hipGetLastError());
        coo_count_kernel<OP, Codec><<<grid, kBlock, 0, s>>>(codec, ca, cb, num_tiles, chunk, split_a,
                                                            split_b, counts, done, length_out);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.mark_length());
        coo_write_kernel<OP, Codec, false><<<grid, kBlock, 0, s>>>(
            codec, ca, va, cb, vb, num_tiles, chunk, split_a, split_b, counts, z[0], z[1], z[2],
            zv, counts + grid, 0, nullptr, nullptr, nullptr, nullptr);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        int64_t len = 0;
        NACHO_TRY(call.wait_length(&len));
        if (len > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;
        *out_nnz = static_cast<int32_t>(len);
        return NACHO_OK;
    };
    if (arity == 2) {
        PackedCodec c{2, 32, 0, 0xffffffffull, 0ull};
        NACHO_TRY(launch(c));
    } else if (bi + bj + bk <= 64) {
        PackedCodec c{3, bj + bk, bk, bj >= 64 ? ~0ull : ((1ull << bj) - 1),
                      bk >= 64 ? ~0ull : ((1ull << bk) - 1)};
        NACHO_TRY(launch(c));
    } else {
        WideCodec c{3};
        NACHO_TRY(launch(c));
    }
    const long long nnz = *out_nnz;
    if (nnz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nnz == 0) {
        for (int d = 0; d < arity; ++d) {
            call.drop_result(z[d]);
            z[d] = nullptr;
        }
        call.drop_result(zv);
        zv = nullptr;
    }
    for (int d = 0; d < 3; ++d) out_coords[d] = z[d];
    *out_val = zv;
    *out_nnz = static_cast<int32_t>(nnz);
    call.commit();
    return NACHO_OK;
}

// ---- 2-D COO through row offsets ---------------------------------------------------------
//
// A 2-D COO operand sorted by (i, j) is a CSR matrix without its offsets.  When the rows are
// not far more than the entries, coo_add / coo_mul build both operands' row offsets (one
// pass over i), run the CSR level merge (csr_merge.hip: pair-count union or spread
// intersection), and take each output's row from the write kernel, which knows it: the
// result is the same sequence of (i, j, value) as the merged-coordinate path.

// pos[r] = the first entry whose row is >= r, r in [0, rows].  Entry p writes the rows after
// the previous entry's row up to its own, and the position nnz closes the last rows (row
// indices clamped to [0, rows]; coordinates must be sorted and in range, as for every
// operand).  Each thread takes kRowOffsetsPer consecutive entries, read with one 16-byte load
// when the array is 16-byte aligned, so a wavefront's loads cover 1 KB contiguously (eight
// entries per thread in two 16-byte loads took 49.3 us for the C2 operands as COO, four
// 44.0 us).  (A merge of the row markers with the entries, balanced whatever the gaps
// between nonempty rows, reloaded one entry per step and was 18x slower.)
constexpr int kRowOffsetsPer = 4;

struct RowOffsetsJob {
    const int *ci;
    int nnz;
    int *pos;
};

// Both operands in one launch: workgroups [0, blocks_a) build A's offsets, the rest B's.
__global__ void coo_row_offsets_kernel(RowOffsetsJob ja, RowOffsetsJob jb, int blocks_a,
                                       int rows) {
    const bool first = static_cast<int>(blockIdx.x) < blocks_a;
    const int *__restrict__ ci = first ? ja.ci : jb.ci;
    const int nnz = first ? ja.nnz : jb.nnz;
    int *__restrict__ pos = first ? ja.pos : jb.pos;
    const int64_t block = first ? blockIdx.x : blockIdx.x - blocks_a;
    const int64_t blocks = first ? blocks_a : gridDim.x - blocks_a;
    const int64_t n_groups = (static_cast<int64_t>(nnz) + kRowOffsetsPer) / kRowOffsetsPer;
    const bool aligned = (reinterpret_cast<uintptr_t>(ci) & 15u) == 0;
    for (int64_t g = block * blockDim.x + threadIdx.x; g < n_groups; g += blocks * blockDim.x) {
        const int64_t p0 = g * kRowOffsetsPer;
        int v[kRowOffsetsPer];
        if (aligned && p0 + kRowOffsetsPer <= nnz) {
            const int4 x0 = *reinterpret_cast<const int4 *>(ci + p0);
            v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        } else {
#pragma unroll
            for (int u = 0; u < kRowOffsetsPer; ++u) {
                v[u] = p0 + u < nnz ? ci[p0 + u] : rows;  // past the end: closes the last rows
            }
        }
        int prev = p0 == 0 ? -1 : min(max(ci[p0 - 1], -1), rows);
#pragma unroll
        for (int u = 0; u < kRowOffsetsPer; ++u) {
            const int64_t p = p0 + u;
            if (p > nnz) break;
            const int cur = min(max(v[u], -1), rows);
            for (int r = prev + 1; r <= cur; ++r) pos[r] = static_cast<int>(p);
            prev = max(prev, cur);
        }
    }
}

// Rows at most this many times the entries take the row-offset path.
constexpr long long kRowPathRowsPerEntry = 4;

template <Op OP>
int coo2_rows(const nacho_coo *a, const nacho_coo *b, nacho_coo *z, void *stream,
              const nacho_allocator *alloc, const char *name) {
    const int rows = a->dim_i_size;
    const int nnz_a = a->nnz, nnz_b = b->nnz;
    const long long cap = (OP == Op::Union) ? static_cast<long long>(nnz_a) + nnz_b
                                            : (nnz_a < nnz_b ? nnz_a : nnz_b);
    Call call(stream, alloc);
    int *pa = nullptr, *pb = nullptr, *pz = nullptr, *zi = nullptr, *zj = nullptr;
    float *zv = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pa));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pb));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pz));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zi));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zj));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zv));
    const hipStream_t s = call.stream();
    NACHO_TRY(call.timer_start(name));
    const unsigned ga = ceil_div(static_cast<size_t>(nnz_a) / kRowOffsetsPer + 1, 256);
    const unsigned gb = ceil_div(static_cast<size_t>(nnz_b) / kRowOffsetsPer + 1, 256);
    coo_row_offsets_kernel<<<ga + gb, 256, 0, s>>>(RowOffsetsJob{a->dim_i_indices, nnz_a, pa},
                                                   RowOffsetsJob{b->dim_i_indices, nnz_b, pb},
                                                   static_cast<int>(ga), rows);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());  // (kernel timing only) before the merge's own interval
    const csr::LevelOperand A{pa, a->dim_j_indices, a->values, nnz_a, nullptr};
    const csr::LevelOperand B{pb, b->dim_j_indices, b->values, nnz_b, nullptr};
    const csr::LevelResult Z{pz, zj, zv, nullptr, nullptr, zi};
    long long nnz = 0;
    NACHO_TRY(csr::merge_level(call, OP == Op::Intersect, true, false, rows, A, B, Z, &nnz, name));
    if (nnz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nnz == 0) {
        call.drop_result(zi);
        call.drop_result(zj);
        call.drop_result(zv);
        zi = zj = nullptr;
        zv = nullptr;
    }
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_i_length = static_cast<int32_t>(nnz);
    z->dim_i_indices = zi;
    z->dim_j_length = static_cast<int32_t>(nnz);
    z->dim_j_indices = zj;
    z->values = zv;
    z->nnz = static_cast<int32_t>(nnz);
    call.commit();
    return NACHO_OK;
}

// ---- COO3 through row offsets ------------------------------------------------------------
//
// A COO3 operand sorted by (i, j, k) is a matrix with rows i and columns (j, k) in
// lexicographic order.  When the j and k extents fit 31 bits together and the largest key
// stays below INT_MAX, the column key j << kbits | k (kbits = bits of the k extent) orders
// entries as (j, k) does, so coo3d_add
// builds both operands' row offsets and keys in one pass, runs the CSR level union on them,
// and the write kernel stores each output key split back into j and k, with its row as i.

struct KeysJob {
    const int *ci, *cj, *ck;
    int nnz;
    int *pos;  // rows + 1 row offsets
    int *key;  // nnz column keys cj << kbits | ck
};

// Row offsets (as coo_row_offsets_kernel) and column keys of both COO3 operands in one
// launch: workgroups [0, blocks_a) take A, the rest B; each thread kRowOffsetsPer consecutive
// entries, whose i, j and k loads are all issued before anything is stored (16-byte loads
// and stores when every array is 16-byte aligned).
__global__ void coo3_keys_kernel(KeysJob ja, KeysJob jb, int blocks_a, int rows, int kbits) {
    const bool first = static_cast<int>(blockIdx.x) < blocks_a;
    const KeysJob &job = first ? ja : jb;
    const int *__restrict__ ci = job.ci;
    const int *__restrict__ cj = job.cj;
    const int *__restrict__ ck = job.ck;
    int *__restrict__ pos = job.pos;
    int *__restrict__ key = job.key;
    const int nnz = job.nnz;
    const int64_t block = first ? blockIdx.x : blockIdx.x - blocks_a;
    const int64_t blocks = first ? blocks_a : gridDim.x - blocks_a;
    const int64_t n_groups = (static_cast<int64_t>(nnz) + kRowOffsetsPer) / kRowOffsetsPer;
    const bool aligned = ((reinterpret_cast<uintptr_t>(ci) | reinterpret_cast<uintptr_t>(cj) |
                           reinterpret_cast<uintptr_t>(ck) | reinterpret_cast<uintptr_t>(key)) &
                          15u) == 0;
    static_assert(kRowOffsetsPer == 4, "one 16-byte group per thread");
    for (int64_t g = block * blockDim.x + threadIdx.x; g < n_groups; g += blocks * blockDim.x) {
        const int64_t p0 = g * kRowOffsetsPer;
        int v[kRowOffsetsPer], kv[kRowOffsetsPer];
        const int before = p0 == 0 ? -1 : ci[p0 - 1];
        if (aligned && p0 + kRowOffsetsPer <= nnz) {
            const int4 i0 = *reinterpret_cast<const int4 *>(ci + p0);
            const int4 j0 = *reinterpret_cast<const int4 *>(cj + p0);
            const int4 k0 = *reinterpret_cast<const int4 *>(ck + p0);
            v[0] = i0.x; v[1] = i0.y; v[2] = i0.z; v[3] = i0.w;
            kv[0] = j0.x << kbits | k0.x; kv[1] = j0.y << kbits | k0.y;
            kv[2] = j0.z << kbits | k0.z; kv[3] = j0.w << kbits | k0.w;
            *reinterpret_cast<int4 *>(key + p0) = make_int4(kv[0], kv[1], kv[2], kv[3]);
        } else {
#pragma unroll
            for (int u = 0; u < kRowOffsetsPer; ++u) {
                const bool in = p0 + u < nnz;
                v[u] = in ? ci[p0 + u] : rows;  // past the end: closes the last rows
                if (in) key[p0 + u] = cj[p0 + u] << kbits | ck[p0 + u];
            }
        }
        int prev = min(max(before, -1), rows);
#pragma unroll
        for (int u = 0; u < kRowOffsetsPer; ++u) {
            const int64_t p = p0 + u;
            if (p > nnz) break;
            const int cur = min(max(v[u], -1), rows);
            for (int r = prev + 1; r <= cur; ++r) pos[r] = static_cast<int>(p);
            prev = max(prev, cur);
        }
    }
}

int coo3_rows(const nacho_coo3 *a, const nacho_coo3 *b, nacho_coo3 *z, void *stream,
              const nacho_allocator *alloc, int kbits, const char *name) {
    const int rows = a->dim_i_size;
    const int nnz_a = a->nnz, nnz_b = b->nnz;
    const long long cap = static_cast<long long>(nnz_a) + nnz_b;
    Call call(stream, alloc);
    int *pa = nullptr, *pb = nullptr, *pz = nullptr, *ka = nullptr, *kb = nullptr;
    int *zi = nullptr, *zj = nullptr, *zk = nullptr;
    float *zv = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pa));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pb));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pz));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(nnz_a, 1)), &ka));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(nnz_b, 1)), &kb));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zi));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zj));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zk));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zv));
    const hipStream_t s = call.stream();
    NACHO_TRY(call.timer_start(name));
    const unsigned ga = ceil_div(static_cast<size_t>(nnz_a) / kRowOffsetsPer + 1, 256);
    const unsigned gb = ceil_div(static_cast<size_t>(nnz_b) / kRowOffsetsPer + 1, 256);
    const KeysJob ja{a->dim_i_indices, a->dim_j_indices, a->dim_k_indices, nnz_a, pa, ka};
    const KeysJob jb{b->dim_i_indices, b->dim_j_indices, b->dim_k_indices, nnz_b, pb, kb};
    coo3_keys_kernel<<<ga + gb, 256, 0, s>>>(ja, jb, static_cast<int>(ga), rows, kbits);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());  // (kernel timing only) before the merge's own interval
    const csr::LevelOperand A{pa, ka, a->values, nnz_a, nullptr};
    const csr::LevelOperand B{pb, kb, b->values, nnz_b, nullptr};
    const csr::LevelResult Z{pz, zj, zv, nullptr, nullptr, zi, zk, kbits};
    long long nnz = 0;
    NACHO_TRY(csr::merge_level(call, false, true, false, rows, A, B, Z, &nnz, name));
    if (nnz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nnz == 0) {
        call.drop_result(zi);
        call.drop_result(zj);
        call.drop_result(zk);
        call.drop_result(zv);
        zi = zj = zk = nullptr;
        zv = nullptr;
    }
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_k_size = a->dim_k_size;
    z->dim_i_length = static_cast<int32_t>(nnz);
    z->dim_i_indices = zi;
    z->dim_j_length = static_cast<int32_t>(nnz);
    z->dim_j_indices = zj;
    z->dim_k_length = static_cast<int32_t>(nnz);
    z->dim_k_indices = zk;
    z->values = zv;
    z->nnz = static_cast<int32_t>(nnz);
    call.commit();
    return NACHO_OK;
}

bool bad_coo(const nacho_coo *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->nnz < 0) return true;
    if (t->dim_i_length != t->nnz || t->dim_j_length != t->nnz) return true;
    if (t->nnz > 0 && (!t->dim_i_indices || !t->dim_j_indices || !t->values)) return true;
    return false;
}

bool bad_coo3(const nacho_coo3 *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_k_size < 0 || t->nnz < 0) {
        return true;
    }
    if (t->dim_i_length != t->nnz || t->dim_j_length != t->nnz || t->dim_k_length != t->nnz) {
        return true;
    }
    if (t->nnz > 0 && (!t->dim_i_indices || !t->dim_j_indices || !t->dim_k_indices || !t->values)) {
        return true;
    }
    return false;
}

// ---- CSR + COO, and the COO3 inner product ------------------------------------------------

// Z = a + b for a CSR a and a COO b (compiler.cpp:122): b's row offsets are built from its i
// coordinates (coo_row_offsets_kernel) and the CSR level union merges the two as csr_add
// does, so the result is the CSR that csr_add gives for a and b converted to CSR.
int coo_csr_add(const nacho_csr *a, const nacho_coo *b, nacho_csr *z, int32_t nb, int32_t tpb,
                void *stream, const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(check_launch_hints(nb, tpb));
    if (csr::bad_csr(a) || bad_coo(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size;
    const long long nnz_a = a->dim_j_length, nnz_b = b->nnz;
    if (nnz_a + nnz_b + rows > static_cast<long long>(INT_MAX) - 2 * csr::kLevelTileSlack) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }
    const long long cap = nnz_a + nnz_b;
    Call call(stream, alloc);
    int *pb = nullptr, *pc = nullptr, *cc = nullptr;
    float *vc = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pb));
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &cc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &vc));
    const hipStream_t s = call.stream();
    NACHO_TRY(call.timer_start("coo_csr_add"));
    const unsigned gb = ceil_div(static_cast<size_t>(nnz_b) / kRowOffsetsPer + 1, 256);
    const RowOffsetsJob jb{b->dim_i_indices, static_cast<int>(nnz_b), pb};
    coo_row_offsets_kernel<<<gb, 256, 0, s>>>(jb, jb, 0, rows);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());  // (kernel timing only) before the merge's own interval
    const csr::LevelOperand A{a->dim_j_offsets, a->dim_j_indices, a->values,
                              a->dim_j_length, nullptr};
    const csr::LevelOperand B{pb, b->dim_j_indices, b->values, b->nnz, nullptr};
    const csr::LevelResult Z{pc, cc, vc, nullptr, nullptr};
    long long nnz = 0;
    NACHO_TRY(csr::merge_level(call, false, true, false, rows, A, B, Z, &nnz, "coo_csr_add"));
    if (nnz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nnz == 0) {
        call.drop_result(cc);
        call.drop_result(vc);
        cc = nullptr;
        vc = nullptr;
    }
    z->dim_i_size = rows;
    z->dim_j_size = a->dim_j_size;
    z->dim_j_offsets = pc;
    z->dim_j_length = static_cast<int32_t>(nnz);
    z->dim_j_indices = cc;
    z->values = vc;
    z->nnz = static_cast<int32_t>(nnz);
    call.commit();
    return NACHO_OK;
}

// Releases a buffer that an entry point returned to the caller, on `stream`, by the rule the
// call that allocated it followed: an allocator without `allocate` means the library's own
// allocator, and an allocator without `release` keeps its buffers.
static void release_result(void *ptr, void *stream, const nacho_allocator *alloc) {
    if (!ptr) return;
    if (alloc && alloc->allocate) {
        if (alloc->release) alloc->release(alloc->ctx, ptr, stream);
    } else {
        (void)nacho_free(ptr, stream);
    }
}

// z = sum of a * b over the (i, j, k) both COO3 operands hold (compiler.cpp:143).  When the
// (j, k) keys fit (as for coo3d_add), both operands become rows i of column keys
// (coo3_keys_kernel) and the CSR level intersection sums its products (LevelResult::dot).
// Otherwise the packed-tuple intersection computes the products, which are then summed.
int coo3_inner_prod(const nacho_coo3 *a, const nacho_coo3 *b, nacho_scalar *z, int32_t nb,
                    int32_t tpb, void *stream, const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_scalar{};
    if (bad_coo3(a) || bad_coo3(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size ||
        a->dim_k_size != b->dim_k_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    NACHO_TRY(check_launch_hints(nb, tpb));
    const long long entries = static_cast<long long>(a->nnz) + b->nnz;
    const int kbits = bits_for_extent(a->dim_k_size);
    const bool keys_fit = a->dim_j_size >= 1 && a->dim_k_size >= 1 &&
                          bits_for_extent(a->dim_j_size) + kbits <= 31 &&
                          ((static_cast<long long>(a->dim_j_size - 1) << kbits) |
                           (a->dim_k_size - 1)) < INT_MAX;
    if (keys_fit &&
        entries + a->dim_i_size <= static_cast<long long>(INT_MAX) - 2 * csr::kLevelTileSlack &&
        a->dim_i_size <= kRowPathRowsPerEntry * entries + (1 << 20)) {
        const int rows = a->dim_i_size;
        const int nnz_a = a->nnz, nnz_b = b->nnz;
        Call call(stream, alloc);
        float *value = nullptr;
        int *pa = nullptr, *pb = nullptr, *ka = nullptr, *kb = nullptr;
        NACHO_TRY(call.result_n(1, &value));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pa));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pb));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(nnz_a, 1)), &ka));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(nnz_b, 1)), &kb));
        const hipStream_t s = call.stream();
        NACHO_TRY(call.timer_start("inner_prod_coo"));
        const unsigned ga = ceil_div(static_cast<size_t>(nnz_a) / kRowOffsetsPer + 1, 256);
        const unsigned gb = ceil_div(static_cast<size_t>(nnz_b) / kRowOffsetsPer + 1, 256);
        const KeysJob ja{a->dim_i_indices, a->dim_j_indices, a->dim_k_indices, nnz_a, pa, ka};
        const KeysJob jb{b->dim_i_indices, b->dim_j_indices, b->dim_k_indices, nnz_b, pb, kb};
        coo3_keys_kernel<<<ga + gb, 256, 0, s>>>(ja, jb, static_cast<int>(ga), rows, kbits);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.collect_timer());  // (kernel timing only) before the merge's interval
        const csr::LevelOperand A{pa, ka, a->values, nnz_a, nullptr};
        const csr::LevelOperand B{pb, kb, b->values, nnz_b, nullptr};
        csr::LevelResult Z{nullptr, nullptr, nullptr, nullptr, nullptr};
        Z.dot = value;
        long long unused = 0;
        NACHO_TRY(csr::merge_level(call, true, true, false, rows, A, B, Z, &unused,
                                   "inner_prod_coo"));
        z->values = value;
        z->nnz = 1;
        call.commit();
        return NACHO_OK;
    }
    // packed-tuple intersection, then the sum of its values
    const int32_t extents[3] = {a->dim_i_size, a->dim_j_size, a->dim_k_size};
    int32_t *out[3] = {nullptr, nullptr, nullptr};
    float *val = nullptr;
    int32_t n = 0;
    NACHO_TRY(coo_binary<Op::Intersect>(
        3, extents, Coords{a->dim_i_indices, a->dim_j_indices, a->dim_k_indices}, a->values,
        a->nnz, Coords{b->dim_i_indices, b->dim_j_indices, b->dim_k_indices}, b->values, b->nnz,
        nb, tpb, stream, alloc, "inner_prod_coo (tuple intersection)", out, &val, &n));
    int rc = NACHO_OK;
    float *value = nullptr;
    {
        Call call(stream, alloc);
        rc = call.result_n(1, &value);
        if (rc == NACHO_OK) rc = csr::sum_values(call, val, n, value);
        if (rc == NACHO_OK) call.commit();
    }
    for (int d = 0; d < 3; ++d) release_result(out[d], stream, alloc);
    release_result(val, stream, alloc);
    if (rc != NACHO_OK) return rc;
    z->values = value;
    z->nnz = 1;
    return NACHO_OK;
}

template <Op OP>
int coo2(const nacho_coo *a, const nacho_coo *b, nacho_coo *z, int32_t nb, int32_t tpb,
         void *stream, const nacho_allocator *alloc, const char *name) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_coo{};
    if (bad_coo(a) || bad_coo(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    NACHO_TRY(check_launch_hints(nb, tpb));
    const long long entries = static_cast<long long>(a->nnz) + b->nnz;
    if (entries + a->dim_i_size <= static_cast<long long>(INT_MAX) - 2 * csr::kLevelTileSlack &&
        a->dim_i_size <= kRowPathRowsPerEntry * entries + (1 << 20)) {
        return coo2_rows<OP>(a, b, z, stream, alloc, name);
    }
    const int32_t extents[3] = {a->dim_i_size, a->dim_j_size, 0};
    int32_t *out[3];
    float *val = nullptr;
    int32_t n = 0;
    NACHO_TRY(coo_binary<OP>(2, extents, Coords{a->dim_i_indices, a->dim_j_indices, nullptr},
                             a->values, a->nnz, Coords{b->dim_i_indices, b->dim_j_indices, nullptr},
                             b->values, b->nnz, nb, tpb, stream, alloc, name, out, &val, &n));
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_i_length = n;
    z->dim_i_indices = out[0];
    z->dim_j_length = n;
    z->dim_j_indices = out[1];
    z->values = val;
    z->nnz = n;
    return NACHO_OK;
}

}  // namespace coo
}  // namespace nacho

extern "C" {

int nacho_gpu_coo_add_f32(const nacho_coo *a, const nacho_coo *b, nacho_coo *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::coo::coo2<nacho::coo::Op::Union>(a, b, z, num_blocks, threads_per_block, stream,
                                                   alloc, "coo_merge_tile_kernel<Union>");
}

int nacho_gpu_coo_mul_f32(const nacho_coo *a, const nacho_coo *b, nacho_coo *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::coo::coo2<nacho::coo::Op::Intersect>(a, b, z, num_blocks, threads_per_block,
                                                       stream, alloc,
                                                       "coo_merge_tile_kernel<Intersect>");
}

int nacho_gpu_coo_csr_add_f32(const nacho_csr *a, const nacho_coo *b, nacho_csr *z,
                              int32_t num_blocks, int32_t threads_per_block, void *stream,
                              const nacho_allocator *alloc) {
    return nacho::coo::coo_csr_add(a, b, z, num_blocks, threads_per_block, stream, alloc);
}

int nacho_gpu_inner_prod_coo_f32(const nacho_coo3 *a, const nacho_coo3 *b, nacho_scalar *z,
                                 int32_t num_blocks, int32_t threads_per_block, void *stream,
                                 const nacho_allocator *alloc) {
    return nacho::coo::coo3_inner_prod(a, b, z, num_blocks, threads_per_block, stream, alloc);
}

int nacho_gpu_coo3d_add_f32(const nacho_coo3 *a, const nacho_coo3 *b, nacho_coo3 *z,
                            int32_t num_blocks, int32_t threads_per_block, void *stream,
                            const nacho_allocator *alloc) {
    using namespace nacho::coo;
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_coo3{};
    if (bad_coo3(a) || bad_coo3(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size ||
        a->dim_k_size != b->dim_k_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    NACHO_TRY(nacho::check_launch_hints(num_blocks, threads_per_block));
    const long long entries = static_cast<long long>(a->nnz) + b->nnz;
    // the row path's column keys stay below INT_MAX, the merge's exhausted-row sentinel
    const int kbits = bits_for_extent(a->dim_k_size);
    const bool keys_fit = a->dim_j_size >= 1 && a->dim_k_size >= 1 &&
                          bits_for_extent(a->dim_j_size) + kbits <= 31 &&
                          ((static_cast<long long>(a->dim_j_size - 1) << kbits) |
                           (a->dim_k_size - 1)) < INT_MAX;
    if (keys_fit &&
        entries + a->dim_i_size <= static_cast<long long>(INT_MAX) - 2 * nacho::csr::kLevelTileSlack &&
        a->dim_i_size <= kRowPathRowsPerEntry * entries + (1 << 20)) {
        return coo3_rows(a, b, z, stream, alloc, kbits, "coo3d_add (row offsets + CSR merge)");
    }
    const int32_t extents[3] = {a->dim_i_size, a->dim_j_size, a->dim_k_size};
    int32_t *out[3];
    float *val = nullptr;
    int32_t n = 0;
    NACHO_TRY(coo_binary<Op::Union>(
        3, extents, Coords{a->dim_i_indices, a->dim_j_indices, a->dim_k_indices}, a->values, a->nnz,
        Coords{b->dim_i_indices, b->dim_j_indices, b->dim_k_indices}, b->values, b->nnz, num_blocks,
        threads_per_block, stream, alloc, "coo_merge_tile_kernel<Union,3>", out, &val, &n));
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_k_size = a->dim_k_size;
    z->dim_i_length = n;
    z->dim_i_indices = out[0];
    z->dim_j_length = n;
    z->dim_j_indices = out[1];
    z->dim_k_length = n;
    z->dim_k_indices = out[2];
    z->values = val;
    z->nnz = n;
    return NACHO_OK;
}

}  // extern "C"
