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
// The work is the merged sequence of both key lists (nnzA + nnzB items).  A partition
// kernel finds every tile's merge-path split (equal keys never split, as the reference's
// balancing step, partition.cpp:964-983); one workgroup per tile stages its keys and values
// in LDS with coalesced loads, splits among lanes in LDS, counts, takes its global offset by
// decoupled look-back, merges again into LDS and writes the unpacked coordinates and values
// coalesced.  Values are one IEEE binary32 add / multiply or a copy, as the reference's
// lattice (compute.cpp:476-491), so results are bit-exact.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "device_utils.hpp"
#include "runtime.hpp"

namespace nacho {
namespace coo {

enum class Op { Union, Intersect };

constexpr int kBlock = 256;
constexpr int kItemsPerLane = 8;
constexpr int kTile = kBlock * kItemsPerLane;
constexpr int kInfoWords = 4;
constexpr int kInfoTicket = 0, kInfoLength = 1, kInfoError = 2;

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

template <typename Codec>
__global__ __launch_bounds__(256) void coo_partition_kernel(Codec codec, Coords ca, int nnz_a,
                                                            Coords cb, int nnz_b, int num_tiles,
                                                            int *__restrict__ split_a,
                                                            int *__restrict__ split_b,
                                                            unsigned long long *__restrict__ status,
                                                            unsigned *__restrict__ info) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < kInfoWords) info[t] = 0u;
    if (t < num_tiles) status[t] = 0ull;
    if (t > num_tiles) return;
    const int total = nnz_a + nnz_b;
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);
    int a, b;
    merge_split([&](int x) { return codec.load(ca, x); }, [&](int y) { return codec.load(cb, y); },
                0, nnz_a, 0, nnz_b, diag, a, b);
    split_a[t] = a;
    split_b[t] = b;
}

template <Op OP, typename Codec>
__global__ __launch_bounds__(kBlock) void coo_merge_tile_kernel(
    Codec codec, Coords ca, const float *__restrict__ va, int nnz_a, Coords cb,
    const float *__restrict__ vb, int nnz_b, const int *__restrict__ split_a,
    const int *__restrict__ split_b, unsigned long long *__restrict__ status,
    unsigned *__restrict__ info, int num_tiles, int *__restrict__ zi, int *__restrict__ zj,
    int *__restrict__ zk, float *__restrict__ zv) {
    using Key = typename Codec::Key;
    constexpr int kCap = kTile + 2;
    constexpr int kLoads = kItemsPerLane + 1;
    static_assert(kLoads * kBlock >= kCap, "staging loop too short");

    __shared__ Key s_key[kCap];  // A's range then B's range
    __shared__ float s_val[kCap];
    __shared__ Key s_okey[kCap];
    __shared__ float s_oval[kCap];
    __shared__ int s_sa[kBlock + 1], s_sb[kBlock + 1];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_tile, s_base;

    const int tid = threadIdx.x;
    if (tid == 0) s_tile = static_cast<int>(atomicAdd(&info[kInfoTicket], 1u));
    __syncthreads();
    const int tile = s_tile;
    const int a0 = split_a[tile], b0 = split_b[tile];
    const int a1 = split_a[tile + 1], b1 = split_b[tile + 1];
    const int na = a1 - a0, nab = na + (b1 - b0);
    const int total = nnz_a + nnz_b;
    const int tile_lo = tile * kTile;
    const int tile_hi = min(tile_lo + kTile, total);

    {
        Key rk[kLoads];
        float rv[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int k = tid + j * kBlock;
            if (k < na) {
                rk[j] = codec.load(ca, a0 + k);
                rv[j] = va[a0 + k];
            } else if (k < nab) {
                rk[j] = codec.load(cb, b0 + k - na);
                rv[j] = vb[b0 + k - na];
            }
        }
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int k = tid + j * kBlock;
            if (k < nab) {
                s_key[k] = rk[j];
                s_val[k] = rv[j];
            }
        }
    }
    __syncthreads();

    auto A = [&](int x) { return s_key[x - a0]; };
    auto B = [&](int y) { return s_key[na + y - b0]; };
    {
        const int g = tile_lo + tid * kItemsPerLane;
        int a, b;
        if (tid == 0) {
            a = a0;
            b = b0;
        } else if (g >= tile_hi) {
            a = a1;
            b = b1;
        } else {
            merge_split(A, B, a0, a1, b0, b1, g, a, b);
        }
        s_sa[tid] = a;
        s_sb[tid] = b;
        if (tid == 0) {
            s_sa[kBlock] = a1;
            s_sb[kBlock] = b1;
        }
    }
    __syncthreads();
    const int as = s_sa[tid], bs = s_sb[tid], ae = s_sa[tid + 1], be = s_sb[tid + 1];

    auto walk = [&](auto emit) {
        int a = as, b = bs;
        while (a < ae && b < be) {
            const Key x = A(a), y = B(b);
            if (x < y) {
                if (OP == Op::Union) emit(x, a, -1);
                ++a;
            } else if (y < x) {
                if (OP == Op::Union) emit(y, -1, b);
                ++b;
            } else {
                emit(x, a, b);
                ++a;
                ++b;
            }
        }
        if (OP == Op::Union) {
            for (; a < ae; ++a) emit(A(a), a, -1);
            for (; b < be; ++b) emit(B(b), -1, b);
        }
    };

    int count = 0;
    walk([&](const Key &, int, int) { ++count; });
    int tile_total = 0;
    const int offset = dev::block_exclusive_sum<kBlock>(count, s_wave, tile_total);
    if (tid < dev::kWave) {
        const uint32_t base = dev::lookback_exclusive(status, tile, static_cast<uint32_t>(tile_total),
                                                      &info[kInfoError]);
        if (tid == 0) s_base = static_cast<int>(base);
    }
    __syncthreads();
    const int base = s_base;
    if (tile == num_tiles - 1 && tid == 0) info[kInfoLength] = static_cast<unsigned>(base + tile_total);

    int o = offset;
    walk([&](const Key &key, int ia, int ib) {
        float v;
        if (ia >= 0 && ib >= 0) {
            const float p = s_val[ia - a0], q = s_val[na + ib - b0];
            v = (OP == Op::Union) ? (p + q) : (p * q);
        } else {
            v = (ia >= 0) ? s_val[ia - a0] : s_val[na + ib - b0];
        }
        s_okey[o] = key;
        s_oval[o] = v;
        ++o;
    });
    __syncthreads();

#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int k = tid + j * kBlock;
        if (k < tile_total) {
            int ci, cj, ck;
            codec.unpack(s_okey[k], ci, cj, ck);
            zi[base + k] = ci;
            zj[base + k] = cj;
            if (codec.arity == 3) zk[base + k] = ck;
            zv[base + k] = s_oval[k];
        }
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
    unsigned long long *status = nullptr;
    int *splits = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles) + kInfoWords / 2, &status));
    NACHO_TRY(call.scratch_n(2 * (static_cast<size_t>(num_tiles) + 1), &splits));
    unsigned *info = reinterpret_cast<unsigned *>(status + num_tiles);
    int *split_a = splits, *split_b = splits + num_tiles + 1;

    int32_t *z[3] = {nullptr, nullptr, nullptr};
    float *zv = nullptr;
    for (int d = 0; d < arity; ++d) NACHO_TRY(call.result_n(static_cast<size_t>(cap), &z[d]));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &zv));

    const hipStream_t s = call.stream();
    const unsigned part_grid = ceil_div(static_cast<size_t>(num_tiles) + 1, 256);
    const int bi = bits_for_extent(extents[0]), bj = bits_for_extent(extents[1]);
    const int bk = arity == 3 ? bits_for_extent(extents[2]) : 0;
    auto launch = [&](auto codec) -> int {
        using Codec = decltype(codec);
        coo_partition_kernel<Codec><<<part_grid, 256, 0, s>>>(codec, ca, nnz_a, cb, nnz_b, num_tiles,
                                                              split_a, split_b, status, info);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_start(kernel_name));
        coo_merge_tile_kernel<OP, Codec><<<num_tiles, kBlock, 0, s>>>(
            codec, ca, va, nnz_a, cb, vb, nnz_b, split_a, split_b, status, info, num_tiles, z[0],
            z[1], z[2], zv);
        NACHO_TRY_HIP(hipGetLastError());
        return call.timer_stop();
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

    unsigned words[kInfoWords] = {};
    NACHO_TRY(call.read_back(words, info, sizeof(words)));
    if (words[kInfoError] != 0) return NACHO_ERR_INTERNAL;
    const long long nnz = words[kInfoLength];
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

template <Op OP>
int coo2(const nacho_coo *a, const nacho_coo *b, nacho_coo *z, int32_t nb, int32_t tpb,
         void *stream, const nacho_allocator *alloc, const char *name) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_coo{};
    if (bad_coo(a) || bad_coo(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
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
