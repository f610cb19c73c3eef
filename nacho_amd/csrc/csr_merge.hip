// CSR elementwise add (union) and multiply (intersection) for gfx950.
//
// Reference path replaced: the generated partition_ij / precompute_ij / compute_ij kernels
// of csr_add and csr_mul (src/backend/partition.cpp:59-336, 813-993;
// src/backend/compute.cpp:151-395, 619-1388) and their host orchestration
// (src/backend/stitch_and_generate.cpp:8-112, 438-527; stitch_and_generate_gpu.cpp:379-715).
// The reference runs one thread per merge-path partition with a serial, uncoalesced merge,
// a count pass, a CUB scan, a blocking length readback and a write pass.  Here:
//
//  * Work is the merged sequence of every row's A entries, B entries and one row-end item,
//    so empty rows and Zipf-heavy rows cost the same per item (the reference counts only
//    nonzeros, tensor.cpp:308-413).  Item count T = nnzA + nnzB + rows.
//  * csr_partition_kernel: one thread per tile boundary finds (row, a, b) for diagonal
//    tile*TILE by a binary search over rows on S(r) = posA[r] + posB[r] + r, then a merge-path
//    search inside the row.  An A/B pair with equal coordinates is never split across tiles
//    (the reference's balancing step, partition.cpp:964-983).  The same kernel clears the
//    look-back status words and the tile ticket, so no memset is needed.
//  * csr_merge_tile_kernel: one workgroup per tile of BLOCK*IPT items.  It stages the tile's
//    crd/val ranges of A and B and its rows' pos entries in LDS with coalesced loads, splits
//    the tile among lanes by the same search in LDS, counts outputs, turns counts into global
//    offsets with a workgroup scan plus decoupled look-back (single pass, no second read of
//    crd), merges again writing results into LDS, and stores crd/val with coalesced writes.
//    Row ends write pos[r+1].
//
// Emission order and values follow the reference's lattice (compute.cpp:476-491,
// 1169-1198, 1297-1337): coordinates ascending within a row; union emits a+b where both
// exist and a copy otherwise; intersection emits a*b only where both exist.  Explicit zeros
// are kept.  Each value is one IEEE binary32 operation, so results are bit-identical to the
// reference's.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "device_utils.hpp"
#include "runtime.hpp"

namespace nacho {
namespace csr {

enum class Op { Union, Intersect };

constexpr int kBlock = 256;
constexpr int kItemsPerLane = 8;
constexpr int kTile = kBlock * kItemsPerLane;

// Per-call info words in scratch, cleared by the partition kernel:
// [0] tile ticket, [1] result length, [2] error flag (look-back gave up).
constexpr int kInfoWords = 4;
constexpr int kInfoTicket = 0, kInfoLength = 1, kInfoError = 2;

// Merge-path split of the merged order of A[aS, aE) and B[bS, bE) (ties: A first) at the
// point where `a + b == D`, followed by the pair rule: if the last A taken equals the next B,
// that B joins this side.  `A(x)` and `B(y)` read coordinates by absolute position.
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

// One thread per tile boundary t in [0, num_tiles]: split of diagonal min(t*TILE, total).
__global__ __launch_bounds__(256) void csr_partition_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, int rows, int total, int num_tiles, int *__restrict__ split_r,
    int *__restrict__ split_a, int *__restrict__ split_b, unsigned long long *__restrict__ status,
    unsigned *__restrict__ info) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < kInfoWords) info[t] = 0u;
    if (t < num_tiles) status[t] = 0ull;
    if (t > num_tiles) return;
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);

    // Largest row r in [0, rows] with S(r) <= diag.
    int lo = 0, hi = rows;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pa[mid] + pb[mid] + mid <= diag) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    const int r = lo;
    int a, b;
    if (r == rows) {
        a = pa[rows];
        b = pb[rows];
    } else {
        const int D = diag - r;  // a + b at the split, in absolute positions
        merge_split([&](int x) { return ca[x]; }, [&](int y) { return cb[y]; }, pa[r], pa[r + 1],
                    pb[r], pb[r + 1], D, a, b);
    }
    split_r[t] = r;
    split_a[t] = a;
    split_b[t] = b;
}

template <Op OP>
__global__ __launch_bounds__(kBlock) void csr_merge_tile_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const float *__restrict__ va,
    const int *__restrict__ pb, const int *__restrict__ cb, const float *__restrict__ vb,
    int total, const int *__restrict__ split_r, const int *__restrict__ split_a,
    const int *__restrict__ split_b, unsigned long long *__restrict__ status,
    unsigned *__restrict__ info, int rows, int *__restrict__ pc, int *__restrict__ cc,
    float *__restrict__ vc) {
    constexpr int kCap = kTile + 2;
    constexpr int kLoads = kItemsPerLane + 1;  // ceil(kCap / kBlock)
    static_assert(kLoads * kBlock >= kCap, "staging loop too short");

    __shared__ int s_crd[kCap];  // A's range then B's range
    __shared__ float s_val[kCap];
    __shared__ int s_pa[kCap];  // pos entries of rows r0..r1
    __shared__ int s_pb[kCap];
    __shared__ int s_oc[kCap];  // staged output
    __shared__ float s_ov[kCap];
    __shared__ int s_sr[kBlock + 1], s_sa[kBlock + 1], s_sb[kBlock + 1];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_tile, s_base;

    const int tid = threadIdx.x;
    if (tid == 0) s_tile = static_cast<int>(atomicAdd(&info[kInfoTicket], 1u));
    __syncthreads();
    const int tile = s_tile;

    const int r0 = split_r[tile], a0 = split_a[tile], b0 = split_b[tile];
    const int r1 = split_r[tile + 1], a1 = split_a[tile + 1], b1 = split_b[tile + 1];
    const int na = a1 - a0, nb = b1 - b0, nab = na + nb, nr = r1 - r0 + 1;
    const int tile_lo = tile * kTile;
    const int tile_hi = min(tile_lo + kTile, total);

    // Stage crd/val of A[a0,a1) ++ B[b0,b1) and pos[r0..r1] of both; loads first, then LDS
    // stores, so every load of a lane is in flight at once.
    {
        int rc[kLoads];
        float rv[kLoads];
        int rpa[kLoads], rpb[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int k = tid + j * kBlock;
            if (k < na) {
                rc[j] = ca[a0 + k];
                rv[j] = va[a0 + k];
            } else if (k < nab) {
                rc[j] = cb[b0 + k - na];
                rv[j] = vb[b0 + k - na];
            }
            if (k < nr) {
                rpa[j] = pa[r0 + k];
                rpb[j] = pb[r0 + k];
            }
        }
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int k = tid + j * kBlock;
            if (k < nab) {
                s_crd[k] = rc[j];
                s_val[k] = rv[j];
            }
            if (k < nr) {
                s_pa[k] = rpa[j];
                s_pb[k] = rpb[j];
            }
        }
    }
    __syncthreads();

    auto A = [&](int x) { return s_crd[x - a0]; };
    auto B = [&](int y) { return s_crd[na + y - b0]; };

    // This lane's starting split: diagonal tile_lo + tid*IPT, found in LDS.
    {
        const int g = tile_lo + tid * kItemsPerLane;
        int r, a, b;
        if (tid == 0) {
            r = r0;
            a = a0;
            b = b0;
        } else if (g >= tile_hi) {
            r = r1;
            a = a1;
            b = b1;
        } else {
            int lo = 0, hi = nr - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_pa[mid] + s_pb[mid] + r0 + mid <= g) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            const int k = lo;
            r = r0 + k;
            const int aS = max(s_pa[k], a0), bS = max(s_pb[k], b0);
            const int aE = (k < nr - 1) ? s_pa[k + 1] : a1;
            const int bE = (k < nr - 1) ? s_pb[k + 1] : b1;
            merge_split(A, B, aS, aE, bS, bE, g - r, a, b);
        }
        s_sr[tid] = r;
        s_sa[tid] = a;
        s_sb[tid] = b;
        if (tid == 0) {
            s_sr[kBlock] = r1;
            s_sa[kBlock] = a1;
            s_sb[kBlock] = b1;
        }
    }
    __syncthreads();

    const int rs = s_sr[tid], as = s_sa[tid], bs = s_sb[tid];
    const int re = s_sr[tid + 1], ae = s_sa[tid + 1], be = s_sb[tid + 1];

    // Walk this lane's share: merge each row's A and B runs, then its row-end item, up to the
    // next lane's split.  `emit(crd, ia, ib)` gets absolute positions (-1 = absent);
    // `row_end(r)` fires when row r's end item is consumed.
    auto walk = [&](auto emit, auto row_end) {
        int r = rs, a = as, b = bs;
        while (true) {
            const int k = r - r0;
            const bool last = r >= re;
            const int aEnd = last ? ae : s_pa[k + 1];
            const int bEnd = last ? be : s_pb[k + 1];
            while (a < aEnd && b < bEnd) {
                const int x = A(a), y = B(b);
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
                for (; a < aEnd; ++a) emit(A(a), a, -1);
                for (; b < bEnd; ++b) emit(B(b), -1, b);
            }
            if (last) break;
            row_end(r);
            ++r;
            a = aEnd;
            b = bEnd;
        }
    };

    int count = 0;
    walk([&](int, int, int) { ++count; }, [&](int) {});

    int tile_total = 0;
    const int offset = dev::block_exclusive_sum<kBlock>(count, s_wave, tile_total);
    if (tid < dev::kWave) {
        const uint32_t base =
            dev::lookback_exclusive(status, tile, static_cast<uint32_t>(tile_total),
                                    &info[kInfoError]);
        if (tid == 0) s_base = static_cast<int>(base);
    }
    __syncthreads();
    const int base = s_base;
    if (tile == 0 && tid == 0) pc[0] = 0;

    int o = offset;
    walk(
        [&](int x, int ia, int ib) {
            float v;
            if (ia >= 0 && ib >= 0) {
                const float p = s_val[ia - a0], q = s_val[na + ib - b0];
                v = (OP == Op::Union) ? (p + q) : (p * q);
            } else {
                v = (ia >= 0) ? s_val[ia - a0] : s_val[na + ib - b0];
            }
            s_oc[o] = x;
            s_ov[o] = v;
            ++o;
        },
        [&](int r) {
            pc[r + 1] = base + o;
            if (r + 1 == rows) info[kInfoLength] = static_cast<unsigned>(base + o);
        });
    __syncthreads();

#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int k = tid + j * kBlock;
        if (k < tile_total) {
            cc[base + k] = s_oc[k];
            vc[base + k] = s_ov[k];
        }
    }
}

bool bad_csr(const nacho_csr *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0) return true;
    if (!t->dim_j_offsets) return true;
    if (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values)) return true;
    return false;
}

template <Op OP>
int csr_binary(const nacho_csr *a, const nacho_csr *b, nacho_csr *z, int32_t num_blocks,
               int32_t threads_per_block, void *stream, const nacho_allocator *alloc,
               const char *kernel_name) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csr(a) || bad_csr(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size;
    const long long nnz_a = a->dim_j_length, nnz_b = b->dim_j_length;
    const long long total = nnz_a + nnz_b + rows;
    if (total > static_cast<long long>(INT_MAX) - 2 * kTile) return NACHO_ERR_INDEX_OVERFLOW;
    const long long cap = (OP == Op::Union) ? nnz_a + nnz_b : (nnz_a < nnz_b ? nnz_a : nnz_b);
    const int num_tiles = total > 0 ? static_cast<int>((total + kTile - 1) / kTile) : 1;

    Call call(stream, alloc);
    unsigned long long *status = nullptr;
    int *splits = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles) + kInfoWords / 2, &status));
    NACHO_TRY(call.scratch_n(3 * (static_cast<size_t>(num_tiles) + 1), &splits));
    unsigned *info = reinterpret_cast<unsigned *>(status + num_tiles);
    int *split_r = splits, *split_a = splits + num_tiles + 1, *split_b = splits + 2 * (num_tiles + 1);

    int *pc = nullptr, *cc = nullptr;
    float *vc = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &cc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &vc));

    const hipStream_t s = call.stream();
    csr_partition_kernel<<<ceil_div(static_cast<size_t>(num_tiles) + 1, 256), 256, 0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, b->dim_j_offsets, b->dim_j_indices, rows,
        static_cast<int>(total), num_tiles, split_r, split_a, split_b, status, info);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_start(kernel_name));
    csr_merge_tile_kernel<OP><<<num_tiles, kBlock, 0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, a->values, b->dim_j_offsets, b->dim_j_indices,
        b->values, static_cast<int>(total), split_r, split_a, split_b, status, info, rows, pc, cc,
        vc);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());

    unsigned words[kInfoWords] = {};
    NACHO_TRY(call.read_back(words, info, sizeof(words)));
    if (words[kInfoError] != 0) return NACHO_ERR_INTERNAL;
    const long long nnz = words[kInfoLength];
    if (nnz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nnz == 0) {
        // Empty result: zeroed offsets, no coordinate/value buffers
        // (stitch_and_generate.cpp:168-220 for the intersection early exit).
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

}  // namespace csr
}  // namespace nacho

extern "C" {

int nacho_gpu_csr_add_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::csr::csr_binary<nacho::csr::Op::Union>(a, b, z, num_blocks, threads_per_block,
                                                         stream, alloc, "csr_merge_tile_kernel<Union>");
}

int nacho_gpu_csr_mul_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::csr::csr_binary<nacho::csr::Op::Intersect>(
        a, b, z, num_blocks, threads_per_block, stream, alloc, "csr_merge_tile_kernel<Intersect>");
}

}  // extern "C"
