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
constexpr int kItemsPerLane = 15;  // odd: lanes' LDS walks spread over banks
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

// Tile inputs staged in LDS: A's crd/val range then B's, and one packed word per row of the
// tile: (max(posA[r], a0) - a0) | (max(posB[r], b0) - b0) << 16.
struct TileSplit {
    int r0, a0, b0, r1, a1, b1;
};

__device__ __forceinline__ TileSplit load_split(const int *__restrict__ split_r,
                                                const int *__restrict__ split_a,
                                                const int *__restrict__ split_b, int tile) {
    return TileSplit{split_r[tile], split_a[tile], split_b[tile],
                     split_r[tile + 1], split_a[tile + 1], split_b[tile + 1]};
}

// Registers of one lane's share of a tile's staged inputs (prefetched one tile ahead).
template <int LOADS>
struct Staged {
    int crd[LOADS];
    float val[LOADS];
    unsigned row[LOADS];
};

template <bool VALUES, int LOADS>
__device__ __forceinline__ void fetch_tile(Staged<LOADS> &st, const TileSplit &sp,
                                           const int *__restrict__ pa, const int *__restrict__ ca,
                                           const float *__restrict__ va,
                                           const int *__restrict__ pb, const int *__restrict__ cb,
                                           const float *__restrict__ vb, int tid) {
    const int na = sp.a1 - sp.a0, nab = na + (sp.b1 - sp.b0), nr = sp.r1 - sp.r0 + 1;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int k = tid + j * kBlock;
        if (k < na) {
            st.crd[j] = ca[sp.a0 + k];
            if (VALUES) st.val[j] = va[sp.a0 + k];
        } else if (k < nab) {
            st.crd[j] = cb[sp.b0 + k - na];
            if (VALUES) st.val[j] = vb[sp.b0 + k - na];
        }
        if (k < nr) {
            const unsigned ra = static_cast<unsigned>(max(pa[sp.r0 + k], sp.a0) - sp.a0);
            const unsigned rb = static_cast<unsigned>(max(pb[sp.r0 + k], sp.b0) - sp.b0);
            st.row[j] = ra | (rb << 16);
        }
    }
}

template <bool VALUES, int LOADS>
__device__ __forceinline__ void stage_tile(const Staged<LOADS> &st, const TileSplit &sp,
                                           int *s_crd, float *s_val, unsigned *s_row, int tid) {
    const int nab = (sp.a1 - sp.a0) + (sp.b1 - sp.b0), nr = sp.r1 - sp.r0 + 1;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int k = tid + j * kBlock;
        if (k < nab) {
            s_crd[k] = st.crd[j];
            if (VALUES) s_val[k] = st.val[j];
        }
        if (k < nr) s_row[k] = st.row[j];
    }
}

// Persistent merge kernel.  Each workgroup takes tiles in ticket order; while it computes
// tile T it already holds the inputs of its next tile N in registers and the split of the
// tile after that, so global-memory latency overlaps computation.
//
// Inside a tile, lane t owns the items [tile_lo + t*IPT, tile_lo + (t+1)*IPT) of the
// merged sequence (lane 0 starts at the tile's own split, the last lane ends at the next
// tile's), found by a merge-path search in LDS.  It walks exactly those items in a fixed,
// unrolled number of steps: take A's head (ties: A first), take B's head, or consume the
// row-end item.  An equal A/B pair is combined when its A entry is taken (the B head is
// peeked) and the B entry is skipped when its turn comes, so a pair may straddle two
// lanes.  Outputs stay in registers with a validity mask until their global offset is known.
template <Op OP, int IPT>
__global__ __launch_bounds__(kBlock) void csr_merge_tile_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const float *__restrict__ va,
    const int *__restrict__ pb, const int *__restrict__ cb, const float *__restrict__ vb,
    int num_tiles, const int *__restrict__ split_r, const int *__restrict__ split_a,
    const int *__restrict__ split_b, unsigned long long *__restrict__ status,
    unsigned *__restrict__ info, int rows, int *__restrict__ pc, int *__restrict__ cc,
    float *__restrict__ vc) {
    constexpr int kTileItems = kBlock * IPT;
    constexpr int kCap = kTileItems + 2;
    constexpr int kLoads = (kCap + kBlock - 1) / kBlock;
    constexpr int kSteps = IPT + 1;
    constexpr int kMax = INT_MAX;  // sentinel head: row exhausted
    static_assert(kCap < 65536, "row offsets are packed in 16 bits");
    static_assert(kSteps <= 32, "masks are 32-bit");

    __shared__ int s_crd[kCap];
    __shared__ float s_val[kCap];
    __shared__ unsigned s_row[kCap];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_next, s_base;

    const int tid = threadIdx.x;
    if (tid == 0) s_next = static_cast<int>(atomicAdd(&info[kInfoTicket], 1u));
    __syncthreads();
    int cur = s_next;
    if (cur >= num_tiles) return;
    TileSplit sp = load_split(split_r, split_a, split_b, cur);
    Staged<kLoads> st;
    fetch_tile<true, kLoads>(st, sp, pa, ca, va, pb, cb, vb, tid);
    __syncthreads();  // every lane has read s_next
    stage_tile<true, kLoads>(st, sp, s_crd, s_val, s_row, tid);
    if (tid == 0) s_next = static_cast<int>(atomicAdd(&info[kInfoTicket], 1u));
    __syncthreads();
    int nxt = s_next;
    TileSplit nsp = sp;
    if (nxt < num_tiles) nsp = load_split(split_r, split_a, split_b, nxt);

    while (true) {
        // Prefetch the next tile's inputs and take the ticket after it.
        if (nxt < num_tiles) fetch_tile<true, kLoads>(st, nsp, pa, ca, va, pb, cb, vb, tid);
        unsigned ticket2 = 0;
        if (tid == 0) ticket2 = atomicAdd(&info[kInfoTicket], 1u);

        const int r0 = sp.r0, a0 = sp.a0, b0 = sp.b0, r1 = sp.r1, a1 = sp.a1, b1 = sp.b1;
        const int na = a1 - a0, nr = r1 - r0 + 1;
        const int tile_lo = cur * kTileItems;
        const int tile_start = a0 + b0 + r0;  // item index of the tile's first item
        const int tile_end = a1 + b1 + r1;    // one past its last item
        auto A = [&](int x) { return s_crd[x - a0]; };
        auto B = [&](int y) { return s_crd[na + y - b0]; };
        auto row_a = [&](int k) { return a0 + static_cast<int>(s_row[k] & 0xffffu); };
        auto row_b = [&](int k) { return b0 + static_cast<int>(s_row[k] >> 16); };

        // This lane's first item and its split (r, a, b).
        const int g_lo = tid == 0 ? tile_start : tile_lo + tid * IPT;
        const int g_hi = min(tile_lo + (tid + 1) * IPT, tile_end);
        const int steps = tid == kBlock - 1 ? tile_end - g_lo : g_hi - g_lo;
        int k = 0, a = a0, b = b0;
        if (tid > 0 && g_lo < tile_end) {
            int lo = 0, hi = nr - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (row_a(mid) + row_b(mid) + r0 + mid <= g_lo) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            k = lo;
            const int aS = row_a(k), bS = row_b(k);
            const int aE = k < nr - 1 ? row_a(k + 1) : a1;
            const int bE = k < nr - 1 ? row_b(k + 1) : b1;
            const int D = g_lo - (r0 + k);
            int slo = max(aS, D - bE), shi = min(aE, D - bS);
            while (slo < shi) {
                const int mid = (slo + shi) >> 1;
                if (A(mid) <= B(D - 1 - mid)) {
                    slo = mid + 1;
                } else {
                    shi = mid;
                }
            }
            a = slo;
            b = D - slo;
        }
        const int rs = r0 + k;  // first row this lane touches
        int aE = k < nr - 1 ? row_a(k + 1) : a1;
        int bE = k < nr - 1 ? row_b(k + 1) : b1;
        int last_a = a > row_a(k) ? A(a - 1) : -1;  // previous A of this row inside the tile
        int xa = a < aE ? A(a) : kMax;
        int xb = b < bE ? B(b) : kMax;

        int out_crd[kSteps];
        float out_val[kSteps];
        unsigned valid = 0, row_ends = 0;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            out_crd[s] = 0;
            out_val[s] = 0.0f;
            if (s < steps) {
                if (xa != kMax || xb != kMax) {
                    if (xa <= xb) {  // take A
                        const bool pair = (xa == xb);
                        float v = 0.0f;
                        if (OP == Op::Union) {
                            v = s_val[a - a0];
                            if (pair) v = v + s_val[na + b - b0];
                        } else if (pair) {
                            v = s_val[a - a0] * s_val[na + b - b0];
                        }
                        out_crd[s] = xa;
                        out_val[s] = v;
                        if (OP == Op::Union || pair) valid |= 1u << s;
                        last_a = xa;
                        ++a;
                        xa = a < aE ? A(a) : kMax;
                    } else {  // take B; skipped when it was combined with the previous A
                        if (OP == Op::Union && last_a != xb) {
                            out_crd[s] = xb;
                            out_val[s] = s_val[na + b - b0];
                            valid |= 1u << s;
                        }
                        ++b;
                        xb = b < bE ? B(b) : kMax;
                    }
                } else {  // row end
                    row_ends |= 1u << s;
                    ++k;
                    aE = k < nr - 1 ? row_a(k + 1) : a1;
                    bE = k < nr - 1 ? row_b(k + 1) : b1;
                    last_a = -1;
                    xa = a < aE ? A(a) : kMax;
                    xb = b < bE ? B(b) : kMax;
                }
            }
        }

        const int count = __popc(valid);
        int tile_total = 0;
        if (tid == 0) s_next = static_cast<int>(ticket2);
        const int offset = dev::block_exclusive_sum<kBlock>(count, s_wave, tile_total);
        if (tid < dev::kWave) {
            const uint32_t base = dev::lookback_exclusive(
                status, cur, static_cast<uint32_t>(tile_total), &info[kInfoError]);
            if (tid == 0) s_base = static_cast<int>(base);
        }
        __syncthreads();
        const int base = s_base;
        const int nxt2 = s_next;
        TileSplit nsp2 = nsp;
        if (nxt2 < num_tiles) nsp2 = load_split(split_r, split_a, split_b, nxt2);
        if (cur == 0 && tid == 0) pc[0] = 0;

        // Row ends: pos[r+1] = global offset of the first output after row r.  Outputs are
        // staged in LDS (the inputs are no longer read) for coalesced stores.
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const unsigned below = (1u << s) - 1u;
            if (row_ends & (1u << s)) {
                const int r = rs + __popc(row_ends & below);
                const int at = base + offset + __popc(valid & below);
                pc[r + 1] = at;
                if (r + 1 == rows) info[kInfoLength] = static_cast<unsigned>(at);
            }
            if (valid & (1u << s)) {
                const int o = offset + __popc(valid & below);
                s_crd[o] = out_crd[s];
                s_val[o] = out_val[s];
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int o = tid + j * kBlock;
            if (o < tile_total) {
                cc[base + o] = s_crd[o];
                vc[base + o] = s_val[o];
            }
        }
        if (nxt >= num_tiles) break;
        __syncthreads();  // staged outputs consumed
        stage_tile<true, kLoads>(st, nsp, s_crd, s_val, s_row, tid);
        __syncthreads();
        cur = nxt;
        sp = nsp;
        nxt = nxt2;
        nsp = nsp2;
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
    auto kernel = csr_merge_tile_kernel<OP, kItemsPerLane>;
    int resident = 0;
    NACHO_TRY(resident_grid(reinterpret_cast<const void *>(kernel), kBlock, &resident));
    const int grid = num_tiles < resident ? num_tiles : resident;
    NACHO_TRY(call.timer_start(kernel_name));
    kernel<<<grid, kBlock, 0, s>>>(a->dim_j_offsets, a->dim_j_indices, a->values,
                                   b->dim_j_offsets, b->dim_j_indices, b->values, num_tiles,
                                   split_r, split_a, split_b, status, info, rows, pc, cc, vc);
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
