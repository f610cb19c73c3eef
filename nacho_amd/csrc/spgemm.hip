// ESC SpGEMM (Z_ik = sum_j A_ij B_jk, CSR x CSR -> CSR) for gfx950 with 64-bit product and
// result offsets.
//
// Reference path replaced: the spgemm kernel (compiler.cpp:145-148), lowered as a scatter
// reduction (compile.cpp:40-72): an expand phase partitioned over the intermediate-product
// count (compile.cpp:122-221, partition.cpp:1039-1193), then CUB DeviceSegmentedSort by column
// within each row, mark_heads / InclusiveSum / extract_offsets and a warp-32 segmented scan
// with atomicAdd (stitch_and_generate_gpu.cpp:14-138, 257-366).  The reference keeps every
// count in int32, which the R-MAT scale-20 square (6.0e9 products, 3.6e9 results) overflows.
//
// Pipeline (every count and offset is int64):
//   1. sizes: len[p] = |row crdA[p] of B| per A entry; exclusive scan -> off[p], P = off[nnzA];
//      row i's products are [row_off[i], row_off[i+1]) in natural (j, k) order.
//   2. segments: a row with at most kShort products is one segment.  A longer row is split by
//      column into nb buckets of 2^shift columns (one device-wide radix digit, k >> shift);
//      each bucket is a segment.  Segments are numbered row-major, bucket-minor, so their
//      concatenation in order is every row's products grouped by column range.
//   3. expand to runs: a product (k, a_ij * b_jk) is never written to memory.  B's rows are
//      cut into runs of equal column bucket; a segment's products are the concatenation of
//      its runs, each run one A entry times a contiguous range of one B row, described by
//      {first B entry, length, a_ij} (a short row's runs are its A entries' whole B rows, in
//      natural order; a long row's runs of bucket b come from B's run table).  A histogram
//      over B's runs gives each long-row segment's products and runs without visiting a
//      product; scans give segment product offsets and run offsets; the run descriptors are
//      then written per segment (4.4e8 of 16 bytes at C4, against 6.0e9 products of 8).
//   4. units: a segment with more than kShort products is a dense unit; smaller segments
//      whose first product falls in the same kShort-aligned window share one sort unit
//      (fewer than 2*kShort products), or one bitmap unit when they are at most
//      kMaxBitmapBuckets narrow column buckets of long rows.  Each kind gets a compacted list.
//   5. reduce: a unit expands its runs, gathering (k, a_ij * b_jk) from B.  A sort unit sorts
//      (segment ordinal, k) in LDS and sums each run of equal keys in float64; a bitmap unit
//      ranks each bucket's columns in an LDS bitmap and sums by rank; a dense unit accumulates
//      its 2^shift-column range in an LDS float64 array (windows of kDenseCols columns) and
//      compacts the touched columns in order.  All write the distinct (k, sum rounded once to
//      float32) at the unit's product offset in an output staging buffer and record the
//      unit's count and the local offset of every row starting in it.
//   6. output, sized one of two ways (output_mode).  Staged: the units write at their product
//      offsets in a staging buffer; a scan of unit counts gives result offsets, each unit's
//      entries are copied, row offsets come from the unit offsets.  Symbolic (columns below
//      2^20): before the runs, a symbolic pass counts every segment's distinct columns from
//      A and B (long rows in an LDS bitmap of the row's columns, short rows in a per-wave LDS
//      hash table); their scan gives segment and row offsets, the result is allocated at its
//      exact size and the units write straight into it.  Every distinct column is kept
//      (structural result, as the reference).
// Summation order inside a segment follows the runs' order and LDS atomics, so values are
// reproducible to within one float32 rounding of the float64 sum (the reference's own order
// is not deterministic either).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "device_utils.hpp"
#include "runtime.hpp"
#include "scan.hpp"

namespace nacho {
namespace spgemm {

constexpr int kBlock = 256;
constexpr int kTile = 4096;             // LDS capacity of a sort unit
constexpr int kPer = kTile / kBlock;    // 16 positions per lane
constexpr int kShort = kTile / 2;       // segments with at most this many products are sorted
constexpr int kOrdBits = 12;            // a sort unit holds fewer than 2^12 segments
constexpr int kDenseBits = 13;          // dense accumulation window: 8192 columns
constexpr int kDenseCols = 1 << kDenseBits;
constexpr int kMaxBucketBits = 10;      // at most 1024 column buckets per long row
constexpr int kMaxBuckets = 1 << kMaxBucketBits;
// A long row's bucket with more products than this is accumulated densely (its 8192-column
// window in LDS) rather than by a bitmap or sort unit.  At C4, 1536 / 2048 (one box, two
// rounds): 95.46 / 95.45 against 96.66 / 95.98 ms; 1024 and 1280 lose.
constexpr int kDenseMin = 1536;
constexpr int kMaxBitmapSegs = 256;     // segments (empty ones included) of a bitmap unit
constexpr int kMaxBitmapBuckets = 32;   // nonempty buckets of a bitmap unit (larger buckets)
constexpr int kBitmapWords = 8192 / 32; // one bit per column of an 8192-column bucket
constexpr int kBitmapBlock = 512;       // threads of a bitmap unit's workgroup
constexpr int kHistGrid = 8192;         // workgroups of the long-row histogram
// Units in list order on one XCD at a time, kXcdGroup consecutive ones per XCD: a long row's
// neighbouring buckets gather adjacent ranges of the same B rows, which then share one L2.
// At C4 the unit kernels fetched 124 -> 105 GB per call (96.97 -> 95.58 ms) with groups of
// 64; one contiguous range per XCD fetched as little but took 102.2 ms (the XCDs' loads no
// longer matched).  Groups of 128 / 256 against 64, one box, two rounds each: 96.10 / 95.88,
// 95.67 / 95.54 against 96.66 / 95.98 ms.
constexpr unsigned kXcdGroup = 256;

static_assert(kTile == 1 << kOrdBits, "segment ordinals must fit kOrdBits");
static_assert(kTile == kBlock * kPer, "a unit's products are kPer per lane");

// ---- small device helpers --------------------------------------------------------------

// LDS index with one pad word per kPer words: a lane's kPer consecutive (blocked) positions
// then start kPer + 1 words after its neighbour's, so blocked accesses are free of bank
// conflicts.
constexpr int kPadded = kTile + kTile / 16;
__device__ __forceinline__ int pad(int i) { return i + (i >> 4); }

using dev::block_exclusive_max;
using dev::last_le;

// ---- 1-2: sizes and segments -----------------------------------------------------------

__global__ void lengths_kernel(const int *__restrict__ crd_a, int64_t nnz_a,
                               const int *__restrict__ pos_b, int64_t *__restrict__ len) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < nnz_a;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int j = crd_a[p];
        len[p] = static_cast<int64_t>(pos_b[j + 1] - pos_b[j]);
    }
}

// row_off[i] = off[posA[i]]; seg_count[i] = segments of row i (1, or nb for a long row).
__global__ void rows_kernel(const int *__restrict__ pos_a, int rows,
                            const int64_t *__restrict__ off, int nb,
                            int64_t *__restrict__ row_off, int64_t *__restrict__ seg_count) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= rows; i += gridDim.x * blockDim.x) {
        row_off[i] = off[pos_a[i]];
        if (i < rows) {
            const int64_t prod = off[pos_a[i + 1]] - off[pos_a[i]];
            seg_count[i] = prod > kShort ? nb : 1;
        }
    }
}

// Segment table: row of each segment, product and run counts (short rows known now: one run
// per A entry whose B row is not empty; long rows counted by the histogram pass) and the
// zeroed fill counters of the long rows' run emission.
__global__ void segments_kernel(const int64_t *__restrict__ row_off,
                                const int64_t *__restrict__ seg_prefix, int rows,
                                const int *__restrict__ pos_a, const int64_t *__restrict__ len,
                                int *__restrict__ seg_row, int64_t *__restrict__ seg_len,
                                int64_t *__restrict__ seg_runs, int64_t *__restrict__ seg_fill) {
    // One row per lane; a long row's segments (one per column bucket) are then written by
    // the whole wavefront, 64 consecutive segments per store, instead of by its own lane.
    const int l = dev::lane();
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + (threadIdx.x - l);
         i0 < rows; i0 += stride) {  // uniform per wavefront
        const int i = static_cast<int>(i0) + l;
        int64_t s0 = 0, s1 = 0, runs = 0, prod = 0;
        if (i < rows) {
            s0 = seg_prefix[i];
            s1 = seg_prefix[i + 1];
            prod = row_off[i + 1] - row_off[i];
            if (prod > 0 && prod <= kShort) {
                for (int p = pos_a[i]; p < pos_a[i + 1]; ++p) runs += len[p] > 0 ? 1 : 0;
            }
            if (s1 - s0 == 1) {  // a short row's single segment
                seg_row[s0] = i;
                seg_len[s0] = prod > kShort ? 0 : prod;
                seg_runs[s0] = runs;
                seg_fill[s0] = 0;
            }
        }
        unsigned long long many = __ballot(i < rows && s1 - s0 > 1);
        while (many) {  // uniform
            const int src = __ffsll(static_cast<long long>(many)) - 1;
            many &= many - 1;
            const int64_t a0 = __shfl(s0, src, dev::kWave), a1 = __shfl(s1, src, dev::kWave);
            const int row = __shfl(i, src, dev::kWave);
            const int64_t plen = __shfl(prod, src, dev::kWave);
            const int64_t prun = __shfl(runs, src, dev::kWave);
            for (int64_t sg = a0 + l; sg < a1; sg += dev::kWave) {
                seg_row[sg] = row;
                seg_len[sg] = plen > kShort ? 0 : plen;
                seg_runs[sg] = prun;
                seg_fill[sg] = 0;
            }
        }
    }
}

// ---- 3a: long-row histogram from B's column-bucket runs --------------------------------
//
// Long rows need their products counted per column bucket before the scatter.  B's rows
// have sorted columns, so each B row is a short list of runs of equal bucket (at most nb,
// however long the row); a long row's bucket counts are the sums of its B rows' run
// lengths.  At C4 (R-MAT 2^20, 128 buckets) this is 4.3e8 run visits instead of 5.9e9
// products.

// flag[p] = 1 where B entry p starts a run: its bucket differs from entry p - 1's.  Row
// starts are flagged by run_row_starts_kernel, launched after this one.
__global__ void run_flags_kernel(const int *__restrict__ crd_b, int64_t nnz_b, int shift,
                                 int64_t *__restrict__ flag) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < nnz_b;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        flag[p] = (p == 0 || (crd_b[p] >> shift) != (crd_b[p - 1] >> shift)) ? 1 : 0;
    }
}

__global__ void run_row_starts_kernel(const int *__restrict__ pos_b, int rows_b,
                                      int64_t *__restrict__ flag) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows_b; r += gridDim.x * blockDim.x) {
        if (pos_b[r] < pos_b[r + 1]) flag[pos_b[r]] = 1;
    }
}

// Run q (numbered by the exclusive scan run_idx of the flags): its bucket (run[q].x) and
// its first B entry; run_start[total runs] = nnz_b closes the last run.  B row k's runs are
// [run_idx[pos_b[k]], run_idx[pos_b[k + 1]]).
__global__ void runs_kernel(const int *__restrict__ crd_b, int64_t nnz_b, int shift,
                            const int64_t *__restrict__ flag, const int64_t *__restrict__ run_idx,
                            int2 *__restrict__ run, int *__restrict__ run_start) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < nnz_b;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (flag[p]) {
            const int64_t q = run_idx[p];
            run[q].x = crd_b[p] >> shift;
            run_start[q] = static_cast<int>(p);
        }
        if (p == 0) run_start[run_idx[nnz_b]] = static_cast<int>(nnz_b);
    }
}

// run[q].y = the length of run q (runs numbered below run_idx[nnz_b]).
__global__ void run_lengths_kernel(const int64_t *__restrict__ run_idx, int64_t nnz_b,
                                   const int *__restrict__ run_start, int2 *__restrict__ run) {
    const int64_t n_runs = run_idx[nnz_b];
    for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < n_runs;
         q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        run[q].y = run_start[q + 1] - run_start[q];
    }
}

// Work blocks of the histogram: kBlock consecutive A entries of one long row.
// nblk[i] = blocks of row i (0 for a short row).
__global__ void hist_blocks_kernel(const int *__restrict__ pos_a, int rows,
                                   const int64_t *__restrict__ row_off,
                                   int64_t *__restrict__ nblk) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += gridDim.x * blockDim.x) {
        const int len = pos_a[i + 1] - pos_a[i];
        nblk[i] = row_off[i + 1] - row_off[i] > kShort ? (len + kBlock - 1) / kBlock : 0;
    }
}

// blk_row[b] = the row of work block b (blocks numbered by the scan blk_off of nblk).
__global__ void hist_rows_kernel(const int64_t *__restrict__ blk_off, int rows,
                                 int *__restrict__ blk_row) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += gridDim.x * blockDim.x) {
        for (int64_t b = blk_off[i]; b < blk_off[i + 1]; ++b) blk_row[b] = i;
    }
}

// B row k's runs, packed (bucket, length) in run[] and first entries in run_start[].
struct BRuns {
    const int64_t *run_idx;  // B row k's runs are [run_idx[pos_b[k]], run_idx[pos_b[k + 1]])
    const int2 *run;
    const int *run_start;
};

// The runs of a work block's A entries, dealt evenly over the workgroup: an A entry's B row
// may hold one run or a hundred (a hub), so one lane per entry leaves most lanes of a
// wavefront waiting for its longest.  Every lane publishes its entry's run count, first run
// and A value; the block's T runs (entry by entry) are then taken kRunsPer per lane per
// round, run j by lane j mod kBlock, which finds the entry owning j with a fixed eight-step
// search of the entries' run offsets in LDS (the kRunsPer searches interleaved).
constexpr int kRunsPer = 4;

struct BlockRuns {
    int off[kBlock];      // exclusive scan of the entries' run counts
    int64_t q0[kBlock];   // first run of the entry's B row in br.run
    float a[kBlock];      // the entry's A value
    int wave[kBlock / dev::kWave];
};

// Publishes this lane's entry (n_runs runs from q0, A value a); returns T.  Ends synchronised.
__device__ __forceinline__ int publish_runs(BlockRuns &sh, int n_runs, int64_t q0, float a) {
    int total = 0;
    const int off = dev::block_exclusive_sum<kBlock>(n_runs, sh.wave, total);
    sh.off[threadIdx.x] = off;
    sh.q0[threadIdx.x] = q0;
    sh.a[threadIdx.x] = a;
    __syncthreads();
    return total;
}

// Run j of the block (j < T): its index in br.run and its entry's A value.
__device__ __forceinline__ void block_run(const BlockRuns &sh, int j, int64_t &q, float &a) {
    int lo = 0;  // last entry whose first run is at or before j (off[0] = 0)
#pragma unroll
    for (int step = kBlock / 2; step > 0; step >>= 1) {
        lo += sh.off[lo + step] <= j ? step : 0;
    }
    q = sh.q0[lo] + (j - sh.off[lo]);
    a = sh.a[lo];
}

// Work blocks strided over the grid (a heavy row's blocks land on different workgroups):
// every thread takes one A entry of the block and adds, per run of its B row, the run's
// length and one run to LDS histograms of the row's buckets; nonzero bins are then added to
// the row's seg_len and seg_runs (zeroed by segments_kernel), stored directly when the row
// has a single block.
__global__ __launch_bounds__(kBlock) void long_hist_kernel(
    const int *__restrict__ pos_a, const int *__restrict__ crd_a,
    const int64_t *__restrict__ blk_off, const int *__restrict__ blk_row, int rows,
    const int *__restrict__ pos_b, BRuns br, int nb, const int64_t *__restrict__ seg_prefix,
    int64_t *__restrict__ seg_len, int64_t *__restrict__ seg_runs) {
    __shared__ int s_hist[kMaxBuckets];
    __shared__ int s_runs[kMaxBuckets];
    __shared__ BlockRuns sh;
    const int64_t n_blk = blk_off[rows];
    for (int64_t blk = blockIdx.x; blk < n_blk; blk += gridDim.x) {
        const int i = blk_row[blk];
        const int64_t first = blk_off[i];
        for (int b = threadIdx.x; b < nb; b += kBlock) {
            s_hist[b] = 0;
            s_runs[b] = 0;
        }
        const int p = pos_a[i] + static_cast<int>(blk - first) * kBlock + threadIdx.x;
        int64_t q0 = 0;
        int n_runs = 0;
        if (p < pos_a[i + 1]) {
            const int k = crd_a[p];
            q0 = br.run_idx[pos_b[k]];
            n_runs = static_cast<int>(br.run_idx[pos_b[k + 1]] - q0);
        }
        // (its barriers also order the clears above before the adds below)
        const int T = publish_runs(sh, n_runs, q0, 0.0f);
        for (int j0 = 0; j0 < T; j0 += kRunsPer * kBlock) {  // uniform
            int2 x[kRunsPer];
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                int64_t q;
                float a;
                block_run(sh, min(j0 + u * kBlock + static_cast<int>(threadIdx.x), T - 1), q, a);
                x[u] = br.run[q];
            }
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                if (j0 + u * kBlock + static_cast<int>(threadIdx.x) < T && x[u].x < nb) {
                    atomicAdd(&s_hist[x[u].x], x[u].y);
                    atomicAdd(&s_runs[x[u].x], 1);
                }
            }
        }
        __syncthreads();
        const int64_t s0 = seg_prefix[i];
        const bool alone = blk_off[i + 1] - first == 1;
        for (int b = threadIdx.x; b < nb; b += kBlock) {
            const int c = s_hist[b], n = s_runs[b];
            if (alone) {
                seg_len[s0 + b] = c;
                seg_runs[s0 + b] = n;
            } else if (c > 0) {
                atomicAdd(reinterpret_cast<unsigned long long *>(&seg_len[s0 + b]),
                          static_cast<unsigned long long>(c));
                atomicAdd(reinterpret_cast<unsigned long long *>(&seg_runs[s0 + b]),
                          static_cast<unsigned long long>(n));
            }
        }
        __syncthreads();  // the histograms are read before the next block clears them
    }
}

// B's columns and value bits as one array of pairs, read by the reduce units' gathers.
__global__ void interleave_kernel(const int *__restrict__ crd_b, const float *__restrict__ val_b,
                                  int64_t nnz_b, int2 *__restrict__ cv_b) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < nnz_b;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        cv_b[p] = make_int2(crd_b[p], __float_as_int(val_b[p]));
    }
}

// ---- 3b: run descriptors -----------------------------------------------------------------

// A run of products: B entries [x, x + y) times the A value with bits z (w unused).
__device__ __forceinline__ int4 make_run(int first, int length, float a) {
    return make_int4(first, length, __float_as_int(a), 0);
}

// Long rows: the same work blocks as the histogram.  Each bucket's runs from the block are
// counted in LDS, a range of the segment's run slots is reserved with one atomic per
// nonempty bucket (none when the row has a single block), and every run is written at the
// next slot of its bucket's range.  The order of runs inside a segment is free: the reduce
// is order-independent (up to float64 rounding).  (Staging a block's runs in LDS to store
// each bucket's range coalesced cost more in occupancy than it saved: 8.4 -> 12.6 ms at C4.)
__global__ __launch_bounds__(kBlock) void long_runs_kernel(
    const int *__restrict__ pos_a, const int *__restrict__ crd_a, const float *__restrict__ val_a,
    const int64_t *__restrict__ blk_off, const int *__restrict__ blk_row, int rows,
    const int *__restrict__ pos_b, BRuns br, int nb, const int64_t *__restrict__ seg_prefix,
    const int64_t *__restrict__ seg_roff, int64_t *__restrict__ seg_fill,
    int4 *__restrict__ desc) {
    __shared__ int s_cnt[kMaxBuckets];
    __shared__ int64_t s_base[kMaxBuckets];
    __shared__ BlockRuns sh;
    const int64_t n_blk = blk_off[rows];
    for (int64_t blk = blockIdx.x; blk < n_blk; blk += gridDim.x) {
        const int i = blk_row[blk];
        const int64_t first = blk_off[i];
        for (int b = threadIdx.x; b < nb; b += kBlock) s_cnt[b] = 0;
        const int p = pos_a[i] + static_cast<int>(blk - first) * kBlock + threadIdx.x;
        int64_t q0 = 0;
        int n_runs = 0;
        float a_mine = 0.0f;
        if (p < pos_a[i + 1]) {
            const int k = crd_a[p];
            a_mine = val_a[p];
            q0 = br.run_idx[pos_b[k]];
            n_runs = static_cast<int>(br.run_idx[pos_b[k + 1]] - q0);
        }
        // (its barriers also order the clears above before the counts below)
        const int T = publish_runs(sh, n_runs, q0, a_mine);
        for (int j0 = 0; j0 < T; j0 += kRunsPer * kBlock) {  // uniform
            int2 x[kRunsPer];
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                int64_t q;
                float a;
                block_run(sh, min(j0 + u * kBlock + static_cast<int>(threadIdx.x), T - 1), q, a);
                x[u] = br.run[q];
            }
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                if (j0 + u * kBlock + static_cast<int>(threadIdx.x) < T && x[u].x < nb) {
                    atomicAdd(&s_cnt[x[u].x], 1);
                }
            }
        }
        __syncthreads();
        const int64_t s0 = seg_prefix[i];
        const bool alone = blk_off[i + 1] - first == 1;
        for (int b = threadIdx.x; b < nb; b += kBlock) {
            const int c = s_cnt[b];
            int64_t at = 0;
            if (c > 0 && !alone) {
                at = static_cast<int64_t>(atomicAdd(
                    reinterpret_cast<unsigned long long *>(&seg_fill[s0 + b]),
                    static_cast<unsigned long long>(c)));
            }
            s_base[b] = seg_roff[s0 + b] + at;
            s_cnt[b] = 0;
        }
        __syncthreads();
        for (int j0 = 0; j0 < T; j0 += kRunsPer * kBlock) {  // uniform
            int2 x[kRunsPer];
            int first_b[kRunsPer];
            float av[kRunsPer];
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                int64_t q;
                block_run(sh, min(j0 + u * kBlock + static_cast<int>(threadIdx.x), T - 1), q,
                          av[u]);
                x[u] = br.run[q];
                first_b[u] = br.run_start[q];
            }
#pragma unroll
            for (int u = 0; u < kRunsPer; ++u) {
                if (j0 + u * kBlock + static_cast<int>(threadIdx.x) < T && x[u].x < nb) {
                    const int64_t slot = s_base[x[u].x] + atomicAdd(&s_cnt[x[u].x], 1);
                    desc[slot] = make_run(first_b[u], x[u].y, av[u]);
                }
            }
        }
        __syncthreads();  // s_cnt, s_base and sh are read before the next block resets them
    }
}

// Short rows: one run per A entry whose B row is not empty, in natural order (the row's
// products in their natural order).  One thread per row.
__global__ void short_runs_kernel(const int *__restrict__ pos_a, const int *__restrict__ crd_a,
                                  const float *__restrict__ val_a, int rows,
                                  const int64_t *__restrict__ row_off,
                                  const int64_t *__restrict__ seg_prefix,
                                  const int64_t *__restrict__ seg_roff,
                                  const int *__restrict__ pos_b, int4 *__restrict__ desc) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += gridDim.x * blockDim.x) {
        const int64_t prod = row_off[i + 1] - row_off[i];
        if (prod == 0 || prod > kShort) continue;
        int64_t slot = seg_roff[seg_prefix[i]];
        for (int p = pos_a[i]; p < pos_a[i + 1]; ++p) {
            const int k = crd_a[p];
            const int b0 = pos_b[k], b1 = pos_b[k + 1];
            if (b1 > b0) desc[slot++] = make_run(b0, b1 - b0, val_a[p]);
        }
    }
}

// A unit's products, expanded from its runs desc[r0, r0 + R) (in segment order): run r
// contributes (cv_b[q].x, a_r * cv_b[q].y) for q in [first_r, first_r + length_r) (cv_b: B's
// columns and value bits interleaved, so a lane's consecutive products are one contiguous
// span of 8-byte pairs), and the unit's
// products [0, n) are the runs' products concatenated.  Lane t of the BLOCK-thread workgroup
// receives positions [t * PER, (t + 1) * PER) in kk / vv (positions >= n repeat position
// n - 1), BLOCK * PER == kTile.  Every run has at least one product, so R <= n <= kTile.
// s_bs and s_a (R entries) and s_mark (kPadded entries) are scratch; ends synchronised, with
// the scratch free.  The product is one float32 multiply a * b, as the reference's
// a_ij * b_jk.
template <int BLOCK, int PER>
__device__ __forceinline__ void expand_runs(const int4 *__restrict__ desc, int64_t r0, int R,
                                            int n, const int2 *__restrict__ cv_b, int *s_bs,
                                            float *s_a, int *s_mark, int *s_wave,
                                            int (&kk)[PER], float (&vv)[PER]) {
    static_assert(BLOCK * PER == kTile, "a unit's products are PER per lane");
    constexpr int kPer = PER;
    const int base = threadIdx.x * kPer;
#pragma unroll
    for (int j = 0; j < kPer; ++j) s_mark[pad(base + j)] = 0;
    int4 d[kPer];
    int mine = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int r = base + j;
        d[j] = r < R ? desc[r0 + r] : make_int4(0, 0, 0, 0);
        mine += d[j].y;
    }
    int total = 0;
    // (its barriers also order the clears above before the marks below)
    int off = dev::block_exclusive_sum<BLOCK>(mine, s_wave, total);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int r = base + j;
        if (r < R) {
            s_bs[r] = d[j].x - off;  // product x of run r is B entry s_bs[r] + x
            s_a[r] = __int_as_float(d[j].z);
            if (d[j].y > 0) s_mark[pad(off)] = r + 1;
            off += d[j].y;
        }
    }
    __syncthreads();
    int m = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) m = max(m, s_mark[pad(base + j)]);
    int cur = block_exclusive_max(m, s_wave);
    int qv[kPer];
    float av[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        cur = max(cur, s_mark[pad(base + j)]);
        const int r = max(cur - 1, 0);
        qv[j] = s_bs[r] + min(base + j, n - 1);  // past n: the last run's last product
        av[j] = s_a[r];
    }
    if (n > 0) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int2 e = cv_b[qv[j]];
            kk[j] = e.x;
            vv[j] = __int_as_float(e.y);
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) vv[j] = av[j] * vv[j];
    } else {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            kk[j] = 0;
            vv[j] = 0.0f;
        }
    }
    __syncthreads();  // every lane is done with the scratch
}

// ---- 4: units --------------------------------------------------------------------------

// A segment is accumulated densely when it has more than kShort products, or more than
// dense_min products and is a column bucket of a long row (dense_min is kShort when buckets
// are wider than one kDenseCols window).  Dense accumulation costs a fixed LDS clear and
// scan of the window plus one atomic per product; sorting costs several passes per product.
__device__ __forceinline__ bool dense_segment(int64_t len, int64_t s,
                                              const int *__restrict__ seg_row,
                                              const int64_t *__restrict__ row_off,
                                              int dense_min) {
    if (len > kShort) return true;
    if (len <= dense_min) return false;
    const int r = seg_row[s];
    return row_off[r + 1] - row_off[r] > kShort;
}

// Units owned by segment s: 1 for a dense segment and for the first nonempty sorted segment
// whose products start in a kShort window (the previous nonempty segment is dense or starts
// in an earlier window); 0 otherwise.
__global__ void unit_count_kernel(const int64_t *__restrict__ seg_len,
                                  const int64_t *__restrict__ seg_off, int64_t n_seg,
                                  const int *__restrict__ seg_row,
                                  const int64_t *__restrict__ row_off, int dense_min,
                                  int64_t *__restrict__ seg_units) {
    for (int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; s < n_seg;
         s += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t len = seg_len[s], start = seg_off[s];
        int64_t u;
        if (len == 0) {
            u = 0;
        } else if (start == 0 || dense_segment(len, s, seg_row, row_off, dense_min)) {
            u = 1;
        } else {
            // previous nonempty segment: last x < s with seg_off[x] < start
            int64_t lo = 0, hi = s - 1;
            while (lo < hi) {
                const int64_t mid = (lo + hi + 1) >> 1;
                if (seg_off[mid] < start) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            const int64_t ps = seg_off[lo];
            u = (dense_segment(start - ps, lo, seg_row, row_off, dense_min) ||
                 ps / kShort != start / kShort)
                    ? 1
                    : 0;
        }
        seg_units[s] = u;
    }
}

// Unit table: first segment and product offset of each unit, and whether it is dense.
__global__ void unit_map_kernel(const int64_t *__restrict__ seg_units,
                                const int64_t *__restrict__ unit_prefix,
                                const int64_t *__restrict__ seg_off,
                                const int64_t *__restrict__ seg_len,
                                const int *__restrict__ seg_row,
                                const int64_t *__restrict__ row_off, int dense_min,
                                int64_t n_seg, int64_t P, int *__restrict__ unit_seg,
                                int64_t *__restrict__ unit_start,
                                int64_t *__restrict__ unit_dense) {
    for (int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; s <= n_seg;
         s += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (s == n_seg) {
            unit_start[unit_prefix[n_seg]] = P;
        } else if (seg_units[s]) {
            const int64_t u = unit_prefix[s];
            unit_seg[u] = static_cast<int>(s);
            unit_start[u] = seg_off[s];
            unit_dense[u] = dense_segment(seg_len[s], s, seg_row, row_off, dense_min) ? 1 : 0;
        }
    }
}

// A unit that is not dense is a bitmap unit when its buckets span at most 8192 columns and
// every one of its (at most kMaxBitmapSegs) segments is a column bucket of a long row: each
// bucket's distinct columns then fit one 8192-bit LDS bitmap.  A bitmap bucket has a fixed
// cost (clearing and scanning its bitmap), so units of many small buckets are sorted
// instead: at most kMaxBitmapBuckets nonempty buckets.  At C4 (units of about 2000
// products) the limits 16 / 32 / 64 / 256 gave a call of 99.6 / 96.6 / 96.9 / 98.0 ms.
__global__ void unit_bitmap_kernel(const int *__restrict__ unit_seg,
                                   const int64_t *__restrict__ unit_dense, int64_t n_units,
                                   int64_t n_seg, const int64_t *__restrict__ seg_len,
                                   const int *__restrict__ seg_row,
                                   const int64_t *__restrict__ row_off, bool narrow_buckets,
                                   int64_t *__restrict__ unit_bitmap) {
    for (int64_t u = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; u < n_units;
         u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t s0 = unit_seg[u];
        const int64_t s1 = u + 1 < n_units ? unit_seg[u + 1] : n_seg;
        bool ok = narrow_buckets && !unit_dense[u] && s1 - s0 <= kMaxBitmapSegs;
        int buckets = 0;
        for (int64_t s = s0; ok && s < s1; ++s) {
            if (seg_len[s] == 0) continue;
            const int r = seg_row[s];
            ok = row_off[r + 1] - row_off[r] > kShort && ++buckets <= kMaxBitmapBuckets;
        }
        unit_bitmap[u] = ok ? 1 : 0;
    }
}

// The three work lists, in unit order: each unit at its rank among units of its kind
// (dense_rank and bitmap_rank are exclusive scans of the kind flags).
__global__ void unit_lists_kernel(const int64_t *__restrict__ unit_dense,
                                  const int64_t *__restrict__ dense_rank,
                                  const int64_t *__restrict__ unit_bitmap,
                                  const int64_t *__restrict__ bitmap_rank, int64_t n_units,
                                  int *__restrict__ dense_list, int *__restrict__ bitmap_list,
                                  int *__restrict__ sort_list) {
    for (int64_t u = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; u < n_units;
         u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t rd = dense_rank[u], rb = bitmap_rank[u];
        if (unit_dense[u]) {
            dense_list[rd] = static_cast<int>(u);
        } else if (unit_bitmap[u]) {
            bitmap_list[rb] = static_cast<int>(u);
        } else {
            sort_list[u - rd - rb] = static_cast<int>(u);
        }
    }
}

// ---- 5a: sort units --------------------------------------------------------------------

// Ascending sort of one lane's kPer (key, value) pairs in registers (bitonic network with
// compile-time indices).
template <typename K>
__device__ __forceinline__ void sort_registers(K (&k)[kPer], float (&v)[kPer]) {
#pragma unroll
    for (int size = 2; size <= kPer; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool ascending = (i & size) == 0;
                    const bool swap = (k[i] > k[j]) == ascending;
                    const K ki = k[i], kj = k[j];
                    const float vi = v[i], vj = v[j];
                    k[i] = swap ? kj : ki;
                    k[j] = swap ? ki : kj;
                    v[i] = swap ? vj : vi;
                    v[j] = swap ? vi : vj;
                }
            }
        }
    }
}

// Merge-path split of output diagonal d over A[0, na) and B[0, nb), equal keys from A first:
// the number of A items among the first d outputs.
// A and B are offsets of the two runs in the padded LDS array.
template <typename K>
__device__ __forceinline__ int merge_split(const K *s_key, int A, int B, int na, int nb, int d) {
    int lo = max(0, d - nb), hi = min(d, na);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (s_key[pad(A + mid)] <= s_key[pad(B + d - 1 - mid)]) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// Ascending sort of n2 (a power of two, kPer <= n2 <= kTile) pairs: lane t holds positions
// [t*kPer, (t+1)*kPer) in k/v (registers), sorts them, then sorted runs of kPer << l are
// merged pairwise through LDS, each lane producing its kPer outputs from a merge-path split.
// On return s_key/s_val hold the sorted sequence and k/v the lane's part of it.
template <typename K>
__device__ __forceinline__ void merge_sort(K (&k)[kPer], float (&v)[kPer], K *s_key,
                                           float *s_val, int n2) {
    const int base = threadIdx.x * kPer;
    const bool active = base < n2;
    sort_registers(k, v);
    if (active) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            s_key[pad(base + u)] = k[u];
            s_val[pad(base + u)] = v[u];
        }
    }
    for (int len = kPer; len < n2; len <<= 1) {
        __syncthreads();
        const int A = base & ~(2 * len - 1);
        const int B = A + len;
        // runs already in order (typically two different segments) merge to themselves: the
        // lane's registers and LDS positions already hold its outputs
        const bool merge = active && s_key[pad(B - 1)] > s_key[pad(B)];
        if (merge) {
            int a = merge_split(s_key, A, B, len, len, base - A);
            int b = (base - A) - a;
            K ka = s_key[pad(A + min(a, len - 1))];
            K kb = s_key[pad(B + min(b, len - 1))];
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const bool take_a = a < len && (b >= len || ka <= kb);
                const int src = take_a ? A + a : B + min(b, len - 1);
                k[u] = take_a ? ka : kb;
                v[u] = s_val[pad(src)];
                a += take_a;
                b += !take_a;
                // the head that advanced, read at an index inside its run, then selected:
                // no branch whose sides wait for their own reads
                const K kn = s_key[pad(take_a ? A + min(a, len - 1) : B + min(b, len - 1))];
                ka = take_a ? kn : ka;
                kb = take_a ? kb : kn;
            }
        }
        __syncthreads();
        if (merge) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                s_key[pad(base + u)] = k[u];
                s_val[pad(base + u)] = v[u];
            }
        }
    }
    __syncthreads();
}

// Exclusive segmented sum across the workgroup's lanes.  Lane input: f = the lane holds a run
// start, s = the sum of its positions after its last start (all of them if none).  Output:
// the sum of the run open where the lane begins (from earlier lanes; 0 if none).
__device__ __forceinline__ double block_segmented_carry(bool f, double s, double *s_sum,
                                                        int *s_flag) {
    const int l = dev::lane();
    const int w = threadIdx.x / dev::kWave;
    int fi = f ? 1 : 0;
    double si = s;
#pragma unroll
    for (int o = 1; o < dev::kWave; o <<= 1) {
        const int fu = __shfl_up(fi, o, dev::kWave);
        const double su = __shfl_up(si, o, dev::kWave);
        if (l >= o) {
            if (!fi) si += su;
            fi |= fu;
        }
    }
    int fe = __shfl_up(fi, 1, dev::kWave);
    double se = __shfl_up(si, 1, dev::kWave);
    if (l == 0) {
        fe = 0;
        se = 0.0;
    }
    if (l == dev::kWave - 1) {
        s_flag[w] = fi;
        s_sum[w] = si;
    }
    __syncthreads();
    double cs = 0.0;
    for (int i = 0; i < w; ++i) cs = s_flag[i] ? s_sum[i] : cs + s_sum[i];
    __syncthreads();
    return fe ? se : cs + se;
}

// One workgroup per sort unit (from the sort list).  Sorts the unit's products by
// (segment ordinal, k), sums each run in float64, writes the distinct entries at the unit's
// start in ukey/uval, the unit's count, and (row_unit, row_local) for rows starting here.
// K is uint32_t when kOrdBits + col_shift <= 32, else uint64_t (col_shift = 32).
template <typename K>
__global__ __launch_bounds__(kBlock) void sort_unit_kernel(
    const int *__restrict__ sort_list, const int *__restrict__ unit_seg,
    const int64_t *__restrict__ unit_start, int64_t n_units,
    int64_t n_seg, const int64_t *__restrict__ seg_len, const int64_t *__restrict__ seg_off,
    const int *__restrict__ seg_row, const int64_t *__restrict__ row_off, int col_shift,
    const int4 *__restrict__ desc, const int64_t *__restrict__ seg_roff,
    const int2 *__restrict__ cv_b, int *__restrict__ ukey,
    float *__restrict__ uval, int64_t *__restrict__ unit_nnz, int *__restrict__ row_unit,
    int *__restrict__ row_local, const int64_t *__restrict__ seg_out) {
    static_assert(sizeof(K) >= sizeof(int), "run starts are staged in s_key");
    __shared__ K s_key[kPadded];
    __shared__ float s_val[kPadded];
    __shared__ int s_mark[kPadded];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ double s_sum[kBlock / dev::kWave];
    __shared__ int s_flag[kBlock / dev::kWave];
    const int64_t u = sort_list[dev::xcd_block<kXcdGroup>()];
    const int s0 = unit_seg[u];
    const int64_t start = unit_start[u];
    const int n = static_cast<int>(unit_start[u + 1] - start);
    const int64_t s_end = u + 1 < n_units ? unit_seg[u + 1] : n_seg;
    {
        // the unit's products from its runs, then staged in LDS (blocked positions)
        int kk[kPer];
        float vv[kPer];
        const int64_t r0 = seg_roff[s0];
        const int R = static_cast<int>(seg_roff[s_end] - r0);
        expand_runs<kBlock, kPer>(desc, r0, R, n, cv_b, reinterpret_cast<int *>(s_key),
                                  s_val, s_mark, s_wave, kk, vv);
        const int lo = threadIdx.x * kPer;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int q = lo + j;
            s_mark[pad(q)] = 0;
            if (q < n) {
                s_key[pad(q)] = static_cast<K>(static_cast<uint32_t>(kk[j]));
                s_val[pad(q)] = vv[j];
            }
        }
    }
    __syncthreads();
    for (int64_t s = s0 + threadIdx.x; s < s_end; s += kBlock) {
        if (seg_len[s] > 0) s_mark[pad(static_cast<int>(seg_off[s] - start))] = static_cast<int>(s) + 1;
    }
    __syncthreads();
    const int base = threadIdx.x * kPer;  // blocked positions of this lane
    int c = 0;
#pragma unroll
    for (int v = 0; v < kPer; ++v) c += s_mark[pad(base + v)] != 0;
    int total = 0;
    int ord = dev::block_exclusive_sum<kBlock>(c, s_wave, total) - 1;
    int n2 = kPer;
    while (n2 < n) n2 <<= 1;
    K rk0[kPer];
    float rv0[kPer];
#pragma unroll
    for (int v = 0; v < kPer; ++v) {
        const int q = base + v;
        ord += s_mark[pad(q)] != 0;
        rk0[v] = q < n ? (static_cast<K>(ord) << col_shift) | s_key[pad(q)] : ~static_cast<K>(0);
        rv0[v] = q < n ? s_val[pad(q)] : 0.0f;
    }
    __syncthreads();
    merge_sort(rk0, rv0, s_key, s_val, n2);
    // Segments keep their positions (sorted by ordinal first), so s_mark still marks them.
    // rk0/rv0 hold this lane's sorted positions; neighbours come from LDS.
    const K prev = base > 0 && base < n ? s_key[pad(base - 1)] : ~static_cast<K>(0);
    unsigned st = 0;
    double acc = 0.0;
#pragma unroll
    for (int v = 0; v < kPer; ++v) {
        const int q = base + v;
        const bool start_run = q < n && (q == 0 || rk0[v] != (v > 0 ? rk0[v - 1] : prev));
        if (start_run) st |= 1u << v;
        const double x = q < n ? static_cast<double>(rv0[v]) : 0.0;
        acc = start_run ? x : acc + x;
    }
    int runs = 0;
    const int rank0 =
        dev::block_exclusive_sum<kBlock>(static_cast<int>(__popc(st)), s_wave, runs);
    const double carry = block_segmented_carry(st != 0, acc, s_sum, s_flag);
    const K next = base + kPer < n ? s_key[pad(base + kPer)] : ~static_cast<K>(0);
    const K mask = (static_cast<K>(1) << col_shift) - 1;
    // second pass: each run's sum is complete at its last position; it goes to the index of
    // the run's start (one entry per run, in order)
    acc = carry;
    int idx = rank0 - 1;
    int ok[kPer];
    float ov[kPer];
    unsigned ends = 0;
    int first_end = 0;  // run index of the lane's first run end (its later ends follow)
#pragma unroll
    for (int v = 0; v < kPer; ++v) {
        const int q = base + v;
        ok[v] = 0;
        ov[v] = 0.0f;
        if (q < n) {
            const bool start_run = (st >> v) & 1u;
            if (start_run) ++idx;
            acc = start_run ? static_cast<double>(rv0[v]) : acc + static_cast<double>(rv0[v]);
            const K after = v + 1 < kPer ? rk0[v + 1] : next;
            if (q + 1 == n || after != rk0[v]) {
                if (ends == 0) first_end = idx;
                ends |= 1u << v;
                ok[v] = static_cast<int>(rk0[v] & mask);
                ov[v] = static_cast<float>(acc);
            }
            // rows starting here: the first position of their first nonempty segment
            if (s_mark[pad(q)]) {
                const int sg = s_mark[pad(q)] - 1;
                const int r = seg_row[sg];
                if (row_off[r] == seg_off[sg]) {
                    row_unit[r] = static_cast<int>(u);
                    row_local[r] = idx;
                }
            }
        }
    }
    // stage the unit's distinct entries in LDS (run j at slot j), then store them coalesced
    __syncthreads();
    int *s_ok = s_mark;
    idx = first_end;
#pragma unroll
    for (int v = 0; v < kPer; ++v) {
        if ((ends >> v) & 1u) {
            s_ok[pad(idx)] = ok[v];
            s_val[pad(idx)] = ov[v];
            ++idx;
        }
    }
    __syncthreads();
    const int64_t out = seg_out ? seg_out[s0] : start;
    for (int j = threadIdx.x; j < runs; j += kBlock) {
        ukey[out + j] = s_ok[pad(j)];
        uval[out + j] = s_val[pad(j)];
    }
    if (threadIdx.x == 0) unit_nnz[u] = runs;
}

// ---- 5b: bitmap units ------------------------------------------------------------------

using dev::wave_sync;

// Marks the columns of a bucket (window offsets s_col[x0, x1)) in bm.
__device__ __forceinline__ void mark_bucket(unsigned *bm, const unsigned short *s_col, int x0,
                                            int x1) {
    const int l = dev::lane();
#pragma unroll
    for (int i = 0; i < kBitmapWords / dev::kWave; ++i) bm[l + i * dev::kWave] = 0u;
    wave_sync();
    for (int xb = x0 + l; xb < x1; xb += 4 * dev::kWave) {  // four reads in flight
        int c[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = s_col[min(xb + j * dev::kWave, x1 - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (xb + j * dev::kWave < x1) atomicOr(&bm[c[j] >> 5], 1u << (c[j] & 31));
        }
    }
    wave_sync();
}

// One workgroup per bitmap unit; one wavefront per bucket at a time.  A bucket's distinct
// columns are the set bits of its 8192-bit window bitmap; the rank of a column (prefix
// popcount) indexes its float64 accumulator, and each product then writes its column at
// its rank, which lists the distinct columns sorted (a loop over each word's set bits
// instead cost 7.7 of the units' 40 ms at C4: a wavefront waits for its lane with the most
// bits; the products are spread evenly).  Accumulators and the listed columns of a bucket
// live in its own product range of the unit; once every bucket is done, a scan of their
// counts gives the output offsets and the workgroup stores the unit's entries with
// consecutive lanes on consecutive outputs.
__global__ __launch_bounds__(kBitmapBlock) void bitmap_unit_kernel(
    const int *__restrict__ bitmap_list, const int *__restrict__ unit_seg,
    const int64_t *__restrict__ unit_start, int64_t n_units, int64_t n_seg,
    const int64_t *__restrict__ seg_len, const int64_t *__restrict__ seg_off,
    const int64_t *__restrict__ seg_prefix, const int *__restrict__ seg_row,
    const int64_t *__restrict__ row_off, int shift, const int4 *__restrict__ desc,
    const int64_t *__restrict__ seg_roff, const int2 *__restrict__ cv_b,
    int *__restrict__ ukey, float *__restrict__ uval,
    int64_t *__restrict__ unit_nnz, int *__restrict__ row_unit, int *__restrict__ row_local,
    const int64_t *__restrict__ seg_out) {
    constexpr int kWaves = kBitmapBlock / dev::kWave;
    constexpr int kPerB = kTile / kBitmapBlock;
    __shared__ double s_acc[kTile];
    __shared__ unsigned short s_col[kTile];  // column offset inside its bucket's window
    __shared__ float s_pv[kPadded];          // product values (padded positions)
    __shared__ unsigned s_bits[kWaves][kBitmapWords];
    __shared__ int s_pre[kWaves][kBitmapWords];
    __shared__ int s_x0[kMaxBitmapSegs + 1];
    __shared__ int s_base[kMaxBitmapSegs];
    __shared__ int s_sid[kMaxBitmapSegs];
    __shared__ int s_out[kMaxBitmapSegs];
    __shared__ int s_wave[kWaves];
    __shared__ int s_next;  // the next bucket to claim
    const int64_t u = bitmap_list[dev::xcd_block<kXcdGroup>()];
    const int64_t s0 = unit_seg[u];
    const int64_t s1 = u + 1 < n_units ? unit_seg[u + 1] : n_seg;
    const int64_t start = unit_start[u];
    const int n = static_cast<int>(unit_start[u + 1] - start);
    // the unit's nonempty buckets in order (at most kMaxBitmapSegs segments: one per lane)
    const int64_t s = s0 + threadIdx.x;
    const bool here = s < s1 && seg_len[s] > 0;
    int n_buckets = 0;
    const int ord = dev::block_exclusive_sum<kBitmapBlock>(here ? 1 : 0, s_wave, n_buckets);
    if (here) {
        s_x0[ord] = static_cast<int>(seg_off[s] - start);
        s_base[ord] = static_cast<int>((s - seg_prefix[seg_row[s]]) << shift);
        s_sid[ord] = static_cast<int>(s);
    }
    if (threadIdx.x == 0) {
        s_x0[n_buckets] = n;
        s_next = kWaves;  // wavefront w starts with bucket w
    }
    // the unit's products from its runs: window offsets (bucket = column >> shift, so the
    // offset is the column's low bits) and values, staged once
    const int low = (1 << shift) - 1;
    {
        int kk[kPerB];
        float vv[kPerB];
        const int64_t r0 = seg_roff[s0];
        const int R = static_cast<int>(seg_roff[s1] - r0);
        expand_runs<kBitmapBlock, kPerB>(desc, r0, R, n, cv_b, reinterpret_cast<int *>(s_acc),
                    reinterpret_cast<float *>(s_acc) + kTile, reinterpret_cast<int *>(s_pv),
                    s_wave, kk, vv);
        const int lo = threadIdx.x * kPerB;
#pragma unroll
        for (int j = 0; j < kPerB; ++j) {
            const int q = lo + j;
            if (q < n) {
                s_col[q] = static_cast<unsigned short>(kk[j] & low);
                s_pv[pad(q)] = vv[j];
            }
        }
    }
    __syncthreads();
    const int w = threadIdx.x / dev::kWave, l = dev::lane();
    unsigned *bm = s_bits[w];
    int *pre = s_pre[w];
    // accumulate each bucket by rank; its distinct columns (window offsets, in order) and
    // their sums are left in its own product range, s_col / s_acc[x0 + rank]
    constexpr int kWordsPerLane = kBitmapWords / dev::kWave;
    // Buckets differ widely in size: a wavefront that finishes one claims the next.
    for (int o = w; o < n_buckets;) {  // uniform per wavefront
        const int x0 = s_x0[o], x1 = s_x0[o + 1];
        for (int x = x0 + l; x < x1; x += dev::kWave) s_acc[x] = 0.0;
        mark_bucket(bm, s_col, x0, x1);
        // exclusive popcount prefix per word; lane l owns words [l*4, l*4 + 4)
        int pc[kWordsPerLane];
        int mine = 0;
#pragma unroll
        for (int i = 0; i < kWordsPerLane; ++i) {
            pc[i] = __popc(bm[l * kWordsPerLane + i]);
            mine += pc[i];
        }
        const int incl = dev::wave_inclusive_sum(mine);
        int run = incl - mine;
#pragma unroll
        for (int i = 0; i < kWordsPerLane; ++i) {
            pre[l * kWordsPerLane + i] = run;
            run += pc[i];
        }
        wave_sync();
        for (int xb = x0 + l; xb < x1; xb += 4 * dev::kWave) {
            // every read of four products first (clamped to the bucket), then the adds
            float vv[4];
            int r[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int x = min(xb + j * dev::kWave, x1 - 1);
                vv[j] = s_pv[pad(x)];
                const int c = s_col[x];
                const int wd = c >> 5;
                r[j] = pre[wd] + __popc(bm[wd] & ((1u << (c & 31)) - 1u));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (xb + j * dev::kWave < x1) atomicAdd(&s_acc[x0 + r[j]], static_cast<double>(vv[j]));
            }
        }
        wave_sync();  // every product value of the bucket is read: its slots take the columns
        // Each product writes its column at its rank into the bucket's own product-value
        // slots (s_pv), so the distinct columns land there in order; products of one column
        // write the same word.  Four products per lane per round, as in the adds above.
        int *s_ocol = reinterpret_cast<int *>(s_pv);
        for (int xb = x0 + l; xb < x1; xb += 4 * dev::kWave) {
            int c[4], r[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int x = min(xb + j * dev::kWave, x1 - 1);
                c[j] = s_col[x];
                const int wd = c[j] >> 5;
                r[j] = pre[wd] + __popc(bm[wd] & ((1u << (c[j] & 31)) - 1u));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (xb + j * dev::kWave < x1) s_ocol[pad(x0 + r[j])] = c[j];
            }
        }
        if (l == dev::kWave - 1) s_out[o] = incl;  // the bucket's distinct columns
        wave_sync();
        int claim = 0;
        if (l == 0) claim = atomicAdd(&s_next, 1);
        o = __shfl(claim, 0, dev::kWave);
    }
    __syncthreads();
    // output offset of each bucket inside the unit
    int total = 0;
    const int cnt = static_cast<int>(threadIdx.x) < n_buckets ? s_out[threadIdx.x] : 0;
    const int off = dev::block_exclusive_sum<kBitmapBlock>(cnt, s_wave, total);
    if (static_cast<int>(threadIdx.x) < n_buckets) s_out[threadIdx.x] = off;
    __syncthreads();
    // the unit's entries, consecutive lanes on consecutive outputs: output i belongs to the
    // last bucket whose offset is at most i (a lane's outputs only move forward)
    int o = 0;
    const int64_t out = seg_out ? seg_out[s0] : start;
    for (int i = threadIdx.x; i < total; i += kBitmapBlock) {
        while (o + 1 < n_buckets && s_out[o + 1] <= i) ++o;
        const int x = s_x0[o] + (i - s_out[o]);
        ukey[out + i] = s_base[o] + reinterpret_cast<const int *>(s_pv)[pad(x)];
        uval[out + i] = static_cast<float>(s_acc[x]);
    }
    // rows starting in this unit, and the unit's count
    if (static_cast<int>(threadIdx.x) < n_buckets) {
        const int sg = s_sid[threadIdx.x];
        const int r = seg_row[sg];
        if (row_off[r] == seg_off[sg]) {
            row_unit[r] = static_cast<int>(u);
            row_local[r] = s_out[threadIdx.x];
        }
    }
    if (threadIdx.x == 0) unit_nnz[u] = total;
}

// ---- 5c: dense units -------------------------------------------------------------------

// One workgroup of kDenseBlock threads per dense unit (from the dense list): the 64 KB
// accumulator allows two resident workgroups per CU, so the workgroup is wide.  The
// segment's column range [bucket << shift, (bucket + 1) << shift) is accumulated kDenseCols
// columns at a time in an LDS float64 array (plus a bitmap of touched columns), then
// compacted in column order, 16 columns per lane.
constexpr int kDenseBlock = 512;
// Products per lane per round: 8 (C4 dense units 16.2 ms; 4: 16.8, 6: 16.2, 12: 16.6,
// 16: 18.5) keeps eight gathers in flight per lane for one run search.
constexpr int kDensePer = 8;

__global__ __launch_bounds__(kDenseBlock) void dense_unit_kernel(
    const int *__restrict__ dense_list, const int *__restrict__ unit_seg,
    const int64_t *__restrict__ unit_start,
    const int64_t *__restrict__ seg_len, const int64_t *__restrict__ seg_prefix,
    const int *__restrict__ seg_row, const int64_t *__restrict__ row_off, int shift, int cols,
    const int4 *__restrict__ desc, const int64_t *__restrict__ seg_roff,
    const int2 *__restrict__ cv_b, int *__restrict__ ukey,
    float *__restrict__ uval, int64_t *__restrict__ unit_nnz, int *__restrict__ row_unit,
    int *__restrict__ row_local, const int64_t *__restrict__ seg_out) {
    __shared__ double s_acc[kDenseCols];
    __shared__ unsigned s_bits[kDenseCols / 32];
    __shared__ int s_wave[kDenseBlock / dev::kWave];
    // a batch of up to kDenseBlock runs: first product offset, B entry of product 0, A value
    __shared__ int s_off[kDenseBlock];
    __shared__ int s_bs[kDenseBlock];
    __shared__ float s_a[kDenseBlock];
    static_assert(kDenseCols / 16 == kDenseBlock, "16 bitmap bits per lane");
    const int64_t u = dense_list[dev::xcd_block<kXcdGroup>()];
    const int s = unit_seg[u];
    const int64_t start = unit_start[u];
    const int row = seg_row[s];
    const int64_t bucket = s - seg_prefix[row];
    const int64_t c_lo = bucket << shift;
    const int64_t c_hi = min(static_cast<int64_t>(cols), (bucket + 1) << shift);
    if (threadIdx.x == 0 && row_off[row] == start) {
        row_unit[row] = static_cast<int>(u);
        row_local[row] = 0;
    }
    int64_t written = seg_out ? seg_out[s] : start;
    const int64_t out0 = written;
    for (int64_t w0 = c_lo; w0 < c_hi; w0 += kDenseCols) {
        for (int i = threadIdx.x; i < kDenseCols; i += kDenseBlock) s_acc[i] = 0.0;
        if (threadIdx.x < kDenseCols / 32) s_bits[threadIdx.x] = 0u;
        __syncthreads();
        // runs in batches of kDenseBlock (one per lane); the batch's products are spread over
        // the lanes, kDensePer consecutive ones per lane per round, each lane finding the run
        // of its first product by a search of the batch's offsets and advancing from there
        for (int64_t rb = seg_roff[s]; rb < seg_roff[s + 1]; rb += kDenseBlock) {
            const int nr = static_cast<int>(min(static_cast<int64_t>(kDenseBlock), seg_roff[s + 1] - rb));
            const int4 d = static_cast<int>(threadIdx.x) < nr ? desc[rb + threadIdx.x]
                                                              : make_int4(0, 0, 0, 0);
            int total = 0;
            const int off = dev::block_exclusive_sum<kDenseBlock>(d.y, s_wave, total);
            s_off[threadIdx.x] = off;
            s_bs[threadIdx.x] = d.x - off;
            s_a[threadIdx.x] = __int_as_float(d.z);
            __syncthreads();
            for (int x0 = threadIdx.x * kDensePer; x0 < total; x0 += kDensePer * kDenseBlock) {
                int lo = 0, hi = nr - 1;  // last run starting at or before x0
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (s_off[mid] <= x0) {
                        lo = mid;
                    } else {
                        hi = mid - 1;
                    }
                }
                int r = lo;
                int qv[kDensePer];
                float av[kDensePer];
#pragma unroll
                for (int q = 0; q < kDensePer; ++q) {
                    const int x = min(x0 + q, total - 1);
                    while (r + 1 < nr && s_off[r + 1] <= x) ++r;
                    qv[q] = s_bs[r] + x;
                    av[q] = s_a[r];
                }
                int kk[kDensePer];
                float vv[kDensePer];
#pragma unroll
                for (int q = 0; q < kDensePer; ++q) {
                    const int2 e = cv_b[qv[q]];
                    kk[q] = e.x;
                    vv[q] = __int_as_float(e.y);
                }
#pragma unroll
                for (int q = 0; q < kDensePer; ++q) {
                    const int64_t c = kk[q] - w0;
                    if (x0 + q < total && c >= 0 && c < kDenseCols) {
                        atomicAdd(&s_acc[c], static_cast<double>(av[q] * vv[q]));
                        atomicOr(&s_bits[c >> 5], 1u << (c & 31));
                    }
                }
            }
            __syncthreads();  // the batch's tables are read before the next batch
        }
        const unsigned half = (s_bits[threadIdx.x >> 1] >> ((threadIdx.x & 1) * 16)) & 0xffffu;
        int total = 0;
        int rank = dev::block_exclusive_sum<kDenseBlock>(static_cast<int>(__popc(half)), s_wave,
                                                         total);
        unsigned m = half;
        while (m) {
            const int bit = __ffs(m) - 1;
            m &= m - 1;
            const int c = threadIdx.x * 16 + bit;
            ukey[written + rank] = static_cast<int>(w0 + c);
            uval[written + rank] = static_cast<float>(s_acc[c]);
            ++rank;
        }
        written += total;
        __syncthreads();
    }
    if (threadIdx.x == 0) unit_nnz[u] = written - out0;
}

// ---- symbolic pass: the result's size before the reduce ----------------------------------
//
// When every column index fits kSymColBits bits, the distinct columns of every segment are
// counted before any unit reduces, from A and B directly (no run descriptors): seg_nnz[s].
// Their exclusive scan gives every segment's result offset, the result is allocated at its
// exact size, and the reduce units write straight into it (a unit's entries are its
// segments' distinct entries in segment order, so the unit starts at its first segment's
// offset).  A row starts at its first segment's offset.  The reference sizes its result the
// same way before reducing into it, from the head flags of its sorted products
// (stitch_and_generate_gpu.cpp:96-126).
//
// Long rows: one workgroup per row (rows claimed from a list, the heaviest first) ORs each
// product's column into a bitmap of the row's columns in LDS (2^20 bits, 128 KB), then counts
// each bucket's bits (a bucket is 8192 columns, 256 words, or the whole row when nb = 1) and
// clears the words it read.  The row's A entries are staged kSymChunk at a time (their B
// rows' starts and product offsets; empty B rows dropped); each wavefront takes an equal
// share of the chunk's products in windows of 64 consecutive products, lane x on product x
// of the window, so that a window's loads are consecutive entries of a few B rows.  The
// entry of lane x's product is the window's first entry plus the number of entries starting
// inside the window at or before x, counted in a 64-bit mask of those starts (an OR over the
// wavefront).  The first entries of kSymBatch windows are searched at once, one lane each,
// and the windows' loads are all issued before their ORs.
// Short rows (at most kShort products): one wavefront per row inserts the columns into an
// open-addressing table of its own in LDS (kSymSlots 32-bit slots, at most half full) and
// counts the keys it added; then it refills the table with the empty key.
constexpr int kSymColBits = 20;
constexpr int kSymBlock = 1024;
constexpr int kSymWords = 1 << (kSymColBits - 5);
constexpr int kSymChunk = kSymBlock;
constexpr int kSymBatch = 16;
constexpr int64_t kSymHeavy = int64_t{1} << 18;  // long rows with more products go first
constexpr int kSymShortBlock = 512;
constexpr int kSymSlots = 4096;
constexpr unsigned kSymEmpty = 0xffffffffu;  // above every column index (< 2^kSymColBits)
static_assert(kSymWords == 32 * kSymBlock, "a thread counts 32 words of the bitmap");
static_assert(kDenseCols / 32 == 8 * 32, "a bucket of 8192 columns is 8 threads' words");
static_assert(kSymSlots >= 2 * kShort, "a short row's table stays at most half full");

// OR of v over the 64 lanes, returned to every lane (DPP inclusive OR scan, then lane 63).
// Every lane must be active.
__device__ __forceinline__ unsigned wave_or(unsigned v) {
    int x = static_cast<int>(v);
    x |= __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x |= __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x |= __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x |= __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x |= __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x |= __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return static_cast<unsigned>(__builtin_amdgcn_readlane(x, dev::kWave - 1));
}

// Entry of lane l's product in a window of 64 products starting at wb, given e0, the entry
// holding product wb: entries e0 + 1 + l (l < 63) may start inside the window (off: their
// first products, ne entries in all, nonempty, so their starts are distinct and > wb).
// Uniform control flow.
__device__ __forceinline__ int window_entry(const int *off, int ne, int e0, int wb, int l) {
    const int e = e0 + 1 + l;
    const int d = e < ne ? off[e] - wb : dev::kWave;
    const bool in = d < dev::kWave;
    const unsigned mlo = wave_or(in && d < 32 ? 1u << d : 0u);
    const unsigned mhi = wave_or(in && d >= 32 ? 1u << (d - 32) : 0u);
    const int cnt = l < 32 ? __popc(mlo & ((2u << l) - 1u))
                           : __popc(mlo) + __popc(mhi & ((2u << (l - 32)) - 1u));
    return e0 + cnt;
}

// Work lists of the symbolic pass.  key1[i] = 2^32 for a long row with more than kSymHeavy
// products, 1 for another long row; key2[i] = 1 for a short row with products.  An empty
// row's segment count is 0.  Zeroes the long-row work counter.
__global__ void sym_flags_kernel(const int64_t *__restrict__ row_off, int rows,
                                 const int64_t *__restrict__ seg_prefix,
                                 int64_t *__restrict__ key1, int64_t *__restrict__ key2,
                                 int64_t *__restrict__ seg_nnz, int *__restrict__ work) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += gridDim.x * blockDim.x) {
        const int64_t prod = row_off[i + 1] - row_off[i];
        key1[i] = prod > kShort ? (prod > kSymHeavy ? (int64_t{1} << 32) : 1) : 0;
        key2[i] = prod > 0 && prod <= kShort ? 1 : 0;
        if (prod == 0) seg_nnz[seg_prefix[i]] = 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *work = 0;
}

// long_list: the heavy long rows, then the others (each group in row order); short_list:
// the short rows with products.  counts[0] / counts[1]: their lengths.  rank1 / rank2 are
// the exclusive scans of key1 / key2 (rank1 packs both groups' ranks, heavy in the high half).
__global__ void sym_lists_kernel(const int64_t *__restrict__ row_off, int rows,
                                 const int64_t *__restrict__ rank1,
                                 const int64_t *__restrict__ rank2, int *__restrict__ long_list,
                                 int *__restrict__ short_list, int64_t *__restrict__ counts) {
    const int64_t t1 = rank1[rows];
    const int64_t n_heavy = t1 >> 32;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += gridDim.x * blockDim.x) {
        const int64_t prod = row_off[i + 1] - row_off[i];
        if (prod > kShort) {
            const int64_t r = rank1[i];
            long_list[prod > kSymHeavy ? (r >> 32) : n_heavy + (r & 0xffffffffll)] = i;
        } else if (prod > 0) {
            short_list[rank2[i]] = i;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        counts[0] = n_heavy + (t1 & 0xffffffffll);
        counts[1] = rank2[rows];
    }
}

// Distinct columns of every bucket of the long rows (see above).  One resident workgroup
// per CU; workgroup g starts with long-list item g and claims its next item from `work`
// (zeroed) when it starts a row, so the next chunk of A entries (the rest of this row's, or
// the claimed item's first) is known in advance: its column loads are issued before this
// chunk's batches and its B row starts after them, off the chunk-to-chunk path.
__global__ __launch_bounds__(kSymBlock) void sym_long_kernel(
    const int *__restrict__ pos_a, const int *__restrict__ crd_a,
    const int *__restrict__ pos_b, const int *__restrict__ crd_b,
    const int *__restrict__ long_list, const int64_t *__restrict__ counts,
    int *__restrict__ work, const int64_t *__restrict__ seg_prefix, int nb, int cols,
    int64_t *__restrict__ seg_nnz) {
    constexpr int kWaves = kSymBlock / dev::kWave;
    __shared__ uint4 s_bm4[kSymWords / 4];
    __shared__ int s_off[kSymChunk + 1];
    __shared__ int s_bs[kSymChunk];
    __shared__ int64_t s_wave[kWaves];
    __shared__ int s_sum[kWaves];
    __shared__ int64_t s_next;  // the item claimed for after the current row
    unsigned *s_bm = reinterpret_cast<unsigned *>(s_bm4);
    const int tid = threadIdx.x, w = tid / dev::kWave, l = dev::lane();
    const int64_t n_long = counts[0];
    int64_t item = blockIdx.x;
    if (item >= n_long) return;  // uniform
    const int words = (cols + 31) >> 5;  // <= kSymWords
    for (int i = tid; i < kSymWords / 4; i += kSymBlock) s_bm4[i] = make_uint4(0u, 0u, 0u, 0u);
    int row = long_list[item];
    int p0 = pos_a[row], p_end = pos_a[row + 1];
    bool row_start = true;
    int bs = 0, len = 0;  // this thread's A entry of the current chunk: its B row
    if (p0 + tid < p_end) {
        const int k = crd_a[p0 + tid];
        bs = pos_b[k];
        len = pos_b[k + 1] - bs;
    }
    for (;;) {
        // (every thread read the previous claim before the last chunk's final barrier; this
        // one is read after this chunk's barriers)
        if (row_start && tid == 0) s_next = static_cast<int64_t>(gridDim.x) + atomicAdd(work, 1);
        // the next chunk, and its column loads (in flight during this chunk)
        int64_t n_item = item;
        int n_row = row, n_p0 = p0 + kSymChunk, n_end = p_end;
        const bool row_done = n_p0 >= p_end;
        if (row_done) {
            __syncthreads();  // the claim
            n_item = s_next;
            if (n_item < n_long) {
                n_row = long_list[n_item];
                n_p0 = pos_a[n_row];
                n_end = pos_a[n_row + 1];
            }
        }
        const bool more = n_item < n_long;
        const int n_k = more && n_p0 + tid < n_end ? crd_a[n_p0 + tid] : -1;
        // one scan for both the nonempty entries' ranks (high half) and product offsets
        // (low half: a chunk's products are at most nnz(B), its B rows being distinct)
        int64_t tot = 0;
        const int64_t ex = dev::block_exclusive_sum<kSymBlock, int64_t>(
            (static_cast<int64_t>(len > 0) << 32) | static_cast<int64_t>(len), s_wave, tot);
        const int ne = static_cast<int>(tot >> 32);
        const int T = static_cast<int>(tot & 0xffffffffll);
        if (len > 0) {
            const int e = static_cast<int>(ex >> 32);
            const int off = static_cast<int>(ex & 0xffffffffll);
            s_off[e] = off;
            s_bs[e] = bs - off;  // product x of entry e is B entry s_bs[e] + x
        }
        if (tid == 0) s_off[ne] = T;
        __syncthreads();
        const int share = (T + kWaves - 1) / kWaves;
        const int lo = min(T, w * share), hi = min(T, lo + share);
        for (int x0 = lo; x0 < hi; x0 += dev::kWave * kSymBatch) {  // uniform per wave
            int first = 0;  // lane j < kSymBatch: the entry of window j's first product
            {
                const int q = x0 + l * dev::kWave;
                if (l < kSymBatch && q < hi) {
                    first = static_cast<int>(dev::last_le(s_off, 0, ne - 1, q));
                }
            }
            int c[kSymBatch];
#pragma unroll
            for (int j = 0; j < kSymBatch; ++j) {
                const int wb = x0 + j * dev::kWave;
                c[j] = -1;
                if (wb < hi) {  // uniform
                    const int e0 = __builtin_amdgcn_readlane(first, j);
                    const int e = window_entry(s_off, ne, e0, wb, l);
                    if (wb + l < hi) c[j] = crd_b[s_bs[e] + wb + l];
                }
            }
#pragma unroll
            for (int j = 0; j < kSymBatch; ++j) {
                if (c[j] >= 0) atomicOr(&s_bm[c[j] >> 5], 1u << (c[j] & 31));
            }
        }
        // the next chunk's B rows (in flight during the barrier and the bucket counts)
        int n_bs = 0, n_len = 0;
        if (n_k >= 0) {
            n_bs = pos_b[n_k];
            n_len = pos_b[n_k + 1] - n_bs;
        }
        __syncthreads();  // the chunk's tables are read; the ORs are done
        if (row_done) {
            // count and clear: thread t holds words [32t, 32t + 32).  The next chunk's scan
            // barrier orders the clears before its ORs.
            int bits = 0;
            if (32 * tid < words) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint4 v = s_bm4[8 * tid + i];
                    bits += __popc(v.x) + __popc(v.y) + __popc(v.z) + __popc(v.w);
                    s_bm4[8 * tid + i] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
            const int64_t s0 = seg_prefix[row];
            if (nb == 1) {
                int total = 0;
                (void)dev::block_exclusive_sum<kSymBlock>(bits, s_sum, total);
                if (tid == 0) seg_nnz[s0] = total;
            } else {  // buckets of 8192 columns: 8 consecutive threads each
                bits += __shfl_xor(bits, 1, dev::kWave);
                bits += __shfl_xor(bits, 2, dev::kWave);
                bits += __shfl_xor(bits, 4, dev::kWave);
                if ((tid & 7) == 0 && (tid >> 3) < nb) seg_nnz[s0 + (tid >> 3)] = bits;
            }
        }
        if (!more) break;  // uniform
        row_start = row_done;
        item = n_item;
        row = n_row;
        p0 = n_p0;
        p_end = n_end;
        bs = n_bs;
        len = n_len;
    }
}

// Distinct columns of every short row (see above): one wavefront per row; wave v of the
// grid takes short-list items v, v + V, v + 2V, ... (V waves), and loads the next item's
// row and offsets while it counts the current one.
__global__ __launch_bounds__(kSymShortBlock) void sym_short_kernel(
    const int *__restrict__ pos_a, const int *__restrict__ crd_a,
    const int *__restrict__ pos_b, const int *__restrict__ crd_b,
    const int *__restrict__ short_list, const int64_t *__restrict__ counts,
    const int64_t *__restrict__ seg_prefix, int64_t *__restrict__ seg_nnz) {
    constexpr int kWaves = kSymShortBlock / dev::kWave;
    __shared__ uint4 s_tab4[kWaves][kSymSlots / 4];
    __shared__ int s_off[kWaves][dev::kWave + 1];
    __shared__ int s_bs[kWaves][dev::kWave];
    const int w = threadIdx.x / dev::kWave, l = dev::lane();
    unsigned *tab = reinterpret_cast<unsigned *>(s_tab4[w]);
    int *off = s_off[w];
    int *bsw = s_bs[w];
    const uint4 empty4 = make_uint4(kSymEmpty, kSymEmpty, kSymEmpty, kSymEmpty);
    const int64_t n_short = counts[1];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
    int64_t item = static_cast<int64_t>(blockIdx.x) * kWaves + w;
    for (int i = l; i < kSymSlots / 4; i += dev::kWave) s_tab4[w][i] = empty4;
    if (item >= n_short) return;  // uniform per wave (no barriers below)
    int row = short_list[item];
    int p_lo = pos_a[row], p_end = pos_a[row + 1];
    for (;;) {
        const int64_t n_item = item + stride;
        const bool more = n_item < n_short;
        int n_row = 0, n_lo = 0, n_end = 0;
        if (more) {  // next item's row and offsets, in flight during this row
            n_row = short_list[n_item];
            n_lo = pos_a[n_row];
            n_end = pos_a[n_row + 1];
        }
        int fresh = 0;
        for (int p0 = p_lo; p0 < p_end; p0 += dev::kWave) {  // 64 A entries at a time
            const int p = p0 + l;
            int bs = 0, len = 0;
            if (p < p_end) {
                const int k = crd_a[p];
                bs = pos_b[k];
                len = pos_b[k + 1] - bs;
            }
            const unsigned long long nz = __ballot(len > 0);
            const int e = static_cast<int>(__popcll(nz & ((1ull << l) - 1ull)));
            const int ne = static_cast<int>(__popcll(nz));
            const int incl = dev::wave_inclusive_sum_dpp(len);
            const int T = __builtin_amdgcn_readlane(incl, dev::kWave - 1);
            if (len > 0) {
                off[e] = incl - len;
                bsw[e] = bs - (incl - len);
            }
            if (l == 0) off[ne] = T;
            wave_sync();
            for (int x0 = 0; x0 < T; x0 += dev::kWave * kSymBatch) {  // uniform
                int first = 0;
                {
                    const int q = x0 + l * dev::kWave;
                    if (l < kSymBatch && q < T) {
                        first = static_cast<int>(dev::last_le(off, 0, ne - 1, q));
                    }
                }
                int c[kSymBatch];
#pragma unroll
                for (int j = 0; j < kSymBatch; ++j) {
                    const int wb = x0 + j * dev::kWave;
                    c[j] = -1;
                    if (wb < T) {  // uniform
                        const int e0 = __builtin_amdgcn_readlane(first, j);
                        const int ee = window_entry(off, ne, e0, wb, l);
                        if (wb + l < T) c[j] = crd_b[bsw[ee] + wb + l];
                    }
                }
#pragma unroll
                for (int j = 0; j < kSymBatch; ++j) {
                    if (c[j] >= 0) {
                        const unsigned key = static_cast<unsigned>(c[j]);
                        unsigned h = (key * 0x9e3779b1u) >> (32 - 12);
                        for (;;) {
                            const unsigned old = atomicCAS(&tab[h], kSymEmpty, key);
                            if (old == kSymEmpty) {
                                ++fresh;
                                break;
                            }
                            if (old == key) break;
                            h = (h + 1u) & (kSymSlots - 1);
                        }
                    }
                }
            }
            wave_sync();  // off / bsw are read before the next 64 entries replace them
        }
        const int total = dev::wave_sum(fresh);
        if (l == 0) seg_nnz[seg_prefix[row]] = total;
        for (int i = l; i < kSymSlots / 4; i += dev::kWave) s_tab4[w][i] = empty4;
        wave_sync();
        if (!more) break;
        item = n_item;
        row = n_row;
        p_lo = n_lo;
        p_end = n_end;
    }
}

// Row offsets from the segment offsets: row i starts at its first segment's offset
// (seg_prefix[rows] = n_seg, whose offset is nnz).
template <typename PosT>
__global__ void seg_pos_kernel(const int64_t *__restrict__ seg_prefix, int rows,
                               const int64_t *__restrict__ seg_out, PosT *__restrict__ pos) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= rows; i += gridDim.x * blockDim.x) {
        pos[i] = static_cast<PosT>(seg_out[seg_prefix[i]]);
    }
}

// ---- 6: output -------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void copy_units_kernel(
    const int64_t *__restrict__ unit_start, const int64_t *__restrict__ unit_nnz,
    const int64_t *__restrict__ unit_out, const int *__restrict__ ukey,
    const float *__restrict__ uval, int *__restrict__ out_crd, float *__restrict__ out_val) {
    const int64_t u = blockIdx.x;
    const int64_t src = unit_start[u], dst = unit_out[u], n = unit_nnz[u];
    for (int64_t x = threadIdx.x; x < n; x += kBlock) {
        out_crd[dst + x] = ukey[src + x];
        out_val[dst + x] = uval[src + x];
    }
}

// Row offsets: a row with products starts at its unit's offset plus its local offset; the
// empty rows just before it share that offset; rows starting at P (and pos[rows]) get nnz.
template <typename PosT>
__global__ void row_pos_kernel(const int64_t *__restrict__ row_off, int rows, int64_t P,
                               int64_t nnz, const int *__restrict__ row_unit,
                               const int *__restrict__ row_local,
                               const int64_t *__restrict__ unit_out, PosT *__restrict__ pos) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= rows; i += gridDim.x * blockDim.x) {
        const int64_t rs = row_off[i];
        if (rs == P) {
            pos[i] = static_cast<PosT>(nnz);
        } else if (row_off[i + 1] > rs) {
            const PosT v = static_cast<PosT>(unit_out[row_unit[i]] + row_local[i]);
            pos[i] = v;
            for (int x = i - 1; x >= 0 && row_off[x] == rs; --x) pos[x] = v;
        }
    }
}

// ---- host ------------------------------------------------------------------------------

bool bad_csr(const nacho_csr *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0) return true;
    if (!t->dim_j_offsets) return true;
    if (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values)) return true;
    return false;
}

unsigned grid_for(int64_t n, int per_block) {
    const int64_t g = (n + per_block - 1) / per_block;
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(g, 1 << 20)));
}

// Bits that hold every column index of a matrix with `cols` columns.
int col_bits(int cols) {
    int b = 1;
    while (b < 31 && (static_cast<int64_t>(1) << b) < cols) ++b;
    return b;
}

// How the result is sized.  Staged: the reduce units write their distinct entries at their
// units' product offsets in a staging buffer of 8 bytes per product, and a copy moves them
// into the result once every unit's count is known.  Symbolic: the symbolic pass counts
// every segment's distinct columns first, and the units write straight into the result
// (no staging buffer; possible when every column fits the pass's 2^kSymColBits-bit row
// bitmap).  At C4 the copy costs 11.0 ms and the symbolic pass 20.6 ms (its long-row kernel
// is bound by the per-row chain of one workgroup per CU), so the staged path is taken
// while its buffer fits in half of the device memory that is free or cached by the
// library, the symbolic one otherwise.  NACHO_SPGEMM_OUTPUT=staged or =symbolic chooses
// one (symbolic only where it applies).
enum class Output { Staged, Symbolic };

Output output_mode(int64_t products, bool symbolic_fits) {
    const char *v = std::getenv("NACHO_SPGEMM_OUTPUT");
    if (v != nullptr && std::strcmp(v, "staged") == 0) return Output::Staged;
    if (!symbolic_fits) return Output::Staged;
    if (v != nullptr && std::strcmp(v, "symbolic") == 0) return Output::Symbolic;
    size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) return Output::Symbolic;
    const double room = (static_cast<double>(free_bytes) + static_cast<double>(nacho_cached_bytes())) / 2;
    return 8.0 * static_cast<double>(products) <= room ? Output::Staged : Output::Symbolic;
}

struct Product {
    int rows = 0, cols = 0;
    int64_t nnz = 0;
    void *pos = nullptr;
    int *crd = nullptr;
    float *val = nullptr;
};

// Runs the pipeline; result offsets are PosT.  With int32 offsets the call fails with
// NACHO_ERR_INDEX_OVERFLOW (before allocating the result) when nnz(Z) exceeds INT_MAX.
template <typename PosT>
int multiply(Call &call, const nacho_csr *a, const nacho_csr *b, Product *z) {
    const hipStream_t st = call.stream();
    const int rows = a->dim_i_size;
    const int cols = b->dim_j_size;
    const int64_t nnz_a = a->dim_j_length;
    const int cb = col_bits(cols);
    // one radix digit over the columns: buckets of 2^shift columns, at most kMaxBuckets
    const int shift = std::max(std::min(kDenseBits, cb), cb - kMaxBucketBits);
    const int nb = cols > 0 ? ((cols - 1) >> shift) + 1 : 1;
    const int dense_min = shift <= kDenseBits ? kDenseMin : kShort;
    const char *name = "spgemm: runs+reduce+output";
    NACHO_TRY(call.timer_start(name));

    // 1-2. products per A entry, per row; segments per row
    int64_t *len = nullptr, *off = nullptr, *row_off = nullptr, *seg_count = nullptr;
    int64_t *seg_prefix = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_a) + 1, &len));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_a) + 1, &off));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &row_off));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &seg_count));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &seg_prefix));
    if (nnz_a > 0) {
        lengths_kernel<<<grid_for(nnz_a, 256), 256, 0, st>>>(a->dim_j_indices, nnz_a,
                                                             b->dim_j_offsets, len);
        NACHO_TRY_HIP(hipGetLastError());
    }
    NACHO_TRY(scan::exclusive_scan_i64(call, len, nnz_a, off));
    rows_kernel<<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, st>>>(
        a->dim_j_offsets, rows, off, nb, row_off, seg_count);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(scan::exclusive_scan_i64(call, seg_count, rows, seg_prefix));
    int64_t P = 0, n_seg = 0;
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.read_back(&P, row_off + rows, sizeof(P)));
    NACHO_TRY(call.read_back(&n_seg, seg_prefix + rows, sizeof(n_seg)));
    NACHO_TRY(call.timer_start(name));
    if (n_seg >= INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;  // segment ids are int32
    const bool symbolic =
        P > 0 && output_mode(P, cb <= kSymColBits &&
                                    b->dim_j_length <= static_cast<int64_t>(INT_MAX) -
                                                           4 * kSymChunk) == Output::Symbolic;

    int64_t n_units = 0;
    int64_t *seg_out = nullptr;  // symbolic pass: result offset of every segment
    int64_t *unit_start = nullptr, *unit_nnz = nullptr, *unit_out = nullptr;
    int *row_unit = nullptr, *row_local = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &row_unit));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &row_local));
    if (P > 0) {
        // segment table
        int *seg_row = nullptr;
        int64_t *seg_len = nullptr, *seg_off = nullptr, *seg_fill = nullptr;
        int64_t *seg_runs = nullptr, *seg_roff = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg), &seg_row));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_len));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_off));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg), &seg_fill));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_runs));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_roff));
        segments_kernel<<<grid_for(rows, 256), 256, 0, st>>>(row_off, seg_prefix, rows,
                                                            a->dim_j_offsets, len, seg_row,
                                                            seg_len, seg_runs, seg_fill);
        NACHO_TRY_HIP(hipGetLastError());

        // symbolic pass: distinct columns per segment, scanned into result offsets
        if (symbolic) {
            int64_t *seg_nnz = nullptr, *keys = nullptr, *ranks = nullptr, *counts = nullptr;
            int *lists = nullptr, *work = nullptr;
            NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_nnz));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &seg_out));
            NACHO_TRY(call.scratch_n(2 * (static_cast<size_t>(rows) + 1), &keys));
            NACHO_TRY(call.scratch_n(2 * (static_cast<size_t>(rows) + 1), &ranks));
            NACHO_TRY(call.scratch_n(2 * static_cast<size_t>(rows) + 2, &lists));
            NACHO_TRY(call.scratch_n(2, &counts));
            NACHO_TRY(call.scratch_n(1, &work));
            int64_t *key2 = keys + (rows + 1), *rank2 = ranks + (rows + 1);
            int *long_list = lists, *short_list = lists + (rows + 1);
            sym_flags_kernel<<<grid_for(rows, 256), 256, 0, st>>>(row_off, rows, seg_prefix,
                                                                 keys, key2, seg_nnz, work);
            NACHO_TRY_HIP(hipGetLastError());
            NACHO_TRY(scan::exclusive_scan_i64(call, keys, rows, ranks));
            NACHO_TRY(scan::exclusive_scan_i64(call, key2, rows, rank2));
            sym_lists_kernel<<<grid_for(rows, 256), 256, 0, st>>>(row_off, rows, ranks, rank2,
                                                                 long_list, short_list, counts);
            NACHO_TRY_HIP(hipGetLastError());
            int g_long = 0, g_short = 0;
            NACHO_TRY(resident_grid(reinterpret_cast<const void *>(sym_long_kernel), kSymBlock,
                                    &g_long));
            NACHO_TRY(resident_grid(reinterpret_cast<const void *>(sym_short_kernel),
                                    kSymShortBlock, &g_short));
            sym_long_kernel<<<static_cast<unsigned>(g_long), kSymBlock, 0, st>>>(
                a->dim_j_offsets, a->dim_j_indices, b->dim_j_offsets, b->dim_j_indices,
                long_list, counts, work, seg_prefix, nb, cols, seg_nnz);
            NACHO_TRY_HIP(hipGetLastError());
            sym_short_kernel<<<static_cast<unsigned>(g_short), kSymShortBlock, 0, st>>>(
                a->dim_j_offsets, a->dim_j_indices, b->dim_j_offsets, b->dim_j_indices,
                short_list, counts, seg_prefix, seg_nnz);
            NACHO_TRY_HIP(hipGetLastError());
            NACHO_TRY(scan::exclusive_scan_i64(call, seg_nnz, n_seg, seg_out));
        }

        // 3. histogram, segment offsets, runs
        int *ukey = nullptr;  // the units' output: staged at product offsets, or the result
        float *uval = nullptr;
        if (!symbolic) {
            NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &ukey));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &uval));
        }
        // long rows' bucket counts from B's runs (P > 0, so B has entries)
        const int64_t nnz_b = b->dim_j_length;
        const int rows_b = b->dim_i_size;
        int64_t *flag = nullptr, *run_idx = nullptr;
        int2 *run = nullptr;
        int *run_start = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b) + 1, &flag));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b) + 1, &run_idx));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b), &run));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b) + 1, &run_start));
        run_flags_kernel<<<grid_for(nnz_b, 256), 256, 0, st>>>(b->dim_j_indices, nnz_b, shift,
                                                               flag);
        NACHO_TRY_HIP(hipGetLastError());
        if (rows_b > 0) {
            run_row_starts_kernel<<<grid_for(rows_b, 256), 256, 0, st>>>(b->dim_j_offsets,
                                                                          rows_b, flag);
            NACHO_TRY_HIP(hipGetLastError());
        }
        NACHO_TRY(scan::exclusive_scan_i64(call, flag, nnz_b, run_idx));
        runs_kernel<<<grid_for(nnz_b, 256), 256, 0, st>>>(b->dim_j_indices, nnz_b, shift, flag,
                                                          run_idx, run, run_start);
        NACHO_TRY_HIP(hipGetLastError());
        run_lengths_kernel<<<grid_for(nnz_b, 256), 256, 0, st>>>(run_idx, nnz_b, run_start, run);
        NACHO_TRY_HIP(hipGetLastError());
        int2 *cv_b = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b), &cv_b));
        interleave_kernel<<<grid_for(nnz_b, 256), 256, 0, st>>>(b->dim_j_indices, b->values,
                                                                nnz_b, cv_b);
        NACHO_TRY_HIP(hipGetLastError());
        int64_t *nblk = nullptr, *blk_off = nullptr;
        int *blk_row = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &nblk));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &blk_off));
        // at most one block per kBlock entries of A, plus one per row
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_a / kBlock + rows + 1), &blk_row));
        hist_blocks_kernel<<<grid_for(rows, 256), 256, 0, st>>>(a->dim_j_offsets, rows, row_off,
                                                               nblk);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(scan::exclusive_scan_i64(call, nblk, rows, blk_off));
        hist_rows_kernel<<<grid_for(rows, 256), 256, 0, st>>>(blk_off, rows, blk_row);
        NACHO_TRY_HIP(hipGetLastError());
        const BRuns br{run_idx, run, run_start};
        long_hist_kernel<<<kHistGrid, kBlock, 0, st>>>(
            a->dim_j_offsets, a->dim_j_indices, blk_off, blk_row, rows, b->dim_j_offsets, br,
            nb, seg_prefix, seg_len, seg_runs);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(scan::exclusive_scan_i64(call, seg_len, n_seg, seg_off));
        NACHO_TRY(scan::exclusive_scan_i64(call, seg_runs, n_seg, seg_roff));
        int64_t n_runs = 0, nnz_sym = 0;
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.read_back(&n_runs, seg_roff + n_seg, sizeof(n_runs)));
        if (symbolic) {
            NACHO_TRY(call.read_back(&nnz_sym, seg_out + n_seg, sizeof(nnz_sym)));
            if (sizeof(PosT) == sizeof(int32_t) && nnz_sym > INT_MAX) {
                return NACHO_ERR_INDEX_OVERFLOW;
            }
            NACHO_TRY(call.result_n(static_cast<size_t>(nnz_sym), &z->crd));
            NACHO_TRY(call.result_n(static_cast<size_t>(nnz_sym), &z->val));
            ukey = z->crd;
            uval = z->val;
        }
        NACHO_TRY(call.timer_start(name));
        int4 *desc = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max<int64_t>(n_runs, 1)), &desc));
        long_runs_kernel<<<kHistGrid, kBlock, 0, st>>>(
            a->dim_j_offsets, a->dim_j_indices, a->values, blk_off, blk_row, rows,
            b->dim_j_offsets, br, nb, seg_prefix, seg_roff, seg_fill, desc);
        NACHO_TRY_HIP(hipGetLastError());
        short_runs_kernel<<<grid_for(rows, 256), 256, 0, st>>>(
            a->dim_j_offsets, a->dim_j_indices, a->values, rows, row_off, seg_prefix, seg_roff,
            b->dim_j_offsets, desc);
        NACHO_TRY_HIP(hipGetLastError());

        // 4. units
        int64_t *seg_units = seg_fill;  // the run fill counters are spent
        int64_t *unit_prefix = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_seg) + 1, &unit_prefix));
        unit_count_kernel<<<grid_for(n_seg, 256), 256, 0, st>>>(
            seg_len, seg_off, n_seg, seg_row, row_off, dense_min, seg_units);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(scan::exclusive_scan_i64(call, seg_units, n_seg, unit_prefix));
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.read_back(&n_units, unit_prefix + n_seg, sizeof(n_units)));
        NACHO_TRY(call.timer_start(name));
        if (n_units > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;
        int *unit_seg = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_units), &unit_seg));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_units) + 1, &unit_start));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_units) + 1, &unit_nnz));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(n_units) + 1, &unit_out));
        int *lists = nullptr;  // dense list, bitmap list, sort list
        int64_t *kinds = nullptr;  // dense flags, their ranks, bitmap flags, their ranks
        NACHO_TRY(call.scratch_n(3 * static_cast<size_t>(n_units), &lists));
        NACHO_TRY(call.scratch_n(4 * (static_cast<size_t>(n_units) + 1), &kinds));
        int64_t *unit_dense = kinds, *dense_rank = kinds + (n_units + 1);
        int64_t *unit_bitmap = kinds + 2 * (n_units + 1), *bitmap_rank = kinds + 3 * (n_units + 1);
        int *dense_list = lists, *bitmap_list = lists + n_units, *sort_list = lists + 2 * n_units;
        unit_map_kernel<<<grid_for(n_seg + 1, 256), 256, 0, st>>>(
            seg_units, unit_prefix, seg_off, seg_len, seg_row, row_off, dense_min, n_seg, P,
            unit_seg, unit_start, unit_dense);
        NACHO_TRY_HIP(hipGetLastError());
        unit_bitmap_kernel<<<grid_for(n_units, 256), 256, 0, st>>>(
            unit_seg, unit_dense, n_units, n_seg, seg_len, seg_row, row_off, shift <= kDenseBits,
            unit_bitmap);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(scan::exclusive_scan_i64(call, unit_dense, n_units, dense_rank));
        NACHO_TRY(scan::exclusive_scan_i64(call, unit_bitmap, n_units, bitmap_rank));
        unit_lists_kernel<<<grid_for(n_units, 256), 256, 0, st>>>(
            unit_dense, dense_rank, unit_bitmap, bitmap_rank, n_units, dense_list, bitmap_list,
            sort_list);
        NACHO_TRY_HIP(hipGetLastError());
        int64_t n_dense = 0, n_bitmap = 0;
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.read_back(&n_dense, dense_rank + n_units, sizeof(n_dense)));
        NACHO_TRY(call.read_back(&n_bitmap, bitmap_rank + n_units, sizeof(n_bitmap)));
        NACHO_TRY(call.timer_start(name));
        const int n_kind[3] = {static_cast<int>(n_dense),
                               static_cast<int>(n_units - n_dense - n_bitmap),
                               static_cast<int>(n_bitmap)};

        // 5. reduce
        const unsigned ug = static_cast<unsigned>(n_units);
        if (n_kind[1] > 0 && cb + kOrdBits <= 32) {
            sort_unit_kernel<uint32_t><<<static_cast<unsigned>(n_kind[1]), kBlock, 0, st>>>(
                sort_list, unit_seg, unit_start, n_units, n_seg, seg_len, seg_off, seg_row,
                row_off, cb, desc, seg_roff, cv_b, ukey, uval, unit_nnz, row_unit, row_local,
                seg_out);
        } else if (n_kind[1] > 0) {
            sort_unit_kernel<uint64_t><<<static_cast<unsigned>(n_kind[1]), kBlock, 0, st>>>(
                sort_list, unit_seg, unit_start, n_units, n_seg, seg_len, seg_off, seg_row,
                row_off, 32, desc, seg_roff, cv_b, ukey, uval, unit_nnz, row_unit, row_local,
                seg_out);
        }
        NACHO_TRY_HIP(hipGetLastError());
        if (n_kind[2] > 0) {
            bitmap_unit_kernel<<<static_cast<unsigned>(n_kind[2]), kBitmapBlock, 0, st>>>(
                bitmap_list, unit_seg, unit_start, n_units, n_seg, seg_len, seg_off, seg_prefix,
                seg_row, row_off, shift, desc, seg_roff, cv_b, ukey, uval, unit_nnz, row_unit,
                row_local, seg_out);
            NACHO_TRY_HIP(hipGetLastError());
        }
        if (n_kind[0] > 0) {
            dense_unit_kernel<<<static_cast<unsigned>(n_kind[0]), kDenseBlock, 0, st>>>(
                dense_list, unit_seg, unit_start, seg_len, seg_prefix, seg_row, row_off, shift,
                cols, desc, seg_roff, cv_b, ukey, uval, unit_nnz, row_unit, row_local, seg_out);
            NACHO_TRY_HIP(hipGetLastError());
        }
        if (symbolic) {
            z->nnz = nnz_sym;  // the units wrote straight into the result
        } else {
            NACHO_TRY(scan::exclusive_scan_i64(call, unit_nnz, n_units, unit_out));
            int64_t nnz = 0;
            NACHO_TRY(call.timer_stop());
            NACHO_TRY(call.read_back(&nnz, unit_out + n_units, sizeof(nnz)));
            if (sizeof(PosT) == sizeof(int32_t) && nnz > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;
            NACHO_TRY(call.timer_start(name));

            // 6. output
            NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &z->crd));
            NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &z->val));
            if (nnz > 0) {
                copy_units_kernel<<<ug, kBlock, 0, st>>>(unit_start, unit_nnz, unit_out, ukey,
                                                         uval, z->crd, z->val);
                NACHO_TRY_HIP(hipGetLastError());
            }
            z->nnz = nnz;
        }
    }
    PosT *pos = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pos));
    if (seg_out) {
        seg_pos_kernel<PosT><<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, st>>>(
            seg_prefix, rows, seg_out, pos);
    } else {
        row_pos_kernel<PosT><<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, st>>>(
            row_off, rows, P, z->nnz, row_unit, row_local, unit_out, pos);
    }
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());

    z->rows = rows;
    z->cols = cols;
    z->pos = pos;
    return NACHO_OK;
}

int check_operands(const nacho_csr *a, const nacho_csr *b, int32_t num_blocks,
                   int32_t threads_per_block) {
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csr(a) || bad_csr(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_j_size != b->dim_i_size) return NACHO_ERR_INVALID_ARGUMENT;
    return NACHO_OK;
}

}  // namespace spgemm
}  // namespace nacho

extern "C" {

int nacho_gpu_spgemm64_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr64 *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc) {
    using namespace nacho;
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr64{};
    NACHO_TRY(spgemm::check_operands(a, b, num_blocks, threads_per_block));
    Call call(stream, alloc);
    spgemm::Product p;
    NACHO_TRY(spgemm::multiply<int64_t>(call, a, b, &p));
    z->dim_i_size = p.rows;
    z->dim_j_size = p.cols;
    z->dim_j_offsets = static_cast<int64_t *>(p.pos);
    z->dim_j_length = p.nnz;
    z->dim_j_indices = p.crd;
    z->values = p.val;
    z->nnz = p.nnz;
    call.commit();
    return NACHO_OK;
}

int nacho_gpu_spgemm_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                         int32_t num_blocks, int32_t threads_per_block, void *stream,
                         const nacho_allocator *alloc) {
    using namespace nacho;
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(spgemm::check_operands(a, b, num_blocks, threads_per_block));
    Call call(stream, alloc);
    spgemm::Product p;
    NACHO_TRY(spgemm::multiply<int32_t>(call, a, b, &p));
    z->dim_i_size = p.rows;
    z->dim_j_size = p.cols;
    z->dim_j_offsets = static_cast<int32_t *>(p.pos);
    z->dim_j_length = static_cast<int32_t>(p.nnz);
    z->dim_j_indices = p.crd;
    z->values = p.val;
    z->nnz = static_cast<int32_t>(p.nnz);
    call.commit();
    return NACHO_OK;
}

}  // extern "C"
