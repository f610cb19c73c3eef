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
//      row i's products are [off[posA[i]], off[posA[i+1]]) in (j, k) order.
//   2. tiles: a row with more than kShort products is cut into tiles of kTile products; the
//      shorter rows whose first product falls in the same kShort-aligned window share one
//      tile (fewer than kTile products, since each has at most kShort).  Tiles cover [0, P)
//      in order: tile t is [tile_start[t], tile_start[t+1]).
//   3. expand: each workgroup writes kTile consecutive products (k, a_ij * b_jk).
//   4. sort: one workgroup per tile sorts by (row ordinal inside the tile, k) in LDS.
//   5. merge: a row longer than one tile merges its sorted tile runs pairwise, level by
//      level (runs of kTile << l), device-wide; the buffers ping-pong and each row starts in
//      the one that makes its last level end in the primary buffer.
//   6. compress: per tile, count the distinct (row, k) runs; scan -> output offsets; then a
//      segmented float64 reduction writes (k, sum rounded once to float32) and the row
//      offsets.  Every distinct column is kept (structural result, as the reference).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <utility>
#include <vector>

#include "device_utils.hpp"
#include "runtime.hpp"
#include "scan.hpp"

namespace nacho {
namespace spgemm {

constexpr int kBlock = 256;
constexpr int kTile = 4096;            // products per sort / merge / compress tile
constexpr int kPer = kTile / kBlock;   // 16 positions per lane
constexpr int kShort = kTile / 2;      // rows with at most this many products share tiles
constexpr int kOrdBits = 12;           // a shared tile holds fewer than 2^12 rows
constexpr int kMaxRowTiles = 1 << 18;  // keeps every in-row merge position below 2^31

static_assert(kTile == 1 << kOrdBits, "row ordinals must fit kOrdBits");

// ---- 1-2: sizes and tiles --------------------------------------------------------------

__global__ void lengths_kernel(const int *__restrict__ crd_a, int64_t nnz_a,
                               const int *__restrict__ pos_b, int64_t *__restrict__ len) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < nnz_a;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int j = crd_a[p];
        len[p] = static_cast<int64_t>(pos_b[j + 1] - pos_b[j]);
    }
}

__global__ void row_off_kernel(const int *__restrict__ pos_a, int rows,
                               const int64_t *__restrict__ off, int64_t *__restrict__ row_off) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= rows; i += gridDim.x * blockDim.x) {
        row_off[i] = off[pos_a[i]];
    }
}

// Tiles owned by row r: ceil(prod / kTile) for a long row; 1 for the first short row whose
// products start in a kShort window (the previous nonempty row is long or starts in an
// earlier window); 0 otherwise.
__device__ inline int64_t row_tile_count(const int64_t *__restrict__ row_off, int r) {
    const int64_t s = row_off[r], prod = row_off[r + 1] - s;
    if (prod == 0) return 0;
    if (prod > kShort) return (prod + kTile - 1) / kTile;
    if (s == 0) return 1;
    int lo = 0, hi = r - 1;  // the previous nonempty row: last x < r with row_off[x] < s
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (row_off[mid] < s) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    const int64_t ps = row_off[lo];
    if (s - ps > kShort) return 1;
    return (ps / kShort != s / kShort) ? 1 : 0;
}

__global__ void row_tiles_kernel(const int64_t *__restrict__ row_off, int rows,
                                 int64_t *__restrict__ row_tiles) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
        row_tiles[r] = row_tile_count(row_off, r);
    }
}

__global__ void tile_map_kernel(const int64_t *__restrict__ row_off,
                                const int64_t *__restrict__ tile_prefix, int rows,
                                int *__restrict__ tile_row, int64_t *__restrict__ tile_start) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r <= rows; r += gridDim.x * blockDim.x) {
        if (r == rows) {
            tile_start[tile_prefix[rows]] = row_off[rows];
            continue;
        }
        const int64_t t0 = tile_prefix[r], t1 = tile_prefix[r + 1];
        for (int64_t t = t0; t < t1; ++t) {
            tile_row[t] = r;
            tile_start[t] = row_off[r] + (t - t0) * kTile;
        }
    }
}

// Merge levels of a row with `tiles` tiles: ceil(log2(tiles)).
__host__ __device__ inline int merge_levels(int64_t tiles) {
    int l = 0;
    while ((static_cast<int64_t>(1) << l) < tiles) ++l;
    return l;
}

// ---- 3: expand -------------------------------------------------------------------------

// Last A entry p in [lo, hi] with off[p] <= q.
__device__ __forceinline__ int64_t entry_of(const int64_t *__restrict__ off, int64_t lo,
                                            int64_t hi, int64_t q) {
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (off[mid] <= q) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    return lo;
}

// Workgroup w writes products [w*kTile, (w+1)*kTile); lane t the kPer consecutive products
// from w*kTile + t*kPer, as 16-byte stores.
__global__ __launch_bounds__(kBlock) void expand_kernel(
    const int *__restrict__ crd_a, const float *__restrict__ val_a, int64_t nnz_a,
    const int64_t *__restrict__ off, int64_t P, const int *__restrict__ pos_b,
    const int *__restrict__ crd_b, const float *__restrict__ val_b, int *__restrict__ key,
    float *__restrict__ val) {
    __shared__ int64_t s_range[2];
    const int64_t c0 = blockIdx.x * static_cast<int64_t>(kTile);
    if (threadIdx.x < 2) {
        const int64_t q = min(c0 + (threadIdx.x ? kTile - 1 : 0), P - 1);
        s_range[threadIdx.x] = entry_of(off, 0, nnz_a - 1, q);
    }
    __syncthreads();
    const int64_t q0 = c0 + static_cast<int64_t>(threadIdx.x) * kPer;
    if (q0 >= P) return;
    int64_t p = entry_of(off, s_range[0], s_range[1], q0);
    int64_t next = off[p + 1];
    float a = val_a[p];
    int64_t bbase = pos_b[crd_a[p]] - off[p];
    int kk[kPer];
    float vv[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int64_t q = q0 + u;
        kk[u] = 0;
        vv[u] = 0.0f;
        if (q < P) {
            if (next <= q) {
                do {
                    ++p;
                    next = off[p + 1];
                } while (next <= q);
                a = val_a[p];
                bbase = pos_b[crd_a[p]] - off[p];
            }
            kk[u] = crd_b[bbase + q];
            vv[u] = a * val_b[bbase + q];
        }
    }
    if (q0 + kPer <= P) {
        int4 *kd = reinterpret_cast<int4 *>(key + q0);
        float4 *vd = reinterpret_cast<float4 *>(val + q0);
#pragma unroll
        for (int u = 0; u < kPer / 4; ++u) {
            kd[u] = make_int4(kk[4 * u], kk[4 * u + 1], kk[4 * u + 2], kk[4 * u + 3]);
            vd[u] = make_float4(vv[4 * u], vv[4 * u + 1], vv[4 * u + 2], vv[4 * u + 3]);
        }
    } else {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            if (q0 + u < P) {
                key[q0 + u] = kk[u];
                val[q0 + u] = vv[u];
            }
        }
    }
}

// ---- tile geometry shared by the sort and compress kernels ------------------------------

struct Tile {
    int row;           // owner row (the long row, or the first row of a shared tile)
    int64_t s, e;      // product range
    int n;             // e - s
    bool shared_tile;  // short rows
};

__device__ __forceinline__ Tile load_tile(const int *__restrict__ tile_row,
                                          const int64_t *__restrict__ tile_start,
                                          const int64_t *__restrict__ row_off, int64_t t) {
    Tile g;
    g.row = tile_row[t];
    g.s = tile_start[t];
    g.e = tile_start[t + 1];
    g.n = static_cast<int>(g.e - g.s);
    g.shared_tile = row_off[g.row + 1] - row_off[g.row] <= kShort;
    return g;
}

// s_mark[q] = r + 1 where row r starts at tile position q (other entries are left as the
// caller cleared them).  A shared tile's rows run from its owner to the next tile's owner.
__device__ __forceinline__ void mark_rows(int *s_mark, const Tile &g,
                                          const int *__restrict__ tile_row,
                                          const int64_t *__restrict__ row_off, int64_t t,
                                          int64_t n_tiles, int rows) {
    if (g.shared_tile) {
        const int r_end = t + 1 < n_tiles ? tile_row[t + 1] : rows;
        for (int r = g.row + threadIdx.x; r < r_end; r += kBlock) {
            const int64_t rs = row_off[r];
            if (rs < g.e && row_off[r + 1] > rs) s_mark[rs - g.s] = r + 1;
        }
    } else if (threadIdx.x == 0 && g.s == row_off[g.row]) {
        s_mark[0] = g.row + 1;
    }
}

// ---- 4: per-tile sort in LDS -----------------------------------------------------------

// Bitonic sort of n2 (a power of two, <= kTile) key/value pairs in LDS, ascending.
template <typename K>
__device__ __forceinline__ void bitonic_sort(K *s_key, float *s_val, int n2) {
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int m = threadIdx.x; m < n2 / 2; m += kBlock) {
                const int i = 2 * m - (m & (stride - 1));
                const int j = i + stride;
                const bool ascending = (i & size) == 0;
                const K ki = s_key[i], kj = s_key[j];
                if ((ki > kj) == ascending) {
                    s_key[i] = kj;
                    s_key[j] = ki;
                    const float vi = s_val[i];
                    s_val[i] = s_val[j];
                    s_val[j] = vi;
                }
            }
            __syncthreads();
        }
    }
}

// K is uint32_t when kOrdBits + col_shift <= 32, else uint64_t (col_shift = 32).  The tile
// is read from buffer 1 and written, sorted, to buffer 1 or 2 (where the row's merge levels
// start); one workgroup reads and writes only its own tile.
template <typename K>
__global__ __launch_bounds__(kBlock) void sort_tiles_kernel(
    const int *__restrict__ tile_row, const int64_t *__restrict__ tile_start, int64_t n_tiles,
    int rows, const int64_t *__restrict__ row_off, const int64_t *__restrict__ tile_prefix,
    int col_shift, int *key1, float *val1, int *__restrict__ key2, float *__restrict__ val2) {
    __shared__ K s_key[kTile];
    __shared__ float s_val[kTile];
    __shared__ int s_wave[kBlock / dev::kWave];
    const int64_t t = blockIdx.x;
    const Tile g = load_tile(tile_row, tile_start, row_off, t);
    const int base = threadIdx.x * kPer;  // blocked positions of this lane
    int ord[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) ord[u] = 0;
    if (g.shared_tile) {
        int *s_mark = reinterpret_cast<int *>(s_val);
        for (int q = threadIdx.x; q < kTile; q += kBlock) s_mark[q] = 0;
        __syncthreads();
        mark_rows(s_mark, g, tile_row, row_off, t, n_tiles, rows);
        __syncthreads();
        int c = 0;
#pragma unroll
        for (int u = 0; u < kPer; ++u) c += s_mark[base + u] != 0;
        int total = 0;
        int run = dev::block_exclusive_sum<kBlock>(c, s_wave, total);
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            run += s_mark[base + u] != 0;
            ord[u] = run - 1;
        }
        __syncthreads();
    }
    int n2 = 1;
    while (n2 < g.n) n2 <<= 1;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int q = base + u;
        if (q < g.n) {
            s_key[q] = (static_cast<K>(ord[u]) << col_shift) |
                       static_cast<K>(static_cast<uint32_t>(key1[g.s + q]));
            s_val[q] = val1[g.s + q];
        } else if (q < n2) {
            s_key[q] = ~static_cast<K>(0);
            s_val[q] = 0.0f;
        }
    }
    __syncthreads();
    bitonic_sort(s_key, s_val, n2);
    const int levels =
        g.shared_tile ? 0 : merge_levels(tile_prefix[g.row + 1] - tile_prefix[g.row]);
    int *kd = (levels & 1) ? key2 : key1;
    float *vd = (levels & 1) ? val2 : val1;
    const K mask = (static_cast<K>(1) << col_shift) - 1;
    for (int q = threadIdx.x; q < g.n; q += kBlock) {
        kd[g.s + q] = static_cast<int>(s_key[q] & mask);
        vd[g.s + q] = s_val[q];
    }
}

// ---- 5: merge levels of long rows -------------------------------------------------------

struct PairGeom {
    int64_t a_begin;  // absolute position of run A; run B follows it
    int a_len, b_len;
    int d0, d1;  // this tile's output range inside the pair
    int u, tiles_in_pair;
};

__device__ __forceinline__ PairGeom pair_geometry(const int64_t *__restrict__ row_off,
                                                  const int64_t *__restrict__ tile_prefix,
                                                  int row, int64_t tile, int level) {
    PairGeom g;
    const int64_t lt = tile - tile_prefix[row];
    const int64_t row_s = row_off[row], row_len = row_off[row + 1] - row_s;
    const int64_t run = static_cast<int64_t>(kTile) << level;
    const int64_t pair = lt >> (level + 1);
    const int64_t pair_s = pair * 2 * run;
    g.a_begin = row_s + pair_s;
    const int64_t a_len = min(run, row_len - pair_s);
    const int64_t b_len = max(static_cast<int64_t>(0), min(run, row_len - pair_s - run));
    g.a_len = static_cast<int>(a_len);
    g.b_len = static_cast<int>(b_len);
    g.u = static_cast<int>(lt - (pair << (level + 1)));
    g.tiles_in_pair = static_cast<int>((a_len + b_len + kTile - 1) / kTile);
    g.d0 = g.u * kTile;
    g.d1 = static_cast<int>(min(static_cast<int64_t>(g.d0) + kTile, a_len + b_len));
    return g;
}

// Merge-path split of output diagonal d over A[0, na) and B[0, nb), equal keys from A first:
// the number of A items among the first d outputs.
template <typename KA, typename KB>
__device__ __forceinline__ int merge_path(KA A, KB B, int na, int nb, int d) {
    int lo = max(0, d - nb), hi = min(d, na);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (A(mid) <= B(d - 1 - mid)) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// Level `level` of a row with `levels` levels reads buffer 2 when (levels - level) is odd.
__device__ __forceinline__ bool reads_buffer2(int levels, int level) {
    return ((levels - level) & 1) != 0;
}

__global__ void level_partition_kernel(const int64_t *__restrict__ tiles, int64_t n_tiles,
                                       const int *__restrict__ tile_row,
                                       const int64_t *__restrict__ row_off,
                                       const int64_t *__restrict__ tile_prefix, int level,
                                       const int *__restrict__ key1,
                                       const int *__restrict__ key2, int *__restrict__ split) {
    for (int64_t x = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; x < n_tiles;
         x += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t tile = tiles[x];
        const int row = tile_row[tile];
        const PairGeom g = pair_geometry(row_off, tile_prefix, row, tile, level);
        const int levels = merge_levels(tile_prefix[row + 1] - tile_prefix[row]);
        const int *A = (reads_buffer2(levels, level) ? key2 : key1) + g.a_begin;
        const int *B = A + g.a_len;
        split[x] = merge_path([&](int i) { return A[i]; }, [&](int i) { return B[i]; }, g.a_len,
                              g.b_len, g.d0);
    }
}

__global__ __launch_bounds__(kBlock) void level_merge_kernel(
    const int64_t *__restrict__ tiles, const int *__restrict__ tile_row,
    const int64_t *__restrict__ row_off, const int64_t *__restrict__ tile_prefix, int level,
    const int *__restrict__ split, int *__restrict__ key1, float *__restrict__ val1,
    int *__restrict__ key2, float *__restrict__ val2) {
    __shared__ int s_key[kTile];
    __shared__ float s_val[kTile];
    const int64_t x = blockIdx.x;
    const int64_t tile = tiles[x];
    const int row = tile_row[tile];
    const PairGeom g = pair_geometry(row_off, tile_prefix, row, tile, level);
    const int levels = merge_levels(tile_prefix[row + 1] - tile_prefix[row]);
    const bool from2 = reads_buffer2(levels, level);
    const int *ks = from2 ? key2 : key1;
    const float *vs = from2 ? val2 : val1;
    int *kd = from2 ? key1 : key2;
    float *vd = from2 ? val1 : val2;
    const int a0 = split[x];
    const int a1 = (g.u + 1 < g.tiles_in_pair) ? split[x + 1] : g.a_len;
    const int b0 = g.d0 - a0, b1 = g.d1 - a1;
    const int na = a1 - a0, nab = na + (b1 - b0), nb = nab - na;
    const int64_t A = g.a_begin + a0, B = g.a_begin + g.a_len + b0;
    for (int q = threadIdx.x; q < nab; q += kBlock) {
        const int64_t src = q < na ? A + q : B + (q - na);
        s_key[q] = ks[src];
        s_val[q] = vs[src];
    }
    __syncthreads();
    // lane t merges output items [t*kPer, (t+1)*kPer) of this tile into registers
    const int d = min(static_cast<int>(threadIdx.x) * kPer, nab);
    int a = merge_path([&](int i) { return s_key[i]; }, [&](int i) { return s_key[na + i]; },
                       na, nb, d);
    int b = d - a;
    int ok[kPer];
    float ov[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const bool take_a = a < na && (b >= nb || s_key[a] <= s_key[na + b]);
        // past the tile's end both sources are spent: read a valid slot, never stored
        const int src = take_a ? a : (b < nb ? na + b : 0);
        ok[u] = s_key[src];
        ov[u] = s_val[src];
        a += take_a;
        b += !take_a;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (d + u < nab) {
            s_key[d + u] = ok[u];
            s_val[d + u] = ov[u];
        }
    }
    __syncthreads();
    const int64_t out = g.a_begin + g.d0;
    for (int q = threadIdx.x; q < nab; q += kBlock) {
        kd[out + q] = s_key[q];
        vd[out + q] = s_val[q];
    }
}

// ---- 6: compress -----------------------------------------------------------------------

// Bit u set: blocked position threadIdx.x*kPer + u starts a run, i.e. a row starts there or
// its key differs from the previous position's (for position 0 of a long row's later tile,
// from the previous tile's last key).
__device__ __forceinline__ unsigned run_starts(const int *s_key, const int *s_mark,
                                               const Tile &g, const int *__restrict__ key) {
    unsigned bits = 0u;
    const int base = threadIdx.x * kPer;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int q = base + u;
        if (q < g.n) {
            bool st;
            if (s_mark[q]) {
                st = true;
            } else if (q > 0) {
                st = s_key[q] != s_key[q - 1];
            } else {
                st = s_key[0] != key[g.s - 1];
            }
            if (st) bits |= 1u << u;
        }
    }
    return bits;
}

__global__ __launch_bounds__(kBlock) void compress_count_kernel(
    const int *__restrict__ tile_row, const int64_t *__restrict__ tile_start, int64_t n_tiles,
    int rows, const int64_t *__restrict__ row_off, const int *__restrict__ key,
    int64_t *__restrict__ tile_count) {
    __shared__ int s_key[kTile];
    __shared__ int s_mark[kTile];
    __shared__ int s_wave[kBlock / dev::kWave];
    const int64_t t = blockIdx.x;
    const Tile g = load_tile(tile_row, tile_start, row_off, t);
    for (int q = threadIdx.x; q < kTile; q += kBlock) {
        s_mark[q] = 0;
        if (q < g.n) s_key[q] = key[g.s + q];
    }
    __syncthreads();
    mark_rows(s_mark, g, tile_row, row_off, t, n_tiles, rows);
    __syncthreads();
    const unsigned st = run_starts(s_key, s_mark, g, key);
    int total = 0;
    (void)dev::block_exclusive_sum<kBlock>(static_cast<int>(__popc(st)), s_wave, total);
    if (threadIdx.x == 0) tile_count[t] = total;
}

// Exclusive segmented sum across the workgroup's lanes.  Lane input: f = the lane holds a run
// start, s = the sum of its positions after its last start (all of them if none).  Output:
// carry_f = an earlier lane holds a start, carry_s = the sum of the run open where the lane
// begins (from the earlier lanes).
__device__ __forceinline__ void block_segmented_carry(bool f, double s, double *s_sum,
                                                      int *s_flag, bool &carry_f,
                                                      double &carry_s) {
    const int l = dev::lane();
    const int w = threadIdx.x / dev::kWave;
    int fi = f ? 1 : 0;
    double si = s;
#pragma unroll
    for (int off = 1; off < dev::kWave; off <<= 1) {
        const int fu = __shfl_up(fi, off, dev::kWave);
        const double su = __shfl_up(si, off, dev::kWave);
        if (l >= off) {
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
    int cf = 0;
    double cs = 0.0;
    for (int i = 0; i < w; ++i) {
        cs = s_flag[i] ? s_sum[i] : cs + s_sum[i];
        cf |= s_flag[i];
    }
    __syncthreads();
    carry_f = (cf | fe) != 0;
    carry_s = fe ? se : cs + se;
}

template <typename PosT>
__global__ __launch_bounds__(kBlock) void compress_write_kernel(
    const int *__restrict__ tile_row, const int64_t *__restrict__ tile_start, int64_t n_tiles,
    int rows, const int64_t *__restrict__ row_off, const int *__restrict__ key,
    const float *__restrict__ val, const int64_t *__restrict__ out_off,
    PosT *__restrict__ out_pos, int *__restrict__ out_crd, float *__restrict__ out_val) {
    __shared__ int s_key[kTile];
    __shared__ float s_val[kTile];
    __shared__ int s_mark[kTile];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ double s_sum[kBlock / dev::kWave];
    __shared__ int s_flag[kBlock / dev::kWave];
    const int64_t t = blockIdx.x;
    const Tile g = load_tile(tile_row, tile_start, row_off, t);
    for (int q = threadIdx.x; q < kTile; q += kBlock) {
        s_mark[q] = 0;
        if (q < g.n) {
            s_key[q] = key[g.s + q];
            s_val[q] = val[g.s + q];
        }
    }
    __syncthreads();
    mark_rows(s_mark, g, tile_row, row_off, t, n_tiles, rows);
    __syncthreads();
    const unsigned st = run_starts(s_key, s_mark, g, key);
    int total = 0;
    const int rank0 = dev::block_exclusive_sum<kBlock>(static_cast<int>(__popc(st)), s_wave, total);
    const int base = threadIdx.x * kPer;
    // lane-local segmented sums
    double part[kPer];
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int q = base + u;
        const double v = q < g.n ? static_cast<double>(s_val[q]) : 0.0;
        acc = (st & (1u << u)) ? v : acc + v;
        part[u] = acc;
    }
    bool carry_f = false;
    double carry_s = 0.0;
    block_segmented_carry(st != 0, acc, s_sum, s_flag, carry_f, carry_s);
    // A run ends at q when q + 1 starts a run or q is the tile's last position; its result
    // goes to the index of its start.  Positions before the tile's first start continue the
    // previous tile's last run, which that tile completes.
    const int64_t out_base = out_off[t];
    const int64_t row_end = g.shared_tile ? g.e : row_off[g.row + 1];
    int rk[kPer];
    float rv[kPer];
    unsigned ends = 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int q = base + u;
        rk[u] = 0;
        rv[u] = 0.0f;
        if (q >= g.n) continue;
        const unsigned upto = st & ((2u << u) - 1);
        if (!carry_f && upto == 0) continue;
        bool end = true;
        if (q + 1 < g.n) {
            end = (u + 1 < kPer) ? (st & (1u << (u + 1))) != 0
                                 : (s_mark[q + 1] != 0 || s_key[q + 1] != s_key[q]);
        }
        if (!end) continue;
        double sum = upto ? part[u] : carry_s + part[u];
        const int k = s_key[q];
        if (q + 1 == g.n) {
            // a long row's run may continue into the following tiles
            for (int64_t x = g.e; x < row_end && key[x] == k; ++x) {
                sum += static_cast<double>(val[x]);
            }
        }
        ends |= 1u << u;
        rk[u] = k;
        rv[u] = static_cast<float>(sum);
    }
    // row offsets: a row's first run; the empty rows just before it share its offset
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int q = base + u;
        if (q < g.n && s_mark[q]) {
            const int r = s_mark[q] - 1;
            const PosT v = static_cast<PosT>(out_base + rank0 + __popc(st & ((1u << u) - 1)));
            out_pos[r] = v;
            const int64_t rs = row_off[r];
            for (int x = r - 1; x >= 0 && row_off[x] == rs; --x) out_pos[x] = v;
        }
    }
    __syncthreads();
    // the run ending at u started at the last start at or before u
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (ends & (1u << u)) {
            const int idx = rank0 + __popc(st & ((2u << u) - 1)) - 1;
            s_key[idx] = rk[u];
            s_val[idx] = rv[u];
        }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < total; q += kBlock) {
        out_crd[out_base + q] = s_key[q];
        out_val[out_base + q] = s_val[q];
    }
}

// Rows that start at P (trailing empty rows, and the final offset) get nnz.
template <typename PosT>
__global__ void tail_pos_kernel(const int64_t *__restrict__ row_off, int rows, int64_t P,
                                int64_t nnz, PosT *__restrict__ out_pos) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r <= rows; r += gridDim.x * blockDim.x) {
        if (row_off[r] == P) out_pos[r] = static_cast<PosT>(nnz);
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
    const hipStream_t s = call.stream();
    const int rows = a->dim_i_size;
    const int64_t nnz_a = a->dim_j_length;
    const char *name = "spgemm: expand+sort+merge+compress";
    NACHO_TRY(call.timer_start(name));

    // 1. products per A entry and per row
    int64_t *len = nullptr, *off = nullptr, *row_off = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_a) + 1, &len));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_a) + 1, &off));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &row_off));
    if (nnz_a > 0) {
        lengths_kernel<<<grid_for(nnz_a, 256), 256, 0, s>>>(a->dim_j_indices, nnz_a,
                                                            b->dim_j_offsets, len);
        NACHO_TRY_HIP(hipGetLastError());
    }
    NACHO_TRY(scan::exclusive_scan_i64(call, len, nnz_a, off));
    row_off_kernel<<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, s>>>(
        a->dim_j_offsets, rows, off, row_off);
    NACHO_TRY_HIP(hipGetLastError());

    // 2. tiles
    int64_t *row_tiles = nullptr, *tile_prefix = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &row_tiles));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &tile_prefix));
    if (rows > 0) {
        row_tiles_kernel<<<grid_for(rows, 256), 256, 0, s>>>(row_off, rows, row_tiles);
        NACHO_TRY_HIP(hipGetLastError());
    }
    NACHO_TRY(scan::exclusive_scan_i64(call, row_tiles, rows, tile_prefix));
    std::vector<int64_t> h_prefix(static_cast<size_t>(rows) + 1);
    NACHO_TRY_HIP(hipMemcpyAsync(h_prefix.data(), tile_prefix, sizeof(int64_t) * (rows + 1),
                                 hipMemcpyDeviceToHost, s));
    int64_t P = 0;
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.read_back(&P, row_off + rows, sizeof(P)));  // synchronises the copy too
    const int64_t T = h_prefix[static_cast<size_t>(rows)];
    NACHO_TRY(call.timer_start(name));

    // merge plan: long rows ordered by level count, so each level's active tiles are a prefix
    std::vector<std::pair<int, int>> long_rows;  // (levels, row)
    int max_levels = 0;
    for (int i = 0; i < rows; ++i) {
        const int64_t nt = h_prefix[static_cast<size_t>(i) + 1] - h_prefix[static_cast<size_t>(i)];
        if (nt > kMaxRowTiles) return NACHO_ERR_INDEX_OVERFLOW;
        const int lv = merge_levels(nt);
        if (lv > 0) long_rows.emplace_back(lv, i);
        max_levels = std::max(max_levels, lv);
    }
    std::stable_sort(long_rows.begin(), long_rows.end(),
                     [](const std::pair<int, int> &x, const std::pair<int, int> &y) {
                         return x.first > y.first;
                     });
    std::vector<int64_t> h_tiles;
    std::vector<int64_t> level_tiles(static_cast<size_t>(max_levels), 0);
    for (const auto &lr : long_rows) {
        const int64_t t0 = h_prefix[static_cast<size_t>(lr.second)];
        const int64_t t1 = h_prefix[static_cast<size_t>(lr.second) + 1];
        for (int64_t t = t0; t < t1; ++t) h_tiles.push_back(t);
        for (int l = 0; l < lr.first; ++l) level_tiles[static_cast<size_t>(l)] += t1 - t0;
    }

    int *key1 = nullptr, *key2 = nullptr, *tile_row = nullptr, *split = nullptr;
    float *val1 = nullptr, *val2 = nullptr;
    int64_t *tile_start = nullptr, *d_tiles = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(T) + 1, &tile_start));
    if (P > 0) {
        NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &key1));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &val1));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(T), &tile_row));
        if (max_levels > 0) {
            NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &key2));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(P), &val2));
            NACHO_TRY(call.scratch_n(h_tiles.size(), &d_tiles));
            NACHO_TRY(call.scratch_n(h_tiles.size(), &split));
            NACHO_TRY_HIP(hipMemcpyAsync(d_tiles, h_tiles.data(),
                                         sizeof(int64_t) * h_tiles.size(),
                                         hipMemcpyHostToDevice, s));
            NACHO_TRY_HIP(hipStreamSynchronize(s));  // h_tiles is pageable host memory
        }
    }
    tile_map_kernel<<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, s>>>(
        row_off, tile_prefix, rows, tile_row, tile_start);
    NACHO_TRY_HIP(hipGetLastError());

    if (P > 0) {
        // 3. expand
        expand_kernel<<<static_cast<unsigned>((P + kTile - 1) / kTile), kBlock, 0, s>>>(
            a->dim_j_indices, a->values, nnz_a, off, P, b->dim_j_offsets, b->dim_j_indices,
            b->values, key1, val1);
        NACHO_TRY_HIP(hipGetLastError());
        // 4. sort
        const int cb = col_bits(b->dim_j_size);
        if (cb + kOrdBits <= 32) {
            sort_tiles_kernel<uint32_t><<<static_cast<unsigned>(T), kBlock, 0, s>>>(
                tile_row, tile_start, T, rows, row_off, tile_prefix, cb, key1, val1, key2, val2);
        } else {
            sort_tiles_kernel<uint64_t><<<static_cast<unsigned>(T), kBlock, 0, s>>>(
                tile_row, tile_start, T, rows, row_off, tile_prefix, 32, key1, val1, key2, val2);
        }
        NACHO_TRY_HIP(hipGetLastError());
        // 5. merge levels
        for (int level = 0; level < max_levels; ++level) {
            const int64_t n = level_tiles[static_cast<size_t>(level)];
            level_partition_kernel<<<grid_for(n, 256), 256, 0, s>>>(
                d_tiles, n, tile_row, row_off, tile_prefix, level, key1, key2, split);
            NACHO_TRY_HIP(hipGetLastError());
            level_merge_kernel<<<static_cast<unsigned>(n), kBlock, 0, s>>>(
                d_tiles, tile_row, row_off, tile_prefix, level, split, key1, val1, key2, val2);
            NACHO_TRY_HIP(hipGetLastError());
        }
    }

    // 6. compress
    int64_t *tile_count = nullptr, *out_off = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(T) + 1, &tile_count));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(T) + 1, &out_off));
    if (T > 0) {
        compress_count_kernel<<<static_cast<unsigned>(T), kBlock, 0, s>>>(
            tile_row, tile_start, T, rows, row_off, key1, tile_count);
        NACHO_TRY_HIP(hipGetLastError());
    }
    NACHO_TRY(scan::exclusive_scan_i64(call, tile_count, T, out_off));
    int64_t nnz = 0;
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.read_back(&nnz, out_off + T, sizeof(nnz)));
    if (sizeof(PosT) == sizeof(int32_t) && nnz > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;
    NACHO_TRY(call.timer_start(name));

    PosT *pos = nullptr;
    int *crd = nullptr;
    float *val = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pos));
    NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &crd));
    NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &val));
    tail_pos_kernel<PosT><<<grid_for(static_cast<int64_t>(rows) + 1, 256), 256, 0, s>>>(
        row_off, rows, P, nnz, pos);
    NACHO_TRY_HIP(hipGetLastError());
    if (T > 0) {
        compress_write_kernel<PosT><<<static_cast<unsigned>(T), kBlock, 0, s>>>(
            tile_row, tile_start, T, rows, row_off, key1, val1, out_off, pos, crd, val);
        NACHO_TRY_HIP(hipGetLastError());
    }
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());

    z->rows = rows;
    z->cols = b->dim_j_size;
    z->nnz = nnz;
    z->pos = pos;
    z->crd = crd;
    z->val = val;
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
