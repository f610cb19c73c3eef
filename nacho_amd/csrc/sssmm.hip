// Masked SpGEMM (sssmm): Z_ik = sum_j a_ij * b_jk * c_ik over the (i, k) stored in C that
// at least one product reaches, for gfx950.
//
// Reference path replaced: sssmm (compiler.cpp:150-153, GPU-only), whose generated kernel
// expands the products of A B restricted to C's pattern through the scatter-reduction path
// (stitch_and_generate_gpu.cpp:14-138).  Its benchmark checks the structure against
// cuSPARSE A*B followed by csr_mul with C (benchmarks/sssmm.py:46-51): the result is C's
// pattern intersected with the product's pattern, and no entry of A B outside C is formed.
//
// Here every mask entry (i, k) is an inner product of row i of A with column k of B.  Both
// operands are indexed by j through per-row / per-column hash tables, so the entry costs
// min(|A_i|, |B_k|) probes: the shorter list is walked and each j is looked up in the other
// operand's table.  On power-law inputs that is far less than expanding every product of
// A B (R-MAT scale 20 squared and masked by itself: 1.1e9 probes against 6.0e9 products).
//
//   count_cols_kernel, scan          column counts of B, column offsets
//   table_sizes_kernel (x2), scans   hash table sizes (power of two >= 2 * length) and bases
//   fill_kernel                      empty tables
//   transpose_kernel                 B's entries into columns (row ids + values), and into
//                                    the per-column tables keyed by row id
//   rows_table_kernel                A's entries into the per-row tables keyed by column id
//   work_kernel, scan                per mask entry: row, probes = min(|A_i|, |B_k|), which
//                                    side is walked, which table is probed
//   chunk_bounds_kernel              first / last mask entry of every 4096-probe chunk
//   probe_kernel                     one chunk per workgroup: load-balanced decode of probes
//                                    to mask entries (max-scan of entry start marks in LDS),
//                                    walk + probe, (a * b) * c per hit in float32 as written,
//                                    segmented wavefront sums in float64, one atomic add per
//                                    entry and wavefront
//   keep_kernel, scan, output_kernel the entries that some product reached, in C's order
//
// Values: each term is rounded as the reference writes it, ((a * b) * c) in float32, and the
// terms of an entry are summed in float64 and rounded once.  The order of the float64 sums
// across wavefronts and chunks follows atomic arrival, so values are reproducible within
// one float32 rounding; the structure is exact.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "device_utils.hpp"
#include "runtime.hpp"
#include "scan.hpp"

namespace nacho {
namespace sssmm {

constexpr int kBlock = 256;
constexpr int kChunk = 4096;       // probes per workgroup
constexpr int kPer = kChunk / kBlock;
constexpr int kBatch = 2;  // probe rounds whose loads are issued together
constexpr uint32_t kEmptyKey = 0xffffffffu;
constexpr uint64_t kEmptySlot = 0x00000000ffffffffull;  // value bits 0, key empty
constexpr uint32_t kWalkB = 0x80000000u;  // entry flag: walk B's column, probe A's row table

using dev::block_exclusive_max;
using dev::last_le;

__device__ __forceinline__ int pad(int i) { return i + (i >> 4); }
constexpr int kPadded = kChunk + kChunk / 16;

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__device__ __forceinline__ void table_insert(uint64_t *table, int64_t base, uint32_t mask,
                                             uint32_t key, float value) {
    const uint64_t word = (static_cast<uint64_t>(__float_as_uint(value)) << 32) | key;
    uint32_t h = mix(key) & mask;
    for (;;) {
        auto *slot = reinterpret_cast<unsigned long long *>(table + base + h);
        if (atomicCAS(slot, static_cast<unsigned long long>(kEmptySlot),
                      static_cast<unsigned long long>(word)) == kEmptySlot) {
            return;
        }
        h = (h + 1) & mask;
    }
}

// Value stored under `key`, or false when the table has no such key.
__device__ __forceinline__ bool table_find(const uint64_t *__restrict__ table, int64_t base,
                                           uint32_t mask, uint32_t key, float *value) {
    uint32_t h = mix(key) & mask;
    for (;;) {
        const uint64_t w = table[base + h];
        const uint32_t k = static_cast<uint32_t>(w);
        if (k == key) {
            *value = __uint_as_float(static_cast<uint32_t>(w >> 32));
            return true;
        }
        if (k == kEmptyKey) return false;
        h = (h + 1) & mask;
    }
}

__global__ void fill_kernel(uint64_t *__restrict__ p, int64_t n, uint64_t v) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        p[i] = v;
    }
}

__global__ void zero_kernel(int64_t *__restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        p[i] = 0;
    }
}

__global__ void zero_int_kernel(int *__restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        p[i] = 0;
    }
}

// Workgroup b counts the columns of entries [b*kSpan, (b+1)*kSpan): columns below kHotCols in
// an LDS histogram flushed with one global atomic per nonzero bin (power-law operands put
// most entries in a few low-numbered hub columns, whose global counters would serialise
// every entry's atomic), the others with a global atomic each.
constexpr int kHotCols = 8192;
constexpr int kSpan = 16 * kBlock;  // entries per workgroup of the two kernels below

__global__ __launch_bounds__(kBlock) void count_cols_kernel(const int *__restrict__ crd,
                                                            int64_t n, int cols,
                                                            unsigned long long *__restrict__ count) {
    __shared__ unsigned hist[kHotCols];
    const int hot = min(cols, kHotCols);
    for (int i = threadIdx.x; i < hot; i += kBlock) hist[i] = 0u;
    __syncthreads();
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kSpan;
    const int64_t hi = min(n, lo + kSpan);
    for (int64_t e = lo + threadIdx.x; e < hi; e += kBlock) {
        const int k = crd[e];
        if (k < hot) {
            atomicAdd(&hist[k], 1u);
        } else {
            atomicAdd(&count[k], 1ull);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < hot; i += kBlock) {
        if (hist[i]) atomicAdd(&count[i], static_cast<unsigned long long>(hist[i]));
    }
}

// Table of a list of `len` entries: the smallest power of two >= 2 * len (0 when empty).
__device__ __forceinline__ int64_t table_size(int64_t len) {
    if (len == 0) return 0;
    int64_t s = 2;
    while (s < 2 * len) s <<= 1;
    return s;
}

// size[x] for the n lists; lengths from an offsets array (pos, n + 1 entries, int32) or from
// counts (int64).
__global__ void table_sizes_kernel(const int *__restrict__ pos, const int64_t *__restrict__ count,
                                   int n, int64_t *__restrict__ size) {
    for (int x = blockIdx.x * blockDim.x + threadIdx.x; x < n; x += gridDim.x * blockDim.x) {
        const int64_t len = pos ? static_cast<int64_t>(pos[x + 1] - pos[x]) : count[x];
        size[x] = table_size(len);
    }
}

// Workgroup b takes entries [lo, hi) = [b*kSpan, (b+1)*kSpan) of a list split by the offsets
// p (n + 1 entries); [r_lo, r_hi] holds the rows of its first and last entry and so bounds
// every entry's row search.  False (for the whole workgroup) when the span is empty.
__device__ __forceinline__ bool span_rows(const int *__restrict__ p, int n, int64_t nnz,
                                          int64_t &lo, int64_t &hi, int &r_lo, int &r_hi) {
    __shared__ int s_rows[2];
    lo = static_cast<int64_t>(blockIdx.x) * kSpan;
    hi = min(nnz, lo + kSpan);
    if (lo >= hi) return false;
    if (threadIdx.x == 0) {
        const int first = static_cast<int>(last_le(p, 0, n - 1, lo));
        s_rows[0] = first;
        s_rows[1] = static_cast<int>(last_le(p, first, n - 1, hi - 1));
    }
    __syncthreads();
    r_lo = s_rows[0];
    r_hi = s_rows[1];
    return true;
}

// B's entries into columns (CSC) and into the per-column tables keyed by row id.
__global__ __launch_bounds__(kBlock) void transpose_kernel(
    const int *__restrict__ pb, int inner, const int *__restrict__ cb,
    const float *__restrict__ vb, int64_t nnz_b, const int64_t *__restrict__ col_off,
    unsigned long long *__restrict__ col_fill, const int64_t *__restrict__ tab_off,
    int *__restrict__ csc_row, float *__restrict__ csc_val, uint64_t *__restrict__ tab_b) {
    int64_t lo, hi;
    int r_lo, r_hi;
    if (!span_rows(pb, inner, nnz_b, lo, hi, r_lo, r_hi)) return;
    for (int64_t e = lo + threadIdx.x; e < hi; e += kBlock) {
        const int j = static_cast<int>(last_le(pb, r_lo, r_hi, e));
        const int k = cb[e];
        const float v = vb[e];
        const int64_t slot = col_off[k] + static_cast<int64_t>(atomicAdd(&col_fill[k], 1ull));
        csc_row[slot] = j;
        csc_val[slot] = v;
        const int64_t size = tab_off[k + 1] - tab_off[k];
        table_insert(tab_b, tab_off[k], static_cast<uint32_t>(size - 1), static_cast<uint32_t>(j),
                     v);
    }
}

// A's entries into the per-row tables keyed by column id.
__global__ __launch_bounds__(kBlock) void rows_table_kernel(
    const int *__restrict__ pa, int rows, const int *__restrict__ ca,
    const float *__restrict__ va, int64_t nnz_a, const int64_t *__restrict__ tab_off,
    uint64_t *__restrict__ tab_a) {
    int64_t lo, hi;
    int r_lo, r_hi;
    if (!span_rows(pa, rows, nnz_a, lo, hi, r_lo, r_hi)) return;
    for (int64_t e = lo + threadIdx.x; e < hi; e += kBlock) {
        const int i = static_cast<int>(last_le(pa, r_lo, r_hi, e));
        const int64_t size = tab_off[i + 1] - tab_off[i];
        table_insert(tab_a, tab_off[i], static_cast<uint32_t>(size - 1),
                     static_cast<uint32_t>(ca[e]), va[e]);
    }
}

// Per mask entry e = (i, k): probes = min(|A_i|, |B_k|) (0 when either is empty), the walked
// list's base, and the probed table's base and mask (kWalkB set when B's column is walked).
__global__ void work_kernel(const int *__restrict__ pc, int rows, const int *__restrict__ cc,
                            int64_t nnz_c, const int *__restrict__ pa,
                            const unsigned long long *__restrict__ col_count,
                            const int64_t *__restrict__ col_off,
                            const int64_t *__restrict__ tab_a_off,
                            const int64_t *__restrict__ tab_b_off, int64_t *__restrict__ work,
                            int64_t *__restrict__ walk_base, int64_t *__restrict__ probe_base,
                            uint32_t *__restrict__ probe_mask) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < nnz_c;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int i = static_cast<int>(last_le(pc, 0, rows - 1, e));
        const int k = cc[e];
        const int64_t la = pa[i + 1] - pa[i];
        const int64_t lb = static_cast<int64_t>(col_count[k]);
        const bool walk_b = lb < la;
        work[e] = (la == 0 || lb == 0) ? 0 : (walk_b ? lb : la);
        walk_base[e] = walk_b ? col_off[k] : static_cast<int64_t>(pa[i]);
        const int64_t t0 = walk_b ? tab_a_off[i] : tab_b_off[k];
        const int64_t t1 = walk_b ? tab_a_off[i + 1] : tab_b_off[k + 1];
        probe_base[e] = t0;
        probe_mask[e] = static_cast<uint32_t>(t1 - t0 - 1) | (walk_b ? kWalkB : 0u);
    }
}

// First and last mask entry of every chunk of kChunk probes.
__global__ void chunk_bounds_kernel(const int64_t *__restrict__ woff, int64_t nnz_c,
                                    int64_t total, int64_t chunks, int64_t *__restrict__ bounds) {
    for (int64_t x = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
         x < 2 * chunks; x += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = x >> 1;
        const int64_t q = (x & 1) ? min((c + 1) * kChunk, total) - 1 : c * kChunk;
        bounds[x] = last_le(woff, 0, nnz_c - 1, q);
    }
}

// Segmented inclusive sum over a wavefront: lanes holding the same `seg` are contiguous.
// Returns the running sums; the last lane of each segment holds the segment's total.
__device__ __forceinline__ void wave_segmented_sum(int seg, double &v, int &h) {
    const int l = dev::lane();
    // every lane takes part in each shuffle (a shuffle under a lane-dependent condition
    // would read inactive lanes)
    const int prev = __shfl_up(seg, 1, dev::kWave);
    int head = (l == 0 || prev != seg) ? l : 0;
#pragma unroll
    for (int o = 1; o < dev::kWave; o <<= 1) {
        const int n = __shfl_up(head, o, dev::kWave);
        if (l >= o) head = max(head, n);
    }
#pragma unroll
    for (int o = 1; o < dev::kWave; o <<= 1) {
        const double nv = __shfl_up(v, o, dev::kWave);
        const int nh = __shfl_up(h, o, dev::kWave);
        if (l - o >= head) {
            v += nv;
            h += nh;
        }
    }
}

__global__ __launch_bounds__(kBlock) void probe_kernel(
    const int64_t *__restrict__ woff, const int64_t *__restrict__ bounds, int64_t total,
    const int64_t *__restrict__ walk_base, const int64_t *__restrict__ probe_base,
    const uint32_t *__restrict__ probe_mask, const int *__restrict__ ca,
    const float *__restrict__ va, const int *__restrict__ csc_row,
    const float *__restrict__ csc_val, const uint64_t *__restrict__ tab_a,
    const uint64_t *__restrict__ tab_b, const float *__restrict__ vc,
    double *__restrict__ acc, int *__restrict__ hit) {
    __shared__ int s_e[kPadded];
    __shared__ int s_wave[kBlock / dev::kWave];
    // neighbouring chunks (a mask row's probes into one table) on one XCD, 64 at a time:
    // probe_kernel fetched 11% less at C4
    const int64_t chunk = dev::xcd_block<64>();
    const int64_t c0 = chunk * kChunk;
    const int n = static_cast<int>(min(static_cast<int64_t>(kChunk), total - c0));
    const int64_t e_lo = bounds[2 * chunk], e_hi = bounds[2 * chunk + 1];
    // decode: s_e[x] = (mask entry of probe c0 + x) - e_lo
    for (int x = threadIdx.x; x < kChunk; x += kBlock) s_e[pad(x)] = 0;
    __syncthreads();
    for (int64_t e = e_lo + 1 + threadIdx.x; e <= e_hi; e += kBlock) {
        const int64_t x = woff[e] - c0;
        if (x >= 0 && x < n) atomicMax(&s_e[pad(static_cast<int>(x))], static_cast<int>(e - e_lo));
    }
    __syncthreads();
    const int base = threadIdx.x * kPer;
    int m = 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) m = max(m, s_e[pad(base + u)]);
    int run = block_exclusive_max(m, s_wave);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        run = max(run, s_e[pad(base + u)]);
        s_e[pad(base + u)] = run;
    }
    __syncthreads();
    // probes, kBlock consecutive ones per round so a wavefront holds 64 consecutive probes.
    // kBatch rounds at a time: each step of a probe's chain of dependent loads (the entry's
    // fields, the walked entry, the table slot) is issued for all of them before the next,
    // so that kBatch chains are in flight per lane.
    static_assert(kPer % kBatch == 0, "rounds come in whole batches");
    for (int r0 = 0; r0 < kPer; r0 += kBatch) {
        bool live[kBatch];
        int64_t e[kBatch], wb[kBatch], tb[kBatch];
        uint32_t pm[kBatch];
#pragma unroll
        for (int g = 0; g < kBatch; ++g) {
            const int x = threadIdx.x + (r0 + g) * kBlock;
            live[g] = x < n;
            e[g] = e_lo + (live[g] ? s_e[pad(x)] : 0);
        }
#pragma unroll
        for (int g = 0; g < kBatch; ++g) {
            const int x = threadIdx.x + (r0 + g) * kBlock;
            pm[g] = probe_mask[e[g]];
            wb[g] = walk_base[e[g]] + (c0 + x - woff[e[g]]);
            tb[g] = probe_base[e[g]];
        }
        uint32_t key[kBatch];
        float own[kBatch];  // the walked entry's value
#pragma unroll
        for (int g = 0; g < kBatch; ++g) {
            key[g] = 0;
            own[g] = 0.0f;
            if (live[g]) {
                const bool walk_b = (pm[g] & kWalkB) != 0;
                key[g] = static_cast<uint32_t>(walk_b ? csc_row[wb[g]] : ca[wb[g]]);
                own[g] = walk_b ? csc_val[wb[g]] : va[wb[g]];
            }
        }
        uint32_t slot[kBatch];
        uint64_t w[kBatch];
#pragma unroll
        for (int g = 0; g < kBatch; ++g) {  // first probe of every table
            const uint32_t mask = pm[g] & ~kWalkB;
            slot[g] = mix(key[g]) & mask;
            w[g] = kEmptySlot;
            if (live[g]) w[g] = ((pm[g] & kWalkB) ? tab_a : tab_b)[tb[g] + slot[g]];
        }
        float cv[kBatch];
#pragma unroll
        for (int g = 0; g < kBatch; ++g) cv[g] = live[g] ? vc[e[g]] : 0.0f;
#pragma unroll
        for (int g = 0; g < kBatch; ++g) {
            double v = 0.0;
            int h = 0;
            if (live[g]) {
                const uint32_t mask = pm[g] & ~kWalkB;
                const uint64_t *tab = (pm[g] & kWalkB) ? tab_a : tab_b;
                uint64_t ww = w[g];
                uint32_t hh = slot[g];
                // collisions: the next two slots per step, both loads issued together (a
                // wavefront waits for its longest chain; the second slot is nearly always in
                // the same line); the first of them that holds the key or is empty ends it
                while (static_cast<uint32_t>(ww) != key[g] &&
                       static_cast<uint32_t>(ww) != kEmptyKey) {
                    const uint32_t h1 = (hh + 1) & mask, h2 = (hh + 2) & mask;
                    const uint64_t w1 = tab[tb[g] + h1], w2 = tab[tb[g] + h2];
                    const bool first = static_cast<uint32_t>(w1) == key[g] ||
                                       static_cast<uint32_t>(w1) == kEmptyKey;
                    ww = first ? w1 : w2;
                    hh = first ? h1 : h2;
                }
                if (static_cast<uint32_t>(ww) == key[g]) {
                    const float other = __uint_as_float(static_cast<uint32_t>(ww >> 32));
                    // a * b with a from A and b from B, as the reference writes it
                    const float ab = (pm[g] & kWalkB) ? other * own[g] : own[g] * other;
                    v = static_cast<double>(ab * cv[g]);
                    h = 1;
                }
            }
            const int seg = live[g] ? static_cast<int>(e[g] - e_lo) : -1;
            wave_segmented_sum(seg, v, h);
            const int l = dev::lane();
            const int next_seg = __shfl_down(seg, 1, dev::kWave);
            const bool tail = live[g] && (l == dev::kWave - 1 || next_seg != seg);
            if (tail && h > 0) {
                atomicAdd(&acc[e[g]], v);
                hit[e[g]] = 1;
            }
        }
    }
}

__global__ void keep_kernel(const int *__restrict__ hit, int64_t n, int64_t *__restrict__ keep) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        keep[e] = hit[e] ? 1 : 0;
    }
}

// Z.pos[r] = kept entries of C before row r; kept entries copied in C's order.
__global__ void output_kernel(const int *__restrict__ pc, int rows, const int *__restrict__ cc,
                              int64_t nnz_c, const int64_t *__restrict__ koff,
                              const int *__restrict__ hit, const double *__restrict__ acc,
                              int *__restrict__ pz, int *__restrict__ cz, float *__restrict__ vz) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t first = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    for (int64_t r = first; r <= rows; r += stride) pz[r] = static_cast<int>(koff[pc[r]]);
    for (int64_t e = first; e < nnz_c; e += stride) {
        if (hit[e]) {
            const int64_t o = koff[e];
            cz[o] = cc[e];
            vz[o] = static_cast<float>(acc[e]);
        }
    }
}

__global__ void zero_pos_kernel(int *__restrict__ p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= n; i += gridDim.x * blockDim.x) p[i] = 0;
}

unsigned grid_for(int64_t n) {
    const int64_t g = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

bool bad_csr(const nacho_csr *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0) return true;
    if (!t->dim_j_offsets) return true;
    if (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values)) return true;
    return false;
}

int multiply(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c, nacho_csr *z,
             int32_t num_blocks, int32_t threads_per_block, void *stream,
             const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csr(a) || bad_csr(b) || bad_csr(c)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_j_size != b->dim_i_size || c->dim_i_size != a->dim_i_size ||
        c->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size, inner = b->dim_i_size, cols = b->dim_j_size;
    const int64_t nnz_a = a->dim_j_length, nnz_b = b->dim_j_length, nnz_c = c->dim_j_length;
    Call call(stream, alloc);
    const hipStream_t st = call.stream();
    const char *name = "sssmm: tables+probe+output";
    int *pz = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pz));
    NACHO_TRY(call.timer_start(name));
    if (nnz_a == 0 || nnz_b == 0 || nnz_c == 0) {
        zero_pos_kernel<<<grid_for(static_cast<int64_t>(rows) + 1), kBlock, 0, st>>>(pz, rows);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.collect_timer());
        z->dim_i_size = rows;
        z->dim_j_size = cols;
        z->dim_j_offsets = pz;
        call.commit();
        return NACHO_OK;
    }

    // columns of B and the table sizes
    int64_t *col_count = nullptr, *col_off = nullptr, *col_fill = nullptr;
    int64_t *tsize_b = nullptr, *toff_b = nullptr, *tsize_a = nullptr, *toff_a = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cols) + 1, &col_count));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cols) + 1, &col_off));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cols) + 1, &col_fill));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cols) + 1, &tsize_b));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cols) + 1, &toff_b));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &tsize_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &toff_a));
    zero_kernel<<<grid_for(cols), kBlock, 0, st>>>(col_count, cols);
    zero_kernel<<<grid_for(cols), kBlock, 0, st>>>(col_fill, cols);
    const unsigned span_grid =
        static_cast<unsigned>(std::max<int64_t>(1, (nnz_b + kSpan - 1) / kSpan));
    count_cols_kernel<<<span_grid, kBlock, 0, st>>>(
        b->dim_j_indices, nnz_b, cols, reinterpret_cast<unsigned long long *>(col_count));
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(scan::exclusive_scan_i64(call, col_count, cols, col_off));
    table_sizes_kernel<<<grid_for(cols), kBlock, 0, st>>>(nullptr, col_count, cols, tsize_b);
    table_sizes_kernel<<<grid_for(rows), kBlock, 0, st>>>(a->dim_j_offsets, nullptr, rows,
                                                          tsize_a);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(scan::exclusive_scan_i64(call, tsize_b, cols, toff_b));
    NACHO_TRY(scan::exclusive_scan_i64(call, tsize_a, rows, toff_a));
    NACHO_TRY(call.timer_stop());
    int64_t sizes[2] = {0, 0};
    NACHO_TRY(call.read_back(&sizes[0], toff_b + cols, sizeof(int64_t)));
    NACHO_TRY(call.read_back(&sizes[1], toff_a + rows, sizeof(int64_t)));
    // A table's mask is kept in 31 bits (bit 31 flags the walked side), so no table may
    // exceed 2^31 slots.  Table sizes are powers of two, so a larger one (2^32 slots or
    // more, for a row or column of more than 2^30 entries) would make its side's total at
    // least 2^32.
    if (sizes[0] >= (int64_t{1} << 32) || sizes[1] >= (int64_t{1} << 32)) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }
    NACHO_TRY(call.timer_start(name));

    // tables and B's columns
    uint64_t *tab_b = nullptr, *tab_a = nullptr;
    int *csc_row = nullptr;
    float *csc_val = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(sizes[0]), &tab_b));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(sizes[1]), &tab_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b), &csc_row));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_b), &csc_val));
    fill_kernel<<<grid_for(sizes[0]), kBlock, 0, st>>>(tab_b, sizes[0], kEmptySlot);
    fill_kernel<<<grid_for(sizes[1]), kBlock, 0, st>>>(tab_a, sizes[1], kEmptySlot);
    transpose_kernel<<<span_grid, kBlock, 0, st>>>(
        b->dim_j_offsets, inner, b->dim_j_indices, b->values, nnz_b, col_off,
        reinterpret_cast<unsigned long long *>(col_fill), toff_b, csc_row, csc_val, tab_b);
    rows_table_kernel<<<static_cast<unsigned>(std::max<int64_t>(1, (nnz_a + kSpan - 1) / kSpan)),
                        kBlock, 0, st>>>(a->dim_j_offsets, rows, a->dim_j_indices, a->values,
                                         nnz_a, toff_a, tab_a);
    NACHO_TRY_HIP(hipGetLastError());

    // probes per mask entry
    int64_t *work = nullptr, *woff = nullptr, *walk_base = nullptr, *probe_base = nullptr;
    uint32_t *probe_mask = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c) + 1, &work));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c) + 1, &woff));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c), &walk_base));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c), &probe_base));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c), &probe_mask));
    work_kernel<<<grid_for(nnz_c), kBlock, 0, st>>>(
        c->dim_j_offsets, rows, c->dim_j_indices, nnz_c, a->dim_j_offsets,
        reinterpret_cast<const unsigned long long *>(col_count), col_off, toff_a, toff_b, work,
        walk_base, probe_base, probe_mask);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(scan::exclusive_scan_i64(call, work, nnz_c, woff));
    NACHO_TRY(call.timer_stop());
    int64_t total = 0;
    NACHO_TRY(call.read_back(&total, woff + nnz_c, sizeof(total)));
    NACHO_TRY(call.timer_start(name));
    const int64_t chunks = (total + kChunk - 1) / kChunk;
    if (chunks > INT_MAX) return NACHO_ERR_INDEX_OVERFLOW;

    // probes
    double *acc = nullptr;
    int *hit = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c), &acc));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(nnz_c), &hit));
    fill_kernel<<<grid_for(nnz_c), kBlock, 0, st>>>(reinterpret_cast<uint64_t *>(acc), nnz_c, 0ull);
    zero_int_kernel<<<grid_for(nnz_c), kBlock, 0, st>>>(hit, nnz_c);
    NACHO_TRY_HIP(hipGetLastError());
    if (chunks > 0) {
        int64_t *bounds = nullptr;
        NACHO_TRY(call.scratch_n(2 * static_cast<size_t>(chunks), &bounds));
        chunk_bounds_kernel<<<grid_for(2 * chunks), kBlock, 0, st>>>(woff, nnz_c, total, chunks,
                                                                     bounds);
        probe_kernel<<<static_cast<unsigned>(chunks), kBlock, 0, st>>>(
            woff, bounds, total, walk_base, probe_base, probe_mask, a->dim_j_indices, a->values,
            csc_row, csc_val, tab_a, tab_b, c->values, acc, hit);
        NACHO_TRY_HIP(hipGetLastError());
    }

    // result
    int64_t *keep = work, *koff = woff;  // the work counts are spent
    keep_kernel<<<grid_for(nnz_c), kBlock, 0, st>>>(hit, nnz_c, keep);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(scan::exclusive_scan_i64(call, keep, nnz_c, koff));
    NACHO_TRY(call.timer_stop());
    int64_t nnz = 0;
    NACHO_TRY(call.read_back(&nnz, koff + nnz_c, sizeof(nnz)));
    NACHO_TRY(call.timer_start(name));
    int *cz = nullptr;
    float *vz = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &cz));
    NACHO_TRY(call.result_n(static_cast<size_t>(nnz), &vz));
    output_kernel<<<grid_for(nnz_c > rows ? nnz_c : static_cast<int64_t>(rows) + 1), kBlock, 0,
                    st>>>(c->dim_j_offsets, rows, c->dim_j_indices, nnz_c, koff, hit, acc, pz,
                          cz, vz);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    NACHO_TRY(call.collect_timer());
    z->dim_i_size = rows;
    z->dim_j_size = cols;
    z->dim_j_offsets = pz;
    z->dim_j_length = static_cast<int32_t>(nnz);
    z->dim_j_indices = cz;
    z->values = vz;
    z->nnz = static_cast<int32_t>(nnz);
    call.commit();
    return NACHO_OK;
}

}  // namespace sssmm
}  // namespace nacho

extern "C" int nacho_gpu_sssmm_f32(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c,
                                   nacho_csr *z, int32_t num_blocks, int32_t threads_per_block,
                                   void *stream, const nacho_allocator *alloc) {
    return nacho::sssmm::multiply(a, b, c, z, num_blocks, threads_per_block, stream, alloc);
}
