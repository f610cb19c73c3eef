// Fused three-way CSR union for csr_add_3 (Z = A + B + C) on gfx950: one merge over the
// three operands, with no intermediate (A + B) in HBM.
//
// Reference path replaced: the csr_add_3 kernel (compiler.cpp:114), whose generated code
// co-iterates the three operands in one loop nest over the lattice of a + b + c
// (compute.cpp:1297-1337, lattice points with absent operands removed); its benchmark
// compares that fused kernel with two chained csr_add calls (benchmarks/csr_add_3.py:21-29).
//
// Structure (the two-operand csr_merge.hip pipeline, widened to three operands):
//  * Items are every row's A, B and C entries plus one row-end item; T = nnzA + nnzB + nnzC
//    + rows items are cut into tiles of kTile.
//  * csr3_partition_kernel: one thread per tile boundary.  The row comes from a binary search
//    on S(r) = posA[r] + posB[r] + posC[r] + r; inside the row, the three-way merge-path
//    split is a nested search: over how many items of the (A, B) merge are taken, each probe
//    finding the (A, B) merge's item at that rank with a two-way merge-path search.  Equal
//    keys order A before B before C.  A key group (equal coordinates in two or three
//    operands) never spans tiles: a split inside a group takes the rest of the group.
//  * csr3_count_kernel / csr3_write_kernel: each workgroup owns a contiguous chunk of tiles;
//    tiles are staged in LDS from registers loaded one tile ahead; lane t walks items
//    [t*IPT, (t+1)*IPT) of its tile from a nested merge-path search in LDS.  A step takes
//    the smallest head (ties A, B, C), or consumes a row end.  The first item of a key group
//    emits (its value is the sum of the group's present values, in the order (a + b) + c,
//    the others are peeked at their heads); later items of the group are skipped by
//    comparing with the previous item's key, so groups may straddle lanes.  The count
//    kernel totals the result length for the early readback and stores every lane's start;
//    the write kernel walks from those starts, stages its outputs in LDS and stores them
//    coalesced.
// Every value is the reference's float32 sum in operand order, so results are bit-exact.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "csr_merge.hpp"
#include "device_utils.hpp"
#include "runtime.hpp"

namespace nacho {
namespace csr3 {

constexpr int kBlock = 256;
constexpr int kIpt = 11;                 // items per lane
constexpr int kTile = kBlock * kIpt;     // 2816 items per tile
constexpr int kCap = kTile + 3;          // a split takes at most two more group members;
                                         // one more slot for the read past the last entry
constexpr int kLoads = (kCap + kBlock - 1) / kBlock;
constexpr int kSteps = kIpt + 2;         // a lane's range plus the group rule's two items
constexpr int kMaxChunk = 64;
constexpr int kPartBlock = 64;           // partition workgroups: boundaries over every CU
constexpr int kMax = INT_MAX;            // head sentinel: that operand's row is exhausted
static_assert(kCap < 65536, "tile-local offsets are packed in 16 bits");

// ---- three-way merge-path split inside one row ------------------------------------------

// The three-way split of one row at in-row diagonal d: how many of the row's A, B and C
// entries (given as [aS, aE), [bS, bE), [cS, cE) through the readers A(), B(), C()) come
// before the d-th item of the row's merged order (ties: A, then B, then C).  Nested search:
// X = the (A, B) merge, Y = C; x = number of X items taken is the largest with
// X[x - 1] <= Y[d - x] (X first on ties); X[q] is found by a two-way split at rank q + 1.
template <typename RA, typename RB, typename RC>
__device__ __forceinline__ void split3(RA A, RB B, RC C, int aS, int aE, int bS, int bE, int cS,
                                       int cE, int d, int &a, int &b, int &c) {
    const int la = aE - aS, lb = bE - bS, lc = cE - cS;
    // a' (A taken) of the plain two-way split of the (A, B) merge at diagonal q
    auto split2 = [&](int q) {
        int lo = max(0, q - lb), hi = min(la, q);
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (A(aS + mid) <= B(bS + q - 1 - mid)) {
                lo = mid + 1;
            } else {
                hi = mid;
            }
        }
        return lo;
    };
    auto x_at = [&](int q) {  // key of item q of the (A, B) merge, q in [0, la + lb)
        const int ta = split2(q + 1), tb = q + 1 - ta;
        const int ka = ta > 0 ? A(aS + ta - 1) : INT_MIN;
        const int kb = tb > 0 ? B(bS + tb - 1) : INT_MIN;
        return max(ka, kb);
    };
    int lo = max(0, d - lc), hi = min(la + lb, d);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (x_at(mid) <= C(cS + d - 1 - mid)) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    const int ta = split2(lo);
    a = aS + ta;
    b = bS + lo - ta;
    c = cS + d - lo;
}

// ---- partition ----------------------------------------------------------------------------

// One thread per tile boundary t in [0, num_tiles]: the split (row, a, b, c) of diagonal
// min(t * kTile, total), moved past the rest of a key group it would cut.  Thread 0 also
// zeroes the accumulator of the count kernel's length total.
__global__ __launch_bounds__(kPartBlock) void csr3_partition_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, const int *__restrict__ pc, const int *__restrict__ cc,
    int rows, int total, int num_tiles, int *__restrict__ split,
    unsigned long long *__restrict__ done) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t > num_tiles) return;
    if (t == 0) *done = 0ull;
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);
    int lo = 0, hi = rows;  // largest row r with S(r) <= diag
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pa[mid] + pb[mid] + pc[mid] + mid <= diag) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    const int r = lo;
    int a = pa[r], b = pb[r], c = pc[r];
    if (r < rows) {
        const int aE = pa[r + 1], bE = pb[r + 1], cE = pc[r + 1];
        const int aS = a, bS = b, cS = c;
        const int d = diag - (aS + bS + cS + r);  // 0 <= d <= row length
        split3([&](int x) { return ca[x]; }, [&](int y) { return cb[y]; },
               [&](int z) { return cc[z]; }, aS, aE, bS, bE, cS, cE, d, a, b, c);
        // key group rule: B or C entries equal to the last key taken join this side
        int last = INT_MIN;
        if (a > aS) last = max(last, ca[a - 1]);
        if (b > bS) last = max(last, cb[b - 1]);
        if (c > cS) last = max(last, cc[c - 1]);
        if (last != INT_MIN) {
            if (b < bE && cb[b] == last) ++b;
            if (c < cE && cc[c] == last) ++c;
        }
    }
    split[4 * t] = r;
    split[4 * t + 1] = a;
    split[4 * t + 2] = b;
    split[4 * t + 3] = c;
}

// ---- tile staging -------------------------------------------------------------------------

struct Split3 {
    int r0, a0, b0, c0, r1, a1, b1, c1;
};

__device__ __forceinline__ Split3 lds_split3(const int *s_split, int i) {
    const int *p = s_split + 4 * i;
    return Split3{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]};
}

struct Staged3 {
    int crd[kLoads];
    int val[kLoads];  // float bits
    int pa[kLoads];
    int pb[kLoads];
    int pc[kLoads];
};

// Loads of one tile, issued unconditionally with clamped indices (lanes past the end
// re-read the last entry), consumed only when staged.
template <bool VALUES>
__device__ __forceinline__ void fetch3(Staged3 &st, const Split3 &sp, const int *__restrict__ pa,
                                       const int *__restrict__ ca, const float *__restrict__ va,
                                       const int *__restrict__ pb, const int *__restrict__ cb,
                                       const float *__restrict__ vb, const int *__restrict__ pc,
                                       const int *__restrict__ cc, const float *__restrict__ vc,
                                       int tid) {
    const int na = sp.a1 - sp.a0, nab = na + (sp.b1 - sp.b0);
    const int n = nab + (sp.c1 - sp.c0), nr = sp.r1 - sp.r0 + 1;
    if (n > 0) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int k = min(tid + j * kBlock, n - 1);
            const int *cp;
            const float *vp;
            int off;
            if (k < na) {
                cp = ca;
                vp = va;
                off = sp.a0 + k;
            } else if (k < nab) {
                cp = cb;
                vp = vb;
                off = sp.b0 + (k - na);
            } else {
                cp = cc;
                vp = vc;
                off = sp.c0 + (k - nab);
            }
            st.crd[j] = cp[off];
            if (VALUES) st.val[j] = __float_as_int(vp[off]);
        }
    }
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int kr = sp.r0 + min(tid + j * kBlock, nr - 1);
        st.pa[j] = pa[kr];
        st.pb[j] = pb[kr];
        st.pc[j] = pc[kr];
    }
}

// LDS layout of a staged tile: s_crd = A's range, then B's, then C's (s_val likewise);
// s_row[k] = (posA[r0+k] clipped to the tile, minus a0) | (the same for B) << 16 and
// s_rowc[k] = the same for C.

template <bool VALUES>
__device__ __forceinline__ void stage3(const Staged3 &st, const Split3 &sp, int *s_crd,
                                       float *s_val, unsigned *s_row, int *s_rowc, int tid) {
    const int n = (sp.a1 - sp.a0) + (sp.b1 - sp.b0) + (sp.c1 - sp.c0);
    const int nr = sp.r1 - sp.r0 + 1;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int k = tid + j * kBlock;
        if (k < n) {
            s_crd[k] = st.crd[j];
            if (VALUES) s_val[k] = __int_as_float(st.val[j]);
        }
        if (k < nr) {
            const unsigned ra = static_cast<unsigned>(max(st.pa[j], sp.a0) - sp.a0);
            const unsigned rb = static_cast<unsigned>(max(st.pb[j], sp.b0) - sp.b0);
            s_row[k] = ra | (rb << 16);
            s_rowc[k] = max(st.pc[j], sp.c0) - sp.c0;
        }
    }
}

// ---- one lane's walk ----------------------------------------------------------------------

struct Lane3Out {
    int crd[kSteps];
    float val[kSteps];
    unsigned valid, row_ends;
    int count;
    int first_row;
};

// A lane's start: (row k | A position << 16, B position | C position << 16), tile-local.
// GIVEN: taken from `start` (the count kernel's); otherwise searched and stored to `start`.
template <bool VALUES, bool COUNT_ONLY, bool GIVEN>
__device__ __forceinline__ void walk3(Lane3Out &out, const Split3 &sp, int tile, const int *s_crd,
                                      const float *s_val, const unsigned *s_row,
                                      const int *s_rowc, int tid, uint2 &start) {
    const int na = sp.a1 - sp.a0, nb = sp.b1 - sp.b0, nc = sp.c1 - sp.c0;
    const int nab = na + nb, n = nab + nc, nr = sp.r1 - sp.r0 + 1;
    // tile-local row starts in the staged arrays (A at [0, na), B at [na, nab), C at
    // [nab, n)); row nr - 1 ends at the tile's end
    auto ra = [&](int k) { return static_cast<int>(s_row[k] & 0xffffu); };
    auto rb = [&](int k) { return na + static_cast<int>(s_row[k] >> 16); };
    auto rc = [&](int k) { return nab + s_rowc[k]; };
    auto ea = [&](int k) { return k < nr - 1 ? ra(k + 1) : na; };
    auto eb = [&](int k) { return k < nr - 1 ? rb(k + 1) : nab; };
    auto ec = [&](int k) { return k < nr - 1 ? rc(k + 1) : n; };
    auto at = [&](int x) { return s_crd[min(x, kCap - 1)]; };

    const int tile_lo = tile * kTile;
    const int tile_start = sp.a0 + sp.b0 + sp.c0 + sp.r0;
    const int tile_end = sp.a1 + sp.b1 + sp.c1 + sp.r1;
    const int g_lo = tid == 0 ? tile_start : tile_lo + tid * kIpt;
    const int steps = tid == kBlock - 1 ? tile_end - g_lo
                                        : min(tile_lo + (tid + 1) * kIpt, tile_end) - g_lo;
    int k = 0, ia = 0, ib = na, ic = nab;
    if (GIVEN) {
        k = min(static_cast<int>(start.x & 0xffffu), nr - 1);
        ia = static_cast<int>(start.x >> 16);
        ib = static_cast<int>(start.y & 0xffffu);
        ic = static_cast<int>(start.y >> 16);
    } else if (tid > 0 && g_lo < tile_end) {
        // the row of item g_lo: largest k with tile_start + ra + rb + rc (local) + k <= g_lo
        const int local = g_lo - tile_start;
        int lo = 0, hi = nr - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ra(mid) + (rb(mid) - na) + (rc(mid) - nab) + mid <= local) {
                lo = mid;
            } else {
                hi = mid - 1;
            }
        }
        k = lo;
        const int d = local - (ra(k) + (rb(k) - na) + (rc(k) - nab) + k);
        split3(at, at, at, ra(k), ea(k), rb(k), eb(k), rc(k), ec(k), d, ia, ib, ic);
    }
    if (!GIVEN) {
        start = make_uint2(static_cast<unsigned>(k) | (static_cast<unsigned>(ia) << 16),
                           static_cast<unsigned>(ib) | (static_cast<unsigned>(ic) << 16));
    }
    out.first_row = sp.r0 + k;
    int aE = ea(k), bE = eb(k), cE = ec(k);
    // key of the item before the lane's first one in its row (a group it continues)
    int last = INT_MIN;
    if (ia > ra(k)) last = max(last, at(ia - 1));
    if (ib > rb(k)) last = max(last, at(ib - 1));
    if (ic > rc(k)) last = max(last, at(ic - 1));
    int xa = ia < aE ? at(ia) : kMax;
    int xb = ib < bE ? at(ib) : kMax;
    int xc = ic < cE ? at(ic) : kMax;
    unsigned valid = 0, row_ends = 0;
    int count = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        if (!COUNT_ONLY) {
            out.crd[s] = 0;
            out.val[s] = 0.0f;
        }
        if (s < steps) {
            if (xa == kMax && xb == kMax && xc == kMax) {  // row end
                row_ends |= 1u << s;
                k = min(k + 1, nr - 1);
                aE = ea(k);
                bE = eb(k);
                cE = ec(k);
                last = INT_MIN;
                xa = ia < aE ? at(ia) : kMax;
                xb = ib < bE ? at(ib) : kMax;
                xc = ic < cE ? at(ic) : kMax;
            } else {
                const int x = min(xa, min(xb, xc));
                const int which = xa == x ? 0 : (xb == x ? 1 : 2);  // ties: A, B, C
                const bool emit = x != last;
                if (COUNT_ONLY) {
                    count += emit;
                } else {
                    out.crd[s] = x;
                    if (VALUES) {
                        // the group's sum in operand order, from its first item
                        float v = s_val[min(which == 0 ? ia : (which == 1 ? ib : ic), kCap - 1)];
                        if (which == 0 && xb == x) v = v + s_val[min(ib, kCap - 1)];
                        if (which <= 1 && xc == x) v = v + s_val[min(ic, kCap - 1)];
                        out.val[s] = v;
                    }
                    valid |= static_cast<unsigned>(emit) << s;
                }
                last = x;
                if (which == 0) {
                    ++ia;
                    xa = ia < aE ? at(ia) : kMax;
                } else if (which == 1) {
                    ++ib;
                    xb = ib < bE ? at(ib) : kMax;
                } else {
                    ++ic;
                    xc = ic < cE ? at(ic) : kMax;
                }
            }
        }
    }
    out.valid = valid;
    out.row_ends = row_ends;
    out.count = COUNT_ONLY ? count : static_cast<int>(__popc(valid));
}

// ---- kernels ------------------------------------------------------------------------------

__device__ __forceinline__ void stage_splits3(int *s_split, const int *__restrict__ split,
                                              int t0, int t1) {
    const int n = 4 * (t1 - t0 + 1);
    for (int i = threadIdx.x; i < n; i += kBlock) s_split[i] = split[4 * t0 + i];
}

// Output count of each chunk, and their sum (the result length) stored to `length_out` by
// the last workgroup.
__global__ __launch_bounds__(kBlock) void csr3_count_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, const int *__restrict__ pc, const int *__restrict__ cc,
    int num_tiles, int chunk, const int *__restrict__ split, unsigned *__restrict__ chunk_count,
    unsigned long long *__restrict__ done, int64_t *__restrict__ length_out,
    uint2 *__restrict__ starts) {
    __shared__ int s_crd[kCap];
    __shared__ unsigned s_row[kCap];
    __shared__ int s_rowc[kCap];
    __shared__ unsigned s_wave[kBlock / dev::kWave];
    __shared__ int s_split[4 * (kMaxChunk + 1)];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) {
        if (tid == 0) {
            chunk_count[blockIdx.x] = 0u;
            dev::add_to_total(0u, done, length_out);
        }
        return;
    }
    stage_splits3(s_split, split, t0, t1);
    __syncthreads();
    Split3 sp = lds_split3(s_split, 0);
    Staged3 st;
    fetch3<false>(st, sp, pa, ca, nullptr, pb, cb, nullptr, pc, cc, nullptr, tid);
    stage3<false>(st, sp, s_crd, nullptr, s_row, s_rowc, tid);
    __syncthreads();
    unsigned mine = 0;
    for (int t = t0; t < t1; ++t) {
        const Split3 nsp = lds_split3(s_split, t + 1 < t1 ? t + 1 - t0 : t - t0);
        if (t + 1 < t1) fetch3<false>(st, nsp, pa, ca, nullptr, pb, cb, nullptr, pc, cc, nullptr, tid);
        Lane3Out lo;
        uint2 start;
        walk3<false, true, false>(lo, sp, t, s_crd, nullptr, s_row, s_rowc, tid, start);
        starts[static_cast<size_t>(t) * kBlock + tid] = start;
        mine += static_cast<unsigned>(lo.count);
        if (t + 1 < t1) {
            __syncthreads();  // every lane is done reading this tile
            stage3<false>(st, nsp, s_crd, nullptr, s_row, s_rowc, tid);
            __syncthreads();
        }
        sp = nsp;
    }
    unsigned total = dev::wave_sum(mine);
    if (dev::lane() == 0) s_wave[tid / dev::kWave] = total;
    __syncthreads();
    if (tid == 0) {
        unsigned all = 0;
#pragma unroll
        for (int w = 0; w < kBlock / dev::kWave; ++w) all += s_wave[w];
        chunk_count[blockIdx.x] = all;
        dev::add_to_total(all, done, length_out);
    }
}

// Writes Z: crd and values at the chunk's offset (the counts of every earlier chunk), pos[r+1]
// at every row end.  Every global write is kept inside the result buffers (`cap` entries,
// `rows` + 1 offsets).
__global__ __launch_bounds__(kBlock) void csr3_write_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const float *__restrict__ va,
    const int *__restrict__ pb, const int *__restrict__ cb, const float *__restrict__ vb,
    const int *__restrict__ pc, const int *__restrict__ cc, const float *__restrict__ vc,
    int num_tiles, int chunk, const int *__restrict__ split,
    const unsigned *__restrict__ chunk_count, const uint2 *__restrict__ starts, int rows,
    long long cap, int *__restrict__ pz, int *__restrict__ cz, float *__restrict__ vz) {
    __shared__ int s_crd[kCap];
    __shared__ float s_val[kCap];
    __shared__ unsigned s_row[kCap];
    __shared__ int s_rowc[kCap];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_split[4 * (kMaxChunk + 1)];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) return;
    stage_splits3(s_split, split, t0, t1);
    int before = 0;
    for (int i = tid; i < static_cast<int>(blockIdx.x); i += kBlock) before += chunk_count[i];
    int base = 0;
    (void)dev::block_exclusive_sum<kBlock>(before, s_wave, base);  // (ends synchronised)
    if (blockIdx.x == 0 && tid == 0) pz[0] = 0;
    Split3 sp = lds_split3(s_split, 0);
    Staged3 st;
    uint2 start = starts[static_cast<size_t>(t0) * kBlock + tid];
    fetch3<true>(st, sp, pa, ca, va, pb, cb, vb, pc, cc, vc, tid);
    stage3<true>(st, sp, s_crd, s_val, s_row, s_rowc, tid);
    __syncthreads();
    for (int t = t0; t < t1; ++t) {
        const Split3 nsp = lds_split3(s_split, t + 1 < t1 ? t + 1 - t0 : t - t0);
        uint2 next_start = start;
        if (t + 1 < t1) {
            fetch3<true>(st, nsp, pa, ca, va, pb, cb, vb, pc, cc, vc, tid);
            next_start = starts[static_cast<size_t>(t + 1) * kBlock + tid];
        }
        Lane3Out lo;
        walk3<true, false, true>(lo, sp, t, s_crd, s_val, s_row, s_rowc, tid, start);
        int tile_total = 0;
        const int offset = dev::block_exclusive_sum<kBlock>(lo.count, s_wave, tile_total);
        // (the scan's barriers also mean every lane is done reading this tile's inputs)
        int o = offset, r = lo.first_row;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (lo.row_ends & (1u << s)) {
                if (r < rows) pz[r + 1] = base + o;
                ++r;
            }
            if (lo.valid & (1u << s)) {
                if (o < kCap) {
                    s_crd[o] = lo.crd[s];
                    s_val[o] = lo.val[s];
                }
                ++o;
            }
        }
        __syncthreads();
        for (int q = tid; q < min(tile_total, kCap); q += kBlock) {
            const long long dst = static_cast<long long>(base) + q;
            if (dst < cap) {
                cz[dst] = s_crd[q];
                vz[dst] = s_val[q];
            }
        }
        base += tile_total;
        __syncthreads();  // staged outputs consumed
        if (t + 1 < t1) {
            stage3<true>(st, nsp, s_crd, s_val, s_row, s_rowc, tid);
            __syncthreads();
        }
        sp = nsp;
        start = next_start;
    }
}

// ---- host ---------------------------------------------------------------------------------

// Z = A + B + C (csr_add_3): the union of three CSR matrices, valued by the reference's
// lattice for (a + b) + c: a sum of the present operands in that order, one float32 add per
// extra operand (compute.cpp:413-491 with absent operands removed).  Partition, count and
// write kernels on the call's stream; the call returns once the count kernel has published
// the result length (the write kernel may still run, ordered before later work on the stream).
int csr_add3_fused(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c, nacho_csr *z,
                   int32_t num_blocks, int32_t threads_per_block, void *stream,
                   const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    auto bad = [](const nacho_csr *t) {
        return !t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0 ||
               !t->dim_j_offsets || (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values));
    };
    if (bad(a) || bad(b) || bad(c)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size ||
        a->dim_i_size != c->dim_i_size || a->dim_j_size != c->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size;
    const long long cap =
        static_cast<long long>(a->dim_j_length) + b->dim_j_length + c->dim_j_length;
    const long long total = cap + rows;
    if (total > static_cast<long long>(INT_MAX) - 2 * kTile) return NACHO_ERR_INDEX_OVERFLOW;
    const int num_tiles = total > 0 ? static_cast<int>((total + kTile - 1) / kTile) : 1;

    Call call(stream, alloc);
    int *pz = nullptr, *cz = nullptr;
    float *vz = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pz));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &cz));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &vz));
    int *split = nullptr;
    NACHO_TRY(call.scratch_n(4 * (static_cast<size_t>(num_tiles) + 1), &split));
    int resident = 0;
    NACHO_TRY(resident_grid(reinterpret_cast<const void *>(csr3_write_kernel), kBlock,
                            &resident));
    int chunk = (num_tiles + resident - 1) / resident;
    if (chunk > kMaxChunk) chunk = kMaxChunk;
    const int grid = (num_tiles + chunk - 1) / chunk;
    unsigned *counts = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 6, &counts));
    unsigned long long *done =
        reinterpret_cast<unsigned long long *>(counts + ((grid + 2) & ~1));
    uint2 *starts = nullptr;  // every lane's start in every tile, from the count kernel
    NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles) * kBlock, &starts));
    int64_t *length_out = nullptr;
    NACHO_TRY(call.length_word(&length_out));

    const hipStream_t s = call.stream();
    NACHO_TRY(call.timer_start("csr_add_3: fused three-way merge"));
    csr3_partition_kernel<<<ceil_div(static_cast<size_t>(num_tiles) + 1, kPartBlock), kPartBlock,
                            0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, b->dim_j_offsets, b->dim_j_indices,
        c->dim_j_offsets, c->dim_j_indices, rows, static_cast<int>(total), num_tiles, split,
        done);
    NACHO_TRY_HIP(hipGetLastError());
    csr3_count_kernel<<<grid, kBlock, 0, s>>>(a->dim_j_offsets, a->dim_j_indices,
                                             b->dim_j_offsets, b->dim_j_indices,
                                             c->dim_j_offsets, c->dim_j_indices, num_tiles,
                                             chunk, split, counts, done, length_out, starts);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.mark_length());
    csr3_write_kernel<<<grid, kBlock, 0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, a->values, b->dim_j_offsets, b->dim_j_indices,
        b->values, c->dim_j_offsets, c->dim_j_indices, c->values, num_tiles, chunk, split,
        counts, starts, rows, cap, pz, cz, vz);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());
    int64_t nz = 0;
    NACHO_TRY(call.wait_length(&nz));
    if (nz > cap) return NACHO_ERR_MALFORMED_INPUT;
    if (nz == 0) {
        call.drop_result(cz);
        call.drop_result(vz);
        cz = nullptr;
        vz = nullptr;
    }
    z->dim_i_size = rows;
    z->dim_j_size = a->dim_j_size;
    z->dim_j_offsets = pz;
    z->dim_j_length = static_cast<int32_t>(nz);
    z->dim_j_indices = cz;
    z->values = vz;
    z->nnz = static_cast<int32_t>(nz);
    call.commit();
    return NACHO_OK;
}

}  // namespace csr3
}  // namespace nacho

extern "C" {

int nacho_gpu_csr_add_3_f32(const nacho_csr *a, const nacho_csr *b, const nacho_csr *c,
                            nacho_csr *z, int32_t num_blocks, int32_t threads_per_block,
                            void *stream, const nacho_allocator *alloc) {
    return nacho::csr3::csr_add3_fused(a, b, c, z, num_blocks, threads_per_block, stream,
                                       alloc);
}

}  // extern "C"
