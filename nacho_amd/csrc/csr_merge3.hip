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
//    comparing with the previous item's key, so groups may straddle lanes.  The write
//    kernel stages its outputs in LDS and stores them coalesced.
//  * The count: where few entries can be duplicates (the rows where two or three operands
//    have entries hold few of them), a row pass and a search per such entry count the
//    duplicates of each write chunk (search mode, below); otherwise the count kernel walks
//    every tile as above and stores every lane's start for the write kernel (tile mode).
//    Either way it totals the result length for the early readback.
// Every value is the reference's float32 sum in operand order, so results are bit-exact.
#include <hip/hip_runtime.h>

#include <algorithm>
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
constexpr int kPartLanes = 8;            // lanes that search one tile boundary together
constexpr int kMax = INT_MAX;            // head sentinel: that operand's row is exhausted
static_assert(kCap < 65536, "tile-local offsets are packed in 16 bits");

// ---- three-way merge-path split inside one row ------------------------------------------

// The three-way split of one row at in-row diagonal d: how many of the row's A, B and C
// entries (given as [aS, aE), [bS, bE), [cS, cE) through the readers A(), B(), C()) come
// before the d-th item of the row's merged order (ties: A, then B, then C).  Nested search:
// X = the (A, B) merge, Y = C; x = number of X items taken is the largest with
// X[x - 1] <= Y[d - x] (X first on ties); X[q] is found by a two-way split at rank q + 1.
// G lanes call it together (dev::group_last_true; G = 1: one lane alone): the outer search
// and the final two-way split are shared by the group, and each lane finds its own X[q] with
// a binary search.
template <int G, typename RA, typename RB, typename RC>
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
    // x: one past the last m in [lo, hi) with X[m] <= Y[d - 1 - m]
    const int lo = max(0, d - lc), hi = min(la + lb, d);
    const int x = dev::group_last_true<G>(
                      lo - 1, hi - 1, [&](int m) { return x_at(m) <= C(cS + d - 1 - m); }) + 1;
    // the two-way split of the (A, B) merge at x
    const int lo2 = max(0, x - lb), hi2 = min(la, x);
    const int ta = dev::group_last_true<G>(
                       lo2 - 1, hi2 - 1, [&](int m) { return A(aS + m) <= B(bS + x - 1 - m); }) + 1;
    a = aS + ta;
    b = bS + x - ta;
    c = cS + d - x;
}

// ---- partition ----------------------------------------------------------------------------

// ---- sparse-overlap count: row pass + duplicate search ------------------------------------
// The union's output count is nnzA + nnzB + nnzC less its duplicates: the B entries whose
// column is in A's row (|A ∩ B|) and the C entries whose column is in A's or B's row
// (|C ∩ (A ∪ B)|).  Duplicates only occur in rows where at least two operands have entries;
// when those rows hold few entries (three C2 operands: 0.8M searches for 50M entries), a
// search per entry of the smaller side counts them without streaming every coordinate
// through a walk.  Per row the searched entries are
//   |A ∩ B|: the smaller of A's and B's entries (A on a tie), each searched in the other;
//   |C ∩ (A ∪ B)|: C's entries, each searched in A and in B, when C has at most as many as A
//            and B together; otherwise A's entries searched in C, and B's entries searched
//            in C and counted only when absent from A.
// Each duplicate is charged to the write chunk holding the searched entry (a key group never
// spans tiles, so that is the chunk that merges it).
// The row pass (extra workgroups of the partition launch) writes one record per row with
// searches; the count kernel totals them (M) and picks the mode it and the write kernel follow:
//   search: M * kSearchRatio <= nnzA + nnzB + nnzC: the count kernel searches every entry,
//           chunk_count receives each write chunk's duplicates, and the write chunk starting
//           at tile t0 starts at output a0 + b0 + c0 of t0's split less the duplicates
//           before it; write lanes search their own starts.
//   count:  the tile walk of csr3_count_kernel (chunk output counts, stored lane starts).
constexpr int kModeCount = 0;
constexpr int kModeSearch = 1;
constexpr int kSearchRatio = 16;
// Ways of the search mode's lower bounds (probes per round + 1).
constexpr int kSearchWays = 8;
constexpr int kRowPassMaxBlocks = 1024;  // workgroups of the row pass (a multiple of kBlock)
constexpr int kRowUnroll = 8;  // row steps of the row pass whose loads are issued together
constexpr int kRowPassMinEntriesPerRow = 8;

struct Rows3 {
    // record k of row-pass workgroup b: rec[2 * (blk_base[b] + k)] = {first search (within
    // b's), posA[r], posB[r], posC[r]} and rec[2 * (blk_base[b] + k) + 1] = {la, lb, lc, 0}
    int4 *rec;
    int *blk_base;   // record region of each workgroup (its first row)
    int *blk_elems;  // searches per workgroup
    int *blk_recs;   // records per workgroup
    int *mode;       // kModeSearch or kModeCount (stored by the count kernel)
    int rows_per_thread;
    int nb;  // workgroups of the row pass
};

// Searches of one row with la, lb, lc entries in A, B and C.
__device__ __forceinline__ int dup_searches(int la, int lb, int lc) {
    const int wb = (la > 0 && lb > 0) ? min(la, lb) : 0;
    const int lab = la + lb;
    return wb + ((lc > 0 && lab > 0) ? min(lc, lab) : 0);
}

// Workgroup `block` of the row pass (one wave): rows_per_thread * 64 consecutive rows;
// nothing waits on other workgroups.  Step j covers rows row0 + j*64 .. +63, one per lane
// (coalesced), so the records come out in row order from one wave scan per step; kRowUnroll
// steps' loads are issued together.
__device__ __forceinline__ void row_pass3(const int *__restrict__ pa, const int *__restrict__ pb,
                                          const int *__restrict__ pc, int rows, const Rows3 &rp,
                                          int block) {
    static_assert(kPartBlock == dev::kWave, "the row pass scans within one wave");
    const int l = threadIdx.x;
    const int rpt = rp.rows_per_thread;
    const long long row0 = static_cast<long long>(block) * kPartBlock * rpt;  // < rows (or 0)
    int4 *out = rp.rec + 2 * row0;
    int e_base = 0, r_base = 0;  // searches and records of the rows before
    for (int j0 = 0; j0 < rpt && rows > 0; j0 += kRowUnroll) {
        int a0[kRowUnroll], a1[kRowUnroll], b0[kRowUnroll], b1[kRowUnroll], c0[kRowUnroll],
            c1[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const long long r = row0 + static_cast<long long>(j0 + u) * dev::kWave + l;
            const long long rc = r < rows ? r : rows - 1;
            a0[u] = pa[rc];
            a1[u] = pa[rc + 1];
            b0[u] = pb[rc];
            b1[u] = pb[rc + 1];
            c0[u] = pc[rc];
            c1[u] = pc[rc + 1];
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const long long r = row0 + static_cast<long long>(j0 + u) * dev::kWave + l;
            const int la = a1[u] - a0[u], lb = b1[u] - b0[u], lc = c1[u] - c0[u];
            const bool in = j0 + u < rpt && r < rows;
            const int w = in ? dup_searches(la, lb, lc) : 0;
            const int e_incl = dev::wave_inclusive_sum(w);
            const int r_incl = dev::wave_inclusive_sum(static_cast<int>(w > 0));
            if (w > 0) {
                int4 *o = out + 2 * (r_base + r_incl - 1);
                o[0] = make_int4(e_base + e_incl - w, a0[u], b0[u], c0[u]);
                o[1] = make_int4(la, lb, lc, 0);
            }
            e_base += __builtin_amdgcn_readlane(e_incl, dev::kWave - 1);
            r_base += __builtin_amdgcn_readlane(r_incl, dev::kWave - 1);
        }
    }
    if (l == 0) {
        rp.blk_base[block] = static_cast<int>(row0);
        rp.blk_elems[block] = e_base;
        rp.blk_recs[block] = r_base;
    }
}

// kPartLanes lanes per tile boundary t in [0, num_tiles]: the split (row, a, b, c) of
// diagonal min(t * kTile, total), moved past the rest of a key group it would cut.  Boundary 0
// also zeroes the accumulator of the count kernel's length total, and the first n_counts
// boundaries the chunk counts (n_counts <= num_tiles + 1).  Workgroups from part_blocks on
// run the row pass.
__global__ __launch_bounds__(kPartBlock) void csr3_partition_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, const int *__restrict__ pc, const int *__restrict__ cc,
    int rows, int total, int num_tiles, int *__restrict__ split,
    unsigned long long *__restrict__ done, unsigned *__restrict__ zero_counts, int n_counts,
    int part_blocks, Rows3 rp) {
    if (static_cast<int>(blockIdx.x) >= part_blocks) {  // the row pass's workgroups
        row_pass3(pa, pb, pc, rows, rp, static_cast<int>(blockIdx.x) - part_blocks);
        return;
    }
    const int t = (static_cast<int>(blockIdx.x) * kPartBlock + static_cast<int>(threadIdx.x)) /
                  kPartLanes;
    if (t > num_tiles) return;  // whole lane groups
    const bool lead = threadIdx.x % kPartLanes == 0;
    if (lead && t < n_counts) zero_counts[t] = 0u;
    if (lead && t == 0) dev::zero_total(done);
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);
    // largest row r with S(r) <= diag (S(0) = 0)
    const int r = dev::group_last_true<kPartLanes>(
        0, rows, [&](int x) { return pa[x] + pb[x] + pc[x] + x <= diag; });
    int a = pa[r], b = pb[r], c = pc[r];
    if (r < rows) {
        const int aE = pa[r + 1], bE = pb[r + 1], cE = pc[r + 1];
        const int aS = a, bS = b, cS = c;
        const int d = diag - (aS + bS + cS + r);  // 0 <= d <= row length
        split3<kPartLanes>([&](int x) { return ca[x]; }, [&](int y) { return cb[y]; },
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
    if (lead) {
        split[4 * t] = r;
        split[4 * t + 1] = a;
        split[4 * t + 2] = b;
        split[4 * t + 3] = c;
    }
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

// Write-kernel staging in one word sequence per array: slot k < n is entry k (A's, then
// B's, then C's: coordinate in s_crd, value in s_val), slot n + k is row r0 + k (s_crd: A's
// and B's tile-local starts packed A | B << 16; s_val, as int bits: C's tile-local start).
// A tile's entries and row ends are at most kTile + 2 items, so n + nr <= kCap.  Lane tid
// loads slots tid + j * kBlock (clamped to the last, consumed only when staged), three
// registers a slot: the rows' third offset is loaded only where a wave holds rows.
struct Slots3 {
    int x[kLoads];  // coordinate, or posA of a row
    int y[kLoads];  // value bits, or posB of a row
    int z[kLoads];  // posC of a row
};

__device__ __forceinline__ void fetch_slots3(Slots3 &st, const Split3 &sp,
                                             const int *__restrict__ pa,
                                             const int *__restrict__ ca,
                                             const float *__restrict__ va,
                                             const int *__restrict__ pb,
                                             const int *__restrict__ cb,
                                             const float *__restrict__ vb,
                                             const int *__restrict__ pc,
                                             const int *__restrict__ cc,
                                             const float *__restrict__ vc, int tid) {
    const int na = sp.a1 - sp.a0, nab = na + (sp.b1 - sp.b0);
    const int n = nab + (sp.c1 - sp.c0), total = n + (sp.r1 - sp.r0 + 1);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int k = min(tid + j * kBlock, total - 1);
        const int *px;
        const int *py;
        int off;
        if (k < na) {
            px = ca;
            py = reinterpret_cast<const int *>(va);
            off = sp.a0 + k;
        } else if (k < nab) {
            px = cb;
            py = reinterpret_cast<const int *>(vb);
            off = sp.b0 + (k - na);
        } else if (k < n) {
            px = cc;
            py = reinterpret_cast<const int *>(vc);
            off = sp.c0 + (k - nab);
        } else {
            px = pa;
            py = pb;
            off = sp.r0 + (k - n);
        }
        st.x[j] = px[off];
        st.y[j] = py[off];
        st.z[j] = k >= n ? pc[off] : 0;
    }
}

__device__ __forceinline__ void stage_slots3(const Slots3 &st, const Split3 &sp, int *s_crd,
                                             float *s_val, int tid) {
    const int n = (sp.a1 - sp.a0) + (sp.b1 - sp.b0) + (sp.c1 - sp.c0);
    const int total = n + (sp.r1 - sp.r0 + 1);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int k = tid + j * kBlock;
        if (k < n) {
            s_crd[k] = st.x[j];
            s_val[k] = __int_as_float(st.y[j]);
        } else if (k < total) {
            const unsigned ra = static_cast<unsigned>(max(st.x[j], sp.a0) - sp.a0);
            const unsigned rb = static_cast<unsigned>(max(st.y[j], sp.b0) - sp.b0);
            s_crd[k] = static_cast<int>(ra | (rb << 16));
            s_val[k] = __int_as_float(max(st.z[j], sp.c0) - sp.c0);
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
// `given`: taken from `start` (the count kernel's); otherwise searched and stored to `start`.
template <bool VALUES, bool COUNT_ONLY>
__device__ __forceinline__ void walk3(Lane3Out &out, const Split3 &sp, int tile, const int *s_crd,
                                      const float *s_val, const unsigned *s_row,
                                      const int *s_rowc, int tid, uint2 &start, bool given) {
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
    if (given) {
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
        split3<1>(at, at, at, ra(k), ea(k), rb(k), eb(k), rc(k), ec(k), d, ia, ib, ic);
    }
    if (!given) {
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
                // (reads at indices always inside the staged arrays, then selects: no
                // nested branches, each waiting for its own read)
                row_ends |= 1u << s;
                k = min(k + 1, nr - 1);
                const int kn = min(k + 1, nr - 1);
                const unsigned wn = s_row[kn];
                const int cn = s_rowc[kn];
                const int ha = at(ia), hb = at(ib), hc = at(ic);
                const bool last_row = k >= nr - 1;
                aE = last_row ? na : static_cast<int>(wn & 0xffffu);
                bE = last_row ? nab : na + static_cast<int>(wn >> 16);
                cE = last_row ? n : nab + cn;
                last = INT_MIN;
                xa = ia < aE ? ha : kMax;
                xb = ib < bE ? hb : kMax;
                xc = ic < cE ? hc : kMax;
            } else {
                const int x = min(xa, min(xb, xc));
                const bool ta = xa == x;  // ties: A, then B, then C
                const bool tb = !ta && xb == x;
                const bool tc = !ta && !tb;
                const bool emit = x != last;
                if (COUNT_ONLY) {
                    count += emit;
                } else {
                    out.crd[s] = x;
                    if (VALUES) {
                        // the group's sum in operand order, from its first item: the three
                        // reads are independent (indices inside the staged arrays), and the
                        // additions the group does not hold are discarded
                        const int own = ta ? ia : (tb ? ib : ic);
                        const float v0 = s_val[min(own, kCap - 1)];
                        const float v1 = s_val[min(ib, kCap - 1)];
                        const float v2 = s_val[min(ic, kCap - 1)];
                        const float vab = v0 + v1;
                        float v = (ta && xb == x) ? vab : v0;
                        const float vabc = v + v2;
                        v = ((ta || tb) && xc == x) ? vabc : v;
                        out.val[s] = v;
                    }
                    valid |= static_cast<unsigned>(emit) << s;
                }
                last = x;
                ia += ta;
                ib += tb;
                ic += tc;
                const int np = ta ? ia : (tb ? ib : ic);  // reload the head that advanced
                const int ne = ta ? aE : (tb ? bE : cE);
                const int h0 = at(np);
                const int h = np < ne ? h0 : kMax;
                xa = ta ? h : xa;
                xb = tb ? h : xb;
                xc = tc ? h : xc;
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

// The row pass's totals staged in LDS by every count workgroup: s_start[b] = searches before
// row-pass workgroup b (s_start[nb] = M), and each workgroup's record count and region.
// Returns the mode (the same in every workgroup); workgroup 0 stores it for the write
// kernel.  Ends synchronised.
__device__ __forceinline__ int stage_rows3(int *s_start, int *s_recs, int *s_base, int *s_wave,
                                           const Rows3 &rp, long long entries) {
    constexpr int kPer = kRowPassMaxBlocks / kBlock;
    const int tid = threadIdx.x;
    const int nb = rp.nb;
    int v[kPer], sum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid * kPer + k;
        v[k] = i < nb ? rp.blk_elems[i] : 0;
        sum += v[k];
        if (i < nb) {
            s_recs[i] = rp.blk_recs[i];
            s_base[i] = rp.blk_base[i];
        }
    }
    int total = 0;
    int off = dev::block_exclusive_sum<kBlock>(sum, s_wave, total);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid * kPer + k;
        if (i < nb) s_start[i] = off;
        off += v[k];
    }
    if (tid == 0) s_start[nb] = total;
    const int mode =
        static_cast<long long>(total) * kSearchRatio <= entries ? kModeSearch : kModeCount;
    if (blockIdx.x == 0 && tid == 0) *rp.mode = mode;
    __syncthreads();
    return mode;
}

// One round of a lower bound of x in c[p, q) (ascending) with kSearchWays - 1 independent
// probes: narrows [p, q] (the answer's range) to under a kSearchWays-th of its length.
__device__ __forceinline__ void lower_bound_round(const int *__restrict__ c, int x, int &p,
                                                  int &q) {
    const int step = (q - p + kSearchWays - 1) / kSearchWays;
    int below = 0;  // probes p + j * step - 1 (j >= 1) inside the range holding less than x
#pragma unroll
    for (int j = 1; j < kSearchWays; ++j) {
        const int at = p + j * step - 1;
        const int v = c[min(at, q - 1)];
        below += (at < q && v < x) ? 1 : 0;
    }
    const int np = p + below * step;
    q = below == kSearchWays - 1 ? q : min(p + (below + 1) * step - 1, q);
    p = np;
}

// Whether x is among c[lo, lo + n) (ascending), with rounds of independent probes, so that
// n entries cost about log_8(n) load latencies.
__device__ __forceinline__ bool holds(const int *__restrict__ c, int lo, int n, int x) {
    int p = lo, q = lo + n;
    while (p < q) lower_bound_round(c, x, p, q);
    return p < lo + n && c[p] == x;
}

// holds(c1, lo1, n1, x) and holds(c2, lo2, n2, x), the two searches' rounds issued together.
__device__ __forceinline__ void holds_both(const int *__restrict__ c1, int lo1, int n1,
                                           const int *__restrict__ c2, int lo2, int n2, int x,
                                           bool &in1, bool &in2) {
    int p1 = lo1, q1 = lo1 + n1, p2 = lo2, q2 = lo2 + n2;
    while (p1 < q1 || p2 < q2) {
        if (p1 < q1) lower_bound_round(c1, x, p1, q1);
        if (p2 < q2) lower_bound_round(c2, x, p2, q2);
    }
    in1 = p1 < lo1 + n1 && c1[p1] == x;
    in2 = p2 < lo2 + n2 && c2[p2] == x;
}

// Search mode of the count kernel: a grid-stride loop over the M searches.  Search e lies in
// row-pass workgroup b (staged offsets) and record k of b (binary search of the records'
// first searches); its place in the row's searches picks the entry and the rows searched
// (see the row pass).  Duplicates are added into chunk_count[write chunk], and the last
// workgroup stores nnzA + nnzB + nnzC less all of them to `length_out`.
__device__ __forceinline__ void dup_search(const int *s_start, const int *s_recs,
                                           const int *s_base, unsigned *s_wsum, int *s_cs,
                                           const Rows3 &rp, const int *__restrict__ ca,
                                           const int *__restrict__ cb, const int *__restrict__ cc,
                                           const int *__restrict__ split, int num_tiles, int chunk,
                                           unsigned *__restrict__ chunk_count,
                                           unsigned long long *__restrict__ done,
                                           int64_t *__restrict__ length_out, long long entries) {
    const int tid = threadIdx.x;
    const int nb = rp.nb;
    const int m_total = s_start[nb];
    const int n_chunks = (num_tiles + chunk - 1) / chunk;
    // the write chunks' first A, B and C positions, staged when they fit (s_cs[(op - 1) *
    // n_chunks + w] for op 1..3)
    const bool staged = 3 * n_chunks <= kCap;
    if (staged) {
        for (int i = tid; i < 3 * n_chunks; i += kBlock) {
            const int op = i / n_chunks, w = i - op * n_chunks;
            s_cs[i] = split[4 * min(w * chunk, num_tiles) + op + 1];
        }
        __syncthreads();
    }
    unsigned found = 0;  // duplicates seen by this wave (uniform in the wave)
    for (long long base = static_cast<long long>(blockIdx.x) * kBlock; base < m_total;
         base += static_cast<long long>(gridDim.x) * kBlock) {
        const long long e = base + tid;
        int chunk_id = -1;
        if (e < m_total) {
            int lo = 0, hi = nb - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_start[mid] <= e) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            const int local = static_cast<int>(e - s_start[lo]);
            const int4 *recs = rp.rec + 2 * static_cast<long long>(s_base[lo]);
            // last record whose first search is at or before `local` (record 0's is 0), with
            // rounds of kSearchWays - 1 independent probes
            int klo = 0, khi = s_recs[lo] - 1;
            while (klo < khi) {
                const int step = (khi - klo + kSearchWays) / kSearchWays;
                int at_or_before = 0;
#pragma unroll
                for (int j = 1; j < kSearchWays; ++j) {
                    const int at = klo + j * step;
                    const int v = recs[2 * min(at, khi)].x;
                    at_or_before += (at <= khi && v <= local) ? 1 : 0;
                }
                khi = min(klo + (at_or_before + 1) * step - 1, khi);
                klo += at_or_before * step;
            }
            const int4 r0 = recs[2 * klo], r1 = recs[2 * klo + 1];
            const int a0 = r0.y, b0 = r0.z, c0 = r0.w, la = r1.x, lb = r1.y, lc = r1.z;
            const int j = local - r0.x;
            const int wb = (la > 0 && lb > 0) ? min(la, lb) : 0;
            const int jc = j - wb;  // index among the row's |C ∩ (A ∪ B)| searches
            int op, pos;  // the searched entry: operand (1 A, 2 B, 3 C) and position
            bool dup;
            if (j < wb) {  // |A ∩ B|
                if (la <= lb) {
                    op = 1;
                    pos = a0 + j;
                    dup = holds(cb, b0, lb, ca[pos]);
                } else {
                    op = 2;
                    pos = b0 + j;
                    dup = holds(ca, a0, la, cb[pos]);
                }
            } else if (lc <= la + lb) {  // |C ∩ (A ∪ B)| by C's entries
                op = 3;
                pos = c0 + jc;
                const int x = cc[pos];
                bool in_a, in_b;
                holds_both(ca, a0, la, cb, b0, lb, x, in_a, in_b);
                dup = in_a || in_b;
            } else if (jc < la) {  // ... by A's entries
                op = 1;
                pos = a0 + jc;
                dup = holds(cc, c0, lc, ca[pos]);
            } else {  // ... by B's entries absent from A
                op = 2;
                pos = b0 + (jc - la);
                const int x = cb[pos];
                bool in_c, in_a;
                holds_both(cc, c0, lc, ca, a0, la, x, in_c, in_a);
                dup = in_c && !in_a;
            }
            if (dup) {
                // the write chunk holding it: last w whose first split is at or before pos
                int wlo = 0, whi = n_chunks - 1;
                const int *cs = s_cs + (op - 1) * n_chunks;
                while (wlo < whi) {
                    const int mid = (wlo + whi + 1) >> 1;
                    if ((staged ? cs[mid] : split[4 * min(mid * chunk, num_tiles) + op]) <= pos) {
                        wlo = mid;
                    } else {
                        whi = mid - 1;
                    }
                }
                chunk_id = wlo;
            }
        }
        // one atomic per distinct write chunk among the wave's duplicates
        unsigned long long pending = __ballot(chunk_id >= 0);
        found += static_cast<unsigned>(__popcll(pending));
        while (pending) {
            const int leader = __ffsll(static_cast<long long>(pending)) - 1;
            const int c = __shfl(chunk_id, leader, dev::kWave);
            const unsigned long long same = __ballot(chunk_id == c);
            if (dev::lane() == leader) {
                atomicAdd(&chunk_count[c], static_cast<unsigned>(__popcll(same)));
            }
            pending &= ~same;
        }
    }
    if (dev::lane() == 0) s_wsum[tid / dev::kWave] = found;
    __syncthreads();
    if (tid == 0) {
        unsigned dups = 0;
#pragma unroll
        for (int w = 0; w < kBlock / dev::kWave; ++w) dups += s_wsum[w];
        dev::subtract_total(dups, done, entries, length_out);
    }
}

// Output count of each chunk, and their sum (the result length) stored to `length_out` by
// the last workgroup.  After a row pass (rp.blk_elems set) the launch first totals it and,
// in search mode, runs dup_search instead (chunk_count then receives each chunk's
// duplicates, and no lane starts are stored).
__global__ __launch_bounds__(kBlock) void csr3_count_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, const int *__restrict__ pc, const int *__restrict__ cc,
    int num_tiles, int chunk, const int *__restrict__ split, unsigned *__restrict__ chunk_count,
    unsigned long long *__restrict__ done, int64_t *__restrict__ length_out,
    uint2 *__restrict__ starts, Rows3 rp, long long entries) {
    __shared__ int s_crd[kCap];
    __shared__ unsigned s_row[kCap];
    __shared__ int s_rowc[kCap];
    __shared__ unsigned s_wave[kBlock / dev::kWave];
    __shared__ int s_iwave[kBlock / dev::kWave];
    __shared__ int s_split[4 * (kMaxChunk + 1)];
    static_assert(kRowPassMaxBlocks + 1 <= kCap && 2 * kRowPassMaxBlocks <= kCap,
                  "the row pass's totals fit the tile arrays");
    const int tid = threadIdx.x;
    if (rp.blk_elems != nullptr) {  // after a row pass
        int *s_start = s_crd;
        int *s_recs = reinterpret_cast<int *>(s_row);
        int *s_base = s_recs + kRowPassMaxBlocks;
        if (stage_rows3(s_start, s_recs, s_base, s_iwave, rp, entries) == kModeSearch) {
            dup_search(s_start, s_recs, s_base, s_wave, s_rowc, rp, ca, cb, cc, split,
                       num_tiles, chunk, chunk_count, done, length_out, entries);
            return;
        }
    }
    // Workgroup w counts write chunk w; the launch may hold more workgroups than write chunks
    // (for the search mode), and those have no chunk.
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) {
        if (tid == 0) dev::add_to_total(0u, done, length_out);
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
        walk3<false, true>(lo, sp, t, s_crd, nullptr, s_row, s_rowc, tid, start, false);
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
    long long cap, int *__restrict__ pz, int *__restrict__ cz, float *__restrict__ vz,
    const int *__restrict__ mode) {
    __shared__ int s_crd[kCap];
    __shared__ float s_val[kCap];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_split[4 * (kMaxChunk + 1)];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * chunk, t1 = min(t0 + chunk, num_tiles);
    if (t0 >= t1) return;
    // the staged rows follow the staged entries (stage_slots3)
    auto rows_a = [&](const Split3 &q) {
        const int n = (q.a1 - q.a0) + (q.b1 - q.b0) + (q.c1 - q.c0);
        return reinterpret_cast<const unsigned *>(s_crd + n);
    };
    auto rows_c = [&](const Split3 &q) {
        const int n = (q.a1 - q.a0) + (q.b1 - q.b0) + (q.c1 - q.c0);
        return reinterpret_cast<const int *>(s_val + n);
    };
    // search mode (see dup_search): chunk_count holds duplicates, and lanes search their starts
    const bool search = mode != nullptr && *mode == kModeSearch;
    stage_splits3(s_split, split, t0, t1);
    int before = 0;
    for (int i = tid; i < static_cast<int>(blockIdx.x); i += kBlock) before += chunk_count[i];
    int base = 0;
    (void)dev::block_exclusive_sum<kBlock>(before, s_wave, base);  // (ends synchronised)
    // outputs before the chunk: its first split's entries less the duplicates before it
    if (search) base = s_split[1] + s_split[2] + s_split[3] - base;
    if (blockIdx.x == 0 && tid == 0) pz[0] = 0;
    Split3 sp = lds_split3(s_split, 0);
    Slots3 st;
    uint2 start = search ? make_uint2(0u, 0u) : starts[static_cast<size_t>(t0) * kBlock + tid];
    fetch_slots3(st, sp, pa, ca, va, pb, cb, vb, pc, cc, vc, tid);
    stage_slots3(st, sp, s_crd, s_val, tid);
    __syncthreads();
    for (int t = t0; t < t1; ++t) {
        const Split3 nsp = lds_split3(s_split, t + 1 < t1 ? t + 1 - t0 : t - t0);
        uint2 next_start = start;
        if (t + 1 < t1) {
            fetch_slots3(st, nsp, pa, ca, va, pb, cb, vb, pc, cc, vc, tid);
            if (!search) next_start = starts[static_cast<size_t>(t + 1) * kBlock + tid];
        }
        Lane3Out lo;
        walk3<true, false>(lo, sp, t, s_crd, s_val, rows_a(sp), rows_c(sp), tid, start, !search);
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
            if (dst >= 0 && dst < cap) {
                cz[dst] = s_crd[q];
                vz[dst] = s_val[q];
            }
        }
        base += tile_total;
        __syncthreads();  // staged outputs consumed
        if (t + 1 < t1) {
            stage_slots3(st, nsp, s_crd, s_val, tid);
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
    NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 4 + 2 * dev::kTotalWords, &counts));
    unsigned long long *done =
        reinterpret_cast<unsigned long long *>(counts + ((grid + 2) & ~1));
    // every lane's start in every tile, from the count kernel's tile walk (count mode)
    uint2 *starts = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles) * kBlock, &starts));
    int64_t *length_out = nullptr;
    NACHO_TRY(call.length_word(&length_out));

    // Row pass (rows holding at least kRowPassMinEntriesPerRow entries on average): at most
    // kRowPassMaxBlocks workgroups of kPartBlock threads, at least 16 rows per thread, one
    // two-int4 record per row with searches, each workgroup's records at its first row.
    Rows3 rp{};
    int row_grid = 0;
    if (static_cast<long long>(rows) * kRowPassMinEntriesPerRow <= cap) {
        const long long per_thread = std::max<long long>(
            16, (static_cast<long long>(rows) + kPartBlock * kRowPassMaxBlocks - 1) /
                    (kPartBlock * kRowPassMaxBlocks));
        const long long per_block = per_thread * kPartBlock;
        row_grid = static_cast<int>(std::max<long long>(1, (rows + per_block - 1) / per_block));
        rp.rows_per_thread = static_cast<int>(per_thread);
        rp.nb = row_grid;
        NACHO_TRY(call.scratch_n(2 * static_cast<size_t>(std::max(rows, 1)), &rp.rec));
        int *words = nullptr;
        NACHO_TRY(call.scratch_n(3 * static_cast<size_t>(row_grid) + 1, &words));
        rp.blk_base = words;
        rp.blk_elems = words + row_grid;
        rp.blk_recs = words + 2 * row_grid;
        rp.mode = words + 3 * row_grid;
    }

    // The count launch: the write chunks, or as many workgroups as it keeps resident when
    // that is more (they only take part in the search mode).
    int count_grid = grid;
    if (row_grid > 0) {
        int count_resident = 0;
        NACHO_TRY(resident_grid(reinterpret_cast<const void *>(csr3_count_kernel), kBlock,
                                &count_resident));
        count_grid = std::max(grid, count_resident);
    }
    const hipStream_t s = call.stream();
    NACHO_TRY(call.timer_start("csr_add_3: fused three-way merge"));
    const int part_blocks = static_cast<int>(
        ceil_div((static_cast<size_t>(num_tiles) + 1) * kPartLanes, kPartBlock));
    csr3_partition_kernel<<<part_blocks + row_grid, kPartBlock, 0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, b->dim_j_offsets, b->dim_j_indices,
        c->dim_j_offsets, c->dim_j_indices, rows, static_cast<int>(total), num_tiles, split,
        done, counts, grid, part_blocks, rp);
    NACHO_TRY_HIP(hipGetLastError());
    csr3_count_kernel<<<count_grid, kBlock, 0, s>>>(a->dim_j_offsets, a->dim_j_indices,
                                             b->dim_j_offsets, b->dim_j_indices,
                                             c->dim_j_offsets, c->dim_j_indices, num_tiles,
                                             chunk, split, counts, done, length_out, starts, rp,
                                             cap);
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.mark_length());
    csr3_write_kernel<<<grid, kBlock, 0, s>>>(
        a->dim_j_offsets, a->dim_j_indices, a->values, b->dim_j_offsets, b->dim_j_indices,
        b->values, c->dim_j_offsets, c->dim_j_indices, c->values, num_tiles, chunk, split,
        counts, starts, rows, cap, pz, cz, vz, rp.mode);
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
