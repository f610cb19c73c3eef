// CSR elementwise add (union) and multiply (intersection) for gfx950, and the level merge
// that CSF3 add chains three times.
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
//    nonzeros, tensor.cpp:308-413).  Item count T = nnzA + nnzB + rows, cut into tiles of
//    kTile items.
//  * csr_partition_kernel: a group of lanes per tile boundary finds (row, a, b) for diagonal
//    tile*kTile by a many-way search over rows on S(r) = posA[r] + posB[r] + r, then a
//    merge-path search inside the row (each round: one probe per lane and a ballot).  An A/B
//    pair with equal coordinates is never split across tiles (the reference's balancing step,
//    partition.cpp:964-983).
//  * csr_pair_count_kernel and csr_write_kernel: each workgroup owns a fixed, contiguous
//    chunk of tiles.  The count kernel reads only coordinates and row offsets and adds each
//    write chunk's output count (a union tile emits na + nb - pairs); the write kernel starts
//    from the sum of the preceding chunks' counts and carries a running offset through its
//    tiles.  No workgroup ever waits on another (an earlier single-pass design with
//    decoupled look-back spent most of its time waiting).
//  * A union value level first runs a row pass (extra workgroups of the partition launch)
//    over the rows where both operands have entries; when those hold few entries, the count
//    kernel searches each of them in the other operand's row instead of walking the tiles
//    (pair_search), and the write kernel derives its chunk offsets from the splits.
//  * Inside a tile (both kernels): the tile's crd/val ranges of A and B and a packed word per
//    row are staged in LDS from registers that were loaded one tile ahead; lane t owns items
//    [t*IPT, (t+1)*IPT) of the tile, found by a merge-path search in LDS, and walks them in a
//    fixed, unrolled number of steps (take A's head with ties to A, take B's head, or consume a
//    row end).  An equal A/B pair is combined when its A entry is taken and its B entry is
//    skipped when reached, so pairs may straddle lanes.  Outputs stay in registers until the
//    workgroup scan gives their offsets, then go through LDS to coalesced stores.
//
// Emission order and values follow the reference's lattice (compute.cpp:476-491,
// 1169-1198, 1297-1337): coordinates ascending within a row; union emits a+b where both
// exist and a copy otherwise; intersection emits a*b only where both exist.  Explicit zeros
// are kept.  Each value is one IEEE binary32 operation, so results are bit-identical to the
// reference's.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "csr_merge.hpp"
#include "device_utils.hpp"
#include "runtime.hpp"

namespace nacho {
namespace csr {

enum class Op { Union, Intersect };

constexpr int kBlock = 256;
constexpr int kItemsPerLane = 15;  // odd: lanes' LDS walks spread over banks
constexpr int kTile = kBlock * kItemsPerLane;
static_assert(kLevelTileSlack >= kTile, "callers' item-count headroom covers merge_level's");
constexpr int kPartBlock = 64;  // threads per workgroup of the partition kernel
// Lanes that search one tile boundary together: each round of the searches costs one
// dependent load and narrows the range (kPartLanes + 1)-fold; wider groups spend more
// divergent loads per round.
constexpr int kPartLanes = 8;


// ---- sparse-overlap union count: row pass + pair search --------------------------------
// A union's output count is na + nb - pairs, and pairs only occur in rows where both
// operands have entries.  When those rows hold few entries (C2: 244K of 33M), searching each
// entry of a row's smaller side in its larger side counts the pairs without streaming every
// coordinate through the count kernel.
//
// The row pass (extra workgroups of the partition kernel's launch) finds those rows and
// writes one record per row; the count kernel totals the entries to search (M) and picks the
// mode it and the write kernel follow:
//   search: M * kSearchRatio <= nnzA + nnzB.  The count kernel searches every such entry
//           (pair_search), adds the pairs into pair_count[write chunk] and publishes the
//           length nnzA + nnzB - pairs; the write kernel's chunk w starts at output
//           split_a[t0] + split_b[t0] - (pairs of chunks before w).
//   count:  the count kernel runs its tile walk (chunk output counts, no lane starts).
// In both modes the write kernel finds its lanes' starts itself (SEARCH).
constexpr int kModeCount = 0;
constexpr int kModeSearch = 1;
constexpr int kSearchRatio = 16;
// Ways of the search mode's lower bounds in the larger side (probes per round + 1).
constexpr int kSearchWays = 8;
// Tile mode of the pair count: a tile whose rows need at least this many searches counts its
// pairs by walking each lane's items instead (about 16 dependent LDS steps per lane against
// about 14 per search); lower when the lane's start is searched anyway (STARTS).
constexpr int kWalkMin = 2 * kBlock;
constexpr int kWalkMinStarts = kBlock;
constexpr int kRowPassMaxBlocks = 1024;  // workgroups of the row pass (a multiple of kBlock)
constexpr int kRowUnroll = 16;  // row steps of the row pass whose loads are issued together
// The row pass reads two offsets per row, so it runs only where rows hold this many entries
// on average: with about one entry per row (a CSF3 k level) its reads cost as much as the
// tile walk it may save, and the few entries per row make the walk's lane starts cheap.
constexpr int kRowPassMinEntriesPerRow = 8;

struct RowPairs {
    // records of row-pass workgroup b at rec[blk_base[b] + k], k < blk_recs[b]:
    // {first entry (within b's entries), smaller side's begin, larger side's begin,
    //  larger side's length | bit 31 set when the smaller side is B}
    // Workgroup b's region starts at its first row, or, when `px` is set, at px[first row]
    // (px: the offsets of the operand with fewer entries, whose entries in b's rows bound
    // b's records), whichever needs less scratch.
    int4 *rec;
    int *rec_row;  // the row of each record (same index as rec)
    const int *px;
    int *blk_base;   // region start per workgroup
    int *blk_elems;  // entries to search per workgroup
    int *blk_recs;   // records per workgroup
    int *mode;       // kModeSearch or kModeCount (stored by the count kernel)
    int rows_per_thread;
    int nb;  // workgroups of the row pass
};

// Workgroup `block` of the row pass (one wave): rows_per_thread * 64 consecutive rows.  It
// runs as extra workgroups of the partition kernel's launch, and nothing in it
// waits for other workgroups: the count kernel, launched next, totals blk_elems and chooses
// the mode.
__device__ __forceinline__ void row_pass_block(const int *__restrict__ pa,
                                               const int *__restrict__ pb, int rows,
                                               const RowPairs &rp, int block) {
    static_assert(kPartBlock == dev::kWave, "the row pass scans within one wave");
    const int l = threadIdx.x;
    const int rpt = rp.rows_per_thread;
    const long long per_block = static_cast<long long>(kPartBlock) * rpt;
    const long long row0 = block * per_block;  // < rows (or 0)
    const int region = rp.px ? rp.px[row0] : static_cast<int>(row0);
    int e_base = 0, r_base = 0;  // entries to search and records of the rows before
    // Step j covers rows row0 + j*64 .. +63, one per lane (coalesced), so the records come out
    // in row order from one wave scan per step; kRowUnroll steps' loads are issued together.
    for (int j0 = 0; j0 < rpt && rows > 0; j0 += kRowUnroll) {
        int a0[kRowUnroll], a1[kRowUnroll], b0[kRowUnroll], b1[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const long long r = row0 + static_cast<long long>(j0 + u) * dev::kWave + l;
            const long long rc = r < rows ? r : rows - 1;
            a0[u] = pa[rc];
            a1[u] = pa[rc + 1];
            b0[u] = pb[rc];
            b1[u] = pb[rc + 1];
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const long long r = row0 + static_cast<long long>(j0 + u) * dev::kWave + l;
            const int la = a1[u] - a0[u], lb = b1[u] - b0[u];
            const bool rec = j0 + u < rpt && r < rows && la > 0 && lb > 0;
            const int e = rec ? min(la, lb) : 0;
            const int e_incl = dev::wave_inclusive_sum(e);
            const int r_incl = dev::wave_inclusive_sum(static_cast<int>(rec));
            if (rec) {
                const bool a_small = la <= lb;
                const int at = region + r_base + r_incl - 1;
                rp.rec[at] = make_int4(e_base + e_incl - e, a_small ? a0[u] : b0[u],
                                       a_small ? b0[u] : a0[u], a_small ? lb : (la | INT_MIN));
                rp.rec_row[at] = static_cast<int>(r);
            }
            e_base += __builtin_amdgcn_readlane(e_incl, dev::kWave - 1);
            r_base += __builtin_amdgcn_readlane(r_incl, dev::kWave - 1);
        }
    }
    if (l == 0) {
        rp.blk_base[block] = region;
        rp.blk_elems[block] = e_base;
        rp.blk_recs[block] = r_base;
    }
}

// kPartLanes lanes per tile boundary t in [0, num_tiles]: split of diagonal
// min(t*TILE, total).  Boundary 0 also zeroes the ticket counter that the next kernel's length
// total uses, and the first n_counts boundaries zero the chunk counts (n_counts <=
// num_tiles + 1).  Workgroups from part_blocks on run the row pass.
__global__ __launch_bounds__(kPartBlock) void csr_partition_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, int rows, int total, int num_tiles, int *__restrict__ split_r,
    int *__restrict__ split_a, int *__restrict__ split_b, unsigned long long *__restrict__ done,
    unsigned *__restrict__ zero_counts, int n_counts, int part_blocks, RowPairs rp) {
    if (static_cast<int>(blockIdx.x) >= part_blocks) {  // the row pass's workgroups
        row_pass_block(pa, pb, rows, rp, static_cast<int>(blockIdx.x) - part_blocks);
        return;
    }
    const int t = (static_cast<int>(blockIdx.x) * kPartBlock + static_cast<int>(threadIdx.x)) /
                  kPartLanes;
    if (t > num_tiles) return;  // whole lane groups
    const bool lead = threadIdx.x % kPartLanes == 0;
    if (lead && t == 0) dev::zero_total(done);  // accumulator of the kernel that totals the length
    if (lead && t < n_counts) zero_counts[t] = 0u;  // chunk counts the count kernel adds into
    const long long d64 = static_cast<long long>(t) * kTile;
    const int diag = d64 > total ? total : static_cast<int>(d64);

    // Largest row r in [0, rows] with S(r) <= diag (S(0) = 0).
    const int r = dev::group_last_true<kPartLanes>(
        0, rows, [&](int x) { return pa[x] + pb[x] + x <= diag; });
    int a, b;
    if (r == rows) {
        a = pa[rows];
        b = pb[rows];
    } else {
        // Merge-path split of the row at a + b == D (ties: A first): a is one past the last
        // x in [lo, hi) with A[x] <= B[D - 1 - x], then the pair rule.
        const int D = diag - r;
        const int aS = pa[r], aE = pa[r + 1], bS = pb[r], bE = pb[r + 1];
        const int lo = max(aS, D - bE), hi = min(aE, D - bS);
        a = dev::group_last_true<kPartLanes>(
                lo - 1, hi - 1, [&](int x) { return ca[x] <= cb[D - 1 - x]; }) + 1;
        b = D - a;
        if (a > aS && b < bE && ca[a - 1] == cb[b]) ++b;
    }
    if (lead) {
        split_r[t] = r;
        split_a[t] = a;
        split_b[t] = b;
    }
}


// ---- tile staging ----------------------------------------------------------------------

struct TileSplit {
    int r0, a0, b0, r1, a1, b1;
};

__device__ __forceinline__ TileSplit load_split(const int *__restrict__ split_r,
                                                const int *__restrict__ split_a,
                                                const int *__restrict__ split_b, int tile) {
    return TileSplit{split_r[tile], split_a[tile], split_b[tile],
                     split_r[tile + 1], split_a[tile + 1], split_b[tile + 1]};
}

// The splits of a workgroup's whole chunk, staged in LDS once: reading them from global
// memory per tile would use scalar loads, whose wait counter is shared with LDS and would
// stall the next LDS access on a memory round trip.
constexpr int kMaxChunk = 64;

__device__ __forceinline__ void stage_splits(int *s_split, const int *__restrict__ split_r,
                                             const int *__restrict__ split_a,
                                             const int *__restrict__ split_b, int t0, int t1) {
    const int n = t1 - t0 + 1;
    for (int i = threadIdx.x; i < n; i += kBlock) {
        s_split[3 * i] = split_r[t0 + i];
        s_split[3 * i + 1] = split_a[t0 + i];
        s_split[3 * i + 2] = split_b[t0 + i];
    }
}

// Every lane reads the same words, so the split is moved to scalar registers.
__device__ __forceinline__ TileSplit lds_split(const int *s_split, int i) {
    auto u = [&](int k) { return __builtin_amdgcn_readfirstlane(s_split[3 * i + k]); };
    return TileSplit{u(0), u(1), u(2), u(3), u(4), u(5)};
}

// A staged tile in LDS is one word array `s_cr` of n + 1 words, n = na + nb + (r1 - r0)
// (at most kTile + 1: the pair rule adds one B entry to a tile): A's coordinates at
// [0, na), B's at [na, na + nb), then the tile's row words s_row = s_cr + na + nb, where
// s_row[k] = (max(posA[r0+k], a0) - a0) | (max(posB[r0+k], b0) - b0) << 16 for k < nr =
// r1 - r0 + 1 (s_row[0] is 0: a0 and b0 lie in row r0).  Values, when the level has them, are
// in s_val at the coordinates' indices.  Entries and rows share the array because a tile's
// items are its entries plus its row ends: a tile of many short rows holds few entries.
//
// Slot k of the n staged words (k >= 1 for rows) is loaded into two registers: A's (or B's)
// coordinate and value bits, or row r0 + 1 + (k - na - nb)'s two offsets.  Lane `tid` loads
// slots tid + j * kBlock, j < kSlots, one tile ahead; slot kSlots * kBlock (a tile of
// kTile + 1 words) is loaded when the tile is staged.
constexpr int kSlots = kTile / kBlock;
constexpr int kCap = kTile + 2;  // n + 1 words
static_assert(kSlots * kBlock == kTile, "a tile is a whole number of slot rounds");

struct Slots {
    int x[kSlots];  // coordinate, or posA of a row
    int y[kSlots];  // value bits, or posB of a row
};

// Global addresses of slot k (0 <= k < n) of the tile `sp`: x from px[off], y from py[off].
__device__ __forceinline__ void slot_source(int k, const TileSplit &sp, int na, int nab,
                                            const int *__restrict__ pa,
                                            const int *__restrict__ ca, const int *__restrict__ va,
                                            const int *__restrict__ pb,
                                            const int *__restrict__ cb, const int *__restrict__ vb,
                                            const int *&px, const int *&py, int &off) {
    if (k < na) {
        px = ca;
        py = va;
        off = sp.a0 + k;
    } else if (k < nab) {
        px = cb;
        py = vb;
        off = sp.b0 + (k - na);
    } else {
        px = pa;
        py = pb;
        off = sp.r0 + 1 + (k - nab);
    }
}

// Loads are issued unconditionally (lanes past the end re-read the last slot) and nothing is
// computed from them until they are stored to LDS, so a whole tile's loads are in flight at
// once.  Levels without values load y for row slots only.
template <bool VALUES>
__device__ __forceinline__ void fetch_slots(Slots &st, const TileSplit &sp,
                                            const int *__restrict__ pa, const int *__restrict__ ca,
                                            const float *__restrict__ va,
                                            const int *__restrict__ pb, const int *__restrict__ cb,
                                            const float *__restrict__ vb, int tid) {
    const int na = sp.a1 - sp.a0, nab = na + (sp.b1 - sp.b0), n = nab + (sp.r1 - sp.r0);
    if (n == 0) return;  // uniform
    const int *vai = reinterpret_cast<const int *>(va);
    const int *vbi = reinterpret_cast<const int *>(vb);
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int k = min(tid + j * kBlock, n - 1);
        const int *px, *py;
        int off;
        slot_source(k, sp, na, nab, pa, ca, vai, pb, cb, vbi, px, py, off);
        st.x[j] = px[off];
        if (VALUES || k >= nab) st.y[j] = py[off];
    }
}

// Row-start bins (when IPT > 0): row k >= 1 of the tile starts at item
// x_k = (a0 + b0 + r0 - tile_lo) + ra_k + rb_k + k counted from the tile's lane grid
// tile_lo = tile * kBlock * IPT, so it is the row of every lane L >= ceil(x_k / IPT) until a
// later row starts.  It is recorded as atomicMax(s_bin[L], tag << 16 | k) for that first L
// (if L < kBlock); after a barrier, lane_first_row turns the bins into each lane's first row
// with one workgroup max-scan, replacing a per-lane binary search over the tile's rows.  The
// tag (distinct per staged tile of a workgroup, increasing) makes stale entries of earlier
// tiles lose every max and read as "no row", so the bins are never cleared.
template <int IPT>
__device__ __forceinline__ void stage_slot(int k, int x, int y, const TileSplit &sp, int nab,
                                           int *s_cr, float *s_val, unsigned *s_bin,
                                           unsigned tag, int tile_lo) {
    if (k < nab) {
        s_cr[k] = x;
        if (s_val) s_val[k] = __int_as_float(y);
    } else {
        const int kr = k - nab + 1;  // tile row
        const unsigned ra = static_cast<unsigned>(max(x, sp.a0) - sp.a0);
        const unsigned rb = static_cast<unsigned>(max(y, sp.b0) - sp.b0);
        s_cr[nab + kr] = static_cast<int>(ra | (rb << 16));
        if (IPT > 0) {
            const int xi = (sp.a0 + sp.b0 + sp.r0 - tile_lo) + static_cast<int>(ra + rb) + kr;
            const int lane = max(1, (xi + IPT - 1) / IPT);
            if (lane < kBlock) atomicMax(&s_bin[lane], (tag << 16) | static_cast<unsigned>(kr));
        }
    }
}

template <bool VALUES, int IPT = 0>
__device__ __forceinline__ void stage_slots(const Slots &st, const TileSplit &sp, int *s_cr,
                                            float *s_val, int tid,
                                            const int *__restrict__ pa, const int *__restrict__ ca,
                                            const float *__restrict__ va,
                                            const int *__restrict__ pb, const int *__restrict__ cb,
                                            const float *__restrict__ vb,
                                            unsigned *s_bin = nullptr, unsigned tag = 0,
                                            int tile_lo = 0) {
    const int na = sp.a1 - sp.a0, nab = na + (sp.b1 - sp.b0), n = nab + (sp.r1 - sp.r0);
    float *sv = VALUES ? s_val : nullptr;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int k = tid + j * kBlock;
        if (k < n) stage_slot<IPT>(k, st.x[j], st.y[j], sp, nab, s_cr, sv, s_bin, tag, tile_lo);
    }
    if (tid == 0) {
        s_cr[nab] = 0;  // row 0's word
        if (n > kSlots * kBlock) {  // the tile's last slot (rare): loaded now
            const int k = kSlots * kBlock;
            const int *px, *py;
            int off;
            slot_source(k, sp, na, nab, pa, ca, reinterpret_cast<const int *>(va), pb, cb,
                        reinterpret_cast<const int *>(vb), px, py, off);
            const int x = px[off];
            const int y = (VALUES || k >= nab) ? py[off] : 0;
            stage_slot<IPT>(k, x, y, sp, nab, s_cr, sv, s_bin, tag, tile_lo);
        }
    }
}

// This lane's first row (tile-local) from the row-start bins of the tile staged with `tag`
// (see stage_slot): the largest row recorded at or before this lane.  Call after the barrier
// that ends the staging.  No barrier: each wave reads the earlier waves' bins itself (at most
// three per lane) and takes their maximum along with its own running maximum.
__device__ __forceinline__ int lane_first_row(const unsigned *s_bin, unsigned tag, int tid) {
    auto row_at = [&](int i) {
        const unsigned v = s_bin[i];
        return (v >> 16) == tag ? static_cast<int>(v & 0xffffu) : 0;
    };
    const int w = tid / dev::kWave, l = tid % dev::kWave;
    int before = 0;
    for (int j = 0; j < w; ++j) before = max(before, row_at(j * dev::kWave + l));  // uniform
    before = __builtin_amdgcn_readlane(dev::wave_inclusive_max_dpp(before), dev::kWave - 1);
    return max(before, dev::wave_inclusive_max_dpp(row_at(tid)));
}

// ---- one lane's walk -------------------------------------------------------------------

// Result of walking a lane's items: outputs in registers (step s fills slot s when bit s of
// `valid` is set), the steps that were row ends, and the first row the lane touched.
template <int STEPS>
struct LaneOut {
    int crd[STEPS];
    float val[STEPS];
    unsigned pos[STEPS];  // (a - a0) | (b - b0) << 16 before the step (child pointers)
    unsigned valid, row_ends;
    int first_row;
};

// Where a lane's walk starts: its first row k (tile-local) and its A and B heads as indices
// into the staged arrays (ia in [0, na], ib in [na, na + nb]), packed k | ia << 16 and ib.
// The count kernel finds them by searching and stores them; the write kernel of the same
// tiles loads them instead of searching again.
struct LaneStart {
    unsigned k_ia;
    unsigned ib;
};

// How a lane finds its start: search for its row and its split in the row; take the row
// (start.k_ia's low half, from the tile's row-start bins) and search in the row only; or take
// the whole start.  The search modes return the start found in `start`.
enum class Start { Search, RowGiven, Given };

template <Op OP, bool VALUES, bool CHILD, int IPT, Start MODE = Start::Search>
__device__ __forceinline__ void walk_lane(LaneOut<IPT + 1> &out, const TileSplit &sp, int tile,
                                          const int *s_crd, const float *s_val,
                                          const unsigned *s_row, int tid, LaneStart &start) {
    constexpr int kSteps = IPT + 1;
    constexpr int kMax = INT_MAX;  // head sentinel: row exhausted on that side
    const int r0 = sp.r0, a0 = sp.a0, b0 = sp.b0, r1 = sp.r1, a1 = sp.a1, b1 = sp.b1;
    const int na = a1 - a0, nr = r1 - r0 + 1;
    auto A = [&](int x) { return s_crd[x - a0]; };
    auto B = [&](int y) { return s_crd[na + y - b0]; };
    auto row_a = [&](int k) { return a0 + static_cast<int>(s_row[k] & 0xffffu); };
    auto row_b = [&](int k) { return b0 + static_cast<int>(s_row[k] >> 16); };

    const int tile_lo = tile * (kBlock * IPT);
    const int tile_start = a0 + b0 + r0;  // item index of the tile's first item
    const int tile_end = a1 + b1 + r1;    // one past its last item
    const int g_lo = tid == 0 ? tile_start : tile_lo + tid * IPT;
    const int steps = tid == kBlock - 1 ? tile_end - g_lo
                                        : min(tile_lo + (tid + 1) * IPT, tile_end) - g_lo;
    int k = 0, a = a0, b = b0;
    if (MODE == Start::Given) {
        k = static_cast<int>(start.k_ia & 0xffffu);
        a = a0 + static_cast<int>(start.k_ia >> 16);
        b = b0 + static_cast<int>(start.ib) - na;
    } else if (tid > 0 && g_lo < tile_end) {
        if (MODE == Start::RowGiven) {
            k = static_cast<int>(start.k_ia & 0xffffu);
        } else {
            int lo = 0, hi = nr - 1;  // row of item g_lo
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (row_a(mid) + row_b(mid) + r0 + mid <= g_lo) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            k = lo;
        }
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
    out.first_row = r0 + k;
    // From here positions are indices into the staged arrays: A's entries at [0, na), B's at
    // [na, na + nb).  A tile holds at most kTile + 1 entries (the pair rule adds one), so
    // every index read below, one past a row's last entry included, is < kCap.
    const int nb = b1 - b0;
    auto end_a = [&](int kk) { return kk < nr - 1 ? static_cast<int>(s_row[kk + 1] & 0xffffu) : na; };
    auto end_b = [&](int kk) {
        return na + (kk < nr - 1 ? static_cast<int>(s_row[kk + 1] >> 16) : nb);
    };
    int ia = a - a0, ib = na + b - b0;
    if (MODE != Start::Given) {
        start.k_ia = static_cast<unsigned>(k) | (static_cast<unsigned>(ia) << 16);
        start.ib = static_cast<unsigned>(ib);
    }
    int iae = end_a(k), ibe = end_b(k);
    int last_a = ia > static_cast<int>(s_row[k] & 0xffffu) ? s_crd[ia - 1] : -1;
    int xa = ia < iae ? s_crd[ia] : kMax;
    int xb = ib < ibe ? s_crd[ib] : kMax;
    unsigned valid = 0, row_ends = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        out.crd[s] = 0;
        out.val[s] = 0.0f;
        out.pos[s] = 0;
        if (s < steps) {
            if (xa == kMax && xb == kMax) {  // row end
                // (reads at indices always inside the staged arrays, then selects: no nested
                // branches, each waiting for its own read)
                row_ends |= 1u << s;
                ++k;
                const unsigned rn = s_row[min(k + 1, nr - 1)];
                const int ha = s_crd[ia], hb = s_crd[ib];
                const bool last_row = k >= nr - 1;
                iae = last_row ? na : static_cast<int>(rn & 0xffffu);
                ibe = na + (last_row ? nb : static_cast<int>(rn >> 16));
                last_a = -1;
                xa = ia < iae ? ha : kMax;
                xb = ib < ibe ? hb : kMax;
            } else {
                const bool take_a = xa <= xb;
                const bool pair = take_a && xa == xb;
                if (CHILD) out.pos[s] = static_cast<unsigned>(ia) | (static_cast<unsigned>(ib - na) << 16);
                out.crd[s] = min(xa, xb);
                if (VALUES) {
                    const float own = s_val[take_a ? ia : ib];
                    const float vb = s_val[ib];  // read even when unpaired: no branch
                    if (OP == Op::Union) {
                        out.val[s] = pair ? own + vb : own;
                    } else {
                        out.val[s] = own * vb;
                    }
                }
                const bool emit = (OP == Op::Union) ? (take_a || last_a != xb) : pair;
                valid |= static_cast<unsigned>(emit) << s;
                if (take_a) last_a = xa;
                ia += take_a;
                ib += !take_a;
                const int np = take_a ? ia : ib;  // reload the head that advanced
                const bool in = np < (take_a ? iae : ibe);
                const int h0 = s_crd[np];  // always read (np < kCap), then mask
                const int h = in ? h0 : kMax;
                xa = take_a ? h : xa;
                xb = take_a ? xb : h;
            }
        }
    }
    out.valid = valid;
    out.row_ends = row_ends;
}

// ---- kernels ---------------------------------------------------------------------------

// Chunk of tiles owned by workgroup w: [w*chunk, min((w+1)*chunk, num_tiles)).
__device__ __forceinline__ void chunk_range(int num_tiles, int chunk, int &t0, int &t1) {
    t0 = blockIdx.x * chunk;
    t1 = min(t0 + chunk, num_tiles);
}

template <int WAVES, typename T>
__device__ __forceinline__ T block_sum(T v, T *s_wave) {
    v = dev::wave_sum(v);
    if (dev::lane() == 0) s_wave[threadIdx.x / dev::kWave] = v;
    __syncthreads();
    T all = 0;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) all += s_wave[i];
    __syncthreads();
    return all;
}

// ---- pair count: the union's count pass ----------------------------------------------
//
// A union tile's output count is na + nb - pairs, and an equal A/B pair never straddles
// tiles, so the count pass only has to find the pairs.  In every row of the tile where both
// operands have entries, each entry of the side with fewer entries (A on a tie) is searched
// in the other side's range of the row (binary search in LDS).  Rows where one side is empty
// cost only their offsets; a row heavy in one operand costs the light side's entries times
// log2 of the heavy side's length.  At C2 (Zipf rows, independent operands) that is 2.4e5
// searches for 3.4e7 items.
//
// Staging reads 16-byte granules: the tile's A range then its B range of coordinates, each
// cut at its array's 16-byte boundaries (a granule holding one element of the range lies in
// the same page as that element, so reading all of it never leaves mapped memory; the extra
// elements are never used), and the row offsets of up to kRowBlock + 1 rows per pass.

// Offset of each array's base address from a 16-byte boundary, in elements (0..3).
struct Misalign {
    int ca, cb, pa, pb;
};

// A 16-byte granule as a native vector (HIP's int4 is a struct over a union, which keeps
// arrays of it in scratch memory).
typedef int grain_t __attribute__((ext_vector_type(4)));

constexpr int kGrains = 4;      // coordinate granules per lane: 4096 entries >= tile + padding
constexpr int kRowGrains = 2;   // row-offset granules per lane per operand: 2048 offsets
constexpr int kRowBlock = kRowGrains * 4 * kBlock - 4;  // rows per pass (their ends included)
constexpr int kGrainCap = kGrains * 4 * kBlock;

__device__ __forceinline__ int grain_first(int lo, int mis) { return ((lo + mis) & ~3) - mis; }
__device__ __forceinline__ int grain_count(int lo, int hi, int mis) {
    return hi > lo ? (hi - grain_first(lo, mis) + 3) >> 2 : 0;
}

// Where a tile's coordinates land in LDS: granule q at s[4q .. 4q + 3], A's granules first;
// A's entry a0 at index offA, B's entry b0 at offB.
struct GrainLayout {
    int firstA, nga, firstB, ngb, offA, offB;
};

__device__ __forceinline__ GrainLayout grain_layout(const TileSplit &sp, int misA, int misB) {
    GrainLayout g;
    g.firstA = grain_first(sp.a0, misA);
    g.nga = grain_count(sp.a0, sp.a1, misA);
    g.firstB = grain_first(sp.b0, misB);
    g.ngb = grain_count(sp.b0, sp.b1, misB);
    g.offA = sp.a0 - g.firstA;
    g.offB = 4 * g.nga + (sp.b0 - g.firstB);
    return g;
}

struct TileGrains {
    grain_t v[kGrains];
};

// Loads are issued unconditionally (lanes past the end re-read the last granule) so that a
// whole tile's loads are in flight at once.
__device__ __forceinline__ void fetch_grains(TileGrains &tg, const GrainLayout &g,
                                             const int *__restrict__ xa,
                                             const int *__restrict__ xb, int tid) {
    const int n = g.nga + g.ngb;
    if (n == 0) return;  // uniform
#pragma unroll
    for (int j = 0; j < kGrains; ++j) {
        const int q = min(tid + j * kBlock, n - 1);
        const int *src = q < g.nga ? xa + g.firstA + 4 * q : xb + g.firstB + 4 * (q - g.nga);
        tg.v[j] = *reinterpret_cast<const grain_t *>(src);
    }
}

__device__ __forceinline__ void store_grains(const TileGrains &tg, const GrainLayout &g,
                                             int *s, int tid) {
    const int n = g.nga + g.ngb;
#pragma unroll
    for (int j = 0; j < kGrains; ++j) {
        const int q = tid + j * kBlock;
        if (q < n) *reinterpret_cast<grain_t *>(s + 4 * q) = tg.v[j];
    }
}

// Row offsets of rows [lo, hi) of both operands (at most kRowBlock + 1 rows).
struct RowGrains {
    grain_t a[kRowGrains], b[kRowGrains];
};

__device__ __forceinline__ void fetch_row_grains(RowGrains &rg, const int *__restrict__ pa,
                                                 const int *__restrict__ pb, int lo, int hi,
                                                 const Misalign &mis, int tid) {
    const int fa = grain_first(lo, mis.pa), na = grain_count(lo, hi, mis.pa);
    const int fb = grain_first(lo, mis.pb), nb = grain_count(lo, hi, mis.pb);
#pragma unroll
    for (int j = 0; j < kRowGrains; ++j) {
        const int qa = min(tid + j * kBlock, na - 1), qb = min(tid + j * kBlock, nb - 1);
        rg.a[j] = *reinterpret_cast<const grain_t *>(pa + fa + 4 * qa);
        rg.b[j] = *reinterpret_cast<const grain_t *>(pb + fb + 4 * qb);
    }
}

// Tile-local starts of rows [lo, hi): s_ra[k] = max(pa[lo + k] - a0, 0), likewise s_rb.
__device__ __forceinline__ void store_row_grains(const RowGrains &rg, int lo, int hi,
                                                 const Misalign &mis, int a0, int b0,
                                                 unsigned short *s_ra, unsigned short *s_rb,
                                                 int tid) {
    const int fa = grain_first(lo, mis.pa), fb = grain_first(lo, mis.pb);
    const int n = hi - lo;
#pragma unroll
    for (int j = 0; j < kRowGrains; ++j) {
        const int q = tid + j * kBlock;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int ka = fa + 4 * q + e - lo, kb = fb + 4 * q + e - lo;
            if (ka >= 0 && ka < n) s_ra[ka] = static_cast<unsigned short>(max(rg.a[j][e] - a0, 0));
            if (kb >= 0 && kb < n) s_rb[kb] = static_cast<unsigned short>(max(rg.b[j][e] - b0, 0));
        }
    }
}

// LDS of the pair count.
struct PairShared {
    int crd[kGrainCap];
    unsigned short ra[kRowBlock + 4], rb[kRowBlock + 4];
    int mpre[kRowBlock + 1];
    int wave[kBlock / dev::kWave];
    unsigned wsum[kBlock / dev::kWave];
};

// LDS of the count kernel's search mode (overlays PairShared).  The M entries to search are
// cut into slices of kBlock entries inside one row-pass workgroup's entries; a slice's
// records (at most kBlock: each holds at least one entry) are staged from `rec` before its
// lanes look up their records.
constexpr int kStageRecs = 2 * kBlock;
struct PairSearchLds {
    int start[kRowPassMaxBlocks + 1];  // entries to search before row-pass workgroup b; [nb] = M
    int recs[kRowPassMaxBlocks];       // records of workgroup b
    int base[kRowPassMaxBlocks];       // region start of workgroup b in rec / rec_row
    int work[kRowPassMaxBlocks + 1];   // slices before workgroup b; [nb] = all slices
    int4 rec[kStageRecs];              // records k0 .. k0 + kStageRecs - 1 of the slice's workgroup
    int rec_row[kStageRecs];
    int last[kBlock / dev::kWave];     // narrowing rounds: last probe <= the slice's first entry
    int wave[kBlock / dev::kWave];
    unsigned wsum[kBlock / dev::kWave];
};
union PairLds {
    PairShared walk;
    PairSearchLds search;
};
static_assert(sizeof(PairSearchLds) <= sizeof(PairShared), "search mode fits the walk's LDS");

// Running totals of a pair-count workgroup.
struct PairTotals {
    unsigned found;    // this lane's pairs since the last flush
    unsigned entries;  // entries of both operands since the last flush (uniform)
    unsigned total;    // the workgroup's output count (thread 0)
};

// One tile of the pair count: stage it from registers (tg, rg), refill the registers with
// tile `t_next`'s loads (split `nsp`, if `has_next`), then count its pairs and, when STARTS,
// store its lanes' write-kernel starts.
template <bool STARTS>
__device__ __forceinline__ void pair_tile(
    PairShared &sh, int t, int t_last, const TileSplit &sp, const GrainLayout &g,
    TileGrains &tg, RowGrains &rg, bool has_next, const TileSplit &nsp,
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, const Misalign &mis, int write_chunk,
    unsigned *__restrict__ chunk_count, uint2 *__restrict__ starts, PairTotals &acc, int tid) {
    const int na = sp.a1 - sp.a0, nb = sp.b1 - sp.b0, nr = sp.r1 - sp.r0 + 1;
    const int offA = g.offA, offB = g.offB;
    store_grains(tg, g, sh.crd, tid);
    store_row_grains(rg, sp.r0, min(sp.r0 + kRowBlock + 1, sp.r1 + 1), mis, sp.a0, sp.b0, sh.ra,
                     sh.rb, tid);
    if (has_next) {  // uniform: tile t_next's loads, in flight during the next two tiles
        const GrainLayout ng = grain_layout(nsp, mis.ca, mis.cb);
        fetch_grains(tg, ng, ca, cb, tid);
        fetch_row_grains(rg, pa, pb, nsp.r0, min(nsp.r0 + kRowBlock + 1, nsp.r1 + 1), mis, tid);
    }
    // this lane's first item in the write kernel, relative to the tile's first item
    const int tile_start = sp.a0 + sp.b0 + sp.r0, tile_end = sp.a1 + sp.b1 + sp.r1;
    const int g_lo = tid == 0 ? tile_start : t * kTile + tid * kItemsPerLane;
    const int rel = g_lo - tile_start;
    bool have_start = g_lo >= tile_end;  // lanes without items keep the tile's start
    LaneStart start{0u, static_cast<unsigned>(na)};
    // this lane's items in the write kernel (for the walk count)
    const int steps = tid == kBlock - 1
                          ? tile_end - g_lo
                          : min(t * kTile + (tid + 1) * kItemsPerLane, tile_end) - g_lo;
    __syncthreads();
    for (int kb = 0; kb < nr; kb += kRowBlock) {  // one pass unless nr > kRowBlock
        const int nrb = min(kRowBlock, nr - kb);
        if (kb > 0) {
            // Further rows of a tile with more than kRowBlock rows: staged here, with plain
            // loads (rare: such a tile holds few entries).
            __syncthreads();
            const int cnt = min(nrb + 1, nr - kb);
            for (int k = tid; k < cnt; k += kBlock) {
                sh.ra[k] = static_cast<unsigned short>(max(pa[sp.r0 + kb + k] - sp.a0, 0));
                sh.rb[k] = static_cast<unsigned short>(max(pb[sp.r0 + kb + k] - sp.b0, 0));
            }
            __syncthreads();
        }
        // Per row: searches to do = the smaller side's entries when both sides have some.
        constexpr int kR = (kRowBlock + kBlock - 1) / kBlock;
        const int per = (nrb + kBlock - 1) / kBlock;  // rows per lane, contiguous
        int m[kR];
        int mine = 0;
#pragma unroll
        for (int i = 0; i < kR; ++i) {
            m[i] = 0;
            const int k = tid * per + i;
            if (i < per && k < nrb) {
                const bool last = kb + k + 1 == nr;
                const int la = (last ? na : sh.ra[k + 1]) - sh.ra[k];
                const int lb = (last ? nb : sh.rb[k + 1]) - sh.rb[k];
                m[i] = (la > 0 && lb > 0) ? min(la, lb) : 0;
                mine += m[i];
            }
        }
        int work = 0;
        int run = dev::block_exclusive_sum<kBlock, int, false>(mine, sh.wave, work);
#pragma unroll
        for (int i = 0; i < kR; ++i) {
            const int k = tid * per + i;
            if (i < per && k < nrb) sh.mpre[k] = run;
            run += m[i];
        }
        __syncthreads();
        // Tiles with many searches (both operands dense in the same rows) count their pairs
        // with a merge walk of each lane's write-kernel items instead (single-pass tiles).
        const bool walk = nr <= kRowBlock && work >= (STARTS ? kWalkMinStarts : kWalkMin);
        for (int j = walk ? work : tid; j < work; j += kBlock) {
            int lo = 0, hi = nrb - 1;  // the row: last k with mpre[k] <= j
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (sh.mpre[mid] <= j) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            const int k = lo;
            const bool last = kb + k + 1 == nr;
            const int sa = sh.ra[k], ea = last ? na : sh.ra[k + 1];
            const int sb = sh.rb[k], eb = last ? nb : sh.rb[k + 1];
            const int nth = j - sh.mpre[k];
            int x, base, l, h;
            if (ea - sa <= eb - sb) {
                x = sh.crd[offA + sa + nth];
                base = offB;
                l = sb;
                h = eb;
            } else {
                x = sh.crd[offB + sb + nth];
                base = offA;
                l = sa;
                h = ea;
            }
            const int end = h;
            while (l < h) {  // first position >= x
                const int mid = (l + h) >> 1;
                if (sh.crd[base + mid] < x) {
                    l = mid + 1;
                } else {
                    h = mid;
                }
            }
            acc.found += (l < end && sh.crd[base + l] == x) ? 1u : 0u;
        }
        // The write kernel's start of this lane, if its first item lies in this pass's rows:
        // the row (last k whose first item is at or before it), then the merge-path split of
        // the row's A and B entries before it (ties: A first).
        const bool last_pass = kb + nrb >= nr;
        if ((STARTS || walk) && !have_start &&
            (last_pass || rel < sh.ra[nrb] + sh.rb[nrb] + kb + nrb)) {
            int lo = 0, hi = nrb - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (sh.ra[mid] + sh.rb[mid] + kb + mid <= rel) {
                    lo = mid;
                } else {
                    hi = mid - 1;
                }
            }
            const int k = lo;
            const bool last = kb + k + 1 == nr;
            const int aS = sh.ra[k], aE = last ? na : sh.ra[k + 1];
            const int bS = sh.rb[k], bE = last ? nb : sh.rb[k + 1];
            const int D = rel - (kb + k);  // entries of the tile before the item
            int slo = max(aS, D - bE), shi = min(aE, D - bS);
            while (slo < shi) {
                const int mid = (slo + shi) >> 1;
                if (sh.crd[offA + mid] <= sh.crd[offB + D - 1 - mid]) {
                    slo = mid + 1;
                } else {
                    shi = mid;
                }
            }
            start = LaneStart{static_cast<unsigned>(kb + k) | (static_cast<unsigned>(slo) << 16),
                              static_cast<unsigned>(na + D - slo)};
            have_start = true;
            if (walk) {  // (kb == 0) count the pairs among this lane's items: a pair at its A
                constexpr int kEnd = INT_MAX;  // head of an exhausted row side
                auto end_a = [&](int r) { return r + 1 < nr ? static_cast<int>(sh.ra[r + 1]) : na; };
                auto end_b = [&](int r) { return r + 1 < nr ? static_cast<int>(sh.rb[r + 1]) : nb; };
                int r = k, ia = slo, ib = D - slo;
                int iae = end_a(r), ibe = end_b(r);
                int xa = ia < iae ? sh.crd[offA + ia] : kEnd;
                int xb = ib < ibe ? sh.crd[offB + ib] : kEnd;
                unsigned pairs = 0;
                // (reads at indices inside the staged arrays, then selects: no nested
                // branches, each waiting for its own read)
                auto crd_at = [&](int x) { return sh.crd[min(x, kGrainCap - 1)]; };
#pragma unroll
                for (int st = 0; st < kItemsPerLane + 1; ++st) {
                    if (st < steps) {
                        if (xa == kEnd && xb == kEnd) {  // row end
                            ++r;
                            const int rn = min(r + 1, nr - 1);
                            const int an = sh.ra[rn], bn = sh.rb[rn];
                            const int ha = crd_at(offA + ia), hb = crd_at(offB + ib);
                            const bool last_row = r + 1 >= nr;
                            iae = last_row ? na : an;
                            ibe = last_row ? nb : bn;
                            xa = ia < iae ? ha : kEnd;
                            xb = ib < ibe ? hb : kEnd;
                        } else {
                            const bool take_a = xa <= xb;
                            pairs += (take_a && xa == xb) ? 1u : 0u;
                            ia += take_a;
                            ib += !take_a;
                            const bool in = take_a ? ia < iae : ib < ibe;
                            const int h0 = crd_at(take_a ? offA + ia : offB + ib);
                            const int h = in ? h0 : kEnd;
                            xa = take_a ? h : xa;
                            xb = take_a ? xb : h;
                        }
                    }
                }
                acc.found += pairs;
            }
        }
    }
    if (STARTS) starts[static_cast<size_t>(t) * kBlock + tid] = make_uint2(start.k_ia, start.ib);
    acc.entries += static_cast<unsigned>(na + nb);
    if (t == t_last || (t + 1) % write_chunk == 0) {  // uniform: end of a write chunk
        const unsigned pairs = block_sum<kBlock / dev::kWave>(acc.found, sh.wsum);
        if (tid == 0) {
            const unsigned c = acc.entries - pairs;
            atomicAdd(&chunk_count[t / write_chunk], c);
            acc.total += c;
        }
        acc.found = 0;
        acc.entries = 0;
    }
    __syncthreads();  // every lane is done with this tile's LDS
}

// The row pass's totals staged in LDS by every count workgroup: sh.start[b] = entries to
// search before workgroup b (sh.start[nb] = M), its records and region start, and
// sh.work[b] = slices of kBlock entries before workgroup b.  Returns the mode (the same in
// every workgroup); workgroup 0 stores it for the write kernel.  Ends synchronised.
__device__ __forceinline__ int stage_row_pass(PairSearchLds &sh, const RowPairs &rp,
                                              long long items) {
    constexpr int kPer = kRowPassMaxBlocks / kBlock;
    const int tid = threadIdx.x;
    const int nb = rp.nb;
    int v[kPer], sum = 0, slices = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid * kPer + k;
        v[k] = i < nb ? rp.blk_elems[i] : 0;
        sum += v[k];
        slices += (v[k] + kBlock - 1) / kBlock;
        if (i < nb) {
            sh.recs[i] = rp.blk_recs[i];
            sh.base[i] = rp.blk_base[i];
        }
    }
    int total = 0, all_slices = 0;
    int off = dev::block_exclusive_sum<kBlock>(sum, sh.wave, total);
    int woff = dev::block_exclusive_sum<kBlock>(slices, sh.wave, all_slices);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid * kPer + k;
        if (i < nb) {
            sh.start[i] = off;
            sh.work[i] = woff;
        }
        off += v[k];
        woff += (v[k] + kBlock - 1) / kBlock;
    }
    if (tid == 0) {
        sh.start[nb] = total;
        sh.work[nb] = all_slices;
    }
    const int mode =
        static_cast<long long>(total) * kSearchRatio <= items ? kModeSearch : kModeCount;
    if (blockIdx.x == 0 && tid == 0) *rp.mode = mode;
    __syncthreads();
    return mode;
}

// First staged record of a slice whose first entry (within its row-pass workgroup) is
// `first`, among the workgroup's `n` records at `rec`: a record k0 with the record holding
// `first` in [k0, k0 + kBlock).  Each round probes kBlock evenly spaced records at once and
// keeps the span after the last probe at or before `first` (records' first entries
// increase, and record 0's is 0).  Uniform in the workgroup; ends synchronised.
__device__ __forceinline__ int first_staged_record(PairSearchLds &sh, const int4 *rec, int n,
                                                   int first) {
    const int tid = threadIdx.x;
    int lo = 0;
    while (n > kBlock) {  // uniform
        const int stride = (n + kBlock - 1) / kBlock;
        const int k = lo + tid * stride;
        const bool le = k < lo + n && rec[k].x <= first;
        const unsigned long long m = __ballot(le);
        if (dev::lane() == 0) sh.last[tid / dev::kWave] = m ? 63 - __clzll(m) + (tid & ~63) : -1;
        __syncthreads();
        int t = -1;
#pragma unroll
        for (int w = 0; w < kBlock / dev::kWave; ++w) t = max(t, sh.last[w]);
        __syncthreads();
        lo += t * stride;  // t >= 0: probe 0 is record lo, at or before `first`
        n = min(stride, n - t * stride);
    }
    return lo;
}

// Search mode of the count kernel.  Slice w (a grid-stride loop over sh.work[nb] slices) is
// slice j of row-pass workgroup b: its entries j * kBlock + tid.  The slice's records are
// staged in LDS; a lane finds its record there (a binary search over the records' first
// entries), reads its smaller-side entry rec.y + (local - rec.x), and a lower bound in the
// larger side tells whether its column is there.  A pair's write chunk is the chunk of the
// tile holding its A entry, merged item a + b + row (the partition keeps pairs inside one
// tile), so no search over the tile splits is needed.
__device__ __forceinline__ void pair_search(PairSearchLds &sh, const int *__restrict__ ca,
                                            const int *__restrict__ cb, const RowPairs &rp,
                                            int write_chunk, unsigned *__restrict__ pair_count,
                                            unsigned long long *__restrict__ done,
                                            int64_t *__restrict__ length_out, long long items) {
    const int tid = threadIdx.x;
    const int nb = rp.nb;
    const int slices = sh.work[nb];
    unsigned found = 0;  // pairs seen by this wave (uniform in the wave)
    for (int w = blockIdx.x; w < slices; w += gridDim.x) {  // uniform
        int b = 0, hi = nb - 1;
        while (b < hi) {
            const int mid = (b + hi + 1) >> 1;
            if (sh.work[mid] <= w) {
                b = mid;
            } else {
                hi = mid - 1;
            }
        }
        const int first = (w - sh.work[b]) * kBlock;
        const int elems = sh.start[b + 1] - sh.start[b];
        const int n_rec = sh.recs[b];
        const int4 *rec = rp.rec + sh.base[b];
        const int *rec_row = rp.rec_row + sh.base[b];
        const int k0 = first_staged_record(sh, rec, n_rec, first);
        const int n_staged = min(kStageRecs, n_rec - k0);
#pragma unroll
        for (int i = 0; i < kStageRecs / kBlock; ++i) {
            const int k = i * kBlock + tid;
            if (k < n_staged) {
                sh.rec[k] = rec[k0 + k];
                sh.rec_row[k] = rec_row[k0 + k];
            }
        }
        __syncthreads();
        const int local = first + tid;
        int chunk_id = -1;
        if (local < elems) {
            int klo = 0, khi = n_staged - 1;
            while (klo < khi) {
                const int mid = (klo + khi + 1) >> 1;
                if (sh.rec[mid].x <= local) {
                    klo = mid;
                } else {
                    khi = mid - 1;
                }
            }
            const int4 rc = sh.rec[klo];
            const bool b_small = rc.w < 0;
            const int l_len = rc.w & INT_MAX;
            const int s_idx = rc.y + (local - rc.x);
            const int x = b_small ? cb[s_idx] : ca[s_idx];
            const int *large = b_small ? ca : cb;
            // Lower bound of x in large[rc.z, rc.z + l_len), kSearchWays - 1 probes per
            // round: the probes of a round are independent loads (the first round's are
            // issued with x's), so a row of n entries costs about log_8(n) load latencies
            // instead of log_2(n).  The answer stays in [p, q].
            int p = rc.z, q = rc.z + l_len;
            while (p < q) {
                const int step = (q - p + kSearchWays - 1) / kSearchWays;
                int below = 0;  // probes p + j * step - 1 (j >= 1) inside the range with large < x
#pragma unroll
                for (int j = 1; j < kSearchWays; ++j) {
                    const int at = p + j * step - 1;
                    const int v = large[min(at, q - 1)];
                    below += (at < q && v < x) ? 1 : 0;
                }
                const int np = p + below * step;
                q = below == kSearchWays - 1 ? q : min(p + (below + 1) * step - 1, q);
                p = np;
            }
            if (p < rc.z + l_len && large[p] == x) {
                // The pair's A entry is merged item a + b + row (A, B and row-end items
                // before it; ties put A first), and the partition keeps the pair in the
                // tile holding that item.
                const int a_idx = b_small ? p : s_idx, b_idx = b_small ? s_idx : p;
                chunk_id = (a_idx + b_idx + sh.rec_row[klo]) / kTile / write_chunk;
            }
        }
        // one atomic per distinct write chunk among the wave's pairs
        unsigned long long pending = __ballot(chunk_id >= 0);
        found += static_cast<unsigned>(__popcll(pending));
        while (pending) {
            const int leader = __ffsll(static_cast<long long>(pending)) - 1;
            const int c = __shfl(chunk_id, leader, dev::kWave);
            const unsigned long long same = __ballot(chunk_id == c);
            if (dev::lane() == leader) atomicAdd(&pair_count[c], static_cast<unsigned>(__popcll(same)));
            pending &= ~same;
        }
        __syncthreads();  // the staged records are rewritten by the next slice
    }
    if (dev::lane() == 0) sh.wsum[tid / dev::kWave] = found;
    __syncthreads();
    if (tid == 0) {
        unsigned pairs = 0;
#pragma unroll
        for (int w = 0; w < kBlock / dev::kWave; ++w) pairs += sh.wsum[w];
        dev::subtract_total(pairs, done, items, length_out);
    }
}

// Output counts of a union level (na + nb - pairs per tile), added into
// chunk_count[tile / write_chunk] (zeroed by the partition kernel): the counts of the write
// kernel's chunks, whose grid is chosen independently of this kernel's (`chunk` tiles per
// workgroup here, two tiles in flight).  Their sum, the result length, goes to `length_out`
// from the last workgroup.  When STARTS, every lane's walk start in the write kernel (row,
// A and B heads) is stored to starts[tile * kBlock + lane], found here by a search over the
// staged rows and a merge-path split inside the row.  Without STARTS and after a row pass
// (rp.blk_elems set), the launch first totals the row pass and, in search mode, runs
// pair_search instead (chunk_count then receives the pairs of each write chunk).
template <bool STARTS>
__global__ __launch_bounds__(kBlock) void csr_pair_count_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const int *__restrict__ pb,
    const int *__restrict__ cb, Misalign mis, int num_tiles, int chunk, int write_chunk,
    const int *__restrict__ split_r, const int *__restrict__ split_a,
    const int *__restrict__ split_b, unsigned *__restrict__ chunk_count,
    unsigned long long *__restrict__ done, int64_t *__restrict__ length_out,
    uint2 *__restrict__ starts, RowPairs rp, int write_grid, long long items) {
    __shared__ PairLds lds;
    __shared__ int s_split[3 * (kMaxChunk + 1)];
    PairShared &sh = lds.walk;

    const int tid = threadIdx.x;
    if (!STARTS && rp.blk_elems != nullptr) {  // after a row pass
        if (stage_row_pass(lds.search, rp, items) == kModeSearch) {  // uniform
            pair_search(lds.search, ca, cb, rp, write_chunk, chunk_count, done, length_out,
                        items);
            return;
        }
    }
    int t0, t1;
    chunk_range(num_tiles, chunk, t0, t1);
    if (t0 >= t1) {
        if (tid == 0) dev::add_to_total(0u, done, length_out);
        return;
    }
    stage_splits(s_split, split_r, split_a, split_b, t0, t1);
    __syncthreads();
    // Two tiles in flight: tiles t0 + 2i go through (tg0, rg0), t0 + 2i + 1 through (tg1, rg1).
    TileGrains tg0, tg1;
    RowGrains rg0, rg1;
    TileSplit sp0 = lds_split(s_split, 0);
    TileSplit sp1 = lds_split(s_split, t0 + 1 < t1 ? 1 : 0);
    GrainLayout g0 = grain_layout(sp0, mis.ca, mis.cb);
    GrainLayout g1 = grain_layout(sp1, mis.ca, mis.cb);
    fetch_grains(tg0, g0, ca, cb, tid);
    fetch_row_grains(rg0, pa, pb, sp0.r0, min(sp0.r0 + kRowBlock + 1, sp0.r1 + 1), mis, tid);
    if (t0 + 1 < t1) {
        fetch_grains(tg1, g1, ca, cb, tid);
        fetch_row_grains(rg1, pa, pb, sp1.r0, min(sp1.r0 + kRowBlock + 1, sp1.r1 + 1), mis, tid);
    }
    PairTotals acc{0u, 0u, 0u};
    for (int t = t0; t < t1; t += 2) {
        const bool n0 = t + 2 < t1, n1 = t + 3 < t1;
        const TileSplit nsp0 = lds_split(s_split, n0 ? t + 2 - t0 : 0);
        pair_tile<STARTS>(sh, t, t1 - 1, sp0, g0, tg0, rg0, n0, nsp0, pa, ca, pb, cb, mis,
                          write_chunk, chunk_count, starts, acc, tid);
        sp0 = nsp0;
        g0 = grain_layout(sp0, mis.ca, mis.cb);
        if (t + 1 < t1) {
            const TileSplit nsp1 = lds_split(s_split, n1 ? t + 3 - t0 : 0);
            pair_tile<STARTS>(sh, t + 1, t1 - 1, sp1, g1, tg1, rg1, n1, nsp1, pa, ca, pb, cb,
                              mis, write_chunk, chunk_count, starts, acc, tid);
            sp1 = nsp1;
            g1 = grain_layout(sp1, mis.ca, mis.cb);
        }
    }
    if (tid == 0) dev::add_to_total(acc.total, done, length_out);
}

// Writes the result: crd/val (VALUES) or crd plus child pointers (CHILD: for output o,
// child_a[o] = next_a[a] and child_b[o] = next_b[b] at the A/B positions a, b reached before
// o, so [child[o], child[o+1]) is the operand's child range under o, empty when absent; a
// null next_a / next_b makes the child pointer the position itself).
//
// SPREAD (intersection only, no count pass): a tile's outputs go to cc/vc at the tile's own
// start position in A (spread_by_a) or B, whose range holds every pair the tile can emit;
// row ends write pos in those coordinates, tile_count[t] receives the tile's length and
// chunk_total[w] the sum over workgroup w's chunk, and the last workgroup to finish stores
// the sum of all chunks, the result length, to `length_out`.  csr_compact_kernel then moves
// each tile to its final offset and corrects its rows' pos.
//
// SEARCH (union without stored lane starts): every lane finds its start from the tile's
// row-start bins and a search inside its row, as the spread intersection does, instead of
// loading it from `starts`.  When `mode` is non-null and holds kModeSearch, chunk_count
// holds each chunk's pairs instead of its output count.
//
// ROWS (value levels): rc receives each output's row, staged in LDS beside the outputs.
template <Op OP, int IPT, bool VALUES, bool CHILD, bool SPREAD, bool SEARCH = false,
          bool ROWS = false>
__global__ __launch_bounds__(kBlock) void csr_write_kernel(
    const int *__restrict__ pa, const int *__restrict__ ca, const float *__restrict__ va,
    const int *__restrict__ pb, const int *__restrict__ cb, const float *__restrict__ vb,
    int nnz_a, int nnz_b, int num_tiles, int chunk, const int *__restrict__ split_r,
    const int *__restrict__ split_a, const int *__restrict__ split_b,
    const unsigned *__restrict__ chunk_count, int rows, int *__restrict__ pc,
    int *__restrict__ cc, float *__restrict__ vc, const int *__restrict__ next_a,
    const int *__restrict__ next_b, int *__restrict__ child_a, int *__restrict__ child_b,
    unsigned *__restrict__ length, int spread_by_a, int64_t *__restrict__ tile_count,
    int64_t *__restrict__ chunk_total, unsigned long long *__restrict__ done,
    int64_t *__restrict__ length_out, const uint2 *__restrict__ starts,
    const int *__restrict__ mode, int *__restrict__ rc, int *__restrict__ ck, int kbits) {
    static_assert(!(VALUES && CHILD), "a level carries values or child pointers, not both");
    static_assert(!(ROWS && !VALUES), "output rows: value levels");
    static_assert(IPT == kItemsPerLane, "the staged tile is kTile items");
    // ck (value levels, optional): outputs stored split, c >> kbits to cc and the low kbits
    // to ck
    static_assert(!SPREAD || (OP == Op::Intersect && !CHILD), "spread output: intersection");
    constexpr int kSteps = IPT + 1;
    constexpr int kLoads = (kCap + kBlock - 1) / kBlock;  // outputs per lane in the stores
    // A third array: the outputs' packed child positions, or their tile-local rows (a tile
    // stages fewer than 2^16 rows).
    constexpr bool kAux = CHILD || ROWS;
    using Aux = typename std::conditional<CHILD, unsigned, unsigned short>::type;
    __shared__ int s_cr[kCap];  // coordinates then row words (see slot staging)
    __shared__ float s_val[VALUES ? kCap : 1];
    __shared__ Aux s_aux[kAux ? kCap : 1];
    __shared__ int s_wave[kBlock / dev::kWave];
    __shared__ int s_split[3 * (kMaxChunk + 1)];
    constexpr bool kOwn = SPREAD || SEARCH;  // lanes find their own starts
    __shared__ unsigned s_bin[kOwn ? kBlock : 1];  // row-start bins (see stage_slot)

    const int tid = threadIdx.x;
    int t0, t1;
    chunk_range(num_tiles, chunk, t0, t1);
    if (t0 >= t1) {
        if (SPREAD) {
            if (tid == 0) {
                chunk_total[blockIdx.x] = 0;
                dev::add_to_total(0u, done, length_out);
            }
        }
        return;
    }
    if (kOwn) s_bin[tid] = 0u;
    stage_splits(s_split, split_r, split_a, split_b, t0, t1);

    // Offset of this chunk: the counts of every earlier chunk.
    int base = 0;
    if (!SPREAD) {
        int before = 0;
        for (int i = tid; i < static_cast<int>(blockIdx.x); i += kBlock) before += chunk_count[i];
        int total = 0;
        (void)dev::block_exclusive_sum<kBlock>(before, s_wave, total);
        base = total;
        if (SEARCH && mode != nullptr && *mode == kModeSearch) {
            // chunk_count holds pairs: outputs before this chunk are its A and B entries
            // before it (the staged splits of tile t0) less the pairs merged among them
            base = s_split[1] + s_split[2] - total;
        }
    } else {
        __syncthreads();  // the staged splits
    }
    if (blockIdx.x == 0 && tid == 0) pc[0] = 0;

    TileSplit sp = lds_split(s_split, 0);  // (the exclusive sum above ended with a barrier)
    Slots st;
    fetch_slots<VALUES>(st, sp, pa, ca, va, pb, cb, vb, tid);
    // A union's lane starts come from its count kernel (loaded one tile ahead); the spread
    // intersection has no count pass, and the SEARCH union has no stored starts: their lanes
    // take their row from the row-start bins and search only inside it.
    constexpr bool kGiven = !kOwn;
    constexpr Start kMode = kOwn ? Start::RowGiven : Start::Given;
    constexpr int kBinIpt = kOwn ? IPT : 0;  // stage_slots fills the bins only then
    stage_slots<VALUES, kBinIpt>(st, sp, s_cr, s_val, tid, pa, ca, va, pb, cb, vb, s_bin, 1u,
                                 t0 * kBlock * IPT);
    __syncthreads();
    TileSplit nsp = lds_split(s_split, t0 + 1 < t1 ? 1 : 0);
    int64_t spread_sum = 0;
    LaneStart cur{0u, 0u}, nxt{0u, 0u};
    if (kGiven) {
        const uint2 v = starts[static_cast<size_t>(t0) * kBlock + tid];
        cur = LaneStart{v.x, v.y};
    } else {
        cur = LaneStart{static_cast<unsigned>(lane_first_row(s_bin, 1u, tid)), 0u};
    }
    for (int t = t0; t < t1; ++t) {
        fetch_slots<VALUES>(st, nsp, pa, ca, va, pb, cb, vb, tid);
        if (kGiven && t + 1 < t1) {
            const uint2 v = starts[static_cast<size_t>(t + 1) * kBlock + tid];
            nxt = LaneStart{v.x, v.y};
        }
        const TileSplit nsp2 = lds_split(s_split, t + 2 < t1 ? t + 2 - t0 : t + 1 < t1 ? t + 1 - t0 : t - t0);
        LaneOut<kSteps> lo;
        const unsigned *s_row =
            reinterpret_cast<const unsigned *>(s_cr) + (sp.a1 - sp.a0) + (sp.b1 - sp.b0);
        walk_lane<OP, VALUES, CHILD, IPT, kMode>(lo, sp, t, s_cr, s_val, s_row, tid, cur);
        if (kGiven) cur = nxt;
        if (SPREAD) base = spread_by_a ? sp.a0 : sp.b0;

        int tile_total = 0;
        // (the scan's barrier also means every lane is done reading this tile's LDS inputs;
        // s_wave is next written after this tile's later barriers)
        const int offset = dev::block_exclusive_sum<kBlock, int, false>(
            static_cast<int>(__popc(lo.valid)), s_wave, tile_total);

        int o = offset, r = lo.first_row;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (lo.row_ends & (1u << s)) {
                pc[r + 1] = base + o;
                ++r;
            }
            if (lo.valid & (1u << s)) {
                s_cr[o] = lo.crd[s];
                if (VALUES) s_val[o] = lo.val[s];
                if (ROWS) s_aux[o] = static_cast<Aux>(r - sp.r0);
                // child pointers: the A / B positions before the output, tile-local, packed;
                // the pointers themselves are gathered by the coalesced store below
                if (CHILD) s_aux[o] = lo.pos[s];
                ++o;
            }
        }
        __syncthreads();
        // Coalesced stores of the staged outputs, in passes of kPass outputs per lane.  Child
        // pointers of a pass's outputs are all gathered before any is stored (lanes past the
        // tile's end repeat its last output); a pass of 8 keeps the gathered pointers in 16
        // registers.
        constexpr int kPass = CHILD ? 8 : kLoads;
        const unsigned low_mask = (1u << kbits) - 1u;  // kbits <= 31
#pragma unroll
        for (int j0 = 0; j0 < kLoads; j0 += kPass) {
            if (j0 * kBlock >= tile_total) break;  // uniform
            int ga[CHILD ? kPass : 1], gb[CHILD ? kPass : 1];
            if (CHILD) {
#pragma unroll
                for (int j = 0; j < kPass; ++j) {
                    const int q = min(tid + (j0 + j) * kBlock, tile_total - 1);
                    const unsigned pq = s_aux[q];
                    const int pa_q = sp.a0 + static_cast<int>(pq & 0xffffu);
                    const int pb_q = sp.b0 + static_cast<int>(pq >> 16);
                    ga[j] = next_a ? next_a[pa_q] : pa_q;
                    gb[j] = next_b ? next_b[pb_q] : pb_q;
                }
            }
#pragma unroll
            for (int j = 0; j < kPass; ++j) {
                const int q = tid + (j0 + j) * kBlock;
                if (q < tile_total) {
                    if (VALUES && ck) {
                        const int c = s_cr[q];
                        cc[base + q] = c >> kbits;
                        ck[base + q] = static_cast<int>(static_cast<unsigned>(c) & low_mask);
                    } else {
                        cc[base + q] = s_cr[q];
                    }
                    if (VALUES) vc[base + q] = s_val[q];
                    if (ROWS) rc[base + q] = sp.r0 + static_cast<int>(s_aux[q]);
                    if (CHILD) {
                        child_a[base + q] = ga[j];
                        child_b[base + q] = gb[j];
                    }
                }
            }
        }
        if (SPREAD && tid == 0) {
            tile_count[t] = tile_total;
            spread_sum += tile_total;
            if (t + 1 == t1) chunk_total[blockIdx.x] = spread_sum;
        }
        base += tile_total;
        if (!SPREAD && t == num_tiles - 1 && tid == 0) {
            *length = static_cast<unsigned>(base);
            if (CHILD) {
                child_a[base] = next_a ? next_a[nnz_a] : nnz_a;
                child_b[base] = next_b ? next_b[nnz_b] : nnz_b;
            }
        }
        __syncthreads();  // staged outputs consumed
        if (t + 1 < t1) {
            const unsigned tag = static_cast<unsigned>(t + 2 - t0);
            stage_slots<VALUES, kBinIpt>(st, nsp, s_cr, s_val, tid, pa, ca, va, pb, cb, vb,
                                         s_bin, tag, (t + 1) * kBlock * IPT);
            __syncthreads();
            if (!kGiven) {
                cur = LaneStart{static_cast<unsigned>(lane_first_row(s_bin, tag, tid)),
                                0u};
            }
        }
        sp = nsp;
        nsp = nsp2;
    }
    // Spread output: the last workgroup to finish stores the result length.
    if (SPREAD && tid == 0) dev::add_to_total(static_cast<uint32_t>(spread_sum), done, length_out);
}

// Moves each tile's outputs from its spread position (csr_write_kernel<SPREAD>) to its final
// offset and shifts the pos entries of the rows ending in the tile (rows
// [split_r[t], split_r[t + 1]), every remaining row for the last tile) by the same amount.
// The offset is the sum of the earlier chunks' totals and of the earlier tiles of its own
// chunk (`chunk` tiles per chunk).  One workgroup per tile; the last one stores the length.
__global__ __launch_bounds__(kBlock) void csr_compact_kernel(
    const int *__restrict__ split_r, const int *__restrict__ split_a,
    const int *__restrict__ split_b, int num_tiles, int chunk, int rows, int spread_by_a,
    const int64_t *__restrict__ tile_count, const int64_t *__restrict__ chunk_total,
    const int *__restrict__ tmp_crd, const float *__restrict__ tmp_val, int *__restrict__ pc,
    int *__restrict__ cc, float *__restrict__ vc, int64_t *__restrict__ length,
    const int *__restrict__ tmp_row, int *__restrict__ rc) {
    __shared__ int64_t s_wave[kBlock / dev::kWave];
    const int t = blockIdx.x;
    const int c = t / chunk;
    // The tile's pairs are loaded first (they do not depend on its offset), so that their
    // loads are in flight while the offset is summed.  A tile holds at most kTile + 1 items.
    constexpr int kMove = (kTile + 1 + kBlock - 1) / kBlock;
    const int from = spread_by_a ? split_a[t] : split_b[t];
    const int n = static_cast<int>(tile_count[t]);
    int mc[kMove];
    float mv[kMove];
#pragma unroll
    for (int k = 0; k < kMove; ++k) {
        const int q = static_cast<int>(threadIdx.x) + k * kBlock;
        mc[k] = 0;
        mv[k] = 0.0f;
        if (q < n) {
            mc[k] = tmp_crd[from + q];
            mv[k] = tmp_val[from + q];
        }
    }
    int64_t before = 0;
    for (int i = threadIdx.x; i < c; i += kBlock) before += chunk_total[i];
    for (int i = c * chunk + static_cast<int>(threadIdx.x); i < t; i += kBlock) before += tile_count[i];
    int64_t to64 = 0;
    (void)dev::block_exclusive_sum<kBlock>(before, s_wave, to64);
    const int to = static_cast<int>(to64);
    if (t == num_tiles - 1 && threadIdx.x == 0) *length = to64 + n;
#pragma unroll
    for (int k = 0; k < kMove; ++k) {
        const int q = static_cast<int>(threadIdx.x) + k * kBlock;
        if (q < n) {
            cc[to + q] = mc[k];
            vc[to + q] = mv[k];
            if (rc) rc[to + q] = tmp_row[from + q];
        }
    }
    const int r_end = t + 1 < num_tiles ? split_r[t + 1] : rows;
    for (int r = split_r[t] + static_cast<int>(threadIdx.x); r < r_end; r += kBlock) {
        pc[r + 1] += to - from;
    }
}

// ---- host ------------------------------------------------------------------------------

// Offset of an int32 array's base from a 16-byte boundary, in elements; int32 arrays must
// be 4-byte aligned.  A null (empty) array counts as aligned.
int misalign(const void *p, int *out) {
    const uintptr_t v = reinterpret_cast<uintptr_t>(p);
    if (v & 3u) return NACHO_ERR_INVALID_ARGUMENT;
    *out = static_cast<int>((v & 15u) >> 2);
    return NACHO_OK;
}

// ---- inner product of a spread intersection -------------------------------------------

// Binary64 sum of the kBlock values of `sh` into sh[0], in a fixed order; ends synchronised.
__device__ __forceinline__ void block_sum_fixed(double *sh) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        __syncthreads();
        if (tid < w) sh[tid] += sh[tid + w];
    }
    __syncthreads();
}

// Workgroups of the two-level sums below: few enough that one workgroup then adds their
// partials in a handful of loads per thread.
constexpr int kDotBlocks = 1024;

// Workgroup b sums the products that tiles [b*T/G, (b+1)*T/G) of the spread intersection
// wrote (tile_count[t] of them each, at the tile's own start position in the smaller
// operand's range) in binary64, in a fixed order: partial[b].
__global__ __launch_bounds__(kBlock) void dot_tiles_kernel(
    const int *__restrict__ split_a, const int *__restrict__ split_b, int by_a,
    const int64_t *__restrict__ tile_count, int num_tiles, const float *__restrict__ prod,
    double *__restrict__ partial) {
    __shared__ double sh[kBlock];
    const long long g = gridDim.x;
    const int t0 = static_cast<int>(num_tiles * static_cast<long long>(blockIdx.x) / g);
    const int t1 = static_cast<int>(num_tiles * (static_cast<long long>(blockIdx.x) + 1) / g);
    double acc = 0.0;
    for (int t = t0; t < t1; ++t) {
        const int base = by_a ? split_a[t] : split_b[t];
        const int n = static_cast<int>(tile_count[t]);
        for (int i = threadIdx.x; i < n; i += kBlock) acc += static_cast<double>(prod[base + i]);
    }
    sh[threadIdx.x] = acc;
    block_sum_fixed(sh);
    if (threadIdx.x == 0) partial[blockIdx.x] = sh[0];
}

// One workgroup: the sum of the n tile partials in a fixed order, rounded once to *dot.
__global__ __launch_bounds__(kBlock) void dot_final_kernel(const double *__restrict__ partial,
                                                           int n, float *__restrict__ dot) {
    __shared__ double sh[kBlock];
    double acc = 0.0;
    for (int i = threadIdx.x; i < n; i += kBlock) acc += partial[i];
    sh[threadIdx.x] = acc;
    block_sum_fixed(sh);
    if (threadIdx.x == 0) *dot = static_cast<float>(sh[0]);
}

// Workgroup b of G sums v[b*n/G, (b+1)*n/G) in binary64, in a fixed order: partial[b].
__global__ __launch_bounds__(kBlock) void sum_blocks_kernel(const float *__restrict__ v,
                                                            long long n,
                                                            double *__restrict__ partial) {
    __shared__ double sh[kBlock];
    const long long g = gridDim.x;
    const long long lo = n * static_cast<long long>(blockIdx.x) / g;
    const long long hi = n * (static_cast<long long>(blockIdx.x) + 1) / g;
    double acc = 0.0;
    for (long long i = lo + threadIdx.x; i < hi; i += kBlock) acc += static_cast<double>(v[i]);
    sh[threadIdx.x] = acc;
    block_sum_fixed(sh);
    if (threadIdx.x == 0) partial[blockIdx.x] = sh[0];
}

int sum_values(Call &call, const float *v, long long n, float *out) {
    const int blocks = static_cast<int>(
        std::max<long long>(1, std::min<long long>(kDotBlocks, (n + kBlock - 1) / kBlock)));
    double *partial = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(blocks), &partial));
    const hipStream_t s = call.stream();
    sum_blocks_kernel<<<blocks, kBlock, 0, s>>>(v, n, partial);
    NACHO_TRY_HIP(hipGetLastError());
    dot_final_kernel<<<1, kBlock, 0, s>>>(partial, blocks, out);
    NACHO_TRY_HIP(hipGetLastError());
    return NACHO_OK;
}

template <Op OP, bool VALUES, bool CHILD, bool SPREAD, bool SEARCH, bool ROWS>
const void *write_kernel_of() {
    return reinterpret_cast<const void *>(
        csr_write_kernel<OP, kItemsPerLane, VALUES, CHILD, SPREAD, SEARCH, ROWS>);
}

int merge_level(Call &call, bool intersect, bool values, bool child, int rows,
                const LevelOperand &A, const LevelOperand &B, const LevelResult &Z,
                long long *out_len, const char *kernel_name, UnionCount count_plan,
                bool *length_pending) {
    if (length_pending) *length_pending = false;
    const long long total = static_cast<long long>(A.len) + B.len + rows;
    if (total > static_cast<long long>(INT_MAX) - 2 * kTile) return NACHO_ERR_INDEX_OVERFLOW;
    const int num_tiles = total > 0 ? static_cast<int>((total + kTile - 1) / kTile) : 1;

    int *splits = nullptr;
    unsigned *counts = nullptr;
    NACHO_TRY(call.scratch_n(3 * (static_cast<size_t>(num_tiles) + 1), &splits));
    int *split_r = splits, *split_a = splits + num_tiles + 1, *split_b = splits + 2 * (num_tiles + 1);

    // How a union level counts (see UnionCount): the row pass and the pair search where
    // rows are long enough, else the tile walk, storing lane starts where the write pass
    // does not search for them.
    const long long items = static_cast<long long>(A.len) + B.len;
    const bool row_pass = !intersect && values && count_plan == UnionCount::kAuto &&
                          static_cast<long long>(rows) * kRowPassMinEntriesPerRow <= items;
    const bool keep_starts =
        !intersect && (!values || (count_plan == UnionCount::kAuto && !row_pass));
    const bool out_rows = values && Z.row != nullptr;
    // The write kernel this level launches.
    const void *write_kernel =
        intersect ? (out_rows ? write_kernel_of<Op::Intersect, true, false, true, false, true>()
                              : write_kernel_of<Op::Intersect, true, false, true, false, false>())
        : !values ? (child ? write_kernel_of<Op::Union, false, true, false, false, false>()
                           : write_kernel_of<Op::Union, false, false, false, false, false>())
        : keep_starts ? (out_rows ? write_kernel_of<Op::Union, true, false, false, false, true>()
                                  : write_kernel_of<Op::Union, true, false, false, false, false>())
                      : (out_rows ? write_kernel_of<Op::Union, true, false, false, true, true>()
                                  : write_kernel_of<Op::Union, true, false, false, true, false>());
    // Grid: as many workgroups of the write kernel as stay resident, each owning a
    // contiguous chunk of tiles.
    int resident = 0;
    NACHO_TRY(resident_grid(write_kernel, kBlock, &resident));
    int chunk = (num_tiles + resident - 1) / resident;
    if (chunk > kMaxChunk) chunk = kMaxChunk;  // more workgroups than resident: still correct
    const int grid = (num_tiles + chunk - 1) / chunk;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 4 + 2 * dev::kTotalWords, &counts));
    unsigned *length = counts + grid;
    // 64-bit accumulator of the length total (8-byte aligned words after the counts).
    unsigned long long *done =
        reinterpret_cast<unsigned long long *>(counts + ((grid + 2) & ~1));
    // The result length goes straight to a pinned host word as soon as the kernel that
    // totals it ends; the host waits for that kernel only, not for the writes after it.
    int64_t *length_out = nullptr;
    NACHO_TRY(call.length_word(&length_out));

    const hipStream_t s = call.stream();
    if (intersect) {
        // One walk: each tile writes its pairs at its own position in the smaller operand's
        // range of a scratch buffer, then one compaction moves them into place.
        if (!values || child || Z.crd_low) return NACHO_ERR_INVALID_ARGUMENT;
        const int by_a = A.len <= B.len ? 1 : 0;
        const size_t cap = static_cast<size_t>(by_a ? A.len : B.len);
        int *tmp_crd = nullptr, *tmp_row = nullptr;
        float *tmp_val = nullptr;
        int64_t *tile_count = nullptr, *chunk_total = nullptr;
        NACHO_TRY(call.scratch_n(cap, &tmp_crd));
        NACHO_TRY(call.scratch_n(cap, &tmp_val));
        if (Z.row) NACHO_TRY(call.scratch_n(cap, &tmp_row));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles), &tile_count));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(grid) + 2, &chunk_total));
        int64_t *len_dev = chunk_total + grid;
        int *pos = Z.pos;
        double *partial = nullptr;
        const int dot_grid = std::min(num_tiles, kDotBlocks);
        if (Z.dot) {
            // the inner product: the spread write's pos and length go to scratch, and the
            // host does not wait for the length
            NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pos));
            NACHO_TRY(call.scratch_n(static_cast<size_t>(dot_grid), &partial));
            length_out = chunk_total + grid + 1;
        }
        NACHO_TRY(call.timer_start(kernel_name));  // the whole device pipeline of this level
        const int part_blocks = static_cast<int>(ceil_div((static_cast<size_t>(num_tiles) + 1) * kPartLanes, kPartBlock));
        csr_partition_kernel<<<part_blocks, kPartBlock, 0, s>>>(
            A.pos, A.crd, B.pos, B.crd, rows, static_cast<int>(total), num_tiles, split_r,
            split_a, split_b, done, nullptr, 0, part_blocks, RowPairs{});
        NACHO_TRY_HIP(hipGetLastError());
#define NACHO_SPREAD_LAUNCH(ROWS)                                                             \
    csr_write_kernel<Op::Intersect, kItemsPerLane, true, false, true, false, ROWS>           \
        <<<grid, kBlock, 0, s>>>(A.pos, A.crd, A.val, B.pos, B.crd, B.val, A.len, B.len,     \
                                 num_tiles, chunk, split_r, split_a, split_b, nullptr, rows, \
                                 pos, tmp_crd, tmp_val, nullptr, nullptr, nullptr, nullptr, \
                                 nullptr, by_a, tile_count, chunk_total, done, length_out,   \
                                 nullptr, nullptr, tmp_row, nullptr, 0)
        if (tmp_row) {
            NACHO_SPREAD_LAUNCH(true);
        } else {
            NACHO_SPREAD_LAUNCH(false);
        }
#undef NACHO_SPREAD_LAUNCH
        NACHO_TRY_HIP(hipGetLastError());
        if (Z.dot) {
            dot_tiles_kernel<<<dot_grid, kBlock, 0, s>>>(split_a, split_b, by_a, tile_count,
                                                         num_tiles, tmp_val, partial);
            NACHO_TRY_HIP(hipGetLastError());
            dot_final_kernel<<<1, kBlock, 0, s>>>(partial, dot_grid, Z.dot);
            NACHO_TRY_HIP(hipGetLastError());
            NACHO_TRY(call.timer_stop());
            NACHO_TRY(call.collect_timer());  // (kernel timing only: waits for the stream)
            *out_len = 0;
            return NACHO_OK;
        }
        NACHO_TRY(call.mark_length());
        csr_compact_kernel<<<num_tiles, kBlock, 0, s>>>(
            split_r, split_a, split_b, num_tiles, chunk, rows, by_a, tile_count, chunk_total,
            tmp_crd, tmp_val, Z.pos, Z.crd, Z.val, len_dev, tmp_row, Z.row);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        if (length_pending) {
            *length_pending = true;
            return NACHO_OK;
        }
        int64_t len = 0;
        NACHO_TRY(call.wait_length(&len));
        *out_len = len;
        return NACHO_OK;
    }
    // Union: the pair count gives the write chunks' output counts (and the length) and, when
    // keep_starts, every lane's walk start; without it the write pass searches for them.
    Misalign mis{};
    NACHO_TRY(misalign(A.crd, &mis.ca));
    NACHO_TRY(misalign(B.crd, &mis.cb));
    NACHO_TRY(misalign(A.pos, &mis.pa));
    NACHO_TRY(misalign(B.pos, &mis.pb));
    if (!values && count_plan != UnionCount::kAuto) return NACHO_ERR_INVALID_ARGUMENT;
    uint2 *starts = nullptr;
    if (keep_starts) NACHO_TRY(call.scratch_n(static_cast<size_t>(num_tiles) * kBlock, &starts));
    RowPairs rp{};
    int row_grid = 0;
    if (row_pass) {
        // at most kRowPassMaxBlocks workgroups of kPartBlock threads, at least 16 rows each
        const long long per_thread = std::max<long long>(
            16, (static_cast<long long>(rows) + kPartBlock * kRowPassMaxBlocks - 1) /
                    (kPartBlock * kRowPassMaxBlocks));
        const long long per_block = per_thread * kPartBlock;
        row_grid = static_cast<int>(std::max<long long>(1, (rows + per_block - 1) / per_block));
        rp.rows_per_thread = static_cast<int>(per_thread);
        rp.nb = row_grid;
        // record regions by row, or by the entries of the operand with fewer of them
        const long long by_rows = static_cast<long long>(row_grid) * per_block;
        const long long by_entries = std::min<long long>(A.len, B.len);
        rp.px = by_entries < by_rows ? (A.len <= B.len ? A.pos : B.pos) : nullptr;
        const size_t n_rec =
            static_cast<size_t>(std::max<long long>(1, std::min(by_rows, by_entries)));
        NACHO_TRY(call.scratch_n(n_rec, &rp.rec));
        NACHO_TRY(call.scratch_n(n_rec, &rp.rec_row));
        int *words = nullptr;
        NACHO_TRY(call.scratch_n(3 * static_cast<size_t>(row_grid) + 1, &words));
        rp.blk_base = words;
        rp.blk_elems = words + row_grid;
        rp.blk_recs = words + 2 * row_grid;
        rp.mode = words + 3 * row_grid;
    }
    // The count kernel's own grid: as many workgroups as it keeps resident (it holds less
    // state than the write kernel, and needs the extra loads in flight).
    int count_resident = 0;
    const void *count_kernel =
        keep_starts ? reinterpret_cast<const void *>(csr_pair_count_kernel<true>)
                    : reinterpret_cast<const void *>(csr_pair_count_kernel<false>);
    NACHO_TRY(resident_grid(count_kernel, kBlock, &count_resident));
    int count_chunk = (num_tiles + count_resident - 1) / count_resident;
    if (count_chunk > kMaxChunk) count_chunk = kMaxChunk;
    const int count_grid = (num_tiles + count_chunk - 1) / count_chunk;
    NACHO_TRY(call.timer_start(kernel_name));  // the whole device pipeline of this level
    const int part_blocks = static_cast<int>(ceil_div((static_cast<size_t>(num_tiles) + 1) * kPartLanes, kPartBlock));
    csr_partition_kernel<<<part_blocks + row_grid, kPartBlock, 0, s>>>(
        A.pos, A.crd, B.pos, B.crd, rows, static_cast<int>(total), num_tiles, split_r, split_a,
        split_b, done, counts, grid, part_blocks, rp);
    NACHO_TRY_HIP(hipGetLastError());
    if (keep_starts) {
        csr_pair_count_kernel<true><<<count_grid, kBlock, 0, s>>>(
            A.pos, A.crd, B.pos, B.crd, mis, num_tiles, count_chunk, chunk, split_r, split_a,
            split_b, counts, done, length_out, starts, RowPairs{}, grid, items);
    } else {
        csr_pair_count_kernel<false><<<count_grid, kBlock, 0, s>>>(
            A.pos, A.crd, B.pos, B.crd, mis, num_tiles, count_chunk, chunk, split_r, split_a,
            split_b, counts, done, length_out, nullptr, rp, grid, items);
    }
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.mark_length());
#define NACHO_WRITE_LAUNCH(OPV, VAL, CHD, SRCH, ROWS)                                            \
    csr_write_kernel<OPV, kItemsPerLane, VAL, CHD, false, SRCH, ROWS><<<grid, kBlock, 0, s>>>(   \
        A.pos, A.crd, A.val, B.pos, B.crd, B.val, A.len, B.len, num_tiles, chunk, split_r,      \
        split_a, split_b, counts, rows, Z.pos, Z.crd, Z.val, A.next, B.next, Z.child_a,         \
        Z.child_b, length, 0, nullptr, nullptr, nullptr, nullptr, starts, rp.mode,             \
        VAL ? Z.row : nullptr, VAL ? Z.crd_low : nullptr, Z.low_bits)
    if (values) {
        if (child) return NACHO_ERR_INVALID_ARGUMENT;
        if (keep_starts) {
            if (Z.row) {
                NACHO_WRITE_LAUNCH(Op::Union, true, false, false, true);
            } else {
                NACHO_WRITE_LAUNCH(Op::Union, true, false, false, false);
            }
        } else if (Z.row) {
            NACHO_WRITE_LAUNCH(Op::Union, true, false, true, true);
        } else {
            NACHO_WRITE_LAUNCH(Op::Union, true, false, true, false);
        }
    } else if (child) {
        NACHO_WRITE_LAUNCH(Op::Union, false, true, false, false);
    } else {
        NACHO_WRITE_LAUNCH(Op::Union, false, false, false, false);
    }
#undef NACHO_WRITE_LAUNCH
    NACHO_TRY_HIP(hipGetLastError());
    NACHO_TRY(call.timer_stop());

    int64_t len = 0;
    NACHO_TRY(call.wait_length(&len));
    *out_len = len;
    return NACHO_OK;
}

size_t merge_level_arena_bytes(long long items) {
    const long long tiles = items > 0 ? (items + kTile - 1) / kTile : 1;
    // splits (3 per boundary), chunk counts (at most one per tile) plus the ticket words,
    // the length word, and 256-byte alignment of each piece
    return static_cast<size_t>(12 * (tiles + 1) + 4 * (tiles + 6) + 8 + 4 * 256);
}

bool bad_csr(const nacho_csr *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0) return true;
    if (!t->dim_j_offsets) return true;
    if (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values)) return true;
    return false;
}

int csr_binary(bool intersect, const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
               int32_t num_blocks, int32_t threads_per_block, void *stream,
               const nacho_allocator *alloc, const char *kernel_name) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csr{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csr(a) || bad_csr(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size;
    const long long nnz_a = a->dim_j_length, nnz_b = b->dim_j_length;
    if (nnz_a + nnz_b + rows > static_cast<long long>(INT_MAX) - 2 * kTile) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }
    const long long cap = intersect ? (nnz_a < nnz_b ? nnz_a : nnz_b) : nnz_a + nnz_b;

    Call call(stream, alloc);
    int *pc = nullptr, *cc = nullptr;
    float *vc = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(rows) + 1, &pc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &cc));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap), &vc));

    const LevelOperand A{a->dim_j_offsets, a->dim_j_indices, a->values, a->dim_j_length, nullptr};
    const LevelOperand B{b->dim_j_offsets, b->dim_j_indices, b->values, b->dim_j_length, nullptr};
    const LevelResult Z{pc, cc, vc, nullptr, nullptr};
    long long nnz = 0;
    NACHO_TRY(merge_level(call, intersect, true, false, rows, A, B, Z, &nnz, kernel_name));
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

// ---- allocation-free csr_add ------------------------------------------------------------
// Scratch of nacho_gpu_csr_add_f32_noalloc: a file-scope device array, one copy per GPU,
// held for the life of the process.  Host code never passes `scratch` itself to a kernel
// (in host code the name is a stand-in, not a device address): it looks up each device's
// address once with hipGetSymbolAddress and uses that.
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// One GPU's `scratch`: its device address (looked up on the first call there) and the lock
// that one call holds from its first launch until its last kernel has finished.
struct ScratchSlot {
    std::mutex busy;
    void *address = nullptr;
};

int scratch_slot(ScratchSlot **out) {
    static std::mutex lookup;
    static ScratchSlot slots[kMaxDevices];
    int device = 0;
    NACHO_TRY_HIP(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices) return NACHO_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(lookup);
    ScratchSlot &slot = slots[device];
    if (!slot.address) {
        void *p = nullptr;
        NACHO_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return NACHO_ERR_INTERNAL;
        slot.address = p;
    }
    *out = &slot;
    return NACHO_OK;
}

// Waits for the stream when the call leaves, on every exit path, so that no kernel of the
// call still reads `scratch` once the slot's lock is released.
struct StreamDrain {
    hipStream_t stream;
    ~StreamDrain() { (void)hipStreamSynchronize(stream); }
};

int csr_add_noalloc(const nacho_csr *a, const nacho_csr *b, nacho_csr *z, int32_t num_blocks,
                    int32_t threads_per_block, void *stream) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    int *pc = z->dim_j_offsets, *cc = z->dim_j_indices;
    float *vc = z->values;
    const long long capacity = z->dim_j_length;
    z->dim_j_length = 0;
    z->nnz = 0;
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csr(a) || bad_csr(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const int rows = a->dim_i_size;
    const long long nnz_a = a->dim_j_length, nnz_b = b->dim_j_length;
    const long long items = nnz_a + nnz_b + rows;
    if (items > static_cast<long long>(INT_MAX) - 2 * kTile) return NACHO_ERR_INDEX_OVERFLOW;
    if (!pc || capacity < nnz_a + nnz_b || (capacity > 0 && (!cc || !vc))) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    if (items > NACHO_NOALLOC_MAX_ITEMS) return NACHO_ERR_SCRATCH_TOO_SMALL;
    if (merge_level_arena_bytes(items) > kNoAllocScratchBytes) return NACHO_ERR_INTERNAL;
    ScratchSlot *slot = nullptr;
    NACHO_TRY(scratch_slot(&slot));
    // Calls on one GPU take turns: the lock is held until the call's kernels have drained
    // (StreamDrain runs after Call's destructor, before the lock is released).
    std::lock_guard<std::mutex> hold(slot->busy);
    StreamDrain drain{static_cast<hipStream_t>(stream)};
    Call call(stream, slot->address, kNoAllocScratchBytes);
    const LevelOperand A{a->dim_j_offsets, a->dim_j_indices, a->values, a->dim_j_length, nullptr};
    const LevelOperand B{b->dim_j_offsets, b->dim_j_indices, b->values, b->dim_j_length, nullptr};
    const LevelResult Z{pc, cc, vc, nullptr, nullptr};
    long long nnz = 0;
    NACHO_TRY(merge_level(call, false, true, false, rows, A, B, Z, &nnz,
                          "csr_add (no-alloc): partition+count+write", UnionCount::kTileWalk));
    if (nnz > nnz_a + nnz_b) return NACHO_ERR_MALFORMED_INPUT;
    z->dim_i_size = rows;
    z->dim_j_size = a->dim_j_size;
    z->dim_j_length = static_cast<int32_t>(nnz);
    z->nnz = static_cast<int32_t>(nnz);
    return NACHO_OK;
}

}  // namespace csr
}  // namespace nacho

extern "C" {

int nacho_gpu_csr_add_f32_noalloc(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                                  int32_t num_blocks, int32_t threads_per_block,
                                  void *stream) {
    return nacho::csr::csr_add_noalloc(a, b, z, num_blocks, threads_per_block, stream);
}


int nacho_gpu_csr_add_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::csr::csr_binary(false, a, b, z, num_blocks, threads_per_block, stream, alloc,
                                  "csr_add: partition+count+write");
}

int nacho_gpu_csr_mul_f32(const nacho_csr *a, const nacho_csr *b, nacho_csr *z,
                          int32_t num_blocks, int32_t threads_per_block, void *stream,
                          const nacho_allocator *alloc) {
    return nacho::csr::csr_binary(true, a, b, z, num_blocks, threads_per_block, stream, alloc,
                                  "csr_mul: partition+count+write");
}

}  // extern "C"
