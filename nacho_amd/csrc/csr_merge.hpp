// Level merge shared by CSR add/mul and CSF3 add (see csr_merge.hip).
#pragma once

#include <cstdint>

#include "runtime.hpp"

namespace nacho {
namespace csr {

// One operand level: `pos` has rows + 1 entries (pos[0] == 0) indexing `crd`/`val`
// (`len` entries).  `next` (optional) is the offsets array of the level below, indexed by
// this level's positions (len + 1 entries); when null, child pointers are the positions.
struct LevelOperand {
    const int *pos;
    const int *crd;
    const float *val;
    int len;
    const int *next;
};

// Result buffers, sized by the caller for the worst case: pos rows + 1, crd/val (and row)
// the union (or intersection) bound, child_a/child_b that bound + 1.
struct LevelResult {
    int *pos;
    int *crd;
    float *val;
    int *child_a;
    int *child_b;
    // Value levels only, optional: the row of every output (a COO result's i coordinate).
    int *row = nullptr;
    // Union value levels only, optional: each output coordinate c is stored split, as
    // c >> low_bits to crd and c & (2^low_bits - 1) to crd_low (a COO3 result's j and k).
    int *crd_low = nullptr;
    int low_bits = 0;
    // Intersection value levels only, optional: the level's inner product instead of its
    // result.  Σ a·b over the pairs (each product one binary32 multiply, as the result's
    // values) is summed in binary64 in a fixed order, rounded once and stored to this device
    // float; pos, crd and val are then not written (they may be null), *out_len is 0, and
    // the host does not wait for the device.
    float *dot = nullptr;
};

// How a union level counts its output before writing it.
enum class UnionCount {
    // Levels without values: a tile walk that also stores every lane's walk start for the
    // write pass (8 bytes per lane and tile).  Value levels whose rows hold at least 8
    // entries on average: a row pass finds the rows where both operands have entries and
    // chooses, on the device, between searching those rows' smaller sides for pairs (few
    // such entries) and the tile walk; the write pass searches for its lanes' starts.
    // Value levels with shorter rows: the tile walk with stored lane starts.
    kAuto,
    // Value levels only: the tile walk without lane starts and no row pass, so that scratch
    // stays at a few bytes per tile (an arena Call).
    kTileWalk,
};

// Headroom merge_level keeps below INT_MAX for its item count (entries of both operands plus
// rows): it refuses larger levels with NACHO_ERR_INDEX_OVERFLOW.
constexpr long long kLevelTileSlack = 4096;

// Merge A and B row by row: union (or intersection) of each row's coordinates, with values
// (a+b / a*b / copies) when `values`, or with child pointers when `child`.  Writes Z.pos for
// every row and returns the result length in *out_len.  The call's kernel timer (if enabled)
// brackets all of the level's kernels under `kernel_name`.
//
// With `length_pending` (intersection value levels), the host does not wait for the length:
// *length_pending is set, *out_len is left alone, and the caller, having queued what it has
// to on the stream, reads the length with call.wait_length before any other level merge of
// the call (and collects the level's timer with call.collect_timer before starting another).
int merge_level(Call &call, bool intersect, bool values, bool child, int rows,
                const LevelOperand &A, const LevelOperand &B, const LevelResult &Z,
                long long *out_len, const char *kernel_name,
                UnionCount count = UnionCount::kAuto, bool *length_pending = nullptr);

// Σ v[0, n) summed in binary64 in a fixed order and rounded once to the device float *out
// (kernels queued on the call's stream; v may be null when n is 0).
int sum_values(Call &call, const float *v, long long n, float *out);

// A CSR descriptor that no entry point can take (negative sizes, missing buffers).
bool bad_csr(const nacho_csr *t);

// Bytes of scratch merge_level takes from an arena Call for a union level of `items` merge
// items (entries of both operands plus rows) without lane starts.
size_t merge_level_arena_bytes(long long items);

}  // namespace csr
}  // namespace nacho
