// CSF3 elementwise add (union at every level) for gfx950.
//
// Reference path replaced: csf_add (compiler.cpp:135), whose generated kernels partition
// three nested levels with runtime exclusion (partition.cpp:286-461, 551-584) and emit the
// i, j and k levels with one count/scan/readback per level (stitch_and_generate_gpu.cpp:
// 641-715).  The union of two trees is computed here as three chained level merges, each
// the CSR merge of csr_merge.hip:
//   i level: one "row" holding both operands' i coordinates; every output i records the
//            positions reached in A and B, which index their j offsets (child pointers);
//   j level: rows are the output i fibres, each row's A/B ranges given by those child
//            pointers; outputs are the result's j coordinates and its j offsets, plus child
//            pointers into the k level;
//   k level: rows are the output (i, j) fibres; outputs are k coordinates, values (a+b or a
//            copy) and the result's k offsets.
// Every coordinate of each level's union is emitted; for operands without empty fibres (what
// to_csf3 builds) no output fibre is empty.
//
// The inner product (inner_prod, compiler.cpp:141) reduces the intersection of the two trees
// to one value: through rows i of (j, k) column keys built from the levels when the keys fit
// 31 bits, otherwise through the i and j unions above and a k level intersection.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "csr_merge.hpp"
#include "device_utils.hpp"
#include "runtime.hpp"

namespace nacho {
namespace csf {

// Offsets of the virtual root "row" of each operand's i level: {0, ni_a, 0, ni_b}.
__global__ void root_offsets_kernel(int *root, int ni_a, int ni_b) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        root[0] = 0;
        root[1] = ni_a;
        root[2] = 0;
        root[3] = ni_b;
    }
}

bool bad_csf3(const nacho_csf3 *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_k_size < 0) return true;
    if (t->dim_i_length < 0 || t->dim_j_length < 0 || t->dim_k_length < 0) return true;
    if (t->nnz != t->dim_k_length) return true;
    if (!t->dim_j_offsets || !t->dim_k_offsets) return true;
    if (t->dim_i_length > 0 && !t->dim_i_indices) return true;
    if (t->dim_j_length > 0 && !t->dim_j_indices) return true;
    if (t->dim_k_length > 0 && (!t->dim_k_indices || !t->values)) return true;
    return false;
}

int csf_add(const nacho_csf3 *a, const nacho_csf3 *b, nacho_csf3 *z, int32_t num_blocks,
            int32_t threads_per_block, void *stream, const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_csf3{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csf3(a) || bad_csf3(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size ||
        a->dim_k_size != b->dim_k_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const long long cap_i = static_cast<long long>(a->dim_i_length) + b->dim_i_length;
    const long long cap_j = static_cast<long long>(a->dim_j_length) + b->dim_j_length;
    const long long cap_k = static_cast<long long>(a->dim_k_length) + b->dim_k_length;
    if (cap_k + cap_j > static_cast<long long>(INT_MAX) - (1 << 16)) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }

    Call call(stream, alloc);
    const hipStream_t s = call.stream();

    // i level
    int *root = nullptr, *root_out = nullptr, *ci_a = nullptr, *ci_b = nullptr;
    NACHO_TRY(call.scratch_n(4, &root));
    NACHO_TRY(call.scratch_n(2, &root_out));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_b));
    int *crd_i = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_i), &crd_i));
    root_offsets_kernel<<<1, 64, 0, s>>>(root, a->dim_i_length, b->dim_i_length);
    NACHO_TRY_HIP(hipGetLastError());
    long long ni = 0;
    {
        const csr::LevelOperand A{root, a->dim_i_indices, nullptr, a->dim_i_length, a->dim_j_offsets};
        const csr::LevelOperand B{root + 2, b->dim_i_indices, nullptr, b->dim_i_length,
                                  b->dim_j_offsets};
        const csr::LevelResult Z{root_out, crd_i, nullptr, ci_a, ci_b};
        NACHO_TRY(csr::merge_level(call, false, false, true, 1, A, B, Z, &ni, "csf_add"));
    }

    // j level: rows = output i fibres
    int *pos_j = nullptr, *crd_j = nullptr, *cj_a = nullptr, *cj_b = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(ni) + 1, &pos_j));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_j), &crd_j));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_j) + 1, &cj_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_j) + 1, &cj_b));
    long long nj = 0;
    {
        const csr::LevelOperand A{ci_a, a->dim_j_indices, nullptr, a->dim_j_length, a->dim_k_offsets};
        const csr::LevelOperand B{ci_b, b->dim_j_indices, nullptr, b->dim_j_length, b->dim_k_offsets};
        const csr::LevelResult Z{pos_j, crd_j, nullptr, cj_a, cj_b};
        NACHO_TRY(csr::merge_level(call, false, false, true, static_cast<int>(ni), A, B, Z, &nj,
                                   "csf_add"));
    }

    // k level: rows = output (i, j) fibres; values
    int *pos_k = nullptr, *crd_k = nullptr;
    float *val = nullptr;
    NACHO_TRY(call.result_n(static_cast<size_t>(nj) + 1, &pos_k));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_k), &crd_k));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_k), &val));
    long long nk = 0;
    {
        const csr::LevelOperand A{cj_a, a->dim_k_indices, a->values, a->dim_k_length, nullptr};
        const csr::LevelOperand B{cj_b, b->dim_k_indices, b->values, b->dim_k_length, nullptr};
        const csr::LevelResult Z{pos_k, crd_k, val, nullptr, nullptr};
        NACHO_TRY(csr::merge_level(call, false, true, false, static_cast<int>(nj), A, B, Z, &nk,
                                   "csf_add"));
    }
    if (ni > cap_i || nj > cap_j || nk > cap_k) return NACHO_ERR_MALFORMED_INPUT;
    if (ni == 0) {
        call.drop_result(crd_i);
        crd_i = nullptr;
    }
    if (nj == 0) {
        call.drop_result(crd_j);
        crd_j = nullptr;
    }
    if (nk == 0) {
        call.drop_result(crd_k);
        call.drop_result(val);
        crd_k = nullptr;
        val = nullptr;
    }
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_k_size = a->dim_k_size;
    z->dim_i_length = static_cast<int32_t>(ni);
    z->dim_i_indices = crd_i;
    z->dim_j_offsets = pos_j;
    z->dim_j_length = static_cast<int32_t>(nj);
    z->dim_j_indices = crd_j;
    z->dim_k_offsets = pos_k;
    z->dim_k_length = static_cast<int32_t>(nk);
    z->dim_k_indices = crd_k;
    z->values = val;
    z->nnz = static_cast<int32_t>(nk);
    call.commit();
    return NACHO_OK;
}

// ---- inner product through row offsets and (j, k) column keys -----------------------------
//
// A CSF3 tensor is a matrix with rows i and columns (j, k) in lexicographic order: its k
// entries in storage order are the row-major entries of that matrix.  When the j and k
// extents fit 31 bits together (key j << kbits | k below INT_MAX), the inner product is the
// level intersection of those two matrices, with no union of the i and j levels first.

struct CsfKeysJob {
    const int *ci, *pj, *cj, *pk, *ck;
    int ni, nj;
    int *pos;  // rows + 1 row offsets (into the k entries)
    int *key;  // nk column keys
};

// Row offsets of both operands: work item p in [0, ni] of an operand gives the rows in
// (ci[p - 1], ci[p]] (ci[-1] = -1, ci[ni] = rows) the k offset of i entry p's first fibre,
// pk[pj[p]] (nk for p = ni).  Items [0, na] are A's, the rest B's.
__global__ void csf_row_offsets_kernel(CsfKeysJob ja, CsfKeysJob jb, int rows) {
    const long long na = static_cast<long long>(ja.ni) + 1;
    const long long nb = static_cast<long long>(jb.ni) + 1;
    for (long long g = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
         g < na + nb; g += static_cast<long long>(gridDim.x) * blockDim.x) {
        const bool first = g < na;
        const int *__restrict__ ci = first ? ja.ci : jb.ci;
        const int *__restrict__ pj = first ? ja.pj : jb.pj;
        const int *__restrict__ pk = first ? ja.pk : jb.pk;
        int *__restrict__ pos = first ? ja.pos : jb.pos;
        const int ni = first ? ja.ni : jb.ni;
        const int p = static_cast<int>(first ? g : g - na);
        const int lo = p == 0 ? -1 : min(max(ci[p - 1], -1), rows);
        const int hi = p == ni ? rows : min(max(ci[p], -1), rows);
        const int at = pk[pj[p]];
        for (int r = lo + 1; r <= hi; ++r) pos[r] = at;
    }
}

// Column keys of both operands: cj[f] << kbits | ck[e] for every k entry e of fibre f.  One
// wavefront per group of 64 consecutive fibres (groups [0, ga) are A's, the rest B's): lane l
// holds fibre f0 + l's offset and j bits, and the wave strides over the group's k entries in
// windows of 64, consecutive lanes on consecutive entries.  An entry's fibre is the last one
// starting at or before it: a ballot counts the fibres starting at or before the window's
// first entry, and the fibres starting inside the window mark their start slot in LDS, so a
// running maximum over the lanes gives each entry the last fibre starting up to it.
//
// Measured alternatives at C5 (19.8M entries in 7.75M fibres per operand): one fibre per
// thread, 515 us; 256 fibres per wave staged in LDS, 164 us; one wave per 1024 entries
// (fibres of a Zipf-heavy i hold about 60 entries) with 1025 staged fibres, 232 us; each
// entry's fibre by a six-step search over the lanes' offsets (ds_bpermute), 148 us; this
// form, 103 us.
__global__ __launch_bounds__(256) void csf_keys_kernel(CsfKeysJob ja, CsfKeysJob jb, int ga,
                                                       int gb, int kbits) {
    constexpr int W = 64;
    __shared__ int s_mark[256 / W][W];  // per wave: the last fibre starting at each window slot
    const int lane = static_cast<int>(threadIdx.x) % W;
    int *mark = s_mark[threadIdx.x / W];
    const long long g = static_cast<long long>(blockIdx.x) * (blockDim.x / W) + threadIdx.x / W;
    if (g >= static_cast<long long>(ga) + gb) return;  // whole waves
    const bool first = g < ga;
    // the operand's fields as plain values (no addressable copy of either job)
    const int *__restrict__ pk = first ? ja.pk : jb.pk;
    const int *__restrict__ cj = first ? ja.cj : jb.cj;
    const int *__restrict__ ck = first ? ja.ck : jb.ck;
    int *__restrict__ key = first ? ja.key : jb.key;
    const int nj = first ? ja.nj : jb.nj;
    const int f0 = static_cast<int>((first ? g : g - ga) * W);
    const int nf = min(W, nj - f0);
    const int f = f0 + min(lane, nf - 1);
    const int start = pk[f];     // lane's fibre start (clamped)
    const int e1 = pk[f0 + nf];  // end of the group's entries
    const int jhi = cj[f] << kbits;
    const int e0 = __shfl(start, 0, W);
    const bool mine = lane < nf;
    mark[lane] = 0;
    dev::wave_sync();
    constexpr int U = 4;  // windows of W entries whose loads are issued together
    for (int base = e0; base < e1; base += U * W) {  // uniform
        int kv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) kv[u] = ck[min(base + u * W + lane, e1 - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // The fibre of entry wb + x is the last fibre starting at or before it: the
            // fibres starting at or before wb (a ballot), then the last one starting inside
            // the window up to x (marks by start slot, the largest fibre winning where
            // empty fibres share a start, and a running maximum over the lanes).
            const int wb = base + u * W;
            const int before = __popcll(__ballot(mine && start <= wb));
            const int d = start - wb;
            if (mine && d > 0 && d < W) atomicMax(&mark[d], lane + 1);
            dev::wave_sync();
            const int m = mark[lane];
            mark[lane] = 0;
            const int run = dev::wave_inclusive_max_dpp(m);
            const int fib = run > 0 ? run - 1 : before - 1;
            const int hi_bits = __shfl(jhi, fib, W);
            const int e = wb + lane;
            if (e < e1) key[e] = hi_bits | kv[u];
            dev::wave_sync();  // the marks are cleared before the next window's
        }
    }
}

// Bits of coordinates below `extent`.
static int extent_bits(int extent) {
    unsigned m = extent > 1 ? static_cast<unsigned>(extent - 1) : 0u;
    int bits = 0;
    while (m) {
        ++bits;
        m >>= 1;
    }
    return bits;
}

// Rows at most this many times the entries take the key path (its row offsets cost one
// write per row).
constexpr long long kKeyPathRowsPerEntry = 4;

// Inner product of two CSF3 tensors: Σ a·b over the (i, j, k) both hold.  When the (j, k)
// keys fit, both operands become rows i of column keys and one level intersection sums the
// products (csf_inner_by_keys).  Otherwise the i and j
// levels are merged as in csf_add (unions carrying child pointers, into scratch), so every
// (i, j) fibre of either operand becomes a row whose A and B ranges are its k entries (empty
// on the side that lacks it); the k level is the intersection of each row's ranges, whose
// products are summed (csr::LevelResult::dot) into the result's single value.
int csf_inner_prod(const nacho_csf3 *a, const nacho_csf3 *b, nacho_scalar *z, int32_t num_blocks,
                   int32_t threads_per_block, void *stream, const nacho_allocator *alloc) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_scalar{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_csf3(a) || bad_csf3(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size ||
        a->dim_k_size != b->dim_k_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const long long cap_i = static_cast<long long>(a->dim_i_length) + b->dim_i_length;
    const long long cap_j = static_cast<long long>(a->dim_j_length) + b->dim_j_length;
    const long long cap_k = static_cast<long long>(a->dim_k_length) + b->dim_k_length;
    if (cap_k + cap_j > static_cast<long long>(INT_MAX) - (1 << 16)) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }

    Call call(stream, alloc);
    const hipStream_t s = call.stream();
    float *value = nullptr;
    NACHO_TRY(call.result_n(1, &value));

    const int kbits = extent_bits(a->dim_k_size);
    const bool keys_fit = a->dim_j_size >= 1 && a->dim_k_size >= 1 &&
                          extent_bits(a->dim_j_size) + kbits <= 31 &&
                          ((static_cast<long long>(a->dim_j_size - 1) << kbits) |
                           (a->dim_k_size - 1)) < INT_MAX;
    const long long entries = static_cast<long long>(a->dim_k_length) + b->dim_k_length;
    if (keys_fit && a->dim_i_size <= kKeyPathRowsPerEntry * entries + (1 << 20) &&
        entries + a->dim_i_size <= static_cast<long long>(INT_MAX) - 2 * csr::kLevelTileSlack) {
        const int rows = a->dim_i_size;
        int *pa = nullptr, *pb = nullptr, *ka = nullptr, *kb = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pa));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(rows) + 1, &pb));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(a->dim_k_length, 1)), &ka));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(std::max(b->dim_k_length, 1)), &kb));
        const CsfKeysJob ja{a->dim_i_indices, a->dim_j_offsets, a->dim_j_indices,
                            a->dim_k_offsets, a->dim_k_indices, a->dim_i_length,
                            a->dim_j_length, pa, ka};
        const CsfKeysJob jb{b->dim_i_indices, b->dim_j_offsets, b->dim_j_indices,
                            b->dim_k_offsets, b->dim_k_indices, b->dim_i_length,
                            b->dim_j_length, pb, kb};
        NACHO_TRY(call.timer_start("inner_prod (row offsets + (j, k) keys)"));
        const long long row_items = static_cast<long long>(a->dim_i_length) + b->dim_i_length + 2;
        csf_row_offsets_kernel<<<static_cast<unsigned>(std::min<long long>(
                                     4096, (row_items + 255) / 256)),
                                 256, 0, s>>>(ja, jb, rows);
        NACHO_TRY_HIP(hipGetLastError());
        const int ga = (a->dim_j_length + 63) / 64, gb = (b->dim_j_length + 63) / 64;
        if (ga + gb > 0) {
            csf_keys_kernel<<<static_cast<unsigned>((ga + gb + 3) / 4), 256, 0, s>>>(
                ja, jb, ga, gb, kbits);
            NACHO_TRY_HIP(hipGetLastError());
        }
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.collect_timer());  // (kernel timing only) before the merge's interval
        const csr::LevelOperand A{pa, ka, a->values, a->dim_k_length, nullptr};
        const csr::LevelOperand B{pb, kb, b->values, b->dim_k_length, nullptr};
        csr::LevelResult Z{nullptr, nullptr, nullptr, nullptr, nullptr};
        Z.dot = value;
        long long unused = 0;
        NACHO_TRY(csr::merge_level(call, true, true, false, rows, A, B, Z, &unused,
                                   "inner_prod"));
        z->values = value;
        z->nnz = 1;
        call.commit();
        return NACHO_OK;
    }

    // i level: union of the root rows, child pointers into the j offsets
    int *root = nullptr, *root_out = nullptr, *ci_a = nullptr, *ci_b = nullptr, *crd_i = nullptr;
    NACHO_TRY(call.scratch_n(4, &root));
    NACHO_TRY(call.scratch_n(2, &root_out));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_b));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i), &crd_i));
    root_offsets_kernel<<<1, 64, 0, s>>>(root, a->dim_i_length, b->dim_i_length);
    NACHO_TRY_HIP(hipGetLastError());
    long long ni = 0;
    {
        const csr::LevelOperand A{root, a->dim_i_indices, nullptr, a->dim_i_length, a->dim_j_offsets};
        const csr::LevelOperand B{root + 2, b->dim_i_indices, nullptr, b->dim_i_length,
                                  b->dim_j_offsets};
        const csr::LevelResult Z{root_out, crd_i, nullptr, ci_a, ci_b};
        NACHO_TRY(csr::merge_level(call, false, false, true, 1, A, B, Z, &ni, "inner_prod"));
    }
    if (ni > cap_i) return NACHO_ERR_MALFORMED_INPUT;

    // j level: rows = union i fibres; child pointers into the k offsets
    int *pos_j = nullptr, *crd_j = nullptr, *cj_a = nullptr, *cj_b = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(ni) + 1, &pos_j));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_j), &crd_j));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_j) + 1, &cj_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_j) + 1, &cj_b));
    long long nj = 0;
    {
        const csr::LevelOperand A{ci_a, a->dim_j_indices, nullptr, a->dim_j_length, a->dim_k_offsets};
        const csr::LevelOperand B{ci_b, b->dim_j_indices, nullptr, b->dim_j_length, b->dim_k_offsets};
        const csr::LevelResult Z{pos_j, crd_j, nullptr, cj_a, cj_b};
        NACHO_TRY(csr::merge_level(call, false, false, true, static_cast<int>(ni), A, B, Z, &nj,
                                   "inner_prod"));
    }
    if (nj > cap_j) return NACHO_ERR_MALFORMED_INPUT;

    // k level: the intersection of every union (i, j) fibre's ranges, reduced to one value
    {
        const csr::LevelOperand A{cj_a, a->dim_k_indices, a->values, a->dim_k_length, nullptr};
        const csr::LevelOperand B{cj_b, b->dim_k_indices, b->values, b->dim_k_length, nullptr};
        csr::LevelResult Z{nullptr, nullptr, nullptr, nullptr, nullptr};
        Z.dot = value;
        long long unused = 0;
        NACHO_TRY(csr::merge_level(call, true, true, false, static_cast<int>(nj), A, B, Z,
                                   &unused, "inner_prod"));
    }
    z->values = value;
    z->nnz = 1;
    call.commit();
    return NACHO_OK;
}

}  // namespace csf
}  // namespace nacho

extern "C" int nacho_gpu_csf_add_f32(const nacho_csf3 *a, const nacho_csf3 *b, nacho_csf3 *z,
                                     int32_t num_blocks, int32_t threads_per_block, void *stream,
                                     const nacho_allocator *alloc) {
    return nacho::csf::csf_add(a, b, z, num_blocks, threads_per_block, stream, alloc);
}

extern "C" int nacho_gpu_inner_prod_f32(const nacho_csf3 *a, const nacho_csf3 *b, nacho_scalar *z,
                                        int32_t num_blocks, int32_t threads_per_block,
                                        void *stream, const nacho_allocator *alloc) {
    return nacho::csf::csf_inner_prod(a, b, z, num_blocks, threads_per_block, stream, alloc);
}
