// DCSR elementwise add (union at both levels) and multiply (intersection at both levels) for
// gfx950.
//
// Reference path replaced: dcsr_add, dcsr_mul and dcsr_mul_without_recursive_partitioning
// (compiler.cpp:124-133).  Their generated kernels partition the two compressed levels
// (partition.cpp:286-461; dcsr_mul re-partitions at the inner intersection) and emit the i
// and j levels with one count/scan/readback per level (stitch_and_generate_gpu.cpp:641-715).
// Both levels are CSR level merges here (csr_merge.hip):
//   add: i level = one "row" holding both operands' row coordinates; each output row records
//        the operands' j offsets reached (child pointers), which are the j level's row
//        offsets; the j level is a CSR add over those rows.
//   mul: the i level is merged as a union whose child pointers are operand positions; the j
//        level is a CSR multiply over the union rows (a row present in one operand only has
//        an empty range on the other side and yields nothing); a compaction then keeps the
//        rows present in both operands.  The i level of the result is therefore the
//        intersection of the operands' row coordinates, and a row whose j intersection is
//        empty is kept with an empty fibre: the generated code counts an output i coordinate
//        at every i lattice point where both operands are present, before and independently
//        of the j level (compute.cpp:945-990).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "csr_merge.hpp"
#include "device_utils.hpp"
#include "runtime.hpp"
#include "scan.hpp"

namespace nacho {
namespace dcsr {

constexpr int kBlock = 256;

// Offsets of the virtual root "row" of each operand's i level: {0, ni_a, 0, ni_b}.
__global__ void root_offsets_kernel(int *root, int ni_a, int ni_b) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        root[0] = 0;
        root[1] = ni_a;
        root[2] = 0;
        root[3] = ni_b;
    }
}

// For union row o in [0, n]: the operands' j offsets at the positions reached (ca/cb are
// positions into the operands' i levels, n + 1 entries each).
__global__ void row_offsets_kernel(const int *__restrict__ ca, const int *__restrict__ cb,
                                   const int *__restrict__ pos_a, const int *__restrict__ pos_b,
                                   int n, int *__restrict__ ja, int *__restrict__ jb) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o > n) return;
    ja[o] = pos_a[ca[o]];
    jb[o] = pos_b[cb[o]];
}

// keep[o] = 1 when union row o is present in both operands.
__global__ void both_present_kernel(const int *__restrict__ ca, const int *__restrict__ cb,
                                    int n, int64_t *__restrict__ keep) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= n) return;
    keep[o] = (ca[o + 1] > ca[o] && cb[o + 1] > cb[o]) ? 1 : 0;
}

// Compacts the kept union rows: row coordinates and j offsets.  Rows that are not kept have
// empty j ranges, so a kept row's range [pos_u[o], pos_u[o + 1]) ends where the next kept
// row's begins and the final offset is pos_u[n].
__global__ void compact_rows_kernel(const int64_t *__restrict__ keep_off,
                                    const int *__restrict__ crd_u, const int *__restrict__ pos_u,
                                    int n, int *__restrict__ crd_i, int *__restrict__ pos_j) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o > n) return;
    const int k = static_cast<int>(keep_off[o]);
    if (o == n) {
        pos_j[k] = pos_u[n];
    } else if (keep_off[o + 1] > keep_off[o]) {
        crd_i[k] = crd_u[o];
        pos_j[k] = pos_u[o];
    }
}

// *dst = *src (a count computed on the device, into the call's side word, which the host
// reads from pinned memory while the stream runs on).
__global__ void store_count_kernel(const int64_t *__restrict__ src, int64_t *__restrict__ dst) {
    if (threadIdx.x == 0 && blockIdx.x == 0) dev::store_system(dst, *src);
}

static unsigned grid_for(long long n) {
    return static_cast<unsigned>((n + kBlock - 1) / kBlock > 0 ? (n + kBlock - 1) / kBlock : 1);
}

bool bad_dcsr(const nacho_dcsr *t) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0) return true;
    if (t->dim_i_length < 0 || t->dim_j_length < 0 || t->nnz != t->dim_j_length) return true;
    if (!t->dim_j_offsets) return true;
    if (t->dim_i_length > 0 && !t->dim_i_indices) return true;
    if (t->dim_j_length > 0 && (!t->dim_j_indices || !t->values)) return true;
    return false;
}

int dcsr_binary(bool intersect, const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z,
                int32_t num_blocks, int32_t threads_per_block, void *stream,
                const nacho_allocator *alloc, const char *name) {
    if (!z) return NACHO_ERR_INVALID_ARGUMENT;
    *z = nacho_dcsr{};
    NACHO_TRY(check_launch_hints(num_blocks, threads_per_block));
    if (bad_dcsr(a) || bad_dcsr(b)) return NACHO_ERR_INVALID_ARGUMENT;
    if (a->dim_i_size != b->dim_i_size || a->dim_j_size != b->dim_j_size) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    const long long cap_i = static_cast<long long>(a->dim_i_length) + b->dim_i_length;
    const long long nnz_a = a->dim_j_length, nnz_b = b->dim_j_length;
    if (cap_i + nnz_a + nnz_b > static_cast<long long>(INT_MAX) - (1 << 16)) {
        return NACHO_ERR_INDEX_OVERFLOW;
    }
    const long long cap_j = intersect ? (nnz_a < nnz_b ? nnz_a : nnz_b) : nnz_a + nnz_b;

    Call call(stream, alloc);
    const hipStream_t s = call.stream();

    // i level: union of the row coordinates; child pointers are j offsets (add) or operand
    // positions (mul)
    int *root = nullptr, *root_out = nullptr, *ci_a = nullptr, *ci_b = nullptr, *crd_u = nullptr;
    NACHO_TRY(call.scratch_n(4, &root));
    NACHO_TRY(call.scratch_n(2, &root_out));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_a));
    NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i) + 1, &ci_b));
    if (intersect) {
        NACHO_TRY(call.scratch_n(static_cast<size_t>(cap_i), &crd_u));
    } else {
        NACHO_TRY(call.result_n(static_cast<size_t>(cap_i), &crd_u));
    }
    root_offsets_kernel<<<1, 64, 0, s>>>(root, a->dim_i_length, b->dim_i_length);
    NACHO_TRY_HIP(hipGetLastError());
    long long nu = 0;
    {
        const csr::LevelOperand A{root, a->dim_i_indices, nullptr, a->dim_i_length,
                                  intersect ? nullptr : a->dim_j_offsets};
        const csr::LevelOperand B{root + 2, b->dim_i_indices, nullptr, b->dim_i_length,
                                  intersect ? nullptr : b->dim_j_offsets};
        const csr::LevelResult Z{root_out, crd_u, nullptr, ci_a, ci_b};
        NACHO_TRY(csr::merge_level(call, false, false, true, 1, A, B, Z, &nu, name));
    }
    if (nu > cap_i) return NACHO_ERR_MALFORMED_INPUT;

    // j-level row offsets over the union rows; for a multiply, also the rows kept (present in
    // both operands), whose count goes to the side word while the j level runs
    const int *ja = ci_a, *jb = ci_b;
    int64_t *keep_off = nullptr;
    if (intersect) {
        int *ra = nullptr, *rb = nullptr;
        int64_t *keep = nullptr, *kept_dev = nullptr;
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nu) + 1, &ra));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nu) + 1, &rb));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nu) + 1, &keep));
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nu) + 1, &keep_off));
        NACHO_TRY(call.side_word(&kept_dev));
        NACHO_TRY(call.timer_start(name));
        row_offsets_kernel<<<grid_for(nu + 1), kBlock, 0, s>>>(
            ci_a, ci_b, a->dim_j_offsets, b->dim_j_offsets, static_cast<int>(nu), ra, rb);
        NACHO_TRY_HIP(hipGetLastError());
        if (nu > 0) {
            both_present_kernel<<<grid_for(nu), kBlock, 0, s>>>(ci_a, ci_b, static_cast<int>(nu),
                                                                 keep);
            NACHO_TRY_HIP(hipGetLastError());
        }
        NACHO_TRY(scan::exclusive_scan_i64(call, keep, nu, keep_off));
        store_count_kernel<<<1, 64, 0, s>>>(keep_off + nu, kept_dev);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        NACHO_TRY(call.collect_timer());  // (kernel timing only) before the j level's interval
        ja = ra;
        jb = rb;
    }

    // j level
    int *pos_u = nullptr, *crd_j = nullptr;
    float *val = nullptr;
    if (intersect) {
        NACHO_TRY(call.scratch_n(static_cast<size_t>(nu) + 1, &pos_u));
    } else {
        NACHO_TRY(call.result_n(static_cast<size_t>(nu) + 1, &pos_u));
    }
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_j), &crd_j));
    NACHO_TRY(call.result_n(static_cast<size_t>(cap_j), &val));
    long long nj = 0;
    bool nj_pending = false;  // multiply: the length is read after the rows are queued
    {
        const csr::LevelOperand A{ja, a->dim_j_indices, a->values, a->dim_j_length, nullptr};
        const csr::LevelOperand B{jb, b->dim_j_indices, b->values, b->dim_j_length, nullptr};
        const csr::LevelResult Z{pos_u, crd_j, val, nullptr, nullptr};
        NACHO_TRY(csr::merge_level(call, intersect, true, false, static_cast<int>(nu), A, B, Z,
                                   &nj, name, csr::UnionCount::kAuto,
                                   intersect ? &nj_pending : nullptr));
    }

    // rows of the result
    int *crd_i = crd_u, *pos_j = pos_u;
    long long ni = nu;
    if (intersect) {
        // The kept rows are compacted into arrays sized for all nu rows, so nothing waits for
        // their count; it and the j level's length are read once the j level's write pass has
        // ended, while its compaction and this one may still run (stream-ordered).
        NACHO_TRY(call.collect_timer());  // (kernel timing only) the j level's interval
        NACHO_TRY(call.result_n(static_cast<size_t>(nu), &crd_i));
        NACHO_TRY(call.result_n(static_cast<size_t>(nu) + 1, &pos_j));
        NACHO_TRY(call.timer_start(name));
        compact_rows_kernel<<<grid_for(nu + 1), kBlock, 0, s>>>(keep_off, crd_u, pos_u,
                                                                static_cast<int>(nu), crd_i,
                                                                pos_j);
        NACHO_TRY_HIP(hipGetLastError());
        NACHO_TRY(call.timer_stop());
        if (nj_pending) {
            int64_t len = 0;
            NACHO_TRY(call.wait_length(&len));
            nj = len;
        }
        int64_t kept = 0;
        NACHO_TRY(call.side_value(&kept));
        ni = kept;
        NACHO_TRY(call.collect_timer());
    }
    if (nj > cap_j || ni > nu) return NACHO_ERR_MALFORMED_INPUT;
    if (ni == 0 && crd_i) {
        call.drop_result(crd_i);
        crd_i = nullptr;
    }
    if (nj == 0) {
        call.drop_result(crd_j);
        call.drop_result(val);
        crd_j = nullptr;
        val = nullptr;
    }
    z->dim_i_size = a->dim_i_size;
    z->dim_j_size = a->dim_j_size;
    z->dim_i_length = static_cast<int32_t>(ni);
    z->dim_i_indices = crd_i;
    z->dim_j_offsets = pos_j;
    z->dim_j_length = static_cast<int32_t>(nj);
    z->dim_j_indices = crd_j;
    z->values = val;
    z->nnz = static_cast<int32_t>(nj);
    call.commit();
    return NACHO_OK;
}

}  // namespace dcsr
}  // namespace nacho

extern "C" {

int nacho_gpu_dcsr_add_f32(const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc) {
    return nacho::dcsr::dcsr_binary(false, a, b, z, num_blocks, threads_per_block, stream,
                                    alloc, "dcsr_add");
}

int nacho_gpu_dcsr_mul_f32(const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z,
                           int32_t num_blocks, int32_t threads_per_block, void *stream,
                           const nacho_allocator *alloc) {
    return nacho::dcsr::dcsr_binary(true, a, b, z, num_blocks, threads_per_block, stream, alloc,
                                    "dcsr_mul");
}

int nacho_gpu_dcsr_mul_without_recursive_partitioning_f32(
    const nacho_dcsr *a, const nacho_dcsr *b, nacho_dcsr *z, int32_t num_blocks,
    int32_t threads_per_block, void *stream, const nacho_allocator *alloc) {
    return nacho::dcsr::dcsr_binary(true, a, b, z, num_blocks, threads_per_block, stream, alloc,
                                    "dcsr_mul");
}

}  // extern "C"
