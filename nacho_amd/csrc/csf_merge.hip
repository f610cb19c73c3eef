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
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "csr_merge.hpp"
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

// Inner product of two CSF3 tensors: Σ a·b over the (i, j, k) both hold.  The i and j
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
