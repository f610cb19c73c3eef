// Input validation on the device: checks a CSR operand against the input contract that the
// merge kernels assume (and that the reference's generated code assumes without checking):
// pos[0] == 0, pos non-decreasing, pos[rows] == length, 0 <= crd < columns, crd strictly
// increasing within each row.
//
// Three small kernels over scratch memory: clear the row-start flags and the error word,
// check every row's offsets and flag where each row starts, then check every coordinate
// against the next one unless a row starts between them.  Offsets outside [0, length] are
// reported, never used as an index.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "runtime.hpp"

namespace nacho {
namespace validate {

constexpr int kBlock = 256;

enum : unsigned {
    kBadFirst = 1u,       // pos[0] != 0
    kBadLast = 2u,        // pos[rows] != length
    kDecreasing = 4u,     // pos[r] > pos[r + 1], or an offset outside [0, length]
    kColumnRange = 8u,    // a coordinate outside [0, columns)
    kUnsorted = 16u,      // coordinates not strictly increasing within a row
};

__global__ void clear_kernel(unsigned char *__restrict__ starts, int64_t n,
                             unsigned *__restrict__ err) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i == 0) *err = 0u;
    for (int64_t x = i; x < n; x += static_cast<int64_t>(gridDim.x) * blockDim.x) starts[x] = 0;
}

__global__ void rows_kernel(const int *__restrict__ pos, int rows, int length,
                            unsigned char *__restrict__ starts, unsigned *__restrict__ err) {
    for (int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; r <= rows;
         r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int p = pos[r];
        unsigned bad = 0u;
        if (r == 0 && p != 0) bad |= kBadFirst;
        if (r == rows && p != length) bad |= kBadLast;
        if (p < 0 || p > length) {
            bad |= kDecreasing;
        } else {
            starts[p] = 1;  // a row (or several empty ones) starts at p
        }
        if (r < rows && p > pos[r + 1]) bad |= kDecreasing;
        if (bad) atomicOr(err, bad);
    }
}

__global__ void entries_kernel(const int *__restrict__ crd, int length, int columns,
                               const unsigned char *__restrict__ starts,
                               unsigned *__restrict__ err) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < length;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int c = crd[e];
        unsigned bad = 0u;
        if (c < 0 || c >= columns) bad |= kColumnRange;
        if (e + 1 < length && !starts[e + 1] && c >= crd[e + 1]) bad |= kUnsorted;
        if (bad) atomicOr(err, bad);
    }
}

unsigned grid_for(int64_t n) {
    const int64_t g = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

int validate_csr(const nacho_csr *t, void *stream) {
    if (!t || t->dim_i_size < 0 || t->dim_j_size < 0 || t->dim_j_length < 0) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    if (!t->dim_j_offsets || (t->dim_j_length > 0 && !t->dim_j_indices)) {
        return NACHO_ERR_INVALID_ARGUMENT;
    }
    if (t->nnz != t->dim_j_length) return NACHO_ERR_INVALID_ARGUMENT;
    Call call(stream, nullptr);
    const int64_t n = static_cast<int64_t>(t->dim_j_length) + 1;
    unsigned char *starts = nullptr;
    unsigned *err = nullptr;
    NACHO_TRY(call.scratch_n(static_cast<size_t>(n), &starts));
    NACHO_TRY(call.scratch_n(1, &err));
    const hipStream_t s = call.stream();
    clear_kernel<<<grid_for(n), kBlock, 0, s>>>(starts, n, err);
    rows_kernel<<<grid_for(static_cast<int64_t>(t->dim_i_size) + 1), kBlock, 0, s>>>(
        t->dim_j_offsets, t->dim_i_size, t->dim_j_length, starts, err);
    if (t->dim_j_length > 0) {
        entries_kernel<<<grid_for(t->dim_j_length), kBlock, 0, s>>>(
            t->dim_j_indices, t->dim_j_length, t->dim_j_size, starts, err);
    }
    NACHO_TRY_HIP(hipGetLastError());
    unsigned bad = 0u;
    NACHO_TRY(call.read_back(&bad, err, sizeof(bad)));
    return bad ? NACHO_ERR_MALFORMED_INPUT : NACHO_OK;
}

}  // namespace validate
}  // namespace nacho

extern "C" int nacho_validate_csr(const nacho_csr *t, void *stream) {
    return nacho::validate::validate_csr(t, stream);
}
