// nacho_hip.hpp — the reference's generated C++ entry points, over the C ABI of nacho_hip.h.
//
// For every GPU kernel <k> the reference writes a header <k>_gpu.h holding
//
//     namespace <k> {
//     using index_t = int32_t;
//     using value_t = float;
//     template <typename index_t, typename value_t> struct a_tensor_format { ... };  // per operand
//     template <typename index_t, typename value_t> struct Z_tensor_format { ... };  // result
//     Z_tensor_format<index_t, value_t> <k>_gpu_i32_f32(const a_tensor_format<index_t, value_t> a,
//                                                      ..., const int32_t num_blocks,
//                                                      const int32_t threads_per_block);
//     }
//
// (namespace and type aliases: src/backend/stitch_and_generate.cpp:229-236; arguments and
// result type: stitch_and_generate.cpp:277-290; prototype: stitch_and_generate.cpp:296-301;
// struct name = tensor name + "_tensor_format": include/backend/tensor.h:141-143; result
// name "Z": include/Kernel.h:67; fields: sizes first, then level arrays in level order, then
// values and nnz, named after the tensor's index variables: src/backend/tensor.cpp:13-61).
//
// This header declares the same namespaces, struct templates and functions for every kernel
// the backend implements, so C++ written against a generated header (the reference's
// nanobind wrappers, generate_bindings.cpp:288-327) compiles against this one unchanged.
// Each function is inline and calls the matching nacho_gpu_<k>_f32.  Differences from the
// generated code:
//   * errors throw std::runtime_error carrying nacho_error_string() (the generated code
//     checks no CUDA call);
//   * results come from the library's caching allocator: release each non-null array with
//     nacho_free(ptr, stream) (the generated code uses cudaMallocAsync, and its bindings free
//     with cudaFreeWrapper, runtime/cuda_utils/cuda_utils.cu:7-11);
//   * work runs on nacho_hip::stream(), settable per thread with nacho_hip::set_stream();
//     the default is the null stream, the generated code's `stream = 0`.
// Only index_t = int32_t and value_t = float are instantiated, as in the reference.
#ifndef NACHO_HIP_HPP
#define NACHO_HIP_HPP

#include <cstdint>

#include "nacho_hip.h"
#include "nacho_hip_runtime.hpp"  // stream(), set_stream(), detail::to_c / from_c / check

namespace nacho_hip {

// ---- tensor formats ---------------------------------------------------------------------
// One template per (format, index variables) the declared kernels use
// (compiler.cpp:21-85): the field names follow the index variables, the field order is the
// generated one, and each layout equals the C descriptor of nacho_hip.h.

#define NACHO_HIP_CSR(NAME, I, J)                                                                \
    template <typename index_t, typename value_t>                                               \
    struct NAME {                                                                               \
        index_t dim_##I##_size;                                                                 \
        index_t dim_##J##_size;                                                                 \
        index_t *dim_##J##_offsets;                                                             \
        index_t dim_##J##_length;                                                               \
        index_t *dim_##J##_indices;                                                             \
        value_t *values;                                                                        \
        index_t nnz;                                                                            \
    };
NACHO_HIP_CSR(csr_ij, i, j)  // CSR over (i, j): csr_1
NACHO_HIP_CSR(csr_jk, j, k)  // CSR over (j, k): csr_2
NACHO_HIP_CSR(csr_ik, i, k)  // CSR over (i, k): csr_3
#undef NACHO_HIP_CSR

template <typename index_t, typename value_t>
struct dcsr_ij {  // DCSR over (i, j)
    index_t dim_i_size;
    index_t dim_j_size;
    index_t dim_i_length;
    index_t *dim_i_indices;
    index_t *dim_j_offsets;
    index_t dim_j_length;
    index_t *dim_j_indices;
    value_t *values;
    index_t nnz;
};

template <typename index_t, typename value_t>
struct csf3_ijk {  // CSF3 over (i, j, k)
    index_t dim_i_size;
    index_t dim_j_size;
    index_t dim_k_size;
    index_t dim_i_length;
    index_t *dim_i_indices;
    index_t *dim_j_offsets;
    index_t dim_j_length;
    index_t *dim_j_indices;
    index_t *dim_k_offsets;
    index_t dim_k_length;
    index_t *dim_k_indices;
    value_t *values;
    index_t nnz;
};

template <typename index_t, typename value_t>
struct coo_ij {  // COO over (i, j): one merged level
    index_t dim_i_size;
    index_t dim_j_size;
    index_t dim_i_length;
    index_t *dim_i_indices;
    index_t dim_j_length;
    index_t *dim_j_indices;
    value_t *values;
    index_t nnz;
};

template <typename index_t, typename value_t>
struct coo3_ijk {  // COO3 over (i, j, k): one merged level
    index_t dim_i_size;
    index_t dim_j_size;
    index_t dim_k_size;
    index_t dim_i_length;
    index_t *dim_i_indices;
    index_t dim_j_length;
    index_t *dim_j_indices;
    index_t dim_k_length;
    index_t *dim_k_indices;
    value_t *values;
    index_t nnz;
};

template <typename index_t, typename value_t>
struct scalar {  // Scalar (format {}): a full reduction's single value, no levels
    value_t *values;  // 1 entry
    index_t nnz;
};

namespace detail {

// a converts to CA, b to CB (default CA), the result from CZ
template <typename Z, typename CZ, typename CA, typename CB = CA, typename A, typename B,
          typename Fn>
inline Z call2(Fn fn, const char *kernel, const A &a, const B &b, int32_t num_blocks,
               int32_t threads_per_block) {
    const CA ca = to_c<CA>(a);
    const CB cb = to_c<CB>(b);
    CZ cz{};
    check(fn(&ca, &cb, &cz, num_blocks, threads_per_block, stream(), nullptr), kernel);
    return from_c<Z>(cz);
}

template <typename Z, typename CZ, typename CA, typename A, typename B, typename C, typename Fn>
inline Z call3(Fn fn, const char *kernel, const A &a, const B &b, const C &c,
               int32_t num_blocks, int32_t threads_per_block) {
    const CA ca = to_c<CA>(a), cb = to_c<CA>(b), cc = to_c<CA>(c);
    CZ cz{};
    check(fn(&ca, &cb, &cc, &cz, num_blocks, threads_per_block, stream(), nullptr), kernel);
    return from_c<Z>(cz);
}

}  // namespace detail
}  // namespace nacho_hip

// ---- the generated namespaces ------------------------------------------------------------

// Two operands a, b and a result Z; CA, CB and CZ are their C descriptors
// (compiler.cpp:112-148).
#define NACHO_HIP_BINARY(K, FA, FB, FZ, CA, CB, CZ)                                              \
    namespace K {                                                                               \
    using index_t = int32_t;                                                                    \
    using value_t = float;                                                                      \
    template <typename I, typename V>                                                           \
    using a_tensor_format = nacho_hip::FA<I, V>;                                                \
    template <typename I, typename V>                                                           \
    using b_tensor_format = nacho_hip::FB<I, V>;                                                \
    template <typename I, typename V>                                                           \
    using Z_tensor_format = nacho_hip::FZ<I, V>;                                                \
    inline Z_tensor_format<index_t, value_t> K##_gpu_i32_f32(                                   \
        const a_tensor_format<index_t, value_t> a, const b_tensor_format<index_t, value_t> b,   \
        const int32_t num_blocks, const int32_t threads_per_block) {                            \
        return nacho_hip::detail::call2<Z_tensor_format<index_t, value_t>, CZ, CA, CB>(         \
            nacho_gpu_##K##_f32, #K, a, b, num_blocks, threads_per_block);                      \
    }                                                                                           \
    }

#define NACHO_HIP_SAME(K, F, FZ, C, CZ) NACHO_HIP_BINARY(K, F, F, FZ, C, C, CZ)
NACHO_HIP_SAME(csr_add, csr_ij, csr_ij, nacho_csr, nacho_csr)                 // compiler.cpp:112
NACHO_HIP_SAME(csr_mul, csr_ij, csr_ij, nacho_csr, nacho_csr)                 // compiler.cpp:116
NACHO_HIP_SAME(coo_add, coo_ij, coo_ij, nacho_coo, nacho_coo)                 // compiler.cpp:118
NACHO_HIP_SAME(coo_mul, coo_ij, coo_ij, nacho_coo, nacho_coo)                 // compiler.cpp:120
NACHO_HIP_BINARY(coo_csr_add, csr_ij, coo_ij, csr_ij, nacho_csr, nacho_coo,
                 nacho_csr)                                                   // compiler.cpp:122
NACHO_HIP_SAME(dcsr_add, dcsr_ij, dcsr_ij, nacho_dcsr, nacho_dcsr)            // compiler.cpp:124
NACHO_HIP_SAME(dcsr_mul, dcsr_ij, dcsr_ij, nacho_dcsr, nacho_dcsr)            // compiler.cpp:126
NACHO_HIP_SAME(dcsr_mul_without_recursive_partitioning, dcsr_ij, dcsr_ij, nacho_dcsr,
               nacho_dcsr)                                                    // compiler.cpp:128-133
NACHO_HIP_SAME(csf_add, csf3_ijk, csf3_ijk, nacho_csf3, nacho_csf3)           // compiler.cpp:135
NACHO_HIP_SAME(coo3d_add, coo3_ijk, coo3_ijk, nacho_coo3, nacho_coo3)         // compiler.cpp:138
NACHO_HIP_SAME(inner_prod, csf3_ijk, scalar, nacho_csf3, nacho_scalar)        // compiler.cpp:141
NACHO_HIP_SAME(inner_prod_coo, coo3_ijk, scalar, nacho_coo3, nacho_scalar)    // compiler.cpp:143
NACHO_HIP_BINARY(spgemm, csr_ij, csr_jk, csr_ik, nacho_csr, nacho_csr,
                 nacho_csr)                                                   // compiler.cpp:145-148
#undef NACHO_HIP_SAME
#undef NACHO_HIP_BINARY

// Three operands a, b, c (compiler.cpp:114, 150-153).
#define NACHO_HIP_TERNARY(K, FA, FB, FC, FZ)                                                     \
    namespace K {                                                                               \
    using index_t = int32_t;                                                                    \
    using value_t = float;                                                                      \
    template <typename I, typename V>                                                           \
    using a_tensor_format = nacho_hip::FA<I, V>;                                                \
    template <typename I, typename V>                                                           \
    using b_tensor_format = nacho_hip::FB<I, V>;                                                \
    template <typename I, typename V>                                                           \
    using c_tensor_format = nacho_hip::FC<I, V>;                                                \
    template <typename I, typename V>                                                           \
    using Z_tensor_format = nacho_hip::FZ<I, V>;                                                \
    inline Z_tensor_format<index_t, value_t> K##_gpu_i32_f32(                                   \
        const a_tensor_format<index_t, value_t> a, const b_tensor_format<index_t, value_t> b,   \
        const c_tensor_format<index_t, value_t> c, const int32_t num_blocks,                    \
        const int32_t threads_per_block) {                                                      \
        return nacho_hip::detail::call3<Z_tensor_format<index_t, value_t>, nacho_csr,           \
                                        nacho_csr>(nacho_gpu_##K##_f32, #K, a, b, c,            \
                                                   num_blocks, threads_per_block);              \
    }                                                                                           \
    }

NACHO_HIP_TERNARY(csr_add_3, csr_ij, csr_ij, csr_ij, csr_ij)  // compiler.cpp:114
NACHO_HIP_TERNARY(sssmm, csr_ij, csr_jk, csr_ik, csr_ik)      // compiler.cpp:150-153
#undef NACHO_HIP_TERNARY

#endif  // NACHO_HIP_HPP
