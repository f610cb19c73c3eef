// Test double for the two headers a generated <k>_gpu_nb.cpp expects from the reference's
// build: nacho_types.h (the Python tensor classes its bindings generator writes) and the
// part of nanobind and runtime/nacho_nb.h those use.  It has just enough surface for the
// wrappers to compile on the host and be called from a test driver: module_::def keeps the
// function pointer, the arrays are (pointer, length) pairs.  Not used by the library.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <map>
#include <string>

namespace nb {
struct arg {
    explicit arg(const char *name) : name(name) {}
    template <typename T>
    arg &operator=(T) {
        return *this;
    }
    const char *name;
};

struct module_ {
    std::map<std::string, void *> functions;
    template <typename F, typename... Args>
    void def(const char *name, F *function, Args &&...) {
        functions[name] = reinterpret_cast<void *>(function);
    }
};
}  // namespace nb

namespace nacho {
template <typename T>
struct ArrayGPU {
    T *ptr = nullptr;
    size_t count = 0;
    T *data() const { return ptr; }
    size_t shape(size_t) const { return count; }
};

template <size_t Rank>
struct ShapeTuple {
    int32_t sizes[Rank];
    const int32_t *data() const { return sizes; }
};

template <typename T, typename Array>
T *borrow(const Array &array) {
    return const_cast<T *>(array.data());
}

template <typename T>
ArrayGPU<T> adopt_gpu(T *data, size_t count) {
    return ArrayGPU<T>{data, count};
}

template <size_t Rank>
ShapeTuple<Rank> make_shape(std::initializer_list<int32_t> sizes) {
    ShapeTuple<Rank> s{};
    size_t i = 0;
    for (int32_t x : sizes) s.sizes[i++] = x;
    return s;
}
}  // namespace nacho

// Class members as the reference's bindings generator names them: after the first tensor
// recorded for the class (generate_bindings.cpp:172-187), a result over (i, j[, k]).
struct CSR_gpu {
    nacho::ArrayGPU<int32_t> dim_j_offsets;
    nacho::ArrayGPU<int32_t> dim_j_indices;
    nacho::ArrayGPU<float> values;
    nacho::ShapeTuple<2> shape;
};

struct DCSR_gpu {
    nacho::ArrayGPU<int32_t> dim_i_indices;
    nacho::ArrayGPU<int32_t> dim_j_offsets;
    nacho::ArrayGPU<int32_t> dim_j_indices;
    nacho::ArrayGPU<float> values;
    nacho::ShapeTuple<2> shape;
};

struct CSF3_gpu {
    nacho::ArrayGPU<int32_t> dim_i_indices;
    nacho::ArrayGPU<int32_t> dim_j_offsets;
    nacho::ArrayGPU<int32_t> dim_j_indices;
    nacho::ArrayGPU<int32_t> dim_k_offsets;
    nacho::ArrayGPU<int32_t> dim_k_indices;
    nacho::ArrayGPU<float> values;
    nacho::ShapeTuple<3> shape;
};

struct COO_gpu {
    nacho::ArrayGPU<int32_t> dim_i_indices;
    nacho::ArrayGPU<int32_t> dim_j_indices;
    nacho::ArrayGPU<float> values;
    nacho::ShapeTuple<2> shape;
};

struct COO3_gpu {
    nacho::ArrayGPU<int32_t> dim_i_indices;
    nacho::ArrayGPU<int32_t> dim_j_indices;
    nacho::ArrayGPU<int32_t> dim_k_indices;
    nacho::ArrayGPU<float> values;
    nacho::ShapeTuple<3> shape;
};

// A full reduction's result: values only, no shape (generate_bindings.cpp:181-183).
struct Scalar_gpu {
    nacho::ArrayGPU<float> values;
};
