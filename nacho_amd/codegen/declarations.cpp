// declarations.cpp — nacho_hipgen's command line: the reference's kernel declarations
// (compiler.cpp:16-156), generated for the GPU target by the HIP generator.
//
//   nacho_hipgen [--kernels name[,name...]] [--output-dir DIR]
//
// Every declaration whose form the HIP library implements gets <k>_gpu.h and
// <k>_gpu_nb.cpp in DIR (default: generated).  The others are listed on stderr as not
// generated; naming one of them with --kernels is an error (exit status 1).
#include <iostream>

#include "hipgen.hpp"

using namespace nacho_hipgen;

static void declare() {
    // Formats of compiler.cpp:21-85 (names become the Python class names).
    Format csr_1 = Format::ordered({{"i", LevelFormat::Dense},
                                    {"j", LevelFormat::Compressed_unique}}).named("CSR");
    Format csr_2 = Format::ordered({{"j", LevelFormat::Dense},
                                    {"k", LevelFormat::Compressed_unique}}).named("CSR");
    Format csr_3 = Format::ordered({{"i", LevelFormat::Dense},
                                    {"k", LevelFormat::Compressed_unique}}).named("CSR");
    Format dcsr = Format::ordered({{"i", LevelFormat::Compressed_unique},
                                   {"j", LevelFormat::Compressed_unique}}).named("DCSR");
    Format csf = Format::ordered({{"i", LevelFormat::Compressed_unique},
                                  {"j", LevelFormat::Compressed_unique},
                                  {"k", LevelFormat::Compressed_unique}}).named("CSF3");
    Format coo = Format::ordered({{"i", LevelFormat::Compressed_non_unique},
                                  {"j", LevelFormat::Singleton_unique}}).named("COO");
    Format coo3d = Format::ordered({{"i", LevelFormat::Compressed_non_unique},
                                    {"j", LevelFormat::Singleton_non_unique},
                                    {"k", LevelFormat::Singleton_unique}}).named("COO3");

    const TensorType csr_f32(csr_1, dType::Float32), csr2_f32(csr_2, dType::Float32),
        csr3_f32(csr_3, dType::Float32), dcsr_f32(dcsr, dType::Float32),
        csf_f32(csf, dType::Float32), coo_f32(coo, dType::Float32),
        coo3d_f32(coo3d, dType::Float32);

    Expr a_csr_ij = Tensor::make(csr_f32, "a"), b_csr_ij = Tensor::make(csr_f32, "b"),
         c_csr_ij = Tensor::make(csr_f32, "c");
    Expr a_dcsr_ij = Tensor::make(dcsr_f32, "a"), b_dcsr_ij = Tensor::make(dcsr_f32, "b");
    Expr b_csr_jk = Tensor::make(csr2_f32, "b");
    Expr a_csf_ijk = Tensor::make(csf_f32, "a"), b_csf_ijk = Tensor::make(csf_f32, "b");
    Expr a_coo_ij = Tensor::make(coo_f32, "a"), b_coo_ij = Tensor::make(coo_f32, "b");
    Expr a_coo_ijk = Tensor::make(coo3d_f32, "a"), b_coo_ijk = Tensor::make(coo3d_f32, "b");
    Expr c_csr_ik = Tensor::make(csr3_f32, "c");

    // element-wise (compiler.cpp:110-138)
    Kernel("csr_add").expr(a_csr_ij + b_csr_ij).emit();
    Kernel("csr_add_3").expr(a_csr_ij + b_csr_ij + c_csr_ij).emit();
    Kernel("csr_mul").expr(a_csr_ij * b_csr_ij).emit();
    Kernel("coo_add").expr(a_coo_ij + b_coo_ij).emit();
    Kernel("coo_mul").expr(a_coo_ij * b_coo_ij).emit();
    Kernel("coo_csr_add").expr(a_csr_ij + b_coo_ij).emit();
    Kernel("dcsr_add").expr(a_dcsr_ij + b_dcsr_ij).emit();
    Kernel("dcsr_mul").expr(a_dcsr_ij * b_dcsr_ij).emit();
    Kernel("dcsr_mul_without_recursive_partitioning")
        .expr(a_dcsr_ij * b_dcsr_ij)
        .recursive_partitioning(false)
        .emit();
    Kernel("csf_add").expr(a_csf_ijk + b_csf_ijk).emit();
    Kernel("coo3d_add").expr(a_coo_ijk + b_coo_ijk).emit();

    // reductions (compiler.cpp:140-153)
    Kernel("inner_prod").expr(Sum::make("i", Sum::make("j", Sum::make("k", a_csf_ijk * b_csf_ijk)))).emit();
    Kernel("inner_prod_coo").expr(Sum::make("i", Sum::make("j", Sum::make("k", a_coo_ijk * b_coo_ijk)))).emit();
    Kernel("spgemm").expr(Sum::make("j", a_csr_ij * b_csr_jk)).targets({Target::GPU}).emit();
    Kernel("sssmm")
        .expr(Sum::make("j", a_csr_ij * b_csr_jk * c_csr_ik))
        .targets({Target::GPU})
        .emit();
}

int main(int argc, char **argv) {
    if (!parse_command_line(argc, argv)) return 1;
    try {
        declare();
    } catch (const UnsupportedForm &e) {
        std::cerr << "nacho_hipgen: " << e.what() << "\n";
        return 1;
    } catch (const std::exception &e) {
        std::cerr << "nacho_hipgen: error: " << e.what() << "\n";
        return 1;
    }
    for (const Emitted &e : emitted()) {
        std::cout << "generated " << e.header << (e.wrapper.empty() ? "" : " " + e.wrapper)
                  << " -> " << e.entry_point << "\n";
    }
    for (const auto &[name, reason] : refused()) {
        std::cerr << "not generated for the GPU target: " << reason << "\n";
    }
    return 0;
}
