// Declarations written against the reference's own API (include/Kernel.h, Frontend.h,
// Format.h), generated for the GPU target through the HIP backend's Kernel::emit
// (nacho_amd/codegen/reference_hook): a renamed sum with its operands reordered and its
// Python name overridden, a product over other index letters, and two forms without a HIP
// kernel (a broadcast that is not an operand of + or *, and a sum of operands over different
// indices).  Prints every refusal; exits 1 when a kernel named by --kernels is refused.
#include <iostream>

#include "Frontend.h"
#include "Kernel.h"
#include "backend/output.h"
#include "gpu_target.hpp"

using namespace nacho;

int main(int argc, char **argv) {
    if (!parse_command_line(argc, argv)) return 2;
    backend::reset_output_directory();
    try {
        const Format csr_xy = Format::ordered({Level("x", LevelFormat::Dense),
                                               Level("y", LevelFormat::Compressed_unique)})
                                  .named("CSR");
        const Format csr_yz = Format::ordered({Level("y", LevelFormat::Dense),
                                               Level("z", LevelFormat::Compressed_unique)})
                                  .named("CSR");
        const TensorType t_xy(csr_xy, dType::Float32), t_yz(csr_yz, dType::Float32);
        Expr p = Tensor::make(t_xy, "p"), q = Tensor::make(t_xy, "q");
        Expr r = Tensor::make(t_yz, "r");
        Kernel("plus_qp")
            .expr(p + q)
            .operand_ordering({"q", "p"})
            .python_name(Target::GPU, "gpu_plus_qp")
            .result_name("W")
            .emit();
        Kernel("times").expr(p * q).targets({Target::GPU}).emit();
        Kernel("cpu_only").expr(p * q).targets({Target::CPU}).emit();
        Kernel("broadcast").expr(bc("z", p)).targets({Target::GPU}).emit();
        Kernel("mixed_sum").expr(p + r).targets({Target::GPU}).emit();
    } catch (const nacho_hipgen::UnsupportedForm &e) {
        std::cout << "error: " << e.what() << "\n";
        return 1;
    }
    for (const auto &[name, reason] : nacho_hipgen::refused()) {
        std::cout << "refused " << name << ": " << reason << "\n";
    }
    return 0;
}
