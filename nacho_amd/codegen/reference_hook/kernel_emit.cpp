// kernel_emit.cpp — the reference's declaration API (include/Kernel.h) with its GPU target on
// the HIP generator.
//
// Linking the reference's own declaration file (compiler.cpp) and its expression front end
// with this file gives a generator that writes the HIP backend's <k>_gpu.h / <k>_gpu_nb.cpp
// for every GPU declaration of that file, unchanged: Kernel(...).expr(...).targets(...)
// .emit() reaches emit_reference_gpu, which is what the GPU branch of the reference's
// Kernel::emit (src/Kernel.cpp:106-130) calls (gpu_target.hpp).  The CPU target stays the
// reference's own lowering and is not generated here.  Option handling, kernel selection and
// refusals are the HIP generator's (nacho_hipgen::parse_command_line, kernel_is_selected,
// refuse), and --output-dir also sets the reference's backend output directory, which
// compiler.cpp's main resets before the declarations run.
#include <algorithm>
#include <utility>

#include "Kernel.h"
#include "backend/output.h"
#include "gpu_target.hpp"

namespace nacho {

const char *target_tag(Target target) { return target == Target::GPU ? "gpu" : "cpu"; }

void set_selected_kernels(std::vector<std::string> names) {
    nacho_hipgen::set_selected_kernels(std::move(names));
}

bool kernel_is_selected(const std::string &name) { return nacho_hipgen::kernel_is_selected(name); }

bool parse_command_line(int argc, char **argv) {
    if (!nacho_hipgen::parse_command_line(argc, argv)) return false;
    backend::set_output_directory(nacho_hipgen::output_directory());
    return true;
}

Kernel::Kernel(std::string name) : name_(std::move(name)) {
    if (name_.empty()) throw std::invalid_argument("Kernel name cannot be empty");
}

Kernel &Kernel::expr(Expr expression) {
    expr_ = std::move(expression);
    return *this;
}

Kernel &Kernel::targets(std::vector<Target> targets) {
    targets_ = std::move(targets);
    return *this;
}

Kernel &Kernel::result_name(std::string name) {
    result_name_ = std::move(name);
    return *this;
}

Kernel &Kernel::operand_ordering(std::vector<std::string> names) {
    operand_ordering_ = std::move(names);
    return *this;
}

Kernel &Kernel::python_name(Target target, std::string name) {
    python_names_.emplace_back(target, std::move(name));
    return *this;
}

Kernel &Kernel::bindings(bool enabled) {
    bindings_ = enabled;
    return *this;
}

Kernel &Kernel::recursive_partitioning(bool enabled) {
    recursive_partitioning_ = enabled;
    return *this;
}

std::string Kernel::python_name_for(Target target) const {
    std::string chosen = std::string(target_tag(target)) + "_" + name_ + "_f32";
    for (const auto &[t, n] : python_names_) {
        if (t == target) chosen = n;
    }
    return chosen;
}

void Kernel::emit() {
    if (!kernel_is_selected(name_)) return;
    if (std::find(targets_.begin(), targets_.end(), Target::GPU) == targets_.end()) return;
    try {
        nacho_hipgen::emit_reference_gpu(name_, expr_, result_name_, operand_ordering_,
                                         python_name_for(Target::GPU), recursive_partitioning_,
                                         bindings_, backend::output_directory());
    } catch (const nacho_hipgen::UnsupportedForm &err) {
        nacho_hipgen::refuse(name_, err.what());
    }
}

}  // namespace nacho
