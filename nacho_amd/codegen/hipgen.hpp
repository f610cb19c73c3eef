// hipgen.hpp — the HIP code generator for nacho's GPU target.
//
// nacho declares each kernel as a tensor expression over formatted operands and generates
// its code per target (compiler.cpp:16-156; Kernel::emit, src/Kernel.cpp:106-130).  For the
// GPU target the reference lowers the expression to CUDA through StitchAndGenerateGPU
// (src/backend/compile.cpp:83-87, include/backend/stitch_and_generate.h:150-236).  This
// generator takes its place for the expression forms the HIP library implements: it reads
// the declaration, picks the library entry point whose semantics match (by the operands'
// formats, the index pattern and the operator, not by the kernel's name), and writes
//
//   <k>_gpu.h       namespace <k> with the generated struct templates and
//                   <k>_gpu_i32_f32(...), an inline call of the C ABI (include/nacho_hip.h);
//   <k>_gpu_nb.cpp  the nanobind wrapper gpu_<k>_f32 and register_<k>_gpu, calling the C ABI
//                   directly (unwrap the Python classes into C descriptors, adopt the result
//                   buffers), compiled as plain C++ and linked with -lnacho_hip.
//
// A declaration of any other form has no HIP kernel behind it and is refused at generation
// time with UnsupportedForm (nothing is written for it).
//
// The front end below keeps the reference's declaration vocabulary (Format::ordered,
// LevelFormat, TensorType, Tensor::make, Sum::make, + and *, Kernel(...).expr().emit(),
// --kernels / --output-dir; include/Kernel.h:10-95), so the declarations of compiler.cpp
// read the same against it.
#pragma once

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace nacho_hipgen {

// ---- formats ----------------------------------------------------------------------------

// The reference's level formats in its order (include/Format.h:14-21), without
// MergedCoordinate, which only its lowering creates.
enum class LevelFormat {
    Dense,
    Compressed_non_unique,
    Compressed_unique,
    Singleton_non_unique,
    Singleton_unique,
};

struct Level {
    std::string index;
    LevelFormat format;
};

class Format {
public:
    static Format ordered(std::vector<Level> levels);
    Format named(std::string name) const;

    const std::vector<Level> &levels() const { return levels_; }
    const std::string &name() const { return name_; }

private:
    std::vector<Level> levels_;
    std::string name_;
};

enum class dType { Float32, Float64 };

struct TensorType {
    TensorType(Format format, dType dtype) : format(std::move(format)), dtype(dtype) {}
    Format format;
    dType dtype;
};

// ---- expressions ------------------------------------------------------------------------

struct ExprNode;

class Expr {
public:
    Expr() = default;
    explicit Expr(std::shared_ptr<const ExprNode> node) : node_(std::move(node)) {}
    const ExprNode *get() const { return node_.get(); }
    bool defined() const { return node_ != nullptr; }

private:
    std::shared_ptr<const ExprNode> node_;
};

struct ExprNode {
    enum class Kind { Tensor, Add, Mul, Sum };
    Kind kind;
    std::string name;                 // tensor name (Tensor) or summed index (Sum)
    std::shared_ptr<TensorType> type; // Tensor only
    Expr lhs, rhs;                    // Add, Mul; Sum keeps its body in lhs
};

struct Tensor {
    static Expr make(const TensorType &type, const std::string &name);
};

struct Sum {
    static Expr make(const std::string &index, Expr body);
};

Expr operator+(const Expr &a, const Expr &b);
Expr operator*(const Expr &a, const Expr &b);

// ---- what the generator reads from a declaration ----------------------------------------

struct Operand {
    std::string name;
    TensorType type;
};

enum class Form {
    Add,            // elementwise sum of the operands
    Mul,            // elementwise product of the operands
    SumOfProducts,  // Sum over one index of a product of the operands
    FullReduction,  // nested Sums over several indices of a product of the operands
};

struct Declaration {
    std::string kernel;
    Form form = Form::Add;
    std::vector<Operand> operands;       // in the expression's order
    std::vector<std::string> ordering;   // parameter order of the entry point
    std::string reduced_index;           // SumOfProducts only
    std::vector<std::string> reduced_indices;  // FullReduction: the summed indices, outer first
    std::string result_name = "Z";
    std::string python_name;             // default gpu_<kernel>_f32
    bool recursive_partitioning = true;
};

// A declaration whose form the HIP library does not implement.
class UnsupportedForm : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

// Flattens an expression into a Declaration (operands, form, reduced index).  Throws
// UnsupportedForm for a mix of + and *, nested or multiple sums, and the like.
Declaration analyse(const std::string &kernel, const Expr &expression);

// The library entry point a declaration maps to and the formats it fixes.
struct Plan {
    std::string entry_point;        // e.g. nacho_gpu_csr_add_f32
    std::string descriptor;         // C descriptor type of the operands, e.g. nacho_csr
    std::map<std::string, std::string> operand_descriptor;  // per operand, when they differ
    std::string result_descriptor;  // C descriptor type of the result
    std::vector<std::string> roles; // operand names in the entry point's argument order
    Format result_format;           // the result's levels (index names from the operands)
    std::string result_class;       // Python class of the result, e.g. CSR_gpu
};

// Throws UnsupportedForm, with the reason, when no entry point implements the declaration.
Plan plan(const Declaration &declaration);

struct Emitted {
    std::string header;   // path of <k>_gpu.h
    std::string wrapper;  // path of <k>_gpu_nb.cpp
    std::string entry_point;
};

// Writes <k>_gpu.h and <k>_gpu_nb.cpp into `output_dir` (which must exist).  Python class
// member names are kept per session as the reference's bindings generator keeps them: the
// first tensor of a class fixes its member names (generate_bindings.cpp:84-170, 172-187).
Emitted emit_gpu(const Declaration &declaration, const std::string &output_dir);

// Forgets the Python classes recorded by earlier emit_gpu calls.
void reset_classes();

// emit_gpu into `output_dir` (created if missing), without the wrapper unless `bindings`,
// recorded in emitted().
Emitted emit_declaration(const Declaration &declaration, bool bindings,
                         const std::string &output_dir);

// Records `kernel` as not generated, with `reason`, in refused(); throws UnsupportedForm when
// the kernel was named by --kernels (a default run lists it and goes on).
void refuse(const std::string &kernel, const std::string &reason);

// ---- the reference's Kernel builder ------------------------------------------------------

enum class Target { CPU, GPU };

class Kernel {
public:
    explicit Kernel(std::string name);
    Kernel &expr(Expr expression);
    Kernel &targets(std::vector<Target> targets);
    Kernel &result_name(std::string name);
    Kernel &operand_ordering(std::vector<std::string> names);
    Kernel &python_name(Target target, std::string name);
    Kernel &bindings(bool enabled);
    Kernel &recursive_partitioning(bool enabled);

    // Generates the GPU target into output_directory() when the kernel is selected and
    // lists GPU among its targets.  The CPU target is not this generator's: a declaration
    // for the CPU alone generates nothing here.  An unsupported form is recorded in
    // refused() (and thrown when the kernel was selected by name).
    void emit();

private:
    std::string name_;
    Expr expr_;
    std::vector<Target> targets_{Target::CPU, Target::GPU};
    std::string result_name_ = "Z";
    std::vector<std::string> ordering_;
    std::string gpu_python_name_;
    bool bindings_ = true;
    bool recursive_partitioning_ = true;
};

void set_selected_kernels(std::vector<std::string> names);
bool kernel_is_selected(const std::string &name);
bool kernel_is_named(const std::string &name);  // selected by --kernels, not by default
void set_output_directory(std::string dir);
const std::string &output_directory();

// Kernels emitted and refused (name, reason) since the start of the process.
const std::vector<Emitted> &emitted();
const std::vector<std::pair<std::string, std::string>> &refused();

// --kernels name[,name...]  --output-dir DIR (default: generated).  Returns false, after
// printing usage, on malformed arguments.
bool parse_command_line(int argc, char **argv);

}  // namespace nacho_hipgen
