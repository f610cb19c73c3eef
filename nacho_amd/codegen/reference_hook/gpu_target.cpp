// gpu_target.cpp — the reference's expression nodes to the HIP generator (see gpu_target.hpp).
#include "gpu_target.hpp"

namespace nacho_hipgen {

namespace {

LevelFormat level_format(::nacho::LevelFormat f) {
    switch (f) {
        case ::nacho::LevelFormat::Dense: return LevelFormat::Dense;
        case ::nacho::LevelFormat::Compressed_non_unique: return LevelFormat::Compressed_non_unique;
        case ::nacho::LevelFormat::Compressed_unique: return LevelFormat::Compressed_unique;
        case ::nacho::LevelFormat::Singleton_non_unique: return LevelFormat::Singleton_non_unique;
        case ::nacho::LevelFormat::Singleton_unique: return LevelFormat::Singleton_unique;
        case ::nacho::LevelFormat::MergedCoordinate: break;
    }
    throw UnsupportedForm("a MergedCoordinate level has no HIP kernel (only the reference's "
                          "lowering creates it)");
}

dType value_type(::nacho::dType t) {
    switch (t) {
        case ::nacho::dType::Float32: return dType::Float32;
        case ::nacho::dType::Float64: return dType::Float64;
        case ::nacho::dType::TemplateT: break;
    }
    throw UnsupportedForm("a tensor of template dtype has no HIP kernel");
}

// An operand of + or *: the reference's front end wraps an operand whose indices the other
// operand lacks in broadcasts (Bc) over those indices (src/Frontend.cpp:12-52).  The
// generator reads the index pattern from the operands' own formats and checks it for the
// whole expression, so these broadcasts carry nothing it needs.
Expr operand(const ::nacho::Expr &e) {
    if (const auto *b = e.as<::nacho::Bc>()) return operand(b->a);
    return from_reference(e);
}

}  // namespace

Expr from_reference(const ::nacho::Expr &e) {
    if (!e.defined()) throw UnsupportedForm("an undefined expression has no HIP kernel");
    if (const auto *t = e.as<::nacho::Tensor>()) {
        std::vector<Level> levels;
        for (const ::nacho::Level &l : t->type.format.levels) {
            if (l.index.indices.size() != 1) {
                throw UnsupportedForm("tensor " + t->name + ": a level over merged indices (" +
                                      l.index.str() + ") has no HIP kernel");
            }
            levels.push_back(Level{l.index.indices[0], level_format(l.format)});
        }
        if (!t->type.format.bc_levels.empty()) {
            throw UnsupportedForm("tensor " + t->name + ": an unordered format has no HIP kernel");
        }
        Format format = Format::ordered(std::move(levels)).named(t->type.format.name);
        return Tensor::make(TensorType(std::move(format), value_type(t->type.dtype)), t->name);
    }
    if (const auto *a = e.as<::nacho::Add>()) return operand(a->a) + operand(a->b);
    if (const auto *m = e.as<::nacho::Mul>()) return operand(m->a) * operand(m->b);
    if (const auto *s = e.as<::nacho::Sum>()) {
        if (s->index.indices.size() != 1) {
            throw UnsupportedForm("a sum over merged indices (" + s->index.str() +
                                  ") has no HIP kernel");
        }
        return Sum::make(s->index.indices[0], from_reference(s->a));
    }
    if (e.as<::nacho::Bc>()) {
        throw UnsupportedForm("a broadcast that is not an operand of + or * has no HIP kernel");
    }
    throw UnsupportedForm("an expression node the HIP generator does not know");
}

Emitted emit_reference_gpu(const std::string &kernel, const ::nacho::Expr &expression,
                           const std::string &result_name,
                           const std::vector<std::string> &operand_ordering,
                           const std::string &python_name, bool recursive_partitioning,
                           bool bindings, const std::string &output_dir) {
    Declaration d = analyse(kernel, from_reference(expression));
    if (!operand_ordering.empty()) d.ordering = operand_ordering;
    d.result_name = result_name;
    d.python_name = python_name;
    d.recursive_partitioning = recursive_partitioning;
    return emit_declaration(d, bindings, output_dir);
}

}  // namespace nacho_hipgen
