// hipgen.cpp — declaration analysis, entry-point matching and the two file writers of the
// HIP code generator (interface and scope in hipgen.hpp).
#include "hipgen.hpp"

#include <algorithm>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <set>
#include <sstream>

namespace nacho_hipgen {

// ---- formats and expressions ------------------------------------------------------------

Format Format::ordered(std::vector<Level> levels) {
    Format f;
    f.levels_ = std::move(levels);
    return f;
}

Format Format::named(std::string name) const {
    Format f = *this;
    f.name_ = std::move(name);
    return f;
}

Expr Tensor::make(const TensorType &type, const std::string &name) {
    auto node = std::make_shared<ExprNode>();
    node->kind = ExprNode::Kind::Tensor;
    node->name = name;
    node->type = std::make_shared<TensorType>(type);
    return Expr(node);
}

Expr Sum::make(const std::string &index, Expr body) {
    auto node = std::make_shared<ExprNode>();
    node->kind = ExprNode::Kind::Sum;
    node->name = index;
    node->lhs = std::move(body);
    return Expr(node);
}

static Expr binary(ExprNode::Kind kind, const Expr &a, const Expr &b) {
    if (!a.defined() || !b.defined()) throw std::invalid_argument("undefined operand expression");
    auto node = std::make_shared<ExprNode>();
    node->kind = kind;
    node->lhs = a;
    node->rhs = b;
    return Expr(node);
}

Expr operator+(const Expr &a, const Expr &b) { return binary(ExprNode::Kind::Add, a, b); }
Expr operator*(const Expr &a, const Expr &b) { return binary(ExprNode::Kind::Mul, a, b); }

// ---- analysis ---------------------------------------------------------------------------

namespace {

const char *kind_word(ExprNode::Kind k) {
    switch (k) {
        case ExprNode::Kind::Tensor: return "a tensor";
        case ExprNode::Kind::Add: return "a sum";
        case ExprNode::Kind::Mul: return "a product";
        case ExprNode::Kind::Sum: return "a reduction";
    }
    return "?";
}

// Leaves of a chain of `kind` nodes, left to right; every leaf must be a tensor.
void flatten(const ExprNode *n, ExprNode::Kind kind, const std::string &kernel,
             std::vector<const ExprNode *> &leaves) {
    if (n->kind == kind) {
        flatten(n->lhs.get(), kind, kernel, leaves);
        flatten(n->rhs.get(), kind, kernel, leaves);
        return;
    }
    if (n->kind != ExprNode::Kind::Tensor) {
        throw UnsupportedForm(kernel + ": " + kind_word(n->kind) + " inside " + kind_word(kind) +
                              " has no HIP kernel (mixed operators)");
    }
    leaves.push_back(n);
}

std::vector<std::string> index_list(const Format &f) {
    std::vector<std::string> out;
    for (const Level &l : f.levels()) out.push_back(l.index);
    return out;
}

// Storage classes the library has descriptors for, recognised by their level formats.
enum class Storage { CSR, DCSR, CSF3, COO, COO3, Other };

Storage storage_of(const Format &f) {
    using L = LevelFormat;
    std::vector<L> k;
    for (const Level &l : f.levels()) k.push_back(l.format);
    if (k == std::vector<L>{L::Dense, L::Compressed_unique}) return Storage::CSR;
    if (k == std::vector<L>{L::Compressed_unique, L::Compressed_unique}) return Storage::DCSR;
    if (k == std::vector<L>{L::Compressed_unique, L::Compressed_unique, L::Compressed_unique})
        return Storage::CSF3;
    if (k == std::vector<L>{L::Compressed_non_unique, L::Singleton_unique}) return Storage::COO;
    if (k == std::vector<L>{L::Compressed_non_unique, L::Singleton_non_unique,
                            L::Singleton_unique})
        return Storage::COO3;
    return Storage::Other;
}

const char *storage_word(Storage s) {
    switch (s) {
        case Storage::CSR: return "CSR (dense, compressed)";
        case Storage::DCSR: return "DCSR (compressed, compressed)";
        case Storage::CSF3: return "CSF3 (compressed x3)";
        case Storage::COO: return "COO (compressed non-unique, singleton)";
        case Storage::COO3: return "COO3 (compressed non-unique, singleton x2)";
        case Storage::Other: return "a level structure the library has no descriptor for";
    }
    return "?";
}

const char *descriptor_of(Storage s) {
    switch (s) {
        case Storage::CSR: return "nacho_csr";
        case Storage::DCSR: return "nacho_dcsr";
        case Storage::CSF3: return "nacho_csf3";
        case Storage::COO: return "nacho_coo";
        case Storage::COO3: return "nacho_coo3";
        case Storage::Other: break;
    }
    return nullptr;
}

// Canonical index names of a descriptor's fields: the C structs of nacho_hip.h are the
// generated structs over (i, j[, k]).
const char *kCanonical[] = {"i", "j", "k"};

Format canonical(const Format &f) {
    std::vector<Level> levels = f.levels();
    for (size_t x = 0; x < levels.size(); ++x) levels[x].index = kCanonical[x];
    return Format::ordered(levels).named(f.name());
}

}  // namespace

Declaration analyse(const std::string &kernel, const Expr &expression) {
    if (!expression.defined()) throw std::invalid_argument(kernel + ": no expression");
    Declaration d;
    d.kernel = kernel;
    const ExprNode *root = expression.get();
    std::vector<const ExprNode *> leaves;
    switch (root->kind) {
        case ExprNode::Kind::Tensor:
            throw UnsupportedForm(kernel + ": a single tensor (a copy) has no HIP kernel");
        case ExprNode::Kind::Add:
            d.form = Form::Add;
            flatten(root, ExprNode::Kind::Add, kernel, leaves);
            break;
        case ExprNode::Kind::Mul:
            d.form = Form::Mul;
            flatten(root, ExprNode::Kind::Mul, kernel, leaves);
            break;
        case ExprNode::Kind::Sum: {
            const ExprNode *body = root;
            while (body->kind == ExprNode::Kind::Sum) {
                d.reduced_indices.push_back(body->name);
                body = body->lhs.get();
            }
            if (d.reduced_indices.size() == 1) {
                d.form = Form::SumOfProducts;
                d.reduced_index = root->name;
            } else {
                d.form = Form::FullReduction;  // plan() checks that nothing is left
            }
            if (body->kind != ExprNode::Kind::Mul) {
                throw UnsupportedForm(kernel + ": only a reduction of a product has a HIP "
                                               "kernel (Sum over " + root->name + " of " +
                                      kind_word(body->kind) + ")");
            }
            flatten(body, ExprNode::Kind::Mul, kernel, leaves);
            break;
        }
    }
    std::set<std::string> seen;
    for (const ExprNode *leaf : leaves) {
        if (!seen.insert(leaf->name).second) {
            throw UnsupportedForm(kernel + ": operand '" + leaf->name +
                                  "' appears twice; pass it as two operands");
        }
        d.operands.push_back(Operand{leaf->name, *leaf->type});
    }
    d.ordering.assign(seen.begin(), seen.end());  // lexicographic, the reference's default
    return d;
}

// ---- matching ---------------------------------------------------------------------------

namespace {

bool has_index(const Format &f, const std::string &x) {
    for (const Level &l : f.levels())
        if (l.index == x) return true;
    return false;
}

}  // namespace

Plan plan(const Declaration &d) {
    const std::string &k = d.kernel;
    for (const Operand &o : d.operands) {
        if (o.type.dtype != dType::Float32) {
            throw UnsupportedForm(k + ": operand '" + o.name +
                                  "' is not float32; the HIP kernels compute in float32");
        }
    }
    Plan p;
    const Storage s0 = storage_of(d.operands.at(0).type.format);
    if (d.form == Form::Add && d.operands.size() == 2 &&
        storage_of(d.operands[1].type.format) != s0) {
        // a CSR operand plus a COO operand (compiler.cpp:122): CSR result
        const Operand *csr = nullptr, *coo = nullptr;
        for (const Operand &o : d.operands) {
            const Storage s = storage_of(o.type.format);
            if (s == Storage::CSR) csr = &o;
            if (s == Storage::COO) coo = &o;
        }
        if (!csr || !coo) {
            throw UnsupportedForm(
                k + ": operands of different formats (" + storage_word(s0) + " and " +
                storage_word(storage_of(d.operands[1].type.format)) +
                ") have a HIP kernel only as a CSR plus a COO");
        }
        if (index_list(csr->type.format) != index_list(coo->type.format)) {
            throw UnsupportedForm(k + ": elementwise operands must share their index order");
        }
        if (index_list(csr->type.format)[0] == index_list(csr->type.format)[1]) {
            throw UnsupportedForm(k + ": an index repeated within one operand (a diagonal) "
                                      "has no HIP kernel");
        }
        p.entry_point = "nacho_gpu_coo_csr_add_f32";
        p.descriptor = p.result_descriptor = "nacho_csr";
        p.operand_descriptor[csr->name] = "nacho_csr";
        p.operand_descriptor[coo->name] = "nacho_coo";
        p.roles = {csr->name, coo->name};
        p.result_format = csr->type.format;
    } else if (d.form == Form::FullReduction) {
        // Sum over every index of a * b, both CSF3 or both COO3 (compiler.cpp:141, 143)
        if (d.operands.size() != 2) {
            throw UnsupportedForm(k + ": a reduction over several indices has a HIP kernel "
                                      "only for the product of two operands");
        }
        const auto idx = index_list(d.operands[0].type.format);
        if (index_list(d.operands[1].type.format) != idx) {
            throw UnsupportedForm(k + ": a reduction over several indices needs both "
                                      "operands in one index order");
        }
        const std::set<std::string> summed(d.reduced_indices.begin(), d.reduced_indices.end());
        if (summed != std::set<std::string>(idx.begin(), idx.end()) ||
            summed.size() != d.reduced_indices.size()) {
            throw UnsupportedForm(k + ": a reduction over more than one index that does not "
                                      "sum every index of its operands once has no HIP kernel");
        }
        const Storage s1 = storage_of(d.operands[1].type.format);
        if (s0 != s1 || (s0 != Storage::CSF3 && s0 != Storage::COO3)) {
            throw UnsupportedForm(k + ": a full reduction has a HIP kernel only over two CSF3 "
                                      "or two COO3 operands");
        }
        p.entry_point = s0 == Storage::CSF3 ? "nacho_gpu_inner_prod_f32"
                                            : "nacho_gpu_inner_prod_coo_f32";
        p.descriptor = descriptor_of(s0);
        p.result_descriptor = "nacho_scalar";
        for (const Operand &o : d.operands) p.roles.push_back(o.name);
        p.result_format = Format::ordered({}).named("Scalar");
    } else if (d.form == Form::Add || d.form == Form::Mul) {
        const auto idx0 = index_list(d.operands[0].type.format);
        for (const Operand &o : d.operands) {
            const Storage s = storage_of(o.type.format);
            if (s != s0) {
                throw UnsupportedForm(k + ": operands of different formats (" +
                                      storage_word(s0) + " and " + storage_word(s) +
                                      ") have no HIP kernel");
            }
            if (index_list(o.type.format) != idx0) {
                throw UnsupportedForm(k + ": elementwise operands must share their index order");
            }
        }
        std::set<std::string> distinct(idx0.begin(), idx0.end());
        if (distinct.size() != idx0.size()) {
            throw UnsupportedForm(k + ": an index repeated within one operand (a diagonal) "
                                      "has no HIP kernel");
        }
        const size_t n = d.operands.size();
        const bool add = d.form == Form::Add;
        std::string entry;
        if (s0 == Storage::CSR && n == 2) entry = add ? "csr_add" : "csr_mul";
        else if (s0 == Storage::CSR && n == 3 && add) entry = "csr_add_3";
        else if (s0 == Storage::COO && n == 2) entry = add ? "coo_add" : "coo_mul";
        else if (s0 == Storage::DCSR && n == 2) {
            entry = add ? "dcsr_add"
                        : (d.recursive_partitioning ? "dcsr_mul"
                                                    : "dcsr_mul_without_recursive_partitioning");
        } else if (s0 == Storage::CSF3 && n == 2 && add) entry = "csf_add";
        else if (s0 == Storage::COO3 && n == 2 && add) entry = "coo3d_add";
        if (entry.empty()) {
            throw UnsupportedForm(k + ": no HIP kernel for " + (add ? "a sum" : "a product") +
                                  " of " + std::to_string(n) + " operands in " +
                                  storage_word(s0));
        }
        p.entry_point = "nacho_gpu_" + entry + "_f32";
        p.descriptor = p.result_descriptor = descriptor_of(s0);
        for (const Operand &o : d.operands) p.roles.push_back(o.name);
        p.result_format = d.operands[0].type.format;
    } else {
        // Sum over j of a_ij * b_jk [* c_ik]: every operand CSR, roles fixed by indices.
        for (const Operand &o : d.operands) {
            if (storage_of(o.type.format) != Storage::CSR) {
                throw UnsupportedForm(k + ": a reduction of a product has a HIP kernel only "
                                          "over CSR operands ('" + o.name + "' is " +
                                      storage_word(storage_of(o.type.format)) + ")");
            }
        }
        const std::string &j = d.reduced_index;
        const Operand *left = nullptr, *right = nullptr, *mask = nullptr;
        for (const Operand &o : d.operands) {
            const auto idx = index_list(o.type.format);
            if (idx[1] == j && idx[0] != j) {
                if (left) throw UnsupportedForm(k + ": two operands end in the reduced index");
                left = &o;
            } else if (idx[0] == j && idx[1] != j) {
                if (right) throw UnsupportedForm(k + ": two operands start with the reduced index");
                right = &o;
            } else if (!has_index(o.type.format, j)) {
                if (mask) throw UnsupportedForm(k + ": more than one operand without the "
                                                    "reduced index");
                mask = &o;
            } else {
                throw UnsupportedForm(k + ": operand '" + o.name + "' uses the reduced index "
                                          "on both levels");
            }
        }
        if (!left || !right) {
            throw UnsupportedForm(k + ": the reduced index " + j + " must be the column index "
                                      "of one operand and the row index of another");
        }
        const std::string i = index_list(left->type.format)[0];
        const std::string kk = index_list(right->type.format)[1];
        if (i == kk) {
            throw UnsupportedForm(k + ": a product whose result index repeats (" + i + ", " +
                                  kk + ") has no HIP kernel");
        }
        if (mask && index_list(mask->type.format) != std::vector<std::string>{i, kk}) {
            throw UnsupportedForm(k + ": the third factor must be indexed (" + i + ", " + kk +
                                  ") like the result");
        }
        p.entry_point = mask ? "nacho_gpu_sssmm_f32" : "nacho_gpu_spgemm_f32";
        p.descriptor = p.result_descriptor = "nacho_csr";
        p.roles = {left->name, right->name};
        if (mask) p.roles.push_back(mask->name);
        const Format &named = (mask ? mask : left)->type.format;
        p.result_format = Format::ordered({{i, LevelFormat::Dense},
                                           {kk, LevelFormat::Compressed_unique}})
                              .named(named.name());
    }
    const std::string cls = p.result_format.name().empty() ? "Tensor" : p.result_format.name();
    p.result_class = cls + "_gpu";
    return p;
}

// ---- struct layout ----------------------------------------------------------------------

namespace {

struct Field {
    std::string name;
    enum class Type { Index, IndexPtr, ValuePtr } type;
};

// Fields of the generated tensor struct of a format, in the generated order
// (src/backend/tensor.cpp:13-61): one size per index in level order, then per level its
// offsets (a compressed level below the first), length and coordinates (a run of a
// compressed non-unique level and its singleton levels carries length and coordinates per
// index, no offsets), then values and nnz.
std::vector<Field> struct_fields(const Format &f) {
    std::vector<Field> out;
    for (const Level &l : f.levels()) out.push_back({"dim_" + l.index + "_size", Field::Type::Index});
    const auto &lv = f.levels();
    for (size_t x = 0; x < lv.size(); ++x) {
        const Level &l = lv[x];
        if (l.format == LevelFormat::Dense) continue;
        if (l.format == LevelFormat::Compressed_unique && x > 0) {
            out.push_back({"dim_" + l.index + "_offsets", Field::Type::IndexPtr});
        }
        out.push_back({"dim_" + l.index + "_length", Field::Type::Index});
        out.push_back({"dim_" + l.index + "_indices", Field::Type::IndexPtr});
    }
    out.push_back({"values", Field::Type::ValuePtr});
    out.push_back({"nnz", Field::Type::Index});
    return out;
}

// One buffer of a Python tensor class: its C descriptor field and the number of elements,
// as an expression over the descriptor `t` (generate_bindings.cpp:84-170).
struct Buffer {
    std::string c_field;
    bool is_value;
    std::string extent;
    std::string length_field;  // descriptor field holding the buffer's length, or ""
};

std::vector<Buffer> class_buffers(const Format &c /* canonical indices */) {
    std::vector<Buffer> out;
    const auto &lv = c.levels();
    std::string last_length = "1";
    for (size_t x = 0; x < lv.size(); ++x) {
        const Level &l = lv[x];
        if (l.format == LevelFormat::Dense) {
            last_length = last_length == "1" ? "t.dim_" + l.index + "_size"
                                             : last_length + " * t.dim_" + l.index + "_size";
            continue;
        }
        if (l.format == LevelFormat::Compressed_unique && x > 0) {
            const Level &parent = lv[x - 1];
            const std::string parent_extent = parent.format == LevelFormat::Dense
                                                  ? "t.dim_" + parent.index + "_size"
                                                  : "t.dim_" + parent.index + "_length";
            out.push_back({"dim_" + l.index + "_offsets", false, parent_extent + " + 1", ""});
        }
        out.push_back({"dim_" + l.index + "_indices", false, "t.dim_" + l.index + "_length",
                       "dim_" + l.index + "_length"});
        last_length = "t.dim_" + l.index + "_length";
    }
    out.push_back({"values", true, last_length, "nnz"});
    return out;
}

struct PyClass {
    std::vector<std::string> members;  // buffer member names, in level order
    size_t rank = 0;
};

std::map<std::string, PyClass> &classes() {
    static std::map<std::string, PyClass> m;
    return m;
}

// The class's member names: those of the first tensor recorded under the class name.
const PyClass &record_class(const std::string &name, const Format &f) {
    PyClass described;
    for (const Level &l : f.levels()) {
        (void)l;
        ++described.rank;
    }
    const Format canon = canonical(f);
    const auto canon_buffers = class_buffers(canon);
    // member names follow the tensor's own index names
    for (const Buffer &b : canon_buffers) {
        std::string m = b.c_field;
        for (size_t x = 0; x < f.levels().size(); ++x) {
            const std::string from = std::string("dim_") + kCanonical[x] + "_";
            if (m.rfind(from, 0) == 0) {
                m = "dim_" + f.levels()[x].index + "_" + m.substr(from.size());
                break;
            }
        }
        described.members.push_back(m);
    }
    auto [it, inserted] = classes().emplace(name, described);
    if (!inserted && (it->second.members.size() != described.members.size() ||
                      it->second.rank != described.rank)) {
        throw std::invalid_argument("two different layouts both map to the Python class '" +
                                    name + "'; name the formats apart");
    }
    return it->second;
}

std::string field_type(const Field &f) {
    switch (f.type) {
        case Field::Type::Index: return "index_t";
        case Field::Type::IndexPtr: return "index_t *";
        case Field::Type::ValuePtr: return "value_t *";
    }
    return "";
}

// "index_t dim_i_size", "index_t *dim_j_offsets"
std::string declare_field(const Field &f) {
    const std::string t = field_type(f);
    return t.back() == '*' ? t + f.name : t + " " + f.name;
}

std::string text_of(const Declaration &d) {
    std::string op = d.form == Form::Add ? " + " : " * ";
    std::string body;
    for (size_t x = 0; x < d.operands.size(); ++x) {
        const Operand &o = d.operands[x];
        body += (x ? op : "") + o.name + "(";
        const auto idx = index_list(o.type.format);
        for (size_t y = 0; y < idx.size(); ++y) body += (y ? "," : "") + idx[y];
        body += ")";
    }
    if (d.form == Form::SumOfProducts) return "Sum(" + d.reduced_index + ", " + body + ")";
    if (d.form == Form::FullReduction) {
        for (auto it = d.reduced_indices.rbegin(); it != d.reduced_indices.rend(); ++it)
            body = "Sum(" + *it + ", " + body + ")";
    }
    return body;
}

std::ofstream open_out(const std::string &path) {
    std::ofstream out(path);
    if (!out) throw std::runtime_error("cannot open '" + path + "' for writing");
    return out;
}

void check_ordering(const Declaration &d) {
    std::vector<std::string> a = d.ordering, b;
    for (const Operand &o : d.operands) b.push_back(o.name);
    std::sort(a.begin(), a.end());
    std::sort(b.begin(), b.end());
    if (a != b) {
        throw std::invalid_argument(d.kernel + ": operand_ordering must name every operand "
                                               "exactly once");
    }
}

const Operand &operand_named(const Declaration &d, const std::string &name) {
    for (const Operand &o : d.operands)
        if (o.name == name) return o;
    throw std::logic_error("no operand " + name);
}

// C descriptor of operand `name`.
const std::string &descriptor_for(const Plan &p, const std::string &name) {
    auto it = p.operand_descriptor.find(name);
    return it == p.operand_descriptor.end() ? p.descriptor : it->second;
}

void write_header(const Declaration &d, const Plan &p, const std::string &path) {
    std::ofstream out = open_out(path);
    const std::string &k = d.kernel;
    out << "// " << k << "_gpu.h — generated by nacho_hipgen for the GPU target (HIP, gfx950).\n"
        << "// Declaration: " << d.result_name << " = " << text_of(d) << "\n"
        << "// " << k << "_gpu_i32_f32 calls " << p.entry_point
        << " in libnacho_hip.so (include/nacho_hip.h):\n"
        << "// link with -lnacho_hip; errors throw std::runtime_error; the call runs on\n"
        << "// nacho_hip::stream(); release each non-null result array with nacho_free.\n"
        << "#pragma once\n\n#include <cstddef>\n#include <cstdint>\n\n"
        << "#include \"nacho_hip.h\"\n#include \"nacho_hip_runtime.hpp\"\n\n"
        << "namespace " << k << " {\n\nusing index_t = int32_t;\nusing value_t = float;\n\n";

    auto write_struct = [&](const std::string &tensor, const Format &f, const std::string &desc) {
        const std::string s = tensor + "_tensor_format";
        out << "template <typename index_t, typename value_t>\nstruct " << s << " {\n";
        const auto fields = struct_fields(f);
        for (const Field &fl : fields) out << "    " << declare_field(fl) << ";\n";
        out << "};\n";
        // the C ABI receives this struct's bytes as `desc`: same size, same offsets
        const auto cfields = struct_fields(canonical(f));
        out << "namespace layout {\nusing " << tensor << " = " << s << "<int32_t, float>;\n"
            << "static_assert(sizeof(" << tensor << ") == sizeof(" << desc << "), \"" << s
            << " and " << desc << " differ\");\n";
        for (size_t x = 0; x < fields.size(); ++x) {
            out << "static_assert(offsetof(" << tensor << ", " << fields[x].name
                << ") == offsetof(" << desc << ", " << cfields[x].name << "), \"" << s << "."
                << fields[x].name << "\");\n";
        }
        out << "}  // namespace layout\n\n";
    };
    for (const std::string &name : d.ordering)
        write_struct(name, operand_named(d, name).type.format, descriptor_for(p, name));
    write_struct(d.result_name, p.result_format, p.result_descriptor);

    const std::string zt = d.result_name + "_tensor_format<index_t, value_t>";
    out << "inline " << zt << " " << k << "_gpu_i32_f32(";
    for (const std::string &name : d.ordering)
        out << "const " << name << "_tensor_format<index_t, value_t> " << name << ", ";
    out << "const int32_t num_blocks, const int32_t threads_per_block) {\n";
    for (const std::string &name : d.ordering) {
        out << "    const " << descriptor_for(p, name) << " desc_" << name
            << " = nacho_hip::detail::to_c<" << descriptor_for(p, name) << ">(" << name
            << ");\n";
    }
    out << "    " << p.result_descriptor << " desc_result{};\n";
    out << "    nacho_hip::detail::check(" << p.entry_point << "(";
    for (const std::string &role : p.roles) out << "&desc_" << role << ", ";
    out << "&desc_result, num_blocks, threads_per_block,\n"
        << "                                 nacho_hip::stream(), nullptr),\n"
        << "                             \"" << k << "\");\n";
    out << "    return nacho_hip::detail::from_c<" << zt << ">(desc_result);\n}\n\n"
        << "}  // namespace " << k << "\n";
}

void write_wrapper(const Declaration &d, const Plan &p, const std::string &path) {
    std::ofstream out = open_out(path);
    const std::string &k = d.kernel;
    const std::string python =
        d.python_name.empty() ? "gpu_" + k + "_f32" : d.python_name;
    out << "// " << k << "_gpu_nb.cpp — generated by nacho_hipgen: nanobind binding of " << k
        << " for the GPU target.\n"
        << "// Declaration: " << d.result_name << " = " << text_of(d) << "\n"
        << "// Calls " << p.entry_point << " (include/nacho_hip.h) directly; compile as C++ "
        << "and link with -lnacho_hip.\n"
        << "// nacho_types.h supplies the Python tensor classes and nacho_nb.h's helpers.\n"
        << "#include <cstddef>\n#include <cstdint>\n\n"
        << "#include \"nacho_types.h\"\n#include \"nacho_hip.h\"\n"
        << "#include \"nacho_hip_runtime.hpp\"\n\nnamespace {\n\n";

    // classes are recorded result first, then operands in parameter order, as the
    // reference's bindings generator records them (generate_bindings.cpp:266-275)
    record_class(p.result_class, p.result_format);
    // one unwrap per operand, one wrap for the result
    for (const std::string &name : d.ordering) {
        const Format &f = operand_named(d, name).type.format;
        const std::string cls = (f.name().empty() ? "Tensor" : f.name()) + "_gpu";
        const PyClass &pc = record_class(cls, f);
        const Format canon = canonical(f);
        const auto bufs = class_buffers(canon);
        out << descriptor_for(p, name) << " unwrap_" << name << "(const " << cls << " &v) {\n"
            << "    " << descriptor_for(p, name) << " t = {};\n";
        for (size_t x = 0; x < canon.levels().size(); ++x) {
            out << "    t.dim_" << kCanonical[x] << "_size = v.shape.data()[" << x << "];\n";
        }
        for (size_t x = 0; x < bufs.size(); ++x) {
            const Buffer &b = bufs[x];
            out << "    t." << b.c_field << " = nacho::borrow<" << (b.is_value ? "float" : "int32_t")
                << ">(v." << pc.members[x] << ");\n";
            if (!b.length_field.empty()) {
                out << "    t." << b.length_field << " = (int32_t)v." << pc.members[x]
                    << ".shape(0);\n";
            }
        }
        out << "    return t;\n}\n\n";
    }
    {
        const std::string &cls = p.result_class;
        const PyClass &pc = record_class(cls, p.result_format);
        const Format canon = canonical(p.result_format);
        const auto bufs = class_buffers(canon);
        out << cls << " wrap_result(const " << p.result_descriptor << " &t) {\n"
            << "    return " << cls << "{\n";
        for (const Buffer &b : bufs) {
            out << "        nacho::adopt_gpu<" << (b.is_value ? "float" : "int32_t") << ">(t."
                << b.c_field << ", (size_t)(" << b.extent << ")),\n";
        }
        // a full reduction has no dimensions left and carries no shape
        // (generate_bindings.cpp:181-183)
        if (!canon.levels().empty()) {
            out << "        nacho::make_shape<" << canon.levels().size() << ">({";
            for (size_t x = 0; x < canon.levels().size(); ++x)
                out << (x ? ", " : "") << "t.dim_" << kCanonical[x] << "_size";
            out << "}),\n";
        }
        out << "    };\n}\n\n";
        (void)pc;
    }

    out << p.result_class << " " << python << "(";
    for (const std::string &name : d.ordering) {
        const Format &f = operand_named(d, name).type.format;
        out << "const " << (f.name().empty() ? "Tensor" : f.name()) << "_gpu &" << name << ", ";
    }
    out << "int32_t num_blocks, int32_t threads_per_block) {\n";
    for (const std::string &name : d.ordering)
        out << "    const " << descriptor_for(p, name) << " desc_" << name << " = unwrap_"
            << name << "(" << name << ");\n";
    out << "    " << p.result_descriptor << " desc_result = {};\n"
        << "    nacho_hip::detail::check(" << p.entry_point << "(";
    for (const std::string &role : p.roles) out << "&desc_" << role << ", ";
    out << "&desc_result, num_blocks,\n"
        << "                                 threads_per_block, nacho_hip::stream(), nullptr),\n"
        << "                             \"" << k << "\");\n"
        << "    return wrap_result(desc_result);\n}\n\n}  // namespace\n\n";

    out << "void register_" << k << "_gpu(nb::module_ &m) {\n"
        << "    m.def(\"" << python << "\", &" << python;
    for (const std::string &name : d.ordering) out << ", nb::arg(\"" << name << "\")";
    out << ",\n          nb::arg(\"num_blocks\") = 256, nb::arg(\"threads_per_block\") = 256);\n}\n";
}

// ---- Kernel builder state ---------------------------------------------------------------

struct Session {
    std::vector<std::string> selected;
    std::string output_dir = "generated";
    std::vector<Emitted> emitted;
    std::vector<std::pair<std::string, std::string>> refused;
};

Session &session() {
    static Session s;
    return s;
}

}  // namespace

void reset_classes() { classes().clear(); }

Emitted emit_gpu(const Declaration &d, const std::string &output_dir) {
    check_ordering(d);
    const Plan p = plan(d);
    Emitted e;
    e.entry_point = p.entry_point;
    e.header = output_dir + "/" + d.kernel + "_gpu.h";
    e.wrapper = output_dir + "/" + d.kernel + "_gpu_nb.cpp";
    write_header(d, p, e.header);
    write_wrapper(d, p, e.wrapper);
    return e;
}

Kernel::Kernel(std::string name) : name_(std::move(name)) {}
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
    ordering_ = std::move(names);
    return *this;
}
Kernel &Kernel::python_name(Target target, std::string name) {
    if (target == Target::GPU) gpu_python_name_ = std::move(name);
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

Emitted emit_declaration(const Declaration &declaration, bool bindings,
                         const std::string &output_dir) {
    std::filesystem::create_directories(output_dir);
    Emitted e = emit_gpu(declaration, output_dir);
    if (!bindings) {
        std::filesystem::remove(e.wrapper);
        e.wrapper.clear();
    }
    session().emitted.push_back(e);
    return e;
}

void refuse(const std::string &kernel, const std::string &reason) {
    session().refused.emplace_back(kernel, reason);
    if (kernel_is_named(kernel)) throw UnsupportedForm(reason);
}

void Kernel::emit() {
    if (!kernel_is_selected(name_)) return;
    if (std::find(targets_.begin(), targets_.end(), Target::GPU) == targets_.end()) return;
    try {
        Declaration d = analyse(name_, expr_);
        if (!ordering_.empty()) d.ordering = ordering_;
        d.result_name = result_name_;
        d.python_name = gpu_python_name_;
        d.recursive_partitioning = recursive_partitioning_;
        emit_declaration(d, bindings_, session().output_dir);
    } catch (const UnsupportedForm &err) {
        refuse(name_, err.what());
    }
}

void set_selected_kernels(std::vector<std::string> names) { session().selected = std::move(names); }

bool kernel_is_selected(const std::string &name) {
    const auto &sel = session().selected;
    return sel.empty() || std::find(sel.begin(), sel.end(), name) != sel.end();
}

bool kernel_is_named(const std::string &name) {
    const auto &sel = session().selected;
    return std::find(sel.begin(), sel.end(), name) != sel.end();
}

void set_output_directory(std::string dir) { session().output_dir = std::move(dir); }
const std::string &output_directory() { return session().output_dir; }
const std::vector<Emitted> &emitted() { return session().emitted; }
const std::vector<std::pair<std::string, std::string>> &refused() { return session().refused; }

bool parse_command_line(int argc, char **argv) {
    auto usage = [&]() {
        std::cerr << "usage: " << (argc > 0 ? argv[0] : "nacho_hipgen")
                  << " [--kernels name[,name...]] [--output-dir DIR]\n";
    };
    std::vector<std::string> selected;
    for (int x = 1; x < argc; ++x) {
        const std::string arg = argv[x];
        if ((arg == "--kernels" || arg == "--output-dir") && x + 1 >= argc) {
            usage();
            return false;
        }
        if (arg == "--kernels") {
            std::stringstream list(argv[++x]);
            std::string item;
            while (std::getline(list, item, ','))
                if (!item.empty()) selected.push_back(item);
        } else if (arg == "--output-dir") {
            set_output_directory(argv[++x]);
        } else {
            usage();
            return false;
        }
    }
    set_selected_kernels(selected);
    return true;
}

}  // namespace nacho_hipgen
