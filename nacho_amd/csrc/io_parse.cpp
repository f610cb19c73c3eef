// Matrix Market (.mtx) and FROSTT (.tns) readers on the host.
//
// Reference: runtime/io/parse.h:28-263 (parse2D, parse3D), exposed to Python as
// nacho.parse2D and nacho.parse3D_i32_f32 (runtime/register_runtime.cpp:20-40).  The same
// results are produced: coordinates in file order converted to 0-based int32, values as
// float32, and for symmetric / skew-symmetric matrices the mirrored off-diagonal entries
// appended after the file's entries in file order (negated for skew-symmetric).  Values of
// .mtx files are read as double and rounded to float (parse.h reads `double val`), values of
// .tns files are read directly as float (parse.h reads `value_t v`).
//
// Differences: the file is read once into memory and parsed with strtoull/strtod instead of
// iostreams, and every failure is returned as an error code rather than terminating the
// process (the reference calls exit(-1) or assert(false)).
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/nacho_hip.h"

namespace {

bool read_file(const char *path, std::string *out) {
    FILE *f = std::fopen(path, "rb");
    if (!f) return false;
    std::string data;
    char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) data.append(buf, n);
    const bool ok = !std::ferror(f);
    std::fclose(f);
    *out = std::move(data);
    return ok;
}

// Whitespace-separated token reader over a NUL-terminated buffer.
struct Cursor {
    const char *p;

    void skip_space() {
        while (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r' || *p == '\v' || *p == '\f') ++p;
    }
    bool token(std::string *t) {
        skip_space();
        const char *s = p;
        while (*p && !(*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r' || *p == '\v' ||
                       *p == '\f')) {
            ++p;
        }
        t->assign(s, p);
        return p != s;
    }
    bool u64(uint64_t *v) {
        skip_space();
        if (*p < '0' || *p > '9') return false;
        char *end = nullptr;
        errno = 0;
        const unsigned long long x = std::strtoull(p, &end, 10);
        if (end == p || errno == ERANGE) return false;
        p = end;
        *v = x;
        return true;
    }
    bool i32(int32_t *v) {
        skip_space();
        char *end = nullptr;
        errno = 0;
        const long x = std::strtol(p, &end, 10);
        if (end == p || errno == ERANGE || x < INT32_MIN || x > INT32_MAX) return false;
        p = end;
        *v = static_cast<int32_t>(x);
        return true;
    }
    bool f64(double *v) {
        skip_space();
        char *end = nullptr;
        const double x = std::strtod(p, &end);
        if (end == p) return false;
        p = end;
        *v = x;
        return true;
    }
    bool f32(float *v) {
        skip_space();
        char *end = nullptr;
        const float x = std::strtof(p, &end);
        if (end == p) return false;
        p = end;
        *v = x;
        return true;
    }
    // Skip the rest of the current line (the reference ignores at most 2048 characters).
    void skip_line() {
        while (*p && *p != '\n') ++p;
        if (*p == '\n') ++p;
    }
};

template <typename T>
T *to_malloc(const std::vector<T> &v) {
    T *p = static_cast<T *>(std::malloc(v.empty() ? 1 : v.size() * sizeof(T)));
    if (p && !v.empty()) std::memcpy(p, v.data(), v.size() * sizeof(T));
    return p;
}

}  // namespace

namespace {

// The readers are called through ctypes and C: a C++ exception must not leave them.
// std::bad_alloc becomes NACHO_ERR_OUT_OF_MEMORY, anything else NACHO_ERR_MALFORMED_INPUT.
template <typename F>
int guarded(F &&body) {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return NACHO_ERR_OUT_OF_MEMORY;
    } catch (...) {
        return NACHO_ERR_MALFORMED_INPUT;
    }
}

int parse2d(const char *path, nacho_coo2d_host *out) {
    std::string text;
    if (!read_file(path, &text)) return NACHO_ERR_IO;
    Cursor c{text.c_str()};
    std::string head, type, formats, field, symmetry;
    if (!c.token(&head) || !c.token(&type) || !c.token(&formats) || !c.token(&field) ||
        !c.token(&symmetry)) {
        return NACHO_ERR_MALFORMED_INPUT;
    }
    if (head != "%%MatrixMarket") return NACHO_ERR_MALFORMED_INPUT;
    if (type != "matrix" && type != "tensor") return NACHO_ERR_UNSUPPORTED;
    if (field != "real") return NACHO_ERR_UNSUPPORTED;
    if (symmetry != "general" && symmetry != "symmetric" && symmetry != "skew-symmetric") {
        return NACHO_ERR_UNSUPPORTED;
    }
    c.skip_line();
    while (*c.p == '%') c.skip_line();
    uint64_t n = 0, m = 0, nnz = 0;
    if (!c.u64(&n) || !c.u64(&m) || !c.u64(&nnz)) return NACHO_ERR_MALFORMED_INPUT;
    if (n > INT32_MAX || m > INT32_MAX) return NACHO_ERR_INDEX_OVERFLOW;
    const bool skew = symmetry == "skew-symmetric";
    const bool symm = symmetry == "symmetric" || skew;
    std::vector<int32_t> row, col;
    std::vector<float> val;
    // Every entry takes at least 6 characters ("1 1 0\n"), so a header that claims more
    // entries than the text can hold does not get to size the buffers.
    const uint64_t room = static_cast<uint64_t>(text.size() / 6);
    const size_t expect = static_cast<size_t>(nnz < room ? nnz : room);
    row.reserve(expect);
    col.reserve(expect);
    val.reserve(expect);
    uint64_t mirrored = 0;
    for (uint64_t e = 0; e < nnz; ++e) {
        uint64_t i = 0, j = 0;
        double v = 0.0;
        if (!c.u64(&i) || !c.u64(&j) || !c.f64(&v)) return NACHO_ERR_MALFORMED_INPUT;
        if (i < 1 || j < 1 || i > n || j > m) return NACHO_ERR_MALFORMED_INPUT;
        row.push_back(static_cast<int32_t>(i - 1));
        col.push_back(static_cast<int32_t>(j - 1));
        val.push_back(static_cast<float>(v));
        mirrored += (i != j);
    }
    if (symm && mirrored) {
        for (uint64_t e = 0; e < nnz; ++e) {
            if (row[e] != col[e]) {
                row.push_back(col[e]);
                col.push_back(row[e]);
                val.push_back(skew ? -val[e] : val[e]);
            }
        }
    }
    if (row.size() > static_cast<size_t>(INT32_MAX)) return NACHO_ERR_INDEX_OVERFLOW;
    out->row = to_malloc(row);
    out->col = to_malloc(col);
    out->data = to_malloc(val);
    if (!out->row || !out->col || !out->data) {
        std::free(out->row);
        std::free(out->col);
        std::free(out->data);
        *out = nacho_coo2d_host{};
        return NACHO_ERR_OUT_OF_MEMORY;
    }
    out->N = static_cast<int32_t>(n);
    out->M = static_cast<int32_t>(m);
    out->nnz = static_cast<int64_t>(row.size());
    return NACHO_OK;
}

int parse3d(const char *path, int32_t n, int32_t m, int32_t k, nacho_coo3d_host *out) {
    std::string text;
    if (!read_file(path, &text)) return NACHO_ERR_IO;
    Cursor c{text.c_str()};
    std::vector<int32_t> ci, cj, ck;
    std::vector<float> val;
    // Entries are read until the first one that does not parse (the reference's
    // `while (file >> i >> j >> k >> v)`); anything after it is ignored.
    for (;;) {
        int32_t i = 0, j = 0, l = 0;
        float v = 0.0f;
        const char *save = c.p;
        if (!c.i32(&i) || !c.i32(&j) || !c.i32(&l) || !c.f32(&v)) {
            c.p = save;
            break;
        }
        if (i < 1 || j < 1 || l < 1 || i > n || j > m || l > k) return NACHO_ERR_MALFORMED_INPUT;
        ci.push_back(i - 1);
        cj.push_back(j - 1);
        ck.push_back(l - 1);
        val.push_back(v);
    }
    out->row = to_malloc(ci);
    out->col = to_malloc(cj);
    out->dep = to_malloc(ck);
    out->data = to_malloc(val);
    if (!out->row || !out->col || !out->dep || !out->data) {
        std::free(out->row);
        std::free(out->col);
        std::free(out->dep);
        std::free(out->data);
        *out = nacho_coo3d_host{};
        return NACHO_ERR_OUT_OF_MEMORY;
    }
    out->N = n;
    out->M = m;
    out->K = k;
    out->nnz = static_cast<int64_t>(ci.size());
    return NACHO_OK;
}

}  // namespace

extern "C" {

void nacho_host_free(void *p) { std::free(p); }

int nacho_parse2d(const char *path, nacho_coo2d_host *out) {
    if (!path || !out) return NACHO_ERR_INVALID_ARGUMENT;
    *out = nacho_coo2d_host{};
    return guarded([&] { return parse2d(path, out); });
}

int nacho_parse3d(const char *path, int32_t n, int32_t m, int32_t k, nacho_coo3d_host *out) {
    if (!path || !out) return NACHO_ERR_INVALID_ARGUMENT;
    *out = nacho_coo3d_host{};
    return guarded([&] { return parse3d(path, n, m, k, out); });
}

}  // extern "C"
