"""The HIP code generator for the GPU target (nacho_amd/codegen).

The reference's declarations (compiler.cpp:16-156) must generate <k>_gpu.h and
<k>_gpu_nb.cpp for every form the library implements and refuse the rest at generation time.
The generated headers compile against include/ and link with libnacho_hip; the generated
nanobind wrappers compile against a test double of nacho_types.h / nanobind
(tests/codegen_double); a call through either reaches the C ABI, which rejects mismatched
shapes on the host (before any HIP call) with an exception naming the kernel.  Declarations
of the reference's vocabulary with other names, index variables and operand orders map to
the entry point their structure implies.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CODEGEN = REPO / "nacho_amd" / "codegen"
DOUBLE = Path(__file__).resolve().parent / "codegen_double"

EXPECTED = {  # kernel of compiler.cpp -> entry point
    "csr_add": "nacho_gpu_csr_add_f32",
    "csr_add_3": "nacho_gpu_csr_add_3_f32",
    "csr_mul": "nacho_gpu_csr_mul_f32",
    "coo_add": "nacho_gpu_coo_add_f32",
    "coo_mul": "nacho_gpu_coo_mul_f32",
    "dcsr_add": "nacho_gpu_dcsr_add_f32",
    "dcsr_mul": "nacho_gpu_dcsr_mul_f32",
    "dcsr_mul_without_recursive_partitioning":
        "nacho_gpu_dcsr_mul_without_recursive_partitioning_f32",
    "csf_add": "nacho_gpu_csf_add_f32",
    "coo3d_add": "nacho_gpu_coo3d_add_f32",
    "spgemm": "nacho_gpu_spgemm_f32",
    "sssmm": "nacho_gpu_sssmm_f32",
    "coo_csr_add": "nacho_gpu_coo_csr_add_f32",
    "inner_prod": "nacho_gpu_inner_prod_f32",
    "inner_prod_coo": "nacho_gpu_inner_prod_coo_f32",
}
REFUSED = {}  # kernel of compiler.cpp -> part of the reason (every declaration has a kernel)
# Python-facing signature of each generated wrapper, in the test double's classes
SIGNATURES = {
    "csr_add": ("CSR_gpu", ["CSR_gpu"] * 2), "csr_add_3": ("CSR_gpu", ["CSR_gpu"] * 3),
    "csr_mul": ("CSR_gpu", ["CSR_gpu"] * 2), "coo_add": ("COO_gpu", ["COO_gpu"] * 2),
    "coo_mul": ("COO_gpu", ["COO_gpu"] * 2), "dcsr_add": ("DCSR_gpu", ["DCSR_gpu"] * 2),
    "dcsr_mul": ("DCSR_gpu", ["DCSR_gpu"] * 2),
    "dcsr_mul_without_recursive_partitioning": ("DCSR_gpu", ["DCSR_gpu"] * 2),
    "csf_add": ("CSF3_gpu", ["CSF3_gpu"] * 2), "coo3d_add": ("COO3_gpu", ["COO3_gpu"] * 2),
    "spgemm": ("CSR_gpu", ["CSR_gpu"] * 2), "sssmm": ("CSR_gpu", ["CSR_gpu"] * 3),
    "coo_csr_add": ("CSR_gpu", ["CSR_gpu", "COO_gpu"]),
    "inner_prod": ("Scalar_gpu", ["CSF3_gpu"] * 2),
    "inner_prod_coo": ("Scalar_gpu", ["COO3_gpu"] * 2),
}


@pytest.fixture(scope="module")
def gxx():
    path = shutil.which("g++")
    if path is None:
        pytest.skip("g++ not available")
    return path


@pytest.fixture(scope="module")
def libdir():
    from nacho_amd import _lib

    if not _lib.LIBRARY_PATH.exists():
        pytest.skip("libnacho_hip.so is not built")
    return _lib.LIBRARY_PATH.parent


@pytest.fixture(scope="module")
def hipgen(tmp_path_factory, gxx):
    out = tmp_path_factory.mktemp("hipgen")
    exe = out / "nacho_hipgen"
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
                    str(CODEGEN / "hipgen.cpp"), str(CODEGEN / "declarations.cpp"),
                    "-o", str(exe)], check=True)
    return exe


@pytest.fixture(scope="module")
def generated(hipgen, tmp_path_factory):
    out = tmp_path_factory.mktemp("generated")
    run = subprocess.run([str(hipgen), "--output-dir", str(out)], capture_output=True,
                         text=True)
    assert run.returncode == 0, run.stderr
    return out, run


def _compile_and_run(gxx, libdir, sources, includes, exe):
    cmd = [gxx, "-std=c++17", "-Wall", "-Werror"] + [f"-I{p}" for p in includes]
    cmd += [str(s) for s in sources] + ["-o", str(exe), f"-L{libdir}", "-lnacho_hip",
                                       f"-Wl,-rpath,{libdir}"]
    subprocess.run(cmd, check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True)


def test_every_implemented_declaration_is_generated(generated):
    out, run = generated
    entries = dict(re.findall(r"/(\w+)_gpu\.h \S+_gpu_nb\.cpp -> (\w+)", run.stdout))
    assert entries == EXPECTED
    for k in EXPECTED:
        assert (out / f"{k}_gpu.h").is_file() and (out / f"{k}_gpu_nb.cpp").is_file()
    for k, why in REFUSED.items():
        line = [x for x in run.stderr.splitlines() if f" {k}: " in x]
        assert len(line) == 1 and why in line[0], run.stderr
        assert not (out / f"{k}_gpu.h").exists() and not (out / f"{k}_gpu_nb.cpp").exists()
    assert sorted(p.name for p in out.iterdir()) == sorted(
        [f"{k}_gpu.h" for k in EXPECTED] + [f"{k}_gpu_nb.cpp" for k in EXPECTED])


def test_generated_namespace_matches_the_reference_signature(generated):
    """namespace <k>, index_t/value_t, <operand>_tensor_format templates with the generated
    field order (tensor.cpp:13-61), Z_tensor_format, and <k>_gpu_i32_f32 taking the operands
    by value in lexicographic order plus the two launch hints."""
    out, _ = generated
    h = (out / "spgemm_gpu.h").read_text()
    assert "namespace spgemm {" in h and "using index_t = int32_t;" in h
    b = h[h.index("struct b_tensor_format {"):]
    b = b[:b.index("};")]
    assert [ln.strip() for ln in b.splitlines()[1:]] == [
        "index_t dim_j_size;", "index_t dim_k_size;", "index_t *dim_k_offsets;",
        "index_t dim_k_length;", "index_t *dim_k_indices;", "value_t *values;", "index_t nnz;"]
    assert ("inline Z_tensor_format<index_t, value_t> spgemm_gpu_i32_f32("
            "const a_tensor_format<index_t, value_t> a, const b_tensor_format<index_t, value_t> b, "
            "const int32_t num_blocks, const int32_t threads_per_block)") in h
    coo = (out / "coo_add_gpu.h").read_text()
    a = coo[coo.index("struct a_tensor_format {"):]
    a = a[:a.index("};")]
    assert [ln.strip() for ln in a.splitlines()[1:]] == [
        "index_t dim_i_size;", "index_t dim_j_size;", "index_t dim_i_length;",
        "index_t *dim_i_indices;", "index_t dim_j_length;", "index_t *dim_j_indices;",
        "value_t *values;", "index_t nnz;"]
    s = (out / "sssmm_gpu.h").read_text()
    assert "nacho_gpu_sssmm_f32(&desc_a, &desc_b, &desc_c, &desc_result" in s


NAMED_UNSUPPORTED = r"""
#include <iostream>
#include "hipgen.hpp"
using namespace nacho_hipgen;

int main(int argc, char **argv) {
    if (!parse_command_line(argc, argv)) return 1;
    Format csf = Format::ordered({{"i", LevelFormat::Compressed_unique},
                                  {"j", LevelFormat::Compressed_unique},
                                  {"k", LevelFormat::Compressed_unique}}).named("CSF3");
    Expr s = Tensor::make(TensorType(csf, dType::Float32), "s");
    Expr t = Tensor::make(TensorType(csf, dType::Float32), "t");
    try {
        Kernel("csf_mul").expr(s * t).emit();
        Kernel("csf_add").expr(s + t).emit();
    } catch (const UnsupportedForm &e) {
        std::cerr << "nacho_hipgen: " << e.what() << "\n";
        return 1;
    }
    for (const auto &[name, reason] : refused()) std::cerr << "not generated: " << reason << "\n";
    return 0;
}
"""


def test_naming_an_unsupported_kernel_fails(gxx, tmp_path):
    """A declaration without a HIP kernel is listed as not generated, and naming it with
    --kernels is an error before anything is written."""
    src = tmp_path / "named.cpp"
    src.write_text(NAMED_UNSUPPORTED)
    exe = tmp_path / "named"
    subprocess.run([gxx, "-std=c++17", "-Wall", "-Werror", f"-I{CODEGEN}", str(src),
                    str(CODEGEN / "hipgen.cpp"), "-o", str(exe)], check=True)
    run = subprocess.run([str(exe), "--kernels", "csf_mul", "--output-dir",
                          str(tmp_path / "o")], capture_output=True, text=True)
    assert run.returncode == 1
    assert "csf_mul: no HIP kernel for a product of 2 operands in CSF3" in run.stderr
    assert not (tmp_path / "o").exists() or not any((tmp_path / "o").iterdir())
    run = subprocess.run([str(exe), "--output-dir", str(tmp_path / "p")], capture_output=True,
                         text=True)
    assert run.returncode == 0 and "not generated: csf_mul: no HIP kernel" in run.stderr
    assert sorted(p.name for p in (tmp_path / "p").iterdir()) == [
        "csf_add_gpu.h", "csf_add_gpu_nb.cpp"]


def test_kernel_selection_and_usage(hipgen, tmp_path):
    run = subprocess.run([str(hipgen), "--kernels", "csr_mul,spgemm", "--output-dir",
                          str(tmp_path)], capture_output=True, text=True)
    assert run.returncode == 0, run.stderr
    assert sorted(p.name for p in tmp_path.iterdir()) == [
        "csr_mul_gpu.h", "csr_mul_gpu_nb.cpp", "spgemm_gpu.h", "spgemm_gpu_nb.cpp"]
    bad = subprocess.run([str(hipgen), "--output-dir"], capture_output=True, text=True)
    assert bad.returncode == 1 and "usage:" in bad.stderr


def test_generated_headers_compile_link_and_reach_the_c_abi(generated, gxx, libdir, tmp_path):
    out, _ = generated
    lines = ["#include <cstdio>", "#include <stdexcept>"]
    lines += [f'#include "{k}_gpu.h"' for k in EXPECTED]
    lines += ["int main() {", "int bad = 0;"]
    # every entry point links
    lines += [f"bad += (void *)&{k}::{k}_gpu_i32_f32 == nullptr;" for k in EXPECTED]
    # calls with mismatched shapes come back as exceptions naming the kernel
    calls = {
        "csr_add": "csr_add::csr_add_gpu_i32_f32({4, 4}, {5, 4}, 256, 256)",
        "csr_mul": "csr_mul::csr_mul_gpu_i32_f32({4, 4}, {4, 5}, 256, 256)",
        "spgemm": "spgemm::spgemm_gpu_i32_f32({4, 3}, {5, 4}, 256, 256)",
        "sssmm": "sssmm::sssmm_gpu_i32_f32({4, 3}, {3, 4}, {4, 5}, 256, 256)",
        "coo_csr_add": "coo_csr_add::coo_csr_add_gpu_i32_f32({4, 4}, {5, 4}, 256, 256)",
        "inner_prod": "inner_prod::inner_prod_gpu_i32_f32({4, 4, 4}, {4, 5, 4}, 256, 256)",
        "inner_prod_coo":
            "inner_prod_coo::inner_prod_coo_gpu_i32_f32({4, 4, 4}, {4, 4, 5}, 256, 256)",
    }
    for k, call in calls.items():
        lines.append(f"try {{ (void){call}; ++bad; std::printf(\"{k} did not throw\\n\"); }}")
        lines.append('catch (const std::runtime_error &e) { std::printf("threw: %s\\n", e.what()); }')
    lines += ["return bad; }"]
    src = tmp_path / "headers.cpp"
    src.write_text("\n".join(lines) + "\n")
    run = _compile_and_run(gxx, libdir, [src], [REPO / "include", out], tmp_path / "headers")
    assert run.returncode == 0, run.stdout + run.stderr
    for k in calls:
        assert f"threw: {k}: nacho: invalid argument" in run.stdout, run.stdout


def test_generated_wrappers_compile_and_reach_the_c_abi(generated, gxx, libdir, tmp_path):
    out, _ = generated
    lines = ["#include <cstdio>", "#include <stdexcept>", '#include "nacho_types.h"']
    lines += [f"void register_{k}_gpu(nb::module_ &m);" for k in EXPECTED]
    lines += ["int main() {", "nb::module_ m;", "int bad = 0;"]
    lines += [f"register_{k}_gpu(m);" for k in EXPECTED]
    lines.append(f"bad += m.functions.size() != {len(EXPECTED)};")
    for k, (res, args) in SIGNATURES.items():
        lines.append(f'bad += m.functions.count("gpu_{k}_f32") != 1;')
    # csr_add and spgemm with mismatched shapes, through the Python-facing signatures
    lines += [
        "using Bin = CSR_gpu (*)(const CSR_gpu &, const CSR_gpu &, int32_t, int32_t);",
        "CSR_gpu x{}, y{};",
        "x.shape = nacho::make_shape<2>({4, 4}); y.shape = nacho::make_shape<2>({5, 4});",
        'for (const char *name : {"gpu_csr_add_f32", "gpu_csr_mul_f32", "gpu_spgemm_f32"}) {',
        "  auto f = reinterpret_cast<Bin>(m.functions.at(name));",
        '  try { (void)f(x, y, 256, 256); ++bad; std::printf("%s did not throw\\n", name); }',
        '  catch (const std::runtime_error &e) { std::printf("threw: %s\\n", e.what()); }',
        "}",
        "return bad; }",
    ]
    src = tmp_path / "wrappers.cpp"
    src.write_text("\n".join(lines) + "\n")
    sources = [src] + [out / f"{k}_gpu_nb.cpp" for k in EXPECTED]
    run = _compile_and_run(gxx, libdir, sources, [REPO / "include", out, DOUBLE],
                           tmp_path / "wrappers")
    assert run.returncode == 0, run.stdout + run.stderr
    for k in ("csr_add", "csr_mul", "spgemm"):
        assert f"threw: {k}: nacho: invalid argument" in run.stdout, run.stdout


CUSTOM = r"""
#include <iostream>
#include "hipgen.hpp"
using namespace nacho_hipgen;

static void attempt(const char *name, Expr e, const std::string &dir,
                    std::vector<std::string> order = {}) {
    try {
        Declaration d = analyse(name, e);
        if (!order.empty()) d.ordering = order;
        Emitted out = emit_gpu(d, dir);
        std::cout << "ok " << name << " " << out.entry_point << "\n";
    } catch (const UnsupportedForm &err) {
        std::cout << "refused " << err.what() << "\n";
    }
}

int main(int argc, char **argv) {
    const std::string dir = argv[1];
    auto csr = [](const char *r, const char *c) {
        return TensorType(Format::ordered({{r, LevelFormat::Dense},
                                           {c, LevelFormat::Compressed_unique}}).named("CSR"),
                          dType::Float32);
    };
    Format csf = Format::ordered({{"i", LevelFormat::Compressed_unique},
                                  {"j", LevelFormat::Compressed_unique},
                                  {"k", LevelFormat::Compressed_unique}}).named("CSF3");
    Expr p = Tensor::make(csr("x", "y"), "p"), q = Tensor::make(csr("x", "y"), "q");
    attempt("merge_xy", q + p, dir);
    Expr a = Tensor::make(csr("l", "m"), "a"), b = Tensor::make(csr("m", "n"), "b");
    attempt("chain", Sum::make("m", b * a), dir);
    Expr c = Tensor::make(csr("l", "n"), "c");
    attempt("masked", Sum::make("m", c * b * a), dir, {"c", "b", "a"});
    Expr s = Tensor::make(TensorType(csf, dType::Float32), "s");
    Expr t = Tensor::make(TensorType(csf, dType::Float32), "t");
    attempt("csf_mul", s * t, dir);
    Expr w = Tensor::make(TensorType(csr("x", "y").format, dType::Float64), "w");
    attempt("double_add", p + w, dir);
    attempt("same_twice", p + p, dir);
    attempt("mixed", (p + q) * Tensor::make(csr("x", "y"), "r"), dir);
    attempt("transposed", p + Tensor::make(csr("y", "x"), "r"), dir);
    attempt("no_shared_index", Sum::make("z", a * b), dir);
    attempt("trace_like", Sum::make("m", a * Tensor::make(csr("m", "l"), "r")), dir);
    attempt("copy", p, dir);
    attempt("four_way", p + q + Tensor::make(csr("x", "y"), "r") +
                            Tensor::make(csr("x", "y"), "u"), dir);
    return 0;
}
"""


def test_declarations_map_by_structure_not_by_name(gxx, libdir, tmp_path):
    gen = tmp_path / "gen"
    gen.mkdir()
    src = tmp_path / "custom.cpp"
    src.write_text(CUSTOM)
    exe = tmp_path / "custom"
    subprocess.run([gxx, "-std=c++17", "-Wall", "-Werror", f"-I{CODEGEN}", str(src),
                    str(CODEGEN / "hipgen.cpp"), "-o", str(exe)], check=True)
    run = subprocess.run([str(exe), str(gen)], capture_output=True, text=True, check=True)
    got = run.stdout.splitlines()
    assert "ok merge_xy nacho_gpu_csr_add_f32" in got
    assert "ok chain nacho_gpu_spgemm_f32" in got
    assert "ok masked nacho_gpu_sssmm_f32" in got
    expect_refused = {
        "csf_mul": "no HIP kernel for a product of 2 operands in CSF3",
        "double_add": "is not float32",
        "same_twice": "appears twice",
        "mixed": "mixed operators",
        "transposed": "share their index order",
        "no_shared_index": "more than one operand without the reduced index",
        "trace_like": "result index repeats",
        "copy": "a single tensor",
        "four_way": "no HIP kernel for a sum of 4 operands",
    }
    for k, why in expect_refused.items():
        line = [x for x in got if x.startswith(f"refused {k}: ")]
        assert len(line) == 1 and why in line[0], (k, got)
    # operands keep the declaration's index names; the entry point's argument order follows
    # the roles (row factor, column factor, mask), the parameters the declared ordering
    h = (gen / "chain_gpu.h").read_text()
    assert "index_t *dim_n_offsets;" in h and "dim_l_size" in h
    assert "nacho_gpu_spgemm_f32(&desc_a, &desc_b, &desc_result" in h
    m = (gen / "masked_gpu.h").read_text()
    assert ("masked_gpu_i32_f32(const c_tensor_format<index_t, value_t> c, "
            "const b_tensor_format<index_t, value_t> b, "
            "const a_tensor_format<index_t, value_t> a,") in m
    assert "nacho_gpu_sssmm_f32(&desc_a, &desc_b, &desc_c, &desc_result" in m
    # and the renamed declaration compiles and reaches csr_add
    drv = tmp_path / "drv.cpp"
    drv.write_text('#include <cstdio>\n#include <stdexcept>\n#include "merge_xy_gpu.h"\n'
                   "int main() { try { (void)merge_xy::merge_xy_gpu_i32_f32({4, 4}, {4, 5}, 256,"
                   " 256); return 1; } catch (const std::runtime_error &e) {"
                   ' std::printf("%s\\n", e.what()); } return 0; }\n')
    run = _compile_and_run(gxx, libdir, [drv], [REPO / "include", gen], tmp_path / "drv")
    assert run.returncode == 0 and "merge_xy: nacho: invalid argument" in run.stdout, run.stdout
