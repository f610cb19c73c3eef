"""The C ABI library loads and exports every function include/nacho_hip.h declares.

Runs on the CPU: only argument-validation paths are called (they return before any HIP
call), no kernels.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "nacho_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nacho_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from nacho_amd import _lib

    return _lib.load()


def test_header_declares_entry_points():
    names = declared_functions()
    assert "nacho_gpu_csr_add_f32" in names and "nacho_gpu_csr_mul_f32" in names
    assert "nacho_free" in names and "nacho_error_string" in names


def test_library_exports_every_declared_symbol(lib):
    from nacho_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (nacho_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for name in declared_functions():
        assert getattr(lib, name) is not None


def test_python_bindings_cover_every_gpu_entry_point():
    from nacho_amd import _lib

    gpu = [n for n in declared_functions() if n.startswith("nacho_gpu_")]
    bound = (set(_lib.ENTRY_POINTS) | set(_lib.ENTRY_POINTS_3) | set(_lib.ENTRY_POINTS_NOALLOC)
             | set(_lib.ENTRY_POINTS_MIXED))
    assert set(gpu) <= bound, set(gpu) - bound


def test_error_strings(lib):
    from nacho_amd import _lib

    assert _lib.error_string(0) == "success"
    assert "invalid" in _lib.error_string(-1)
    assert "int32" in _lib.error_string(-2)
    assert lib.nacho_version().decode().startswith("nacho-mi355x")


def test_invalid_arguments_rejected_without_a_device(lib):
    from nacho_amd import _lib

    z = _lib.CsrDesc()
    good = _lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), 0, None, None, 0)
    fn = lib.nacho_gpu_csr_add_f32
    # null operand
    assert fn(None, ctypes.byref(good), ctypes.byref(z), 256, 256, None, None) == -1
    # null result
    assert fn(ctypes.byref(good), ctypes.byref(good), None, 256, 256, None, None) == -1
    # bad launch hints (the reference's num_blocks / threads_per_block)
    assert fn(ctypes.byref(good), ctypes.byref(good), ctypes.byref(z), 0, 256, None, None) == -1
    assert fn(ctypes.byref(good), ctypes.byref(good), ctypes.byref(z), 256, -1, None, None) == -1
    # shape mismatch
    other = _lib.CsrDesc(5, 4, ctypes.c_void_p(0x1000), 0, None, None, 0)
    assert fn(ctypes.byref(good), ctypes.byref(other), ctypes.byref(z), 256, 256, None,
              None) == -1
    # missing crd with a positive length
    bad = _lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), 3, None, None, 3)
    assert lib.nacho_gpu_csr_mul_f32(ctypes.byref(bad), ctypes.byref(good), ctypes.byref(z),
                                     256, 256, None, None) == -1
    # int32 overflow of the work count is refused before any allocation
    huge = _lib.CsrDesc(2**31 - 2, 4, ctypes.c_void_p(0x1000), 2**30, ctypes.c_void_p(0x2000),
                        ctypes.c_void_p(0x3000), 2**30)
    assert fn(ctypes.byref(huge), ctypes.byref(huge), ctypes.byref(z), 256, 256, None,
              None) == -2
    assert z.dim_j_offsets is None and z.nnz == 0


def test_device_copy_rejects_misaligned_buffers_without_a_device(lib):
    v = ctypes.c_void_p
    assert lib.nacho_device_copy(v(0x1000), v(0x2000), 0, None) == 0  # nothing to copy
    assert lib.nacho_device_copy(None, v(0x2000), 32, None) == -1
    assert lib.nacho_device_copy(v(0x1000), None, 32, None) == -1
    assert lib.nacho_device_copy(v(0x1004), v(0x2000), 32, None) == -1  # dst misaligned
    assert lib.nacho_device_copy(v(0x1000), v(0x2008), 32, None) == -1  # src misaligned
    assert lib.nacho_device_copy(v(0x1000), v(0x2000), 24, None) == -1  # not 16-byte units


def test_csr_add_3_arguments_rejected_without_a_device(lib):
    """The fused three-way union checks its third operand like the other two, and refuses
    a total item count past int32 before any allocation."""
    from nacho_amd import _lib

    z = _lib.CsrDesc()
    good = _lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), 0, None, None, 0)
    other = _lib.CsrDesc(4, 5, ctypes.c_void_p(0x1000), 0, None, None, 0)
    fn = lib.nacho_gpu_csr_add_3_f32
    r = ctypes.byref
    assert fn(r(good), r(good), None, r(z), 256, 256, None, None) == -1
    assert fn(r(good), r(good), r(other), r(z), 256, 256, None, None) == -1
    assert fn(r(good), r(good), r(good), None, 256, 256, None, None) == -1
    assert fn(r(good), r(good), r(good), r(z), 256, 0, None, None) == -1
    third = 2**30  # three operands of 2^30 entries: 3 * 2^30 items overflow int32
    huge = _lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), third, ctypes.c_void_p(0x2000),
                        ctypes.c_void_p(0x3000), third)
    assert fn(r(huge), r(huge), r(huge), r(z), 256, 256, None, None) == -2
    assert z.dim_j_offsets is None and z.nnz == 0


def test_struct_layouts_match_the_header():
    """ctypes mirrors of the descriptors have the C layout (offsets of pointer fields)."""
    from nacho_amd import _lib

    assert _lib.CsrDesc.dim_j_offsets.offset == 8
    assert _lib.CsrDesc.dim_j_indices.offset == 24
    assert ctypes.sizeof(_lib.CsrDesc) == 48
    assert ctypes.sizeof(_lib.Csr64Desc) == 48


def test_every_descriptor_layout_matches_the_c_compiler(tmp_path):
    """Field offsets and sizes of every ctypes descriptor equal what gcc computes from
    include/nacho_hip.h."""
    import shutil
    import subprocess

    from nacho_amd import _lib

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    pairs = {"nacho_csr": _lib.CsrDesc, "nacho_csr64": _lib.Csr64Desc,
             "nacho_coo": _lib.CooDesc, "nacho_coo3": _lib.Coo3Desc,
             "nacho_dcsr": _lib.DcsrDesc, "nacho_csf3": _lib.Csf3Desc,
             "nacho_scalar": _lib.ScalarDesc,
             "nacho_coo2d_host": _lib.Coo2dHost, "nacho_coo3d_host": _lib.Coo3dHost}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "nacho_hip.h"',
             "int main(void) {"]
    for cname, desc in pairs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in desc._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    include = Path(__file__).resolve().parent.parent / "include"
    subprocess.run([gcc, f"-I{include}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        cname, field, value = line.split()
        desc = pairs[cname]
        got = ctypes.sizeof(desc) if field == "size" else getattr(desc, field).offset
        assert got == int(value), f"{cname}.{field}: ctypes {got}, C {value}"


def test_cpp_shim_matches_the_generated_signatures(tmp_path):
    """include/nacho_hip.hpp compiles as C++17, its format templates have the C descriptors'
    layout field by field, every generated-style entry point links against the library, and
    a failing call (mismatched shapes, rejected before any HIP call) throws."""
    import shutil

    from nacho_amd import _lib

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    pairs = {  # shim format -> (C descriptor, {shim field: C field})
        "nacho_hip::csr_ij<int32_t, float>": ("nacho_csr", {}),
        "nacho_hip::csr_jk<int32_t, float>": ("nacho_csr", {
            "dim_j_size": "dim_i_size", "dim_k_size": "dim_j_size",
            "dim_k_offsets": "dim_j_offsets", "dim_k_length": "dim_j_length",
            "dim_k_indices": "dim_j_indices"}),
        "nacho_hip::csr_ik<int32_t, float>": ("nacho_csr", {
            "dim_k_size": "dim_j_size", "dim_k_offsets": "dim_j_offsets",
            "dim_k_length": "dim_j_length", "dim_k_indices": "dim_j_indices"}),
        "nacho_hip::dcsr_ij<int32_t, float>": ("nacho_dcsr", {}),
        "nacho_hip::csf3_ijk<int32_t, float>": ("nacho_csf3", {}),
        "nacho_hip::coo_ij<int32_t, float>": ("nacho_coo", {}),
        "nacho_hip::coo3_ijk<int32_t, float>": ("nacho_coo3", {}),
        "nacho_hip::scalar<int32_t, float>": ("nacho_scalar", {}),
    }
    descs = {"nacho_csr": _lib.CsrDesc, "nacho_dcsr": _lib.DcsrDesc,
             "nacho_csf3": _lib.Csf3Desc, "nacho_coo": _lib.CooDesc, "nacho_coo3": _lib.Coo3Desc,
             "nacho_scalar": _lib.ScalarDesc}
    lines = ["#include <cstddef>", "#include <cstdio>", '#include "nacho_hip.hpp"',
             "int main() {", "int bad = 0;"]
    for shim, (cname, rename) in pairs.items():
        inverse = {v: k for k, v in rename.items()}
        lines.append(f"{{ using F = {shim}; static_assert(sizeof(F) == sizeof({cname}), \"size\");")
        for field, _ in descs[cname]._fields_:
            sf = inverse.get(field, field)
            lines.append(f"if (offsetof(F, {sf}) != offsetof({cname}, {field})) "
                         f"{{ std::printf(\"{shim}.{sf}\\n\"); ++bad; }}")
        lines.append("}")
    lines += [
        "void *fns[] = {",
        "  (void *)&csr_add::csr_add_gpu_i32_f32, (void *)&csr_mul::csr_mul_gpu_i32_f32,",
        "  (void *)&csr_add_3::csr_add_3_gpu_i32_f32, (void *)&coo_add::coo_add_gpu_i32_f32,",
        "  (void *)&coo_mul::coo_mul_gpu_i32_f32, (void *)&coo3d_add::coo3d_add_gpu_i32_f32,",
        "  (void *)&dcsr_add::dcsr_add_gpu_i32_f32, (void *)&dcsr_mul::dcsr_mul_gpu_i32_f32,",
        "  (void *)&dcsr_mul_without_recursive_partitioning::"
        "dcsr_mul_without_recursive_partitioning_gpu_i32_f32,",
        "  (void *)&csf_add::csf_add_gpu_i32_f32, (void *)&spgemm::spgemm_gpu_i32_f32,",
        "  (void *)&sssmm::sssmm_gpu_i32_f32, (void *)&coo_csr_add::coo_csr_add_gpu_i32_f32,",
        "  (void *)&inner_prod::inner_prod_gpu_i32_f32,",
        "  (void *)&inner_prod_coo::inner_prod_coo_gpu_i32_f32};",
        "for (void *f : fns) bad += f == nullptr;",
        "csr_add::a_tensor_format<int32_t, float> a{4, 4, nullptr, 0, nullptr, nullptr, 0};",
        "csr_add::b_tensor_format<int32_t, float> b{5, 4, nullptr, 0, nullptr, nullptr, 0};",
        "try { (void)csr_add::csr_add_gpu_i32_f32(a, b, 256, 256); ++bad; std::printf(\"no throw\\n\"); }",
        "catch (const std::runtime_error &e) { std::printf(\"threw: %s\\n\", e.what()); }",
        "return bad; }",
    ]
    src = tmp_path / "shim.cpp"
    src.write_text("\n".join(lines))
    exe = tmp_path / "shim"
    include = REPO / "include"
    libdir = _lib.LIBRARY_PATH.parent
    subprocess.run([gxx, "-std=c++17", f"-I{include}", str(src), "-o", str(exe),
                    f"-L{libdir}", "-lnacho_hip", f"-Wl,-rpath,{libdir}"], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "threw: csr_add: " in run.stdout


class _CountingAllocator:
    """A caller allocator that hands out fake device addresses and returns NULL from the
    `fail_at`-th request on; it records every pointer handed out and every release."""

    def __init__(self, fail_at):
        from nacho_amd import _lib

        self.fail_at = fail_at
        self.handed, self.released, self.requests = [], [], 0
        self._next = 0x10000000

        def allocate(ctx, nbytes, stream):
            self.requests += 1
            if self.requests >= self.fail_at:
                return None
            p = self._next
            self._next += (nbytes + 0xFFF) & ~0xFFF or 0x1000
            self.handed.append(p)
            return p

        def release(ctx, ptr, stream):
            self.released.append(ptr)

        self.struct = _lib.Allocator(None, _lib.Allocator._fields_[1][1](allocate),
                                     _lib.Allocator._fields_[2][1](release))


@pytest.mark.parametrize("entry", ["nacho_gpu_csr_add_f32", "nacho_gpu_csr_mul_f32"])
@pytest.mark.parametrize("fail_at", [1, 2, 3])
def test_allocator_failure_releases_everything(lib, entry, fail_at):
    """The caller's allocator returning NULL gives NACHO_ERR_OUT_OF_MEMORY, a zeroed result
    and a release of every buffer the call had obtained (the result arrays are the first
    three requests, before any HIP call)."""
    from nacho_amd import _lib

    alloc = _CountingAllocator(fail_at)
    a = _lib.CsrDesc(8, 8, ctypes.c_void_p(0x1000), 5, ctypes.c_void_p(0x2000),
                     ctypes.c_void_p(0x3000), 5)
    z = _lib.CsrDesc()
    rc = getattr(lib, entry)(ctypes.byref(a), ctypes.byref(a), ctypes.byref(z), 256, 256, None,
                             ctypes.byref(alloc.struct))
    assert rc == -3, _lib.error_string(rc)
    assert alloc.requests == fail_at
    assert sorted(alloc.handed) == sorted(alloc.released)
    assert z.dim_j_offsets is None and z.dim_j_indices is None and z.values is None
    assert z.nnz == 0 and z.dim_j_length == 0


def test_validate_csr_rejects_host_visible_faults(lib):
    """nacho_validate_csr refuses null pointers, negative sizes and nnz != dim_j_length
    before touching the device."""
    from nacho_amd import _lib

    r = ctypes.byref
    fn = lib.nacho_validate_csr
    assert fn(None, None) == -1
    assert fn(r(_lib.CsrDesc(4, 4, None, 0, None, None, 0)), None) == -1
    assert fn(r(_lib.CsrDesc(-1, 4, ctypes.c_void_p(0x1000), 0, None, None, 0)), None) == -1
    assert fn(r(_lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), 3, None, None, 3)), None) == -1
    assert fn(r(_lib.CsrDesc(4, 4, ctypes.c_void_p(0x1000), 3, ctypes.c_void_p(0x2000), None,
                             2)), None) == -1


def test_record_stream_rejects_unknown_buffers(lib):
    """nacho_record_stream only accepts live buffers of the library's allocator."""
    assert lib.nacho_record_stream(None, None) == -1
    assert lib.nacho_record_stream(ctypes.c_void_p(0x1234000), None) == -1
