"""The HIP generator behind the reference's own declaration API (nacho_amd/codegen/reference_hook).

The hook is what the GPU branch of the reference's Kernel::emit calls (src/Kernel.cpp:106-130):
it converts the reference's expression nodes (include/Frontend.h:73-116) to the generator's
and emits the GPU target.  Here it is compiled against the reference's headers, with the
reference's expression front end and output helpers built from their own sources where they
lie (src/Frontend.cpp, Format.cpp, Printer.cpp, Visitor.cpp, Mutator.cpp, CIN.cpp, Seq.cpp,
llir/*.cpp, backend/output.cpp, backend/generate_bindings.cpp), and linked with the
reference's unchanged declaration file compiler.cpp.  The program it makes must write, for
every GPU declaration there, exactly the files nacho_hipgen writes.  A second program
declares kernels through the same API with options the reference offers (operand order,
Python name, result name, targets) and forms without a HIP kernel.  Skipped where the
reference tree is absent (the GPU machine); nothing of the reference is copied.
"""

import concurrent.futures
import filecmp
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CODEGEN = REPO / "nacho_amd" / "codegen"
HOOK = CODEGEN / "reference_hook"
REFERENCE = Path("/root/reference")
FRONT_END = ["Frontend", "Format", "Printer", "Visitor", "Mutator", "CIN", "Seq",
             "llir/Function", "llir/LLIR", "backend/output", "backend/generate_bindings"]

pytestmark = pytest.mark.skipif(not (REFERENCE / "compiler.cpp").exists() or
                                shutil.which("g++") is None,
                                reason="the reference tree (or g++) is not here")


def _compile_all(sources, out):
    """Objects of `sources` (C++20, the reference's include directory and the generator's)."""
    gxx = shutil.which("g++")
    flags = ["-std=c++20", "-O1", f"-I{REFERENCE / 'include'}", f"-I{CODEGEN}", f"-I{HOOK}"]

    def one(i_src):
        i, src = i_src
        obj = out / f"{i}_{Path(src).stem}.o"
        subprocess.run([gxx, *flags, "-c", str(src), "-o", str(obj)], check=True,
                       capture_output=True, text=True)
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=6) as pool:
        return list(pool.map(one, enumerate(sources)))


@pytest.fixture(scope="module")
def common_objects(tmp_path_factory):
    out = tmp_path_factory.mktemp("reference_hook_objs")
    sources = [REFERENCE / "src" / f"{name}.cpp" for name in FRONT_END]
    sources += [HOOK / "gpu_target.cpp", HOOK / "kernel_emit.cpp", CODEGEN / "hipgen.cpp"]
    return _compile_all(sources, out)


def _link(objects, main_source, out):
    exe = out / "generator"
    main_obj = _compile_all([main_source], out)
    subprocess.run([shutil.which("g++"), *map(str, objects), *map(str, main_obj), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


@pytest.fixture(scope="module")
def nacho_hipgen(tmp_path_factory):
    from nacho_amd import build

    return build.build_codegen()


def test_reference_compiler_cpp_generates_what_nacho_hipgen_does(common_objects, nacho_hipgen,
                                                                 tmp_path):
    exe = _link(common_objects, REFERENCE / "compiler.cpp", tmp_path)
    ref_out, own_out = tmp_path / "from_reference", tmp_path / "from_hipgen"
    run = subprocess.run([str(exe), "--output-dir", str(ref_out)], capture_output=True,
                         text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    subprocess.run([str(nacho_hipgen), "--output-dir", str(own_out)], check=True,
                   capture_output=True, text=True)
    names = sorted(p.name for p in ref_out.iterdir())
    assert names == sorted(p.name for p in own_out.iterdir())
    assert len(names) == 30  # 15 GPU declarations, a header and a wrapper each
    for name in names:
        assert filecmp.cmp(ref_out / name, own_out / name, shallow=False), name
    # --kernels selects through the same API
    sel = tmp_path / "selected"
    subprocess.run([str(exe), "--kernels", "spgemm,csr_mul", "--output-dir", str(sel)],
                   check=True, capture_output=True, text=True)
    assert sorted(p.name for p in sel.iterdir()) == [
        "csr_mul_gpu.h", "csr_mul_gpu_nb.cpp", "spgemm_gpu.h", "spgemm_gpu_nb.cpp"]


def test_reference_api_options_and_refusals(common_objects, tmp_path):
    exe = _link(common_objects, Path(__file__).parent / "codegen_ref" / "declare_extra.cpp",
                tmp_path)
    out = tmp_path / "out"
    run = subprocess.run([str(exe), "--output-dir", str(out)], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert sorted(p.name for p in out.iterdir()) == [
        "plus_qp_gpu.h", "plus_qp_gpu_nb.cpp", "times_gpu.h", "times_gpu_nb.cpp"]
    header = (out / "plus_qp_gpu.h").read_text()
    # operands in the declared order, the result named W, the entry point chosen by structure
    assert "W_tensor_format" in header and "nacho_gpu_csr_add_f32" in header
    sig = header[header.index("plus_qp_gpu_i32_f32("):]
    assert sig.index("q_tensor_format") < sig.index("p_tensor_format")
    assert '"gpu_plus_qp"' in (out / "plus_qp_gpu_nb.cpp").read_text()
    assert "nacho_gpu_csr_mul_f32" in (out / "times_gpu.h").read_text()
    refused = [line for line in run.stdout.splitlines() if line.startswith("refused ")]
    assert len(refused) == 2, run.stdout
    assert refused[0].startswith("refused broadcast: a broadcast")
    assert refused[1].startswith("refused mixed_sum: ")
    named = subprocess.run([str(exe), "--kernels", "broadcast", "--output-dir",
                            str(tmp_path / "named")], capture_output=True, text=True)
    assert named.returncode == 1 and "broadcast" in named.stdout
