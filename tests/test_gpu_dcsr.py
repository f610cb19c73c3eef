"""GPU parity of dcsr_add / dcsr_mul (two CSR level merges) against the oracle, bit-exact."""

import numpy as np
import pytest
import scipy.sparse as sp
import torch

from oracle import oracle
from tests.test_oracle_dcsr import assert_dcsr_equal, dcsr_of, random_dcsr

pytestmark = pytest.mark.gpu

ENTRY = {"add": "gpu_dcsr_add_f32", "mul": "gpu_dcsr_mul_f32",
         "mul_nrp": "gpu_dcsr_mul_without_recursive_partitioning_f32"}


def to_gpu(levels, val, shape, device):
    import nacho_amd

    ci, pj, cj = levels
    t = lambda x, d: torch.from_numpy(np.ascontiguousarray(x)).to(dtype=d, device=device)  # noqa: E731
    return nacho_amd.DCSR_gpu(t(ci, torch.int32), t(pj, torch.int32), t(cj, torch.int32),
                              t(val, torch.float32), torch.tensor(shape, dtype=torch.int32))


def run(op, shape, a, b, device):
    import nacho_amd

    print(f"[gpu] dcsr {op} shape={shape} rows=({len(a[0][0])},{len(b[0][0])}) "
          f"nnz=({len(a[1])},{len(b[1])})", flush=True)
    z = getattr(nacho_amd, ENTRY[op])(to_gpu(*a, shape, device), to_gpu(*b, shape, device))
    torch.cuda.synchronize()
    assert tuple(z.shape.tolist()) == tuple(shape)
    levels = tuple(getattr(z, n).cpu().numpy()
                   for n in ("dim_i_indices", "dim_j_offsets", "dim_j_indices"))
    return levels, z.values.cpu().numpy()


def want(op, a, b):
    return oracle.port_dcsr_binary("add" if op == "add" else "mul", *a, *b)


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(5))
def test_random(gpu, op, seed):
    rng = np.random.default_rng(500 + seed)
    rows = int(rng.choice([1, 9, 4000, 300000]))
    cols = int(rng.choice([1, 17, 5000, 1 << 20]))
    density = float(rng.choice([1e-5, 1e-3, 0.05])) if rows * cols < 1e10 else 1e-5
    a, b = (random_dcsr(rng, rows, cols, density) for _ in range(2))
    assert_dcsr_equal(run(op, (rows, cols), a, b, gpu), want(op, a, b), f"{op} seed={seed}")


@pytest.mark.parametrize("op", ["add", "mul", "mul_nrp"])
def test_reference_smoke_case(gpu, op):
    rng = np.random.default_rng(0)
    shape = (200, 180)
    ms = [sp.random(*shape, density=0.05, format="csr", dtype=np.float32,
                    random_state=rng.integers(2**31)) for _ in range(2)]
    a, b = dcsr_of(ms[0]), dcsr_of(ms[1])
    assert_dcsr_equal(run(op, shape, a, b, gpu), want(op, a, b), f"smoke {op}")


@pytest.mark.parametrize("op", ["add", "mul"])
def test_empty_operands(gpu, op):
    e = ((np.zeros(0, np.int32), np.zeros(1, np.int32), np.zeros(0, np.int32)),
         np.zeros(0, np.float32))
    b = random_dcsr(np.random.default_rng(1), 60, 50, 0.1)
    assert_dcsr_equal(run(op, (60, 50), e, b, gpu), want(op, e, b), "a empty")
    assert_dcsr_equal(run(op, (60, 50), b, e, gpu), want(op, b, e), "b empty")
    assert_dcsr_equal(run(op, (60, 50), e, e, gpu), want(op, e, e), "both empty")


def test_mul_keeps_rows_with_empty_intersection(gpu):
    a = ((np.array([1, 4, 6], np.int32), np.array([0, 2, 3, 4], np.int32),
          np.array([0, 5, 2, 9], np.int32)), np.array([1, 2, 3, 4], np.float32))
    b = ((np.array([1, 2, 6], np.int32), np.array([0, 1, 2, 4], np.int32),
          np.array([3, 7, 1, 9], np.int32)), np.array([5, 6, 7, 8], np.float32))
    got = run("mul", (8, 10), a, b, gpu)
    assert list(got[0][0]) == [1, 6] and list(got[0][1]) == [0, 0, 1]
    assert_dcsr_equal(got, want("mul", a, b), "empty fibre kept")
    assert_dcsr_equal(run("add", (8, 10), a, b, gpu), want("add", a, b), "add")


@pytest.mark.parametrize("op", ["add", "mul"])
def test_disjoint_and_identical_rows(gpu, op):
    rng = np.random.default_rng(9)
    m = sp.random(5000, 3000, density=0.01, format="csr", dtype=np.float32, random_state=3)
    even = sp.diags((np.arange(5000) % 2 == 0).astype(np.float32)) @ m
    odd = sp.diags((np.arange(5000) % 2 == 1).astype(np.float32)) @ m
    a, b = dcsr_of(sp.csr_matrix(even)), dcsr_of(sp.csr_matrix(odd))
    assert_dcsr_equal(run(op, (5000, 3000), a, b, gpu), want(op, a, b), "disjoint rows")
    c = (a[0], rng.uniform(-1, 1, len(a[1])).astype(np.float32))
    assert_dcsr_equal(run(op, (5000, 3000), a, c, gpu), want(op, a, c), "same structure")


@pytest.mark.parametrize("op", ["add", "mul"])
def test_c2_rows_as_dcsr(gpu, op):
    """The C2 (add) / C3 (mul) generators (2^20 rows, ~16.7M nnz per operand), rows
    compressed: most Zipf rows are empty."""
    from nacho_amd import synth

    rows = cols = 1 << 20
    ops = synth.c2_operands() if op == "add" else synth.c3_operands()
    mats = [dcsr_of(sp.csr_matrix((val, crd, pos), shape=(rows, cols)))
            for pos, crd, val in ops]
    assert_dcsr_equal(run(op, (rows, cols), *mats, gpu), want(op, *mats), f"C2 dcsr {op}")


def _hypersparse(rng, rows, cols, n_rows, shared=None):
    """DCSR levels with n_rows stored rows scattered over [0, rows) (plus the rows in
    `shared`), 1-5 entries each."""
    ids = set(rng.choice(rows, size=n_rows, replace=False).tolist())
    if shared is not None:
        ids |= set(shared)
    ci = np.array(sorted(ids), np.int32)
    lens = rng.integers(1, 6, len(ci))
    pj = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cj = np.concatenate([np.sort(rng.choice(cols, size=int(k), replace=False)) for k in lens])
    return (ci, pj, cj.astype(np.int32)), rng.uniform(-1, 1, len(cj)).astype(np.float32)


@pytest.mark.parametrize("op", ["add", "mul"])
def test_hypersparse_rows(gpu, op):
    """A row extent of 2^30 with a few thousand stored rows per operand (half of them shared,
    some with an empty column intersection): nothing may scale with the row extent."""
    rng = np.random.default_rng(31)
    rows, cols = 1 << 30, 64
    shared = rng.choice(rows, size=1500, replace=False).tolist()
    a = _hypersparse(rng, rows, cols, 1500, shared)
    b = _hypersparse(rng, rows, cols, 1500, shared)
    assert_dcsr_equal(run(op, (rows, cols), a, b, gpu), want(op, a, b), f"hypersparse {op}")
