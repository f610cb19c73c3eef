"""GPU parity of coo_csr_add (CSR a + COO b -> CSR, reference compiler.cpp:122) against the
oracle, bit-exact: the result is csr_add of a and b converted to CSR (values one binary32
add where both hold a coordinate, copies otherwise)."""

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import assert_csr_equal, check_csr_invariants, random_csr
from tests.test_gpu_csr import from_gpu, to_gpu

pytestmark = pytest.mark.gpu


def run(a, b, rows, cols, device):
    import nacho_amd

    print(f"[gpu] coo_csr_add rows={rows} cols={cols} nnz=({len(a[1])},{len(b[1])})",
          flush=True)
    pos, crd, val = (np.asarray(x) for x in b)
    bi = np.repeat(np.arange(rows, dtype=np.int32), np.diff(pos))
    bc = nacho_amd.COO_gpu(torch.from_numpy(bi).to(device),
                           torch.from_numpy(np.asarray(crd, np.int32)).to(device),
                           torch.from_numpy(np.asarray(val, np.float32)).to(device),
                           torch.tensor([rows, cols], dtype=torch.int32))
    z = nacho_amd.gpu_coo_csr_add_f32(to_gpu(a, rows, cols, device), bc)
    assert isinstance(z, nacho_amd.CSR_gpu) and tuple(z.shape.tolist()) == (rows, cols)
    return from_gpu(z)


@pytest.mark.parametrize("seed", range(6))
def test_random(gpu, seed):
    rng = np.random.default_rng(700 + seed)
    rows, cols = int(rng.choice([1, 17, 1000, 50000])), int(rng.choice([1, 40, 30000]))
    density = float(rng.choice([0.0, 0.001, 0.05, 0.3]))
    a, b = random_csr(rng, rows, cols, density), random_csr(rng, rows, cols, density)
    got = run(a, b, rows, cols, gpu)
    assert_csr_equal(got, oracle.closed_csr_binary("add", rows, cols, *a, *b), f"seed={seed}")
    check_csr_invariants(got[0], got[1], rows, cols)


def test_reference_smoke_case(gpu):
    """tests/smoke.py case_coo_csr_add: two 200 x 180 random CSR at density 0.05, the right
    one passed as COO; compared with scipy a + b."""
    import scipy.sparse as sp

    rng = np.random.default_rng(0)

    def random_sp():
        m = sp.random(200, 180, density=0.05, format="csr", dtype=np.float32,
                      random_state=int(rng.integers(2**31)))
        m.sum_duplicates()
        m.sort_indices()
        return m

    a, b = random_sp(), random_sp()
    ta = (a.indptr.astype(np.int32), a.indices.astype(np.int32), a.data.astype(np.float32))
    tb = (b.indptr.astype(np.int32), b.indices.astype(np.int32), b.data.astype(np.float32))
    got = run(ta, tb, 200, 180, gpu)
    want = (a + b).tocsr()
    want.sort_indices()
    assert np.array_equal(got[0], want.indptr) and np.array_equal(got[1], want.indices)
    assert np.allclose(got[2], want.data, rtol=1e-6, atol=0)
    assert_csr_equal(got, oracle.port_csr_binary("add", 200, *ta, *tb), "smoke")


def test_one_side_empty(gpu):
    rng = np.random.default_rng(3)
    rows, cols = 500, 600
    a = random_csr(rng, rows, cols, 0.02)
    e = (np.zeros(rows + 1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    assert_csr_equal(run(a, e, rows, cols, gpu), a, "b empty")
    assert_csr_equal(run(e, a, rows, cols, gpu), a, "a empty")
    got = run(e, e, rows, cols, gpu)
    assert len(got[1]) == 0 and np.all(got[0] == 0)


def test_c2_full_size(gpu):
    """The C2 operands, the right one as COO: the same result as csr_add (bit-exact against
    the multi-threaded C restatement)."""
    from nacho_amd import synth

    rows = synth.C2_ROWS
    a, b = synth.c2_operands()
    got = run(a, b, rows, rows, gpu)
    assert_csr_equal(got, oracle.port_csr_binary("add", rows, *a, *b, nthreads=16), "C2")
