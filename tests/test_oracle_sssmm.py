"""Pins the masked SpGEMM oracle (nacho_oracle.c: oracle_sssmm) on the CPU.

sssmm (compiler.cpp:150-153) is GPU-only in the reference; its benchmark checks the result's
structure against cuSPARSE A*B followed by csr_mul with the mask (benchmarks/sssmm.py:46-51).
The oracle is pinned against scipy (structure = pattern(A) pattern(B) ∩ pattern(C), values
c * (A B) in float64), against a brute-force triple loop with the same per-term float32
rounding on tiny inputs (bit-exact), and against special cases: a full mask reduces to the
SpGEMM result scaled by c, a mask disjoint from the product gives an empty result, and the
row-list restriction computes only the listed rows.
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle
from tests.helpers import random_csr


def assert_struct(got, want, what=""):
    for name, g, w in zip(("pos", "crd"), got[:2], want[:2]):
        np.testing.assert_array_equal(np.asarray(g, np.int64), np.asarray(w, np.int64),
                                      err_msg=f"{what}: {name}")


@pytest.mark.parametrize("seed", range(5))
def test_scipy(seed):
    rng = np.random.default_rng(70 + seed)
    n, m, q = (int(rng.integers(1, 400)) for _ in range(3))
    a = random_csr(rng, n, m, float(rng.choice([0.01, 0.05, 0.2])))
    b = random_csr(rng, m, q, float(rng.choice([0.01, 0.05, 0.2])))
    c = random_csr(rng, n, q, float(rng.choice([0.01, 0.1, 0.5])))
    got = oracle.port_sssmm(n, q, a, b, c)
    want = oracle.closed_sssmm_f64(n, m, q, a, b, c)
    assert_struct(got, want, f"seed={seed}")
    np.testing.assert_allclose(got[2], want[2], rtol=1e-5, atol=1e-6)


def test_brute_force_tiny():
    rng = np.random.default_rng(3)
    for trial in range(30):
        n, m, q = (int(rng.integers(1, 7)) for _ in range(3))
        a, b, c = (random_csr(rng, *s, 0.5) for s in ((n, m), (m, q), (n, q)))
        w_pos, w_crd, w_val = [0], [], []
        for i in range(n):
            for p in range(c[0][i], c[0][i + 1]):
                k = c[1][p]
                acc, hit = 0.0, False
                for x in range(a[0][i], a[0][i + 1]):
                    j = a[1][x]
                    for y in range(b[0][j], b[0][j + 1]):
                        if b[1][y] == k:
                            ab = np.float32(a[2][x] * b[2][y])
                            acc += float(np.float32(ab * c[2][p]))
                            hit = True
                if hit:
                    w_crd.append(k)
                    w_val.append(np.float32(acc))
            w_pos.append(len(w_crd))
        got = oracle.port_sssmm(n, q, a, b, c)
        assert_struct(got, (w_pos, w_crd), f"trial {trial}")
        np.testing.assert_array_equal(got[2].view(np.int32),
                                      np.asarray(w_val, np.float32).view(np.int32))


def test_full_mask_is_spgemm_scaled():
    rng = np.random.default_rng(4)
    a, b = random_csr(rng, 60, 50, 0.1), random_csr(rng, 50, 70, 0.1)
    pz, cz, vz = oracle.port_spgemm(60, 50, 70, *a, *b)
    c = (pz.astype(np.int32), cz, np.ones(len(cz), np.float32))  # mask = the product pattern
    got = oracle.port_sssmm(60, 70, a, b, c)
    assert_struct(got, (pz, cz), "full mask")
    np.testing.assert_allclose(got[2], vz, rtol=1e-6)


def test_disjoint_mask_and_row_list():
    rng = np.random.default_rng(5)
    a, b = random_csr(rng, 40, 30, 0.1), random_csr(rng, 30, 20, 0.1)
    pz, cz, _ = oracle.port_spgemm(40, 30, 20, *a, *b)
    dense = sp.csr_matrix((np.ones(len(cz)), cz, pz), shape=(40, 20)).toarray()
    comp = sp.csr_matrix(1.0 - dense)
    c = (comp.indptr.astype(np.int32), comp.indices.astype(np.int32),
         np.ones(comp.nnz, np.float32))
    got = oracle.port_sssmm(40, 20, a, b, c)
    assert got[0].tolist() == [0] * 41 and len(got[1]) == 0
    full = oracle.port_sssmm(40, 20, a, b, (pz.astype(np.int32), cz, np.ones(len(cz), np.float32)))
    part = oracle.port_sssmm(40, 20, a, b, (pz.astype(np.int32), cz, np.ones(len(cz), np.float32)),
                             row_list=[3, 17])
    lens = np.diff(part[0])
    assert set(np.flatnonzero(lens)) <= {3, 17}
    for r in (3, 17):
        np.testing.assert_array_equal(part[1][part[0][r]:part[0][r + 1]],
                                      full[1][full[0][r]:full[0][r + 1]])
