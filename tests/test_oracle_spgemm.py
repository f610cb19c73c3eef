"""Pins the CPU SpGEMM oracle (oracle_spgemm, ESC semantics: every distinct (i, k) reached by
a product is kept, values are float32 products summed in float64 and rounded once).

The reference has no CPU SpGEMM (compiler.cpp:145-148 declares it GPU-only) and commits no
golden vectors, so the oracle is pinned against: a brute-force triple loop on tiny inputs,
scipy's float64 product (structure from the 0/1 pattern product, so cancelled entries stay),
exact algebraic cases (identity, permutation, diagonal scaling, outer products) and the
reference smoke case's shapes (tests/smoke.py:21, 213-218: 200x180 @ 180x200, density 0.05).
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle
from tests.helpers import check_csr_invariants, csr_from_rows, random_csr


def brute_force(rows, inner, cols, a, b):
    pa, ca, va = a
    pb, cb, vb = b
    out = {}
    for i in range(rows):
        for p in range(pa[i], pa[i + 1]):
            j = int(ca[p])
            for q in range(pb[j], pb[j + 1]):
                k = int(cb[q])
                out[(i, k)] = out.get((i, k), 0.0) + float(np.float32(va[p]) * np.float32(vb[q]))
    return out


def as_dict(pos, crd, val):
    return {(r, int(crd[p])): float(val[p])
            for r in range(len(pos) - 1) for p in range(pos[r], pos[r + 1])}


def assert_close_to_closed(rows, inner, cols, a, b, z):
    pos, crd, val = z
    cp, cc, cv = oracle.closed_spgemm_f64(rows, inner, cols, *a, *b)
    np.testing.assert_array_equal(pos, cp)
    np.testing.assert_array_equal(crd, cc)
    np.testing.assert_allclose(val.astype(np.float64), cv, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("seed", range(4))
def test_port_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    rows, inner, cols = 7 + seed, 6, 9
    a = random_csr(rng, rows, inner, 0.4)
    b = random_csr(rng, inner, cols, 0.4)
    z = oracle.port_spgemm(rows, inner, cols, *a, *b)
    check_csr_invariants(*z[:2], rows, cols)
    got = as_dict(*z)
    want = brute_force(rows, inner, cols, a, b)
    assert got.keys() == want.keys()
    for k in want:
        assert got[k] == pytest.approx(want[k], rel=1e-6, abs=1e-7)


@pytest.mark.parametrize("shape,density", [((200, 180, 200), 0.05), ((300, 250, 90), 0.03),
                                           ((64, 1000, 64), 0.2), ((1, 50, 1000), 0.5)])
def test_port_matches_scipy(shape, density):
    rows, inner, cols = shape
    rng = np.random.default_rng(rows + inner)
    a = random_csr(rng, rows, inner, density)
    b = random_csr(rng, inner, cols, density)
    z = oracle.port_spgemm(rows, inner, cols, *a, *b)
    assert_close_to_closed(rows, inner, cols, a, b, z)


def test_port_threads_agree():
    rng = np.random.default_rng(5)
    a = random_csr(rng, 500, 400, 0.02)
    b = random_csr(rng, 400, 300, 0.02)
    z1 = oracle.port_spgemm(500, 400, 300, *a, *b, nthreads=1)
    z4 = oracle.port_spgemm(500, 400, 300, *a, *b, nthreads=4)
    for x, y in zip(z1, z4):
        np.testing.assert_array_equal(x, y)


def test_identity_and_permutation_exact():
    rng = np.random.default_rng(2)
    n = 40
    a = random_csr(rng, n, n, 0.1)
    eye = csr_from_rows(n, n, [[i] for i in range(n)], np.ones(n, np.float32))
    z = oracle.port_spgemm(n, n, n, *a, *eye)
    for x, y in zip(z, a):
        np.testing.assert_array_equal(x, y)
    # P A with P a row permutation: rows of A reordered, values bit-identical
    perm = rng.permutation(n)
    pm = csr_from_rows(n, n, [[int(perm[i])] for i in range(n)], np.ones(n, np.float32))
    z = oracle.port_spgemm(n, n, n, *pm, *a)
    want = to_rows(a)
    got = to_rows(z)
    for i in range(n):
        assert got[i] == want[int(perm[i])]


def to_rows(t):
    pos, crd, val = t
    return [list(zip(crd[pos[r]:pos[r + 1]].tolist(), val[pos[r]:pos[r + 1]].tolist()))
            for r in range(len(pos) - 1)]


def test_outer_product_is_dense_block():
    # column vector (5 x 1) times row vector (1 x 7): every (i, k) present, value u_i * v_k
    u = np.arange(1, 6, dtype=np.float32) / 3
    v = np.arange(1, 8, dtype=np.float32) / 5
    a = csr_from_rows(5, 1, [[0]] * 5, u)
    b = csr_from_rows(1, 7, [list(range(7))], v)
    pos, crd, val = oracle.port_spgemm(5, 1, 7, *a, *b)
    np.testing.assert_array_equal(pos, np.arange(0, 36, 7))
    np.testing.assert_array_equal(crd, np.tile(np.arange(7), 5))
    np.testing.assert_array_equal(val, (u[:, None] * v[None, :]).ravel())


def test_cancellation_keeps_entry():
    # row 0: 1*x + (-1)*x = 0 at column 3 -> kept with value 0 (structural result)
    a = csr_from_rows(1, 2, [[0, 1]], np.array([1.0, -1.0], np.float32))
    b = csr_from_rows(2, 5, [[3], [3]], np.array([2.5, 2.5], np.float32))
    pos, crd, val = oracle.port_spgemm(1, 2, 5, *a, *b)
    assert pos.tolist() == [0, 1] and crd.tolist() == [3] and val.tolist() == [0.0]


def test_empty_operands():
    a = csr_from_rows(3, 4, [[], [], []])
    b = csr_from_rows(4, 5, [[1], [], [2], []])
    pos, crd, val = oracle.port_spgemm(3, 4, 5, *a, *b)
    assert pos.tolist() == [0, 0, 0, 0] and len(crd) == 0 and len(val) == 0
    # inner dimension 0
    a = csr_from_rows(2, 0, [[], []])
    b = (np.zeros(1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    pos, crd, val = oracle.port_spgemm(2, 0, 3, *a, *b)
    assert pos.tolist() == [0, 0, 0] and len(crd) == 0


def test_float64_accumulation_beats_float32():
    # 1 + 2^-24 * 2^k terms: a float32 running sum loses the small terms, float64 keeps them
    n = 4096
    va = np.ones(n, np.float32)
    va[0] = 1.0
    vb = np.full(n, np.float32(2.0 ** -24), np.float32)
    vb[0] = 1.0
    a = csr_from_rows(1, n, [list(range(n))], va)
    b = csr_from_rows(n, 1, [[0]] * n, vb)
    pos, crd, val = oracle.port_spgemm(1, n, 1, *a, *b)
    exact = 1.0 + (n - 1) * 2.0 ** -24
    assert val[0] == np.float32(exact)
    f32 = np.float32(0)
    for x in va * vb:
        f32 = np.float32(f32 + x)
    assert f32 != val[0]  # sequential float32 drops every small term


def test_rmat_small_matches_scipy():
    from nacho_amd import synth

    pos, crd, val = synth.rmat_csr(10, seed=3)
    n = 1 << 10
    z = oracle.port_spgemm(n, n, n, pos, crd, val, pos, crd, val)
    assert_close_to_closed(n, n, n, (pos, crd, val), (pos, crd, val), z)
    # positive values: no cancellation, so scipy's own product has the same structure
    c = sp.csr_matrix((val.astype(np.float64), crd, pos), shape=(n, n))
    c = c @ c
    assert c.nnz == len(z[1])
