"""Pins the DCSR oracle (nacho_oracle.c: oracle_dcsr_binary) on the CPU.

dcsr_add / dcsr_mul (compiler.cpp:124-133) have no golden vectors in the reference; its
tests/smoke.py:149-167 re-expands the DCSR result to CSR and compares with scipy's
`a + b` / `a.multiply(b)`.  The oracle is checked here against:
  * that smoke comparison on the smoke generator's 200x180, density 0.05 operands;
  * the closed form (oracle.closed_dcsr_binary): row ids = union / intersection of the
    operands' row ids, entries = the CSR closed form of the expanded matrices;
  * a dictionary evaluation of the two-level lattice on tiny inputs;
  * hand-built cases: a row stored in both operands whose column intersection is empty is
    kept with an empty fibre (mul); disjoint row sets; empty operands.
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle


def dcsr_of(m):
    """scipy CSR -> DCSR levels (crd_i, pos_j, crd_j) and values, dropping empty rows
    (python/nacho/convert.py:34-53)."""
    m = sp.csr_matrix(m)
    m.sort_indices()
    lengths = np.diff(m.indptr)
    present = np.flatnonzero(lengths > 0)
    pos = np.zeros(len(present) + 1, np.int64)
    pos[1:] = np.cumsum(lengths[present])
    return ((present.astype(np.int32), pos.astype(np.int32), m.indices.astype(np.int32)),
            m.data.astype(np.float32))


def expand(levels, val, shape):
    ci, pj, cj = levels
    indptr = np.zeros(shape[0] + 1, np.int64)
    indptr[np.asarray(ci, np.int64) + 1] = np.diff(np.asarray(pj, np.int64))
    return sp.csr_matrix((val, cj, np.cumsum(indptr)), shape=shape)


def random_dcsr(rng, rows, cols, density, empty_row_frac=0.5, max_nnz=4_000_000):
    """About density * rows * cols distinct uniform entries (at most max_nnz), values in
    [-1, 1), then about empty_row_frac of the rows emptied (so they are not stored)."""
    n = min(int(round(density * rows * cols)), max_nnz)
    keys = np.unique(rng.integers(0, rows * cols, size=n, dtype=np.int64))
    r, c = keys // cols, keys % cols
    keep = rng.random(rows) >= empty_row_frac
    sel = keep[r]
    r, c = r[sel], c[sel]
    val = rng.uniform(-1, 1, len(r)).astype(np.float32)
    val[val == 0] = np.float32(0.5)  # no explicit zeros: scipy would keep them anyway
    return dcsr_of(sp.csr_matrix((val, (r, c)), shape=(rows, cols)))


def assert_dcsr_equal(got, want, what=""):
    (gl, gv), (wl, wv) = got, want
    for name, g, w in zip(("crd_i", "pos_j", "crd_j"), gl, wl):
        np.testing.assert_array_equal(np.asarray(g, np.int64), np.asarray(w, np.int64),
                                      err_msg=f"{what}: {name}")
    np.testing.assert_array_equal(np.asarray(gv, np.float32).view(np.int32),
                                  np.asarray(wv, np.float32).view(np.int32),
                                  err_msg=f"{what}: values (bits)")


@pytest.mark.parametrize("op", ["add", "mul"])
def test_reference_smoke_comparison(op):
    rng = np.random.default_rng(0)
    shape = (200, 180)
    ms = []
    for _ in range(2):
        m = sp.random(*shape, density=0.05, format="csr", dtype=np.float32,
                      random_state=rng.integers(2**31))
        m.sum_duplicates()
        m.sort_indices()
        ms.append(m)
    (al, av), (bl, bv) = dcsr_of(ms[0]), dcsr_of(ms[1])
    levels, val = oracle.port_dcsr_binary(op, al, av, bl, bv)
    got = expand(levels, val, shape)
    want = ms[0] + ms[1] if op == "add" else ms[0].multiply(ms[1])
    want = sp.csr_matrix(want)
    want.eliminate_zeros()
    assert abs(got - want).max() < 1e-4 if want.nnz else got.nnz == 0


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(5))
def test_closed_form(op, seed):
    rng = np.random.default_rng(100 + seed)
    rows, cols = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
    density = float(rng.choice([0.0005, 0.01, 0.1]))
    (al, av), (bl, bv) = (random_dcsr(rng, rows, cols, density) for _ in range(2))
    got = oracle.port_dcsr_binary(op, al, av, bl, bv)
    want = oracle.closed_dcsr_binary(op, rows, cols, al, av, bl, bv)
    assert_dcsr_equal(got, want, f"{op} seed={seed}")


@pytest.mark.parametrize("op", ["add", "mul"])
def test_brute_force_tiny(op):
    rng = np.random.default_rng(7)
    for trial in range(30):
        rows, cols = int(rng.integers(1, 9)), int(rng.integers(1, 9))
        (al, av), (bl, bv) = (random_dcsr(rng, rows, cols, 0.4, 0.3) for _ in range(2))

        def entries(levels, val):
            ci, pj, cj = levels
            return {int(i): {int(cj[p]): np.float32(val[p]) for p in range(pj[q], pj[q + 1])}
                    for q, i in enumerate(ci)}

        ea, eb = entries(al, av), entries(bl, bv)
        ids = sorted(ea.keys() | eb.keys()) if op == "add" else sorted(ea.keys() & eb.keys())
        w_ci, w_pj, w_cj, w_v = [], [0], [], []
        for i in ids:
            ra, rb = ea.get(i, {}), eb.get(i, {})
            cs = sorted(ra.keys() | rb.keys()) if op == "add" else sorted(ra.keys() & rb.keys())
            for c in cs:
                if c in ra and c in rb:
                    w_v.append(ra[c] + rb[c] if op == "add" else ra[c] * rb[c])
                else:
                    w_v.append(ra.get(c, rb.get(c)))
                w_cj.append(c)
            w_ci.append(i)
            w_pj.append(len(w_cj))
        want = ((w_ci, w_pj, w_cj), np.asarray(w_v, np.float32))
        assert_dcsr_equal(oracle.port_dcsr_binary(op, al, av, bl, bv), want, f"trial {trial}")


def test_mul_keeps_rows_with_empty_intersection():
    a = ((np.array([1, 4, 6], np.int32), np.array([0, 2, 3, 4], np.int32),
          np.array([0, 5, 2, 9], np.int32)), np.array([1, 2, 3, 4], np.float32))
    b = ((np.array([1, 2, 6], np.int32), np.array([0, 1, 2, 4], np.int32),
          np.array([3, 7, 1, 9], np.int32)), np.array([5, 6, 7, 8], np.float32))
    (ci, pj, cj), v = oracle.port_dcsr_binary("mul", *a, *b)
    assert list(ci) == [1, 6] and list(pj) == [0, 0, 1] and list(cj) == [9]
    assert v.tolist() == [np.float32(4) * np.float32(8)]
    (ci, pj, cj), v = oracle.port_dcsr_binary("add", *a, *b)
    assert list(ci) == [1, 2, 4, 6] and list(pj) == [0, 3, 4, 5, 7]
    assert list(cj) == [0, 3, 5, 7, 2, 1, 9]


@pytest.mark.parametrize("op", ["add", "mul"])
def test_empty_operands(op):
    e = ((np.zeros(0, np.int32), np.zeros(1, np.int32), np.zeros(0, np.int32)),
         np.zeros(0, np.float32))
    rng = np.random.default_rng(5)
    b = random_dcsr(rng, 50, 40, 0.1)
    (ci, pj, cj), v = oracle.port_dcsr_binary(op, *e, *e)
    assert len(ci) == 0 and list(pj) == [0] and len(cj) == 0 and len(v) == 0
    got = oracle.port_dcsr_binary(op, *e, *b)
    if op == "mul":
        assert len(got[0][0]) == 0 and list(got[0][1]) == [0]
    else:
        assert_dcsr_equal(got, b, "a empty")
