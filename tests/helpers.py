"""Operand builders and checks shared by the test modules."""

from __future__ import annotations

import numpy as np
import scipy.sparse as sp


def random_csr(rng, rows, cols, density, dtype=np.float32):
    """Sorted, distinct-column CSR as (pos, crd, val) numpy arrays."""
    m = sp.random(rows, cols, density=density, format="csr", dtype=dtype,
                  random_state=int(rng.integers(2**31)))
    m.sum_duplicates()
    m.sort_indices()
    return (m.indptr.astype(np.int32), m.indices.astype(np.int32),
            (m.data * 2 - 1).astype(np.float32))


def csr_from_rows(rows, cols, row_lists, vals=None):
    """CSR from a list of per-row column lists (each sorted distinct)."""
    pos = np.zeros(rows + 1, np.int32)
    crd = []
    for r, cs in enumerate(row_lists):
        pos[r + 1] = pos[r] + len(cs)
        crd.extend(cs)
    crd = np.asarray(crd, np.int32)
    if vals is None:
        vals = np.arange(1, len(crd) + 1, dtype=np.float32) / 7.0
    return pos, crd, np.asarray(vals, np.float32)


def to_scipy(pos, crd, val, shape):
    return sp.csr_matrix((val, crd, pos), shape=shape)


def check_csr_invariants(pos, crd, rows, cols):
    """pos[0] = 0, monotone, pos[rows] = nnz; columns strictly increasing, in range."""
    pos = np.asarray(pos, np.int64)
    crd = np.asarray(crd, np.int64)
    assert len(pos) == rows + 1
    assert pos[0] == 0 and pos[-1] == len(crd)
    assert np.all(np.diff(pos) >= 0)
    if len(crd):
        assert crd.min() >= 0 and crd.max() < cols
        inc = np.diff(crd) > 0
        starts = np.zeros(len(crd), bool)
        starts[pos[:-1][pos[:-1] < len(crd)]] = True
        assert np.all(inc | starts[1:]), "columns not strictly increasing within a row"


def brute_force_binary(op, rows, a, b):
    """Dictionary evaluation of the union (add) / intersection (mul) lattice."""
    def entries(t):
        pos, crd, val = t
        return {(r, int(crd[p])): np.float32(val[p])
                for r in range(rows) for p in range(pos[r], pos[r + 1])}

    ea, eb = entries(a), entries(b)
    out = {}
    keys = (ea.keys() | eb.keys()) if op == "add" else (ea.keys() & eb.keys())
    for k in keys:
        if k in ea and k in eb:
            out[k] = np.float32(ea[k] + eb[k]) if op == "add" else np.float32(ea[k] * eb[k])
        else:
            out[k] = ea.get(k, eb.get(k))
    return out


def csr_to_dict(rows, pos, crd, val):
    return {(r, int(crd[p])): np.float32(val[p])
            for r in range(rows) for p in range(pos[r], pos[r + 1])}


def assert_csr_equal(got, want, what=""):
    """Bit-exact equality of (pos, crd, val) triples (values compared as bit patterns)."""
    gp, gc, gv = (np.asarray(x) for x in got)
    wp, wc, wv = (np.asarray(x) for x in want)
    assert np.array_equal(gp.astype(np.int64), wp.astype(np.int64)), f"{what}: pos differs"
    assert np.array_equal(gc.astype(np.int64), wc.astype(np.int64)), f"{what}: crd differs"
    assert gv.dtype == np.float32 and wv.dtype == np.float32
    assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), f"{what}: values differ"
