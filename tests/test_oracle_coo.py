"""Pins the COO / COO3 oracle (C restatement of the reference's merged-coordinate pipeline).

Checked against the numpy closed form (union / intersection of packed tuple keys), a
dictionary brute force, and the reference's own smoke cases for coo_add and coo3d_add
(reference tests/smoke.py: 200 x 180 at density 0.05; shape (40, 30, 25) with 900 draws,
compared against a coordinate dictionary of summed values).
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle


def random_coo(rng, shape, n):
    coords = np.unique(np.stack([rng.integers(0, e, n) for e in shape], axis=1), axis=0)
    vals = rng.uniform(-1, 1, len(coords)).astype(np.float32)
    return tuple(coords[:, d].astype(np.int32) for d in range(len(shape))), vals


def assert_coo_equal(got, want, what=""):
    (gc, gv), (wc, wv) = got, want
    assert len(gc) == len(wc)
    for d, (x, y) in enumerate(zip(gc, wc)):
        assert np.array_equal(np.asarray(x, np.int64), np.asarray(y, np.int64)), \
            f"{what}: coordinate {d} differs"
    assert np.array_equal(np.asarray(gv, np.float32).view(np.uint32),
                          np.asarray(wv, np.float32).view(np.uint32)), f"{what}: values differ"


@pytest.mark.parametrize("arity", [2, 3])
@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(5))
def test_port_matches_closed_form(arity, op, seed):
    rng = np.random.default_rng(seed)
    shape = tuple(int(rng.integers(1, 60)) for _ in range(arity))
    n = int(rng.integers(0, 3000))
    a, va = random_coo(rng, shape, n)
    b, vb = random_coo(rng, shape, n)
    want = oracle.closed_coo_binary(op, shape, a, va, b, vb)
    for t in (1, 2, 7, 64, 1000):
        assert_coo_equal(oracle.port_coo_binary(op, a, va, b, vb, nthreads=t), want,
                         f"arity={arity} op={op} seed={seed} threads={t}")


def test_brute_force_tiny():
    rng = np.random.default_rng(3)
    for _ in range(30):
        shape = (4, 3, 5)
        a, va = random_coo(rng, shape, 12)
        b, vb = random_coo(rng, shape, 12)
        ea = {tuple(int(x[p]) for x in a): va[p] for p in range(len(va))}
        eb = {tuple(int(x[p]) for x in b): vb[p] for p in range(len(vb))}
        crd, val = oracle.port_coo_binary("add", a, va, b, vb, nthreads=3)
        got = {tuple(int(x[p]) for x in crd): val[p] for p in range(len(val))}
        assert got.keys() == ea.keys() | eb.keys()
        assert list(got.keys()) == sorted(got.keys())
        for k, v in got.items():
            want = np.float32(ea[k] + eb[k]) if (k in ea and k in eb) else ea.get(k, eb.get(k))
            assert np.float32(v).view(np.uint32) == np.float32(want).view(np.uint32)


def test_reference_smoke_coo_add():
    rng = np.random.default_rng(0)
    mats = []
    for _ in range(2):
        m = sp.random(200, 180, density=0.05, format="csr", dtype=np.float32,
                      random_state=rng.integers(2**31))
        m.sum_duplicates()
        m.sort_indices()
        mats.append(m.tocoo())
    a, b = mats
    crd, val = oracle.port_coo_binary("add", (a.row.astype(np.int32), a.col.astype(np.int32)),
                                      a.data, (b.row.astype(np.int32), b.col.astype(np.int32)),
                                      b.data)
    got = sp.coo_matrix((val, crd), shape=(200, 180)).tocsr()
    want = (a.tocsr() + b.tocsr())
    want.eliminate_zeros()
    diff = abs(got - want)
    assert diff.nnz == 0 or diff.max() < 1e-4


def test_reference_smoke_coo3d_add():
    rng = np.random.default_rng(0)
    shape = (40, 30, 25)

    def random_coo_3d():
        coords = np.unique(np.stack([rng.integers(0, e, 900) for e in shape], axis=1), axis=0)
        return coords, rng.random(coords.shape[0]).astype(np.float32)

    (ac, av), (bc, bv) = random_coo_3d(), random_coo_3d()
    expected = {tuple(int(x) for x in c): float(v) for c, v in zip(ac, av)}
    for c, v in zip(bc, bv):
        key = tuple(int(x) for x in c)
        expected[key] = expected.get(key, 0.0) + float(v)
    crd, val = oracle.port_coo_binary("add", tuple(ac[:, d].astype(np.int32) for d in range(3)),
                                      av, tuple(bc[:, d].astype(np.int32) for d in range(3)), bv)
    got = {(int(i), int(j), int(k)): float(v) for i, j, k, v in zip(*crd, val)}
    assert got.keys() == expected.keys()
    assert all(abs(got[k] - expected[k]) < 1e-4 for k in expected)


def test_planted_lexicographic_mistake_is_caught():
    """Ordering by (j, i) instead of (i, j) — a transposed key — is rejected."""
    rng = np.random.default_rng(11)
    a, va = random_coo(rng, (20, 20), 80)
    b, vb = random_coo(rng, (20, 20), 80)
    want = oracle.closed_coo_binary("add", (20, 20), a, va, b, vb)
    (ci, cj), v = oracle.port_coo_binary("add", a, va, b, vb)
    order = np.lexsort((ci, cj))  # sorted by j first
    with pytest.raises(AssertionError):
        assert_coo_equal(((ci[order], cj[order]), v[order]), want)
