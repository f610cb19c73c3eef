"""Pins the csr_add_3 oracle (nacho_oracle.c: oracle_csr_add3) on the CPU.

The reference's own check of csr_add_3 (benchmarks/csr_add_3.py) compares it with torch's
A + B + C.  Here the C restatement is checked against the numpy closed form (union of the
three key sets, values (a + b) + c over the present operands), against scipy's
(A + B) + C after pruning zeros, against a dictionary brute force on tiny inputs, and
against a case where float32 addition order is visible.
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle
from tests.helpers import random_csr


def assert_csr_equal(got, want, what=""):
    for name, g, w in zip(("pos", "crd"), got[:2], want[:2]):
        np.testing.assert_array_equal(np.asarray(g, np.int64), np.asarray(w, np.int64),
                                      err_msg=f"{what}: {name}")
    np.testing.assert_array_equal(np.asarray(got[2], np.float32).view(np.int32),
                                  np.asarray(want[2], np.float32).view(np.int32),
                                  err_msg=f"{what}: values (bits)")


@pytest.mark.parametrize("seed", range(6))
def test_closed_form(seed):
    rng = np.random.default_rng(40 + seed)
    rows, cols = int(rng.integers(1, 2000)), int(rng.integers(1, 2000))
    ops = [random_csr(rng, rows, cols, float(rng.choice([0.001, 0.02, 0.2]))) for _ in range(3)]
    got = oracle.port_csr_add3(rows, *ops)
    want = oracle.closed_csr_add3(rows, cols, *ops)
    assert_csr_equal(got, want, f"seed={seed}")


def test_scipy_sum_on_smoke_sized_operands():
    rng = np.random.default_rng(0)
    ops = [random_csr(rng, 200, 180, 0.05) for _ in range(3)]
    pos, crd, val = oracle.port_csr_add3(200, *ops)
    got = sp.csr_matrix((val, crd, pos), shape=(200, 180))
    mats = [sp.csr_matrix((v, c, p), shape=(200, 180)) for p, c, v in ops]
    want = (mats[0] + mats[1]) + mats[2]
    want.eliminate_zeros()
    got.eliminate_zeros()
    assert (got != want).nnz == 0


def test_brute_force_tiny():
    rng = np.random.default_rng(9)
    for trial in range(40):
        rows, cols = int(rng.integers(1, 6)), int(rng.integers(1, 7))
        ops = [random_csr(rng, rows, cols, 0.5) for _ in range(3)]
        ents = [{(r, int(c[q])): np.float32(v[q]) for r in range(rows)
                 for q in range(p[r], p[r + 1])} for p, c, v in ops]
        keys = sorted(ents[0].keys() | ents[1].keys() | ents[2].keys())
        w_pos, w_crd, w_val = [0] * (rows + 1), [], []
        for r, c in keys:
            present = [e[(r, c)] for e in ents if (r, c) in e]
            v = present[0]
            for x in present[1:]:
                v = np.float32(v + x)
            w_crd.append(c)
            w_val.append(v)
            w_pos[r + 1] += 1
        want = (np.cumsum(w_pos), w_crd, np.asarray(w_val, np.float32))
        assert_csr_equal(oracle.port_csr_add3(rows, *ops), want, f"trial {trial}")


def test_addition_order_is_a_plus_b_then_c():
    one = lambda v: (np.array([0, 1], np.int32), np.array([3], np.int32),  # noqa: E731
                     np.array([v], np.float32))
    _, _, val = oracle.port_csr_add3(1, one(1e8), one(-1e8), one(1.0))
    assert val.tolist() == [1.0]  # a + (b + c) would give 0 in float32
    _, _, val = oracle.port_csr_add3(1, one(1.0), one(1e8), one(-1e8))
    assert val.tolist() == [0.0]  # (1 + 1e8) rounds to 1e8


def test_empty_operands():
    rng = np.random.default_rng(2)
    e = (np.zeros(31, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    b = random_csr(rng, 30, 20, 0.1)
    assert_csr_equal(oracle.port_csr_add3(30, e, b, e), b, "only b")
    pos, crd, val = oracle.port_csr_add3(30, e, e, e)
    assert pos.tolist() == [0] * 31 and len(crd) == 0
