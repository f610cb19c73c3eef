"""Pins the CSR oracle (C restatement of the reference's CPU csr_add / csr_mul pipeline).

The restatement (oracle/nacho_oracle.c) is checked against checks that do not share its
algorithm: the numpy closed form of a sorted union / intersection, a dictionary brute
force on tiny inputs, scipy (the reference's own smoke-test comparison,
tests/smoke.py:110-123 and 146-157 of the reference), and structural invariants.  The
partition count is varied from 1 to more threads than items, so every boundary case of the
reference's partitioner (count == 0, count >= total_work, pairs split at a diagonal) is
exercised.  Planted-mistake tests show each check rejects a plausible wrong answer.
"""

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle
from tests.helpers import (assert_csr_equal, brute_force_binary, check_csr_invariants,
                           csr_from_rows, csr_to_dict, random_csr)

THREADS = [1, 2, 3, 8, 17, 64, 257]


def run_both(op, rows, cols, a, b, nthreads):
    port = oracle.port_csr_binary(op, rows, *a, *b, nthreads=nthreads)
    closed = oracle.closed_csr_binary(op, rows, cols, *a, *b)
    return port, closed


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(6))
def test_port_matches_closed_form_random(op, seed):
    rng = np.random.default_rng(seed)
    rows, cols = int(rng.integers(1, 300)), int(rng.integers(1, 300))
    density = float(rng.choice([0.001, 0.02, 0.1, 0.5]))
    a = random_csr(rng, rows, cols, density)
    b = random_csr(rng, rows, cols, density)
    for t in THREADS:
        port, closed = run_both(op, rows, cols, a, b, t)
        assert_csr_equal(port, closed, f"{op} seed={seed} threads={t}")
        check_csr_invariants(port[0], port[1], rows, cols)


@pytest.mark.parametrize("op", ["add", "mul"])
def test_port_matches_brute_force_tiny(op):
    rng = np.random.default_rng(42)
    for _ in range(40):
        rows, cols = int(rng.integers(1, 9)), int(rng.integers(1, 9))
        a = random_csr(rng, rows, cols, 0.4)
        b = random_csr(rng, rows, cols, 0.4)
        want = brute_force_binary(op, rows, a, b)
        for t in (1, 2, 5, 40):
            pos, crd, val = oracle.port_csr_binary(op, rows, *a, *b, nthreads=t)
            got = csr_to_dict(rows, pos, crd, val)
            assert got.keys() == want.keys()
            for k in want:
                assert np.float32(got[k]).view(np.uint32) == np.float32(want[k]).view(np.uint32)


@pytest.mark.parametrize("op", ["add", "mul"])
def test_reference_smoke_case_against_scipy(op):
    """The reference's smoke case: 200 x 180 at density 0.05, RNG default_rng(0), compared
    with scipy after pruning zeros from the expected side (reference tests/smoke.py)."""
    rng = np.random.default_rng(0)

    def smoke_csr():
        m = sp.random(200, 180, density=0.05, format="csr", dtype=np.float32,
                      random_state=rng.integers(2**31))
        m.sum_duplicates()
        m.sort_indices()
        return m

    a, b = smoke_csr(), smoke_csr()
    ta = (a.indptr.astype(np.int32), a.indices.astype(np.int32), a.data)
    tb = (b.indptr.astype(np.int32), b.indices.astype(np.int32), b.data)
    pos, crd, val = oracle.port_csr_binary(op, 200, *ta, *tb)
    got = sp.csr_matrix((val, crd, pos), shape=(200, 180))
    want = (a + b) if op == "add" else a.multiply(b)
    want = want.tocsr()
    want.eliminate_zeros()
    got.eliminate_zeros()
    diff = abs(got - want)
    assert diff.nnz == 0 or diff.max() < 1e-4
    # and exactly: the union/intersection structure with values as single f32 ops
    assert_csr_equal((pos, crd, val), oracle.closed_csr_binary(op, 200, 180, *ta, *tb))


def test_c1_config_port_matches_closed_and_scipy():
    from nacho_amd import synth

    a, b = synth.c1_operands()
    port = oracle.port_csr_binary("add", 4096, *a, *b, nthreads=8)
    assert_csr_equal(port, oracle.closed_csr_binary("add", 4096, 4096, *a, *b), "C1")
    want = (sp.csr_matrix((a[2], a[1], a[0]), shape=(4096, 4096))
            + sp.csr_matrix((b[2], b[1], b[0]), shape=(4096, 4096))).tocsr()
    want.sort_indices()
    got = sp.csr_matrix((port[2], port[1], port[0]), shape=(4096, 4096))
    # scipy drops exact zeros; U[-1,1] sums are never exactly zero here
    assert got.nnz == want.nnz
    assert np.array_equal(got.indices, want.indices)
    assert np.array_equal(got.data.view(np.uint32), want.data.astype(np.float32).view(np.uint32))


EDGE_CASES = {
    "both_empty": (4, 5, [[], [], [], []], [[], [], [], []]),
    "a_empty": (3, 6, [[], [], []], [[0, 5], [], [2]]),
    "no_rows": (0, 4, [], []),
    "all_overlap": (3, 8, [[0, 3, 7], [1], [2, 4]], [[0, 3, 7], [1], [2, 4]]),
    "no_overlap": (2, 8, [[0, 2, 4, 6], [1]], [[1, 3, 5, 7], [0]]),
    "one_long_row": (2, 20000, [list(range(0, 20000, 2)), []],
                     [list(range(0, 20000, 3)), [5]]),
    "many_empty_rows": (5000, 10, [[] for _ in range(4999)] + [[1, 2]],
                        [[3]] + [[] for _ in range(4999)]),
}


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("name", sorted(EDGE_CASES))
def test_edge_cases(op, name):
    rows, cols, ra, rb = EDGE_CASES[name]
    a = csr_from_rows(rows, cols, ra)
    b = csr_from_rows(rows, cols, rb)
    for t in (1, 4, 33):
        port, closed = run_both(op, rows, cols, a, b, t)
        assert_csr_equal(port, closed, f"{name} threads={t}")
    if name == "no_overlap" and op == "mul":
        assert len(port[1]) == 0 and not port[0].any()  # early-exit shape: zeroed offsets


def test_explicit_zeros_are_kept():
    """a + (-a) keeps every coordinate with value 0.0 (the reference never prunes)."""
    a = csr_from_rows(2, 5, [[0, 3], [4]], [1.5, -2.0, 0.25])
    b = csr_from_rows(2, 5, [[0, 3], [4]], [-1.5, 2.0, -0.25])
    pos, crd, val = oracle.port_csr_binary("add", 2, *a, *b)
    assert list(crd) == [0, 3, 4] and not val.any() and list(pos) == [0, 2, 3]


# ---- planted mistakes: each plausible error in an oracle answer is rejected ----------

def _planted(op, a, b, rows, cols):
    good = oracle.port_csr_binary(op, rows, *a, *b, nthreads=3)
    closed = oracle.closed_csr_binary(op, rows, cols, *a, *b)
    return good, closed


def test_planted_wrong_value_op_is_caught():
    rng = np.random.default_rng(7)
    a, b = random_csr(rng, 50, 40, 0.3), random_csr(rng, 50, 40, 0.3)
    (pos, crd, val), closed = _planted("add", a, b, 50, 40)
    # recompute the result with subtraction at matched coordinates (a sign error)
    ka = {(r, c): v for r in range(50) for c, v in zip(a[1][a[0][r]:a[0][r + 1]],
                                                       a[2][a[0][r]:a[0][r + 1]])}
    kb = {(r, c): v for r in range(50) for c, v in zip(b[1][b[0][r]:b[0][r + 1]],
                                                       b[2][b[0][r]:b[0][r + 1]])}
    bad = val.copy()
    for r in range(50):
        for p in range(pos[r], pos[r + 1]):
            k = (r, int(crd[p]))
            if k in ka and k in kb:
                bad[p] = np.float32(ka[k] - kb[k])
    with pytest.raises(AssertionError):
        assert_csr_equal((pos, crd, bad), closed)


def test_planted_dropped_entry_and_shifted_pos_are_caught():
    rng = np.random.default_rng(8)
    a, b = random_csr(rng, 30, 30, 0.3), random_csr(rng, 30, 30, 0.3)
    (pos, crd, val), closed = _planted("add", a, b, 30, 30)
    with pytest.raises(AssertionError):  # a dropped union term (B-only entry lost)
        assert_csr_equal((pos, np.delete(crd, 3), np.delete(val, 3)), closed)
    shifted = pos.copy()
    shifted[5] += 1  # an off-by-one row boundary
    with pytest.raises(AssertionError):
        assert_csr_equal((shifted, crd, val), closed)
    with pytest.raises(AssertionError):  # a transposed operand
        at = sp.csr_matrix((a[2], a[1], a[0]), shape=(30, 30)).T.tocsr()
        at.sort_indices()
        ta = (at.indptr.astype(np.int32), at.indices.astype(np.int32), at.data)
        assert_csr_equal(oracle.port_csr_binary("add", 30, *ta, *b), closed)
