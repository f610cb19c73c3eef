"""The range-parallel oracle restatements (oracle_csf3_union_mt, oracle_dcsr_binary_mt,
oracle_csr_add3_mt: the CPU baselines, one partition per thread with count and write
passes as the reference's CPU target runs, stitch_and_generate_cpu.cpp:26-31, 138-154)
return exactly what the serial lattices return, which their own tests pin.  Thread counts
from 1 to more threads than top-level items; skewed, empty and one-sided operands."""

import numpy as np
import pytest

from nacho_amd.convert import csf3_levels
from oracle import oracle
from tests.helpers import random_csr
from tests.test_oracle_csf import assert_csf_equal, random_coords
from tests.test_oracle_dcsr import assert_dcsr_equal, random_dcsr
from tests.test_oracle_csr3 import assert_csr_equal

THREADS = [1, 2, 3, 8, 64]


def skewed_coords(rng, shape, n):
    """Mode 0 Zipf-like: one fibre holds most entries, as in the C5 generator."""
    i = np.minimum(rng.zipf(1.3, n) - 1, shape[0] - 1)
    coords = np.stack([i, rng.integers(0, shape[1], n), rng.integers(0, shape[2], n)], axis=1)
    coords = np.unique(coords, axis=0)
    return coords.astype(np.int32), rng.uniform(-1, 1, len(coords)).astype(np.float32)


@pytest.mark.parametrize("nt", THREADS)
@pytest.mark.parametrize("case", ["uniform", "skewed", "a_empty", "both_empty", "same"])
def test_csf3_union_mt_equals_serial(nt, case):
    rng = np.random.default_rng(7)
    shape = (60, 40, 30)
    if case == "skewed":
        ac, av = skewed_coords(rng, shape, 4000)
        bc, bv = skewed_coords(rng, shape, 3000)
    else:
        ac, av = random_coords(rng, shape, 3000)
        bc, bv = random_coords(rng, shape, 2500)
    if case in ("a_empty", "both_empty"):
        ac, av = ac[:0], av[:0]
    if case == "both_empty":
        bc, bv = bc[:0], bv[:0]
    if case == "same":
        bc, bv = ac, -av
    la, lb = csf3_levels(ac), csf3_levels(bc)
    want = oracle.port_csf3_union(la, av, lb, bv)
    got = oracle.port_csf3_union(la, av, lb, bv, nthreads=nt)
    assert_csf_equal(got, want, f"csf3 mt nt={nt} {case}")


@pytest.mark.parametrize("nt", THREADS)
@pytest.mark.parametrize("op", ["add", "mul"])
def test_dcsr_binary_mt_equals_serial(nt, op):
    rng = np.random.default_rng(8)
    for rows, cols, density in ((300, 200, 0.05), (50, 4000, 0.2), (1, 10, 0.5)):
        a = random_dcsr(rng, rows, cols, density)
        b = random_dcsr(rng, rows, cols, density)
        want = oracle.port_dcsr_binary(op, *a, *b)
        got = oracle.port_dcsr_binary(op, *a, *b, nthreads=nt)
        assert_dcsr_equal(got, want, f"dcsr {op} mt nt={nt} rows={rows}")


@pytest.mark.parametrize("nt", THREADS)
def test_csr_add3_mt_equals_serial(nt):
    rng = np.random.default_rng(9)
    for rows, cols, density in ((500, 700, 0.02), (3, 5000, 0.3), (2000, 50, 0.0)):
        ops = [random_csr(rng, rows, cols, density) for _ in range(3)]
        want = oracle.port_csr_add3(rows, *ops)
        got = oracle.port_csr_add3(rows, *ops, nthreads=nt)
        assert_csr_equal(got, want, f"add3 mt nt={nt} rows={rows}")
