"""Pins the inner-product oracle (oracle_csf3_inner / oracle_coo3_inner): the full
reductions inner_prod and inner_prod_coo (reference compiler.cpp:141, 143).

Checked against the key-intersection closed form (numpy), against a dictionary brute force
(the reference's own smoke case: tests/smoke.py _expected_inner_product over shape
(40, 30, 25) with 900 draws), against special cases the mathematics fixes (an operand with
itself is its sum of squares; disjoint operands give 0; a single shared coordinate gives
that one product), and with mistakes planted in the operands the oracle sees (a dropped or
shifted shared coordinate must move the result).
"""

import numpy as np
import pytest

from nacho_amd.convert import csf3_levels
from oracle import oracle


def random_coords(rng, shape, n):
    coords = np.unique(np.stack([rng.integers(0, e, n) for e in shape], axis=1), axis=0)
    return coords.astype(np.int32), rng.uniform(-1, 1, len(coords)).astype(np.float32)


def both(shape, ac, av, bc, bv, nthreads=0):
    csf = oracle.port_csf3_inner(csf3_levels(ac), av, csf3_levels(bc), bv, nthreads=nthreads)
    coo = oracle.port_coo3_inner(tuple(ac[:, d] for d in range(3)), av,
                                 tuple(bc[:, d] for d in range(3)), bv, nthreads=nthreads)
    return csf, coo


def closed(shape, ac, av, bc, bv):
    return oracle.closed_inner(shape, tuple(ac[:, d] for d in range(3)), av,
                               tuple(bc[:, d] for d in range(3)), bv)


def close(x, y, scale):
    # float64 sums of the same float32 products in different orders
    return abs(x - y) <= 1e-12 * max(1.0, scale)


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("nthreads", [1, 3, 0])
def test_port_matches_closed_form(seed, nthreads):
    rng = np.random.default_rng(seed)
    shape = tuple(int(rng.integers(1, 40)) for _ in range(3))
    n = int(rng.integers(0, 5000))
    ac, av = random_coords(rng, shape, n)
    bc, bv = random_coords(rng, shape, n)
    want = closed(shape, ac, av, bc, bv)
    scale = float(np.abs(av).sum() + np.abs(bv).sum())
    csf, coo = both(shape, ac, av, bc, bv, nthreads)
    assert close(csf, want, scale), (csf, want)
    assert close(coo, want, scale), (coo, want)


def test_reference_smoke_case():
    rng = np.random.default_rng(0)
    shape = (40, 30, 25)

    def random_coo_3d():
        coords = np.unique(np.stack([rng.integers(0, e, 900) for e in shape], axis=1), axis=0)
        return coords.astype(np.int32), rng.random(coords.shape[0]).astype(np.float32)

    (ac, av), (bc, bv) = random_coo_3d(), random_coo_3d()
    a_entries = {tuple(int(x) for x in c): float(v) for c, v in zip(ac, av)}
    expected = sum(a_entries[k] * float(v) for c, v in zip(bc, bv)
                   if (k := tuple(int(x) for x in c)) in a_entries)
    csf, coo = both(shape, ac, av, bc, bv)
    # the brute force multiplies in float64; the oracle's products are float32
    assert abs(csf - expected) <= 1e-6 * max(1.0, abs(expected))
    assert abs(coo - expected) <= 1e-6 * max(1.0, abs(expected))
    assert close(csf, coo, abs(expected))


def test_self_product_is_sum_of_squares():
    rng = np.random.default_rng(5)
    shape = (50, 20, 30)
    ac, av = random_coords(rng, shape, 3000)
    want = float(np.sum((av * av).astype(np.float64)))
    csf, coo = both(shape, ac, av, ac, av)
    assert close(csf, want, want) and close(coo, want, want)


def test_disjoint_and_empty():
    rng = np.random.default_rng(6)
    shape = (30, 30, 30)
    ac, av = random_coords(rng, shape, 2000)
    bc = ac.copy()
    bc[:, 2] = (bc[:, 2] + shape[2]) + 1  # every k outside A's range
    bc = bc[np.lexsort((bc[:, 2], bc[:, 1], bc[:, 0]))]
    big = (30, 30, 2 * shape[2] + 2)
    assert both(big, ac, av, bc, av) == (0.0, 0.0)
    e = np.zeros((0, 3), np.int32)
    ev = np.zeros(0, np.float32)
    assert both(shape, e, ev, ac, av) == (0.0, 0.0)
    assert both(shape, e, ev, e, ev) == (0.0, 0.0)


def test_single_shared_coordinate():
    ac = np.array([[0, 0, 0], [1, 2, 3], [4, 5, 6]], np.int32)
    bc = np.array([[1, 2, 3], [4, 5, 7], [9, 9, 9]], np.int32)
    av = np.array([1.5, 2.25, -3.0], np.float32)
    bv = np.array([-0.5, 8.0, 2.0], np.float32)
    assert both((10, 10, 10), ac, av, bc, bv) == (2.25 * -0.5, 2.25 * -0.5)


@pytest.mark.parametrize("mistake", ["drop", "shift_k", "swap_j"])
def test_planted_mistakes_are_caught(mistake):
    """A plausible slip in walking the levels (a shared coordinate missed, an off-by-one k,
    a j taken from the wrong fibre) changes what the oracle computes, and the closed form
    over the true operands tells the two apart."""
    rng = np.random.default_rng(11)
    shape = (20, 20, 20)
    ac, av = random_coords(rng, shape, 4000)
    keep = rng.random(len(ac)) < 0.6
    bc, bv = ac[keep], rng.uniform(0.5, 1.5, int(keep.sum())).astype(np.float32)
    want = closed(shape, ac, av, bc, bv)
    wrong = bc.copy()
    if mistake == "drop":
        wrong, wbv = wrong[1:], bv[1:]
    elif mistake == "shift_k":
        wrong[:, 2] = np.minimum(wrong[:, 2] + 1, shape[2] - 1)
        wrong, idx = np.unique(wrong, axis=0, return_index=True)
        wbv = bv[idx]
    else:
        wrong[:, 1] = shape[1] - 1 - wrong[:, 1]
        order = np.lexsort((wrong[:, 2], wrong[:, 1], wrong[:, 0]))
        wrong, wbv = wrong[order], bv[order]
    csf, coo = both(shape, ac, av, wrong, wbv)
    assert not close(csf, want, 1.0) and not close(coo, want, 1.0)
