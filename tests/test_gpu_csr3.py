"""GPU parity of csr_add_3 (A + B + C) against the oracle, bit-exact."""

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import csr_from_rows, random_csr
from tests.test_oracle_csr3 import assert_csr_equal

pytestmark = pytest.mark.gpu


def run(rows, cols, ops, device):
    import nacho_amd

    print(f"[gpu] csr_add_3 rows={rows} cols={cols} nnz={[len(o[1]) for o in ops]}", flush=True)
    t = [nacho_amd.CSR_gpu(*(torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in o),
                           torch.tensor([rows, cols], dtype=torch.int32)) for o in ops]
    z = nacho_amd.gpu_csr_add_3_f32(*t)
    torch.cuda.synchronize()
    return (z.dim_j_offsets.cpu().numpy(), z.dim_j_indices.cpu().numpy(), z.values.cpu().numpy())


@pytest.mark.parametrize("seed", range(6))
def test_random(gpu, seed):
    rng = np.random.default_rng(700 + seed)
    rows = int(rng.choice([1, 13, 3000, 200000]))
    cols = int(rng.choice([1, 29, 4000, 1 << 20]))
    density = min(0.3, 3e6 / max(1, rows * cols))
    ops = [random_csr(rng, rows, cols, density * float(rng.uniform(0.2, 1))) for _ in range(3)]
    assert_csr_equal(run(rows, cols, ops, gpu), oracle.port_csr_add3(rows, *ops), f"seed={seed}")


def test_overlaps_and_order(gpu):
    a = csr_from_rows(3, 10, [[1, 2, 5], [], [0, 9]], [1e8, 2, 3, 4, 5])
    b = csr_from_rows(3, 10, [[2, 5], [4], [9]], [-1, -1e8, 7, 8])
    c = csr_from_rows(3, 10, [[1, 5, 7], [4], []], [1, 1, 2, 3])
    assert_csr_equal(run(3, 10, [a, b, c], gpu), oracle.port_csr_add3(3, a, b, c), "hand")
    e = (np.zeros(4, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    assert_csr_equal(run(3, 10, [e, b, e], gpu), oracle.port_csr_add3(3, e, b, e), "only b")
    got = run(3, 10, [e, e, e], gpu)
    assert got[0].tolist() == [0, 0, 0, 0] and len(got[1]) == 0


def test_c2_triple(gpu):
    """Three C2 operands (Zipf(1.6) rows, 16.7M nnz each, seeds 1, 2, 4)."""
    from nacho_amd import synth

    rows = synth.C2_ROWS
    ops = [synth.zipf_csr(rows, s) for s in (1, 2, 4)]
    assert_csr_equal(run(rows, rows, ops, gpu), oracle.port_csr_add3(rows, *ops), "C2 triple")


@pytest.mark.parametrize("pattern", ["same", "strided", "dense_rows"])
def test_key_groups_across_tiles(gpu, pattern):
    """Long rows where most keys occur in two or three operands, so that tile and lane
    boundaries fall inside key groups (a group must still produce one entry)."""
    rng = np.random.default_rng(7)
    if pattern == "same":  # one row, every key in all three operands
        rows, cols = 1, 40000
        keys = [np.arange(cols)] * 3
        ops = [csr_from_rows(rows, cols, [k.tolist()], rng.standard_normal(len(k)).tolist())
               for k in keys]
    elif pattern == "strided":  # A: even keys, B: multiples of 3, C: every key
        rows, cols = 2, 30011
        ops = []
        for step in (2, 3, 1):
            k = np.arange(0, cols, step)
            ops.append(csr_from_rows(rows, cols, [k.tolist(), k[: len(k) // 2].tolist()],
                                     rng.standard_normal(len(k) + len(k) // 2).tolist()))
    else:  # many short dense rows with full overlap, and empty rows between
        rows, cols = 5000, 7
        lists = [[list(range(cols)) if r % 3 else [] for r in range(rows)] for _ in range(3)]
        ops = [csr_from_rows(rows, cols, l, rng.standard_normal(sum(map(len, l))).tolist())
               for l in lists]
    assert_csr_equal(run(rows, cols, ops, gpu), oracle.port_csr_add3(rows, *ops), pattern)


def test_duplicate_search_branches(gpu):
    """Many rows that hold one operand only (so the count searches for duplicates instead of
    walking every tile), and rows that take each search branch: A smaller or larger than B,
    C at most A + B (C's entries searched) or more (A's and B's searched in C, B's counted
    only when absent from A), empty A or B, keys in two and in all three operands."""
    rng = np.random.default_rng(11)
    rows, cols = 2000, 5000
    shapes = [(3, 10, 2), (10, 3, 50), (0, 5, 20), (5, 0, 3), (12, 12, 40), (7, 2, 0)]
    lists = [[], [], []]
    for r in range(rows):
        if r < 1880:  # one operand, 100 entries
            for o in range(3):
                lists[o].append(sorted(rng.choice(cols, 100, replace=False).tolist())
                                if r % 3 == o else [])
        else:  # overlapping rows, keys from a small pool
            for o, n in enumerate(shapes[r % len(shapes)]):
                lists[o].append(sorted(rng.choice(64, n, replace=False).tolist()))
    ops = [csr_from_rows(rows, cols, l, rng.standard_normal(sum(map(len, l))).tolist())
           for l in lists]
    assert_csr_equal(run(rows, cols, ops, gpu), oracle.port_csr_add3(rows, *ops), "branches")
