"""GPU parity of coo_add / coo_mul / coo3d_add against the oracle (bit-exact).

Covers both key encodings of the kernel: packed 64-bit keys (every COO, and COO3 whose
extents fit 64 bits) and the wide (i<<32|j, k) key for COO3 with huge extents.
"""

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.test_oracle_coo import assert_coo_equal, random_coo

pytestmark = pytest.mark.gpu


def to_gpu(crd, val, shape, device):
    import nacho_amd

    bufs = [torch.from_numpy(np.asarray(c, np.int32)).to(device) for c in crd]
    bufs.append(torch.from_numpy(np.asarray(val, np.float32)).to(device))
    cls = nacho_amd.COO_gpu if len(crd) == 2 else nacho_amd.COO3_gpu
    return cls(*bufs, torch.tensor(list(shape), dtype=torch.int32))


def run(op, shape, a, va, b, vb, device):
    import nacho_amd

    if len(shape) == 2:
        fn = nacho_amd.gpu_coo_add_f32 if op == "add" else nacho_amd.gpu_coo_mul_f32
    else:
        assert op == "add"
        fn = nacho_amd.gpu_coo3d_add_f32
    print(f"[gpu] coo{len(shape)} {op} shape={shape} nnz=({len(va)},{len(vb)})", flush=True)
    z = fn(to_gpu(a, va, shape, device), to_gpu(b, vb, shape, device))
    torch.cuda.synchronize()
    names = ["dim_i_indices", "dim_j_indices", "dim_k_indices"][:len(shape)]
    crd = tuple(getattr(z, n).cpu().numpy() for n in names)
    assert tuple(z.shape.tolist()) == tuple(shape)
    return crd, z.values.cpu().numpy()


@pytest.mark.parametrize("op", ["add", "mul"])
@pytest.mark.parametrize("seed", range(4))
def test_coo2_random(gpu, op, seed):
    rng = np.random.default_rng(200 + seed)
    shape = (int(rng.choice([1, 50, 5000, 2**20])), int(rng.choice([1, 70, 2**20])))
    n = int(rng.choice([0, 10, 3000, 300000]))
    a, va = random_coo(rng, shape, n)
    b, vb = random_coo(rng, shape, n)
    got = run(op, shape, a, va, b, vb, gpu)
    assert_coo_equal(got, oracle.closed_coo_binary(op, shape, a, va, b, vb), f"seed={seed}")


@pytest.mark.parametrize("seed", range(4))
def test_coo3_random(gpu, seed):
    rng = np.random.default_rng(300 + seed)
    shape = tuple(int(rng.choice([1, 13, 1000, 100000])) for _ in range(3))
    n = int(rng.choice([0, 5, 4000, 500000]))
    a, va = random_coo(rng, shape, n)
    b, vb = random_coo(rng, shape, n)
    got = run("add", shape, a, va, b, vb, gpu)
    assert_coo_equal(got, oracle.port_coo_binary("add", a, va, b, vb), f"seed={seed}")


@pytest.mark.parametrize("shape", [(7, 2**16, 2**15), (7, 2**16, 2**15 - 1),
                                   (7, 2**16 + 1, 2**15), (3, 1000, 1), (2**23, 50, 50),
                                   (7, 1, 2**31 - 1), (7, 1, 2**30 + 3)])
def test_coo3_column_key_bounds(gpu, shape):
    """(j, k) keys of 31 bits whose largest is INT_MAX (the merge's sentinel: packed path)
    and of 32 bits (packed path), a k extent of one (no k bits: row-offset path), far more
    rows than entries (packed path), and a j extent of one with k keys of 31 bits (row-offset
    path; the result's k is the key's low 31 bits)."""
    rng = np.random.default_rng(sum(shape))
    n = 30000
    coords = np.unique(np.stack([rng.integers(0, e, size=n) for e in shape], axis=1), axis=0)
    coords[-1] = [e - 1 for e in shape]  # the largest key
    coords = np.unique(coords, axis=0)
    split = rng.random(len(coords)) < 0.6
    both = rng.random(len(coords)) < 0.3
    a, b = coords[split | both], coords[~split | both]
    va = rng.uniform(-1, 1, len(a)).astype(np.float32)
    vb = rng.uniform(-1, 1, len(b)).astype(np.float32)
    ta = tuple(a[:, d].astype(np.int32) for d in range(3))
    tb = tuple(b[:, d].astype(np.int32) for d in range(3))
    got = run("add", shape, ta, va, tb, vb, gpu)
    assert_coo_equal(got, oracle.port_coo_binary("add", ta, va, tb, vb), f"shape={shape}")


def test_coo3_wide_keys(gpu):
    """Extents whose bit widths sum past 64 take the wide-key path."""
    rng = np.random.default_rng(9)
    shape = (2**31 - 1, 2**31 - 1, 2**31 - 1)
    n = 20000
    coords = np.unique(rng.integers(0, 1000, size=(n, 3)) * np.array([1, 1, 1]) +
                       np.array([2**30, 7, 2**31 - 1001]), axis=0)
    split = rng.random(len(coords)) < 0.6
    both = rng.random(len(coords)) < 0.3
    a = coords[split | both]
    b = coords[~split | both]
    va = rng.uniform(-1, 1, len(a)).astype(np.float32)
    vb = rng.uniform(-1, 1, len(b)).astype(np.float32)
    ta = tuple(a[:, d].astype(np.int32) for d in range(3))
    tb = tuple(b[:, d].astype(np.int32) for d in range(3))
    got = run("add", shape, ta, va, tb, vb, gpu)
    assert_coo_equal(got, oracle.port_coo_binary("add", ta, va, tb, vb), "wide")


def test_empty_and_disjoint(gpu):
    e = (np.zeros(0, np.int32), np.zeros(0, np.int32))
    got = run("add", (5, 5), e, np.zeros(0, np.float32), e, np.zeros(0, np.float32), gpu)
    assert all(len(c) == 0 for c in got[0]) and len(got[1]) == 0
    a = (np.array([0, 1], np.int32), np.array([0, 1], np.int32))
    b = (np.array([0, 1], np.int32), np.array([1, 0], np.int32))
    got = run("mul", (2, 2), a, np.ones(2, np.float32), b, np.ones(2, np.float32), gpu)
    assert all(len(c) == 0 for c in got[0])


def test_c5_coo3_reduced(gpu):
    """The C5 generator (Zipf(1.3) mode-0) at 2M draws per operand."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = (synth.zipf3_coords(2_000_000, synth.C5_SHAPE, s) for s in (1, 2))
    ta = tuple(ac[:, d] for d in range(3))
    tb = tuple(bc[:, d] for d in range(3))
    got = run("add", synth.C5_SHAPE, ta, av, tb, bv, gpu)
    assert_coo_equal(got, oracle.port_coo_binary("add", ta, av, tb, bv, nthreads=16), "C5 2M")


def _coo_of(csr):
    pos, crd, val = csr
    rows = np.repeat(np.arange(len(pos) - 1, dtype=np.int32), np.diff(pos))
    return (rows, crd), val


@pytest.mark.parametrize("op", ["add", "mul"])
def test_c2_c3_full_size(gpu, op):
    """C2 (coo_add) and C3 (coo_mul) operands as COO at their full size (16.7M nnz each)."""
    from nacho_amd import synth

    ops = synth.c2_operands() if op == "add" else synth.c3_operands()
    (ta, va), (tb, vb) = (_coo_of(t) for t in ops)
    shape = (synth.C2_ROWS, synth.C2_ROWS)
    got = run(op, shape, ta, va, tb, vb, gpu)
    assert_coo_equal(got, oracle.port_coo_binary(op, ta, va, tb, vb, nthreads=16), f"C{op}")


def test_c5_coo3_full_size(gpu):
    """The C5 configuration at its full size (20M draws per operand)."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = synth.c5_operands()
    ta = tuple(ac[:, d] for d in range(3))
    tb = tuple(bc[:, d] for d in range(3))
    got = run("add", synth.C5_SHAPE, ta, av, tb, bv, gpu)
    assert_coo_equal(got, oracle.port_coo_binary("add", ta, av, tb, bv, nthreads=16), "C5")
