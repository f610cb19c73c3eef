"""GPU parity of the masked SpGEMM (sssmm) against the oracle: structure exact, values within
rel 1e-5 / abs 1e-6 (the summation order differs)."""

import os

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import random_csr

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def upload(t, shape, device):
    import nacho_amd

    return nacho_amd.CSR_gpu(*(torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in t),
                             torch.tensor(shape, dtype=torch.int32))


def run(a, b, c, shapes, device):
    import nacho_amd

    print(f"[gpu] sssmm shapes={shapes} nnz={[len(t[1]) for t in (a, b, c)]}", flush=True)
    z = nacho_amd.gpu_sssmm_f32(*(upload(t, s, device) for t, s in zip((a, b, c), shapes)))
    torch.cuda.synchronize()
    return z.dim_j_offsets.cpu().numpy(), z.dim_j_indices.cpu().numpy(), z.values.cpu().numpy()


def check(got, want, what):
    np.testing.assert_array_equal(got[0].astype(np.int64), np.asarray(want[0], np.int64),
                                  err_msg=f"{what}: pos")
    np.testing.assert_array_equal(got[1], want[1], err_msg=f"{what}: crd")
    np.testing.assert_allclose(got[2], want[2], rtol=RTOL, atol=ATOL, err_msg=f"{what}: val")


@pytest.mark.parametrize("seed", range(6))
def test_random(gpu, seed):
    rng = np.random.default_rng(900 + seed)
    n, m, q = (int(rng.choice([1, 7, 300, 5000])) for _ in range(3))
    a = random_csr(rng, n, m, min(0.3, 40.0 / max(m, 1)))
    b = random_csr(rng, m, q, min(0.3, 40.0 / max(q, 1)))
    c = random_csr(rng, n, q, min(0.5, 60.0 / max(q, 1)))
    check(run(a, b, c, ((n, m), (m, q), (n, q)), gpu), oracle.port_sssmm(n, q, a, b, c),
          f"seed={seed}")


@pytest.mark.parametrize("scale", [10, 14])
def test_rmat_masked_by_itself(gpu, scale):
    """A, A, A as the reference benchmark runs square matrices (hub rows and columns)."""
    from nacho_amd import synth

    a = synth.rmat_csr(scale, seed=3)
    n = len(a[0]) - 1
    check(run(a, a, a, ((n, n),) * 3, gpu), oracle.port_sssmm(n, n, a, a, a), f"rmat {scale}")


def test_full_disjoint_and_empty_masks(gpu):
    rng = np.random.default_rng(5)
    a, b = random_csr(rng, 200, 150, 0.05), random_csr(rng, 150, 180, 0.05)
    pz, cz, vz = oracle.port_spgemm(200, 150, 180, *a, *b)
    full = (pz.astype(np.int32), cz, rng.uniform(0.5, 1.5, len(cz)).astype(np.float32))
    shapes = ((200, 150), (150, 180), (200, 180))
    check(run(a, b, full, shapes, gpu), oracle.port_sssmm(200, 180, a, b, full), "full mask")
    dense = np.zeros((200, 180), bool)
    rows = np.repeat(np.arange(200), np.diff(pz))
    dense[rows, cz] = True
    r, k = np.nonzero(~dense)
    pos = np.searchsorted(r, np.arange(201)).astype(np.int32)
    disjoint = (pos, k.astype(np.int32), np.ones(len(k), np.float32))
    got = run(a, b, disjoint, shapes, gpu)
    assert got[0].tolist() == [0] * 201 and len(got[1]) == 0
    e = (np.zeros(201, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    got = run(a, b, e, shapes, gpu)
    assert got[0].tolist() == [0] * 201 and len(got[1]) == 0


def test_shape_mismatch_raises(gpu):
    rng = np.random.default_rng(6)
    a, b, c = random_csr(rng, 5, 4, 0.5), random_csr(rng, 5, 6, 0.5), random_csr(rng, 5, 6, 0.5)
    with pytest.raises(RuntimeError, match="invalid argument"):
        run(a, b, c, ((5, 4), (5, 6), (5, 6)), gpu)


def test_repeatable(gpu):
    from nacho_amd import synth

    a = synth.rmat_csr(13, seed=4)
    n = len(a[0]) - 1
    first = run(a, a, a, ((n, n),) * 3, gpu)
    second = run(a, a, a, ((n, n),) * 3, gpu)
    np.testing.assert_array_equal(first[1], second[1])
    np.testing.assert_allclose(first[2], second[2], rtol=2.5e-7, atol=0)


def test_c4_masked_by_itself(gpu):
    """R-MAT 2^20 (the C4 operand) as A, B and mask: every row against the oracle (6.0e9
    products; the oracle runs on all rows with the host's cores)."""
    from nacho_amd import synth

    a = synth.c4_operand()
    n = len(a[0]) - 1
    pz, cz, vz = run(a, a, a, ((n, n),) * 3, gpu)
    threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    want = oracle.port_sssmm(n, n, a, a, a, nthreads=threads)
    check((pz, cz, vz), want, "C4 masked by itself")
    assert pz[-1] <= len(a[1])
