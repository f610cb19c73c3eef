"""GPU parity of csf_add (three chained level merges) against the oracle, bit-exact."""

import numpy as np
import pytest
import torch

from nacho_amd.convert import csf3_levels
from oracle import oracle
from tests.test_oracle_csf import assert_csf_equal, random_coords

pytestmark = pytest.mark.gpu


def run(shape, ac, av, bc, bv, device):
    import nacho_amd

    print(f"[gpu] csf_add shape={shape} nnz=({len(av)},{len(bv)})", flush=True)
    z = nacho_amd.gpu_csf_add_f32(nacho_amd.to_csf3(ac, av, shape, device),
                                  nacho_amd.to_csf3(bc, bv, shape, device))
    torch.cuda.synchronize()
    levels = tuple(getattr(z, n).cpu().numpy() for n in
                   ("dim_i_indices", "dim_j_offsets", "dim_j_indices", "dim_k_offsets",
                    "dim_k_indices"))
    assert tuple(z.shape.tolist()) == tuple(shape)
    return levels, z.values.cpu().numpy()


def want(ac, av, bc, bv):
    return oracle.port_csf3_union(csf3_levels(ac), av, csf3_levels(bc), bv)


@pytest.mark.parametrize("seed", range(6))
def test_random(gpu, seed):
    rng = np.random.default_rng(400 + seed)
    shape = tuple(int(rng.choice([1, 7, 300, 20000])) for _ in range(3))
    n = int(rng.choice([1, 50, 5000, 400000]))
    ac, av = random_coords(rng, shape, n)
    bc, bv = random_coords(rng, shape, n)
    assert_csf_equal(run(shape, ac, av, bc, bv, gpu), want(ac, av, bc, bv), f"seed={seed}")


def test_reference_smoke_case(gpu):
    rng = np.random.default_rng(0)
    shape = (40, 30, 25)

    def random_coo_3d():
        coords = np.unique(np.stack([rng.integers(0, e, 900) for e in shape], axis=1), axis=0)
        return coords.astype(np.int32), rng.random(coords.shape[0]).astype(np.float32)

    (ac, av), (bc, bv) = random_coo_3d(), random_coo_3d()
    assert_csf_equal(run(shape, ac, av, bc, bv, gpu), want(ac, av, bc, bv), "smoke")


def test_one_operand_empty(gpu):
    rng = np.random.default_rng(3)
    e = np.zeros((0, 3), np.int32)
    bc, bv = random_coords(rng, (9, 9, 9), 100)
    got = run((9, 9, 9), e, np.zeros(0, np.float32), bc, bv, gpu)
    assert_csf_equal(got, want(e, np.zeros(0, np.float32), bc, bv), "a empty")
    got = run((9, 9, 9), e, np.zeros(0, np.float32), e, np.zeros(0, np.float32), gpu)
    assert len(got[0][0]) == 0 and list(got[0][1]) == [0] and len(got[1]) == 0


def test_identical_structure(gpu):
    rng = np.random.default_rng(4)
    ac, av = random_coords(rng, (50, 60, 70), 30000)
    bv = rng.uniform(-1, 1, len(av)).astype(np.float32)
    assert_csf_equal(run((50, 60, 70), ac, av, ac, bv, gpu), want(ac, av, ac, bv), "same")


def test_c5_reduced(gpu):
    """The C5 generator (Zipf(1.3) mode 0) at 2M draws per operand."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = (synth.zipf3_coords(2_000_000, synth.C5_SHAPE, s) for s in (1, 2))
    assert_csf_equal(run(synth.C5_SHAPE, ac, av, bc, bv, gpu), want(ac, av, bc, bv), "C5 2M")


def test_c5_full_size(gpu):
    """The C5 configuration at its full size (20M draws per operand)."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = synth.c5_operands()
    assert_csf_equal(run(synth.C5_SHAPE, ac, av, bc, bv, gpu), want(ac, av, bc, bv), "C5 full")
