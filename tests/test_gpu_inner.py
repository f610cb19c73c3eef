"""GPU parity of inner_prod (CSF3) and inner_prod_coo (COO3) against the oracle.

The GPU sums the float32 products in float64 in a fixed order and rounds once; the oracle
(oracle_csf3_inner / oracle_coo3_inner, pinned in test_oracle_inner.py) sums the same
products in float64 in another order.  Tolerance: the float32 rounding of the result
(1.2e-7 relative) plus 1e-12 of the sum of |a * b| for the two float64 orders.
"""

import numpy as np
import pytest
import torch

from nacho_amd.convert import csf3_levels
from oracle import oracle
from tests.test_oracle_inner import random_coords

pytestmark = pytest.mark.gpu


def gpu_inner(kind, shape, ac, av, bc, bv, device):
    import nacho_amd

    print(f"[gpu] inner_prod {kind} shape={shape} nnz=({len(av)},{len(bv)})", flush=True)
    if kind == "csf":
        z = nacho_amd.gpu_inner_prod_f32(nacho_amd.to_csf3(ac, av, shape, device),
                                         nacho_amd.to_csf3(bc, bv, shape, device))
    else:
        z = nacho_amd.gpu_inner_prod_coo_f32(nacho_amd.to_coo3(ac, av, shape, device),
                                             nacho_amd.to_coo3(bc, bv, shape, device))
    assert isinstance(z, nacho_amd.Scalar_gpu)
    torch.cuda.synchronize()
    vals = z.values.cpu().numpy()
    assert vals.dtype == np.float32 and vals.shape == (1,)
    return float(vals[0])


def want_inner(kind, ac, av, bc, bv):
    if kind == "csf":
        return oracle.port_csf3_inner(csf3_levels(ac), av, csf3_levels(bc), bv, nthreads=16)
    return oracle.port_coo3_inner(tuple(ac[:, d] for d in range(3)), av,
                                  tuple(bc[:, d] for d in range(3)), bv, nthreads=16)


def assert_close(got, want, ac, av, bc, bv, what):
    scale = float(np.abs(av.astype(np.float64)).max(initial=0.0)
                  * np.abs(bv.astype(np.float64)).max(initial=0.0)) * min(len(av), len(bv))
    tol = 1.2e-7 * abs(want) + 1e-12 * scale
    assert abs(got - want) <= tol, f"{what}: got {got!r}, want {want!r} (tol {tol:.3g})"
    assert np.float32(got) == got


KINDS = ["csf", "coo"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("seed", range(4))
def test_random(gpu, kind, seed):
    rng = np.random.default_rng(900 + seed)
    shape = tuple(int(rng.choice([1, 7, 300, 20000])) for _ in range(3))
    n = int(rng.choice([1, 50, 5000, 400000]))
    ac, av = random_coords(rng, shape, n)
    bc, bv = random_coords(rng, shape, n)
    got = gpu_inner(kind, shape, ac, av, bc, bv, gpu)
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, f"{kind} seed={seed}")


@pytest.mark.parametrize("kind", KINDS)
def test_reference_smoke_case(gpu, kind):
    rng = np.random.default_rng(0)
    shape = (40, 30, 25)

    def random_coo_3d():
        coords = np.unique(np.stack([rng.integers(0, e, 900) for e in shape], axis=1), axis=0)
        return coords.astype(np.int32), rng.random(coords.shape[0]).astype(np.float32)

    (ac, av), (bc, bv) = random_coo_3d(), random_coo_3d()
    got = gpu_inner(kind, shape, ac, av, bc, bv, gpu)
    a_entries = {tuple(int(x) for x in c): float(v) for c, v in zip(ac, av)}
    expected = sum(a_entries[k] * float(v) for c, v in zip(bc, bv)
                   if (k := tuple(int(x) for x in c)) in a_entries)
    assert abs(got - expected) <= 1e-4 * max(1.0, abs(expected))  # the reference's TOLERANCE
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, "smoke")


@pytest.mark.parametrize("kind", KINDS)
def test_empty_and_disjoint(gpu, kind):
    rng = np.random.default_rng(12)
    shape = (30, 30, 64)
    ac, av = random_coords(rng, (30, 30, 30), 2000)
    e, ev = np.zeros((0, 3), np.int32), np.zeros(0, np.float32)
    assert gpu_inner(kind, shape, e, ev, ac, av, gpu) == 0.0
    assert gpu_inner(kind, shape, ac, av, e, ev, gpu) == 0.0
    assert gpu_inner(kind, shape, e, ev, e, ev, gpu) == 0.0
    bc = ac.copy()
    bc[:, 2] += 31  # same (i, j) fibres, every k beyond A's
    assert gpu_inner(kind, shape, ac, av, bc, av, gpu) == 0.0


@pytest.mark.parametrize("kind", KINDS)
def test_self_product(gpu, kind):
    """a . a = the sum of squares (every coordinate pairs with itself)."""
    rng = np.random.default_rng(13)
    shape = (200, 300, 100)
    ac, av = random_coords(rng, shape, 300000)
    got = gpu_inner(kind, shape, ac, av, ac, av, gpu)
    want = float(np.sum((av * av).astype(np.float64)))
    assert_close(got, want, ac, av, ac, av, "self")


@pytest.mark.parametrize("kind", KINDS)
def test_wide_keys(gpu, kind):
    """(j, k) keys that do not fit 31 bits: COO3 takes the packed-tuple intersection and sums
    its products, CSF3 the i and j level unions and the k level intersection."""
    rng = np.random.default_rng(14)
    shape = (50, 1 << 20, 1 << 20)
    ac, av = random_coords(rng, shape, 100000)
    keep = rng.random(len(ac)) < 0.5
    bc = ac[keep]
    bv = rng.uniform(-1, 1, len(bc)).astype(np.float32)
    got = gpu_inner(kind, shape, ac, av, bc, bv, gpu)
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, f"{kind} wide keys")


@pytest.mark.parametrize("kind", KINDS)
def test_sparse_rows(gpu, kind):
    """Few i coordinates spread over many rows (row offsets with long empty gaps), j and k
    extents of one (keys of no bits)."""
    rng = np.random.default_rng(16)
    shape = (1 << 20, 1, 1)
    ac, av = random_coords(rng, shape, 3000)
    bc, bv = random_coords(rng, shape, 3000)
    got = gpu_inner(kind, shape, ac, av, bc, bv, gpu)
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, f"{kind} sparse rows")


def test_c5_reduced(gpu):
    """Both layouts on the C5 generator (Zipf(1.3) mode 0) at 2M draws per operand."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = (synth.zipf3_coords(2_000_000, synth.C5_SHAPE, s) for s in (1, 2))
    csf = gpu_inner("csf", synth.C5_SHAPE, ac, av, bc, bv, gpu)
    coo = gpu_inner("coo", synth.C5_SHAPE, ac, av, bc, bv, gpu)
    want = want_inner("csf", ac, av, bc, bv)
    assert_close(csf, want, ac, av, bc, bv, "csf C5 2M")
    assert_close(coo, want, ac, av, bc, bv, "coo C5 2M")


@pytest.mark.parametrize("kind", KINDS)
def test_c5_full_size(gpu, kind):
    """The C5 operand pair at full size (20M draws each), and each operand with itself."""
    from nacho_amd import synth

    (ac, av), (bc, bv) = synth.c5_operands()
    got = gpu_inner(kind, synth.C5_SHAPE, ac, av, bc, bv, gpu)
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, f"{kind} C5")
    got = gpu_inner(kind, synth.C5_SHAPE, ac, av, ac, av, gpu)
    want = float(np.sum((av * av).astype(np.float64)))
    assert_close(got, want, ac, av, ac, av, f"{kind} C5 self")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("smaller", ["a", "b"])
def test_subset_operand(gpu, kind, smaller):
    """One operand a subset of the other's coordinates: the products are spread over the
    smaller operand's positions, whichever side that is."""
    rng = np.random.default_rng(15)
    shape = (300, 400, 500)
    big, bigv = random_coords(rng, shape, 200000)
    keep = rng.random(len(big)) < 0.3
    small = big[keep]
    smallv = rng.uniform(-1, 1, len(small)).astype(np.float32)
    ac, av, bc, bv = (small, smallv, big, bigv) if smaller == "a" else (big, bigv, small, smallv)
    got = gpu_inner(kind, shape, ac, av, bc, bv, gpu)
    assert_close(got, want_inner(kind, ac, av, bc, bv), ac, av, bc, bv, f"{kind} {smaller}")


def test_csf_empty_fibres(gpu):
    """CSF3 operands with many empty (i, j) fibres (legal for the C ABI, never built by
    to_csf3): runs of fibres with no k entries between the ones that have them, so that a
    range of k entries spans more fibres than the key kernel stages."""
    import nacho_amd

    shape = (4, 60000, 50)

    def levels_with_gaps(seed):
        r = np.random.default_rng(seed)
        ci = np.array([0, 2, 3], np.int32)
        pj, cj, pk, ck, val = [0], [], [0], [], []
        for _ in ci:
            js = np.sort(r.choice(shape[1], 20000, replace=False))
            for n, j in enumerate(js):
                cj.append(j)
                if n % 10 == 0:  # one fibre in ten holds entries
                    ks = np.sort(r.choice(shape[2], int(r.integers(1, 4)), replace=False))
                    ck.extend(ks)
                    val.extend(r.uniform(-1, 1, len(ks)))
                pk.append(len(ck))
            pj.append(len(cj))
        return ((ci, np.array(pj, np.int32), np.array(cj, np.int32), np.array(pk, np.int32),
                 np.array(ck, np.int32)), np.array(val, np.float32))

    (la, va), (lb, vb) = levels_with_gaps(1), levels_with_gaps(2)
    lb = (lb[0], lb[1], la[2], lb[3], lb[4])  # the same j coordinates, so fibres pair
    # (B keeps its own k offsets: its entries sit under every tenth fibre as well)

    def gpu_csf(levels, val):
        bufs = [torch.from_numpy(np.asarray(x, np.int32)).to(gpu) for x in levels]
        return nacho_amd.CSF3_gpu(*bufs, torch.from_numpy(val).to(gpu),
                                  torch.tensor(list(shape), dtype=torch.int32))

    print(f"[gpu] inner_prod csf empty fibres nnz=({len(va)},{len(vb)})", flush=True)
    z = nacho_amd.gpu_inner_prod_f32(gpu_csf(la, va), gpu_csf(lb, vb))
    got = float(z.values.cpu().numpy()[0])
    want = oracle.port_csf3_inner(la, va, lb, vb, nthreads=4)
    scale = float(np.abs(va).max() * np.abs(vb).max()) * min(len(va), len(vb))
    assert abs(got - want) <= 1.2e-7 * abs(want) + 1e-12 * scale, (got, want)


@pytest.mark.parametrize("with_release", [True, False])
def test_wide_keys_coo_through_a_caller_allocator(gpu, with_release):
    """inner_prod_coo with (j, k) keys wider than 31 bits (the packed-tuple intersection,
    whose result buffers the entry point frees itself) through the C ABI with a caller
    allocator: every buffer but the result goes back through `release`, and an allocator
    without `release` keeps its buffers."""
    import ctypes

    from nacho_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(15)
    shape = (50, 1 << 20, 1 << 20)
    ac, av = random_coords(rng, shape, 20000)
    bc = ac[rng.random(len(ac)) < 0.5]
    bv = rng.uniform(-1, 1, len(bc)).astype(np.float32)
    keep, handed, released = {}, [], []

    @ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p)
    def allocate(ctx, nbytes, stream):
        t = torch.empty(int(nbytes), dtype=torch.uint8, device=gpu)
        keep[t.data_ptr()] = t
        handed.append(t.data_ptr())
        return t.data_ptr()

    @ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)
    def release(ctx, ptr, stream):
        released.append(ptr)

    alloc = _lib.Allocator(None, allocate, release) if with_release else \
        _lib.Allocator(None, allocate, ctypes.cast(None, _lib.Allocator._fields_[2][1]))

    def desc(c, v):
        cols = [torch.from_numpy(np.ascontiguousarray(c[:, d])).to(gpu) for d in range(3)]
        vals = torch.from_numpy(v).to(gpu)
        keep[id(cols[0])] = (cols, vals)
        n = len(v)
        return _lib.Coo3Desc(shape[0], shape[1], shape[2], n, cols[0].data_ptr(), n,
                             cols[1].data_ptr(), n, cols[2].data_ptr(), vals.data_ptr(), n)

    da, db = desc(ac, av), desc(bc, bv)
    z = _lib.ScalarDesc()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    print(f"[gpu] inner_prod_coo wide keys, caller allocator, release={with_release}",
          flush=True)
    rc = lib.nacho_gpu_inner_prod_coo_f32(ctypes.byref(da), ctypes.byref(db), ctypes.byref(z),
                                          256, 256, ctypes.c_void_p(stream),
                                          ctypes.byref(alloc))
    assert rc == 0, _lib.error_string(rc)
    torch.cuda.synchronize()
    assert z.nnz == 1 and z.values in keep
    got = float(keep[z.values].view(torch.float32)[:1].cpu().numpy()[0])
    assert_close(got, want_inner("coo", ac, av, bc, bv), ac, av, bc, bv, "caller allocator")
    if with_release:
        assert sorted(released) == sorted(p for p in handed if p != z.values)
    else:
        assert not released
