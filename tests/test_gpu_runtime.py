"""GPU tests of the runtime around the kernels: input validation (nacho_validate_csr and the
validation mode) and stream-ordered buffer reuse across streams (nacho_record_stream)."""

import numpy as np
import pytest
import torch

from tests.helpers import csr_from_rows, random_csr
from tests.test_gpu_csr import to_gpu

pytestmark = pytest.mark.gpu


def _malformed_cases():
    rows, cols = 4, 6
    good = csr_from_rows(rows, cols, [[0, 2], [], [1, 3, 5], [4]])
    cases = {"good": good}
    pos, crd, val = (x.copy() for x in good)
    crd[3], crd[4] = crd[4], crd[3]  # row 2 unsorted
    cases["unsorted"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    crd[3] = crd[2]  # row 2: duplicate column
    cases["duplicate"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    crd[0] = cols  # column out of range
    cases["column_range"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    pos[2], pos[3] = 4, 2  # offsets decrease
    cases["decreasing"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    pos[0] = 1
    cases["first_offset"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    pos[4] = 5  # last offset short of nnz
    cases["last_offset"] = (pos, crd, val)
    pos, crd, val = (x.copy() for x in good)
    pos[1] = 99  # an offset past nnz (reported, never used as an index)
    cases["offset_past_end"] = (pos, crd, val)
    return rows, cols, cases


@pytest.mark.parametrize("case", ["good", "unsorted", "duplicate", "column_range", "decreasing",
                                  "first_offset", "last_offset", "offset_past_end"])
def test_validate_csr(gpu, case):
    import nacho_amd

    rows, cols, cases = _malformed_cases()
    print(f"[gpu] validate_csr case={case}", flush=True)
    t = to_gpu(cases[case], rows, cols, gpu)
    if case == "good":
        nacho_amd.validate_csr(t)
    else:
        with pytest.raises(ValueError, match="input contract"):
            nacho_amd.validate_csr(t)


def test_validate_csr_large_valid_operand(gpu):
    import nacho_amd

    rng = np.random.default_rng(5)
    a = random_csr(rng, 20000, 30000, 0.002)
    nacho_amd.validate_csr(to_gpu(a, 20000, 30000, gpu))


def test_validation_mode_guards_the_entry_points(gpu):
    import nacho_amd

    rows, cols, cases = _malformed_cases()
    good, bad = (to_gpu(cases[k], rows, cols, gpu) for k in ("good", "unsorted"))
    nacho_amd.set_validation(True)
    try:
        with pytest.raises(ValueError):
            nacho_amd.gpu_csr_add_f32(good, bad)
        with pytest.raises(ValueError):
            nacho_amd.gpu_csr_mul_f32(bad, good)
        z = nacho_amd.gpu_csr_add_f32(good, good)
        torch.cuda.synchronize()
        assert z.dim_j_indices.numel() == cases["good"][1].size
    finally:
        nacho_amd.set_validation(False)


def test_record_stream_orders_reuse_after_a_side_stream(gpu):
    """A result read on a side stream (behind a long spin) and then dropped: with
    record_stream, the next call on the main stream, which reuses the freed blocks and
    writes different values into them, must not overwrite them before the side stream's
    read."""
    import nacho_amd

    rng = np.random.default_rng(11)
    rows, cols = 4000, 5000
    a = random_csr(rng, rows, cols, 0.01)
    b = random_csr(rng, rows, cols, 0.01)
    na = (a[0], a[1], -a[2])
    nb = (b[0], b[1], -b[2])
    ga, gb, gna, gnb = (to_gpu(t, rows, cols, gpu) for t in (a, b, na, nb))
    main = torch.cuda.current_stream(gpu)
    side = torch.cuda.Stream(gpu)
    reuse = []
    for trial in range(3):
        z = nacho_amd.gpu_csr_add_f32(ga, gb)
        expected = z.values.clone()
        ptr = z.values.data_ptr()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            torch.cuda._sleep(20_000_000)
            seen = z.values.clone()
        z.record_stream(side)
        del z
        z2 = nacho_amd.gpu_csr_add_f32(gna, gnb)  # same sizes: reuses the freed blocks
        # z's values block, which the side stream reads, taken by either array of z2 (both are
        # of one size class)
        reused = ptr in (z2.values.data_ptr(), z2.dim_j_indices.data_ptr())
        reuse.append(reused)
        torch.cuda.synchronize()
        print(f"[gpu] record_stream trial={trial} reused={reused}", flush=True)
        assert torch.equal(seen, expected)
        assert torch.equal(z2.values, -expected)
        del z2
    # the ordering was exercised: some trial's second call wrote into the recorded block
    assert any(reuse), reuse


def test_cache_limit_returns_memory_to_the_driver(gpu):
    """With a cap of 0 nothing released stays cached; without a cap the call's released
    buffers stay for reuse until nacho_release_cached_memory; results stay correct."""
    import nacho_amd
    from oracle import oracle
    from tests.helpers import assert_csr_equal
    from tests.test_gpu_csr import from_gpu

    rng = np.random.default_rng(21)
    rows, cols = 20000, 20000
    a, b = random_csr(rng, rows, cols, 0.002), random_csr(rng, rows, cols, 0.002)
    want = oracle.closed_csr_binary("add", rows, cols, *a, *b)
    ga, gb = to_gpu(a, rows, cols, gpu), to_gpu(b, rows, cols, gpu)
    try:
        print("[gpu] cache limit 0", flush=True)
        nacho_amd.set_cache_limit(0)
        assert nacho_amd.cached_bytes() == 0
        for _ in range(3):
            z = nacho_amd.gpu_csr_add_f32(ga, gb)
            assert_csr_equal(from_gpu(z), want, "limit 0")
            del z
            torch.cuda.synchronize()
            assert nacho_amd.cached_bytes() == 0
        print("[gpu] cache unlimited", flush=True)
        nacho_amd.set_cache_limit(None)
        z = nacho_amd.gpu_csr_add_f32(ga, gb)
        assert_csr_equal(from_gpu(z), want, "unlimited")
        del z
        torch.cuda.synchronize()
        assert nacho_amd.cached_bytes() > 0
        held = nacho_amd.cached_bytes()
        nacho_amd.set_cache_limit(held // 2)  # trims at once
        assert nacho_amd.cached_bytes() <= held // 2
    finally:
        nacho_amd.set_cache_limit(None)
    nacho_amd.release_cached_memory()
    assert nacho_amd.cached_bytes() == 0


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, (1 << 24) + 16 * 1000])
def test_device_copy_is_exact(gpu, nbytes):
    """nacho_device_copy (the bandwidth reference of the roofline) copies every byte and
    nothing past the end, whole passes and a partial last pass alike."""
    import ctypes

    from nacho_amd import _lib

    lib = _lib.load()
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=gpu)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    print(f"[gpu] device copy {nbytes} bytes", flush=True)
    rc = lib.nacho_device_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                               nbytes, ctypes.c_void_p(stream))
    assert rc == 0, _lib.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert not dst[nbytes:].any()
