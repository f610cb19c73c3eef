"""GPU parity of the ESC SpGEMM (gfx950 kernels through the C ABI) against the CPU oracle.

Bar: structure (pos, crd) exact; values within rel 1e-5 / abs 1e-6 of the float64-accumulated
oracle (the GPU sums float32 products in float64 and rounds once, so it sits far inside).
Cases cover the reference smoke shapes (tests/smoke.py:213-218), the tile geometry (rows
sharing tiles, rows of exactly one tile, rows needing several merge levels, runs of equal
columns crossing tiles), wide column ranges (64-bit sort keys), empty operands and the full
R-MAT scale-20 square, checked row by row against the oracle and by a size-independent
checksum.
"""

import os

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import check_csr_invariants, csr_from_rows, random_csr

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def to_gpu(t, rows, cols, device):
    import nacho_amd

    pos, crd, val = t
    return nacho_amd.CSR_gpu(torch.from_numpy(np.asarray(pos, np.int32)).to(device),
                             torch.from_numpy(np.asarray(crd, np.int32)).to(device),
                             torch.from_numpy(np.asarray(val, np.float32)).to(device),
                             torch.tensor([rows, cols], dtype=torch.int32))


def spgemm(a, b, rows, inner, cols, device, wide=True):
    import nacho_amd

    fn = nacho_amd.gpu_spgemm64_f32 if wide else nacho_amd.gpu_spgemm_f32
    print(f"[gpu] spgemm{'64' if wide else ''} {rows}x{inner} @ {inner}x{cols} "
          f"nnz=({len(a[1])},{len(b[1])})", flush=True)
    z = fn(to_gpu(a, rows, inner, device), to_gpu(b, inner, cols, device))
    torch.cuda.synchronize()
    assert tuple(z.shape.tolist()) == (rows, cols)
    return (z.dim_j_offsets.cpu().numpy(), z.dim_j_indices.cpu().numpy(),
            z.values.cpu().numpy())


@pytest.fixture(params=["staged", "symbolic"])
def output_mode(request, monkeypatch):
    """Both ways of sizing the result: staged output and copy, or the symbolic pass first
    (NACHO_SPGEMM_OUTPUT; by default the library picks by free memory)."""
    monkeypatch.setenv("NACHO_SPGEMM_OUTPUT", request.param)
    return request.param


def check(rows, inner, cols, a, b, z, what):
    pos, crd, val = z
    check_csr_invariants(pos, crd, rows, cols)
    wp, wc, wv = oracle.port_spgemm(rows, inner, cols, *a, *b)
    np.testing.assert_array_equal(np.asarray(pos, np.int64), wp, err_msg=f"{what}: pos")
    np.testing.assert_array_equal(crd, wc, err_msg=f"{what}: crd")
    np.testing.assert_allclose(val, wv, rtol=RTOL, atol=ATOL, err_msg=f"{what}: values")


def run_and_check(gpu, rows, inner, cols, a, b, what, wide=True):
    z = spgemm(a, b, rows, inner, cols, gpu, wide)
    check(rows, inner, cols, a, b, z, what)
    return z


@pytest.mark.parametrize("wide", [True, False])
def test_reference_smoke_case(gpu, wide, output_mode):
    rng = np.random.default_rng(0)
    a = random_csr(rng, 200, 180, 0.05)
    b = random_csr(rng, 180, 200, 0.05)
    z = run_and_check(gpu, 200, 180, 200, a, b, "smoke", wide)
    assert z[0].dtype == (np.int64 if wide else np.int32)


@pytest.mark.parametrize("shape,density,seed", [((1000, 800, 1200), 0.01, 1),
                                                ((3000, 3000, 3000), 0.003, 2),
                                                ((64, 5000, 64), 0.3, 3),
                                                ((1, 300, 20000), 0.5, 4),
                                                ((20000, 50, 1), 0.2, 5)])
def test_random_shapes(gpu, shape, density, seed, output_mode):
    rows, inner, cols = shape
    rng = np.random.default_rng(seed)
    a = random_csr(rng, rows, inner, density)
    b = random_csr(rng, inner, cols, density)
    run_and_check(gpu, rows, inner, cols, a, b, f"random{shape}")


def product_rows(lengths, cols, rng):
    """A (len(lengths) x len(lengths)) diagonal-pattern A times B whose row r has lengths[r]
    distinct columns: row r of the product has exactly lengths[r] products."""
    n = len(lengths)
    a = csr_from_rows(n, n, [[r] for r in range(n)],
                      rng.uniform(0.5, 1.5, n).astype(np.float32))
    rows_b = [np.sort(rng.choice(cols, size=L, replace=False)).tolist() for L in lengths]
    nb = sum(lengths)
    b = csr_from_rows(n, cols, rows_b, rng.uniform(-1, 1, nb).astype(np.float32))
    return a, b


def test_tile_boundaries(gpu, output_mode):
    """Rows of exactly 1, kShort, kShort+1, one tile, one tile + 1 and several tiles of
    products, with empty rows between (tiles: 4096 products; short rows: <= 2048)."""
    rng = np.random.default_rng(7)
    lengths = [0, 1, 2047, 2048, 0, 2049, 4095, 4096, 4097, 0, 0, 8192, 8193, 3, 12289,
               20481, 1, 1, 1, 2, 40000, 0, 5, 0]
    a, b = product_rows(lengths, 50000, rng)
    n = len(lengths)
    run_and_check(gpu, n, n, 50000, a, b, "tile boundaries")


def test_many_short_rows_share_tiles(gpu, output_mode):
    rng = np.random.default_rng(8)
    lengths = rng.integers(0, 40, 30000)
    lengths[rng.random(30000) < 0.3] = 0
    lengths[:5] = 0
    lengths[-7:] = 0
    a, b = product_rows(lengths.tolist(), 500, rng)
    n = len(lengths)
    run_and_check(gpu, n, n, 500, a, b, "short rows")


def test_long_runs_cross_tiles(gpu):
    """One row with 9000 A entries whose B rows all hold columns {5, 7}: two runs of 9000
    equal columns crossing tile boundaries (and merge levels)."""
    rng = np.random.default_rng(9)
    inner = 9000
    a = csr_from_rows(2, inner, [list(range(inner)), [3, 17]],
                      rng.uniform(-1, 1, inner + 2).astype(np.float32))
    b = csr_from_rows(inner, 10, [[5, 7]] * inner,
                      rng.uniform(-1, 1, 2 * inner).astype(np.float32))
    pos, crd, val = run_and_check(gpu, 2, inner, 10, a, b, "long runs")
    assert pos.tolist() == [0, 2, 4] and crd.tolist() == [5, 7, 5, 7]


def _hub_operands(rng, cols):
    """A with a heavy row (3000 A entries, every third B row empty, about 3.5e5 products:
    several staged chunks, above the heavy-row threshold), a row of 1025 entries, rows with
    products just around the short-row limit, and empty rows; B's rows have 0-400 distinct
    columns in [0, cols)."""
    inner = 4000
    lens_b = rng.integers(1, 400, inner)
    lens_b[::3] = 0
    rows_b = [np.sort(rng.choice(cols, size=int(L), replace=False)).tolist() for L in lens_b]
    nnz_b = int(lens_b.sum())
    b = csr_from_rows(inner, cols, rows_b, rng.uniform(-1, 1, nnz_b).astype(np.float32))
    rows_a = [sorted(rng.choice(inner, size=3000, replace=False).tolist()), [],
              sorted(rng.choice(inner, size=1025, replace=False).tolist()),
              [1, 2], [0, 3, 6], []]
    # a short row of exactly kShort (2048) products and a long one of kShort + 1
    for target in (2048, 2049):
        row, total = [], 0
        for j in rng.permutation(inner):
            if lens_b[j] > 0 and total + lens_b[j] <= target:
                row.append(int(j))
                total += int(lens_b[j])
            if total == target:
                break
        rows_a.append(sorted(row))
    rows = len(rows_a)
    nnz_a = sum(len(r) for r in rows_a)
    a = csr_from_rows(rows, inner, rows_a, rng.uniform(0.5, 1.5, nnz_a).astype(np.float32))
    return rows, inner, a, b


@pytest.mark.parametrize("cols", [1 << 20, (1 << 20) - 5, 8192, 8193])
def test_symbolic_pass_hub_rows(gpu, cols, monkeypatch):
    """The symbolic pass sizes the result (columns fit its 2^20-bit row bitmap): long rows
    staged in several chunks with empty B rows among their A entries, a row above the
    heavy-row threshold, short rows at the short-row limit; one bucket (cols <= 8192) and
    8192-column buckets with a partial last one."""
    monkeypatch.setenv("NACHO_SPGEMM_OUTPUT", "symbolic")
    rng = np.random.default_rng(cols % 997)
    rows, inner, a, b = _hub_operands(rng, cols)
    run_and_check(gpu, rows, inner, cols, a, b, f"symbolic hub rows cols={cols}")


def test_staged_and_symbolic_outputs_agree(gpu, monkeypatch):
    """NACHO_SPGEMM_OUTPUT=staged runs the units into a staging buffer at their product
    offsets and copies them to the result; =symbolic sizes the result first with the
    symbolic pass.  Both match the oracle and each other's structure exactly."""
    from nacho_amd import synth

    n = 1 << 14
    t = synth.rmat_csr(14, seed=6)
    rng = np.random.default_rng(11)
    rows, inner, a, b = _hub_operands(rng, 1 << 20)
    for what, args in (("rmat14", (n, n, n, t, t)), ("hub rows", (rows, inner, 1 << 20, a, b))):
        z = {}
        for mode in ("staged", "symbolic"):
            monkeypatch.setenv("NACHO_SPGEMM_OUTPUT", mode)
            z[mode] = run_and_check(gpu, *args, f"{what} {mode}")
        np.testing.assert_array_equal(z["staged"][0], z["symbolic"][0])
        np.testing.assert_array_equal(z["staged"][1], z["symbolic"][1])
        np.testing.assert_allclose(z["staged"][2], z["symbolic"][2], rtol=RTOL, atol=ATOL)


def test_wide_columns_use_64bit_keys(gpu):
    """cols > 2^20 leaves fewer than 12 free key bits, so the 64-bit sort key path runs."""
    rng = np.random.default_rng(10)
    rows, inner, cols = 4000, 3000, 3_000_000
    a = random_csr(rng, rows, inner, 0.002)
    pb = np.zeros(inner + 1, np.int32)
    lens = rng.integers(0, 30, inner)
    pb[1:] = np.cumsum(lens)
    cb = np.concatenate([np.sort(rng.choice(cols, size=L, replace=False)) for L in lens])
    vb = rng.uniform(-1, 1, len(cb)).astype(np.float32)
    run_and_check(gpu, rows, inner, cols, a, (pb, cb.astype(np.int32), vb), "wide cols")


def test_cancellation_keeps_entry(gpu, output_mode):
    a = csr_from_rows(1, 2, [[0, 1]], np.array([1.0, -1.0], np.float32))
    b = csr_from_rows(2, 5, [[3], [3]], np.array([2.5, 2.5], np.float32))
    pos, crd, val = spgemm(a, b, 1, 2, 5, gpu)
    assert pos.tolist() == [0, 1] and crd.tolist() == [3] and val.tolist() == [0.0]


@pytest.mark.parametrize("wide", [True, False])
def test_empty_operands(gpu, wide, output_mode):
    a = csr_from_rows(3, 4, [[], [], []])
    b = csr_from_rows(4, 5, [[1], [], [2], []])
    pos, crd, val = spgemm(a, b, 3, 4, 5, gpu, wide)
    assert pos.tolist() == [0, 0, 0, 0] and len(crd) == 0 and len(val) == 0
    # A's columns hit only empty rows of B
    a = csr_from_rows(3, 4, [[1, 3], [], [1]])
    pos, crd, val = spgemm(a, b, 3, 4, 5, gpu, wide)
    assert pos.tolist() == [0, 0, 0, 0] and len(crd) == 0
    # no rows at all
    a = csr_from_rows(0, 4, [])
    pos, crd, val = spgemm(a, b, 0, 4, 5, gpu, wide)
    assert pos.tolist() == [0]


def test_identity_exact(gpu, output_mode):
    rng = np.random.default_rng(11)
    n = 5000
    a = random_csr(rng, n, n, 0.002)
    eye = csr_from_rows(n, n, [[i] for i in range(n)], np.ones(n, np.float32))
    pos, crd, val = spgemm(a, eye, n, n, n, gpu)
    np.testing.assert_array_equal(pos, a[0])
    np.testing.assert_array_equal(crd, a[1])
    np.testing.assert_array_equal(val, a[2])


def test_dimension_mismatch_raises(gpu):
    import nacho_amd

    a = csr_from_rows(2, 3, [[0], [1]])
    b = csr_from_rows(4, 3, [[0], [], [], []])
    with pytest.raises(Exception):
        nacho_amd.gpu_spgemm64_f32(to_gpu(a, 2, 3, gpu), to_gpu(b, 4, 3, gpu))


def test_rmat_medium(gpu, output_mode):
    from nacho_amd import synth

    n = 1 << 15
    pos, crd, val = synth.rmat_csr(15, seed=4)
    t = (pos, crd, val)
    run_and_check(gpu, n, n, n, t, t, "rmat15")


def test_repeatable(gpu, output_mode):
    """Structure is identical run to run; values agree to within one float32 rounding of the
    float64 sums (their summation order follows the scatter's arrival order)."""
    from nacho_amd import synth

    n = 1 << 13
    t = synth.rmat_csr(13, seed=5)
    z1 = spgemm(t, t, n, n, n, gpu)
    z2 = spgemm(t, t, n, n, n, gpu)
    np.testing.assert_array_equal(z1[0], z2[0])
    np.testing.assert_array_equal(z1[1], z2[1])
    np.testing.assert_allclose(z1[2], z2[2], rtol=2.5e-7, atol=0)


def test_dense_windows_and_wide_keys(gpu):
    """cols = 2^24 + 3: column buckets of 2^15 columns, so a dense bucket is accumulated in
    four 8192-column windows, and sort keys need 64 bits."""
    rng = np.random.default_rng(13)
    cols = (1 << 24) + 3
    inner = 600
    # B rows: 40 columns in [0, 32768) (bucket 0) and a few spread over the whole range
    rows_b = []
    for _ in range(inner):
        near = rng.choice(32768, size=40, replace=False)
        far = rng.choice(cols, size=3, replace=False)
        rows_b.append(np.unique(np.concatenate([near, far])).tolist())
    b = csr_from_rows(inner, cols, rows_b,
                      rng.uniform(-1, 1, sum(len(r) for r in rows_b)).astype(np.float32))
    # row 0: every B row (24000+ products, dense bucket 0); row 1: a short row; row 2 empty
    a = csr_from_rows(3, inner, [list(range(inner)), [5, 77, 300], []],
                      rng.uniform(0.5, 1.5, inner + 3).astype(np.float32))
    run_and_check(gpu, 3, inner, cols, a, b, "dense windows")


def _oracle_threads():
    return max(1, min(len(os.sched_getaffinity(0)), 16))


def _row_blocks(zpos, max_rows, max_entries):
    """Cut [0, rows) into consecutive row ranges of at most `max_rows` rows and, where a
    single row allows it, at most `max_entries` result entries (by the offsets `zpos`)."""
    rows = len(zpos) - 1
    r0 = 0
    while r0 < rows:
        limit = min(rows, r0 + max_rows)
        r1 = int(np.searchsorted(zpos, zpos[r0] + max_entries, side="right")) - 1
        r1 = max(r0 + 1, min(r1, limit))
        yield r0, r1
        r0 = r1


def _first_bad(got_c, want_c, got_v, want_v):
    """Index of the first entry whose column differs or whose value is out of tolerance
    (rel 1e-5 / abs 1e-6), or -1.  Device tensors of equal length."""
    bad = got_c != want_c
    bad |= (got_v - want_v).abs() > ATOL + RTOL * want_v.abs()
    bad |= got_v.isnan() != want_v.isnan()
    if not bool(bad.any().item()):
        return -1
    return int(torch.argmax(bad.to(torch.uint8)).item())


def test_c4_full_size(gpu):
    """R-MAT scale 20 squared: 6.0e9 products, 3.6e9 results (int64 offsets).  Every row is
    compared with the oracle: in row blocks (at most 2^16 rows or 2^28 entries each) the
    oracle runs on the same rows of A, its offsets are compared on the host and its columns
    and values, uploaded, on the device; nnz(C) must equal the oracle's total.  The row-sum identity sum_ik C_ik = sum_j colsum(A)_j rowsum(A)_j checks
    the values once more as a whole, and the int32 entry point must refuse the result."""
    import nacho_amd
    from nacho_amd import synth

    n = 1 << 20
    pos, crd, val = synth.c4_operand()
    a_gpu = to_gpu((pos, crd, val), n, n, gpu)
    print("[gpu] spgemm64 C4", flush=True)
    z = nacho_amd.gpu_spgemm64_f32(a_gpu, a_gpu)
    torch.cuda.synchronize()
    zpos = z.dim_j_offsets
    nnz = int(zpos[-1].item())
    assert nnz == z.values.numel() == z.dim_j_indices.numel()
    assert nnz > 2**31  # the reason for 64-bit offsets
    zpos_h = zpos.cpu().numpy()
    assert zpos_h[0] == 0 and bool(np.all(zpos_h[1:] >= zpos_h[:-1]))
    # checksum over every value
    total = float(z.values.to(torch.float64).sum().item())
    v64 = val.astype(np.float64)
    lens = np.diff(pos).astype(np.int64)
    row_of = np.repeat(np.arange(n), lens)
    colsum = np.bincount(crd, weights=v64, minlength=n)
    rowsum = np.bincount(row_of, weights=v64, minlength=n)
    want = float(np.dot(colsum, rowsum))
    # every entry is rounded once to float32 (relative error <= 2^-24)
    assert total == pytest.approx(want, rel=1e-7)
    # every row against the oracle, block by block (the comparison runs on the device)
    threads = _oracle_threads()
    oracle_total = 0
    for r0, r1 in _row_blocks(zpos_h, 1 << 16, 1 << 28):
        s, e = int(zpos_h[r0]), int(zpos_h[r1])
        a0, a1 = int(pos[r0]), int(pos[r1])
        wp, wc, wv = oracle.port_spgemm(r1 - r0, n, n, pos[r0:r1 + 1] - pos[r0],
                                        crd[a0:a1], val[a0:a1], pos, crd, val,
                                        nthreads=threads)
        oracle_total += int(wp[-1])
        np.testing.assert_array_equal(zpos_h[r0:r1 + 1] - s, wp,
                                      err_msg=f"offsets of rows [{r0}, {r1})")
        wc_d = torch.from_numpy(wc).to(gpu)
        wv_d = torch.from_numpy(wv).to(gpu)
        gc, gv = z.dim_j_indices[s:e], z.values[s:e]
        bad = _first_bad(gc, wc_d, gv, wv_d)
        if bad >= 0:
            r = r0 + int(np.searchsorted(wp, bad, side="right")) - 1
            pytest.fail(f"row {r}, entry {bad - int(wp[r - r0])}: got column "
                        f"{int(gc[bad].item())} value {float(gv[bad].item())!r}, oracle "
                        f"column {int(wc[bad])} value {float(wv[bad])!r}")
        del wp, wc, wv, wc_d, wv_d
    assert oracle_total == nnz
    del z
    try:
        with pytest.raises(RuntimeError, match="exceeds int32"):
            nacho_amd.gpu_spgemm_f32(a_gpu, a_gpu)
    finally:
        torch.cuda.synchronize()
        nacho_amd.release_cached_memory()


def test_c4_symbolic_matches_staged(gpu, monkeypatch):
    """The C4 square with the symbolic pass sizing the result (the path taken when the
    staging buffer would not fit) equals the staged path's result, which
    test_c4_full_size checks row by row against the oracle: offsets and columns exactly,
    values within the tolerance (the two runs' float64 sums may differ in order)."""
    import nacho_amd
    from nacho_amd import synth

    n = 1 << 20
    pos, crd, val = synth.c4_operand()
    a_gpu = to_gpu((pos, crd, val), n, n, gpu)
    z = {}
    for mode in ("staged", "symbolic"):
        monkeypatch.setenv("NACHO_SPGEMM_OUTPUT", mode)
        print(f"[gpu] spgemm64 C4 {mode}", flush=True)
        z[mode] = nacho_amd.gpu_spgemm64_f32(a_gpu, a_gpu)
        torch.cuda.synchronize()
    staged, symbolic = z.pop("staged"), z.pop("symbolic")
    try:
        assert torch.equal(staged.dim_j_offsets, symbolic.dim_j_offsets)
        assert torch.equal(staged.dim_j_indices, symbolic.dim_j_indices)
        nnz = staged.values.numel()
        step = 1 << 28
        for i in range(0, nnz, step):
            x = staged.values[i:i + step].to(torch.float64)
            y = symbolic.values[i:i + step].to(torch.float64)
            assert bool(((x - y).abs() <= ATOL + RTOL * y.abs()).all()), f"values [{i}, +{step})"
    finally:
        del staged, symbolic
        torch.cuda.synchronize()
        nacho_amd.release_cached_memory()
