"""Real-data path on the GPU, against the oracle (bit-exact): a Matrix Market file read by
parse2D, converted with to_csr and added / multiplied on the device; and generated files of
more than 1M entries prepared as `bench.py --workload mtx|tns` prepares them (.mtx pairs
clipped to a common shape; a .tns file sorted, summed and paired with its shifted copy)."""

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op", ["add", "mul"])
def test_mtx_file_through_csr_kernels(gpu, tmp_path, op):
    import nacho_amd
    from nacho_amd import io

    rng = np.random.default_rng(11)
    a = sp.random(3000, 3000, density=0.002, format="coo", random_state=1)
    a = sp.triu(a + a.T, format="coo")  # symmetric upper triangle; the reader mirrors it
    a.data = rng.uniform(-1, 1, a.nnz)
    f = tmp_path / "a.mtx"
    scipy.io.mmwrite(str(f), a, symmetry="symmetric")
    ta = io.parse_matrix(f, device="cpu")
    tb = (ta.to_dense() * 2.0 + torch.diag(torch.ones(3000))).to_sparse_csr()
    print(f"[gpu] mtx {op} nnz=({ta.values().numel()},{tb.values().numel()})", flush=True)
    fn = nacho_amd.gpu_csr_add_f32 if op == "add" else nacho_amd.gpu_csr_mul_f32
    z = fn(nacho_amd.to_csr(ta, gpu), nacho_amd.to_csr(tb, gpu))
    torch.cuda.synchronize()
    np_of = lambda t: (t.crow_indices().numpy().astype(np.int32),  # noqa: E731
                       t.col_indices().numpy().astype(np.int32),
                       t.values().numpy().astype(np.float32))
    pos, crd, val = oracle.port_csr_binary(op, 3000, *np_of(ta), *np_of(tb))
    np.testing.assert_array_equal(z.dim_j_offsets.cpu().numpy(), pos)
    np.testing.assert_array_equal(z.dim_j_indices.cpu().numpy(), crd)
    np.testing.assert_array_equal(z.values.cpu().numpy().view(np.int32), val.view(np.int32))


def _write_mtx(path, rows, cols, r, c, v):
    """A general `coordinate real` Matrix Market file, entries in the order given."""
    with open(path, "w") as f:
        f.write("%%MatrixMarket matrix coordinate real general\n")
        f.write(f"{rows} {cols} {len(v)}\n")
        np.savetxt(f, np.column_stack((r + 1, c + 1, v)), fmt="%d %d %.9g")


def _write_tns(path, coords, v):
    with open(path, "w") as f:
        np.savetxt(f, np.column_stack((coords + 1, v)), fmt="%d %d %d %.9g")


def _random_entries(rng, rows, cols, n):
    """n random (row, col, value) in shuffled order, with some coordinates repeated (the
    reader sums repeats)."""
    r = rng.integers(0, rows, n)
    c = rng.integers(0, cols, n)
    rep = rng.choice(n, n // 50, replace=False)  # 2% repeat an earlier coordinate
    r[rep[1:]] = r[rep[:-1]]
    c[rep[1:]] = c[rep[:-1]]
    v = rng.uniform(-1, 1, n).astype(np.float32)
    return r, c, v


def test_large_mtx_pair_as_the_bench_runs_it(gpu, tmp_path):
    """Two generated .mtx files of 1.2M entries and different shapes, read, summed over
    repeats and clipped to a common shape as `bench.py --workload mtx` does, then csr_add
    and csr_mul against the oracle (bit-exact)."""
    import nacho_amd
    from nacho_amd import io

    rng = np.random.default_rng(21)
    files = []
    for name, (rows, cols) in (("a.mtx", (300_000, 250_000)), ("b.mtx", (280_000, 260_000))):
        r, c, v = _random_entries(rng, rows, cols, 1_200_000)
        # share a quarter of A's coordinates so the multiply has work
        if name == "b.mtx":
            k = len(v) // 4
            keep = ra < 280_000
            r[:k], c[:k] = ra[keep][:k], ca[keep][:k]
        else:
            ra, ca = r.copy(), c.copy()
        _write_mtx(tmp_path / name, rows, cols, r, c, v)
        files.append(tmp_path / name)
    ta, tb = (io.parse_matrix(f, device="cpu") for f in files)
    assert ta.values().numel() >= 1_000_000 and tb.values().numel() >= 1_000_000
    rows, cols, a, b = io.clip_to_common_shape(ta, tb)
    assert (rows, cols) == (280_000, 260_000)

    def up(t):
        return nacho_amd.CSR_gpu(*(torch.from_numpy(x).to(gpu) for x in t),
                                 torch.tensor([rows, cols], dtype=torch.int32))

    for op, fn in (("add", nacho_amd.gpu_csr_add_f32), ("mul", nacho_amd.gpu_csr_mul_f32)):
        print(f"[gpu] mtx pair {op} {rows}x{cols} nnz=({len(a[1])},{len(b[1])})", flush=True)
        z = fn(up(a), up(b))
        torch.cuda.synchronize()
        pos, crd, val = oracle.port_csr_binary(op, rows, *a, *b)
        if op == "mul":
            assert len(crd) > 100_000
        np.testing.assert_array_equal(z.dim_j_offsets.cpu().numpy(), pos)
        np.testing.assert_array_equal(z.dim_j_indices.cpu().numpy(), crd)
        np.testing.assert_array_equal(z.values.cpu().numpy().view(np.int32), val.view(np.int32))


def test_large_tns_as_the_bench_runs_it(gpu, tmp_path):
    """A generated .tns file of 1.2M unsorted entries (with repeats), read without dims,
    sorted and summed, paired with its shifted copy as `bench.py --workload tns` does, then
    csf_add and coo3d_add against the oracle (bit-exact)."""
    import nacho_amd
    from nacho_amd import io
    from nacho_amd.convert import csf3_levels

    rng = np.random.default_rng(22)
    shape = (5_000, 4_000, 3_000)
    n = 1_200_000
    coords = np.column_stack([rng.integers(0, s, n) for s in shape])
    coords[rng.choice(n, n // 50, replace=False)] = coords[0]  # repeats
    coords[0] = np.array(shape) - 1  # the shape is taken from the largest coordinates
    v = rng.uniform(-1, 1, n).astype(np.float32)
    f = tmp_path / "t.tns"
    _write_tns(f, coords, v)
    raw_c, raw_v = io.load_frostt(f, (2**31 - 1,) * 3)
    dims = io.frostt_shape(raw_c)
    assert dims == shape and len(raw_v) == n
    ac, av = io.coalesce_coordinates(raw_c, raw_v, dims)
    bc, bv = io.shift_coordinates(ac, av, dims)
    assert len(av) >= 1_000_000
    print(f"[gpu] tns csf_add / coo3d_add shape={dims} nnz=({len(av)},{len(bv)})", flush=True)
    z = nacho_amd.gpu_csf_add_f32(nacho_amd.to_csf3(ac, av, dims, gpu),
                                  nacho_amd.to_csf3(bc, bv, dims, gpu))
    torch.cuda.synchronize()
    want_levels, want_val = oracle.port_csf3_union(csf3_levels(ac), av, csf3_levels(bc), bv)
    got = [getattr(z, k).cpu().numpy() for k in ("dim_i_indices", "dim_j_offsets",
                                                   "dim_j_indices", "dim_k_offsets",
                                                   "dim_k_indices")]
    for g, w in zip(got, want_levels):
        np.testing.assert_array_equal(g, w)
    np.testing.assert_array_equal(z.values.cpu().numpy().view(np.int32), want_val.view(np.int32))
    del z
    z = nacho_amd.gpu_coo3d_add_f32(nacho_amd.to_coo3(ac, av, dims, gpu),
                                    nacho_amd.to_coo3(bc, bv, dims, gpu))
    torch.cuda.synchronize()
    wc, wv = oracle.port_coo_binary("add", tuple(ac[:, d] for d in range(3)), av,
                                    tuple(bc[:, d] for d in range(3)), bv, nthreads=16)
    for d, k in enumerate(("dim_i_indices", "dim_j_indices", "dim_k_indices")):
        np.testing.assert_array_equal(getattr(z, k).cpu().numpy(), wc[d])
    np.testing.assert_array_equal(z.values.cpu().numpy().view(np.int32), wv.view(np.int32))
