"""Matrix Market / FROSTT readers (nacho_parse2d / nacho_parse3d, host C++), CPU only.

The reference readers (runtime/io/parse.h:28-263) have no tests of their own; these pin the
C++ readers against scipy.io.mmread, against the C library's strtof for .tns values, and
against the reference's documented handling of symmetric and skew-symmetric files (mirrored
off-diagonal entries appended after the file's entries, in file order).
"""

import ctypes

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

import nacho_amd
from nacho_amd import io


def write(path, text):
    path.write_text(text)
    return str(path)


def test_general_matches_scipy(tmp_path):
    rng = np.random.default_rng(1)
    m = sp.random(300, 200, density=0.03, format="coo", random_state=2)
    m.data = rng.normal(size=m.nnz) * 10.0 ** rng.integers(-30, 30, m.nnz)
    f = tmp_path / "g.mtx"
    scipy.io.mmwrite(str(f), m, comment="written by scipy", precision=17)
    got = nacho_amd.parse2D(str(f))
    want = scipy.io.mmread(str(f)).tocoo()
    assert (got.N, got.M) == want.shape
    np.testing.assert_array_equal(got.row.numpy(), want.row)
    np.testing.assert_array_equal(got.col.numpy(), want.col)
    np.testing.assert_array_equal(got.data.numpy().view(np.int32),
                                  want.data.astype(np.float32).view(np.int32))
    assert got.row.dtype == torch.int32 and got.data.dtype == torch.float32


def test_symmetric_and_skew_mirror_in_file_order(tmp_path):
    text = ("%%MatrixMarket matrix coordinate real {}\n% comment\n%another\n"
            "4 4 4\n1 1 1.5\n3 1 -2.0\n4 2 0.25\n2 4 7\n")
    sym = nacho_amd.parse2D(write(tmp_path / "s.mtx", text.format("symmetric")))
    assert sym.row.tolist() == [0, 2, 3, 1, 0, 1, 3]
    assert sym.col.tolist() == [0, 0, 1, 3, 2, 3, 1]
    assert sym.data.tolist() == [1.5, -2.0, 0.25, 7.0, -2.0, 0.25, 7.0]
    skew = nacho_amd.parse2D(write(tmp_path / "k.mtx", text.format("skew-symmetric")))
    assert skew.row.tolist() == sym.row.tolist() and skew.col.tolist() == sym.col.tolist()
    assert skew.data.tolist() == [1.5, -2.0, 0.25, 7.0, 2.0, -0.25, -7.0]
    # scipy agrees on the matrix (order aside)
    want = scipy.io.mmread(str(tmp_path / "s.mtx")).toarray()
    got = sp.coo_matrix((sym.data.numpy(), (sym.row.numpy(), sym.col.numpy())), shape=(4, 4))
    np.testing.assert_array_equal(got.toarray(), want)


@pytest.mark.parametrize("header", [
    "%%MatrixMarket matrix coordinate pattern general",
    "%%MatrixMarket matrix coordinate integer general",
    "%%MatrixMarket matrix coordinate complex general",
    "%%MatrixMarket matrix coordinate real hermitian",
    "%%MatrixMarket vector coordinate real general",
])
def test_unsupported_variants_raise(tmp_path, header):
    with pytest.raises(RuntimeError, match="unsupported"):
        nacho_amd.parse2D(write(tmp_path / "u.mtx", header + "\n2 2 1\n1 1 1\n"))


def test_malformed_and_missing_files_raise(tmp_path):
    with pytest.raises(RuntimeError, match="malformed"):
        nacho_amd.parse2D(write(tmp_path / "b.mtx", "%%Matrix matrix coordinate real general\n"))
    with pytest.raises(RuntimeError, match="malformed"):
        nacho_amd.parse2D(write(tmp_path / "t.mtx", "%%MatrixMarket matrix coordinate real "
                                                    "general\n2 2 3\n1 1 1\n2 2 2\n"))
    with pytest.raises(RuntimeError, match="malformed"):
        nacho_amd.parse2D(write(tmp_path / "r.mtx", "%%MatrixMarket matrix coordinate real "
                                                    "general\n2 2 1\n3 1 1\n"))
    with pytest.raises(RuntimeError, match="opened or read"):
        nacho_amd.parse2D(str(tmp_path / "missing.mtx"))


def test_empty_matrix(tmp_path):
    got = nacho_amd.parse2D(write(tmp_path / "e.mtx",
                                  "%%MatrixMarket matrix coordinate real general\n5 6 0\n"))
    assert (got.N, got.M) == (5, 6) and got.row.numel() == 0 and got.data.numel() == 0


def test_tns_values_are_strtof_and_reading_stops_at_first_bad_entry(tmp_path):
    strtof = ctypes.CDLL(None).strtof
    strtof.restype = ctypes.c_float
    strtof.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]
    rng = np.random.default_rng(3)
    lines, want = [], []
    for _ in range(500):
        i, j, k = (int(rng.integers(1, n + 1)) for n in (7, 8, 9))
        v = f"{rng.normal() * 10.0 ** rng.integers(-20, 20):.12e}"
        lines.append(f"{i} {j}\t{k}  {v}")
        want.append((i - 1, j - 1, k - 1, np.float32(strtof(v.encode(), None))))
    text = "\n".join(lines) + "\n# trailing comment\n1 1 1 5.0\n"
    got = nacho_amd.parse3D_i32_f32(write(tmp_path / "x.tns", text), 7, 8, 9)
    assert got.nnz == 500 and (got.N, got.M, got.K) == (7, 8, 9)
    assert got.row.tolist() == [w[0] for w in want]
    assert got.col.tolist() == [w[1] for w in want]
    assert got.dep.tolist() == [w[2] for w in want]
    np.testing.assert_array_equal(got.data.numpy().view(np.int32),
                                  np.array([w[3] for w in want], np.float32).view(np.int32))
    with pytest.raises(RuntimeError, match="malformed"):
        nacho_amd.parse3D_i32_f32(write(tmp_path / "o.tns", "1 1 10 1.0\n"), 7, 8, 9)


def test_parse_matrix_and_frostt_helpers(tmp_path):
    m = sp.random(50, 40, density=0.1, format="coo", random_state=4, dtype=np.float32)
    f = tmp_path / "m.mtx"
    scipy.io.mmwrite(str(f), m)
    csr = io.parse_matrix(f, device="cpu")
    want = scipy.io.mmread(str(f)).tocsr().astype(np.float32)
    want.sort_indices()
    np.testing.assert_array_equal(csr.crow_indices().numpy(), want.indptr)
    np.testing.assert_array_equal(csr.col_indices().numpy(), want.indices)
    np.testing.assert_array_equal(csr.values().numpy(), want.data)

    shape = (5, 6, 7)
    rng = np.random.default_rng(5)
    coords = np.unique(np.stack([rng.integers(0, n, 80) for n in shape], axis=1), axis=0)
    vals = rng.uniform(-1, 1, len(coords)).astype(np.float32)
    tns = tmp_path / "t.tns"
    tns.write_text("".join(f"{i + 1} {j + 1} {k + 1} {v!r}\n" for (i, j, k), v in
                           zip(coords.tolist(), vals.tolist())))
    c, v = io.load_frostt(tns, shape)
    np.testing.assert_array_equal(c, coords)
    sc, sv = io.shift_coordinates(c, v, shape)
    brute = {}
    for (i, j, k), x in zip(c.tolist(), v.tolist()):
        key = (min(i + 1, shape[0] - 1), min(j + 1, shape[1] - 1), min(k + 1, shape[2] - 1))
        brute[key] = brute.get(key, 0.0) + x
    assert [tuple(x) for x in sc.tolist()] == sorted(brute)
    np.testing.assert_allclose(sv, [brute[k] for k in sorted(brute)], rtol=1e-6)


def test_header_claiming_huge_nnz_is_an_error_not_a_crash(tmp_path):
    """A header that claims 1e15 entries must not size the buffers from the header (which
    would throw through the C ABI and end the process): the reader sizes by the file and
    reports the missing entries as malformed input."""
    text = "%%MatrixMarket matrix coordinate real general\n3 3 1000000000000000\n1 1 1.0\n"
    f = write(tmp_path / "huge.mtx", text)
    with pytest.raises(RuntimeError, match="malformed"):
        nacho_amd.parse2D(f)
    # the same through the C ABI, with the error code
    from nacho_amd import _lib

    out = _lib.Coo2dHost()
    assert _lib.load().nacho_parse2d(f.encode(), ctypes.byref(out)) == -4
    assert out.nnz == 0 and not out.row


def test_parse_matrix_builds_csr_and_coo(tmp_path):
    """parse_matrix (the benchmarks' operand builder) sorts entries by (row, column) and
    sums duplicates in file order."""
    text = ("%%MatrixMarket matrix coordinate real general\n3 4 5\n"
            "3 2 1.0\n1 4 2.0\n1 1 3.0\n3 2 0.5\n2 3 -1.0\n")
    f = write(tmp_path / "p.mtx", text)
    csr = io.parse_matrix(f, device="cpu")
    assert csr.crow_indices().tolist() == [0, 2, 3, 4]
    assert csr.col_indices().tolist() == [0, 3, 2, 1]
    assert csr.values().tolist() == [3.0, 2.0, -1.0, 1.5]
    coo = io.parse_matrix(f, return_coo=True, device="cpu")
    assert coo.is_coalesced()
    np.testing.assert_array_equal(coo.to_dense().numpy(), csr.to_dense().numpy())


def test_clip_to_common_shape_keeps_leading_rows_and_widens():
    """benchmarks/csr_add.py:33-42, 59-65: rows = min, cols = max, entries of the dropped
    rows removed."""
    from nacho_amd import io

    a = torch.tensor([[1.0, 0, 2], [0, 3, 0], [4, 0, 0]]).to_sparse_csr()
    b = torch.tensor([[0, 5.0, 0, 0], [6, 0, 0, 7]]).to_sparse_csr()
    rows, cols, ta, tb = io.clip_to_common_shape(a, b)
    assert (rows, cols) == (2, 4)
    np.testing.assert_array_equal(ta[0], [0, 2, 3])
    np.testing.assert_array_equal(ta[1], [0, 2, 1])
    np.testing.assert_array_equal(ta[2], np.float32([1, 2, 3]))
    np.testing.assert_array_equal(tb[0], [0, 1, 3])
    assert ta[0].dtype == np.int32 and ta[1].dtype == np.int32 and ta[2].dtype == np.float32


def test_coalesce_and_shape_of_an_unsorted_tensor():
    from nacho_amd import io

    c = np.array([[2, 1, 1], [0, 0, 0], [2, 1, 1], [1, 5, 2]], np.int32)
    v = np.float32([1, 2, 3, 4])
    assert io.frostt_shape(c) == (3, 6, 3)
    got_c, got_v = io.coalesce_coordinates(c, v, (3, 6, 3))
    np.testing.assert_array_equal(got_c, [[0, 0, 0], [1, 5, 2], [2, 1, 1]])
    np.testing.assert_array_equal(got_v, np.float32([2, 4, 4]))
    # the wide-shape branch (lexicographic sort) gives the same result
    wide = (2**31 - 1,) * 3
    wc, wv = io.coalesce_coordinates(c, v, wide)
    np.testing.assert_array_equal(wc, got_c)
    np.testing.assert_array_equal(wv, got_v)
    assert io.frostt_shape(np.zeros((0, 3), np.int32)) == (1, 1, 1)
