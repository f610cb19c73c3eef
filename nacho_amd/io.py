"""Matrix Market / FROSTT readers and the real-data helpers built on them.

`parse2D` and `parse3D_i32_f32` keep the names, arguments and result fields of the
reference's readers (runtime/io/parse.h:28-263, registered as nacho.parse2D and
nacho.parse3D_i32_f32 at runtime/register_runtime.cpp:20-40): coordinates in file order,
0-based int32, float32 values, as torch CPU tensors.  They run the library's C++ reader
(nacho_parse2d / nacho_parse3d in libnacho_hip.so) and raise RuntimeError where the
reference would terminate the process.

`parse_matrix`, `load_frostt`, `shift_coordinates` and `clip_to_common_shape` restate the
benchmark helpers that turn those files into operands (benchmarks/common/parser.py:87-99,
benchmarks/common/frostt.py:11-44, benchmarks/csr_add.py:33-42), for local files: this
package downloads nothing.  `coalesce_coordinates` and `frostt_shape` prepare a .tns file
whose entries are unsorted or whose dims are not given.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


@dataclass(frozen=True)
class COO2D:
    """Result of parse2D (reference class COO2D): row, col, data and the shape N x M."""

    row: torch.Tensor
    col: torch.Tensor
    data: torch.Tensor
    N: int
    M: int


@dataclass(frozen=True)
class COO3D_parsed:  # noqa: N801 (the reference's class name)
    """Result of parse3D_i32_f32 (reference class COO3D_parsed)."""

    row: torch.Tensor
    col: torch.Tensor
    dep: torch.Tensor
    data: torch.Tensor
    N: int
    M: int
    K: int
    nnz: int


def _host_array(lib, ptr, n, ctype, dtype) -> torch.Tensor:
    """Copy a library-owned host array into a torch tensor and release it."""
    try:
        if n == 0:
            return torch.zeros(0, dtype=dtype)
        arr = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctype)), shape=(n,))
        return torch.from_numpy(arr.copy())
    finally:
        lib.nacho_host_free(ptr)


def parse2D(filename: str) -> COO2D:  # noqa: N802 (the reference's name)
    """Read a `coordinate real` Matrix Market file (general, symmetric or skew-symmetric)."""
    lib = _lib.load()
    out = _lib.Coo2dHost()
    rc = lib.nacho_parse2d(os.fsencode(str(filename)), ctypes.byref(out))
    _lib.check(rc, f"parse2D({filename!s})")
    n = int(out.nnz)
    return COO2D(_host_array(lib, out.row, n, ctypes.c_int32, torch.int32),
                 _host_array(lib, out.col, n, ctypes.c_int32, torch.int32),
                 _host_array(lib, out.data, n, ctypes.c_float, torch.float32),
                 int(out.N), int(out.M))


def parse3D_i32_f32(filename: str, N: int, M: int, K: int) -> COO3D_parsed:  # noqa: N802,N803
    """Read a FROSTT .tns file ("i j k value" lines, 1-based) of shape (N, M, K)."""
    lib = _lib.load()
    out = _lib.Coo3dHost()
    rc = lib.nacho_parse3d(os.fsencode(str(filename)), int(N), int(M), int(K),
                           ctypes.byref(out))
    _lib.check(rc, f"parse3D_i32_f32({filename!s})")
    n = int(out.nnz)
    return COO3D_parsed(_host_array(lib, out.row, n, ctypes.c_int32, torch.int32),
                        _host_array(lib, out.col, n, ctypes.c_int32, torch.int32),
                        _host_array(lib, out.dep, n, ctypes.c_int32, torch.int32),
                        _host_array(lib, out.data, n, ctypes.c_float, torch.float32),
                        int(out.N), int(out.M), int(out.K), n)


def parse_matrix(path, return_coo: bool = False, device="cuda") -> torch.Tensor:
    """A .mtx file as a torch sparse tensor (CSR, or coalesced COO when return_coo): the
    operand builder of the reference's matrix benchmarks (benchmarks/common/parser.py:87-99),
    which takes a matrix name where this takes the file's path.

    Entries are ordered by one int64 key row * columns + column on the host; entries that
    share a key (possible in general files) are summed in file order."""
    m = parse2D(str(path))
    key = m.row.to(torch.int64) * int(m.M) + m.col.to(torch.int64)
    key, order = torch.sort(key, stable=True)
    uniq, slot = torch.unique_consecutive(key, return_inverse=True)
    vals = torch.zeros(uniq.numel(), dtype=torch.float32).index_add_(0, slot, m.data[order])
    rows, cols = uniq // int(m.M), uniq % int(m.M)
    if return_coo:
        out = torch.sparse_coo_tensor(torch.stack((rows, cols)), vals, (m.N, m.M),
                                      is_coalesced=True)
        return out.to(device)
    crow = torch.zeros(int(m.N) + 1, dtype=torch.int64)
    torch.cumsum(torch.bincount(rows, minlength=int(m.N)), 0, out=crow[1:])
    return torch.sparse_csr_tensor(crow, cols, vals, (m.N, m.M)).to(device)


def load_frostt(path, dims):
    """A .tns file as (int32 coordinates of shape (nnz, 3), float32 values): the loader of
    the reference's tensor benchmarks (benchmarks/common/frostt.py:11-24), which takes a
    tensor name where this takes the file's path."""
    t = parse3D_i32_f32(str(path), *dims)
    return np.column_stack((t.row.numpy(), t.col.numpy(), t.dep.numpy())), t.data.numpy()


def _sorted_distinct(coords64, values, shape, dtype):
    """Rows of `coords64` (int64, shape (n, 3)) lexicographically sorted, with the values of
    equal rows summed in their sorted order.

    Coordinates become one int64 key (mode 0 most significant) when the shape allows it,
    else a three-column lexicographic sort gives the same order."""
    ext = np.asarray(shape, dtype=np.int64)
    if int(ext[0]) * int(ext[1]) * int(ext[2]) < (1 << 62):
        key = (coords64[:, 0] * ext[1] + coords64[:, 1]) * ext[2] + coords64[:, 2]
        order = np.argsort(key, kind="stable")
        key = key[order]
        head = np.ones(len(key), dtype=bool)
        head[1:] = key[1:] != key[:-1]
    else:
        order = np.lexsort((coords64[:, 2], coords64[:, 1], coords64[:, 0]))
        m = coords64[order]
        head = np.ones(len(m), dtype=bool)
        head[1:] = (m[1:] != m[:-1]).any(axis=1)
    first = np.flatnonzero(head)
    ordered = np.asarray(values)[order]
    summed = np.add.reduceat(ordered, first) if len(first) else ordered
    return coords64[order][first].astype(dtype), summed


def shift_coordinates(coordinates, values, shape):
    """The second operand of the reference's tensor benchmarks
    (benchmarks/common/frostt.py:27-44): every coordinate moved one step along each mode,
    stopping at the last index, then entries that land on the same coordinate summed (in
    their sorted order), lexicographically sorted."""
    c = np.asarray(coordinates)
    ext = np.asarray(shape, dtype=np.int64)
    moved = np.minimum(c.astype(np.int64) + 1, ext - 1)
    return _sorted_distinct(moved, values, shape, c.dtype)


def coalesce_coordinates(coordinates, values, shape):
    """(i, j, k) rows in the form to_csf3 / to_coo3 take: sorted, distinct, the values of
    repeated coordinates summed.  A FROSTT file need not be sorted or free of repeats."""
    c = np.asarray(coordinates)
    return _sorted_distinct(c.astype(np.int64), values, shape, c.dtype)


def frostt_shape(coordinates):
    """Shape of a tensor given without its dims: one past the largest coordinate per mode."""
    c = np.asarray(coordinates)
    if len(c) == 0:
        return (1, 1, 1)
    return tuple(int(x) + 1 for x in c.max(axis=0))


def clip_to_common_shape(a: torch.Tensor, b: torch.Tensor):
    """Two CSR matrices restricted to their common number of rows and declared as wide as
    the wider one, as the reference's matrix benchmarks pair them
    (benchmarks/csr_add.py:33-42, 59-65).  Returns (rows, cols, a, b) with each operand a
    (pos, crd, val) triple of int32 / int32 / float32 numpy arrays."""
    rows = min(int(a.shape[0]), int(b.shape[0]))
    cols = max(int(a.shape[1]), int(b.shape[1]))

    def clip(m):
        crow = m.crow_indices().cpu()
        nnz = int(crow[rows])
        return (crow[:rows + 1].numpy().astype(np.int32),
                m.col_indices().cpu()[:nnz].numpy().astype(np.int32),
                m.values().cpu()[:nnz].numpy().astype(np.float32))

    return rows, cols, clip(a), clip(b)
