"""Matrix Market / FROSTT readers and the real-data helpers built on them.

`parse2D` and `parse3D_i32_f32` keep the names, arguments and result fields of the
reference's readers (runtime/io/parse.h:28-263, registered as nacho.parse2D and
nacho.parse3D_i32_f32 at runtime/register_runtime.cpp:20-40): coordinates in file order,
0-based int32, float32 values, as torch CPU tensors.  They run the library's C++ reader
(nacho_parse2d / nacho_parse3d in libnacho_hip.so) and raise RuntimeError where the
reference would terminate the process.

`parse_matrix`, `load_frostt` and `shift_coordinates` restate the benchmark helpers that
turn those files into operands (benchmarks/common/parser.py:87-99,
benchmarks/common/frostt.py:11-44), for local files: this package downloads nothing.
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
    """A .mtx file as a torch sparse tensor, CSR unless return_coo
    (benchmarks/common/parser.py:87-99; here the argument is the file's path)."""
    coo = parse2D(str(path))
    row = coo.row.to(dtype=torch.long, device=device)
    col = coo.col.to(dtype=torch.long, device=device)
    values = coo.data.to(dtype=torch.float32, device=device)
    tensor = torch.sparse_coo_tensor(torch.stack([row, col], dim=0), values, (coo.N, coo.M))
    return tensor if return_coo else tensor.to_sparse_csr()


def load_frostt(path, dims):
    """A .tns file as (coordinates shaped (nnz, 3), values) (benchmarks/common/frostt.py:11-24;
    here the argument is the file's path)."""
    parsed = parse3D_i32_f32(str(path), *dims)
    coordinates = np.stack([parsed.row.numpy(), parsed.col.numpy(), parsed.dep.numpy()], axis=1)
    return coordinates, parsed.data.numpy()


def shift_coordinates(coordinates, values, shape):
    """A second operand from the first: every coordinate advanced by one and clamped to the
    extent, duplicates summed, lexicographically sorted (benchmarks/common/frostt.py:27-44)."""
    coordinates = np.asarray(coordinates)
    shifted = np.minimum(coordinates + 1, np.array(shape, dtype=coordinates.dtype) - 1)
    order = np.lexsort((shifted[:, 2], shifted[:, 1], shifted[:, 0]))
    shifted, ordered = shifted[order], np.asarray(values)[order]
    starts = np.ones(len(shifted), dtype=bool)
    starts[1:] = np.any(shifted[1:] != shifted[:-1], axis=1)
    run_starts = np.flatnonzero(starts)
    return shifted[run_starts], np.add.reduceat(ordered, run_starts) if len(run_starts) else ordered
