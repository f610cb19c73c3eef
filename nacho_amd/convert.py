"""Building GPU tensors from torch tensors / coordinate arrays.

Same names, arguments and buffer order as the reference's converters
(python/nacho/convert.py:23-118): index arrays become int32, values float32, and the shape
is a host int32 tensor.  This backend replaces the GPU target only, so `device` must name a
HIP device ("cuda" or "cuda:N" in torch); asking for "cpu" raises.
"""

from __future__ import annotations

import numpy as np
import torch

from .tensors import COO3_gpu, COO_gpu, CSF3_gpu, CSR_gpu, DCSR_gpu

__all__ = ["to_csr", "to_dcsr", "to_coo", "to_coo3", "to_csf3"]


def _gpu(device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"nacho_amd builds GPU tensors only; got device {device!s}")
    return device


def _shape(*sizes):
    return torch.tensor(list(sizes), dtype=torch.int32)


def to_csr(csr: torch.Tensor, device="cuda") -> CSR_gpu:
    """torch sparse CSR -> CSR_gpu (python/nacho/convert.py:23-31)."""
    device = _gpu(device)
    return CSR_gpu(
        csr.crow_indices().to(dtype=torch.int32, device=device).contiguous(),
        csr.col_indices().to(dtype=torch.int32, device=device).contiguous(),
        csr.values().to(dtype=torch.float32, device=device).contiguous(),
        _shape(csr.shape[0], csr.shape[1]),
    )


def to_dcsr(csr: torch.Tensor, device="cuda") -> DCSR_gpu:
    """torch sparse CSR -> DCSR_gpu: the row dimension is compressed too, so empty rows are
    dropped and the remaining row ids stored (python/nacho/convert.py:34-53)."""
    device = _gpu(device)
    indptr = csr.crow_indices().to(dtype=torch.int64, device="cpu")
    lengths = indptr[1:] - indptr[:-1]
    present = (lengths > 0).nonzero(as_tuple=False).squeeze(-1)
    offsets = torch.zeros(present.numel() + 1, dtype=torch.int64)
    offsets[1:] = lengths[present].cumsum(0)
    return DCSR_gpu(
        present.to(dtype=torch.int32, device=device).contiguous(),
        offsets.to(dtype=torch.int32, device=device).contiguous(),
        csr.col_indices().to(dtype=torch.int32, device=device).contiguous(),
        csr.values().to(dtype=torch.float32, device=device).contiguous(),
        _shape(csr.shape[0], csr.shape[1]),
    )


def to_coo(coo: torch.Tensor, device="cuda") -> COO_gpu:
    """torch sparse COO -> COO_gpu; coalesced so coordinates are sorted and distinct
    (python/nacho/convert.py:57-67)."""
    device = _gpu(device)
    coo = coo.coalesce()
    indices = coo.indices()
    return COO_gpu(
        indices[0].to(dtype=torch.int32, device=device).contiguous(),
        indices[1].to(dtype=torch.int32, device=device).contiguous(),
        coo.values().to(dtype=torch.float32, device=device).contiguous(),
        _shape(coo.shape[0], coo.shape[1]),
    )


def _tensor(array, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(array)).to(dtype=dtype, device=device)


def to_coo3(coordinates, values, shape, device="cuda") -> COO3_gpu:
    """Sorted, distinct (i, j, k) rows of `coordinates` -> COO3_gpu
    (python/nacho/convert.py:70-87)."""
    device = _gpu(device)
    coordinates = np.asarray(coordinates)
    return COO3_gpu(
        _tensor(coordinates[:, 0], torch.int32, device),
        _tensor(coordinates[:, 1], torch.int32, device),
        _tensor(coordinates[:, 2], torch.int32, device),
        _tensor(values, torch.float32, device),
        torch.tensor(list(shape), dtype=torch.int32),
    )


def csf3_levels(coordinates):
    """Level arrays of the CSF3 tree of sorted, distinct (i, j, k) coordinates:
    (crd_i, pos_j, crd_j, pos_k, crd_k), as in python/nacho/convert.py:90-118."""
    coordinates = np.asarray(coordinates)
    n = coordinates.shape[0]
    if n == 0:
        empty = np.zeros(0, dtype=np.int64)
        return empty, np.zeros(1, np.int64), empty, np.zeros(1, np.int64), empty
    i, j, k = (coordinates[:, c].astype(np.int64) for c in range(3))
    new_ij = np.ones(n, dtype=bool)
    new_ij[1:] = (i[1:] != i[:-1]) | (j[1:] != j[:-1])
    ij_starts = np.flatnonzero(new_ij)
    ij_i, ij_j = i[ij_starts], j[ij_starts]
    new_i = np.ones(len(ij_starts), dtype=bool)
    new_i[1:] = ij_i[1:] != ij_i[:-1]
    i_starts = np.flatnonzero(new_i)
    pos_j = np.append(i_starts, len(ij_starts))
    pos_k = np.append(ij_starts, n)
    return ij_i[i_starts], pos_j, ij_j, pos_k, k


def to_csf3(coordinates, values, shape, device="cuda") -> CSF3_gpu:
    """Sorted, distinct (i, j, k) rows of `coordinates` -> CSF3_gpu: every level compressed,
    each storing the coordinates present under its parent plus the parent's offsets
    (python/nacho/convert.py:90-118)."""
    device = _gpu(device)
    crd_i, pos_j, crd_j, pos_k, crd_k = csf3_levels(coordinates)
    return CSF3_gpu(
        _tensor(crd_i, torch.int32, device),
        _tensor(pos_j, torch.int32, device),
        _tensor(crd_j, torch.int32, device),
        _tensor(pos_k, torch.int32, device),
        _tensor(crd_k, torch.int32, device),
        _tensor(values, torch.float32, device),
        torch.tensor(list(shape), dtype=torch.int32),
    )
