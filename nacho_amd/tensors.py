"""GPU tensor classes with the reference's Python names and fields.

The reference generates one nanobind class per (format, device): its constructor takes the
level buffers in level order, then `values`, then a host int32 `shape`, and exposes them as
read-only attributes (src/backend/generate_bindings.cpp:84-154, 177-254).  These classes keep
those names, argument orders and field names for the GPU target:

    CSR_gpu(dim_j_offsets, dim_j_indices, values, shape)
    COO_gpu(dim_i_indices, dim_j_indices, values, shape)
    COO3_gpu(dim_i_indices, dim_j_indices, dim_k_indices, values, shape)
    DCSR_gpu(dim_i_indices, dim_j_offsets, dim_j_indices, values, shape)
    CSF3_gpu(dim_i_indices, dim_j_offsets, dim_j_indices, dim_k_offsets, dim_k_indices,
             values, shape)

plus CSR64_gpu, the same as CSR_gpu with int64 offsets, for SpGEMM results longer than 2^31
(the reference is int32-only), and Scalar_gpu(values), a full reduction's single value: no
levels and no shape (generate_bindings.cpp:181-183).  Buffers are torch tensors on a HIP device ("cuda" in torch).
"""

from __future__ import annotations

import torch

from . import _device

_I32, _I64, _F32 = torch.int32, torch.int64, torch.float32


def _shape(shape, rank: int, name: str) -> torch.Tensor:
    t = torch.as_tensor(shape, dtype=_I32)
    if t.device.type != "cpu":
        t = t.cpu()
    if t.dim() != 1 or t.numel() != rank:
        raise ValueError(f"{name}: shape must have {rank} entries, got {tuple(t.shape)}")
    if (t < 0).any():
        raise ValueError(f"{name}: negative dimension in shape {t.tolist()}")
    return t.contiguous()


class _GpuTensor:
    """Common machinery: named device buffers (checked dtype/device) plus a host shape."""

    _fields: tuple[tuple[str, torch.dtype], ...] = ()
    _rank = 0

    def __init__(self, *buffers, shape=None):
        cls = type(self).__name__
        if len(buffers) != len(self._fields):
            raise TypeError(f"{cls} takes {len(self._fields)} buffers and a shape")
        device = None
        for (name, dtype), buf in zip(self._fields, buffers):
            _device.require_device_tensor(buf, dtype, f"{cls}.{name}")
            if device is None:
                device = buf.device
            elif buf.device != device:
                raise ValueError(f"{cls}: buffers on different devices ({device}, {buf.device})")
            object.__setattr__(self, "_" + name, buf)
        object.__setattr__(self, "_shape", _shape(shape, self._rank, cls))
        object.__setattr__(self, "_dims", tuple(int(x) for x in self._shape.tolist()))
        object.__setattr__(self, "_device", device)

    @classmethod
    def _trusted(cls, buffers, shape_list, device):
        """Build from buffers the library just produced (already checked): no validation."""
        obj = object.__new__(cls)
        for (name, _), buf in zip(cls._fields, buffers):
            object.__setattr__(obj, "_" + name, buf)
        object.__setattr__(obj, "_shape", None)  # built on first access
        object.__setattr__(obj, "_dims", tuple(int(x) for x in shape_list))
        object.__setattr__(obj, "_device", device)
        return obj

    @property
    def shape(self) -> torch.Tensor:
        if self._shape is None:
            object.__setattr__(self, "_shape", torch.tensor(self._dims, dtype=_I32))
        return self._shape

    @property
    def device(self) -> torch.device:
        return self._device

    def record_stream(self, stream) -> None:
        """Mark every buffer as used by `stream` (a torch.cuda.Stream), like torch's
        Tensor.record_stream: a buffer the library allocated is then reused, after it is
        released, only by work ordered after `stream`'s work queued until the release.
        Buffers torch allocated are passed to torch's own record_stream."""
        for name, _ in self._fields:
            buf = getattr(self, "_" + name)
            if buf.numel() == 0:
                continue
            try:
                _device.record_stream(buf, stream)
            except ValueError:
                buf.record_stream(stream)

    def __setattr__(self, name, value):
        raise AttributeError(f"{type(self).__name__} fields are read-only")

    def __repr__(self):
        parts = ", ".join(f"{n}[{getattr(self, n).numel()}]" for n, _ in self._fields)
        return f"{type(self).__name__}({parts}, shape={list(self._dims)})"


def _field(name):
    return property(lambda self: getattr(self, "_" + name))


def _make(cls_name, fields, rank, doc):
    ns = {"_fields": tuple(fields), "_rank": rank, "__doc__": doc}
    for name, _ in fields:
        ns[name] = _field(name)

    def __init__(self, *args):
        if len(args) != len(fields) + 1:
            raise TypeError(f"{cls_name}({', '.join(n for n, _ in fields)}, shape)")
        _GpuTensor.__init__(self, *args[:-1], shape=args[-1])

    ns["__init__"] = __init__
    return type(cls_name, (_GpuTensor,), ns)


CSR_gpu = _make(
    "CSR_gpu",
    [("dim_j_offsets", _I32), ("dim_j_indices", _I32), ("values", _F32)],
    2,
    "CSR matrix {i: Dense, j: Compressed_unique} on the GPU (reference class CSR_gpu).",
)

CSR64_gpu = _make(
    "CSR64_gpu",
    [("dim_j_offsets", _I64), ("dim_j_indices", _I32), ("values", _F32)],
    2,
    "CSR matrix with int64 offsets, for results with more than 2^31 entries.",
)

COO_gpu = _make(
    "COO_gpu",
    [("dim_i_indices", _I32), ("dim_j_indices", _I32), ("values", _F32)],
    2,
    "COO matrix {i: Compressed_non_unique, j: Singleton_unique} (reference class COO_gpu).",
)

COO3_gpu = _make(
    "COO3_gpu",
    [("dim_i_indices", _I32), ("dim_j_indices", _I32), ("dim_k_indices", _I32),
     ("values", _F32)],
    3,
    "COO order-3 tensor (reference class COO3_gpu).",
)

DCSR_gpu = _make(
    "DCSR_gpu",
    [("dim_i_indices", _I32), ("dim_j_offsets", _I32), ("dim_j_indices", _I32),
     ("values", _F32)],
    2,
    "DCSR matrix {i, j: Compressed_unique}: only rows with entries are stored "
    "(reference class DCSR_gpu).",
)

CSF3_gpu = _make(
    "CSF3_gpu",
    [("dim_i_indices", _I32), ("dim_j_offsets", _I32), ("dim_j_indices", _I32),
     ("dim_k_offsets", _I32), ("dim_k_indices", _I32), ("values", _F32)],
    3,
    "CSF order-3 tensor, every level compressed (reference class CSF3_gpu).",
)


class Scalar_gpu(_GpuTensor):
    """A full reduction's single value on the GPU (reference class Scalar_gpu, the format {}
    named "Scalar", compiler.cpp:75): one `values` buffer of one element and, having no
    dimensions left, no shape (generate_bindings.cpp:181-183)."""

    _fields = (("values", _F32),)
    _rank = 0
    values = _field("values")

    def __init__(self, values):
        _GpuTensor.__init__(self, values, shape=torch.zeros(0, dtype=_I32))
        if values.numel() != 1:
            raise ValueError(f"Scalar_gpu.values holds one element, got {values.numel()}")

    @property
    def shape(self):
        raise AttributeError("Scalar_gpu has no shape: a full reduction has no dimensions")

    def item(self) -> float:
        """The value, copied to the host (waits for the stream that produced it)."""
        return float(self.values.item())
