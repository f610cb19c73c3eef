"""Device plumbing between torch and the C ABI: streams, and adopting result buffers.

Result buffers come back from libnacho_hip.so as raw device pointers owned by the caller
(allocated by the library's caching allocator over hipMalloc).  `adopt` wraps one in a torch
tensor without copying; when the last tensor referencing it is collected the buffer is
released with `nacho_free` on the stream it was produced on.  Work on another stream that
reads a result must be announced with `record_stream` (torch's own `Tensor.record_stream`
only tracks torch's allocator): the library then orders the buffer's reuse after that
stream's work at release time.  This is the counterpart of the
reference's `adopt_gpu` capsule (runtime/nacho_nb.h:50-58).  A zero-length result is a
NULL pointer and becomes an empty tensor (runtime/nacho_nb.h:37-39).
"""

from __future__ import annotations

import ctypes

import torch
import torch.utils.dlpack

from . import _lib

_TYPESTR = {torch.int32: "<i4", torch.int64: "<i8", torch.float32: "<f4"}
_ITEMSIZE = {torch.int32: 4, torch.int64: 8, torch.float32: 4}


class _OwnedBuffer:
    """Owner of one device allocation, exposed through __cuda_array_interface__."""

    __slots__ = ("ptr", "stream", "count", "dtype", "__weakref__")

    def __init__(self, ptr: int, count: int, dtype: torch.dtype, stream: int):
        self.ptr = ptr
        self.count = count
        self.dtype = dtype
        self.stream = stream

    @property
    def __cuda_array_interface__(self):
        return {
            "shape": (self.count,),
            "typestr": _TYPESTR[self.dtype],
            "data": (self.ptr, False),
            "version": 2,
        }

    def __del__(self):
        if self.ptr:
            try:
                _lib.load().nacho_free(ctypes.c_void_p(self.ptr), ctypes.c_void_p(self.stream))
            except Exception:  # interpreter shutdown: the process is ending anyway
                pass
            self.ptr = 0


# ---- DLPack route (used when torch does not take __cuda_array_interface__) -----------

class _DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int), ("device_id", ctypes.c_int32)]


class _DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class _DLTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device", _DLDevice), ("ndim", ctypes.c_int32),
                ("dtype", _DLDataType), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("strides", ctypes.POINTER(ctypes.c_int64)), ("byte_offset", ctypes.c_uint64)]


class _DLManagedTensor(ctypes.Structure):
    pass


_DL_DELETER = ctypes.CFUNCTYPE(None, ctypes.POINTER(_DLManagedTensor))
_DLManagedTensor._fields_ = [("dl_tensor", _DLTensor), ("manager_ctx", ctypes.c_void_p),
                             ("deleter", _DL_DELETER)]

_KDL_ROCM = 10
_DL_CODE = {torch.int32: (0, 32), torch.int64: (0, 64), torch.float32: (2, 32)}
_DL_LIVE: dict[int, tuple] = {}  # address of managed struct -> (struct, shape, owner)
_CAPSULE_NAME = b"dltensor"


def _dl_release(managed_ptr):
    _DL_LIVE.pop(ctypes.cast(managed_ptr, ctypes.c_void_p).value, None)


_DL_RELEASE = _DL_DELETER(_dl_release)

_capsule_new = ctypes.pythonapi.PyCapsule_New
_capsule_new.restype = ctypes.py_object
_capsule_new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


def _adopt_dlpack(owner: _OwnedBuffer, device: torch.device) -> torch.Tensor:
    shape = (ctypes.c_int64 * 1)(owner.count)
    code, bits = _DL_CODE[owner.dtype]
    managed = _DLManagedTensor()
    managed.dl_tensor.data = owner.ptr
    managed.dl_tensor.device = _DLDevice(_KDL_ROCM, device.index or 0)
    managed.dl_tensor.ndim = 1
    managed.dl_tensor.dtype = _DLDataType(code, bits, 1)
    managed.dl_tensor.shape = shape
    managed.dl_tensor.strides = None
    managed.dl_tensor.byte_offset = 0
    managed.manager_ctx = None
    managed.deleter = _DL_RELEASE
    address = ctypes.addressof(managed)
    _DL_LIVE[address] = (managed, shape, owner)
    capsule = _capsule_new(address, _CAPSULE_NAME, None)
    return torch.utils.dlpack.from_dlpack(capsule)


_ROUTE = None  # "cai" (__cuda_array_interface__) or "dlpack", fixed after the first success


def adopt(ptr: int | None, count: int, dtype: torch.dtype, device: torch.device,
          stream: int) -> torch.Tensor:
    """Tensor of `count` elements over a library-allocated device buffer (takes ownership)."""
    global _ROUTE
    if not ptr:
        return torch.empty(0, dtype=dtype, device=device)
    owner = _OwnedBuffer(ptr, count, dtype, stream)
    tensor = None
    # (the caller has made `device` current: gpu_<k> entry points run under it)
    if _ROUTE in (None, "cai"):
        try:
            tensor = torch.as_tensor(owner, device=device)
            _ROUTE = "cai"
        except (TypeError, RuntimeError, ValueError):
            if _ROUTE == "cai":
                raise
            tensor = None
    if tensor is None:
        tensor = _adopt_dlpack(owner, device)
        _ROUTE = "dlpack"
    if tensor.data_ptr() != ptr or tensor.numel() != count or tensor.dtype != dtype:
        raise RuntimeError("torch did not adopt the device buffer in place")
    return tensor


def record_stream(t: torch.Tensor, stream) -> None:
    """Mark the library-allocated buffer under `t` as used by `stream` (a torch.cuda.Stream
    or a raw hipStream_t), so that its reuse after release waits for work queued on that
    stream until then."""
    if t.numel() == 0:
        return
    raw = stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)
    rc = _lib.load().nacho_record_stream(ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(raw))
    if rc != 0:
        raise ValueError("record_stream: the tensor does not start a buffer that libnacho_hip "
                         f"allocated ({_lib.error_string(rc)})")


def adoption_route() -> str | None:
    """How result buffers are handed to torch in this process (None before the first)."""
    return _ROUTE


def current_stream(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on `device`, as an integer."""
    return int(torch.cuda.current_stream(device).cuda_stream)


class on_device:
    """Make `device` the current HIP device for the block, switching (and restoring) only
    when it is not current already: torch.cuda.device() switches unconditionally, which
    costs tens of microseconds per call."""

    __slots__ = ("index", "prev")

    def __init__(self, device: torch.device):
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        current = torch.cuda.current_device()
        if current != self.index:
            self.prev = current
            torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def require_device_tensor(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a GPU tensor, got device {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if t.dim() != 1 or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous 1-D tensor")
    return t


def ptr(t: torch.Tensor) -> int | None:
    return t.data_ptr() if t.numel() > 0 else None
