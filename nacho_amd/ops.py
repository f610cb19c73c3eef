"""`gpu_<kernel>_f32` entry points with the reference's Python signatures.

The reference's generated wrapper (src/backend/generate_bindings.cpp:288-327) unwraps each
operand class into the kernel's tensor struct, calls `<k>::<k>_gpu_i32_f32(operands...,
num_blocks, threads_per_block)` and adopts the returned buffers.  These functions do the
same through the C ABI of libnacho_hip.so: borrow operand buffers, call the entry point on
torch's current stream, adopt the result buffers.  There is no CPU fallback: a missing
library raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _device, _lib
from .tensors import COO3_gpu, COO_gpu, CSF3_gpu, CSR64_gpu, CSR_gpu, DCSR_gpu, Scalar_gpu

_I32, _I64, _F32 = torch.int32, torch.int64, torch.float32


def _p(t: torch.Tensor):
    return ctypes.c_void_p(_device.ptr(t))


def _same_device(*tensors):
    device = tensors[0].device
    for t in tensors[1:]:
        if t.device != device:
            raise ValueError(f"operands on different devices: {device} and {t.device}")
    return device


# ---- descriptor conversion -----------------------------------------------------------

def _csr_desc(t: CSR_gpu) -> _lib.CsrDesc:
    rows, cols = t._dims
    if t.dim_j_offsets.numel() != rows + 1:
        raise ValueError(f"CSR_gpu: dim_j_offsets has {t.dim_j_offsets.numel()} entries, "
                         f"expected rows + 1 = {rows + 1}")
    n = t.dim_j_indices.numel()
    if t.values.numel() != n:
        raise ValueError("CSR_gpu: dim_j_indices and values differ in length")
    return _lib.CsrDesc(rows, cols, _p(t.dim_j_offsets), n, _p(t.dim_j_indices), _p(t.values), n)


def _coo_desc(t: COO_gpu) -> _lib.CooDesc:
    rows, cols = t._dims
    n = t.values.numel()
    if t.dim_i_indices.numel() != n or t.dim_j_indices.numel() != n:
        raise ValueError("COO_gpu: coordinate and value arrays differ in length")
    return _lib.CooDesc(rows, cols, n, _p(t.dim_i_indices), n, _p(t.dim_j_indices),
                        _p(t.values), n)


def _coo3_desc(t: COO3_gpu) -> _lib.Coo3Desc:
    si, sj, sk = t._dims
    n = t.values.numel()
    if any(x.numel() != n for x in (t.dim_i_indices, t.dim_j_indices, t.dim_k_indices)):
        raise ValueError("COO3_gpu: coordinate and value arrays differ in length")
    return _lib.Coo3Desc(si, sj, sk, n, _p(t.dim_i_indices), n, _p(t.dim_j_indices), n,
                         _p(t.dim_k_indices), _p(t.values), n)


def _dcsr_desc(t: DCSR_gpu) -> _lib.DcsrDesc:
    rows, cols = t._dims
    ni, nj = t.dim_i_indices.numel(), t.dim_j_indices.numel()
    if t.dim_j_offsets.numel() != ni + 1:
        raise ValueError(f"DCSR_gpu: dim_j_offsets has {t.dim_j_offsets.numel()} entries, "
                         f"expected stored rows + 1 = {ni + 1}")
    if t.values.numel() != nj:
        raise ValueError("DCSR_gpu: dim_j_indices and values differ in length")
    return _lib.DcsrDesc(rows, cols, ni, _p(t.dim_i_indices), _p(t.dim_j_offsets), nj,
                         _p(t.dim_j_indices), _p(t.values), nj)


def _csf3_desc(t: CSF3_gpu) -> _lib.Csf3Desc:
    si, sj, sk = t._dims
    ni, nj, nk = t.dim_i_indices.numel(), t.dim_j_indices.numel(), t.dim_k_indices.numel()
    if t.dim_j_offsets.numel() != ni + 1 or t.dim_k_offsets.numel() != nj + 1:
        raise ValueError("CSF3_gpu: offsets arrays must have parent length + 1 entries")
    if t.values.numel() != nk:
        raise ValueError("CSF3_gpu: dim_k_indices and values differ in length")
    return _lib.Csf3Desc(si, sj, sk, ni, _p(t.dim_i_indices), _p(t.dim_j_offsets), nj,
                         _p(t.dim_j_indices), _p(t.dim_k_offsets), nk, _p(t.dim_k_indices),
                         _p(t.values), nk)


def _cached_desc(t, desc_fn):
    """The operand's C descriptor, rebuilt only when a buffer's address or length changed
    since it was last built for this object (its fields are read-only, but a buffer could
    be resized in place): repeated calls on the same operands skip the size checks and the
    ctypes construction."""
    key = tuple((b.data_ptr(), b.numel()) for b in (getattr(t, "_" + n) for n, _ in t._fields))
    cached = t.__dict__.get("_cdesc")
    if cached is not None and cached[0] is desc_fn and cached[1] == key:
        return cached[2]
    d = desc_fn(t)
    object.__setattr__(t, "_cdesc", (desc_fn, key, d))
    return d


# ---- result adoption -----------------------------------------------------------------

def _adopt_csr(z: _lib.CsrDesc, device, stream) -> CSR_gpu:
    rows, n = z.dim_i_size, z.dim_j_length
    return CSR_gpu._trusted((_device.adopt(z.dim_j_offsets, rows + 1, _I32, device, stream),
                             _device.adopt(z.dim_j_indices, n, _I32, device, stream),
                             _device.adopt(z.values, n, _F32, device, stream)),
                            [z.dim_i_size, z.dim_j_size], device)


def _adopt_csr64(z: _lib.Csr64Desc, device, stream) -> CSR64_gpu:
    rows, n = z.dim_i_size, z.dim_j_length
    return CSR64_gpu._trusted((_device.adopt(z.dim_j_offsets, rows + 1, _I64, device, stream),
                               _device.adopt(z.dim_j_indices, n, _I32, device, stream),
                               _device.adopt(z.values, n, _F32, device, stream)),
                              [z.dim_i_size, z.dim_j_size], device)


def _adopt_coo(z: _lib.CooDesc, device, stream) -> COO_gpu:
    n = z.nnz
    return COO_gpu._trusted((_device.adopt(z.dim_i_indices, n, _I32, device, stream),
                             _device.adopt(z.dim_j_indices, n, _I32, device, stream),
                             _device.adopt(z.values, n, _F32, device, stream)),
                            [z.dim_i_size, z.dim_j_size], device)


def _adopt_coo3(z: _lib.Coo3Desc, device, stream) -> COO3_gpu:
    n = z.nnz
    return COO3_gpu._trusted((_device.adopt(z.dim_i_indices, n, _I32, device, stream),
                              _device.adopt(z.dim_j_indices, n, _I32, device, stream),
                              _device.adopt(z.dim_k_indices, n, _I32, device, stream),
                              _device.adopt(z.values, n, _F32, device, stream)),
                             [z.dim_i_size, z.dim_j_size, z.dim_k_size], device)


def _adopt_dcsr(z: _lib.DcsrDesc, device, stream) -> DCSR_gpu:
    ni, nj = z.dim_i_length, z.dim_j_length
    return DCSR_gpu._trusted((_device.adopt(z.dim_i_indices, ni, _I32, device, stream),
                              _device.adopt(z.dim_j_offsets, ni + 1, _I32, device, stream),
                              _device.adopt(z.dim_j_indices, nj, _I32, device, stream),
                              _device.adopt(z.values, nj, _F32, device, stream)),
                             [z.dim_i_size, z.dim_j_size], device)


def _adopt_csf3(z: _lib.Csf3Desc, device, stream) -> CSF3_gpu:
    ni, nj, nk = z.dim_i_length, z.dim_j_length, z.dim_k_length
    return CSF3_gpu._trusted((_device.adopt(z.dim_i_indices, ni, _I32, device, stream),
                              _device.adopt(z.dim_j_offsets, ni + 1, _I32, device, stream),
                              _device.adopt(z.dim_j_indices, nj, _I32, device, stream),
                              _device.adopt(z.dim_k_offsets, nj + 1, _I32, device, stream),
                              _device.adopt(z.dim_k_indices, nk, _I32, device, stream),
                              _device.adopt(z.values, nk, _F32, device, stream)),
                             [z.dim_i_size, z.dim_j_size, z.dim_k_size], device)


def _adopt_scalar(z: _lib.ScalarDesc, device, stream) -> Scalar_gpu:
    return Scalar_gpu._trusted((_device.adopt(z.values, 1, _F32, device, stream),), [], device)


# ---- input validation ----------------------------------------------------------------

_VALIDATE = False


def set_validation(enable: bool) -> None:
    """Validation mode: when enabled, every `gpu_` entry point first checks its CSR operands
    on the device (nacho_validate_csr) and raises ValueError for a malformed one.  Off by
    default: like the reference's generated code, the kernels trust operand contents."""
    global _VALIDATE
    _VALIDATE = bool(enable)


def validate_csr(t: CSR_gpu) -> None:
    """Check a CSR operand against the input contract (pos[0] == 0, pos non-decreasing,
    pos[rows] == nnz, 0 <= crd < columns, crd strictly increasing per row); raises
    ValueError if it is malformed."""
    if not isinstance(t, CSR_gpu):
        raise TypeError(f"validate_csr: expected CSR_gpu, got {type(t).__name__}")
    desc = _csr_desc(t)
    with _device.on_device(t.device):
        rc = _lib.load().nacho_validate_csr(ctypes.byref(desc),
                                            ctypes.c_void_p(_device.current_stream(t.device)))
    if rc == -4:  # NACHO_ERR_MALFORMED_INPUT
        raise ValueError("CSR operand violates the input contract (offsets, column range or "
                         "per-row order)")
    _lib.check(rc, "nacho_validate_csr")


def _maybe_validate(*operands):
    if _VALIDATE:
        for t in operands:
            if isinstance(t, CSR_gpu):
                validate_csr(t)


# ---- generic call --------------------------------------------------------------------

_ENTRIES: dict = {}


def _entry(name):
    """The library's entry point `name` (looked up once)."""
    fn = _ENTRIES.get(name)
    if fn is None:
        fn = getattr(_lib.load(), name, None)
        if fn is None:
            raise RuntimeError(f"{name} is not exported by {_lib.LIBRARY_PATH.name}")
        _ENTRIES[name] = fn
    return fn


def _call(entry, a, b, cls, desc_fn, result_desc, adopt_fn, num_blocks, threads_per_block,
          cls_b=None, desc_fn_b=None):
    """One two-operand entry point: a (class `cls`) and b (class `cls_b`, default `cls`)."""
    cls_b = cls_b or cls
    desc_fn_b = desc_fn_b or desc_fn
    for name, t, c in (("a", a, cls), ("b", b, cls_b)):
        if not isinstance(t, c):
            raise TypeError(f"{entry}: operand {name} must be {c.__name__}, "
                            f"got {type(t).__name__}")
    _maybe_validate(a, b)
    device = _same_device(a, b)
    fn = _entry(entry)
    da, db = _cached_desc(a, desc_fn), _cached_desc(b, desc_fn_b)
    z = result_desc()
    with _device.on_device(device):
        stream = _device.current_stream(device)
        rc = fn(ctypes.byref(da), ctypes.byref(db), ctypes.byref(z), int(num_blocks),
                int(threads_per_block), ctypes.c_void_p(stream), None)
        _lib.check(rc, entry)
        return adopt_fn(z, device, stream)


def gpu_csr_add_f32(a: CSR_gpu, b: CSR_gpu, num_blocks: int = 256,
                    threads_per_block: int = 256) -> CSR_gpu:
    """Z = a + b (sorted union per row; explicit zeros kept).  compiler.cpp:112."""
    return _call("nacho_gpu_csr_add_f32", a, b, CSR_gpu, _csr_desc, _lib.CsrDesc, _adopt_csr,
                 num_blocks, threads_per_block)


def _call3(entry, a, b, c, num_blocks, threads_per_block) -> CSR_gpu:
    for name, t in (("a", a), ("b", b), ("c", c)):
        if not isinstance(t, CSR_gpu):
            raise TypeError(f"{entry}: operand {name} must be CSR_gpu, got {type(t).__name__}")
    _maybe_validate(a, b, c)
    device = _same_device(a, b, c)
    fn = _entry(entry)
    da, db, dc = (_cached_desc(t, _csr_desc) for t in (a, b, c))
    z = _lib.CsrDesc()
    with _device.on_device(device):
        stream = _device.current_stream(device)
        rc = fn(ctypes.byref(da), ctypes.byref(db), ctypes.byref(dc), ctypes.byref(z),
                int(num_blocks), int(threads_per_block), ctypes.c_void_p(stream), None)
        _lib.check(rc, entry)
        return _adopt_csr(z, device, stream)


def gpu_csr_add_3_f32(a: CSR_gpu, b: CSR_gpu, c: CSR_gpu, num_blocks: int = 256,
                      threads_per_block: int = 256) -> CSR_gpu:
    """Z = a + b + c (sorted union of three; values (a + b) + c over the present operands).
    compiler.cpp:114."""
    return _call3("nacho_gpu_csr_add_3_f32", a, b, c, num_blocks, threads_per_block)


def gpu_sssmm_f32(a: CSR_gpu, b: CSR_gpu, c: CSR_gpu, num_blocks: int = 256,
                  threads_per_block: int = 256) -> CSR_gpu:
    """Masked SpGEMM Z_ik = sum_j a_ij b_jk c_ik over the entries of c that a product reaches.
    compiler.cpp:150-153."""
    return _call3("nacho_gpu_sssmm_f32", a, b, c, num_blocks, threads_per_block)


def gpu_csr_mul_f32(a: CSR_gpu, b: CSR_gpu, num_blocks: int = 256,
                    threads_per_block: int = 256) -> CSR_gpu:
    """Z = a * b elementwise (sorted intersection per row).  compiler.cpp:116."""
    return _call("nacho_gpu_csr_mul_f32", a, b, CSR_gpu, _csr_desc, _lib.CsrDesc, _adopt_csr,
                 num_blocks, threads_per_block)


def gpu_coo_add_f32(a: COO_gpu, b: COO_gpu, num_blocks: int = 256,
                    threads_per_block: int = 256) -> COO_gpu:
    """Z = a + b over COO (union of (i, j)).  compiler.cpp:118."""
    return _call("nacho_gpu_coo_add_f32", a, b, COO_gpu, _coo_desc, _lib.CooDesc, _adopt_coo,
                 num_blocks, threads_per_block)


def gpu_coo_mul_f32(a: COO_gpu, b: COO_gpu, num_blocks: int = 256,
                    threads_per_block: int = 256) -> COO_gpu:
    """Z = a * b over COO (intersection of (i, j)).  compiler.cpp:120."""
    return _call("nacho_gpu_coo_mul_f32", a, b, COO_gpu, _coo_desc, _lib.CooDesc, _adopt_coo,
                 num_blocks, threads_per_block)


def gpu_coo3d_add_f32(a: COO3_gpu, b: COO3_gpu, num_blocks: int = 256,
                      threads_per_block: int = 256) -> COO3_gpu:
    """Z = a + b over COO3 (union of (i, j, k)).  compiler.cpp:138."""
    return _call("nacho_gpu_coo3d_add_f32", a, b, COO3_gpu, _coo3_desc, _lib.Coo3Desc,
                 _adopt_coo3, num_blocks, threads_per_block)


def gpu_dcsr_add_f32(a: DCSR_gpu, b: DCSR_gpu, num_blocks: int = 256,
                     threads_per_block: int = 256) -> DCSR_gpu:
    """Z = a + b over DCSR (union of row ids, then of each row's columns).
    compiler.cpp:124."""
    return _call("nacho_gpu_dcsr_add_f32", a, b, DCSR_gpu, _dcsr_desc, _lib.DcsrDesc,
                 _adopt_dcsr, num_blocks, threads_per_block)


def gpu_dcsr_mul_f32(a: DCSR_gpu, b: DCSR_gpu, num_blocks: int = 256,
                     threads_per_block: int = 256) -> DCSR_gpu:
    """Z = a * b over DCSR: rows stored in both operands, each with the intersection of its
    columns (kept when that is empty).  compiler.cpp:126."""
    return _call("nacho_gpu_dcsr_mul_f32", a, b, DCSR_gpu, _dcsr_desc, _lib.DcsrDesc,
                 _adopt_dcsr, num_blocks, threads_per_block)


def gpu_dcsr_mul_without_recursive_partitioning_f32(
        a: DCSR_gpu, b: DCSR_gpu, num_blocks: int = 256,
        threads_per_block: int = 256) -> DCSR_gpu:
    """The same product as gpu_dcsr_mul_f32 (the reference variant differs only in how it
    partitions work).  compiler.cpp:128-133."""
    return _call("nacho_gpu_dcsr_mul_without_recursive_partitioning_f32", a, b, DCSR_gpu,
                 _dcsr_desc, _lib.DcsrDesc, _adopt_dcsr, num_blocks, threads_per_block)


def gpu_csf_add_f32(a: CSF3_gpu, b: CSF3_gpu, num_blocks: int = 256,
                    threads_per_block: int = 256) -> CSF3_gpu:
    """Z = a + b over CSF3 (union at every level).  compiler.cpp:135."""
    return _call("nacho_gpu_csf_add_f32", a, b, CSF3_gpu, _csf3_desc, _lib.Csf3Desc,
                 _adopt_csf3, num_blocks, threads_per_block)


def gpu_coo_csr_add_f32(a: CSR_gpu, b: COO_gpu, num_blocks: int = 256,
                        threads_per_block: int = 256) -> CSR_gpu:
    """Z = a + b for a CSR a and a COO b (sorted, no duplicates), giving CSR.
    compiler.cpp:122."""
    return _call("nacho_gpu_coo_csr_add_f32", a, b, CSR_gpu, _csr_desc, _lib.CsrDesc,
                 _adopt_csr, num_blocks, threads_per_block, cls_b=COO_gpu,
                 desc_fn_b=_coo_desc)


def gpu_inner_prod_f32(a: CSF3_gpu, b: CSF3_gpu, num_blocks: int = 256,
                       threads_per_block: int = 256) -> Scalar_gpu:
    """z = sum_ijk a_ijk * b_ijk over CSF3 operands (float32 products summed in float64,
    rounded once).  compiler.cpp:141."""
    return _call("nacho_gpu_inner_prod_f32", a, b, CSF3_gpu, _csf3_desc, _lib.ScalarDesc,
                 _adopt_scalar, num_blocks, threads_per_block)


def gpu_inner_prod_coo_f32(a: COO3_gpu, b: COO3_gpu, num_blocks: int = 256,
                           threads_per_block: int = 256) -> Scalar_gpu:
    """The same inner product over COO3 operands.  compiler.cpp:143."""
    return _call("nacho_gpu_inner_prod_coo_f32", a, b, COO3_gpu, _coo3_desc, _lib.ScalarDesc,
                 _adopt_scalar, num_blocks, threads_per_block)


def gpu_spgemm_f32(a: CSR_gpu, b: CSR_gpu, num_blocks: int = 256,
                   threads_per_block: int = 256) -> CSR_gpu:
    """Z_ik = sum_j a_ij b_jk (ESC SpGEMM), int32 result.  compiler.cpp:145-148."""
    return _call("nacho_gpu_spgemm_f32", a, b, CSR_gpu, _csr_desc, _lib.CsrDesc, _adopt_csr,
                 num_blocks, threads_per_block)


def gpu_spgemm64_f32(a: CSR_gpu, b: CSR_gpu, num_blocks: int = 256,
                     threads_per_block: int = 256) -> CSR64_gpu:
    """The same product with int64 result offsets, for results beyond 2^31 entries."""
    return _call("nacho_gpu_spgemm64_f32", a, b, CSR_gpu, _csr_desc, _lib.Csr64Desc,
                 _adopt_csr64, num_blocks, threads_per_block)


def release_cached_memory() -> None:
    """Return the default allocator's cached, unused device buffers to the driver."""
    _lib.check(_lib.load().nacho_release_cached_memory(), "nacho_release_cached_memory")


def set_cache_limit(nbytes: int | None) -> None:
    """Cap the bytes the library's caching allocator keeps for reuse (None: no cap, the
    default).  Past the cap, released buffers go back to the driver (after a device
    synchronise), so that torch's allocator in the same process can use that memory."""
    limit = ctypes.c_size_t(-1).value if nbytes is None else int(nbytes)
    if limit < 0:
        raise ValueError("cache limit must be >= 0")
    _lib.check(_lib.load().nacho_set_cache_limit(limit), "nacho_set_cache_limit")


def cached_bytes() -> int:
    """Bytes the library's caching allocator holds for reuse now."""
    return int(_lib.load().nacho_cached_bytes())


def set_kernel_timing(enable: bool) -> None:
    _lib.load().nacho_set_kernel_timing(1 if enable else 0)


def last_kernel_ms() -> float:
    return float(_lib.load().nacho_last_kernel_ms())
