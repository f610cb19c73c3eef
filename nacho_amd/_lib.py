"""ctypes view of the C ABI in include/nacho_hip.h (libnacho_hip.so).

Loading fails loudly when the library has not been built: there is no fallback path.
The structures below mirror the C descriptors field for field.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libnacho_hip.so"

c_int32_p = ctypes.POINTER(ctypes.c_int32)
c_int64_p = ctypes.POINTER(ctypes.c_int64)
c_float_p = ctypes.POINTER(ctypes.c_float)


class CsrDesc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_j_offsets", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int32),
        ("dim_j_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class Csr64Desc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_j_offsets", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int64),
        ("dim_j_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int64),
    ]


class CooDesc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_i_length", ctypes.c_int32),
        ("dim_i_indices", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int32),
        ("dim_j_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class Coo3Desc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_k_size", ctypes.c_int32),
        ("dim_i_length", ctypes.c_int32),
        ("dim_i_indices", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int32),
        ("dim_j_indices", ctypes.c_void_p),
        ("dim_k_length", ctypes.c_int32),
        ("dim_k_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class DcsrDesc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_i_length", ctypes.c_int32),
        ("dim_i_indices", ctypes.c_void_p),
        ("dim_j_offsets", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int32),
        ("dim_j_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class Csf3Desc(ctypes.Structure):
    _fields_ = [
        ("dim_i_size", ctypes.c_int32),
        ("dim_j_size", ctypes.c_int32),
        ("dim_k_size", ctypes.c_int32),
        ("dim_i_length", ctypes.c_int32),
        ("dim_i_indices", ctypes.c_void_p),
        ("dim_j_offsets", ctypes.c_void_p),
        ("dim_j_length", ctypes.c_int32),
        ("dim_j_indices", ctypes.c_void_p),
        ("dim_k_offsets", ctypes.c_void_p),
        ("dim_k_length", ctypes.c_int32),
        ("dim_k_indices", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class ScalarDesc(ctypes.Structure):
    _fields_ = [
        ("values", ctypes.c_void_p),
        ("nnz", ctypes.c_int32),
    ]


class Coo2dHost(ctypes.Structure):
    _fields_ = [
        ("N", ctypes.c_int32),
        ("M", ctypes.c_int32),
        ("nnz", ctypes.c_int64),
        ("row", ctypes.c_void_p),
        ("col", ctypes.c_void_p),
        ("data", ctypes.c_void_p),
    ]


class Coo3dHost(ctypes.Structure):
    _fields_ = [
        ("N", ctypes.c_int32),
        ("M", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("nnz", ctypes.c_int64),
        ("row", ctypes.c_void_p),
        ("col", ctypes.c_void_p),
        ("dep", ctypes.c_void_p),
        ("data", ctypes.c_void_p),
    ]


class Allocator(ctypes.Structure):
    _fields_ = [
        ("ctx", ctypes.c_void_p),
        ("allocate", ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p)),
        ("release", ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)),
    ]


# entry point name -> (operand descriptor, result descriptor)
ENTRY_POINTS = {
    "nacho_gpu_csr_add_f32": (CsrDesc, CsrDesc),
    "nacho_gpu_csr_mul_f32": (CsrDesc, CsrDesc),
    "nacho_gpu_coo_add_f32": (CooDesc, CooDesc),
    "nacho_gpu_coo_mul_f32": (CooDesc, CooDesc),
    "nacho_gpu_coo3d_add_f32": (Coo3Desc, Coo3Desc),
    "nacho_gpu_dcsr_add_f32": (DcsrDesc, DcsrDesc),
    "nacho_gpu_dcsr_mul_f32": (DcsrDesc, DcsrDesc),
    "nacho_gpu_dcsr_mul_without_recursive_partitioning_f32": (DcsrDesc, DcsrDesc),
    "nacho_gpu_csf_add_f32": (Csf3Desc, Csf3Desc),
    "nacho_gpu_inner_prod_f32": (Csf3Desc, ScalarDesc),
    "nacho_gpu_inner_prod_coo_f32": (Coo3Desc, ScalarDesc),
    "nacho_gpu_spgemm_f32": (CsrDesc, CsrDesc),
    "nacho_gpu_spgemm64_f32": (CsrDesc, Csr64Desc),
}

# entry points whose two operands differ in format: name -> (a, b, result)
ENTRY_POINTS_MIXED = {
    "nacho_gpu_coo_csr_add_f32": (CsrDesc, CooDesc, CsrDesc),
}

# three-operand entry points (a, b, c, z, ...)
ENTRY_POINTS_3 = {
    "nacho_gpu_csr_add_3_f32": (CsrDesc, CsrDesc),
    "nacho_gpu_sssmm_f32": (CsrDesc, CsrDesc),
}

# allocation-free entry points (a, b, z, num_blocks, threads_per_block, stream): the caller
# passes the result buffers in z
ENTRY_POINTS_NOALLOC = {
    "nacho_gpu_csr_add_f32_noalloc": (CsrDesc, CsrDesc),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"{LIBRARY_PATH.name} is not built (expected at {LIBRARY_PATH}); "
            "run `python -m nacho_amd.build` — nacho_amd has no non-HIP fallback")
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (operand, result) in ENTRY_POINTS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(operand), ctypes.POINTER(operand), ctypes.POINTER(result),
                       ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                       ctypes.POINTER(Allocator)]
    for name, (da, db, result) in ENTRY_POINTS_MIXED.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(da), ctypes.POINTER(db), ctypes.POINTER(result),
                       ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                       ctypes.POINTER(Allocator)]
    for name, (operand, result) in ENTRY_POINTS_3.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(operand)] * 3 + [
            ctypes.POINTER(result), ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
            ctypes.POINTER(Allocator)]
    for name, (operand, result) in ENTRY_POINTS_NOALLOC.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(operand), ctypes.POINTER(operand), ctypes.POINTER(result),
                       ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.nacho_parse2d.restype = ctypes.c_int
    lib.nacho_parse2d.argtypes = [ctypes.c_char_p, ctypes.POINTER(Coo2dHost)]
    lib.nacho_parse3d.restype = ctypes.c_int
    lib.nacho_parse3d.argtypes = [ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32,
                                  ctypes.c_int32, ctypes.POINTER(Coo3dHost)]
    lib.nacho_host_free.restype = None
    lib.nacho_host_free.argtypes = [ctypes.c_void_p]
    lib.nacho_free.restype = ctypes.c_int
    lib.nacho_free.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.nacho_release_cached_memory.restype = ctypes.c_int
    lib.nacho_release_cached_memory.argtypes = []
    lib.nacho_set_cache_limit.restype = ctypes.c_int
    lib.nacho_set_cache_limit.argtypes = [ctypes.c_size_t]
    lib.nacho_cached_bytes.restype = ctypes.c_size_t
    lib.nacho_cached_bytes.argtypes = []
    lib.nacho_error_string.restype = ctypes.c_char_p
    lib.nacho_error_string.argtypes = [ctypes.c_int]
    lib.nacho_device_copy.restype = ctypes.c_int
    lib.nacho_device_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p]
    lib.nacho_version.restype = ctypes.c_char_p
    lib.nacho_version.argtypes = []
    lib.nacho_set_kernel_timing.restype = None
    lib.nacho_set_kernel_timing.argtypes = [ctypes.c_int]
    lib.nacho_last_kernel_ms.restype = ctypes.c_float
    lib.nacho_last_kernel_ms.argtypes = []
    lib.nacho_last_kernel_name.restype = ctypes.c_char_p
    lib.nacho_last_kernel_name.argtypes = []
    lib.nacho_validate_csr.restype = ctypes.c_int
    lib.nacho_validate_csr.argtypes = [ctypes.POINTER(CsrDesc), ctypes.c_void_p]
    lib.nacho_record_stream.restype = ctypes.c_int
    lib.nacho_record_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    _lib = lib
    return lib


def error_string(code: int) -> str:
    return load().nacho_error_string(code).decode()


def check(code: int, what: str) -> None:
    if code != 0:
        raise RuntimeError(f"{what} failed: {error_string(code)} (code {code})")
