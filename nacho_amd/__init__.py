"""nacho_amd — MI355X (gfx950) backend for nacho's GPU target.

Python surface of the reference (`import nacho`; python/nacho/__init__.py) for the GPU
target: the tensor classes, the `gpu_<kernel>_f32` entry points, the converters and the
Matrix Market / FROSTT readers.  Every `gpu_` entry point runs hand-written HIP kernels from
libnacho_hip.so through its C ABI (include/nacho_hip.h); nothing here computes on the CPU
except the file readers (host C++ in the same library).
"""

from .convert import to_coo, to_coo3, to_csf3, to_csr, to_dcsr  # noqa: F401
from .ops import (  # noqa: F401
    cached_bytes,
    gpu_coo3d_add_f32,
    gpu_coo_add_f32,
    gpu_coo_csr_add_f32,
    gpu_coo_mul_f32,
    gpu_csf_add_f32,
    gpu_csr_add_3_f32,
    gpu_csr_add_f32,
    gpu_csr_mul_f32,
    gpu_dcsr_add_f32,
    gpu_dcsr_mul_f32,
    gpu_dcsr_mul_without_recursive_partitioning_f32,
    gpu_inner_prod_coo_f32,
    gpu_inner_prod_f32,
    gpu_spgemm64_f32,
    gpu_sssmm_f32,
    gpu_spgemm_f32,
    last_kernel_ms,
    release_cached_memory,
    set_cache_limit,
    set_kernel_timing,
    set_validation,
    validate_csr,
)
from ._device import record_stream  # noqa: F401
from .io import COO2D, COO3D_parsed, parse2D, parse3D_i32_f32  # noqa: F401
from .tensors import (  # noqa: F401
    COO3_gpu, COO_gpu, CSF3_gpu, CSR64_gpu, CSR_gpu, DCSR_gpu, Scalar_gpu)

__version__ = "0.1.0"
