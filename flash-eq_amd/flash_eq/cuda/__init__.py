"""Import path of the reference's op binding (``flash_eq.cuda``), kept for API compatibility.

On this build the op runs HIP kernels for gfx950; the module name is the
reference's public import path, not a CUDA dependency.
"""
from .block_diagonal import block_diagonal_cuda, CUDANotAvailableError

__all__ = ["block_diagonal_cuda", "CUDANotAvailableError"]
