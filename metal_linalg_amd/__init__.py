"""metal_linalg for the AMD Instinct MI355X (gfx950).

Batched fp32 QR, symmetric eigendecomposition, thin SVD, Cholesky, LU with
solve and inverse, and triangular solve, computed by hand-written HIP kernels
behind the reference library's C ABI (libmetal_linalg.so,
include/metal_linalg/c_api.h).  ``metal_linalg_amd.api`` calls it on numpy
arrays (host memory) or torch tensors on the GPU (in place);
``metal_linalg_amd._lib`` is the raw ctypes binding.

Importing the package does not load the library (so that the build step can
run first); the first use of ``api`` or ``_lib`` does, and raises ImportError
if it has not been built.  There is no fallback: every call runs on the GPU.
"""

import importlib

__all__ = ["api", "build"]


def __getattr__(name):
    if name in ("api", "_lib", "build"):
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
