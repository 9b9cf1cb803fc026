"""Array-level calls over the C ABI.

Each function takes a numpy array (host memory: the library stages it through
HBM) or a torch tensor on the GPU (device memory: read and written in place),
float32 with shape [..., M, N], and returns outputs of the same kind.  The
semantics are the C ABI's (include/metal_linalg/c_api.h): NaN output and the
info bits for a non-finite matrix, LAPACK-style info for Cholesky and LU.
A non-OK status raises MetalLinalgError carrying the status and message.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class MetalLinalgError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"metal_linalg status {status}: {message}")
        self.status = status


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


class _Arrays:
    """Allocation and pointers for one call, on the input's side."""

    def __init__(self, a):
        self.torch = _is_torch(a)
        if self.torch:
            import torch

            if a.dtype != torch.float32:
                a = a.to(torch.float32)
            self.a = a.contiguous()
            self.device = self.a.device
            # pinned host input -> pinned host outputs: the library then moves
            # them over PCIe directly, with no copy through its own staging
            self.pinned = self.device.type == "cpu" and self.a.is_pinned()
        else:
            self.a = np.ascontiguousarray(a, dtype=np.float32)
        self.keep = [self.a]

    def like(self, x):
        if self.torch:
            import torch

            if not _is_torch(x):
                x = torch.as_tensor(x)
            x = x.to(device=self.device, dtype=torch.float32).contiguous()
            if self.pinned and not x.is_pinned():
                x = x.pin_memory()
        else:
            x = np.ascontiguousarray(x, dtype=np.float32)
        self.keep.append(x)
        return x

    def empty(self, shape, dtype="f32"):
        if self.torch:
            import torch

            dt = torch.float32 if dtype == "f32" else torch.int32
            if self.pinned:
                x = torch.empty(shape, dtype=dt, pin_memory=True)
            else:
                x = torch.empty(shape, dtype=dt, device=self.device)
        else:
            x = np.empty(shape, dtype=np.float32 if dtype == "f32" else np.uint32)
        self.keep.append(x)
        return x

    def call(self, fn, *args):
        """fn(*args) under the library lock.  For tensors on the GPU the
        library's stream first waits for what torch has enqueued on its
        current stream so far, this call's input conversions included: an
        event, not a host synchronisation, and none at all when that stream
        has nothing pending (the wait costs ~20 us per call).  The library
        returns when its results are complete."""
        with _lib.lock:
            if self.torch and self.device.type == "cuda":
                import torch

                stream = torch.cuda.current_stream(self.device)
                if not stream.query():
                    _check(_lib.hip_stream_wait(stream.cuda_stream))
            _check(fn(*args))

    @staticmethod
    def ptr(x):
        if x is None:
            return None
        if _is_torch(x):
            return x.data_ptr() if x.numel() else None
        return x.ctypes.data if x.size else None

    def u32(self, x):
        """uint32 view of an int32 torch tensor (torch has no uint32 ops)."""
        if x is None:
            return None
        return x


def _check(rc: int):
    if rc != _lib.OK:
        raise MetalLinalgError(rc, _lib.last_error().decode())


def _dims(a):
    if a.ndim < 2:
        raise ValueError(f"expected [..., M, N], got shape {tuple(a.shape)}")
    lead = tuple(a.shape[:-2])
    b = 1
    for d in lead:
        b *= int(d)
    return lead, b, int(a.shape[-2]), int(a.shape[-1])


def qr(a, mode: str = "reduced"):
    """(Q, R); Q is None for mode 'r'."""
    arr = _Arrays(a)
    lead, b, m, n = _dims(arr.a)
    k = min(m, n)
    code = _lib.QR_MODES[mode]
    qc = 0 if code == 1 else (m if code == 2 else k)
    rr = m if code == 2 else k
    q = arr.empty(lead + (m, qc)) if qc else None
    r = arr.empty(lead + (rr, n))
    arr.call(_lib.qr_with_mode, arr.ptr(arr.a), b, m, n, code, arr.ptr(q), arr.ptr(r))
    return q, r


def eigh(a, lower: bool = True, vectors: bool = True):
    """(w ascending, V with eigenvectors as columns or None, info)."""
    arr = _Arrays(a)
    lead, b, n, n2 = _dims(arr.a)
    if n != n2:
        raise ValueError("eigh needs square matrices")
    w = arr.empty(lead + (n,))
    v = arr.empty(lead + (n, n)) if vectors else None
    info = arr.empty(lead, "u32")
    arr.call(_lib.eigh, arr.ptr(arr.a), b, n, int(bool(lower)), arr.ptr(w), arr.ptr(v), arr.ptr(info))
    return w, v, info


def svd(a, vectors: bool = True):
    """(U, s descending, Vt, info); U and Vt None without vectors."""
    arr = _Arrays(a)
    lead, b, m, n = _dims(arr.a)
    k = min(m, n)
    s = arr.empty(lead + (k,))
    u = arr.empty(lead + (m, k)) if vectors else None
    vt = arr.empty(lead + (k, n)) if vectors else None
    info = arr.empty(lead, "u32")
    arr.call(_lib.svd, arr.ptr(arr.a), b, m, n, arr.ptr(u), arr.ptr(s), arr.ptr(vt), arr.ptr(info))
    return u, s, vt, info


def cholesky(a, upper: bool = False):
    """(L or U, info)."""
    arr = _Arrays(a)
    lead, b, n, _ = _dims(arr.a)
    l = arr.empty(lead + (n, n))
    info = arr.empty(lead, "u32")
    arr.call(_lib.cholesky, arr.ptr(arr.a), b, n, int(bool(upper)), arr.ptr(l), arr.ptr(info))
    return l, info


def lu_factor(a):
    """(LU packed, pivots 0-based, info)."""
    arr = _Arrays(a)
    lead, b, n, _ = _dims(arr.a)
    lu = arr.empty(lead + (n, n))
    piv = arr.empty(lead + (n,), "u32")
    info = arr.empty(lead, "u32")
    arr.call(_lib.lu_factor, arr.ptr(arr.a), b, n, arr.ptr(lu), arr.ptr(piv), arr.ptr(info))
    return lu, piv, info


def solve(a, rhs):
    """(X, info) for A X = B, B [..., n, nrhs]."""
    arr = _Arrays(a)
    lead, b, n, _ = _dims(arr.a)
    rhs = arr.like(rhs)
    nrhs = int(rhs.shape[-1])
    x = arr.empty(tuple(rhs.shape))
    info = arr.empty(lead, "u32")
    arr.call(_lib.solve, arr.ptr(arr.a), b, n, arr.ptr(rhs), nrhs, arr.ptr(x), arr.ptr(info))
    return x, info


def inv(a):
    """(A^-1, info)."""
    arr = _Arrays(a)
    lead, b, n, _ = _dims(arr.a)
    x = arr.empty(lead + (n, n))
    info = arr.empty(lead, "u32")
    arr.call(_lib.inv, arr.ptr(arr.a), b, n, arr.ptr(x), arr.ptr(info))
    return x, info


def solve_triangular(a, rhs, upper: bool = False, unit: bool = False):
    arr = _Arrays(a)
    lead, b, n, _ = _dims(arr.a)
    rhs = arr.like(rhs)
    nrhs = int(rhs.shape[-1])
    x = arr.empty(tuple(rhs.shape))
    arr.call(_lib.solve_triangular, arr.ptr(arr.a), b, n, arr.ptr(rhs), nrhs, int(bool(upper)), int(bool(unit)),
             arr.ptr(x))
    return x


# The reference's north-star entry-point names (its MLX API:
# include/metal_linalg/qr.h:22-24, eigh.h:29-35, svd.h:33-37, cholesky.h:24-33,
# lu.h:24-45, triangular.h:20-21), here over numpy arrays and torch tensors.
def qr_accelerated(a, mode: str = "reduced"):
    return qr(a, mode)


def eigh_accelerated(a, lower: bool = True):
    w, v, _ = eigh(a, lower, True)
    return w, v


def eigvalsh_accelerated(a, lower: bool = True):
    return eigh(a, lower, False)[0]


def svd_accelerated(a):
    u, s, vt, _ = svd(a, True)
    return u, s, vt


def svdvals_accelerated(a):
    return svd(a, False)[1]


def cholesky_ex_accelerated(a, upper: bool = False):
    return cholesky(a, upper)


def lu_factor_accelerated(a):
    lu, piv, _ = lu_factor(a)
    return lu, piv


def solve_accelerated(a, rhs):
    return solve(a, rhs)[0]


def inv_accelerated(a):
    return inv(a)[0]


def solve_triangular_accelerated(a, rhs, upper: bool = False, unit: bool = False):
    return solve_triangular(a, rhs, upper, unit)
