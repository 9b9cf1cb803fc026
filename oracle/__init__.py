"""ORACLE -- test infrastructure, not product code.

ctypes front end of ``lapack_batch.cpp``, the CPU restatement of the reference
library's LAPACK-batched CPU path (see that file's header for the reference
lines each function follows).  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg import this package, as the checker
and as the timed host baseline; ``metal_linalg_amd`` never does.

All functions take and return numpy arrays (float32, row-major, C-contiguous)
with the reference C API's shapes and semantics.
"""

from __future__ import annotations

import ctypes
import glob
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(BUILD_DIR, "liboracle.so")
SOURCES = [os.path.join(HERE, "lapack_batch.cpp"), os.path.join(HERE, "lu_netlib.cpp")]


def build(force: bool = True) -> str:
    """Compile lapack_batch.cpp and lu_netlib.cpp with g++ into
    oracle/_build/liboracle.so (no FMA contraction: LAPACK's Fortran order)."""
    if not force and os.path.exists(LIB_PATH):
        return LIB_PATH
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-shared", "-fPIC", "-pthread", *SOURCES, "-o", tmp,
           "-ldl"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lapack_path() -> str:
    """LAPACK to load: $ORACLE_LAPACK, else scipy's bundled OpenBLAS."""
    env = os.environ.get("ORACLE_LAPACK")
    if env:
        return env
    import scipy

    libs = os.path.join(os.path.dirname(os.path.dirname(scipy.__file__)), "scipy.libs")
    found = sorted(glob.glob(os.path.join(libs, "libscipy_openblas*.so")))
    if not found:
        raise RuntimeError(f"oracle: no OpenBLAS under {libs}; set ORACLE_LAPACK")
    return found[0]


_lib = None
_u32 = ctypes.c_uint32
_p = ctypes.c_void_p


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    L.oracle_last_error.restype = ctypes.c_char_p
    L.oracle_lapack_config.restype = ctypes.c_char_p
    L.oracle_init.argtypes = [ctypes.c_char_p]
    L.oracle_set_threads.argtypes = [_u32]
    L.oracle_threads.restype = _u32
    L.oracle_qr.argtypes = [_p, _u32, _u32, _u32, ctypes.c_int, _p, _p]
    L.oracle_eigh.argtypes = [_p, _u32, _u32, ctypes.c_int, _p, _p, _p]
    L.oracle_svd.argtypes = [_p, _u32, _u32, _u32, _p, _p, _p, _p]
    L.oracle_cholesky.argtypes = [_p, _u32, _u32, ctypes.c_int, _p, _p]
    L.oracle_lu_factor.argtypes = [_p, _u32, _u32, _p, _p, _p]
    L.oracle_solve.argtypes = [_p, _u32, _u32, _p, _u32, _p, _p]
    L.oracle_inv.argtypes = [_p, _u32, _u32, _p, _p]
    L.oracle_solve_triangular.argtypes = [_p, _u32, _u32, _p, _u32, ctypes.c_int, ctypes.c_int, _p]
    L.oracle_lu_netlib_factor.argtypes = [_p, _u32, _u32, _p, _p, _p]
    L.oracle_lu_netlib_solve.argtypes = [_p, _u32, _u32, _p, _u32, _p, _p]
    L.oracle_lu_netlib_inv.argtypes = [_p, _u32, _u32, _p, _p]
    if L.oracle_init(lapack_path().encode()) != 0:
        raise RuntimeError(L.oracle_last_error().decode())
    _lib = L
    return L


def config() -> str:
    return lib().oracle_lapack_config().decode()


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def threads() -> int:
    return int(lib().oracle_threads())


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data


def _check(rc):
    if rc != 0:
        raise RuntimeError(f"oracle status {rc}: {lib().oracle_last_error().decode()}")


def _shape3(a):
    if a.ndim < 2:
        raise ValueError("need [..., rows, cols]")
    lead = a.shape[:-2]
    b = int(np.prod(lead)) if lead else 1
    return lead, b, a.shape[-2], a.shape[-1]


def qr(a, mode: str = "reduced"):
    """(Q, R) as metal_linalg_qr_with_mode; Q is None for mode 'r'."""
    a = _c(a)
    lead, b, m, n = _shape3(a)
    k = min(m, n)
    code = {"reduced": 0, "r": 1, "complete": 2}[mode]
    qc = 0 if code == 1 else (m if code == 2 else k)
    rr = m if code == 2 else k
    q = np.empty(lead + (m, qc), np.float32) if qc else None
    r = np.empty(lead + (rr, n), np.float32)
    _check(lib().oracle_qr(_ptr(a), b, m, n, code, _ptr(q), _ptr(r)))
    return q, r


def eigh(a, lower: bool = True, vectors: bool = True):
    """(w, V, info) as metal_linalg_eigh; V is None without vectors."""
    a = _c(a)
    lead, b, n, n2 = _shape3(a)
    assert n == n2
    w = np.empty(lead + (n,), np.float32)
    v = np.empty(lead + (n, n), np.float32) if vectors else None
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_eigh(_ptr(a), b, n, int(bool(lower)), _ptr(w), _ptr(v), _ptr(info)))
    return w, v, info


def svd(a, vectors: bool = True):
    """(U, s, Vt, info) as metal_linalg_svd; U, Vt None without vectors."""
    a = _c(a)
    lead, b, m, n = _shape3(a)
    k = min(m, n)
    s = np.empty(lead + (k,), np.float32)
    u = np.empty(lead + (m, k), np.float32) if vectors else None
    vt = np.empty(lead + (k, n), np.float32) if vectors else None
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_svd(_ptr(a), b, m, n, _ptr(u), _ptr(s), _ptr(vt), _ptr(info)))
    return u, s, vt, info


def cholesky(a, upper: bool = False):
    a = _c(a)
    lead, b, n, _ = _shape3(a)
    l = np.empty_like(a)
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_cholesky(_ptr(a), b, n, int(bool(upper)), _ptr(l), _ptr(info)))
    return l, info


def lu_factor(a):
    a = _c(a)
    lead, b, n, _ = _shape3(a)
    lu = np.empty_like(a)
    piv = np.empty(lead + (n,), np.uint32)
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_lu_factor(_ptr(a), b, n, _ptr(lu), _ptr(piv), _ptr(info)))
    return lu, piv, info


def solve(a, rhs):
    a, rhs = _c(a), _c(rhs)
    lead, b, n, _ = _shape3(a)
    nrhs = rhs.shape[-1]
    x = np.empty_like(rhs)
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_solve(_ptr(a), b, n, _ptr(rhs), nrhs, _ptr(x), _ptr(info)))
    return x, info


def inv(a):
    a = _c(a)
    lead, b, n, _ = _shape3(a)
    x = np.empty_like(a)
    info = np.empty(lead, np.uint32)
    _check(lib().oracle_inv(_ptr(a), b, n, _ptr(x), _ptr(info)))
    return x, info


def solve_triangular(a, rhs, upper: bool = False, unit: bool = False):
    a, rhs = _c(a), _c(rhs)
    lead, b, n, _ = _shape3(a)
    nrhs = rhs.shape[-1]
    x = np.empty_like(rhs)
    _check(lib().oracle_solve_triangular(_ptr(a), b, n, _ptr(rhs), nrhs, int(bool(upper)), int(bool(unit)), _ptr(x)))
    return x


# ---- netlib LAPACK restatement (lu_netlib.cpp): the pin for non-finite LU inputs ----

def lu_netlib_factor(a):
    """(LU, pivots, info) by netlib's sgetf2 rule (ISAMAX: strict '>', NaN never taken)."""
    a = _c(a)
    lead, b, n, _ = _shape3(a)
    lu = np.empty_like(a)
    piv = np.empty(lead + (n,), np.uint32)
    info = np.empty(lead, np.uint32)
    lib().oracle_lu_netlib_factor(_ptr(a), b, n, _ptr(lu), _ptr(piv), _ptr(info))
    return lu, piv, info


def lu_netlib_solve(a, rhs):
    a, rhs = _c(a), _c(rhs)
    lead, b, n, _ = _shape3(a)
    x = np.empty_like(rhs)
    info = np.empty(lead, np.uint32)
    lib().oracle_lu_netlib_solve(_ptr(a), b, n, _ptr(rhs), rhs.shape[-1], _ptr(x), _ptr(info))
    return x, info


def lu_netlib_inv(a):
    a = _c(a)
    lead, b, n, _ = _shape3(a)
    x = np.empty_like(a)
    info = np.empty(lead, np.uint32)
    lib().oracle_lu_netlib_inv(_ptr(a), b, n, _ptr(x), _ptr(info))
    return x, info
