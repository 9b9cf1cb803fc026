"""The library's C ABI (include/metal_linalg/c_api.h, hip_ext.h) through ctypes.

Mirrors the reference's PyTorch binding loader
(reference: python-torch/metal_linalg_torch/_lib.py:1-140): one shared
library, every call serialised by one lock, the policy structs field for
field.  The library computes on the GPU only; loading it needs no GPU (the
device is opened at the first decomposition), so symbol checks run anywhere.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.environ.get("METAL_LINALG_LIBRARY") or os.path.join(HERE, "libmetal_linalg.so")

if not os.path.exists(PATH):
    raise ImportError(f"metal_linalg_amd: {PATH} is not built; run `python -m metal_linalg_amd.build` "
                      f"(or __graft_entry__.build()) first")

# torch ships its own libamdhip64.so.7 under the same soname as ROCm's.  One
# process must hold one HIP runtime, or device pointers from torch are
# unknown to the library's: when torch is installed it is loaded first, so
# that the library binds to the runtime torch already uses.
try:
    import torch  # noqa: F401
except ImportError:
    pass

lib = ctypes.CDLL(PATH)
lock = threading.RLock()

_u32, _p, _cstr, _int = ctypes.c_uint32, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int

OK, INVALID_ARGUMENT, RUNTIME_ERROR, OUT_OF_MEMORY = 0, 1, 2, 3
NO_LIMIT = 0xFFFFFFFF
QR_MODES = {"reduced": 0, "r": 1, "complete": 2}


def _fn(name, restype, *argtypes):
    f = getattr(lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


last_error = _fn("metal_linalg_last_error", _cstr)
qr = _fn("metal_linalg_qr", _int, _p, _u32, _u32, _u32, _p, _p)
qr_with_mode = _fn("metal_linalg_qr_with_mode", _int, _p, _u32, _u32, _u32, _int, _p, _p)
eigh = _fn("metal_linalg_eigh", _int, _p, _u32, _u32, _int, _p, _p, _p)
svd = _fn("metal_linalg_svd", _int, _p, _u32, _u32, _u32, _p, _p, _p, _p)
cholesky = _fn("metal_linalg_cholesky", _int, _p, _u32, _u32, _int, _p, _p)
lu_factor = _fn("metal_linalg_lu_factor", _int, _p, _u32, _u32, _p, _p, _p)
solve = _fn("metal_linalg_solve", _int, _p, _u32, _u32, _p, _u32, _p, _p)
inv = _fn("metal_linalg_inv", _int, _p, _u32, _u32, _p, _p)
solve_triangular = _fn("metal_linalg_solve_triangular", _int, _p, _u32, _u32, _p, _u32, _int, _int, _p)

buffer_contents = _fn("metal_linalg_buffer_contents", _p, _p, ctypes.c_uint64, ctypes.c_uint64)
know_buffer = _fn("metal_linalg_know_buffer", _int, _p, _p)
forget_buffer = _fn("metal_linalg_forget_buffer", None, _p, _p)

device_name = _fn("metal_linalg_device_name", _cstr)
gpu_core_count = _fn("metal_linalg_gpu_core_count", _u32)
set_calibration_notices = _fn("metal_linalg_set_calibration_notices", None, _int)
calibration_message = _fn("metal_linalg_calibration_message", _cstr, _cstr)
cpu_threads = _fn("metal_linalg_cpu_threads", _u32)
set_cpu_threads = _fn("metal_linalg_set_cpu_threads", None, _u32)
cpu_only = _fn("metal_linalg_cpu_only", _int)
set_cpu_only = _fn("metal_linalg_set_cpu_only", None, _int)

qr_backend = _fn("metal_linalg_qr_backend", _cstr, _u32, _u32, _u32)
eigh_backend = _fn("metal_linalg_eigh_backend", _cstr, _u32, _u32)
eigvalsh_backend = _fn("metal_linalg_eigvalsh_backend", _cstr, _u32, _u32)
svd_backend = _fn("metal_linalg_svd_backend", _cstr, _u32, _u32, _u32)
svdvals_backend = _fn("metal_linalg_svdvals_backend", _cstr, _u32, _u32, _u32)
cholesky_backend = _fn("metal_linalg_cholesky_backend", _cstr, _u32, _u32)
lu_backend = _fn("metal_linalg_lu_backend", _cstr, _u32, _u32)
trsm_backend = _fn("metal_linalg_trsm_backend", _cstr, _u32, _u32, _u32)

qr_policy_source = _fn("metal_linalg_qr_policy_source", _cstr)
eigh_policy_source = _fn("metal_linalg_eigh_policy_source", _cstr)
svd_policy_source = _fn("metal_linalg_svd_policy_source", _cstr)
cholesky_policy_source = _fn("metal_linalg_cholesky_policy_source", _cstr)
lu_policy_source = _fn("metal_linalg_lu_policy_source", _cstr)
trsm_policy_source = _fn("metal_linalg_trsm_policy_source", _cstr)

# HIP extensions (hip_ext.h)
hip_set_timing = _fn("metal_linalg_hip_set_timing", None, _int)
hip_reset_timing = _fn("metal_linalg_hip_reset_timing", None)
hip_kernel_time = _fn("metal_linalg_hip_kernel_time", _int, _cstr, ctypes.POINTER(ctypes.c_uint64),
                      ctypes.POINTER(ctypes.c_double))
hip_kernel_names = _fn("metal_linalg_hip_kernel_names", _cstr)
hip_arch = _fn("metal_linalg_hip_arch", _cstr)
_ll = ctypes.c_longlong
hip_sgemm = _fn("metal_linalg_hip_sgemm", _int, _int, _int, _int, _int, _int, ctypes.c_float, _p, _int, _ll, _p, _int,
                _ll, ctypes.c_float, _p, _int, _ll, _int)
hip_sytrd = _fn("metal_linalg_hip_sytrd", _int, _p, _u32, _int, _p, _p)


def _struct(name, fields):
    return type(name, (ctypes.Structure,), {"_fields_": [(f, _u32) for f in fields]})


# Field for field as in c_api.h (the reference's order).
QR_FIELDS = ("m_crossover_small_batch", "m_crossover_large_batch", "batch_threshold",
             "gpu_max_k", "gpu_min_batch_times_k", "gpu_min_batch", "gpu_cores", "concurrent_matrices",
             "gpu_large_min_k", "gpu_large_max_batch", "gpu_min_k", "share_min_batch")
EIGH_FIELDS = ("simd_max_n", "block_min_n", "block_min_n_batched", "block_min_batch",
               "gpu_max_n", "gpu_min_batch_times_n", "gpu_min_batch", "gpu_cores",
               "values_gpu_max_n", "values_gpu_min_batch_times_n", "values_gpu_min_batch",
               "tridiag_min_n", "values_tridiag_min_n", "ql_min_n", "ql_max_n",
               "tridiag_max_batch", "values_tridiag_max_batch", "share_min_batch",
               "gpu_big_batch_max_n", "gpu_big_batch_min", "values_band_min_n", "values_band_width",
               "band_min_n", "tridiag_batch_min_n", "tridiag_batch_max_n", "tridiag_batch_min_batch",
               "values_tridiag_batch_min_n", "values_tridiag_batch_max_n", "values_tridiag_batch_min_batch",
               "share_min_n")
SVD_FIELDS = ("qr_min_rows", "qr_min_k", "block_min_k", "block_min_k_batched", "block_min_batch",
              "gpu_max_k", "gpu_min_batch_times_k", "gpu_min_batch", "gpu_cores",
              "bidiag_min_k", "values_bidiag_min_k", "bidiag_max_batch", "values_bidiag_max_batch",
              "gk_min_k", "gk_max_k", "gpu_max_l",
              "values_gpu_max_k", "values_gpu_min_batch_times_k", "values_gpu_min_batch", "values_gpu_max_l",
              "share_min_batch", "gpu_big_batch_max_k", "gpu_big_batch_min", "values_band_min_k",
              "values_band_width", "band_min_k", "bidiag_batch_min_k", "bidiag_batch_max_k",
              "bidiag_batch_min_batch", "bidiag_batch_max_l", "values_bidiag_batch_min_k",
              "values_bidiag_batch_max_k", "values_bidiag_batch_min_batch", "values_bidiag_batch_max_l",
              "share_min_k")
CHOLESKY_FIELDS = ("simd_max_n", "blocked_min_n", "blocked_max_batch", "gpu_max_n", "gpu_min_batch_times_n",
                   "gpu_min_batch", "gpu_min_n", "gpu_large_min_n", "gpu_large_max_batch", "gpu_cores")
LU_FIELDS = ("gpu_min_n", "gpu_max_batch", "gpu_solve_min_rhs", "gpu_cores")
TRSM_FIELDS = ("gpu_min_n", "gpu_min_rhs", "gpu_max_batch", "gpu_cores")
INFORMATIONAL = {"gpu_cores", "concurrent_matrices"}

POLICIES = {}
for _what, _fields in (("qr", QR_FIELDS), ("eigh", EIGH_FIELDS), ("svd", SVD_FIELDS),
                       ("cholesky", CHOLESKY_FIELDS), ("lu", LU_FIELDS), ("trsm", TRSM_FIELDS)):
    _S = _struct(f"{_what}_policy", _fields)
    POLICIES[_what] = (_S, _fields, _fn(f"metal_linalg_{_what}_policy_get", _S),
                       _fn(f"metal_linalg_{_what}_policy_set", None, ctypes.POINTER(_S)))


def get_policy(what):
    _, fields, get, _ = POLICIES[what]
    with lock:
        p = get()
    return {f: getattr(p, f) for f in fields}


def set_policy(what, values):
    S, fields, get, set_ = POLICIES[what]
    unknown = set(values) - set(fields)
    if unknown:
        raise TypeError(f"unknown {what} policy field(s): {', '.join(sorted(unknown))}")
    with lock:
        p = get()
        for f, v in values.items():
            if f not in INFORMATIONAL:
                setattr(p, f, int(v))
        set_(ctypes.byref(p))


def kernel_time(name: str):
    """(launches, total_ms) of a timed kernel since the last reset."""
    n = ctypes.c_uint64()
    ms = ctypes.c_double()
    hip_kernel_time(name.encode(), ctypes.byref(n), ctypes.byref(ms))
    return int(n.value), float(ms.value)


def kernel_names():
    s = hip_kernel_names().decode()
    return [x for x in s.split("\n") if x]
