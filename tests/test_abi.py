"""The drop-in boundary, without a GPU: libmetal_linalg.so loads and exports
every function include/metal_linalg/*.h declares; argument errors give the
reference's statuses and messages; the routing and policy calls answer as
the reference's do (its C-API test, tests/test_c_api.c:158-417, restated)."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "metal_linalg", h) for h in ("c_api.h", "hip_ext.h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(metal_linalg_[a-z0-9_]+)\s*\(", text))
    return sorted(n for n in names if not n.startswith("metal_linalg_INFO"))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 53, names   # 47 reference entry points + 6 HIP extensions
    missing = [n for n in names if not hasattr(lib.lib, n)]
    assert not missing, missing


def test_reference_symbol_set_is_declared():
    # The 41 symbols the reference's Swift package and the 46 its PyTorch
    # binding bind all live in c_api.h: every decomposition, device,
    # routing and policy call.
    names = set(declared_functions())
    for n in ["qr", "qr_with_mode", "eigh", "svd", "cholesky", "lu_factor", "solve", "inv", "solve_triangular",
              "last_error", "buffer_contents", "know_buffer", "forget_buffer", "device_name", "gpu_core_count",
              "set_calibration_notices", "calibration_message", "set_cpu_threads", "cpu_threads",
              "set_cpu_only", "cpu_only"]:
        assert "metal_linalg_" + n in names
    for w in ["qr", "eigh", "svd", "cholesky", "lu", "trsm"]:
        for suffix in ["_policy_get", "_policy_set", "_policy_source", "_backend"]:
            assert f"metal_linalg_{w}{suffix}" in names
    assert "metal_linalg_eigvalsh_backend" in names and "metal_linalg_svdvals_backend" in names


def test_struct_layouts(lib):
    # field counts as the reference's c_api.h
    for what, count in {"qr": 12, "eigh": 30, "svd": 35, "cholesky": 10, "lu": 4, "trsm": 4}.items():
        S = lib.policy_struct(what)
        assert ctypes.sizeof(S) == 4 * count


def test_argument_errors(lib):
    q = np.zeros(4, np.float32)
    r = np.zeros(4, np.float32)
    a = np.eye(2, dtype=np.float32)
    s = np.zeros(2, np.float32)
    u = np.zeros(4, np.float32)
    assert lib.qr(None, 1, 2, 2, q.ctypes.data, r.ctypes.data) == lib.INVALID_ARGUMENT
    assert len(lib.last_error()) > 0
    assert lib.svd(a.ctypes.data, 1, 2, 2, u.ctypes.data, s.ctypes.data, None, None) == lib.INVALID_ARGUMENT
    assert lib.qr_with_mode(a.ctypes.data, 1, 2, 2, 7, q.ctypes.data, r.ctypes.data) == lib.INVALID_ARGUMENT
    assert lib.qr_with_mode(a.ctypes.data, 1, 2, 2, 2, None, r.ctypes.data) == lib.INVALID_ARGUMENT
    assert lib.cholesky(None, 1, 2, 0, q.ctypes.data, None) == lib.INVALID_ARGUMENT
    assert lib.solve(a.ctypes.data, 1, 2, None, 1, q.ctypes.data, None) == lib.INVALID_ARGUMENT
    # an empty batch needs no buffers (and no device)
    assert lib.qr(None, 0, 2, 2, None, None) == lib.OK


def test_metal_buffer_helpers_are_inert(lib):
    assert lib.buffer_contents(None, 0, 16) is None
    assert lib.know_buffer(None, None) == 0
    lib.forget_buffer(None, None)


def test_cpu_only_flag(lib, api):
    assert lib.cpu_only() == 0
    lib.set_cpu_only(1)
    try:
        assert lib.cpu_only() == 1
        for name in (lib.qr_backend(32, 32, 10), lib.eigh_backend(64, 10), lib.svd_backend(8, 8, 2),
                     lib.cholesky_backend(16, 4), lib.lu_backend(100, 9), lib.trsm_backend(64, 64, 1)):
            assert name == b"cpu"
        with pytest.raises(api.MetalLinalgError) as e:
            api.qr(np.eye(3, dtype=np.float32)[None])
        assert e.value.status == lib.RUNTIME_ERROR and b"CPU-only" in lib.last_error()
    finally:
        lib.set_cpu_only(0)
    assert lib.cpu_only() == 0


def test_routing_follows_policies(lib):
    """tests/test_c_api.c:211-417, the routing and policy part, as behaviour."""
    lm = lib.get_policy("lu")
    lib.set_policy("lu", {"gpu_min_n": 100, "gpu_max_batch": 0})
    assert lib.lu_backend(100, 9) == b"blocked"
    assert lib.lu_policy_source() == b"user"
    lib.set_policy("lu", lm)

    measured = lib.get_policy("eigh")
    p = dict(measured, gpu_max_n=0)
    lib.set_policy("eigh", p)
    assert lib.eigh_backend(8, 4096) == b"cpu"
    assert lib.eigh_policy_source() == b"user"
    p.update(gpu_max_n=lib.NO_LIMIT, gpu_min_batch_times_n=0, gpu_min_batch=1)
    lib.set_policy("eigh", p)
    assert lib.eigh_backend(8, 4096) != b"cpu"
    p["values_band_min_n"] = 2048
    lib.set_policy("eigh", p)
    assert lib.get_policy("eigh")["values_band_min_n"] == 2048
    q = dict(measured, gpu_max_n=0, tridiag_min_n=1024, tridiag_max_batch=4, band_min_n=3072,
             tridiag_batch_min_n=96, tridiag_batch_max_n=512, tridiag_batch_min_batch=64)
    lib.set_policy("eigh", q)
    assert lib.eigh_backend(4096, 1) == b"band"
    assert lib.eigh_backend(2048, 1) == b"tridiag"
    assert lib.eigh_backend(256, 64) == b"tridiag_batch"
    assert lib.eigvalsh_backend(256, 64) != b"tridiag_batch"
    p2 = dict(measured, gpu_max_n=0, tridiag_min_n=256, band_min_n=0)
    lib.set_policy("eigh", p2)
    assert lib.eigh_backend(512, 1) == b"tridiag"
    assert lib.eigh_backend(128, 1) == b"cpu"
    lib.set_policy("eigh", measured)
    assert lib.get_policy("eigh")["gpu_max_n"] == measured["gpu_max_n"]

    svd_measured = lib.get_policy("svd")
    sp = dict(svd_measured, gpu_max_k=0, bidiag_min_k=256, band_min_k=0, values_bidiag_min_k=0)
    lib.set_policy("svd", sp)
    assert lib.svd_backend(512, 512, 1) == b"bidiag"
    assert lib.svdvals_backend(512, 512, 1) == b"cpu"
    sp = dict(svd_measured, gpu_max_k=64, gpu_min_batch_times_k=0, gpu_min_batch=1, gpu_max_l=lib.NO_LIMIT,
              gk_min_k=8, gk_max_k=48, gpu_big_batch_min=0)
    lib.set_policy("svd", sp)
    assert lib.svd_backend(40, 24, 16) == b"golub_kahan"
    assert lib.svd_backend(4000, 16, 16) == b"qr_golub_kahan"
    assert lib.svd_backend(49, 49, 16) == b"jacobi"
    sp2 = dict(sp, gpu_max_k=0, gpu_big_batch_max_k=0, bidiag_batch_min_k=64, bidiag_batch_max_k=256,
               bidiag_batch_min_batch=32, bidiag_batch_max_l=512)
    lib.set_policy("svd", sp2)
    assert lib.svd_backend(256, 128, 32) == b"bidiag_batch"
    assert lib.svd_backend(600, 128, 32) != b"bidiag_batch"
    assert lib.svdvals_backend(256, 128, 32) != b"bidiag_batch"
    sp3 = dict(sp, band_min_k=1536, bidiag_min_k=1024, gpu_max_k=0)
    lib.set_policy("svd", sp3)
    assert lib.svd_backend(2048, 2048, 1) == b"band"
    assert lib.svd_backend(1200, 1200, 1) == b"bidiag"
    lib.set_policy("svd", svd_measured)

    cm = lib.get_policy("cholesky")
    lib.set_policy("cholesky", dict(cm, gpu_max_n=0, gpu_large_min_n=0))
    assert lib.cholesky_backend(16, 4096) == b"cpu"
    assert lib.cholesky_policy_source() == b"user"
    lib.set_policy("cholesky", dict(cm, gpu_max_n=lib.NO_LIMIT, gpu_min_batch_times_n=0, gpu_min_batch=1,
                                    gpu_min_n=0, simd_max_n=32, blocked_min_n=1024, blocked_max_batch=2))
    assert lib.cholesky_backend(24, 64) == b"simd"
    assert lib.cholesky_backend(200, 64) == b"threadgroup"
    assert lib.cholesky_backend(2048, 1) == b"blocked"
    lib.set_policy("cholesky", cm)


def test_calibration_message(lib):
    lib.svd_policy_source()
    msg = lib.calibration_message(b"SVD")
    src = lib.svd_policy_source()
    assert msg is not None
    assert (src.startswith(b"tuned:") == (msg == b"")) or src.startswith(b"env:") or src == b"user" \
        or lib.device_name() == b""
    assert lib.calibration_message(None) == b""


def test_cpu_threads(lib):
    lib.set_cpu_threads(3)
    assert lib.cpu_threads() == 3
    lib.set_cpu_threads(0)
    assert lib.cpu_threads() >= 1
