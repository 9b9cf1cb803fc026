"""Execution follows the routed backend.  For Cholesky, LU (factor, solve,
inverse) and the triangular solve, n <= 128 has two GPU routes: the batched
kernels, or the one-matrix-at-a-time blocked path when the policy row says
"blocked" (rows measured by metal_linalg_amd/tuning/sweep.py).  The kernels
that run are read from the library's per-kernel timers, and the blocked path
is checked against the oracle at n <= 128, where the default rows rarely
send it."""

import contextlib

import numpy as np
import pytest

from _util import bound, gaussian, lu_residual, near_tie, rel_recon, to_np, u32

pytestmark = pytest.mark.gpu
NO_LIMIT = 0xFFFFFFFF


@contextlib.contextmanager
def policies(lib, **over):
    saved = {w: lib.get_policy(w) for w in over}
    try:
        for w, fields in over.items():
            lib.set_policy(w, fields)
        yield
    finally:
        for w, fields in saved.items():
            lib.set_policy(w, fields)


def kernels_run(lib, fn):
    lib.hip_reset_timing()
    lib.hip_set_timing(1)
    try:
        fn()
    finally:
        lib.hip_set_timing(0)
    return set(lib.kernel_names())


BLOCKED = dict(cholesky={"blocked_min_n": 1, "blocked_max_batch": 0}, lu={"gpu_min_n": 1, "gpu_max_batch": 0},
               trsm={"gpu_min_n": 1, "gpu_min_rhs": 0, "gpu_max_batch": 0})
BATCHED = dict(cholesky={"blocked_min_n": NO_LIMIT}, lu={"gpu_min_n": 0}, trsm={"gpu_min_n": 0})


@pytest.mark.parametrize("n", [33, 64, 100])
def test_routes_pick_the_kernels(cuda, api, lib, n):
    a = gaussian((4, n, n), seed=n) + np.float32(2 * n) * np.eye(n, dtype=np.float32)
    spd = (a @ np.swapaxes(a, -1, -2)).astype(np.float32)
    b = gaussian((4, n, 3), seed=n + 1)
    with policies(lib, **BLOCKED):
        assert lib.cholesky_backend(n, 4) == b"blocked" and lib.lu_backend(n, 4) == b"blocked"
        assert lib.trsm_backend(n, 3, 4) == b"blocked"
        assert "chol_diag" in kernels_run(lib, lambda: api.cholesky(spd))
        assert "lu_panel" in kernels_run(lib, lambda: api.lu_factor(a))
        assert "trsm_blocked" in kernels_run(lib, lambda: api.solve_triangular(a, b))
    with policies(lib, **BATCHED):
        assert lib.cholesky_backend(n, 4) != b"blocked" and lib.lu_backend(n, 4) == b"cpu"
        assert "chol_small" in kernels_run(lib, lambda: api.cholesky(spd))
        assert "lu_small_factor" in kernels_run(lib, lambda: api.lu_factor(a))
        assert "trsm_small" in kernels_run(lib, lambda: api.solve_triangular(a, b))


@pytest.mark.parametrize("n", [8, 33, 64, 100, 128])
def test_blocked_path_at_batched_sizes(cuda, api, lib, oracle, n):
    """The blocked path, forced, against the oracle where the batched
    kernels usually run."""
    g = gaussian((3, n, n), seed=200 + n)
    spd = (g @ np.swapaxes(g, -1, -2) / n + np.eye(n)).astype(np.float32)
    b = gaussian((3, n, 5), seed=300 + n)
    dom = g + np.float32(n) * np.eye(n, dtype=np.float32)
    with policies(lib, **BLOCKED):
        l, info = api.cholesky(spd)
        lo, io = oracle.cholesky(spd)
        assert np.array_equal(u32(info), io) and np.all(io == 0)
        assert rel_recon(spd, l.astype(np.float64) @ np.swapaxes(l, -1, -2)).max() <= bound(n)
        lu, piv, info = api.lu_factor(g)
        lo, po, io = oracle.lu_factor(g)
        assert np.array_equal(u32(info), io)
        assert lu_residual(g, lu, piv).max() <= bound(n)
        for i in range(3):
            if not np.array_equal(u32(piv)[i], po[i]):
                assert near_tie(g[i], u32(piv)[i], po[i], rel=1e-5)
        x, _ = api.solve(dom, b)
        xo, _ = oracle.solve(dom, b)
        assert (np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))).max() <= 1e-4
        v, _ = api.inv(dom)
        vo, _ = oracle.inv(dom)
        assert (np.abs(v - vo).max(axis=(-2, -1)) / np.abs(vo).max(axis=(-2, -1))).max() <= 1e-4
        t = api.solve_triangular(dom, b, True, False)
        to = oracle.solve_triangular(dom, b, True, False)
        assert (np.abs(t - to).max(axis=(-2, -1)) / np.abs(to).max(axis=(-2, -1))).max() <= 1e-4


def test_default_rows_follow_the_sweep(cuda, lib):
    """The tuned rows in use are the ones the sweep wrote."""
    import re, os

    inc = open(os.path.join(os.path.dirname(lib.__file__), "csrc", "tuned_gfx950.inc")).read()
    val = lambda name: int(re.search(name + r" = (0x[0-9A-Fa-f]+|\d+)", inc).group(1), 0)
    c, l, t = lib.get_policy("cholesky"), lib.get_policy("lu"), lib.get_policy("trsm")
    assert c["blocked_min_n"] == val("kCholeskyBlockedMinN") and c["blocked_max_batch"] == val("kCholeskyBlockedMaxBatch")
    assert l["gpu_min_n"] == val("kLuBlockedMinN") and l["gpu_max_batch"] == val("kLuBlockedMaxBatch")
    assert t["gpu_min_n"] == val("kTrsmBlockedMinN") and t["gpu_max_batch"] == val("kTrsmBlockedMaxBatch")
