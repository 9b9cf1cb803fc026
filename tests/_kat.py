"""The reference C-API test's known answers (tests/golden/c_api_known_answers.json),
as checks that run against any backend with the oracle's call signatures:
the oracle on the CPU, and the HIP library through its C ABI on the GPU."""

from __future__ import annotations

import json
import math
import os

import numpy as np

from _util import to_np, u32

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c_api_known_answers.json")


def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def near(x, y, tol):
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    return np.all(np.abs(x - y) <= tol * (1 + np.abs(y)))


def arr(x):
    return np.array([[float(v) for v in row] for row in x], np.float32) if not isinstance(x[0][0], list) else \
        np.array([[[float(v) for v in row] for row in m] for m in x], np.float32)


def check_qr(be, g, tol):
    a = arr(g["a"])
    q, r = (to_np(x) for x in be.qr(a, "reduced"))
    assert q.shape == (2, 3, 2) and r.shape == (2, 2, 2)
    for b in range(2):
        assert r[b, 1, 0] == 0.0
        assert near(q[b] @ r[b], a[b], tol)
    _, r_alone = be.qr(a, "r")
    assert near(to_np(r_alone), r, tol)
    qc, rc = (to_np(x) for x in be.qr(a, "complete"))
    assert qc.shape == (2, 3, 3) and rc.shape == (2, 3, 2)
    for b in range(2):
        assert np.all(rc[b, 2] == 0.0)
        assert np.abs(qc[b].T @ qc[b] - np.eye(3)).max() < 1e-5
        assert near(qc[b] @ rc[b], a[b], tol)
        assert near(qc[b][:, :2], q[b], tol)


def check_eigh(be, g, tol):
    a = arr([g["a"]])
    w, v, info = be.eigh(a, True, True)
    w, v, info = to_np(w)[0], to_np(v)[0], u32(info)[0]
    assert near(w, g["w"], tol)
    assert near(abs(v[0, 0]), g["first_vector_abs"], tol) and near(v[0, 0], -v[1, 0], tol)
    assert (info >> 16) & 1 and not (info >> 17) & 1
    w2, v2, _ = be.eigh(a, False, False)
    assert v2 is None and near(to_np(w2)[0], g["w"], tol)


def check_svd(be, g, tol):
    a = arr([g["a"]])
    u, s, vt, info = be.svd(a, True)
    u, s, vt = to_np(u)[0], to_np(s)[0], to_np(vt)[0]
    assert near(s, g["s"], tol)
    assert near((u * s) @ vt, a[0], tol)
    assert (u32(info)[0] >> 16) & 1


def check_cholesky(be, g, tol):
    a = arr(g["a"])
    l, info = be.cholesky(a, False)
    l, info = to_np(l), u32(info)
    assert near(l[0], g["l0"], tol) and l[0, 0, 1] == 0.0
    assert list(info) == g["info"]
    assert np.isnan(l[1]).all()
    uu, _ = be.cholesky(a[:1], True)
    uu = to_np(uu)
    assert near(uu[0], g["u0"], tol) and uu[0, 1, 0] == 0.0


def check_lu(be, g, tol):
    a = arr(g["a"])
    lu, piv, info = be.lu_factor(a)
    lu, piv, info = to_np(lu), u32(piv), u32(info)
    assert list(piv[0]) == g["pivots0"]
    assert near(lu[0], g["lu0"], tol)
    assert list(info) == g["info"]
    x, _ = be.solve(a[:1], np.array(g["solve_b"], np.float32).reshape(1, 2, 1))
    assert near(to_np(x).ravel(), g["solve_x"], tol)
    xi, info = be.inv(a)
    xi, info = to_np(xi), u32(info)
    assert near(xi[0], g["inv0"], tol)
    assert np.isnan(xi[1]).all() and info[1] == 2


def check_trsm(be, g, tol):
    a = arr([g["a"]])
    b = np.array(g["b"], np.float32).reshape(1, 2, 1)
    x = to_np(be.solve_triangular(a, b, False, False))
    assert near(x.ravel(), g["x"], tol)


def check_eigh_nan(be, g, tol):
    a = np.array([[[float(v) for v in row] for row in m] for m in g["a"]], np.float32)
    w, _, info = be.eigh(a, True, False)
    w, info = to_np(w), u32(info)
    assert not np.isnan(w[0]).any() and np.isnan(w[1]).all()
    assert [bool((i >> 17) & 1) for i in info] == g["info_nonfinite"]


def check_svd_ones(be, g):
    for m, n in g["ones_shapes"]:
        a = np.ones((1, m, n), np.float32)
        _, s, _, _ = be.svd(a, True)
        s = to_np(s)[0]
        assert abs(s[0] - math.sqrt(m * n)) <= 1e-5 * math.sqrt(m * n)
        assert np.all(np.abs(s[1:]) <= 1e-5 * math.sqrt(m * n))


ALL = {
    "qr": check_qr,
    "eigh": check_eigh,
    "svd": check_svd,
    "cholesky": check_cholesky,
    "lu": check_lu,
    "solve_triangular": check_trsm,
    "eigh_nan": check_eigh_nan,
}


def run(be, which):
    g = golden()
    tol = g["tolerance_rel"]
    if which == "svd_closed_forms":
        check_svd_ones(be, g["svd_closed_forms"])
    else:
        ALL[which](be, g[which], tol)
