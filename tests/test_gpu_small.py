"""Cholesky, LU, solve, inverse and triangular solve parity on the GPU
(BASELINE config 4 and the reference's edge cases), through the C ABI,
against the oracle on identical inputs.  Integer outputs (info, pivots) are
compared exactly; pivots may differ only where partial pivoting faces a
near-tie that fp32 rounding order decides, which the test then proves."""

import numpy as np
import pytest

import _kat
from _util import (bound, config4_lu, config4_spd, first_difference, gaussian, lu_residual, near_tie, rel_recon,
                   to_np, u32)

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


@pytest.mark.parametrize("which", ["cholesky", "lu", "solve_triangular"])
def test_known_answers(cuda, api, which):
    _kat.run(api, which)


def test_config4_cholesky(cuda, api, oracle):
    torch = cuda
    a, bad = config4_spd()
    l, info = api.cholesky(dev(torch, a), False)
    l, info = to_np(l), u32(info)
    lo, io = oracle.cholesky(a, False)
    assert np.array_equal(info, io)
    assert np.array_equal(np.nonzero(info)[0], bad) and np.all(info[bad] == 16)
    assert np.isnan(l[bad]).all() and (l[bad].view(np.uint32) == 0x7FC00000).all()
    ok = np.setdiff1d(np.arange(a.shape[0]), bad)
    recon = rel_recon(a[ok], l[ok].astype(np.float64) @ np.swapaxes(l[ok], -1, -2))
    print(f"[chol config4] recon max {recon.max():.3e} bound {bound(16):.3e}")
    assert recon.max() <= bound(16)
    assert np.all(np.triu(l[ok], 1) == 0)
    d = np.abs(l[ok] - lo[ok]).max(axis=(-2, -1)) / np.abs(lo[ok]).max(axis=(-2, -1))
    assert d.max() <= bound(16)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 13, 16, 17, 31, 32, 33, 47, 64, 65, 100, 128])
@pytest.mark.parametrize("upper", [False, True])
def test_cholesky_shapes(cuda, api, oracle, n, upper):
    rng = np.random.default_rng(n)
    bm = rng.standard_normal((50, n, n)).astype(np.float32)
    a = (bm @ np.swapaxes(bm, -1, -2) + n * np.eye(n, dtype=np.float32)).astype(np.float32)
    junk = a.copy()
    iu = np.triu_indices(n, 1) if not upper else np.tril_indices(n, -1)
    junk[:, iu[0], iu[1]] = np.nan   # the unread triangle holds NaN
    l, info = api.cholesky(junk, upper)
    lo, io = oracle.cholesky(a, upper)
    assert np.array_equal(u32(info), io) and np.all(io == 0)
    full = np.swapaxes(l, -1, -2) @ l.astype(np.float64) if upper else l.astype(np.float64) @ np.swapaxes(l, -1, -2)
    assert rel_recon(a, full).max() <= bound(n)
    other = np.tril(l, -1) if upper else np.triu(l, 1)
    assert np.all(other == 0)


@pytest.mark.parametrize("n", [16, 64, 100])
def test_cholesky_info_minors(cuda, api, oracle, n):
    rng = np.random.default_rng(4)
    bm = rng.standard_normal((3, n, n)).astype(np.float32)
    a = (bm @ np.swapaxes(bm, -1, -2) + n * np.eye(n, dtype=np.float32)).astype(np.float32)
    for k in (1, n // 2 + 1, n):
        bad = a.copy()
        bad[1, k - 1, k - 1] = -1e3
        l, info = api.cholesky(bad, False)
        assert list(u32(info)) == [0, k, 0] == list(oracle.cholesky(bad, False)[1])
        assert np.isnan(l[1]).all() and not np.isnan(l[[0, 2]]).any()
    for val, expect in ((np.inf, 1), (np.nan, 1)):
        x = a[:1].copy()
        x[0, 0, 0] = val
        _, info = api.cholesky(x, False)
        assert u32(info)[0] == expect == oracle.cholesky(x, False)[1][0]
    x = a[:1].copy()
    x[0, 9, 3] = np.nan   # read, below the diagonal: reaches pivot 10 first
    _, info = api.cholesky(x, False)
    assert u32(info)[0] == oracle.cholesky(x, False)[1][0] == 10


def test_config4_lu_solve_trsm(cuda, api, oracle):
    torch = cuda
    a, b = config4_lu()
    da, db = dev(torch, a), dev(torch, b)
    lu, piv, info = api.lu_factor(da)
    lu, piv, info = to_np(lu), u32(piv), u32(info)
    luo, pivo, infoo = oracle.lu_factor(a)
    assert np.array_equal(info, infoo) and np.all(info == 0)
    res = lu_residual(a, lu, piv)
    print(f"[lu config4] PA-LU max {res.max():.3e} bound {bound(16):.3e}")
    assert res.max() <= bound(16)
    # pivots are index outputs: identical to LAPACK's, except where a
    # difference is proven to start at a near-tie (each one printed)
    differ = np.nonzero(np.any(piv != pivo, axis=-1))[0]
    print(f"[lu config4] pivot sequences differing from LAPACK's: {len(differ)} of {a.shape[0]}")
    for i in differ:
        print(f"[lu config4]   matrix {i}: first difference at step {first_difference(piv[i], pivo[i])}")
        assert near_tie(a[i], piv[i], pivo[i], rel=1e-5), i
    same = np.setdiff1d(np.arange(a.shape[0]), differ)
    d = np.abs(lu[same] - luo[same]).max(axis=(-2, -1)) / np.abs(luo[same]).max(axis=(-2, -1))
    assert d.max() <= 1e-4

    x, sinfo = api.solve(da, db)
    x = to_np(x).astype(np.float64)
    xo, _ = oracle.solve(a, b)
    assert np.all(u32(sinfo) == 0)
    r = np.linalg.norm(a.astype(np.float64) @ x - b, axis=(-2, -1)) / (
        np.linalg.norm(a.astype(np.float64), axis=(-2, -1)) * np.linalg.norm(x, axis=(-2, -1)))
    print(f"[solve config4] backward error max {r.max():.3e}")
    assert r.max() <= bound(16)

    # trsm on the factors: unit-lower L, then upper U (the oracle's factors, so both read identical bytes)
    y = api.solve_triangular(dev(torch, luo), db, False, True)
    yo = oracle.solve_triangular(luo, b, False, True)
    y = to_np(y)
    assert (np.abs(y - yo).max(axis=(-2, -1)) / np.abs(yo).max(axis=(-2, -1))).max() <= 1e-5
    z = to_np(api.solve_triangular(dev(torch, luo), dev(torch, yo), True, False))
    zo = oracle.solve_triangular(luo, yo, True, False)
    U = np.triu(luo.astype(np.float64))
    rz = np.linalg.norm(U @ z - yo, axis=(-2, -1)) / (np.linalg.norm(U, axis=(-2, -1)) * np.linalg.norm(z, axis=(-2, -1)))
    assert rz.max() <= bound(16)
    assert (np.abs(z - zo).max(axis=(-2, -1)) / np.abs(zo).max(axis=(-2, -1))).max() <= 1e-3


@pytest.mark.parametrize("n", [1, 2, 3, 7, 8, 16, 23, 32, 33, 50, 64])
@pytest.mark.parametrize("nrhs", [1, 4, 17, 40, 70])
def test_solve_shapes(cuda, api, oracle, n, nrhs):
    a = gaussian((40, n, n), seed=n * 7 + nrhs) + np.float32(2 * n) * np.eye(n, dtype=np.float32)
    b = gaussian((40, n, nrhs), seed=nrhs)
    x, info = api.solve(a, b)
    assert np.all(u32(info) == 0)
    r = np.linalg.norm(a.astype(np.float64) @ x - b, axis=(-2, -1)) / (
        np.linalg.norm(a.astype(np.float64), axis=(-2, -1)) * np.linalg.norm(x.astype(np.float64), axis=(-2, -1)))
    assert r.max() <= bound(n)
    xo, _ = oracle.solve(a, b)
    assert (np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))).max() <= 1e-4
    for upper in (False, True):
        for unit in (False, True):
            junk = a.copy()
            iu = np.tril_indices(n, -1) if upper else np.triu_indices(n, 1)
            junk[:, iu[0], iu[1]] = np.nan
            if unit:
                junk[:, np.arange(n), np.arange(n)] = np.nan
            y = api.solve_triangular(junk, b, upper, unit)
            yo = oracle.solve_triangular(a, b, upper, unit)
            assert not np.isnan(y).any()
            assert (np.abs(y - yo).max(axis=(-2, -1)) / np.abs(yo).max(axis=(-2, -1))).max() <= 1e-4


@pytest.mark.parametrize("n", [1, 2, 5, 16, 32, 33, 64, 65, 128])
def test_lu_inv_shapes(cuda, api, oracle, n):
    a = gaussian((60, n, n), seed=n + 100)
    lu, piv, info = api.lu_factor(a)
    assert lu_residual(a, lu, piv).max() <= bound(n)
    assert np.array_equal(u32(info), oracle.lu_factor(a)[2])
    xi, info = api.inv(a)
    xo, _ = oracle.inv(a)
    e = np.abs(a.astype(np.float64) @ xi - np.eye(n)).max(axis=(-2, -1)) / (
        np.abs(a).max(axis=(-2, -1)) * np.abs(xi).max(axis=(-2, -1)) * n)
    assert e.max() <= bound(n)


@pytest.mark.parametrize("n", [5, 40])
def test_singular_lu_gives_nan_for_that_matrix(cuda, api, oracle, n):
    a = gaussian((3, n, n), seed=41)
    a[1, :, 2] = 0.0
    b = gaussian((3, n, 2), seed=42)
    lu, piv, info = api.lu_factor(a)
    assert np.array_equal(u32(info), oracle.lu_factor(a)[2]) and u32(info)[1] == 3
    x, info = api.solve(a, b)
    assert np.isnan(x[1]).all() and not np.isnan(x[[0, 2]]).any() and u32(info)[1] == 3
    xi, info = api.inv(a)
    assert np.isnan(xi[1]).all() and not np.isnan(xi[[0, 2]]).any()
    z = np.zeros((1, 4, 4), np.float32)
    _, piv, info = api.lu_factor(z)
    assert list(u32(piv)[0]) == [0, 1, 2, 3] and u32(info)[0] == 1


def test_host_and_device_pointers_agree(cuda, api):
    torch = cuda
    a, bad = config4_spd(batch=300)
    l1, i1 = api.cholesky(a)
    l2, i2 = api.cholesky(dev(torch, a))
    assert np.array_equal(l1, to_np(l2), equal_nan=True) and np.array_equal(u32(i1), u32(i2))


@pytest.mark.parametrize("n", [33, 48, 64, 65, 100, 128])
def test_lu_factor_one_matrix_per_wave(cuda, api, oracle, n):
    """33 <= n <= 128: the batched factorization with one matrix per wave
    (n <= 64) or per workgroup; a zero column in one matrix gives LAPACK's
    info there and nowhere else."""
    rng = np.random.default_rng(300 + n)
    a = rng.standard_normal((64, n, n)).astype(np.float32)
    k = n // 2
    a[5, :, k - 1] = 0.0
    lu, piv, info = api.lu_factor(a)
    lu, piv, info = to_np(lu), u32(piv), u32(info)
    lo, po, io = oracle.lu_factor(a)
    assert np.array_equal(info, io) and info[5] == k and np.count_nonzero(info) == 1
    res = lu_residual(a, lu, piv)
    assert res.max() <= bound(n), res.max()
    differ = np.nonzero(np.any(piv != po, axis=-1))[0]
    print(f"[lu n={n}] pivot sequences differing from LAPACK's: {len(differ)} of {a.shape[0]}")
    for i in differ:
        print(f"[lu n={n}]   matrix {i}: first difference at step {first_difference(piv[i], po[i])}")
        assert near_tie(a[i], piv[i], po[i], rel=1e-5), i
    same = np.setdiff1d(np.arange(a.shape[0]), differ)
    d = np.abs(lu[same] - lo[same]).max(axis=(-2, -1)) / np.abs(lo[same]).max(axis=(-2, -1))
    assert d.max() <= 1e-3


@pytest.mark.parametrize("n,nrhs", [(65, 3), (100, 70), (128, 8)])
@pytest.mark.parametrize("upper", [False, True])
@pytest.mark.parametrize("unit", [False, True])
def test_solve_triangular_one_workgroup(cuda, api, oracle, n, nrhs, upper, unit):
    """65 <= n <= 128: the triangle and the right-hand sides in LDS; the
    other triangle (and a unit diagonal) hold NaN and must not be read."""
    # off-diagonal entries of size 1/n keep the unit-diagonal triangles well
    # conditioned at this n (N(0,1) entries grow the solution exponentially)
    a = (gaussian((24, n, n), seed=n + nrhs) / np.float32(n) + np.float32(2) * np.eye(n, dtype=np.float32)).astype(
        np.float32)
    b = gaussian((24, n, nrhs), seed=nrhs + 1)
    junk = a.copy()
    iu = np.tril_indices(n, -1) if upper else np.triu_indices(n, 1)
    junk[:, iu[0], iu[1]] = np.nan
    if unit:
        junk[:, np.arange(n), np.arange(n)] = np.nan
    y = api.solve_triangular(junk, b, upper, unit)
    yo = oracle.solve_triangular(a, b, upper, unit)
    assert not np.isnan(y).any()
    assert (np.abs(y - yo).max(axis=(-2, -1)) / np.abs(yo).max(axis=(-2, -1))).max() <= 1e-4


@pytest.mark.parametrize("n", [65, 100, 128])
@pytest.mark.parametrize("nrhs", [1, 17, 70])
def test_solve_one_workgroup(cuda, api, oracle, n, nrhs):
    """65 <= n <= 128: factor, permutation and substitutions in one workgroup
    per matrix (right-hand sides beyond 64 in a second workgroup); a matrix
    with a zero column gives NaN there and LAPACK's info."""
    a = gaussian((24, n, n), seed=n * 7 + nrhs) + np.float32(2 * n) * np.eye(n, dtype=np.float32)
    a[3, :, n // 2] = 0.0
    b = gaussian((24, n, nrhs), seed=nrhs)
    x, info = api.solve(a, b)
    xo, io = oracle.solve(a, b)
    assert np.array_equal(u32(info), io) and u32(info)[3] == n // 2 + 1 and np.count_nonzero(u32(info)) == 1
    assert np.isnan(x[3]).all()
    ok = np.setdiff1d(np.arange(a.shape[0]), [3])
    x, xo, a, b = x[ok], xo[ok], a[ok], b[ok]
    r = np.linalg.norm(a.astype(np.float64) @ x - b, axis=(-2, -1)) / (
        np.linalg.norm(a.astype(np.float64), axis=(-2, -1)) * np.linalg.norm(x.astype(np.float64), axis=(-2, -1)))
    assert r.max() <= bound(n)
    assert (np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))).max() <= 1e-4

