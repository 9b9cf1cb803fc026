"""Pins the oracle (oracle/lapack_batch.cpp) before anything is checked
against it: the reference C-API test's known answers, closed forms,
invariants on seeded inputs, an independent LAPACK (numpy's own OpenBLAS
build) for values, brute-force partial pivoting for LU pivots, the
reference's special cases (NaN isolation, non-SPD info, singular LU), and
planted mistakes that the checks must catch.  CPU only."""

import math

import numpy as np
import pytest

import _kat
from _util import (bound, eigh_residuals, gaussian, lu_residual, lu_unpack, orthogonality, qr_residuals,
                   rel_recon, svd_residuals, symmetrize, values_close)


@pytest.mark.parametrize("which", list(_kat.ALL) + ["svd_closed_forms"])
def test_known_answers(oracle, which):
    _kat.run(oracle, which)


@pytest.mark.parametrize("m,n", [(32, 32), (48, 20), (20, 48), (1, 5), (7, 1), (64, 64)])
def test_qr_invariants(oracle, m, n):
    a = gaussian((50, m, n), seed=m * 100 + n)
    q, r = oracle.qr(a)
    recon, ortho = qr_residuals(a, q, r)
    k = min(m, n)
    assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(k)
    assert np.all(np.tril(r[..., :k, :k], -1) == 0)
    _, r_alone = oracle.qr(a, "r")
    np.testing.assert_allclose(r_alone, r, rtol=0, atol=1e-5 * np.abs(r).max())
    qc, rc = oracle.qr(a, "complete")
    assert qc.shape == (50, m, m) and rc.shape == (50, m, n)
    assert orthogonality(qc).max() <= bound(m)
    assert rel_recon(a, qc.astype(np.float64) @ rc).max() <= bound(max(m, n))


def test_qr_nan_isolation_and_magnitudes(oracle):
    a = gaussian((6, 16, 16), seed=11)
    a[1, 3, 4] = np.nan
    a[4, 0, 0] = np.inf
    a[2] *= 1e-30
    a[3] *= 1e30
    q, r = oracle.qr(a)
    assert np.isnan(q[1]).all() and np.isnan(r[1]).all() and np.isnan(r[4]).all()
    ok = [0, 2, 3, 5]
    recon, ortho = qr_residuals(a[ok], q[ok], r[ok])
    assert recon.max() <= bound(16) and ortho.max() <= bound(16)


@pytest.mark.parametrize("n", [2, 16, 64])
def test_eigh_invariants_and_independent_values(oracle, n):
    g = gaussian((40, n, n), seed=n)
    s = ((g + np.swapaxes(g, -1, -2)) / 2).astype(np.float32)
    w, v, info = oracle.eigh(s, True, True)
    recon, ortho = eigh_residuals(s, w, v)
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert np.all(np.diff(w, axis=-1) >= 0)
    assert np.all(info == (1 | (1 << 16)))
    ref = np.linalg.eigvalsh(s.astype(np.float64))   # numpy's own LAPACK build, in double
    assert values_close(w, ref).max() <= 1e-5
    w2, v2, _ = oracle.eigh(s, True, False)
    assert v2 is None and values_close(w2, w).max() <= 1e-5


def test_eigh_reads_one_triangle(oracle):
    g = gaussian((8, 12, 12), seed=5)
    junk = g.copy()
    junk[:, np.triu_indices(12, 1)[0], np.triu_indices(12, 1)[1]] = np.nan   # upper holds NaN
    w, v, info = oracle.eigh(junk, True, True)
    assert not np.isnan(w).any()
    ref = np.linalg.eigvalsh(symmetrize(g, lower=True))
    assert values_close(w, ref).max() <= 1e-5
    w_up, _, _ = oracle.eigh(np.swapaxes(junk, -1, -2).copy(), False, False)
    assert values_close(w_up, ref).max() <= 1e-5


def test_eigh_closed_form_2x2(oracle):
    rng = np.random.default_rng(3)
    a, b, c = rng.standard_normal((3, 100))
    m = np.stack([np.stack([a, b], -1), np.stack([b, c], -1)], -2).astype(np.float32)
    w, _, _ = oracle.eigh(m, True, False)
    a, b, c = (m[:, 0, 0].astype(np.float64), m[:, 1, 0].astype(np.float64), m[:, 1, 1].astype(np.float64))
    mid, rad = (a + c) / 2, np.hypot((a - c) / 2, b)
    ref = np.stack([mid - rad, mid + rad], -1)
    assert values_close(w, ref).max() <= 1e-5


def test_eigh_nan_matrix(oracle):
    s = gaussian((3, 8, 8), seed=9)
    s = (s + np.swapaxes(s, -1, -2)) / 2
    s[1, 5, 2] = np.nan   # in the lower triangle
    w, v, info = oracle.eigh(s, True, True)
    assert np.isnan(w[1]).all() and np.isnan(v[1]).all() and info[1] == (1 << 17)
    assert not np.isnan(w[[0, 2]]).any()


@pytest.mark.parametrize("m,n", [(128, 64), (64, 64), (40, 90), (6, 4)])
def test_svd_invariants_and_independent_values(oracle, m, n):
    a = gaussian((30, m, n), seed=m + n)
    u, s, vt, info = oracle.svd(a, True)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    k = min(m, n)
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert np.all(np.diff(s, axis=-1) <= 0) and np.all(s >= 0)
    ref = np.linalg.svd(a.astype(np.float64), compute_uv=False)
    assert values_close(s, ref).max() <= 1e-5
    _, s2, _, _ = oracle.svd(a, False)
    assert values_close(s2, s).max() <= 1e-5


def test_svd_rank_one_closed_form(oracle):
    rng = np.random.default_rng(8)
    x, y = rng.standard_normal((20, 7, 1)), rng.standard_normal((20, 1, 5))
    a = (x @ y).astype(np.float32)
    _, s, _, _ = oracle.svd(a, True)
    ref = np.linalg.norm(x[..., 0], axis=-1) * np.linalg.norm(y[:, 0], axis=-1)
    assert np.all(np.abs(s[:, 0] - ref) <= 1e-5 * ref)
    assert np.all(s[:, 1:] <= 1e-5 * ref[:, None])


def test_cholesky_invariants_and_info(oracle):
    n = 16
    rng = np.random.default_rng(4)
    bm = rng.standard_normal((64, n, n)).astype(np.float32)
    a = (bm @ np.swapaxes(bm, -1, -2) + n * np.eye(n, dtype=np.float32)).astype(np.float32)
    l, info = oracle.cholesky(a, False)
    assert np.all(info == 0)
    assert rel_recon(a, l.astype(np.float64) @ np.swapaxes(l, -1, -2)).max() <= bound(n)
    assert np.all(np.triu(l, 1) == 0)
    u, _ = oracle.cholesky(a, True)
    np.testing.assert_allclose(u, np.swapaxes(l, -1, -2), rtol=0, atol=1e-5 * np.abs(l).max())
    # non-PD at the minors of order 1, n/2+1 and n (test_cholesky.cpp:163-222)
    for k in (1, n // 2 + 1, n):
        bad = a[:3].copy()
        bad[1, k - 1, k - 1] = -1e3
        lb, ib = oracle.cholesky(bad, False)
        assert list(ib) == [0, k, 0]
        assert np.isnan(lb[1]).all() and not np.isnan(lb[[0, 2]]).any()
    inf = a[:1].copy()
    inf[0, 0, 0] = np.inf
    _, ii = oracle.cholesky(inf, False)
    assert ii[0] == 1


def gepp_pivots(a):
    """Partial pivoting in float64, first maximum on ties (LAPACK isamax)."""
    a = a.astype(np.float64).copy()
    n = a.shape[0]
    piv = []
    for k in range(n):
        p = k + int(np.argmax(np.abs(a[k:, k])))
        piv.append(p)
        a[[k, p]] = a[[p, k]]
        if a[k, k] != 0:
            a[k + 1:, k] /= a[k, k]
            a[k + 1:, k + 1:] -= np.outer(a[k + 1:, k], a[k, k + 1:])
    return piv


def test_lu_pivots_and_residual(oracle):
    a = gaussian((300, 6, 6), seed=21)
    lu, piv, info = oracle.lu_factor(a)
    assert np.all(info == 0)
    for b in range(300):
        assert list(piv[b]) == gepp_pivots(a[b]), b
    assert lu_residual(a, lu, piv).max() <= bound(6)
    a16 = gaussian((200, 16, 16), seed=22)
    lu, piv, info = oracle.lu_factor(a16)
    assert lu_residual(a16, lu, piv).max() <= bound(16)


def test_solve_inv_trsm(oracle):
    n = 16
    a = gaussian((100, n, n), seed=31)
    b = gaussian((100, n, 4), seed=32)
    x, info = oracle.solve(a, b)
    assert np.all(info == 0)
    res = np.linalg.norm(a.astype(np.float64) @ x - b, axis=(-2, -1)) / (
        np.linalg.norm(a.astype(np.float64), axis=(-2, -1)) * np.linalg.norm(x.astype(np.float64), axis=(-2, -1)))
    assert res.max() <= bound(n)
    xi, _ = oracle.inv(a)
    assert np.abs(a.astype(np.float64) @ xi - np.eye(n)).max() <= 1e-3
    lu, piv, _ = oracle.lu_factor(a)
    lower = oracle.solve_triangular(lu, b, False, True)
    ref = np.linalg.solve(np.tril(lu.astype(np.float64), -1) + np.eye(n), b.astype(np.float64))
    assert np.abs(lower - ref).max() <= 1e-4 * np.abs(ref).max()
    upper = oracle.solve_triangular(lu, b, True, False)
    ref = np.linalg.solve(np.triu(lu.astype(np.float64)), b.astype(np.float64))
    assert (np.abs(upper - ref).max(axis=(-2, -1)) / np.abs(ref).max(axis=(-2, -1))).max() <= 1e-3


def test_singular_lu_gives_nan_for_that_matrix(oracle):
    a = gaussian((3, 5, 5), seed=41)
    a[1, :, 2] = 0.0
    b = gaussian((3, 5, 2), seed=42)
    _, _, info = oracle.lu_factor(a)
    assert info[0] == 0 and info[1] > 0 and info[2] == 0
    x, info = oracle.solve(a, b)
    assert np.isnan(x[1]).all() and not np.isnan(x[[0, 2]]).any()
    xi, _ = oracle.inv(a)
    assert np.isnan(xi[1]).all() and not np.isnan(xi[[0, 2]]).any()


def test_planted_mistakes_are_caught(oracle):
    """The measures above fail on plausible mistakes (made here, on the CPU)."""
    a = gaussian((4, 16, 16), seed=51)
    q, r = oracle.qr(a)
    qt = np.swapaxes(q, -1, -2).copy()             # transposed operand
    assert qr_residuals(a, qt, r)[0].max() > bound(16)
    q2 = q.copy()
    q2[..., 3] *= -1                               # a sign dropped in one column
    assert qr_residuals(a, q2, r)[0].max() > bound(16)
    s = ((a + np.swapaxes(a, -1, -2)) / 2).astype(np.float32)
    w, v, _ = oracle.eigh(s, True, True)
    w2 = w.copy()
    w2[:, [0, 1]] = w2[:, [1, 0]]                  # wrong order / index
    assert eigh_residuals(s, w2, v)[0].max() > bound(16)
    lu, piv, _ = oracle.lu_factor(a)
    piv2 = piv.copy()
    piv2[:, 0] = (piv2[:, 0] + 1) % 16             # wrong pivot index
    assert lu_residual(a, lu, piv2).max() > bound(16)
    assert lu_residual(a, np.swapaxes(lu, -1, -2).copy(), piv).max() > bound(16)


def test_threads_do_not_change_results(oracle):
    a = gaussian((257, 20, 20), seed=61)
    before = oracle.threads()
    oracle.set_threads(1)
    q1, r1 = oracle.qr(a)
    oracle.set_threads(0)
    q2, r2 = oracle.qr(a)
    oracle.set_threads(before if before else 0)
    assert np.array_equal(q1, q2) and np.array_equal(r1, r2)
