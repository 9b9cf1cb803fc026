"""Pins the netlib restatement of LU / solve / inverse (oracle/lu_netlib.cpp),
the checker for non-finite LU inputs, before any GPU result is compared with
it.  CPU only.

- Finite inputs: the same pivots as the OpenBLAS-backed oracle (the
  reference's CPU path restated) except at proven near-ties, and factors,
  solutions and inverses within fp32 tolerance of it.
- ISAMAX's rule in closed form: the first of equal magnitudes; a NaN never
  taken over a number; a NaN on the diagonal kept; an infinity taken; an
  all-NaN column keeps its diagonal.
- Non-finite inputs against an independent pure-Python sgetf2 loop (float32,
  numpy per column), which shares no code with the C++ restatement: pivots,
  info and the NaN / Inf positions identical.
- Closed forms for solve and inverse: a NaN in one right-hand-side column
  makes that column of x NaN and no other; an upper triangle with one NaN
  above the diagonal has an all-NaN inverse (0 * NaN in the rank-1 update);
  inv of diag(Inf, 2, 4) = diag(0, 0.5, 0.25).
- A planted mistake (ISAMAX taking the last of equal magnitudes, or taking a
  NaN) is caught by the checks above.
"""

import numpy as np
import pytest

from _util import bound, gaussian, lu_residual

F32 = np.float32


def py_getf2(a, last_of_ties=False, nan_wins=False):
    """Independent sgetf2 (float32): ISAMAX, swap, scale, rank-1 update.
    The two flags plant mistakes in the pivot rule."""
    a = np.array(a, dtype=F32, copy=True)
    n = a.shape[0]
    piv = np.zeros(n, np.uint32)
    info = 0
    with np.errstate(all="ignore"):
        for k in range(n):
            col = np.abs(a[k:, k])
            p, smax = 0, col[0]
            for i in range(1, col.size):
                v = col[i]
                better = v > smax or (last_of_ties and v == smax) or (nan_wins and np.isnan(v))
                if better:
                    p, smax = i, v
            p += k
            piv[k] = p
            if a[p, k] != 0:
                if p != k:
                    a[[k, p]] = a[[p, k]]
                if abs(a[k, k]) >= np.finfo(F32).tiny:
                    a[k + 1:, k] = a[k + 1:, k] * (F32(1) / a[k, k])
                else:
                    a[k + 1:, k] = a[k + 1:, k] / a[k, k]
            elif info == 0:
                info = k + 1
            a[k + 1:, k + 1:] = a[k + 1:, k + 1:] - np.outer(a[k + 1:, k], a[k, k + 1:]).astype(F32)
    return a, piv, info


def near_tie(a, piv_x, piv_y, rel=1e-4):
    """The first step where two pivot sequences part is a near-tie of
    column magnitudes (float64 elimination along piv_y)."""
    a = a.astype(np.float64).copy()
    for k in range(a.shape[0]):
        if piv_x[k] != piv_y[k]:
            m1, m2 = abs(a[piv_x[k], k]), abs(a[piv_y[k], k])
            return abs(m1 - m2) <= rel * max(m1, m2)
        p = piv_y[k]
        a[[k, p]] = a[[p, k]]
        if a[k, k] != 0:
            a[k + 1:, k] /= a[k, k]
            a[k + 1:, k + 1:] -= np.outer(a[k + 1:, k], a[k, k + 1:])
    return True


@pytest.mark.parametrize("n", [3, 16, 48, 100])
def test_finite_inputs_match_the_lapack_oracle(oracle, n):
    a = gaussian((120, n, n), seed=700 + n)
    lu, piv, info = oracle.lu_netlib_factor(a)
    luo, pivo, infoo = oracle.lu_factor(a)
    assert np.array_equal(info, infoo) and np.all(info == 0)
    differ = np.nonzero(np.any(piv != pivo, axis=-1))[0]
    for i in differ:
        assert near_tie(a[i], piv[i], pivo[i]), i
    assert len(differ) <= 1
    assert lu_residual(a, lu, piv).max() <= bound(n)
    same = np.setdiff1d(np.arange(a.shape[0]), differ)
    d = np.abs(lu[same] - luo[same]).max(axis=(-2, -1)) / np.abs(luo[same]).max(axis=(-2, -1))
    assert d.max() <= 1e-3
    # two backward-stable solves differ by at most ~ n eps cond(A) relative
    cond = np.linalg.cond(a.astype(np.float64))
    rhs = gaussian((120, n, 5), seed=800 + n)
    x, xi = oracle.lu_netlib_solve(a, rhs)
    xo, _ = oracle.solve(a, rhs)
    assert np.all(xi == 0)
    dx = np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))
    assert np.all(dx <= 4 * n * np.finfo(F32).eps * cond)
    v, vi = oracle.lu_netlib_inv(a)
    vo, _ = oracle.inv(a)
    assert np.all(vi == 0)
    dv = np.abs(v - vo).max(axis=(-2, -1)) / np.abs(vo).max(axis=(-2, -1))
    assert np.all(dv <= 4 * n * np.finfo(F32).eps * cond)
    e = np.abs(a.astype(np.float64) @ v - np.eye(n)).max(axis=(-2, -1)) / (
        np.abs(a).max(axis=(-2, -1)) * np.abs(v).max(axis=(-2, -1)) * n)
    assert e.max() <= bound(n)


def test_pivot_rule_closed_forms(oracle):
    rest = gaussian((4, 3), seed=1)

    def first_pivot(col):
        a = np.concatenate([np.array(col, F32)[:, None], rest], axis=1)
        _, piv, info = oracle.lu_netlib_factor(a[None])
        return int(piv[0, 0]), int(info[0])

    assert first_pivot([1, -1, 1, 0.5]) == (0, 0)           # ties: the first
    assert first_pivot([0.5, -1, 1, 1]) == (1, 0)
    assert first_pivot([0.5, np.nan, 3, -3]) == (2, 0)      # NaN below: never taken
    assert first_pivot([np.nan, 5, -7, 1]) == (0, 0)        # NaN on the diagonal: kept
    assert first_pivot([2, np.inf, -np.inf, 1]) == (1, 0)   # infinities: the first
    assert first_pivot([0, 0, np.nan, 0]) == (0, 1)         # zero pivot kept, info 1

    # NaN on the diagonal: every multiplier and the whole trailing block NaN,
    # every later pivot its diagonal
    a = gaussian((1, 6, 6), seed=2)
    a[0, 0, 0] = np.nan
    lu, piv, info = oracle.lu_netlib_factor(a)
    assert list(piv[0]) == list(range(6)) and info[0] == 0
    assert np.isnan(lu[0, 1:, :]).all() and np.array_equal(lu[0, 0, 1:], a[0, 0, 1:])
    # an all-NaN column: its diagonal is the pivot
    a = gaussian((1, 6, 6), seed=3)
    a[0, :, 2] = np.nan
    _, piv, _ = oracle.lu_netlib_factor(a)
    assert piv[0, 2] == 2
    # an infinite pivot: multipliers finite / inf = 0, U's first row the pivot row
    a = gaussian((1, 5, 5), seed=4)
    a[0, 3, 0] = np.inf
    lu, piv, _ = oracle.lu_netlib_factor(a)
    assert piv[0, 0] == 3 and np.all(lu[0, 1:, 0] == 0)
    assert np.array_equal(lu[0, 0], a[0, 3])


CASES = [(np.nan, (0, 0)), (np.nan, (3, 3)), (np.nan, (6, 1)), (np.nan, (1, 6)), (np.inf, (0, 0)),
         (np.inf, (5, 2)), (-np.inf, (2, 2)), (-np.inf, (7, 0)), (np.inf, (0, 7))]


def nonfinite_batch(n, seed):
    base = gaussian((n, n), seed=seed)
    out = []
    for val, (i, j) in CASES:
        x = base.copy()
        x[i % n, j % n] = val
        out.append(x)
    x = base.copy()
    x[:, 4 % n] = np.nan
    out.append(x)
    x = base.copy()
    x[2 % n, :] = np.inf
    out.append(x)
    x = base.copy()
    x[1 % n, 1 % n] = np.nan
    x[5 % n, 3 % n] = -np.inf
    out.append(x)
    return np.stack(out)


@pytest.mark.parametrize("n", [5, 9])
def test_nonfinite_factor_matches_independent_loop(oracle, n):
    a = nonfinite_batch(n, seed=n)
    lu, piv, info = oracle.lu_netlib_factor(a)
    for b in range(a.shape[0]):
        lp, pp, ip = py_getf2(a[b])
        assert np.array_equal(piv[b], pp), b
        assert info[b] == ip, b
        assert np.array_equal(np.isnan(lu[b]), np.isnan(lp)), b
        assert np.array_equal(np.isinf(lu[b]), np.isinf(lp)), b


def test_planted_pivot_mistakes_are_caught(oracle):
    a = nonfinite_batch(9, seed=9)
    _, piv, _ = oracle.lu_netlib_factor(a)
    caught_nan = any(not np.array_equal(piv[b], py_getf2(a[b], nan_wins=True)[1]) for b in range(a.shape[0]))
    assert caught_nan
    ties = np.array([[1, 2, 3], [-1, 5, 1], [1, 1, 7]], F32)
    assert oracle.lu_netlib_factor(ties[None])[1][0, 0] != py_getf2(ties, last_of_ties=True)[1][0]


def test_solve_and_inverse_closed_forms(oracle):
    n = 6
    a = gaussian((1, n, n), seed=5) + F32(4) * np.eye(n, dtype=F32)
    rhs = gaussian((1, n, 3), seed=6)
    rhs[0, 2, 1] = np.nan
    x, info = oracle.lu_netlib_solve(a, rhs)
    assert info[0] == 0 and np.isnan(x[0, :, 1]).all() and not np.isnan(x[0][:, [0, 2]]).any()
    ref = np.linalg.solve(a[0].astype(np.float64), np.nan_to_num(rhs[0].astype(np.float64))[:, [0, 2]])
    assert np.abs(x[0][:, [0, 2]] - ref).max() <= 1e-4 * np.abs(ref).max()

    # an upper triangle with one NaN above the diagonal, at (i, j): the
    # rank-1 update of step i forms 0 * NaN down column j, so U(j, j) is NaN
    # and sgetri's column loop carries it into every column: all NaN; the
    # pivots stay on the diagonal up to j
    u = np.triu(gaussian((n, n), seed=7)) + F32(3) * np.eye(n, dtype=F32)
    u[1, 3] = np.nan
    lu, piv, info = oracle.lu_netlib_factor(u[None])
    assert info[0] == 0 and list(piv[0, :4]) == [0, 1, 2, 3]
    assert np.isnan(lu[0, 2:, 3]).all() and not np.isnan(lu[0, :, :3]).any()
    v, info = oracle.lu_netlib_inv(u[None])
    assert info[0] == 0 and np.isnan(v[0]).all()

    d = np.diag(np.array([np.inf, 2, 4], F32))[None]
    v, info = oracle.lu_netlib_inv(d)
    assert info[0] == 0 and np.array_equal(v[0], np.diag(np.array([0, 0.5, 0.25], F32)))


def test_singular_gives_nan(oracle):
    a = gaussian((3, 7, 7), seed=8)
    a[1, :, 3] = 0
    _, _, info = oracle.lu_netlib_factor(a)
    assert list(info) == [0, 4, 0] == list(oracle.lu_factor(a)[2])
    x, info = oracle.lu_netlib_solve(a, gaussian((3, 7, 2), seed=9))
    assert np.isnan(x[1]).all() and not np.isnan(x[[0, 2]]).any()
    v, _ = oracle.lu_netlib_inv(a)
    assert np.isnan(v[1]).all() and not np.isnan(v[[0, 2]]).any()
