"""LU factor, solve and inverse on non-finite inputs, on the GPU through the
C ABI, against the netlib restatement (oracle/lu_netlib.cpp, pinned in
tests/test_oracle_netlib.py).  The reference runs sgetrf / sgetrs / sgetri on
such input with no scan (src/lu_cpu.mm:72-157): the pivot rule (ISAMAX: the
first of equal magnitudes, a NaN never taken over a number, a NaN on the
diagonal kept) decides where NaN and Inf land.  Compared exactly: info,
pivots, and the positions of NaN and of +-Inf in every output.

Inputs: a Gaussian matrix with NaN, +Inf or -Inf put on the diagonal, below
it, and on the entry that partial pivoting would take in column 0 and in a
later column; an all-NaN column; an all-Inf row; a NaN with a -Inf.  Every
kernel regime is covered: n <= 32 (several matrices per wave), 33-64 (one per
wave), 65-128 (one per workgroup), and the blocked path (n > 128)."""

import numpy as np
import pytest

from _util import config4_lu, gaussian, near_tie, to_np, u32

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def pivot_rows(oracle, a):
    """The original row index that partial pivoting takes at each step."""
    _, piv, _ = oracle.lu_netlib_factor(a[None])
    perm = np.arange(a.shape[0])
    out = []
    for k, p in enumerate(piv[0]):
        perm[[k, p]] = perm[[p, k]]
        out.append(int(perm[k]))
    return out


def nonfinite_cases(oracle, n, seed):
    """[cases, n, n] and a label per case."""
    base = gaussian((n, n), seed=seed)
    k = n // 2
    j = n // 3
    rows = pivot_rows(oracle, base)
    spots = [("diag0", 0, 0), ("diagk", k, k), ("below", n - 1, 0), ("below_k", min(k + 3, n - 1), k),
             ("pivot_col0", rows[0], 0), ("pivot_colj", rows[j], j), ("above", 0, n - 1)]
    mats, labels = [], []
    for name, v in (("nan", np.nan), ("+inf", np.inf), ("-inf", -np.inf)):
        for where, r, c in spots:
            x = base.copy()
            x[r, c] = v
            mats.append(x)
            labels.append(f"{name}@{where}({r},{c})")
    x = base.copy()
    x[:, j] = np.nan
    mats.append(x)
    labels.append(f"nan column {j}")
    x = base.copy()
    x[k, :] = np.inf
    mats.append(x)
    labels.append(f"inf row {k}")
    x = base.copy()
    x[1 % n, 0] = np.nan
    x[n - 1, k] = -np.inf
    mats.append(x)
    labels.append("nan and -inf")
    return np.stack(mats), labels


def same_positions(x, ref):
    x, ref = to_np(x), np.asarray(ref)
    return (np.array_equal(np.isnan(x), np.isnan(ref)) and np.array_equal(np.isposinf(x), np.isposinf(ref))
            and np.array_equal(np.isneginf(x), np.isneginf(ref)))


def check_factor(a, labels, lu, piv, info, oracle, tag):
    lo, po, io = oracle.lu_netlib_factor(a)
    lu, piv, info = to_np(lu), u32(piv), u32(info)
    assert np.array_equal(info, io), (tag, info, io)
    differ = [b for b in range(a.shape[0]) if not np.array_equal(piv[b], po[b])]
    for b in differ:
        print(f"[{tag}] {labels[b]}: pivots part from netlib's at step "
              f"{int(np.nonzero(piv[b] != po[b])[0][0])}")
        assert near_tie(a[b], piv[b], po[b]), (tag, labels[b], piv[b], po[b])
    for b in range(a.shape[0]):
        if b in differ:
            continue
        assert same_positions(lu[b], lo[b]), (tag, labels[b], np.argwhere(np.isnan(lu[b]) != np.isnan(lo[b]))[:5])
    print(f"[{tag}] {a.shape[0]} non-finite matrices: info and NaN/Inf positions identical, "
          f"pivot sequences differing: {len(differ)}")
    return differ


@pytest.mark.parametrize("n", [5, 16, 32, 48, 64, 65, 100, 128, 200, 300])
def test_lu_factor_nonfinite(cuda, api, oracle, n):
    a, labels = nonfinite_cases(oracle, n, seed=900 + n)
    lu, piv, info = api.lu_factor(dev(cuda, a))
    differ = check_factor(a, labels, lu, piv, info, oracle, f"lu_factor n={n}")
    assert len(differ) == 0


@pytest.mark.parametrize("n", [5, 16, 32, 48, 64, 65, 100, 128, 200, 300])
def test_solve_and_inverse_nonfinite(cuda, api, oracle, n):
    a, labels = nonfinite_cases(oracle, n, seed=900 + n)
    rhs = gaussian((a.shape[0], n, 3), seed=950 + n)
    x, info = api.solve(dev(cuda, a), dev(cuda, rhs))
    xo, io = oracle.lu_netlib_solve(a, rhs)
    assert np.array_equal(u32(info), io)
    x = to_np(x)
    for b in range(a.shape[0]):
        assert same_positions(x[b], xo[b]), ("solve", n, labels[b])
    v, info = api.inv(dev(cuda, a))
    vo, io = oracle.lu_netlib_inv(a)
    assert np.array_equal(u32(info), io)
    v = to_np(v)
    for b in range(a.shape[0]):
        assert same_positions(v[b], vo[b]), ("inv", n, labels[b])
    print(f"[solve/inv n={n}] {a.shape[0]} non-finite matrices: info and NaN/Inf positions identical")


def test_config4_batch_with_nonfinite_matrices(cuda, api, oracle):
    """Config 4's 8192 x 16 x 16 batch with 23 non-finite matrices in it:
    the finite matrices' pivots equal LAPACK's (a difference only at a
    proven near-tie, printed), the non-finite ones netlib's."""
    a, b = config4_lu()
    cases, labels = nonfinite_cases(oracle, 16, seed=5)
    where = np.linspace(100, a.shape[0] - 100, len(cases)).astype(int)
    a[where] = cases
    lu, piv, info = api.lu_factor(dev(cuda, a))
    lu, piv, info = to_np(lu), u32(piv), u32(info)
    check_factor(a[where], labels, lu[where], piv[where], info[where], oracle, "config4 non-finite")
    finite = np.setdiff1d(np.arange(a.shape[0]), where)
    lo, po, io = oracle.lu_factor(a[finite])
    assert np.array_equal(info[finite], io)
    differ = np.nonzero(np.any(piv[finite] != po, axis=-1))[0]
    print(f"[config4] finite matrices whose pivots differ from LAPACK's: {len(differ)} of {finite.size}")
    for i in differ:
        step = int(np.nonzero(piv[finite[i]] != po[i])[0][0])
        print(f"[config4]   matrix {finite[i]}: first difference at step {step} (near-tie proven below)")
        assert near_tie(a[finite[i]], piv[finite[i]], po[i], rel=1e-5), finite[i]
    x, sinfo = api.solve(dev(cuda, a), dev(cuda, b))
    xo, io = oracle.lu_netlib_solve(a[where], b[where])
    x = to_np(x)
    assert np.array_equal(u32(sinfo)[where], io)
    for k, m in enumerate(where):
        assert same_positions(x[m], xo[k]), labels[k]
    assert np.isfinite(x[finite]).all()


@pytest.mark.parametrize("n", [16, 48, 100, 128, 300])
def test_inverse_in_place(cuda, api, lib, oracle, n):
    """x aliasing a on the device: every kernel reads the whole matrix
    before it writes any of x (the reference's inv_cpu works on a copy)."""
    a = gaussian((40, n, n), seed=1000 + n) + np.float32(n) * np.eye(n, dtype=np.float32)
    t = dev(cuda, a)
    info = cuda.empty(40, dtype=cuda.int32, device="cuda")
    with lib.lock:
        rc = lib.inv(t.data_ptr(), 40, n, t.data_ptr(), info.data_ptr())
    assert rc == lib.OK
    cuda.cuda.synchronize()
    x = to_np(t)
    xo, io = oracle.inv(a)
    assert np.array_equal(u32(info), io)
    e = np.abs(a.astype(np.float64) @ x - np.eye(n)).max(axis=(-2, -1))
    print(f"[inv in place n={n}] max |A X - I| {e.max():.3e}")
    assert e.max() <= 1e-4
    assert (np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))).max() <= 1e-4


@pytest.mark.parametrize("n,nrhs", [(16, 4), (48, 70), (100, 8), (128, 70), (300, 5)])
def test_solve_in_place(cuda, api, lib, oracle, n, nrhs):
    """x aliasing b on the device (the reference's solve_cpu reads b into
    its own workspace, src/lu_cpu.mm:123-126)."""
    a = gaussian((12, n, n), seed=1100 + n) + np.float32(n) * np.eye(n, dtype=np.float32)
    b = gaussian((12, n, nrhs), seed=1200 + n)
    ta, tb = dev(cuda, a), dev(cuda, b)
    info = cuda.empty(12, dtype=cuda.int32, device="cuda")
    with lib.lock:
        rc = lib.solve(ta.data_ptr(), 12, n, tb.data_ptr(), nrhs, tb.data_ptr(), info.data_ptr())
    assert rc == lib.OK
    cuda.cuda.synchronize()
    x = to_np(tb)
    xo, io = oracle.solve(a, b)
    assert np.array_equal(u32(info), io)
    assert (np.abs(x - xo).max(axis=(-2, -1)) / np.abs(xo).max(axis=(-2, -1))).max() <= 1e-4
