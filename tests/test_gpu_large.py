"""The large-matrix (blocked) regime on the GPU, BASELINE config 5 and the
blocked paths' edge cases, through the C ABI, against the oracle."""

import numpy as np
import pytest

from _util import bound, config5_matrix, config5_spd, gaussian, rel_recon, to_np, u32

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def spd(n, batch, seed):
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((batch, n, n))
    return (g @ np.swapaxes(g, -1, -2) / n + np.eye(n)).astype(np.float32)


@pytest.mark.parametrize("n", [33, 64, 100, 128, 129, 255, 300, 512])
@pytest.mark.parametrize("upper", [False, True])
def test_cholesky_blocked_shapes(cuda, api, oracle, n, upper):
    a = spd(n, 2, n)
    junk = a.copy()
    iu = np.triu_indices(n, 1) if not upper else np.tril_indices(n, -1)
    junk[:, iu[0], iu[1]] = np.nan
    l, info = api.cholesky(junk, upper)
    lo, io = oracle.cholesky(a, upper)
    assert np.array_equal(u32(info), io) and np.all(io == 0)
    full = np.swapaxes(l, -1, -2) @ l.astype(np.float64) if upper else l.astype(np.float64) @ np.swapaxes(l, -1, -2)
    assert rel_recon(a, full).max() <= bound(n)
    other = np.tril(l, -1) if upper else np.triu(l, 1)
    assert np.all(other == 0)
    assert (np.abs(l - lo).max(axis=(-2, -1)) / np.abs(lo).max(axis=(-2, -1))).max() <= 1e-4


@pytest.mark.parametrize("k", [1, 64, 128, 129, 200, 300])
def test_cholesky_blocked_info(cuda, api, oracle, k):
    n = 300
    a = spd(n, 1, 7)
    a[0, k - 1, k - 1] = -5.0
    l, info = api.cholesky(a, False)
    lo, io = oracle.cholesky(a, False)
    assert u32(info)[0] == io[0] == k
    assert np.isnan(l).all()


def test_config5_cholesky(cuda, api, oracle):
    torch = cuda
    g = config5_matrix()
    a = config5_spd(g)
    l, info = api.cholesky(dev(torch, a[None]), False)
    l, info = to_np(l)[0], u32(info)[0]
    assert info == 0
    lo, io = oracle.cholesky(a[None], False)
    recon = rel_recon(a, l.astype(np.float64) @ l.T.astype(np.float64))
    d = np.abs(l - lo[0]).max() / np.abs(lo[0]).max()
    print(f"[chol config5] recon {recon:.3e} (bound {bound(4096):.3e}) max|L - L_oracle|/max|L| {d:.3e}")
    assert recon <= bound(4096) and d <= 1e-4
    assert np.all(np.triu(l, 1) == 0)
