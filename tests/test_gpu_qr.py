"""QR parity on the GPU, through the C ABI: the HIP kernels against the
oracle on identical seeded inputs (config 1 of BASELINE.json and the
reference's QR edge cases).  Comparisons are sign-invariant: reconstruction
and orthogonality <= 50 n eps_f32, |diag R| against the oracle's, R exactly
upper triangular, NaN isolation bit for bit."""

import numpy as np
import pytest

import _kat
from _util import bound, config1_qr, gaussian, orthogonality, qr_residuals, rel_recon, to_np

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def test_known_answers(cuda, api):
    _kat.run(api, "qr")


def test_config1_parity(cuda, api, oracle):
    torch = cuda
    a = config1_qr()
    q, r = api.qr(dev(torch, a))
    torch.cuda.synchronize()
    q, r = to_np(q), to_np(r)
    recon, ortho = qr_residuals(a, q, r)
    print(f"[qr config1] recon max {recon.max():.3e} ortho max {ortho.max():.3e} bound {bound(32):.3e}")
    assert recon.max() <= bound(32) and ortho.max() <= bound(32)
    assert np.all(np.tril(r, -1) == 0)
    qo, ro = oracle.qr(a)
    d = np.abs(np.abs(np.diagonal(r, axis1=-2, axis2=-1)) - np.abs(np.diagonal(ro, axis1=-2, axis2=-1)))
    scale = np.abs(ro).max(axis=(-2, -1))[:, None]
    assert (d / scale).max() <= bound(32)


def test_host_and_device_pointers_agree(cuda, api):
    torch = cuda
    a = gaussian((500, 24, 20), seed=7)
    qh, rh = api.qr(a)
    qd, rd = api.qr(dev(torch, a))
    assert np.array_equal(qh, to_np(qd)) and np.array_equal(rh, to_np(rd))


@pytest.mark.parametrize("m,n", [(1, 1), (2, 3), (5, 5), (8, 3), (3, 8), (16, 16), (31, 17), (17, 31),
                                 (32, 32), (33, 33), (64, 40), (40, 64), (64, 64), (64, 1), (1, 64)])
@pytest.mark.parametrize("mode", ["reduced", "r", "complete"])
def test_shapes_and_modes(cuda, api, oracle, m, n, mode):
    a = gaussian((37, m, n), seed=m * 131 + n)
    q, r = api.qr(a, mode)
    qo, ro = oracle.qr(a, mode)
    k = min(m, n)
    assert r.shape == ro.shape and (q is None) == (qo is None)
    if q is not None:
        assert q.shape == qo.shape
        assert orthogonality(q).max() <= bound(max(k, q.shape[-1]))
        assert rel_recon(a, q.astype(np.float64) @ r).max() <= bound(max(m, n))
    assert np.all(np.tril(r[..., :k, :], -1) == 0) and np.all(r[..., k:, :] == 0)
    # R agrees with the oracle's up to the signs of its rows
    sgn = np.sign(np.diagonal(r[..., :k, :k], axis1=-2, axis2=-1) * np.diagonal(ro[..., :k, :k], axis1=-2, axis2=-1))
    sgn[sgn == 0] = 1
    diff = np.abs(r[..., :k, :] * sgn[..., None] - ro[..., :k, :]).max(axis=(-2, -1))
    assert (diff / np.maximum(np.abs(ro).max(axis=(-2, -1)), 1e-30)).max() <= 1e-4


def test_nan_isolation_and_magnitudes(cuda, api):
    a = gaussian((8, 32, 32), seed=11)
    a[1, 3, 4] = np.nan
    a[4, 0, 0] = np.inf
    a[5, 31, 31] = -np.inf
    a[2] *= np.float32(1e-30)
    a[3] *= np.float32(1e37)
    a[6] *= np.float32(1e-38)   # subnormal territory after scaling stays exact
    q, r = api.qr(a)
    for b in (1, 4, 5):
        assert np.isnan(q[b]).all() and np.isnan(r[b]).all()
        assert (q[b].view(np.uint32) == 0x7FC00000).all()
    ok = [0, 2, 3, 6, 7]
    recon, ortho = qr_residuals(a[ok], q[ok], r[ok])
    assert recon.max() <= bound(32) and ortho.max() <= bound(32)
    assert not np.isnan(q[ok]).any()


def test_structured_inputs(cuda, api):
    n = 32
    z = np.zeros((1, n, n), np.float32)
    eye = np.eye(n, dtype=np.float32)[None]
    ones = np.ones((1, n, n), np.float32)
    rank1 = (np.arange(1, n + 1, dtype=np.float32)[:, None] * np.linspace(-1, 1, n, dtype=np.float32)[None])[None]
    a = np.concatenate([z, eye, ones, rank1, ones * 1e-20, ones * 1e20])
    q, r = api.qr(a)
    assert not np.isnan(q).any() and not np.isnan(r).any()
    assert orthogonality(q).max() <= bound(n)
    recon = rel_recon(a, q.astype(np.float64) @ r)
    assert recon[1:].max() <= bound(n)
    assert np.all(r[0] == 0)


def test_empty_and_large_batch(cuda, api):
    q, r = api.qr(np.zeros((0, 4, 4), np.float32))
    assert q.shape == (0, 4, 4)
    a = gaussian((70001, 4, 3), seed=3)   # grid of many workgroups, ragged tail
    q, r = api.qr(a)
    recon, ortho = qr_residuals(a, q, r)
    assert recon.max() <= bound(4) and ortho.max() <= bound(3)


def test_complete_with_no_columns_is_identity(cuda, api):
    q, r = api.qr(np.zeros((2, 3, 0), np.float32), "complete")
    assert np.array_equal(q, np.broadcast_to(np.eye(3, dtype=np.float32), (2, 3, 3)))
