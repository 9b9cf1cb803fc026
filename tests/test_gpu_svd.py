"""Thin SVD parity on the GPU (BASELINE config 3 and the reference's SVD edge
cases), through the C ABI, against the oracle on identical inputs:
reconstruction and orthogonality <= 50 n eps_f32, singular values within
1e-5 of the largest, NaN isolation and the info flag bits."""

import numpy as np
import pytest

import _kat
from _util import bound, config3_svd, gaussian, orthogonality, svd_residuals, to_np, u32, values_close

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


@pytest.mark.parametrize("which", ["svd", "svd_closed_forms"])
def test_known_answers(cuda, api, which):
    _kat.run(api, which)


def test_config3_parity(cuda, api, oracle):
    torch = cuda
    a = config3_svd()
    u, s, vt, info = api.svd(dev(torch, a), True)
    u, s, vt, info = to_np(u), to_np(s), to_np(vt), u32(info)
    uo, so, vto, io = oracle.svd(a, True)
    assert np.all((info >> 16) & 1) and not np.any((info >> 17) & 1)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    print(f"[svd config3] recon max {recon.max():.3e} orthoU {ou.max():.3e} orthoV {ov.max():.3e} "
          f"values max {close.max():.3e} bound {bound(128):.3e}; sweeps mean {np.mean(info & 0xFFFF):.1f}")
    assert recon.max() <= bound(128)
    assert ou.max() <= bound(64) and ov.max() <= bound(64)
    assert close.max() <= 1e-5
    assert np.all(np.diff(s, axis=-1) <= 0) and np.all(s >= 0)
    # rank-deficient flag: set unless s_min > 32 FLT_EPSILON s_max (the reference
    # kernel's rule, Svd_GolubKahan.metal:793-795), judged on the oracle's values
    # away from the threshold
    thr = 32 * np.finfo(np.float32).eps * so[:, 0]
    expect = ~(so[:, -1] > thr)
    clear = np.abs(so[:, -1] - thr) > 1e-5 * so[:, 0]
    deficient = ((info >> 18) & 1).astype(bool)
    assert np.array_equal(deficient[clear], expect[clear])
    assert deficient.sum() >= a.shape[0] // 4   # at least the 16-zero quarter


def test_values_only(cuda, api, oracle):
    a = config3_svd(batch=128)
    _, s1, _, _ = api.svd(a, True)
    u, s2, vt, info = api.svd(a, False)
    assert u is None and vt is None
    assert values_close(s2, s1).max() <= 1e-6
    _, so, _, _ = oracle.svd(a, False)
    assert values_close(s2, so).max() <= 1e-5


@pytest.mark.parametrize("m,n", [(1, 1), (2, 3), (3, 2), (5, 5), (8, 8), (16, 16), (17, 9), (9, 17), (32, 32),
                                 (33, 20), (64, 64), (100, 64), (128, 64), (128, 1), (1, 128), (64, 128),
                                 (128, 33), (40, 90)])
def test_shapes(cuda, api, oracle, m, n):
    a = gaussian((30, m, n), seed=m * 1000 + n)
    u, s, vt, info = api.svd(a, True)
    k = min(m, n)
    assert u.shape == (30, m, k) and s.shape == (30, k) and vt.shape == (30, k, n)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    assert recon.max() <= bound(max(m, n))
    assert ou.max() <= bound(k) and ov.max() <= bound(k)
    _, so, _, _ = oracle.svd(a, False)
    assert values_close(s, so).max() <= 1e-5


def test_structured(cuda, api, oracle):
    n = 64
    m = 128
    rng = np.random.default_rng(9)
    z = np.zeros((m, n), np.float32)
    ones = np.ones((m, n), np.float32)
    rank1 = np.outer(rng.standard_normal(m), rng.standard_normal(n)).astype(np.float32)
    eye = np.eye(m, n, dtype=np.float32)
    graded = (rng.standard_normal((m, n)) * (10.0 ** np.linspace(-6, 0, n))[None, :]).astype(np.float32)
    a = np.stack([z, ones, rank1, eye, graded])
    u, s, vt, info = api.svd(a, True)
    so = oracle.svd(a, False)[1]
    assert np.all((u32(info) >> 16) & 1)
    assert values_close(s, so).max() <= 1e-5
    recon, ou, ov = svd_residuals(a, u, s, vt)
    recon[0] = 0.0
    assert recon.max() <= bound(m)
    assert ou.max() <= bound(n) and ov.max() <= bound(n)
    assert abs(s[1, 0] - np.sqrt(m * n)) <= 1e-5 * np.sqrt(m * n)


def test_nan_isolation_and_magnitudes(cuda, api, oracle):
    a = gaussian((7, 48, 24), seed=31)
    a[2, 5, 5] = np.nan
    a[4, 0, 23] = -np.inf
    scales = np.array([1, 1e-30, 1, 1e30, 1, 1e-20, 1e37], np.float32)
    a = (a.astype(np.float64) * scales[:, None, None]).astype(np.float32)
    u, s, vt, info = api.svd(a, True)
    info = u32(info)
    for b in (2, 4):
        assert np.isnan(s[b]).all() and np.isnan(u[b]).all() and np.isnan(vt[b]).all() and info[b] == (1 << 17)
    ok = [0, 1, 3, 5, 6]
    assert not np.isnan(s[ok]).any()
    recon, ou, ov = svd_residuals(a[ok], u[ok], s[ok], vt[ok])
    assert recon.max() <= bound(48) and ou.max() <= bound(24) and ov.max() <= bound(24)
    assert values_close(s[ok], oracle.svd(a[ok], False)[1]).max() <= 1e-5


def test_host_and_device_pointers_agree(cuda, api):
    torch = cuda
    a = config3_svd(batch=40)
    u1, s1, vt1, _ = api.svd(a, True)
    u2, s2, vt2, _ = api.svd(dev(torch, a), True)
    assert np.array_equal(s1, to_np(s2)) and np.array_equal(u1, to_np(u2)) and np.array_equal(vt1, to_np(vt2))


# ---- beyond the batched kernel's 128 rows: QR, then the SVD of R ----

@pytest.mark.parametrize("m,n,batch", [(129, 64, 6), (300, 40, 5), (1000, 64, 3), (4096, 16, 2), (40, 300, 5),
                                       (64, 1000, 2), (2000, 1, 3)])
def test_tall_and_wide(cuda, api, oracle, m, n, batch):
    a = gaussian((batch, m, n), seed=m * 7 + n)
    u, s, vt, info = api.svd(a, True)
    uo, so, vto, io = oracle.svd(a, True)
    info = u32(info)
    assert np.all((info >> 16) & 1) and not np.any((info >> 17) & 1)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    k = min(m, n)
    print(f"[svd {m}x{n}] recon {recon.max():.3e} orthoU {ou.max():.3e} orthoV {ov.max():.3e} values {close.max():.3e}")
    assert u.shape == (batch, m, k) and vt.shape == (batch, k, n)
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert close.max() <= 1e-5
    assert np.all(np.diff(s, axis=-1) <= 0) and np.all(s >= 0)
    _, s2, _, _ = api.svd(a, False)
    assert values_close(s2, s).max() <= 1e-6


def test_tall_special(cuda, api, oracle):
    rng = np.random.default_rng(41)
    m, n = 700, 48
    mats = [np.zeros((m, n), np.float32), rng.standard_normal((m, n)).astype(np.float32),
            (rng.standard_normal((m, 8)) @ rng.standard_normal((8, n))).astype(np.float32),   # rank 8
            (rng.standard_normal((m, n)) * 1e30).astype(np.float32)]
    a = np.stack(mats)
    a[1, 5, 7] = np.nan
    u, s, vt, info = api.svd(a, True)
    info = u32(info)
    assert np.isnan(s[1]).all() and np.isnan(u[1]).all() and np.isnan(vt[1]).all() and info[1] == (1 << 17)
    ok = [0, 2, 3]
    assert not np.isnan(s[ok]).any() and not np.isnan(u[ok]).any()
    _, so, _, _ = oracle.svd(a[ok], True)
    recon, ou, ov = svd_residuals(a[ok], u[ok], s[ok], vt[ok])
    recon[0] = 0.0   # zero matrix: nothing to reconstruct
    assert recon.max() <= bound(m) and ou.max() <= bound(n) and ov.max() <= bound(n)
    assert values_close(s[ok], so).max() <= 1e-5
    assert (info[2] >> 18) & 1   # rank-deficient


# ---- min(M, N) > 64 beyond the batched windows: bidiagonalisation, then the
# Golub-Kahan tridiagonal's eigenpairs (5000 and 4500 rows: past 4096, the
# fix-up's QR of U is a tree of blocked QRs) ----

@pytest.mark.parametrize("m,n", [(65, 65), (100, 80), (80, 100), (300, 130), (130, 513), (1024, 1024), (5000, 100),
                                 (90, 4500)])
def test_large(cuda, api, oracle, m, n):
    a = gaussian((1, m, n), seed=m * 3 + n)
    u, s, vt, info = api.svd(a, True)
    uo, so, vto, io = oracle.svd(a, True)
    info = u32(info)
    k = min(m, n)
    assert info[0] & (1 << 16) and not info[0] & (1 << 17)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    print(f"[svd large {m}x{n}] recon {recon.max():.3e} orthoU {ou.max():.3e} orthoV {ov.max():.3e} "
          f"values {close.max():.3e} bound {bound(max(m, n)):.3e}")
    assert u.shape == (1, m, k) and vt.shape == (1, k, n)
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert close.max() <= 1e-5
    assert np.all(np.diff(s, axis=-1) <= 0) and np.all(s >= 0)
    _, s2, _, _ = api.svd(a, False)
    assert values_close(s2, s).max() <= 1e-5


def test_large_tall_rank_deficient(cuda, api, oracle):
    """5000 x 120 of rank 60: the zero cluster's columns are rebuilt from the
    QR of U, past 4096 rows a tree of blocked QRs."""
    rng = np.random.default_rng(47)
    m, n = 5000, 120
    a = (rng.standard_normal((m, 60)) @ rng.standard_normal((60, n))).astype(np.float32)[None]
    u, s, vt, info = api.svd(a, True)
    _, so, _, _ = oracle.svd(a, False)
    info = u32(info)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    print(f"[svd large tall rank 60] recon {recon.max():.3e} orthoU {ou.max():.3e} orthoV {ov.max():.3e} "
          f"values {close.max():.3e} info {info[0]:#x}")
    assert recon.max() <= bound(m) and ou.max() <= bound(n) and ov.max() <= bound(n)
    assert close.max() <= 1e-5 and (info[0] >> 18) & 1


def test_large_special(cuda, api, oracle):
    rng = np.random.default_rng(43)
    m, n = 300, 200
    cases = {
        "rank 50": (rng.standard_normal((m, 50)) @ rng.standard_normal((50, n))).astype(np.float32),
        "zero": np.zeros((m, n), np.float32),
        "graded": ((rng.standard_normal((m, n)) * 10.0 ** np.linspace(0, -6, n)[None, :])).astype(np.float32),
        "1e30": (rng.standard_normal((m, n)) * 1e30).astype(np.float32),
    }
    for name, x in cases.items():
        a = x[None]
        u, s, vt, info = api.svd(a, True)
        info = u32(info)
        _, so, _, _ = oracle.svd(a, True)
        recon, ou, ov = svd_residuals(a, u, s, vt)
        if name == "zero":
            recon[:] = 0.0
        print(f"[svd large {name}] recon {recon.max():.3e} orthoU {ou.max():.3e} orthoV {ov.max():.3e} "
              f"values {values_close(s, so).max():.3e} info {info[0]:#x}")
        assert recon.max() <= bound(m) and ou.max() <= bound(n) and ov.max() <= bound(n)
        assert values_close(s, so).max() <= 1e-5
        if name in ("rank 50", "zero"):
            assert info[0] & (1 << 18)
    a = rng.standard_normal((1, m, n)).astype(np.float32)
    a[0, 3, 4] = np.inf
    u, s, vt, info = api.svd(a, True)
    assert np.isnan(s).all() and np.isnan(u).all() and np.isnan(vt).all() and u32(info)[0] == (1 << 17)
