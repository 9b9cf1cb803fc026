"""Parity of the batched mid-size thin SVD (65 <= min(m, n) <= 128,
max(m, n) <= 128; one-sided Jacobi, one workgroup per matrix) on the GPU,
through the C ABI, against the oracle on identical seeded inputs.

The reference runs this window on its golub_kahan kernel
(src/svd_golub_kahan.mm:205-211, K up to about 83); before this kernel the
build ran it one matrix at a time through the large-matrix path.  Bounds are
the north star's: reconstruction ||A - U diag(s) V^T|| / ||A|| and the
orthogonality of U and V within 50 n eps_f32, singular values within 1e-5
of the largest, descending and non-negative; info bit 16 on every finite
matrix, bit 18 by the rank-deficient rule (s_min <= 32 FLT_EPSILON s_max,
judged on the oracle's values away from the threshold); a NaN or an
infinity gives all-NaN outputs and info = 1 << 17 without touching the
neighbours.  The batch >= 1024 cases are the window the kernel exists for."""

import numpy as np
import pytest

from _util import bound, gaussian, random_orthogonal, svd_residuals, to_np, u32, values_close

pytestmark = pytest.mark.gpu

QNAN = 0x7FC00000


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def check(api, oracle, a, tag):
    m, n = a.shape[-2:]
    k = min(m, n)
    u, s, vt, info = api.svd(a, True)
    _, so, _, _ = oracle.svd(a, False)
    info = u32(info)
    assert u.shape == a.shape[:-2] + (m, k) and vt.shape == a.shape[:-2] + (k, n)
    assert np.all((info >> 16) & 1) and not np.any((info >> 17) & 1)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    print(f"[svd_mid {tag} {a.shape}] recon {recon.max():.2e} orthoU {ou.max():.2e} orthoV {ov.max():.2e} "
          f"values {close.max():.2e} bound {bound(max(m, n)):.2e}; sweeps {np.mean(info & 0xFFFF):.1f}")
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert close.max() <= 1e-5
    assert np.all(np.diff(s, axis=-1) <= 0) and np.all(s >= 0)
    _, s2, _, info2 = api.svd(a, False)
    assert values_close(s2, s).max() <= 1e-6
    return u, s, vt, info, so


@pytest.mark.parametrize("m,n", [(65, 65), (66, 65), (65, 66), (80, 100), (100, 80), (97, 97), (127, 97),
                                 (128, 65), (65, 128), (100, 100), (128, 128)])
def test_shapes(cuda, api, oracle, m, n):
    a = gaussian((12, m, n), seed=m * 5 + n)
    check(api, oracle, a, "shape")


@pytest.mark.parametrize("m,n", [(128, 128), (128, 80), (80, 128)])
def test_batch_1024(cuda, api, oracle, m, n):
    torch = cuda
    a = gaussian((1024, m, n), seed=m * 11 + n)
    u, s, vt, info = api.svd(dev(torch, a), True)
    torch.cuda.synchronize()
    u, s, vt, info = to_np(u), to_np(s), to_np(vt), u32(info)
    uh, sh, vth, ih = api.svd(a, True)   # host pointers: the pipelined path, the same bytes
    assert np.array_equal(s.view(np.uint32), sh.view(np.uint32)) and np.array_equal(u.view(np.uint32),
                                                                                     uh.view(np.uint32))
    assert np.array_equal(vt.view(np.uint32), vth.view(np.uint32)) and np.array_equal(info, u32(ih))
    _, so, _, _ = oracle.svd(a, False)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    close = values_close(s, so)
    k = min(m, n)
    print(f"[svd_mid batch 1024 {m}x{n}] recon {recon.max():.2e} orthoU {ou.max():.2e} orthoV {ov.max():.2e} "
          f"values {close.max():.2e}; sweeps {np.mean(info & 0xFFFF):.1f} max {np.max(info & 0xFFFF)}")
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert close.max() <= 1e-5 and np.all((info >> 16) & 1)


def test_spectra_and_rank_flag(cuda, api, oracle):
    """Config 3's spectra at 128 x 96: s log-uniform in [1e-6, 1], a quarter
    with the 16 smallest exactly zero; the rank-deficient bit against the
    oracle's values."""
    rng = np.random.default_rng(3)
    batch, m, n = 64, 128, 96
    a = np.empty((batch, m, n), np.float64)
    for b in range(batch):
        sv = np.sort(10.0 ** rng.uniform(-6, 0, size=n))[::-1].copy()
        if b % 4 == 0:
            sv[-16:] = 0.0
        a[b] = (random_orthogonal(rng, m, n) * sv) @ random_orthogonal(rng, n, n).T
    a = a.astype(np.float32)
    u, s, vt, info, so = check(api, oracle, a, "config3 spectra")
    thr = 32 * np.finfo(np.float32).eps * so[:, 0]
    expect = ~(so[:, -1] > thr)
    clear = np.abs(so[:, -1] - thr) > 1e-5 * so[:, 0]
    deficient = ((info >> 18) & 1).astype(bool)
    assert np.array_equal(deficient[clear], expect[clear])
    assert deficient[::4].all()


@pytest.mark.parametrize("m,n", [(100, 100), (128, 70), (70, 128)])
def test_structured(cuda, api, oracle, m, n):
    """Zero (every column completed), identity-like, rank one, repeated
    singular values, a zero column, graded columns."""
    rng = np.random.default_rng(m + n)
    k = min(m, n)
    eye = np.zeros((m, n), np.float32)
    eye[np.arange(k), np.arange(k)] = 1.0
    rank1 = np.outer(rng.standard_normal(m), rng.standard_normal(n)).astype(np.float32)
    rep = ((random_orthogonal(rng, m, k) * np.repeat([3.0, 1.0], (k + 1) // 2)[:k])
           @ random_orthogonal(rng, n, k).T).astype(np.float32)
    zcol = rng.standard_normal((m, n)).astype(np.float32)
    zcol[:, 5] = 0.0
    graded = (rng.standard_normal((m, n)) * 10.0 ** np.linspace(0, -6, n)[None, :]).astype(np.float32)
    a = np.stack([np.zeros((m, n), np.float32), eye, rank1, rep, zcol, graded])
    u, s, vt, info = api.svd(a, True)
    _, so, _, _ = oracle.svd(a, False)
    info = u32(info)
    assert np.all((info >> 16) & 1)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    recon[0] = 0.0   # the zero matrix: no relative reconstruction
    print(f"[svd_mid structured {m}x{n}] recon {np.array2string(recon, precision=2)} orthoU "
          f"{np.array2string(ou, precision=2)} orthoV {np.array2string(ov, precision=2)}")
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(k) and ov.max() <= bound(k)
    assert values_close(s, so).max() <= 1e-5
    assert np.all(s[0] == 0) and (info[0] >> 18) & 1 and (info[2] >> 18) & 1


@pytest.mark.parametrize("m,n", [(128, 128), (80, 100)])
def test_magnitudes(cuda, api, oracle, m, n):
    g = gaussian((6, m, n), seed=29)
    scales = np.array([1e-30, 1e-20, 1e-5, 1e5, 1e20, 1e37], np.float32)
    a = (g.astype(np.float64) * scales[:, None, None]).astype(np.float32)
    check(api, oracle, a, "magnitudes")


@pytest.mark.parametrize("m,n", [(128, 128), (65, 100)])
def test_nonfinite_isolation(cuda, api, m, n):
    a = gaussian((6, m, n), seed=m + n)
    cu, cs, cvt, ci = api.svd(a, True)
    a[1, 0, 0] = np.nan
    a[3, m - 1, n - 1] = np.inf
    a[4, m // 2, 3] = -np.inf
    u, s, vt, info = api.svd(a, True)
    info = u32(info)
    for b in (1, 3, 4):
        assert (u[b].view(np.uint32) == QNAN).all() and (s[b].view(np.uint32) == QNAN).all()
        assert (vt[b].view(np.uint32) == QNAN).all() and info[b] == (1 << 17)
    for b in (0, 2, 5):
        assert np.array_equal(u[b].view(np.uint32), cu[b].view(np.uint32))
        assert np.array_equal(s[b].view(np.uint32), cs[b].view(np.uint32))
        assert np.array_equal(vt[b].view(np.uint32), cvt[b].view(np.uint32))
        assert info[b] == u32(ci)[b]


def test_batch_position(cuda, api):
    torch = cuda
    a = gaussian((100, 90, 70), seed=41)
    r1 = [to_np(x) for x in api.svd(dev(torch, a), True)]
    r2 = [to_np(x) for x in api.svd(dev(torch, a[::-1].copy()), True)]
    for x1, x2 in zip(r1, r2):
        assert np.array_equal(x1.view(np.uint32), x2[::-1].view(np.uint32))
