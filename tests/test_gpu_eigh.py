"""Symmetric eigendecomposition parity on the GPU (BASELINE config 2 and the
reference's eigh edge cases), through the C ABI, against the oracle on
identical inputs: residual and orthogonality <= 50 n eps_f32, eigenvalues
within 1e-5 of the largest, NaN isolation and the info flag bits."""

import numpy as np
import pytest

import _kat
from _util import bound, config2_eigh, eigh_residuals, gaussian, orthogonality, symmetrize, to_np, u32, values_close

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


@pytest.mark.parametrize("which", ["eigh", "eigh_nan"])
def test_known_answers(cuda, api, which):
    _kat.run(api, which)


def test_config2_parity(cuda, api, oracle):
    torch = cuda
    a = config2_eigh()
    w, v, info = api.eigh(dev(torch, a), True, True)
    w, v, info = to_np(w), to_np(v), u32(info)
    wo, vo, io = oracle.eigh(a, True, True)
    bad = 7
    assert np.isnan(w[bad]).all() and np.isnan(v[bad]).all() and info[bad] == (1 << 17)
    ok = np.setdiff1d(np.arange(a.shape[0]), [bad])
    assert not np.isnan(w[ok]).any() and not np.isnan(v[ok]).any()
    assert np.all((info[ok] >> 16) & 1) and not np.any((info[ok] >> 17) & 1)
    recon, ortho = eigh_residuals(symmetrize(a[ok]), w[ok], v[ok])
    close = values_close(w[ok], wo[ok])
    print(f"[eigh config2] recon max {recon.max():.3e} ortho max {ortho.max():.3e} values max {close.max():.3e} "
          f"bound {bound(64):.3e}; QL iterations mean {np.mean(info[ok] & 0xFFFF):.1f}")
    assert recon.max() <= bound(64) and ortho.max() <= bound(64)
    assert close.max() <= 1e-5
    assert np.all(np.diff(w[ok], axis=-1) >= 0)


def test_values_only_matches_vectors(cuda, api):
    a = config2_eigh(batch=256, nan_index=None)
    w1, _, _ = api.eigh(a, True, True)
    w2, v2, _ = api.eigh(a, True, False)
    assert v2 is None
    assert values_close(w2, w1).max() <= 1e-6


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 13, 16, 17, 31, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("lower", [True, False])
def test_shapes_and_triangles(cuda, api, oracle, n, lower):
    g = gaussian((40, n, n), seed=n * 3 + lower)
    junk = g.copy()
    iu = np.triu_indices(n, 1) if lower else np.tril_indices(n, -1)
    junk[:, iu[0], iu[1]] = np.nan   # the unread triangle holds NaN
    w, v, info = api.eigh(junk, lower, True)
    wo, _, _ = oracle.eigh(g, lower, False)
    s = symmetrize(g, lower)
    assert not np.isnan(w).any() and not np.isnan(v).any()
    recon, ortho = eigh_residuals(s, w, v)
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert values_close(w, wo).max() <= 1e-5


def with_spectrum(rng, spec):
    n = len(spec)
    q, r = np.linalg.qr(rng.standard_normal((n, n)))
    q = q * np.sign(np.diag(r))
    return ((q * spec) @ q.T).astype(np.float32)


def test_structured_spectra(cuda, api, oracle):
    rng = np.random.default_rng(17)
    n = 64
    mats = [np.zeros((n, n), np.float32), np.eye(n, dtype=np.float32), np.ones((n, n), np.float32),
            with_spectrum(rng, np.repeat([1.0, -2.0, 3.0, 0.5], n // 4)),               # repeated
            with_spectrum(rng, 1.0 + 1e-6 * np.arange(n)),                              # clustered
            with_spectrum(rng, 10.0 ** np.linspace(-6, 0, n)),                          # graded
            np.diag(np.arange(n, dtype=np.float32)),                                    # already diagonal
            (np.diag(np.full(n, 2.0)) - np.diag(np.ones(n - 1), 1) - np.diag(np.ones(n - 1), -1)).astype(np.float32)]
    a = np.stack(mats)
    w, v, info = api.eigh(a, True, True)
    wo, _, _ = oracle.eigh(a, True, False)
    assert np.all((u32(info) >> 16) & 1)
    recon, ortho = eigh_residuals(a, w, v)
    recon[0] = 0.0 if np.abs(w[0]).max() == 0 else recon[0]
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert values_close(w, wo).max() <= 1e-5
    assert np.abs(w[2, -1] - n) <= 1e-5 * n and np.abs(w[2, :-1]).max() <= 1e-5 * n


def test_magnitudes(cuda, api, oracle):
    g = gaussian((6, 32, 32), seed=23)
    s = (g + np.swapaxes(g, -1, -2)) / 2
    scales = np.array([1e-30, 1e-20, 1e-5, 1e5, 1e20, 1e37], np.float32)
    a = (s.astype(np.float64) * scales[:, None, None]).astype(np.float32)
    w, v, _ = api.eigh(a, True, True)
    wo, _, _ = oracle.eigh(a, True, False)
    recon, ortho = eigh_residuals(a, w, v)
    assert recon.max() <= bound(32) and ortho.max() <= bound(32)
    assert values_close(w, wo).max() <= 1e-5


def test_inf_and_host_pointers(cuda, api):
    torch = cuda
    a = config2_eigh(batch=64, nan_index=None)
    a[5, 10, 3] = np.inf     # read (lower)
    a[9, 3, 10] = np.inf     # unread (upper): ignored
    w, v, info = api.eigh(a, True, True)
    info = u32(info)
    assert np.isnan(w[5]).all() and info[5] == (1 << 17)
    assert not np.isnan(w[9]).any() and (info[9] >> 16) & 1
    w2, v2, info2 = api.eigh(dev(torch, a), True, True)
    assert np.array_equal(w, to_np(w2), equal_nan=True) and np.array_equal(v, to_np(v2), equal_nan=True)


def test_result_does_not_depend_on_batch_position(cuda, api):
    """A matrix's eigenpairs are bit-identical wherever it sits in the batch
    (the kernels' inverse-iteration start vector is the same for every
    matrix), so a batch split into chunks gives the whole batch's result."""
    from _util import config2_eigh

    a = config2_eigh(batch=300, n=64, seed=12)
    w1, v1, i1 = (to_np(x) for x in api.eigh(cuda.from_numpy(a).to("cuda")))
    w2, v2, i2 = (to_np(x) for x in api.eigh(cuda.from_numpy(a[::-1].copy()).to("cuda")))
    assert np.array_equal(w1.view(np.uint32), w2[::-1].view(np.uint32))
    assert np.array_equal(v1.view(np.uint32), v2[::-1].view(np.uint32))
    assert np.array_equal(i1, i2[::-1])


@pytest.mark.parametrize("n", [16, 32, 64])
def test_large_groups_of_close_eigenvalues(cuda, api, oracle, n):
    """Half the spectrum one eigenvalue and half another (groups of n / 2
    for the Gram-Schmidt rounds), and a group spread over 1e-7: the
    inverse-iteration shifts inside a group are set apart (sstein's rule),
    so every member converges to its own vector of the group."""
    rng = np.random.default_rng(n + 1)
    mats = [with_spectrum(rng, np.repeat([2.0, -1.0], n // 2)),
            with_spectrum(rng, np.concatenate([1.0 + 1e-7 * np.arange(n // 2), np.linspace(-3, -2, n - n // 2)])),
            with_spectrum(rng, np.repeat([0.0, 5.0], n // 2))]
    a = np.stack(mats)
    w, v, info = api.eigh(a, True, True)
    wo, _, _ = oracle.eigh(a, True, False)
    recon, ortho = eigh_residuals(a, w, v)
    print(f"[eigh groups n={n}] recon {np.array2string(recon, precision=2)} ortho {np.array2string(ortho, precision=2)}")
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert values_close(w, wo).max() <= 1e-5
