"""Parity of the batched mid-size symmetric eigendecomposition (65 <= n <=
128, one workgroup of two waves per matrix) on the GPU, through the C ABI,
against the oracle on identical seeded inputs.

The reference runs this window on its eigh_ql kernel (src/eigh_ql.mm:151-163,
n up to about 87); before this kernel the build ran it one matrix at a time
through the blocked path.  Bounds are the north star's: residual
||A - V diag(w) V^T|| / ||A|| and orthogonality ||V^T V - I|| within
50 n eps_f32, eigenvalues within 1e-5 of the largest, ascending; a NaN or an
infinity in the read triangle gives all-NaN w and V with info = 1 << 17 and
leaves the other matrices bit-identical; info bit 16 on every finite
matrix.  The batch >= 1024 cases are the window the kernel exists for."""

import numpy as np
import pytest

from _util import bound, eigh_residuals, gaussian, orthogonality, symmetrize, to_np, u32, values_close

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def sym(batch, n, seed):
    g = gaussian((batch, n, n), seed=seed).astype(np.float64)
    return ((g + np.swapaxes(g, -1, -2)) / 2).astype(np.float32)


def check(api, oracle, a, lower=True, tag="", full=None):
    """Vectors and values-only against the oracle; `full` the symmetric
    matrices the read triangle stands for (default: a itself)."""
    n = a.shape[-1]
    s = a if full is None else full
    w, v, info = api.eigh(a, lower, True)
    wo, _, _ = oracle.eigh(s, lower, False)
    info = u32(info)
    assert not np.isnan(w).any() and not np.isnan(v).any()
    assert np.all((info >> 16) & 1) and not np.any((info >> 17) & 1)
    recon, ortho = eigh_residuals(symmetrize(s, lower), w, v)
    close = values_close(w, wo)
    print(f"[eigh_mid {tag} {a.shape} lower={lower}] recon {recon.max():.2e} ortho {ortho.max():.2e} "
          f"values {close.max():.2e} bound {bound(n):.2e}; bisection steps {np.mean(info & 0xFFFF):.1f}")
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert close.max() <= 1e-5
    assert np.all(np.diff(w, axis=-1) >= 0)
    w2, v2, info2 = api.eigh(a, lower, False)
    assert v2 is None
    assert values_close(w2, w).max() <= 1e-6
    assert np.array_equal(u32(info2) >> 16, info >> 16)
    return w, v, info


@pytest.mark.parametrize("n", [65, 71, 80, 96, 97, 100, 112, 127, 128])
@pytest.mark.parametrize("lower", [True, False])
def test_shapes_and_triangles(cuda, api, oracle, n, lower):
    a = sym(24, n, seed=n * 7 + lower)
    junk = a.copy()
    iu = np.triu_indices(n, 1) if lower else np.tril_indices(n, -1)
    junk[:, iu[0], iu[1]] = np.nan   # the unread triangle holds NaN
    check(api, oracle, junk, lower, "shape", full=a)


@pytest.mark.parametrize("n", [128, 100, 65])
def test_batch_1024(cuda, api, oracle, n):
    torch = cuda
    a = sym(1024, n, seed=1000 + n)
    w, v, info = api.eigh(dev(torch, a), True, True)
    torch.cuda.synchronize()
    w, v, info = to_np(w), to_np(v), u32(info)
    wh, vh, ih = api.eigh(a, True, True)   # host pointers: the pipelined path, the same bytes
    assert np.array_equal(w.view(np.uint32), wh.view(np.uint32)) and np.array_equal(v.view(np.uint32),
                                                                                     vh.view(np.uint32))
    assert np.array_equal(info, u32(ih))
    wo, _, _ = oracle.eigh(a, True, False)
    recon, ortho = eigh_residuals(a, w, v)
    close = values_close(w, wo)
    print(f"[eigh_mid batch 1024 n={n}] recon {recon.max():.2e} ortho {ortho.max():.2e} values {close.max():.2e}")
    assert recon.max() <= bound(n) and ortho.max() <= bound(n) and close.max() <= 1e-5
    assert np.all((info >> 16) & 1)


def with_spectrum(rng, spec):
    n = len(spec)
    q, r = np.linalg.qr(rng.standard_normal((n, n)))
    q = q * np.sign(np.diag(r))
    return ((q * spec) @ q.T).astype(np.float32)


@pytest.mark.parametrize("n", [65, 100, 128])
def test_structured_spectra(cuda, api, oracle, n):
    """Zero, identity, all-ones (rank one), repeated and clustered
    eigenvalues (large groups for the Gram-Schmidt rounds, across the two
    waves), graded, already diagonal, and the second-difference matrix."""
    rng = np.random.default_rng(n)
    mats = [np.zeros((n, n), np.float32), np.eye(n, dtype=np.float32), np.ones((n, n), np.float32),
            with_spectrum(rng, np.repeat([1.0, -2.0, 3.0, 0.5], (n + 3) // 4)[:n]),
            with_spectrum(rng, 1.0 + 1e-6 * np.arange(n)),
            with_spectrum(rng, 10.0 ** np.linspace(-6, 0, n)),
            np.diag(np.arange(n, dtype=np.float32) % 7),
            (np.diag(np.full(n, 2.0)) - np.diag(np.ones(n - 1), 1) - np.diag(np.ones(n - 1), -1)).astype(np.float32),
            (np.eye(n) + np.outer(np.ones(n), np.ones(n)) / n).astype(np.float32)]
    a = np.stack(mats)
    w, v, info = api.eigh(a, True, True)
    wo, _, _ = oracle.eigh(a, True, False)
    assert np.all((u32(info) >> 16) & 1)
    recon, ortho = eigh_residuals(a, w, v)
    recon[0] = 0.0 if np.abs(w[0]).max() == 0 else recon[0]
    print(f"[eigh_mid structured n={n}] recon {np.array2string(recon, precision=2)} ortho "
          f"{np.array2string(ortho, precision=2)}")
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert values_close(w, wo).max() <= 1e-5
    assert np.abs(w[2, -1] - n) <= 1e-5 * n and np.abs(w[2, :-1]).max() <= 1e-5 * n


@pytest.mark.parametrize("n", [80, 128])
def test_magnitudes(cuda, api, oracle, n):
    s = sym(6, n, seed=23 + n)
    scales = np.array([1e-30, 1e-20, 1e-5, 1e5, 1e20, 1e37], np.float32)
    a = (s.astype(np.float64) * scales[:, None, None]).astype(np.float32)
    w, v, _ = api.eigh(a, True, True)
    wo, _, _ = oracle.eigh(a, True, False)
    recon, ortho = eigh_residuals(a, w, v)
    assert recon.max() <= bound(n) and ortho.max() <= bound(n)
    assert values_close(w, wo).max() <= 1e-5


@pytest.mark.parametrize("n", [65, 128])
def test_nonfinite_isolation(cuda, api, n):
    a = sym(8, n, seed=5 + n)
    clean_w, clean_v, clean_i = api.eigh(a, True, True)
    a[1, n - 1, 0] = np.nan      # read (lower)
    a[3, 10, 3] = np.inf         # read
    a[4, 5, 5] = -np.inf         # read, diagonal
    a[6, 3, 10] = np.inf         # unread (upper): ignored
    w, v, info = api.eigh(a, True, True)
    info = u32(info)
    for b in (1, 3, 4):
        assert (w[b].view(np.uint32) == 0x7FC00000).all() and (v[b].view(np.uint32) == 0x7FC00000).all()
        assert info[b] == (1 << 17)
    for b in (0, 2, 5, 6, 7):
        assert np.array_equal(w[b].view(np.uint32), clean_w[b].view(np.uint32))
        assert np.array_equal(v[b].view(np.uint32), clean_v[b].view(np.uint32))
        assert info[b] == u32(clean_i)[b]


def test_batch_position_and_chunking(cuda, api):
    """A matrix's eigenpairs are bit-identical wherever it sits in the batch
    and whatever the batch size."""
    torch = cuda
    a = sym(200, 90, seed=12)
    w1, v1, i1 = (to_np(x) for x in api.eigh(dev(torch, a)))
    w2, v2, i2 = (to_np(x) for x in api.eigh(dev(torch, a[::-1].copy())))
    assert np.array_equal(w1.view(np.uint32), w2[::-1].view(np.uint32))
    assert np.array_equal(v1.view(np.uint32), v2[::-1].view(np.uint32))
    assert np.array_equal(i1, i2[::-1])
    w3, v3, _ = api.eigh(a[77:78])
    assert np.array_equal(w3[0].view(np.uint32), w1[77].view(np.uint32))
    assert np.array_equal(v3[0].view(np.uint32), v1[77].view(np.uint32))
