"""Parity of the batched mid-size QR (m, n <= 128 with one of them above 64:
two waves per matrix, a column per thread) on the GPU, through the C ABI,
against the oracle on identical seeded inputs.

The reference factors such batches with one threadgroup per matrix
(shaders/QR_Householder.metal:665-847, any number of columns up to 4096
rows); before this kernel the build ran them one matrix at a time through
the blocked path.  Comparisons are sign-invariant: reconstruction and
orthogonality within the north star's 50 max(m, n) eps_f32, R within 1e-4 of
the oracle's (relative to its largest entry) once the row signs agree, R
exactly upper triangular, and a matrix holding a NaN or an infinity written
as all quiet NaN 0x7FC00000 without touching its neighbours.  Wide matrices
(m < n) give Q m x m and R m x n."""

import numpy as np
import pytest

from _util import bound, gaussian, qr_residuals, to_np

pytestmark = pytest.mark.gpu

QNAN = 0x7FC00000


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def r_matches_oracle(r, ro):
    """max over matrices of max |D R - R_o| / max |R_o|, D the row signs."""
    k = min(r.shape[-2:])
    sgn = np.sign(np.diagonal(r[..., :k, :k], axis1=-2, axis2=-1).astype(np.float64) *
                  np.diagonal(ro[..., :k, :k], axis1=-2, axis2=-1))
    sgn[sgn == 0] = 1
    diff = np.abs(r.astype(np.float64) * sgn[..., None] - ro).max(axis=(-2, -1))
    return float((diff / np.maximum(np.abs(ro).max(axis=(-2, -1)), 1e-30)).max())


def check(api, oracle, a, mode, tag):
    m, n = a.shape[-2:]
    k = min(m, n)
    q, r = api.qr(a, mode)
    qo, ro = oracle.qr(a, mode)
    assert r.shape == ro.shape == a.shape[:-2] + (k, n)
    assert np.all(np.tril(r, -1) == 0) and not np.isnan(r).any()
    rdiff = r_matches_oracle(r, ro)
    msg = f"[qr_mid {tag} {a.shape} {mode}] R vs oracle {rdiff:.2e}"
    if q is not None:
        assert q.shape == a.shape[:-2] + (m, k)
        recon, ortho = qr_residuals(a, q, r)
        msg += f" recon {recon.max():.2e} ortho {ortho.max():.2e} bound {bound(max(m, n)):.2e}"
        print(msg)
        assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(max(m, n))
    else:
        assert qo is None
        print(msg)
    assert rdiff <= 1e-4
    return q, r


@pytest.mark.parametrize("m,n", [(65, 65), (128, 128), (128, 65), (100, 97), (127, 80), (70, 33), (128, 1),
                                 (65, 128), (80, 100), (1, 128), (33, 70), (128, 127)])
@pytest.mark.parametrize("mode", ["reduced", "r"])
def test_shapes_and_modes(cuda, api, oracle, m, n, mode):
    check(api, oracle, gaussian((5, m, n), seed=m * 7 + n), mode, "shape")


@pytest.mark.parametrize("m,n", [(128, 128), (128, 96), (96, 128)])
def test_batch_1024(cuda, api, oracle, m, n):
    """A batch the kernel exists for, device pointers, with the host-pointer
    (pipelined) path giving the same bytes."""
    torch = cuda
    a = gaussian((1024, m, n), seed=m + 3 * n)
    q, r = api.qr(dev(torch, a), "reduced")
    torch.cuda.synchronize()
    q, r = to_np(q), to_np(r)
    qh, rh = api.qr(a, "reduced")
    assert np.array_equal(q.view(np.uint32), qh.view(np.uint32)) and np.array_equal(r.view(np.uint32),
                                                                                     rh.view(np.uint32))
    qo, ro = oracle.qr(a, "reduced")
    recon, ortho = qr_residuals(a, q, r)
    rdiff = r_matches_oracle(r, ro)
    print(f"[qr_mid batch 1024 {m}x{n}] recon {recon.max():.2e} ortho {ortho.max():.2e} R vs oracle {rdiff:.2e}")
    assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(max(m, n)) and rdiff <= 1e-4


@pytest.mark.parametrize("m,n", [(128, 128), (100, 70), (70, 100)])
def test_complete_when_wide_or_square(cuda, api, oracle, m, n):
    """complete mode where Q is m x min(m, n) anyway (m <= n): the same kernel."""
    if m > n:
        pytest.skip("complete Q of a tall matrix is m x m: the blocked path")
    check(api, oracle, gaussian((3, m, n), seed=5 * m + n), "complete", "complete")


@pytest.mark.parametrize("m,n", [(128, 128), (100, 80), (80, 100)])
def test_nonfinite_isolation(cuda, api, m, n):
    a = gaussian((6, m, n), seed=m * 3 + n)
    qc, rc = api.qr(a, "reduced")
    a[1, 0, 0] = np.nan
    a[3, m - 1, n - 1] = np.inf
    a[4, m // 2, 3] = -np.inf
    q, r = api.qr(a, "reduced")
    for b in (1, 3, 4):
        assert (q[b].view(np.uint32) == QNAN).all() and (r[b].view(np.uint32) == QNAN).all()
    for b in (0, 2, 5):
        assert np.array_equal(q[b].view(np.uint32), qc[b].view(np.uint32))
        assert np.array_equal(r[b].view(np.uint32), rc[b].view(np.uint32))


@pytest.mark.parametrize("m,n", [(128, 128), (100, 80)])
def test_structured_inputs(cuda, api, oracle, m, n):
    """Zero (Q = I's first columns, R = 0), a zero column, rank one, graded
    columns, and 1e-30 / 1e30 scalings (a power of two taken out inside)."""
    rng = np.random.default_rng(m + n)
    k = min(m, n)
    zero = np.zeros((m, n), np.float32)
    zcol = rng.standard_normal((m, n)).astype(np.float32)
    zcol[:, 3] = 0.0
    rank1 = np.outer(rng.standard_normal(m), rng.standard_normal(n)).astype(np.float32)
    graded = (rng.standard_normal((m, n)) * 10.0 ** np.linspace(0, -6, n)[None, :]).astype(np.float32)
    tiny = (rng.standard_normal((m, n)) * 1e-30).astype(np.float32)
    huge = (rng.standard_normal((m, n)) * 1e30).astype(np.float32)
    a = np.stack([zero, zcol, rank1, graded, tiny, huge])
    q, r = api.qr(a, "reduced")
    assert np.array_equal(q[0], np.eye(m, k, dtype=np.float32)) and np.all(r[0] == 0)
    recon, ortho = qr_residuals(a[1:], q[1:], r[1:])
    print(f"[qr_mid structured {m}x{n}] recon {np.array2string(recon, precision=2)} "
          f"ortho {np.array2string(ortho, precision=2)}")
    assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(max(m, n))
    _, ro = oracle.qr(a[[1, 3, 4, 5]], "reduced")
    assert r_matches_oracle(r[[1, 3, 4, 5]], ro) <= 1e-4


def test_batch_position(cuda, api):
    torch = cuda
    a = gaussian((100, 110, 90), seed=41)
    q1, r1 = [to_np(x) for x in api.qr(dev(torch, a), "reduced")]
    q2, r2 = [to_np(x) for x in api.qr(dev(torch, a[::-1].copy()), "reduced")]
    assert np.array_equal(q1.view(np.uint32), q2[::-1].view(np.uint32))
    assert np.array_equal(r1.view(np.uint32), r2[::-1].view(np.uint32))
