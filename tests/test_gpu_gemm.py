"""The fp32 MFMA GEMM the blocked factorisations build on, against a float64
product: every transpose combination, ragged edges, strided batches,
alpha/beta.  Bound per element: 2 K eps (|A||B|)_ij + eps |beta C_ij|.
Products with K <= 128 on a small grid run the 64 x 64 whole-K kernel
(every case here with K <= 128 except 2900 x 2900 x 64, which has enough
128 x 128 tiles to stay on the main kernel)."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run(lib, ta, tb, a, b, c, alpha, beta, batch=1):
    m = c.shape[-2]
    n = c.shape[-1]
    k = a.shape[-2] if ta else a.shape[-1]
    lda, ldb, ldc = a.shape[-1], b.shape[-1], c.shape[-1]
    sa = a.shape[-2] * a.shape[-1] if a.ndim == 3 else 0
    sb = b.shape[-2] * b.shape[-1] if b.ndim == 3 else 0
    sc = m * n
    rc = lib.hip_sgemm(int(ta), int(tb), m, n, k, alpha, a.ctypes.data, lda, sa, b.ctypes.data, ldb, sb, beta,
                       c.ctypes.data, ldc, sc, batch)
    assert rc == 0, lib.last_error()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (128, 128, 16), (130, 70, 33), (257, 384, 100), (64, 513, 7),
                                   (600, 200, 257), (200, 300, 128), (2900, 2900, 64)])
def test_gemm(cuda, lib, ta, tb, m, n, k):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    batch = 2
    a = rng.standard_normal((batch, k, m) if ta else (batch, m, k)).astype(np.float32)
    b = rng.standard_normal((batch, n, k) if tb else (batch, k, n)).astype(np.float32)
    c = rng.standard_normal((batch, m, n)).astype(np.float32)
    alpha, beta = np.float32(-1.5), np.float32(0.5)
    opa = np.swapaxes(a, -1, -2) if ta else a
    opb = np.swapaxes(b, -1, -2) if tb else b
    ref = alpha * (opa.astype(np.float64) @ opb) + beta * c.astype(np.float64)
    mag = np.abs(alpha) * (np.abs(opa).astype(np.float64) @ np.abs(opb)) + np.abs(beta * c)
    out = c.copy()
    run(lib, ta, tb, a, b, out, alpha, beta, batch)
    eps = np.finfo(np.float32).eps
    assert np.all(np.abs(out - ref) <= 2 * (k + 2) * eps * mag + 1e-30)


def test_gemm_beta_zero_ignores_c(cuda, lib):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((70, 40)).astype(np.float32)
    b = rng.standard_normal((40, 90)).astype(np.float32)
    c = np.full((70, 90), np.nan, np.float32)
    run(lib, False, False, a, b, c, np.float32(1), np.float32(0))
    assert np.abs(c - a.astype(np.float64) @ b).max() <= 1e-4


@pytest.mark.parametrize("m", [100, 2000])
def test_gemm_in_place(cuda, lib, m):
    """C = A X^T written over A (device memory, as the blocked Cholesky's
    L21 = A21 X^T): every row of A is read whole before it is overwritten."""
    torch = cuda
    rng = np.random.default_rng(m)
    a = rng.standard_normal((m, 128)).astype(np.float32)
    x = rng.standard_normal((128, 128)).astype(np.float32)
    ref = a.astype(np.float64) @ x.astype(np.float64).T
    ad = torch.from_numpy(a).to("cuda")
    xd = torch.from_numpy(x).to("cuda")
    rc = lib.hip_sgemm(0, 1, m, 128, 128, np.float32(1), ad.data_ptr(), 128, 0, xd.data_ptr(), 128, 0,
                       np.float32(0), ad.data_ptr(), 128, 0, 1)
    assert rc == 0, lib.last_error()
    torch.cuda.synchronize()
    out = ad.cpu().numpy()
    mag = np.abs(a).astype(np.float64) @ np.abs(x).T
    eps = np.finfo(np.float32).eps
    assert np.all(np.abs(out - ref) <= 2 * 130 * eps * mag)
