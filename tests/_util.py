"""Shared test helpers: seeded inputs for the five BASELINE configs and the
sign- and order-invariant parity measures, all evaluated in float64.

Inputs come from numpy's PCG64 generator with the seeds fixed here; the GPU
path and the oracle always read the same float32 bytes.  The bounds are the
north star's: reconstruction and orthogonality <= 50 * n * eps_f32, values
within 1e-5 of the largest.
"""

from __future__ import annotations

import numpy as np

EPS32 = float(np.finfo(np.float32).eps)


def bound(n: int) -> float:
    """50 * n * eps_f32, the north star's residual bound for size n."""
    return 50.0 * n * EPS32


def gaussian(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def to_np(x):
    if x is None:
        return None
    if type(x).__module__.startswith("torch"):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def u32(x):
    """An info/pivot array (uint32, or int32 from torch) as uint32."""
    x = to_np(x)
    return x.view(np.uint32) if x.dtype == np.int32 else x.astype(np.uint32)


# ---- configs ----

def config1_qr(batch=10000, n=32, seed=1):
    return gaussian((batch, n, n), seed)


def config2_eigh(batch=4096, n=64, seed=2, nan_index=7):
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((batch, n, n))
    s = (g + np.swapaxes(g, -1, -2)) / 2
    picks = rng.choice(batch, size=max(1, batch // 10), replace=False)
    ks = rng.uniform(-30, 37, size=picks.size)
    s[picks] *= (10.0 ** ks)[:, None, None]
    s = s.astype(np.float32)
    if nan_index is not None and nan_index < batch:
        s[nan_index] = np.nan
    return s


def random_orthogonal(rng, m, n):
    q, r = np.linalg.qr(rng.standard_normal((m, n)))
    return q * np.sign(np.diag(r))


def config3_svd(batch=2048, m=128, n=64, seed=3):
    rng = np.random.default_rng(seed)
    a = np.empty((batch, m, n), np.float64)
    deficient = set(rng.choice(batch, size=batch // 4, replace=False).tolist())
    for b in range(batch):
        u = random_orthogonal(rng, m, n)
        v = random_orthogonal(rng, n, n)
        s = np.sort(10.0 ** rng.uniform(-6, 0, size=n))[::-1].copy()
        if b in deficient:
            s[-16:] = 0.0
        a[b] = (u * s) @ v.T
    return a.astype(np.float32)


def config4_spd(batch=8192, n=16, seed=4):
    rng = np.random.default_rng(seed)
    bm = rng.standard_normal((batch, n, n)).astype(np.float32)
    a = (bm @ np.swapaxes(bm, -1, -2) + n * np.eye(n, dtype=np.float32)).astype(np.float32)
    bad = rng.choice(batch, size=max(1, batch // 100), replace=False)
    a[bad, n - 1, n - 1] = -a[bad, n - 1, n - 1]
    return a, np.sort(bad)


def config4_lu(batch=8192, n=16, nrhs=4, seed=5):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((batch, n, n)).astype(np.float32)
    b = rng.standard_normal((batch, n, nrhs)).astype(np.float32)
    return a, b


# ---- invariants (float64), one value per matrix ----

def fro(x, axes=(-2, -1)):
    return np.sqrt(np.sum(np.square(x, dtype=np.float64), axis=axes))


def rel_recon(a, approx):
    a = a.astype(np.float64)
    d = fro(a - approx)
    nrm = fro(a)
    return np.where(nrm > 0, d / np.where(nrm > 0, nrm, 1), d)


def orthogonality(q):
    """||Q^T Q - I||_F per matrix (columns of Q)."""
    q = q.astype(np.float64)
    k = q.shape[-1]
    g = np.swapaxes(q, -1, -2) @ q
    return fro(g - np.eye(k))


def qr_residuals(a, q, r):
    return rel_recon(a, q.astype(np.float64) @ r.astype(np.float64)), orthogonality(q)


def eigh_residuals(a, w, v):
    recon = (v.astype(np.float64) * w.astype(np.float64)[..., None, :]) @ np.swapaxes(v.astype(np.float64), -1, -2)
    return rel_recon(a, recon), orthogonality(v)


def svd_residuals(a, u, s, vt):
    recon = (u.astype(np.float64) * s.astype(np.float64)[..., None, :]) @ vt.astype(np.float64)
    return rel_recon(a, recon), orthogonality(u), orthogonality(np.swapaxes(vt, -1, -2))


def values_close(x, ref, rel=1e-5):
    """max |x - ref| / max|ref| per matrix (value lists already sorted alike)."""
    x = x.astype(np.float64)
    ref = ref.astype(np.float64)
    scale = np.max(np.abs(ref), axis=-1)
    d = np.max(np.abs(x - ref), axis=-1)
    return np.where(scale > 0, d / np.where(scale > 0, scale, 1), d)


def symmetrize(a, lower=True):
    """The symmetric matrix a routine reading one triangle sees."""
    a = a.astype(np.float64)
    t = np.tril(a) if lower else np.triu(a)
    d = np.tril(np.triu(a))
    return t + np.swapaxes(t, -1, -2) - d


def lu_unpack(lu, piv):
    """(P, L, U) with P A = L U from packed LU and 0-based sequential swaps."""
    lu = lu.astype(np.float64)
    n = lu.shape[-1]
    L = np.tril(lu, -1) + np.eye(n)
    U = np.triu(lu)
    batch_shape = lu.shape[:-2]
    perm = np.broadcast_to(np.arange(n), batch_shape + (n,)).copy()
    piv = u32(piv).astype(np.int64)
    flat_perm = perm.reshape(-1, n)
    flat_piv = piv.reshape(-1, n)
    for b in range(flat_perm.shape[0]):
        p = flat_perm[b]
        for i in range(n):
            j = flat_piv[b, i]
            p[i], p[j] = p[j], p[i]
    return flat_perm.reshape(batch_shape + (n,)), L, U


def lu_residual(a, lu, piv):
    perm, L, U = lu_unpack(lu, piv)
    pa = np.take_along_axis(a.astype(np.float64), perm[..., :, None], axis=-2)
    return rel_recon(pa, L @ U)


def config5_matrix(n=4096, seed=6):
    """G, iid N(0,1), the single large matrix of config 5."""
    return gaussian((n, n), seed)


def config5_spd(g):
    """G G^T / n + I, in float64, rounded to float32."""
    n = g.shape[0]
    g64 = g.astype(np.float64)
    return (g64 @ g64.T / n + np.eye(n)).astype(np.float32)


def near_tie(a, piv_x, piv_y, rel=1e-4):
    """True when the first step at which two partial-pivoting sequences part
    is a near-tie of column magnitudes: elimination in float64 along piv_y
    up to that step, then |a[piv_x[k], k]| and |a[piv_y[k], k]| within rel
    of each other (a NaN or an infinity never ties)."""
    a = a.astype(np.float64).copy()
    with np.errstate(all="ignore"):
        for k in range(a.shape[0]):
            if piv_x[k] != piv_y[k]:
                m1, m2 = abs(a[piv_x[k], k]), abs(a[piv_y[k], k])
                return bool(np.isfinite(m1) and np.isfinite(m2) and abs(m1 - m2) <= rel * max(m1, m2))
            p = piv_y[k]
            a[[k, p]] = a[[p, k]]
            if a[k, k] != 0:
                a[k + 1:, k] /= a[k, k]
            a[k + 1:, k + 1:] -= np.outer(a[k + 1:, k], a[k, k + 1:])
    return True


def first_difference(piv_x, piv_y):
    d = np.nonzero(np.asarray(piv_x) != np.asarray(piv_y))[0]
    return int(d[0]) if d.size else -1
