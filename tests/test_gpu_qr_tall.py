"""Parity of the batched tall QR (n <= 64 columns, 65 rows and beyond) on
the GPU, through the C ABI, against the oracle on identical seeded inputs.

The reference factors such batches with one threadgroup per matrix
(shaders/QR_Householder.metal:665-847, up to 4096 rows); this build uses one
wave per block of up to 128 rows and a reduction tree of block QRs beyond.
Comparisons are sign-invariant (QR is unique up to the signs of R's rows for
a full-rank matrix): reconstruction and orthogonality within the north star's
50 max(m, n) eps_f32, R within 1e-4 of the oracle's (relative to its largest
entry) once the row signs agree, R exactly upper triangular, and a matrix
holding a NaN or an infinity written as all quiet NaN 0x7FC00000 without
touching its neighbours.  The batch >= 1024 cases are the mid-size batched
windows (65-128 rows, and 1000 rows) the kernel exists for."""

import numpy as np
import pytest

from _util import bound, gaussian, orthogonality, qr_residuals, rel_recon, to_np

pytestmark = pytest.mark.gpu

QNAN = 0x7FC00000


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def r_matches_oracle(r, ro):
    """max over matrices of max |R D - R_o| / max |R_o|, D the row signs."""
    k = r.shape[-1]
    sgn = np.sign(np.diagonal(r[..., :k, :k], axis1=-2, axis2=-1) * np.diagonal(ro[..., :k, :k], axis1=-2, axis2=-1))
    sgn[sgn == 0] = 1
    diff = np.abs(r[..., :k, :].astype(np.float64) * sgn[..., None] - ro[..., :k, :]).max(axis=(-2, -1))
    return float((diff / np.maximum(np.abs(ro).max(axis=(-2, -1)), 1e-30)).max())


def check_against_oracle(api, oracle, a, mode, tag):
    m, n = a.shape[-2:]
    q, r = api.qr(a, mode)
    qo, ro = oracle.qr(a, mode)
    assert r.shape == ro.shape == a.shape[:-2] + (n, n)
    assert np.all(np.tril(r, -1) == 0)
    assert not np.isnan(r).any()
    rdiff = r_matches_oracle(r, ro)
    msg = f"[qr_tall {tag} {a.shape} {mode}] R vs oracle {rdiff:.2e}"
    if q is not None:
        assert q.shape == a.shape
        recon, ortho = qr_residuals(a, q, r)
        msg += f" recon {recon.max():.2e} ortho {ortho.max():.2e} bound {bound(max(m, n)):.2e}"
        print(msg)
        assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(max(m, n))
    else:
        assert qo is None
        print(msg)
    assert rdiff <= 1e-4
    return q, r


@pytest.mark.parametrize("m,n", [(65, 1), (65, 64), (66, 64), (100, 40), (127, 5), (128, 64), (128, 1),
                                 (129, 64), (129, 1), (200, 7), (257, 33), (300, 64), (1000, 20), (4096, 64),
                                 (5000, 3), (8320, 64)])
@pytest.mark.parametrize("mode", ["reduced", "r"])
def test_shapes_and_modes(cuda, api, oracle, m, n, mode):
    batch = 33 if m * n <= 300 * 64 else 5
    a = gaussian((batch, m, n), seed=m * 977 + n)
    check_against_oracle(api, oracle, a, mode, "shape")


@pytest.mark.parametrize("m,n", [(128, 64), (100, 40), (65, 32), (1000, 20)])
def test_batch_1024(cuda, api, oracle, m, n):
    a = gaussian((1024, m, n), seed=m + 31 * n)
    torch = cuda
    q, r = api.qr(dev(torch, a))
    torch.cuda.synchronize()
    q, r = to_np(q), to_np(r)
    qh, rh = api.qr(a)   # host pointers: the pipelined path, the same bytes
    assert np.array_equal(q, qh) and np.array_equal(r, rh)
    recon, ortho = qr_residuals(a, q, r)
    qo, ro = oracle.qr(a)
    rdiff = r_matches_oracle(r, ro)
    print(f"[qr_tall batch 1024 {m}x{n}] recon {recon.max():.2e} ortho {ortho.max():.2e} R vs oracle {rdiff:.2e}")
    assert recon.max() <= bound(max(m, n)) and ortho.max() <= bound(max(m, n))
    assert rdiff <= 1e-4 and np.all(np.tril(r, -1) == 0)


def test_4096_rows_batch_1024(cuda, api, oracle):
    """The reference's largest batched QR shape, 4096 x 64, at batch 1024:
    residuals on the GPU in float64 for the whole batch, R against the
    oracle for a sample of 16 matrices."""
    torch = cuda
    m, n, batch = 4096, 64, 1024
    g = torch.Generator(device="cuda").manual_seed(4096)
    a = torch.randn((batch, m, n), device="cuda", generator=g, dtype=torch.float32)
    q, r = api.qr(a)
    torch.cuda.synchronize()
    assert not torch.isnan(q).any() and not torch.isnan(r).any()
    assert bool((torch.tril(r, -1) == 0).all())
    recon = torch.empty(batch, dtype=torch.float64, device="cuda")
    ortho = torch.empty(batch, dtype=torch.float64, device="cuda")
    eye = torch.eye(n, dtype=torch.float64, device="cuda")
    for b0 in range(0, batch, 128):
        ad, qd, rd = (t[b0:b0 + 128].double() for t in (a, q, r))
        recon[b0:b0 + 128] = torch.linalg.norm(ad - qd @ rd, dim=(-2, -1)) / torch.linalg.norm(ad, dim=(-2, -1))
        ortho[b0:b0 + 128] = torch.linalg.norm(qd.transpose(-1, -2) @ qd - eye, dim=(-2, -1))
    print(f"[qr_tall 4096x64 batch 1024] recon {recon.max().item():.2e} ortho {ortho.max().item():.2e}")
    assert recon.max().item() <= bound(m) and ortho.max().item() <= bound(m)
    pick = list(range(0, batch, 64))
    sample = to_np(a[pick])
    qo, ro = oracle.qr(sample)
    assert r_matches_oracle(to_np(r[pick]), ro) <= 1e-4


@pytest.mark.parametrize("m,n,where", [(100, 40, (99, 39)), (128, 64, (0, 0)), (300, 64, (150, 3)),
                                       (4096, 16, (4095, 15)), (4096, 16, (0, 7)), (1000, 20, (640, 0))])
def test_nonfinite_isolation(cuda, api, m, n, where):
    a = gaussian((6, m, n), seed=m + n)
    clean_q, clean_r = api.qr(a)
    a[1][where] = np.nan
    a[3][where] = np.inf
    a[4][where] = -np.inf
    q, r = api.qr(a)
    for b in (1, 3, 4):
        assert (q[b].view(np.uint32) == QNAN).all() and (r[b].view(np.uint32) == QNAN).all()
        qr_only = api.qr(a[b:b + 1], "r")[1]
        assert (qr_only.view(np.uint32) == QNAN).all()
    for b in (0, 2, 5):   # neighbours unchanged, bit for bit
        assert np.array_equal(q[b], clean_q[b]) and np.array_equal(r[b], clean_r[b])


@pytest.mark.parametrize("m", [100, 300, 4096])
def test_structured_inputs(cuda, api, m):
    """Zero, rank-one, repeated-column and extreme-magnitude matrices: Q stays
    orthonormal (every block of the tree has at least n rows, so its Q is
    orthonormal whatever the rank), A = Q R."""
    n = 16
    rng = np.random.default_rng(m)
    z = np.zeros((m, n), np.float32)
    rank1 = np.outer(rng.standard_normal(m), rng.standard_normal(n)).astype(np.float32)
    rep = rng.standard_normal((m, n)).astype(np.float32)
    rep[:, 8:] = rep[:, :8]
    tiny = gaussian((m, n), seed=1, scale=1e-30)
    huge = gaussian((m, n), seed=2, scale=1e30)
    sub = gaussian((m, n), seed=3, scale=1e-38)
    eye = np.zeros((m, n), np.float32)
    eye[np.arange(n), np.arange(n)] = 1.0
    bottom = np.zeros((m, n), np.float32)   # all mass in the last rows (the tree's last block)
    bottom[-n:] = rng.standard_normal((n, n))
    a = np.stack([z, rank1, rep, tiny, huge, sub, eye, bottom])
    q, r = api.qr(a)
    assert not np.isnan(q).any() and not np.isnan(r).any()
    ortho = orthogonality(q)
    recon = rel_recon(a, q.astype(np.float64) @ r.astype(np.float64))
    print(f"[qr_tall structured m={m}] ortho {np.array2string(ortho, precision=2)} recon "
          f"{np.array2string(recon, precision=2)}")
    assert ortho.max() <= bound(m)
    assert recon[1:].max() <= bound(m)
    assert np.all(r[0] == 0)
    assert np.all(np.tril(r, -1) == 0)


def test_batch_position_and_host_device(cuda, api):
    """A matrix's result does not depend on its position in the batch or on
    the batch size, nor on whether the pointers are host or device memory."""
    torch = cuda
    a = gaussian((50, 700, 24), seed=5)
    q, r = api.qr(a)
    q1, r1 = api.qr(a[17:18])
    assert np.array_equal(q[17], q1[0]) and np.array_equal(r[17], r1[0])
    qd, rd = api.qr(dev(torch, a))
    assert np.array_equal(q, to_np(qd)) and np.array_equal(r, to_np(rd))


@pytest.mark.parametrize("m,n", [(5000, 20), (20, 5000), (1000, 64)])
def test_tall_svd_beyond_4096_rows(cuda, api, oracle, m, n):
    """SVD of tall matrices past the batched kernel: A = Q R by the tall QR,
    then the SVD of R; 5000 rows, past the blocked QR's 4096, now fit."""
    from _util import svd_residuals, values_close

    a = gaussian((4, m, n), seed=m * 3 + n)
    u, s, vt, info = api.svd(a)
    _, so, _, _ = oracle.svd(a)
    recon, ou, ov = svd_residuals(a, u, s, vt)
    print(f"[svd tall {m}x{n}] recon {recon.max():.2e} ortho {ou.max():.2e}/{ov.max():.2e} "
          f"s vs oracle {values_close(s, so).max():.2e}")
    assert recon.max() <= bound(max(m, n)) and ou.max() <= bound(max(m, n)) and ov.max() <= bound(max(m, n))
    assert values_close(s, so).max() <= 1e-5
