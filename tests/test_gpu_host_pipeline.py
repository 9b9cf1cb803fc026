"""Host pointers through the pipelined path: a batch of host (numpy)
buffers runs in chunks through pinned staging, the transfers of one chunk
overlapping the kernels of another.  Results must be bit-identical to the
same call on device buffers (the same kernels on the same matrices; no
result depends on a matrix's position in the batch), including info words
and NaN outputs, across many chunks and a partial last chunk."""

import numpy as np
import pytest

from _util import config1_qr, config2_eigh, config4_lu, config4_spd, to_np, u32

pytestmark = pytest.mark.gpu


def dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def same(x, y):
    x, y = to_np(x), to_np(y)
    return x.shape == y.shape and np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_eigh_host_matches_device(cuda, api):
    a = config2_eigh(batch=3001, n=64, seed=31)   # ~9 chunks of ~500, the last partial
    wh, vh, ih = api.eigh(a)
    wd, vd, idv = api.eigh(dev(cuda, a))
    assert same(wh, wd) and same(vh, vd) and np.array_equal(u32(ih), u32(idv))


def test_qr_host_matches_device(cuda, api):
    a = config1_qr(batch=7777, seed=32)
    for mode in ("reduced", "r"):
        qh, rh = api.qr(a, mode)
        qd, rd = api.qr(dev(cuda, a), mode)
        assert same(rh, rd) and (qh is None or same(qh, qd))


def test_small_family_host_matches_device(cuda, api):
    a, _ = config4_spd(batch=9000, seed=33)
    lh, ih = api.cholesky(a)
    ld, idv = api.cholesky(dev(cuda, a))
    assert same(lh, ld) and np.array_equal(u32(ih), u32(idv))
    g, b = config4_lu(batch=9000, seed=34)
    luh, ph, ih = api.lu_factor(g)
    lud, pd, idv = api.lu_factor(dev(cuda, g))
    assert same(luh, lud) and np.array_equal(u32(ph), u32(pd)) and np.array_equal(u32(ih), u32(idv))
    xh, _ = api.solve(g, b)
    xd, _ = api.solve(dev(cuda, g), dev(cuda, b))
    assert same(xh, xd)
    vh, _ = api.inv(g)
    vd, _ = api.inv(dev(cuda, g))
    assert same(vh, vd)
    th = api.solve_triangular(g, b, True, False)
    td = api.solve_triangular(dev(cuda, g), dev(cuda, b), True, False)
    assert same(th, td)


def test_svd_host_matches_device_and_mixed_pointers(cuda, api, lib):
    from _util import config3_svd

    a = config3_svd(batch=700, seed=35)
    uh, sh, vh, ih = api.svd(a)
    ud, sd, vd, idv = api.svd(dev(cuda, a))
    assert same(uh, ud) and same(sh, sd) and same(vh, vd) and np.array_equal(u32(ih), u32(idv))
    # input on the device, outputs in host memory: the device slice is read
    # in place per chunk, the host ones staged
    s = np.empty((700, 64), np.float32)
    info = np.empty(700, np.uint32)
    ta = dev(cuda, a)
    with lib.lock:
        rc = lib.svd(ta.data_ptr(), 700, 128, 64, None, s.ctypes.data, None, info.ctypes.data)
    assert rc == lib.OK
    _, s2, _, i2 = api.svd(ta, vectors=False)
    assert same(s, s2) and np.array_equal(info, u32(i2))


def test_pinned_host_buffers(cuda, api):
    """Pinned host tensors in and out: the transfers read and write the
    caller's buffers directly (no staging copy); same bits as on device."""
    a = config2_eigh(batch=1500, n=64, seed=36)
    pa = cuda.from_numpy(a).pin_memory()
    wp, vp, ip = api.eigh(pa)
    assert wp.is_pinned() and vp.is_pinned()
    wd, vd, idv = api.eigh(dev(cuda, a))
    assert same(wp, wd) and same(vp, vd) and np.array_equal(u32(ip), u32(idv))
    g, b = config4_lu(batch=5000, seed=37)
    xp, _ = api.solve(cuda.from_numpy(g).pin_memory(), cuda.from_numpy(b))   # b pinned by the call
    xd, _ = api.solve(dev(cuda, g), dev(cuda, b))
    assert same(xp, xd)


def test_pinned_host_buffers_many_chunks(cuda, api):
    """Every host buffer pinned: all chunks are queued at once over four
    device slots, each reused once its previous chunk's download is done.
    Ten chunks (QR, ~2730 matrices each) and six (eigh, 1024 each), the last
    partial: same bits as the device call."""
    a = config1_qr(batch=25001, seed=38)
    qp, rp = api.qr(cuda.from_numpy(a).pin_memory())
    assert qp.is_pinned() and rp.is_pinned()
    qd, rd = api.qr(dev(cuda, a))
    assert same(qp, qd) and same(rp, rd)
    e = config2_eigh(batch=5500, n=64, seed=39)
    wp, vp, ip = api.eigh(cuda.from_numpy(e).pin_memory())
    wd, vd, idv = api.eigh(dev(cuda, e))
    assert same(wp, wd) and same(vp, vd) and np.array_equal(u32(ip), u32(idv))
