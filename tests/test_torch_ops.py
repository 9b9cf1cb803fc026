"""The torch custom operators (torch.ops.metal_linalg.*, the reference's
python-torch binding): registration and fake shapes on the CPU; on the GPU,
forward parity with the C-ABI calls and gradients against torch.linalg's own
autograd in float64 on the CPU (losses invariant to the eigen/singular vector
signs, so that the comparison is well defined)."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import metal_linalg_amd.torch_ops  # noqa: F401  (registers the operators)
from metal_linalg_amd import api
from _util import to_np

ops = torch.ops.metal_linalg


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = torch.empty(3, 10, 6)
        s = torch.empty(2, 5, 5)
        b = torch.empty(2, 5, 3)
        assert [t.shape for t in ops.qr(a)] == [(3, 10, 6), (3, 6, 6)]
        assert [t.shape for t in ops.qr(a, "complete")] == [(3, 10, 10), (3, 10, 6)]
        assert [t.shape for t in ops.eigh(s)] == [(2, 5), (2, 5, 5)]
        assert ops.eigvalsh(s).shape == (2, 5)
        assert [t.shape for t in ops.svd(a)] == [(3, 10, 6), (3, 6), (3, 6, 6)]
        assert ops.svdvals(a).shape == (3, 6)
        l, info = ops.cholesky(s)
        assert l.shape == (2, 5, 5) and info.shape == (2,) and info.dtype == torch.int32
        assert [t.shape for t in ops.lu_factor(s)] == [(2, 5, 5), (2, 5), (2,)]
        assert ops.solve(s, b)[0].shape == (2, 5, 3)
        assert ops.inv(s)[0].shape == (2, 5, 5)
        assert ops.solve_triangular(s, b, True, False).shape == (2, 5, 3)


def _rand(shape, seed, scale=1.0):
    g = np.random.default_rng(seed).standard_normal(shape) * scale
    return g


def _grads(fn_ours, fn_ref, x, seed):
    """d loss / d x for ours (float32 on the GPU) and the reference (float64
    on the CPU), loss = a fixed random linear functional of fn's outputs."""
    xg = torch.tensor(x, dtype=torch.float32, device="cuda", requires_grad=True)
    xr = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    outs = fn_ours(xg)
    refs = fn_ref(xr)
    rng = np.random.default_rng(seed)
    loss_g, loss_r = 0, 0
    for o, r in zip(outs, refs):
        c = rng.standard_normal(tuple(r.shape))
        loss_g = loss_g + (o * torch.tensor(c, dtype=torch.float32, device="cuda")).sum()
        loss_r = loss_r + (r * torch.tensor(c, dtype=torch.float64)).sum()
    loss_g.backward()
    loss_r.backward()
    return xg.grad.double().cpu().numpy(), xr.grad.numpy()


def _close(g, r, tol):
    err = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
    print(f"  grad rel err {err:.2e}")
    assert err <= tol


@pytest.mark.gpu
def test_forward_matches_c_abi(cuda):
    a = torch.tensor(_rand((4, 12, 7), 1), dtype=torch.float32, device="cuda")
    q, r = ops.qr(a)
    q2, r2 = api.qr(a)
    assert torch.equal(q, q2) and torch.equal(r, r2)
    s = a[:, :7, :] @ a[:, :7, :].mT.contiguous() + 7 * torch.eye(7, device="cuda")
    w, v = ops.eigh(s)
    w2, v2, _ = api.eigh(s)
    assert torch.equal(w, w2) and torch.equal(v, v2)
    l, info = ops.cholesky(s)
    assert info.dtype == torch.int32 and int(info.abs().sum()) == 0
    # CPU tensors go through the host-pointer path and give the same values
    wc, vc = ops.eigh(s.cpu())
    assert wc.device.type == "cpu" and np.array_equal(to_np(wc), to_np(w))


@pytest.mark.gpu
def test_orders_after_torch_stream(cuda):
    """The input is still being written by work queued on torch's current
    stream (a chain of 4096^3 products, milliseconds each) when the operator
    is called: the library's stream waits for it through an event, and the
    results equal those on the settled input, bit for bit."""
    base = torch.tensor(_rand((256, 64, 64), 5), dtype=torch.float32, device="cuda")
    sym = (base + base.mT).contiguous()
    ref_w, ref_v, _ = api.eigh(sym)
    ref_q, ref_r = api.qr(base)
    torch.cuda.synchronize()
    for op in ("eigh", "qr"):
        big = torch.randn(4096, 4096, device="cuda")
        for _ in range(8):
            big = (big @ big) * (1.0 / 64)
        zero = torch.nan_to_num(big[0, 0], nan=0.0, posinf=0.0, neginf=0.0) * 0.0
        a = torch.zeros_like(base)
        a.copy_((sym if op == "eigh" else base) + zero)   # written only after the chain
        if op == "eigh":
            w, v = ops.eigh(a)
            assert torch.equal(w, ref_w) and torch.equal(v, ref_v)
        else:
            q, r = ops.qr(a)
            assert torch.equal(q, ref_q) and torch.equal(r, ref_r)


@pytest.mark.gpu
def test_gradients(cuda):
    x = _rand((3, 9, 6), 2)
    sq = lambda t: t * t   # sign-invariant functions of vectors
    print("qr")
    g, r = _grads(lambda t: [sq(y) for y in ops.qr(t)], lambda t: [sq(y) for y in torch.linalg.qr(t)], x, 11)
    _close(g, r, 2e-3)
    print("qr wide")
    wide = _rand((3, 5, 8), 5)
    g, r = _grads(lambda t: [sq(y) for y in ops.qr(t)], lambda t: [sq(y) for y in torch.linalg.qr(t)], wide, 20)
    _close(g, r, 2e-3)
    print("svd")
    g, r = _grads(lambda t: [sq(y) for y in ops.svd(t)], lambda t: [sq(y) for y in torch.linalg.svd(t, full_matrices=False)],
                  x, 12)
    _close(g, r, 2e-3)
    print("svdvals")
    g, r = _grads(lambda t: [ops.svdvals(t)], lambda t: [torch.linalg.svdvals(t)], x, 13)
    _close(g, r, 1e-4)
    y = _rand((3, 6, 6), 3)
    sym = y + np.swapaxes(y, -1, -2)
    print("eigh")
    g, r = _grads(lambda t: [sq(z) for z in ops.eigh(t)], lambda t: [sq(z) for z in torch.linalg.eigh(t)], sym, 14)
    # both read the lower triangle: compare the symmetric part
    _close(np.tril(g) + np.swapaxes(np.tril(g, -1), -1, -2), np.tril(r) + np.swapaxes(np.tril(r, -1), -1, -2), 2e-3)
    print("eigvalsh")
    g, r = _grads(lambda t: [ops.eigvalsh(t)], lambda t: [torch.linalg.eigvalsh(t)], sym, 15)
    _close(np.tril(g) + np.swapaxes(np.tril(g, -1), -1, -2), np.tril(r) + np.swapaxes(np.tril(r, -1), -1, -2), 1e-4)
    spd = y @ np.swapaxes(y, -1, -2) + 6 * np.eye(6)
    print("cholesky")
    g, r = _grads(lambda t: [ops.cholesky(t)[0]], lambda t: [torch.linalg.cholesky(t)], spd, 16)
    _close(np.tril(g) + np.swapaxes(np.tril(g, -1), -1, -2), np.tril(r) + np.swapaxes(np.tril(r, -1), -1, -2), 1e-3)
    dom = y + 8 * np.eye(6)
    print("inv")
    g, r = _grads(lambda t: [ops.inv(t)[0]], lambda t: [torch.linalg.inv(t)], dom, 17)
    _close(g, r, 1e-4)
    rhs = _rand((3, 6, 4), 4)
    print("solve")
    bg = torch.tensor(rhs, dtype=torch.float32, device="cuda")
    br = torch.tensor(rhs, dtype=torch.float64)
    g, r = _grads(lambda t: [ops.solve(t, bg)[0]], lambda t: [torch.linalg.solve(t, br)], dom, 18)
    _close(g, r, 1e-4)
    print("solve_triangular")
    low = np.tril(dom)
    g, r = _grads(lambda t: [ops.solve_triangular(t, bg, False, False)],
                  lambda t: [torch.linalg.solve_triangular(t.tril(), br, upper=False)], low, 19)
    _close(np.tril(g), np.tril(r), 1e-4)
