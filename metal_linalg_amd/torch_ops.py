"""The decompositions as torch custom operators: torch.ops.metal_linalg.*.

The MI355X counterpart of the reference's PyTorch binding
(reference: python-torch/metal_linalg_torch/_ops.py): the same operator
names, arguments and outputs (qr, eigh, eigvalsh, svd, svdvals, cholesky,
lu_factor, solve, inv, solve_triangular), over this build's C ABI.

A GPU tensor (ROCm: device type "cuda") is read and written in place by the
library on its own stream, which first waits (through an event, without
blocking the host) for the work queued on torch's current stream, as that may
still be writing the input; the call returns when the results are complete.  A CPU tensor goes through the C ABI's host-pointer
path (staged through device memory), so CPU tensors work too, computed on the
GPU.  Every operator has a fake (meta) implementation giving torch.compile the
output shapes, and the differentiable ones carry the backward formulas below
(the usual ones for each decomposition, as torch.linalg's), so that they train
like the built-in operators.  Integer outputs (info, pivots) are int32 holding
the C ABI's uint32 values.

Importing this module registers the operators.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from . import api

__all__ = ["qr", "eigh", "eigvalsh", "svd", "svdvals", "cholesky", "lu_factor", "solve", "inv", "solve_triangular"]


def _f32(a: Tensor) -> Tensor:
    return a.detach().to(torch.float32).contiguous()


def _back(x, like: Tensor) -> Tensor:
    """A result of api.* as a tensor on like's device (int32 for integers)."""
    if x is None:
        return torch.empty(0, device=like.device, dtype=torch.float32)
    if isinstance(x, Tensor):
        return x
    x = np.asarray(x)
    if x.dtype == np.uint32:
        x = x.view(np.int32)
    return torch.from_numpy(np.ascontiguousarray(x)).to(like.device)


def _run(fn, a: Tensor, *rest):
    """fn over device tensors in place (api orders the library's stream after
    torch's current one), or over host arrays for CPU tensors."""
    if a.device.type == "cuda":
        return fn(a, *rest)
    return fn(a.numpy(), *[r.numpy() for r in rest])


def _lead_k(a):
    *lead, m, n = a.shape
    return list(lead), m, n, min(m, n)


def _qr_shapes(a, mode):
    lead, m, n, k = _lead_k(a)
    if mode == "r":
        return [0], lead + [k, n]
    if mode == "complete":
        return lead + [m, m], lead + [m, n]
    return lead + [m, k], lead + [k, n]


# ---------------------------------------------------------------- QR --------

@torch.library.custom_op("metal_linalg::qr", mutates_args=(), schema="(Tensor a, str mode='reduced') -> (Tensor, Tensor)")
def qr(a: Tensor, mode: str = "reduced") -> tuple[Tensor, Tensor]:
    a = _f32(a)
    q, r = _run(lambda x: api.qr(x, mode), a)
    return _back(q, a), _back(r, a)


@qr.register_fake
def _(a, mode="reduced"):
    qs, rs = _qr_shapes(a, mode)
    return a.new_empty(qs, dtype=torch.float32), a.new_empty(rs, dtype=torch.float32)


def _copyltu(m: Tensor) -> Tensor:
    """The lower triangle mirrored into the upper (diagonal kept)."""
    low = m.tril(-1)
    return low + low.mT + torch.diag_embed(m.diagonal(dim1=-2, dim2=-1))


def _qr_setup(ctx, inputs, output):
    a, mode = inputs
    q, r = output
    ctx.mode = mode
    ctx.save_for_backward(q, r)


def _qr_tall_grad(q, r, gq, gr):
    """A = Q R with M >= N (R square, invertible): gA = (gQ + Q copyltu(M)) R^-T,
    M = R gR^T - gQ^T Q."""
    mm = r @ gr.mT.contiguous() - gq.mT.contiguous() @ q
    b = gq + q @ _copyltu(mm)
    return torch.linalg.solve_triangular(r, b.mT.contiguous(), upper=True, left=True).mT


def _qr_backward(ctx, gq, gr):
    q, r = ctx.saved_tensors
    m, n = q.shape[-2], r.shape[-1]
    if ctx.mode != "reduced":
        raise NotImplementedError("metal_linalg.qr: the backward is defined for mode='reduced'")
    gq = torch.zeros_like(q) if gq is None else gq
    gr = torch.zeros_like(r) if gr is None else gr
    if m >= n:
        return _qr_tall_grad(q, r, gq, gr).contiguous(), None
    # wide: A = [X Y] with X = Q R1 (square) and Y = Q R2, R2 = Q^T Y.  Y's
    # part: gY = Q gR2; through R2 the loss also depends on Q: gQ += Y gR2^T.
    r1, r2 = r[..., :m], r[..., m:]
    gr1, gr2 = gr[..., :m], gr[..., m:]
    y = q @ r2
    gx = _qr_tall_grad(q, r1, gq + y @ gr2.mT.contiguous(), gr1)
    gy = q @ gr2
    return torch.cat([gx, gy], dim=-1).contiguous(), None


qr.register_autograd(_qr_backward, setup_context=_qr_setup)


# -------------------------------------------------------------- eigh --------

def _square(a, name):
    if a.shape[-1] != a.shape[-2]:
        raise ValueError(f"metal_linalg.{name}: square matrices expected, got {tuple(a.shape)}")


@torch.library.custom_op("metal_linalg::eigh", mutates_args=(), schema="(Tensor a, bool lower=True) -> (Tensor, Tensor)")
def eigh(a: Tensor, lower: bool = True) -> tuple[Tensor, Tensor]:
    _square(a, "eigh")
    a = _f32(a)
    w, v, _ = _run(lambda x: api.eigh(x, lower, True), a)
    return _back(w, a), _back(v, a)


@eigh.register_fake
def _(a, lower=True):
    lead, m, n, _ = _lead_k(a)
    return a.new_empty(lead + [n], dtype=torch.float32), a.new_empty(lead + [n, n], dtype=torch.float32)


@torch.library.custom_op("metal_linalg::eigvalsh", mutates_args=(), schema="(Tensor a, bool lower=True) -> Tensor")
def eigvalsh(a: Tensor, lower: bool = True) -> Tensor:
    _square(a, "eigvalsh")
    a = _f32(a)
    w, _, _ = _run(lambda x: api.eigh(x, lower, False), a)
    return _back(w, a)


@eigvalsh.register_fake
def _(a, lower=True):
    lead, m, n, _ = _lead_k(a)
    return a.new_empty(lead + [n], dtype=torch.float32)


def _eigh_grad(w, v, gw, gv):
    # A = V diag(w) V^T: gA = V (diag(gw) + skew(V^T gV) / E) V^T, E_ij = w_j - w_i
    inner = torch.zeros_like(v) if gw is None else torch.diag_embed(gw)
    if gv is not None:
        k = v.mT.contiguous() @ gv
        e = w.unsqueeze(-2) - w.unsqueeze(-1)
        e.diagonal(dim1=-2, dim2=-1).fill_(float("inf"))
        inner = inner + (k - k.mT) / (2.0 * e)
    return v @ inner @ v.mT.contiguous()


def _eigh_setup(ctx, inputs, output):
    ctx.save_for_backward(*output)


def _eigh_backward(ctx, gw, gv):
    w, v = ctx.saved_tensors
    return _eigh_grad(w, v, gw, gv), None


eigh.register_autograd(_eigh_backward, setup_context=_eigh_setup)


def _eigvalsh_setup(ctx, inputs, output):
    a, lower = inputs
    ctx.lower = lower
    ctx.save_for_backward(a)


def _eigvalsh_backward(ctx, gw):
    (a,) = ctx.saved_tensors
    w, v = eigh(a, ctx.lower)
    return _eigh_grad(w, v, gw, None), None


eigvalsh.register_autograd(_eigvalsh_backward, setup_context=_eigvalsh_setup)


# --------------------------------------------------------------- SVD --------

@torch.library.custom_op("metal_linalg::svd", mutates_args=(), schema="(Tensor a) -> (Tensor, Tensor, Tensor)")
def svd(a: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    a = _f32(a)
    u, s, vt, _ = _run(lambda x: api.svd(x, True), a)
    return _back(u, a), _back(s, a), _back(vt, a)


@svd.register_fake
def _(a):
    lead, m, n, k = _lead_k(a)
    f = torch.float32
    return a.new_empty(lead + [m, k], dtype=f), a.new_empty(lead + [k], dtype=f), a.new_empty(lead + [k, n], dtype=f)


@torch.library.custom_op("metal_linalg::svdvals", mutates_args=(), schema="(Tensor a) -> Tensor")
def svdvals(a: Tensor) -> Tensor:
    a = _f32(a)
    _, s, _, _ = _run(lambda x: api.svd(x, False), a)
    return _back(s, a)


@svdvals.register_fake
def _(a):
    lead, m, n, k = _lead_k(a)
    return a.new_empty(lead + [k], dtype=torch.float32)


def _svd_grad(u, s, vh, gu, gs, gvh):
    # thin real SVD A = U diag(s) V^T (Townsend's formula):
    # gA = U [F o (J - J^T) S + diag(gs) + S F o (K - K^T)] V^T
    #      + (I - U U^T) gU S^-1 V^T + U S^-1 gV^T (I - V V^T),
    # J = U^T gU, K = V^T gV, F_ij = 1 / (s_j^2 - s_i^2) off the diagonal
    v = vh.mT.contiguous()
    inner = torch.diag_embed(gs) if gs is not None else torch.zeros(s.shape + s.shape[-1:], dtype=s.dtype,
                                                                     device=s.device)
    s2 = s * s
    f = s2.unsqueeze(-2) - s2.unsqueeze(-1)
    f.diagonal(dim1=-2, dim2=-1).fill_(float("inf"))
    f = 1.0 / f
    sd = torch.diag_embed(s)
    ga = torch.zeros(u.shape[:-1] + v.shape[-2:-1], dtype=u.dtype, device=u.device)
    if gu is not None:
        j = u.mT.contiguous() @ gu
        inner = inner + (f * (j - j.mT)) @ sd
        proj = gu - u @ j
        ga = ga + (proj / s.unsqueeze(-2)) @ vh
    if gvh is not None:
        gv = gvh.mT.contiguous()
        k = v.mT.contiguous() @ gv
        inner = inner + sd @ (f * (k - k.mT))
        proj = gv - v @ k
        ga = ga + u @ (proj / s.unsqueeze(-2)).mT.contiguous()
    return ga + u @ inner @ vh


def _svd_setup(ctx, inputs, output):
    ctx.save_for_backward(*output)


def _svd_backward(ctx, gu, gs, gvh):
    u, s, vh = ctx.saved_tensors
    return _svd_grad(u, s, vh, gu, gs, gvh)


svd.register_autograd(_svd_backward, setup_context=_svd_setup)


def _svdvals_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])


def _svdvals_backward(ctx, gs):
    (a,) = ctx.saved_tensors
    u, s, vh = svd(a)
    return u @ torch.diag_embed(gs) @ vh


svdvals.register_autograd(_svdvals_backward, setup_context=_svdvals_setup)


# ---------------------------------------------------------- Cholesky --------

@torch.library.custom_op("metal_linalg::cholesky", mutates_args=(),
                         schema="(Tensor a, bool upper=False) -> (Tensor, Tensor)")
def cholesky(a: Tensor, upper: bool = False) -> tuple[Tensor, Tensor]:
    _square(a, "cholesky")
    a = _f32(a)
    l, info = _run(lambda x: api.cholesky(x, upper), a)
    return _back(l, a), _back(info, a)


@cholesky.register_fake
def _(a, upper=False):
    lead, m, n, _ = _lead_k(a)
    return a.new_empty(lead + [n, n], dtype=torch.float32), a.new_empty(lead, dtype=torch.int32)


def _cholesky_setup(ctx, inputs, output):
    ctx.upper = inputs[1]
    ctx.save_for_backward(output[0])


def _cholesky_backward(ctx, gl, ginfo):
    (l,) = ctx.saved_tensors
    if ctx.upper:   # U = L^T
        l, gl = l.mT.contiguous(), gl.mT.contiguous()
    # A = L L^T: gA = sym(L^-T Phi(L^T gL) L^-1), Phi = lower triangle with
    # the diagonal halved
    p = l.mT.contiguous() @ gl
    p = p.tril() - 0.5 * torch.diag_embed(p.diagonal(dim1=-2, dim2=-1))
    x = torch.linalg.solve_triangular(l.mT.contiguous(), p, upper=True)                       # L^-T P
    x = torch.linalg.solve_triangular(l.mT.contiguous(), x.mT.contiguous(), upper=True).mT   # (L^-T P) L^-1
    return 0.5 * (x + x.mT), None


cholesky.register_autograd(_cholesky_backward, setup_context=_cholesky_setup)


# ------------------------------------------------------ LU, solve, inv ------

@torch.library.custom_op("metal_linalg::lu_factor", mutates_args=(), schema="(Tensor a) -> (Tensor, Tensor, Tensor)")
def lu_factor(a: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    _square(a, "lu_factor")
    a = _f32(a)
    lu, piv, info = _run(api.lu_factor, a)
    return _back(lu, a), _back(piv, a), _back(info, a)


@lu_factor.register_fake
def _(a):
    lead, m, n, _ = _lead_k(a)
    return (a.new_empty(lead + [n, n], dtype=torch.float32), a.new_empty(lead + [n], dtype=torch.int32),
            a.new_empty(lead, dtype=torch.int32))


@torch.library.custom_op("metal_linalg::solve", mutates_args=(), schema="(Tensor a, Tensor b) -> (Tensor, Tensor)")
def solve(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor]:
    _square(a, "solve")
    a, b = _f32(a), _f32(b)
    x, info = _run(api.solve, a, b)
    return _back(x, a), _back(info, a)


@solve.register_fake
def _(a, b):
    lead, m, n, _ = _lead_k(a)
    return b.new_empty(list(b.shape), dtype=torch.float32), a.new_empty(lead, dtype=torch.int32)


def _solve_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], output[0])


def _solve_backward(ctx, gx, ginfo):
    a, x = ctx.saved_tensors
    gb, _ = solve(a.mT.contiguous(), gx.contiguous())   # A^-T gX
    return -gb @ x.mT.contiguous(), gb


solve.register_autograd(_solve_backward, setup_context=_solve_setup)


@torch.library.custom_op("metal_linalg::inv", mutates_args=(), schema="(Tensor a) -> (Tensor, Tensor)")
def inv(a: Tensor) -> tuple[Tensor, Tensor]:
    _square(a, "inv")
    a = _f32(a)
    x, info = _run(api.inv, a)
    return _back(x, a), _back(info, a)


@inv.register_fake
def _(a):
    lead, m, n, _ = _lead_k(a)
    return a.new_empty(lead + [n, n], dtype=torch.float32), a.new_empty(lead, dtype=torch.int32)


def _inv_setup(ctx, inputs, output):
    ctx.save_for_backward(output[0])


def _inv_backward(ctx, gx, ginfo):
    (x,) = ctx.saved_tensors
    xt = x.mT.contiguous()
    return -xt @ gx @ xt


inv.register_autograd(_inv_backward, setup_context=_inv_setup)


@torch.library.custom_op("metal_linalg::solve_triangular", mutates_args=(),
                         schema="(Tensor a, Tensor b, bool upper=False, bool unit=False) -> Tensor")
def solve_triangular(a: Tensor, b: Tensor, upper: bool = False, unit: bool = False) -> Tensor:
    _square(a, "solve_triangular")
    a, b = _f32(a), _f32(b)
    x = _run(lambda p, q: api.solve_triangular(p, q, upper, unit), a, b)
    return _back(x, a)


@solve_triangular.register_fake
def _(a, b, upper=False, unit=False):
    return b.new_empty(list(b.shape), dtype=torch.float32)


def _trsm_setup(ctx, inputs, output):
    ctx.upper, ctx.unit = inputs[2], inputs[3]
    ctx.save_for_backward(inputs[0], output)


def _trsm_backward(ctx, gx):
    a, x = ctx.saved_tensors
    # X = T^-1 B: gB = T^-T gX (the transpose swaps the triangle), gA = -gB X^T
    # on T's triangle (strictly, for a unit diagonal)
    gb = solve_triangular(a.mT.contiguous(), gx.contiguous(), not ctx.upper, ctx.unit)
    ga = -gb @ x.mT.contiguous()
    ga = ga.triu(1 if ctx.unit else 0) if ctx.upper else ga.tril(-1 if ctx.unit else 0)
    return ga, gb, None, None


solve_triangular.register_autograd(_trsm_backward, setup_context=_trsm_setup)
