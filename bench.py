"""Benchmark of the MI355X metal_linalg hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one synchronous C-ABI call over one batch of synthetic input that
is already resident in HBM (torch tensors on cuda:0, passed as device
pointers; the output buffers allocated once before the steps, as a C caller
holds them).  W untimed steps, then K timed steps between two
synchronisations.  One JSON line on stdout: `value` = matrices/s over the
timed steps; `roofline` = the dominant kernel's algorithmic bytes (or flops)
per launch over its average duration, timed with HIP events on the
library's launch stream over K more steps after the timed ones (events
between the launches of a multi-launch call lengthen it, so they stay out of
the timed steps; `ms_per_step_kernel_events` is that second pass's time per
step).  The batched kernels are limited by VALU instruction issue rather
than HBM bytes, so `roofline.valu_issue` adds their measured VALU
instruction count per call as issue time on 1024 SIMDs at 2.4 GHz, and its
fraction of the measured kernel time.  `cpu_baseline` = the oracle
(the reference's LAPACK-batched CPU path restated) on the host's cores over
a bounded sample of the same workload.

Workloads are BASELINE.json's configs; the default is the one the headline
metric is quoted on.  Data: synthetic, seeded (tests/_util.py generators).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "batched matrices/s (QR/eigh/SVD/chol/LU) + fp32 GFLOP/s & % peak at n=4096"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
FP32_MFMA_PEAK_TFS = 157.3     # MI355X dense fp32 matrix, published

# HBM bytes per launch of the dominant kernel, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes scaled by a 256 MiB copy kernel's readings (FETCH_SIZE
# x1.9998, WRITE_SIZE x1.0); the runs and the scaling are in
# profiles/<kernel>_<workload>.md.  Workloads not yet counted report null.
TRAFFIC_BYTES = {
    "eigh": 241_899_491, # profiles/eigh_small_eigh.md
    "svd": 511_817_149, # profiles/svd_svd.md
    "qr": 123_540_339, # profiles/qr_small_qr.md
    "qr128x64": 672_378_494, # profiles/qr_tall_qr128x64.md
    "qr4096x64": 2_627_819_140, # profiles/qr_tall_qr4096x64.md
    "eigh128": 2_753_827_916, # profiles/eigh_mid_eigh128.md
    "svd128": 807_681_288, # profiles/svd_jacobi_svd128.md
    "qr128": 812_645_786, # profiles/qr_mid_qr128.md
}

# The batched kernels are bound by instruction issue, not HBM: VALU
# instructions per call (rocprofv3 --pmc SQ_INSTS_VALU, summed over the
# call's kernels; profiles/valu_instructions.md).  A wave64 VALU instruction
# occupies its SIMD for 4 cycles; MI355X has 1024 SIMDs at 2.4 GHz.
VALU_INSTRUCTIONS = {
    "qr": 24_295_000,
    "eigh": 131_263_967,
    "svd": 278_065_237,
    "qr128x64": 388_014_080,
    "eigh128": 830_838_762,
    "svd128": 9_048_489_876,
    "qr128": 488_611_840,
}
SIMDS, CLOCK_HZ = 1024, 2.4e9


class Workload:
    """name, inputs, the device call, and the accounting for one config.

    bytes_per_call / flops_per_call are the algorithmic HBM bytes / flops of
    the roofline kernel(s) per call.  `unit` is "matrices/s" for the batched
    configs and "GFLOP/s" for the single large matrix, where `nominal_flops`
    (the textbook count of the whole decomposition) per call is the numerator.
    """

    def __init__(self, name, desc, batch, make, call, kernel, bytes_per_call, flops_per_call, bound, oracle_call,
                 shape, unit="matrices/s", nominal_flops=None):
        self.name, self.desc, self.batch = name, desc, batch
        self.make, self.call, self.kernel = make, call, kernel
        self.bytes_per_call, self.flops_per_call, self.bound = bytes_per_call, flops_per_call, bound
        self.oracle_call, self.shape = oracle_call, shape
        self.unit, self.nominal_flops = unit, nominal_flops

    def rate(self, calls, seconds):
        if self.unit == "GFLOP/s":
            return self.nominal_flops * calls / seconds / 1e9
        return self.batch * calls / seconds


def blocked_lu_gemm_flops(n, nb=128):
    """Flops of the blocked LU's matrix-core updates: per panel the trailing
    A22 -= L21 U12 (the in-panel updates are thin VALU kernels)."""
    f = 0
    for pj in range(0, n, nb):
        pe = min(pj + nb, n)
        nc = n - pe
        f += 2 * nc * nc * (pe - pj)
    return f


def blocked_chol_gemm_flops(n, nb=128):
    """Flops of the blocked Cholesky's matrix-core updates: per panel, the
    TRSM as a product (2 m2 nb^2) and the lower half of the SYRK (m2^2 nb)."""
    f = 0
    for j in range(0, n, nb):
        b = min(nb, n - j)
        m2 = n - j - b
        f += 2 * m2 * b * b + m2 * m2 * b
    return f


def workloads():
    import _util as U

    w = {}

    def qr_make():
        return {"a": U.config1_qr()}

    def qr_call(api, t):
        return api.qr(t["a"], "reduced")

    w["qr"] = Workload(
        "qr", "qr_with_mode reduced, 10000 x 32x32 fp32 N(0,1) (BASELINE config 1)", 10000, qr_make, qr_call,
        "qr_small", 10000 * (3 * 32 * 32 * 4), 10000 * 87381, "hbm",
        lambda o, h, n: o.qr(h["a"][:n], "reduced"), {"batch": 10000, "rows": 32, "cols": 32})

    def eigh_make():
        return {"a": U.config2_eigh()}

    w["eigh"] = Workload(
        "eigh", "eigh lower with vectors, 4096 x 64x64 fp32 symmetric, 10% scaled by 10^U(-30,37), "
                "one NaN matrix (BASELINE config 2)", 4096, eigh_make,
        lambda api, t: api.eigh(t["a"], True, True), "eigh_small", 4096 * (16384 + 256 + 16384 + 4),
        4096 * 9 * 64 ** 3, "hbm",
        lambda o, h, n: o.eigh(h["a"][:n], True, True), {"batch": 4096, "n": 64})

    def svd_make():
        return {"a": U.config3_svd()}

    w["svd"] = Workload(
        "svd", "thin SVD with vectors, 2048 x 128x64 fp32, s log-uniform in [1e-6, 1], 25% rank-deficient "
               "(BASELINE config 3)", 2048, svd_make,
        lambda api, t: api.svd(t["a"], True), ["svd_bidiag", "svd_bdsqr", "svd_backtransform"], 2048 * (32768 + 32768 + 256 + 16384 + 4),
        2048 * (6 * 128 * 64 * 64 + 20 * 64 ** 3), "hbm",
        lambda o, h, n: o.svd(h["a"][:n], True), {"batch": 2048, "rows": 128, "cols": 64})

    def chol_make():
        a, _ = U.config4_spd()
        return {"a": a}

    w["cholesky"] = Workload(
        "cholesky", "cholesky lower, 8192 x 16x16 SPD fp32, 1% non-SPD (BASELINE config 4)", 8192, chol_make,
        lambda api, t: api.cholesky(t["a"], False), "chol_small", 8192 * (1024 + 1024 + 4), 8192 * 1365, "hbm",
        lambda o, h, n: o.cholesky(h["a"][:n], False), {"batch": 8192, "n": 16})

    def lu_make():
        a, b = U.config4_lu()
        return {"a": a, "b": b}

    w["lu"] = Workload(
        "lu", "lu_factor, 8192 x 16x16 fp32 N(0,1) (BASELINE config 4)", 8192, lu_make,
        lambda api, t: api.lu_factor(t["a"]), "lu_small_factor", 8192 * (1024 + 1024 + 64 + 4), 8192 * 2731, "hbm",
        lambda o, h, n: o.lu_factor(h["a"][:n]), {"batch": 8192, "n": 16})
    w["solve"] = Workload(
        "solve", "solve, 8192 x 16x16 fp32 with 4 right-hand sides (BASELINE config 4)", 8192, lu_make,
        lambda api, t: api.solve(t["a"], t["b"]), "lu_small_solve", 8192 * (1024 + 256 + 256 + 4),
        8192 * (2731 + 2 * 16 * 16 * 4), "hbm",
        lambda o, h, n: o.solve(h["a"][:n], h["b"][:n]), {"batch": 8192, "n": 16, "nrhs": 4})
    def mid_make(spd):
        def make():
            rng = np.random.default_rng(7 if spd else 8)
            g = rng.standard_normal((4096, 128, 128), dtype=np.float32)
            if spd:
                g = (np.matmul(g, np.swapaxes(g, -1, -2)) + np.float32(128) * np.eye(128, dtype=np.float32))
            return {"a": np.ascontiguousarray(g, dtype=np.float32)}
        return make

    # batched shapes beyond the configs: one matrix per workgroup in LDS
    w["cholesky128"] = Workload(
        "cholesky128", "cholesky lower, 4096 x 128x128 SPD fp32 (G G^T + 128 I)", 4096, mid_make(True),
        lambda api, t: api.cholesky(t["a"], False), "chol_small", 4096 * (65536 + 65536 + 4), 4096 * 699051, "hbm",
        lambda o, h, n: o.cholesky(h["a"][:n], False), {"batch": 4096, "n": 128})
    w["lu128"] = Workload(
        "lu128", "lu_factor, 4096 x 128x128 fp32 N(0,1)", 4096, mid_make(False),
        lambda api, t: api.lu_factor(t["a"]), "lu_small_factor", 4096 * (65536 + 65536 + 512 + 4), 4096 * 1398101,
        "hbm", lambda o, h, n: o.lu_factor(h["a"][:n]), {"batch": 4096, "n": 128})
    w["trsm"] = Workload(
        "trsm", "solve_triangular lower unit, 8192 x 16x16 fp32, 4 right-hand sides (BASELINE config 4)", 8192,
        lu_make, lambda api, t: api.solve_triangular(t["a"], t["b"], False, True), "trsm_small",
        8192 * (1024 + 256 + 256), 8192 * 1024, "hbm",
        lambda o, h, n: o.solve_triangular(h["a"][:n], h["b"][:n], False, True), {"batch": 8192, "n": 16, "nrhs": 4})

    # the batched tall QR (one wave per block of up to 128 rows, a reduction
    # tree of block QRs beyond): the reference's QR window past its register
    # kernel, 65 to 4096 rows with at most 64 columns
    def tall_make(batch, m, n, seed):
        def make():
            return {"a": U.gaussian((batch, m, n), seed=seed)}
        return make

    def tall_flops(m, n):
        # Householder R (2 m n^2 - 2 n^3 / 3) and the formation of Q (the same)
        return 4 * m * n * n - 4 * n ** 3 // 3

    for (tb, tm, tn) in ((8192, 128, 64), (256, 4096, 64)):
        tname = f"qr{tm}x{tn}"
        w[tname] = Workload(
            tname, f"qr_with_mode reduced, {tb} x {tm}x{tn} fp32 N(0,1) (the batched tall QR window)", tb,
            tall_make(tb, tm, tn, tm + tn), lambda api, t: api.qr(t["a"], "reduced"), "qr_tall",
            tb * (2 * tm * tn * 4 + tn * tn * 4), tb * tall_flops(tm, tn), "hbm",
            lambda o, h, n: o.qr(h["a"][:n], "reduced"), {"batch": tb, "rows": tm, "cols": tn})

    # the batched mid-size QR (m, n <= 128, a workgroup of two waves per
    # matrix): the reference's batched QR past 64 columns
    w["qr128"] = Workload(
        "qr128", "qr_with_mode reduced, 4096 x 128x128 fp32 N(0,1) (the batched mid-size QR window)", 4096,
        tall_make(4096, 128, 128, 131), lambda api, t: api.qr(t["a"], "reduced"), "qr_mid",
        4096 * 3 * 128 * 128 * 4, 4096 * tall_flops(128, 128), "hbm",
        lambda o, h, n: o.qr(h["a"][:n], "reduced"), {"batch": 4096, "rows": 128, "cols": 128})

    # the batched mid-size eigh (65 <= n <= 128, a workgroup of two waves
    # per matrix): the reference's eigh_ql window past 64
    def sym_make(batch, n, seed):
        def make():
            g = U.gaussian((batch, n, n), seed=seed).astype(np.float64)
            return {"a": ((g + np.swapaxes(g, -1, -2)) / 2).astype(np.float32)}
        return make

    w["eigh128"] = Workload(
        "eigh128", "eigh lower with vectors, 4096 x 128x128 fp32 (G + G^T)/2, G ~ N(0,1) (the batched mid-size "
                   "eigh window)", 4096, sym_make(4096, 128, 128),
        lambda api, t: api.eigh(t["a"], True, True), "eigh_mid", 4096 * (2 * 128 * 128 * 4 + 128 * 4 + 4),
        4096 * (4 * 128 ** 3 // 3 + 2 * 128 ** 3), "hbm",
        lambda o, h, n: o.eigh(h["a"][:n], True, True), {"batch": 4096, "n": 128})

    # the batched mid-size SVD (65 <= min(m, n) <= 128, one-sided Jacobi
    # in LDS): the reference's golub_kahan window past 64
    w["svd128"] = Workload(
        "svd128", "thin SVD with vectors, 4096 x 128x128 fp32 N(0,1) (the batched mid-size SVD window)", 4096,
        tall_make(4096, 128, 128, 257), lambda api, t: api.svd(t["a"], True), "svd_jacobi",
        4096 * (3 * 128 * 128 * 4 + 128 * 4 + 4), 4096 * 22 * 128 ** 3, "hbm",
        lambda o, h, n: o.svd(h["a"][:n], True), {"batch": 4096, "rows": 128, "cols": 128})

    def chol5_make():
        return {"a": U.config5_spd(U.config5_matrix())}

    n5 = 4096
    w["cholesky4096"] = Workload(
        "cholesky4096", "cholesky lower, one 4096x4096 SPD fp32 G G^T/n + I, G ~ N(0,1) (BASELINE config 5)", 1,
        chol5_make, lambda api, t: api.cholesky(t["a"], False), "gemm_mfma", None,
        blocked_chol_gemm_flops(n5), "mfma", lambda o, h, n: o.cholesky(h["a"][None], False), {"n": n5},
        unit="GFLOP/s", nominal_flops=n5 ** 3 / 3)

    def lu5_make():
        return {"a": U.config5_matrix()}

    w["lu4096"] = Workload(
        "lu4096", "lu_factor, one 4096x4096 fp32 G ~ N(0,1) (BASELINE config 5)", 1, lu5_make,
        lambda api, t: api.lu_factor(t["a"]), "gemm_mfma", None, blocked_lu_gemm_flops(n5), "mfma",
        lambda o, h, n: o.lu_factor(h["a"][None]), {"n": n5}, unit="GFLOP/s", nominal_flops=2 * n5 ** 3 / 3)

    def qr5_make():
        return {"a": U.config5_matrix()}

    def qr_gemm_flops(n, nb=128):
        # the trailing updates and the formation of Q as products:
        # per panel W = V^T A2, A2 -= V W, and the same for Q2
        f = 0
        for pj in range(0, n, nb):
            pe = min(pj + nb, n)
            b, rows, n2, nq = pe - pj, n - pj, n - pe, n - pj
            f += 4 * rows * b * n2 + 4 * rows * b * nq
        return f

    def eigh5_make():
        g = U.config5_matrix()
        return {"a": ((g.astype(np.float64) + g.T) / 2).astype(np.float32)}

    def eigh_gemm_flops(n, nb=64):
        # the matrix-core products: the reduction's trailing updates
        # (A22 -= V W^T + W V^T per panel), the Newton-Schulz step (Z^T Z and
        # Z M) and the back-transformation (V^T Z2 and Z2 -= V W2 per panel)
        f = 4 * n ** 3
        for j0 in range(0, n - 1, nb):
            b = min(nb, n - 1 - j0)
            n2 = n - min(j0 + nb, n)
            f += 4 * n2 * n2 * nb + 4 * (n - j0 - 1) * b * n
        return f

    w["eigh4096"] = Workload(
        "eigh4096", "eigh lower with vectors, one 4096x4096 fp32 (G + G^T)/2, G ~ N(0,1) (BASELINE config 5)", 1,
        eigh5_make, lambda api, t: api.eigh(t["a"], True, True), "gemm_mfma", None, eigh_gemm_flops(n5), "mfma",
        lambda o, h, n: o.eigh(h["a"][None], True, True), {"n": n5}, unit="GFLOP/s",
        nominal_flops=(4 * n5 ** 3) // 3 + 2 * n5 ** 3)

    w["qr4096"] = Workload(
        "qr4096", "qr_with_mode reduced, one 4096x4096 fp32 G ~ N(0,1) (BASELINE config 5)", 1, qr5_make,
        lambda api, t: api.qr(t["a"], "reduced"), "gemm_mfma", None, qr_gemm_flops(n5), "mfma",
        lambda o, h, n: o.qr(h["a"][None], "reduced"), {"n": n5}, unit="GFLOP/s", nominal_flops=8 * n5 ** 3 / 3)

    def bidiag_bytes(m, k):
        # the one-stage bidiagonalisation's HBM floor: per column the
        # trailing block is read and written by the left update and read
        # again by the product A v (it outgrows on-chip memory), 4 B each
        return sum(4 * (2 * (m - j) * (k - j) + (m - j - 1) * (k - j - 1)) for j in range(k))

    # the large single-matrix SVD (not a BASELINE config): rate by the
    # nominal count of bidiagonalisation (8/3 n^3) and the two reflector
    # back-transforms (2 n^3 each), as LAPACK's sgebrd + sormbr
    w["svd4096"] = Workload(
        "svd4096", "thin SVD with vectors, one 4096x4096 fp32 G ~ N(0,1) (the large single-matrix SVD)", 1,
        qr5_make, lambda api, t: api.svd(t["a"], True), "svd_bidiag_large", bidiag_bytes(n5, n5), None, "hbm",
        lambda o, h, n: o.svd(h["a"][None], True), {"n": n5}, unit="GFLOP/s",
        nominal_flops=8 * n5 ** 3 // 3 + 4 * n5 ** 3)
    return w


class CAbi:
    """The workloads' calls made as a C caller makes them: device pointers
    straight into the C ABI, output buffers allocated once (`allocate`, before
    any step) and written again by every call.  A step then holds the library
    call alone; the inputs are resident and torch has nothing pending on its
    stream, so no stream ordering is asked for (the Python API in
    `metal_linalg_amd.api` adds its output allocations and, when torch's
    stream has work pending, an event wait; `ms_per_step_python_api` times
    it)."""

    def __init__(self, lib):
        self.lib, self.bufs, self.dry = lib, {}, False

    def _out(self, key, specs):
        if key not in self.bufs:
            import torch

            self.bufs[key] = [None if shape is None else
                              torch.empty(shape, dtype=torch.float32 if dt == "f32" else torch.int32, device="cuda")
                              for shape, dt in specs]
        return self.bufs[key]

    def _call(self, fn, *args):
        if self.dry:
            return
        rc = fn(*[a.data_ptr() if hasattr(a, "data_ptr") else a for a in args])
        if rc != self.lib.OK:
            raise RuntimeError(self.lib.last_error().decode())

    def allocate(self, wl, dev):
        self.dry = True
        try:
            wl.call(self, dev)
        finally:
            self.dry = False

    @staticmethod
    def _dims(a):
        b = 1
        for d in a.shape[:-2]:
            b *= int(d)
        return tuple(a.shape[:-2]), b, int(a.shape[-2]), int(a.shape[-1])

    def qr(self, a, mode="reduced"):
        lead, b, m, n = self._dims(a)
        k = min(m, n)
        code = self.lib.QR_MODES[mode]
        qc = 0 if code == 1 else (m if code == 2 else k)
        rr = m if code == 2 else k
        q, r = self._out(("qr", a.shape, mode), [(lead + (m, qc) if qc else None, "f32"), (lead + (rr, n), "f32")])
        self._call(self.lib.qr_with_mode, a, b, m, n, code, q, r)

    def eigh(self, a, lower=True, vectors=True):
        lead, b, n, _ = self._dims(a)
        w, v, info = self._out(("eigh", a.shape, vectors),
                               [(lead + (n,), "f32"), (lead + (n, n) if vectors else None, "f32"), (lead, "u32")])
        self._call(self.lib.eigh, a, b, n, int(bool(lower)), w, v, info)

    def svd(self, a, vectors=True):
        lead, b, m, n = self._dims(a)
        k = min(m, n)
        u, s, vt, info = self._out(("svd", a.shape, vectors),
                                   [(lead + (m, k) if vectors else None, "f32"), (lead + (k,), "f32"),
                                    (lead + (k, n) if vectors else None, "f32"), (lead, "u32")])
        self._call(self.lib.svd, a, b, m, n, u, s, vt, info)

    def cholesky(self, a, upper=False):
        lead, b, n, _ = self._dims(a)
        l, info = self._out(("cholesky", a.shape), [(lead + (n, n), "f32"), (lead, "u32")])
        self._call(self.lib.cholesky, a, b, n, int(bool(upper)), l, info)

    def lu_factor(self, a):
        lead, b, n, _ = self._dims(a)
        lu, piv, info = self._out(("lu", a.shape), [(lead + (n, n), "f32"), (lead + (n,), "u32"), (lead, "u32")])
        self._call(self.lib.lu_factor, a, b, n, lu, piv, info)

    def solve(self, a, rhs):
        lead, b, n, _ = self._dims(a)
        x, info = self._out(("solve", a.shape, rhs.shape), [(tuple(rhs.shape), "f32"), (lead, "u32")])
        self._call(self.lib.solve, a, b, n, rhs, int(rhs.shape[-1]), x, info)

    def solve_triangular(self, a, rhs, upper=False, unit=False):
        lead, b, n, _ = self._dims(a)
        (x,) = self._out(("trsm", a.shape, rhs.shape), [(tuple(rhs.shape), "f32")])
        self._call(self.lib.solve_triangular, a, b, n, rhs, int(rhs.shape[-1]), int(bool(upper)), int(bool(unit)), x)


def _arrays(x):
    if x is None:
        return []
    if isinstance(x, dict):
        return [v for v in x.values() if hasattr(v, "nbytes")]
    if isinstance(x, (tuple, list)):
        return [v for v in x if v is not None and hasattr(v, "nbytes")]
    return [x] if hasattr(x, "nbytes") else []


def host_pointer_path(wl, api, host, reps):
    """The call on host (numpy) buffers: staged through pinned memory in
    chunks by the library.  Beside it, the PCIe bound for the same bytes:
    pinned torch copies of the inputs to the device and of the outputs back,
    the two directions on two streams at once (the link is full duplex)."""
    import torch

    out = wl.call(api, host)   # warm-up: pinned and device staging allocated
    in_bytes = sum(a.nbytes for a in _arrays(host))
    out_bytes = sum(a.nbytes for a in _arrays(out))
    t0 = time.perf_counter()
    for _ in range(reps):
        wl.call(api, host)
    t_call = (time.perf_counter() - t0) / reps
    # the caller's buffers pinned (torch pin_memory tensors in and out): the
    # transfers read and write them directly
    pinned = {k: (torch.from_numpy(v).pin_memory() if isinstance(v, np.ndarray) else v) for k, v in host.items()}
    wl.call(api, pinned)
    t0 = time.perf_counter()
    for _ in range(reps):
        wl.call(api, pinned)
    t_pinned = (time.perf_counter() - t0) / reps
    h_in = torch.empty(max(1, in_bytes), dtype=torch.uint8, pin_memory=True)
    d_in = torch.empty(max(1, in_bytes), dtype=torch.uint8, device="cuda")
    d_out = torch.empty(max(1, out_bytes), dtype=torch.uint8, device="cuda")
    h_out = torch.empty(max(1, out_bytes), dtype=torch.uint8, pin_memory=True)
    s_up, s_down = torch.cuda.Stream(), torch.cuda.Stream()

    def both():
        with torch.cuda.stream(s_up):
            d_in.copy_(h_in, non_blocking=True)
        with torch.cuda.stream(s_down):
            h_out.copy_(d_out, non_blocking=True)

    both()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        both()
    torch.cuda.synchronize()
    t_pcie = (time.perf_counter() - t0) / reps
    total = in_bytes + out_bytes
    return {"value": round(wl.rate(1, t_call), 2), "unit": wl.unit, "ms_per_call": round(t_call * 1e3, 3),
            "host_bytes_per_call": total, "gb_s": round(total / t_call / 1e9, 2),
            "pcie_bound": {"ms_per_call": round(t_pcie * 1e3, 3), "gb_s": round(total / t_pcie / 1e9, 2),
                           "rate": round(wl.rate(1, t_pcie), 2),
                           "how": "pinned torch copies of the same bytes, inputs up and outputs down at once"},
            "frac_of_pcie_bound": round(t_pcie / t_call, 4),
            "pinned_buffers": {"value": round(wl.rate(1, t_pinned), 2), "ms_per_call": round(t_pinned * 1e3, 3),
                               "gb_s": round(total / t_pinned / 1e9, 2),
                               "frac_of_pcie_bound": round(t_pcie / t_pinned, 4)}}


def host_cpus() -> str:
    """The CPU model and the cores this process may run on."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return f"{model}, {allowed} logical CPUs allowed"


def cpu_baseline(wl, host, seconds):
    """The oracle on the host: a one-thread sample, then the pool of
    OMP_NUM_THREADS workers (the reference's lapack_batches); both after a
    warm-up pass that loads the workers' LAPACK copies."""
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)

    def rate(t, n, secs):
        oracle.set_threads(t)
        wl.oracle_call(oracle, host, n)   # warm-up (and the workers' LAPACK copies)
        count, t0 = 0, time.perf_counter()
        while True:
            wl.oracle_call(oracle, host, n)
            count += n
            if time.perf_counter() - t0 >= secs:
                break
        dt = time.perf_counter() - t0
        return wl.rate(count / wl.batch, dt), count, dt

    if wl.batch == 1:   # one large matrix: LAPACK's own threads, as the reference
        many, cn, sn = rate(threads, 1, seconds)
        return {"value": round(many, 2), "unit": wl.unit, "cores": threads, "kind": "port",
                "sample": f"{cn} factorisation(s) in {sn:.2f} s, LAPACK on {threads} threads; host: {host_cpus()}; "
                          f"{oracle.config()}"}
    # one thread on a sub-batch (a whole-batch pass can take seconds there)
    one, c1, s1 = rate(1, max(1, wl.batch // 8), seconds / 2)
    many, cn, sn = rate(threads, wl.batch, seconds)
    copies = int(oracle.lib().oracle_lapack_copies())
    return {"value": round(many, 2), "unit": wl.unit, "cores": threads, "kind": "port",
            "sample": f"{cn} matrices ({cn // wl.batch} passes over the {wl.batch}-matrix batch) in {sn:.2f} s on "
                      f"{threads} worker threads ({copies} private LAPACK copies); one thread: {one:.6g} {wl.unit} "
                      f"({c1} matrices in {s1:.2f} s), so {many / one:.2f}x on {threads} threads; host: "
                      f"{host_cpus()}; {oracle.config()}"}


# The other BASELINE configs, timed in the default run beside the headline
# (device pointers through the C ABI, as the headline's steps): config 1,
# config 3, config 4's four calls and config 5's four 4096 x 4096 calls.
OTHER_CONFIGS = [("qr", 20), ("svd", 10), ("cholesky", 20), ("lu", 20), ("solve", 20), ("trsm", 20),
                 ("cholesky4096", 5), ("lu4096", 3), ("qr4096", 3), ("eigh4096", 2)]


def other_configs(_lib, skip):
    """{workload: rate, time per call and roofline fraction} for the configs
    other than `skip`; each one's failure is reported in its entry."""
    import torch

    out = {}
    for name, steps in OTHER_CONFIGS:
        if name == skip:
            continue
        try:
            wl = workloads()[name]
            dev = {k: torch.from_numpy(np.ascontiguousarray(v)).to("cuda") for k, v in wl.make().items()}
            cabi = CAbi(_lib)
            cabi.allocate(wl, dev)
            wl.call(cabi, dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                wl.call(cabi, dev)
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - t0
            names = wl.kernel if isinstance(wl.kernel, (list, tuple)) else [wl.kernel]
            _lib.hip_reset_timing()
            _lib.hip_set_timing(1)
            for _ in range(steps):
                wl.call(cabi, dev)
            torch.cuda.synchronize()
            _lib.hip_set_timing(0)
            kernel_s = sum(_lib.kernel_time(k)[1] for k in names) / 1e3 / steps
            if wl.bound == "hbm":
                frac = wl.bytes_per_call / kernel_s / 1e9 / HBM_PEAK_GBS
            else:
                frac = wl.flops_per_call / kernel_s / 1e12 / FP32_MFMA_PEAK_TFS
            out[name] = {"value": round(wl.rate(steps, elapsed), 2), "unit": wl.unit,
                         "ms_per_call": round(elapsed * 1e3 / steps, 4),
                         "kernel_us_per_call": round(kernel_s * 1e6, 2), "roofline_bound": wl.bound,
                         "roofline_frac": round(frac, 5), "steps": steps}
            del dev, cabi
        except Exception as e:   # reported, not fatal: the headline line is printed regardless
            out[name] = {"error": f"{type(e).__name__}: {e}"}
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="eigh")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-host-path", action="store_true",
                    help="skip the host-pointer leg (for profiler runs that count only the device calls)")
    ap.add_argument("--cpu-seconds", type=float, default=2.0, help="wall seconds of the CPU baseline sample")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip timing the other BASELINE configs (they run by default beside the headline)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the batch would shard across GPUs with no exchange, which no run here measures)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible; the library has no CPU path to measure", file=sys.stderr)
        sys.exit(1)
    from metal_linalg_amd import _lib, api

    wl = workloads()[args.workload]
    host = wl.make()
    dev = {k: torch.from_numpy(np.ascontiguousarray(v)).to("cuda") for k, v in host.items()}
    torch.cuda.synchronize()

    cabi = CAbi(_lib)
    cabi.allocate(wl, dev)
    for _ in range(args.warmup):
        wl.call(cabi, dev)
    torch.cuda.synchronize()

    # the timed steps, with no events between the path's launches
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        wl.call(cabi, dev)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # the same steps again with a HIP event pair around each of the path's
    # kernels (on the library's stream), for their durations; the events
    # lengthen a multi-launch call, so this pass is not the one timed above
    _lib.hip_reset_timing()
    _lib.hip_set_timing(1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        wl.call(cabi, dev)
    torch.cuda.synchronize()
    elapsed_events = time.perf_counter() - t1
    _lib.hip_set_timing(0)

    # the same steps through the Python API (new output tensors per call)
    wl.call(api, dev)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for _ in range(args.steps):
        wl.call(api, dev)
    torch.cuda.synchronize()
    elapsed_api = time.perf_counter() - t2

    # the path's kernels (one name, or several launched once per call each)
    names = wl.kernel if isinstance(wl.kernel, (list, tuple)) else [wl.kernel]
    per = [_lib.kernel_time(k) for k in names]
    launches = sum(p[0] for p in per)
    kernel_ms = sum(p[1] for p in per)
    other = {n: _lib.kernel_time(n) for n in _lib.kernel_names()}
    # per call: the roofline kernels' summed HIP-event time over the timed steps
    kernel_s_per_call = (kernel_ms / 1e3) / args.steps
    avg_kernel_s = (kernel_ms / 1e3) / max(launches, 1)
    ms_per_step = elapsed * 1e3 / args.steps
    value = wl.rate(args.steps, elapsed)

    if wl.bound == "hbm":
        achieved = wl.bytes_per_call / kernel_s_per_call / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": TRAFFIC_BYTES.get(wl.name)}
    else:
        achieved = wl.flops_per_call / kernel_s_per_call / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 4), "peak": FP32_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_MFMA_PEAK_TFS, 5), "traffic": None}
    roof["kernel"] = "+".join(names)
    roof["kernel_avg_us"] = round(avg_kernel_s * 1e6, 3)
    roof["launches"] = launches
    roof["launches_per_call"] = launches / args.steps
    roof["kernel_us_per_call"] = round(kernel_s_per_call * 1e6, 3)
    roof["algorithmic_bytes_per_launch"] = wl.bytes_per_call
    roof["algorithmic_flops_per_launch"] = wl.flops_per_call
    if wl.name in VALU_INSTRUCTIONS:
        issue_s = VALU_INSTRUCTIONS[wl.name] * 4 / (SIMDS * CLOCK_HZ)
        roof["valu_issue"] = {"instructions_per_call": VALU_INSTRUCTIONS[wl.name],
                              "issue_us_per_call": round(issue_s * 1e6, 1),
                              "frac": round(issue_s / kernel_s_per_call, 4)}

    # host-pointer (PCIe-inclusive) rate, for the record; never `value`
    host_path = None if args.no_host_path else host_pointer_path(wl, api, host, max(1, min(5, args.steps)))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(wl, host, args.cpu_seconds)

    # the other configs, in the default run only (a profiler run names its
    # workload and skips the host path)
    others = None
    if not args.no_other_configs and not args.no_host_path and args.workload == "eigh":
        others = other_configs(_lib, wl.name)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "ms_per_step_kernel_events": round(elapsed_events * 1e3 / args.steps, 5),
        "ms_per_step_python_api": round(elapsed_api * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) per BASELINE.json configs; device-resident inputs)",
        "config": dict({"workload": wl.desc}, **wl.shape),
        "roofline": roof,
        "cpu_baseline": cpu,
        "host_pointer_rate": host_path["value"] if host_path else None,
        "host_pointer": host_path,
        "kernels": {k: {"launches": v[0], "total_ms": round(v[1], 4)} for k, v in other.items()},
        "other_configs": others,
        "device": _lib.device_name().decode(),
        "arch": _lib.hip_arch().decode(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
