"""Routing sweep for the MI355X: the batched kernels against the
one-matrix-at-a-time blocked path.

For Cholesky, LU (factor) and the triangular solve, every n up to the
batched kernels' 128 has two GPU routes: one launch for the whole batch
(a wave or a workgroup per matrix), or the blocked path, one matrix after
another.  The first wins on large batches, the second can win on a few
large matrices (it spreads one matrix over the whole device).  This sweep
times both over a grid of n and batch on device buffers and writes the
policy rows that pick the faster:

    python -m metal_linalg_amd.tuning.sweep [--quick]

  -> metal_linalg_amd/csrc/tuned_gfx950.inc   the rows (rebuild the library)
  -> metal_linalg_amd/tuning/gfx950_sweep.csv the timings they came from

Each point is the median of repeated synchronous calls after two warm-ups
(the reference's sweeps time the same way: tuning/sweep_timing.h:1-103);
the rows are fitted to the reference's routing rules (src/cholesky.mm:
143-148 blocked when n >= blocked_min_n and batch <= blocked_max_batch;
src/lu.mm:119-121 and src/trsm.mm:136-138 likewise with gpu_min_n and
gpu_max_batch) by choosing, among the grid's values, the pair with the
smallest summed slowdown against the faster route at every point.
"""

from __future__ import annotations

import argparse
import datetime
import os
import statistics
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
INC = os.path.join(PKG, "csrc", "tuned_gfx950.inc")
CSV = os.path.join(HERE, "gfx950_sweep.csv")
NO_LIMIT = 0xFFFFFFFF


def _time(fn, reps):
    import torch

    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _inputs(torch, which, n, batch, rng):
    g = rng.standard_normal((batch, n, n)).astype(np.float32)
    if which == "cholesky":
        g = g @ np.swapaxes(g, -1, -2) + np.float32(n) * np.eye(n, dtype=np.float32)
    if which == "trsm":
        g = g / np.float32(n) + np.float32(2) * np.eye(n, dtype=np.float32)
    b = rng.standard_normal((batch, n, 8)).astype(np.float32)
    return torch.from_numpy(g).to("cuda"), torch.from_numpy(b).to("cuda")


# (policy name, fields forcing the blocked path, fields forcing the batched kernels)
FORCE = {
    "cholesky": ("cholesky", {"blocked_min_n": 1, "blocked_max_batch": 0}, {"blocked_min_n": NO_LIMIT}),
    "lu": ("lu", {"gpu_min_n": 1, "gpu_max_batch": 0}, {"gpu_min_n": 0}),
    "trsm": ("trsm", {"gpu_min_n": 1, "gpu_min_rhs": 0, "gpu_max_batch": 0}, {"gpu_min_n": 0}),
}


def sweep(quick=False):
    import torch

    from metal_linalg_amd import _lib, api

    assert torch.cuda.is_available(), "the sweep runs on the GPU"
    ns = {"cholesky": [33, 48, 64, 96, 128] if quick else [33, 48, 64, 80, 96, 112, 128],
          "lu": [16, 32, 64, 128] if quick else [8, 16, 32, 48, 64, 80, 96, 112, 128],
          "trsm": [16, 32, 64, 128] if quick else [8, 16, 32, 48, 64, 80, 96, 112, 128]}
    batches = [1, 4, 16, 64, 256] if quick else [1, 2, 4, 8, 16, 32, 64, 128, 256, 512]
    call = {"cholesky": lambda a, b: api.cholesky(a, False),
            "lu": lambda a, b: api.lu_factor(a),
            "trsm": lambda a, b: api.solve_triangular(a, b, False, False)}
    rng = np.random.default_rng(2024)
    rows = []
    for which in ("cholesky", "lu", "trsm"):
        pol, blocked, batched = FORCE[which]
        saved = _lib.get_policy(pol)
        try:
            for n in ns[which]:
                slow = False   # blocked slower than 4x the batched at a smaller batch: stop timing it
                for batch in batches:
                    a, b = _inputs(torch, which, n, batch, rng)
                    reps = 9 if batch <= 64 else 5
                    _lib.set_policy(pol, batched)
                    tb = _time(lambda: call[which](a, b), reps)
                    tk = float("nan")
                    if not slow:
                        _lib.set_policy(pol, blocked)
                        tk = _time(lambda: call[which](a, b), reps)
                        slow = tk > 4 * tb
                    rows.append((which, n, batch, tb * 1e3, tk * 1e3))
                    print(f"[sweep] {which} n={n} batch={batch}: batched {tb * 1e3:.3f} ms, "
                          f"blocked {tk * 1e3:.3f} ms", flush=True)
        finally:
            _lib.set_policy(pol, saved)
    return rows


def fit(rows, which):
    """(min_n, max_batch) minimising the summed slowdown over the grid."""
    pts = [(n, b, tb, tk) for w, n, b, tb, tk in rows if w == which]
    ns = sorted({p[0] for p in pts})
    bs = sorted({p[1] for p in pts})
    best = None
    for min_n in ns + [NO_LIMIT]:
        for max_b in [0] + bs:
            loss = 0.0
            for n, b, tb, tk in pts:
                blocked = n >= min_n and (max_b == 0 or b <= max_b)
                t = tk if blocked else tb
                fast = tb if not (tk == tk) else min(tb, tk)
                loss += (t / fast) if t == t else 1e9   # NaN: never timed, far slower
            if best is None or loss < best[0] - 1e-12:
                best = (loss, min_n, max_b)
    return best[1], best[2]


def write(rows, stamp):
    with open(CSV, "w") as f:
        f.write("decomposition,n,batch,batched_ms,blocked_ms\n")
        for r in rows:
            f.write(f"{r[0]},{r[1]},{r[2]},{r[3]:.4f},{r[4]:.4f}\n")
    fits = {w: fit(rows, w) for w in ("cholesky", "lu", "trsm")}
    # the blocked path takes every n above the batched kernels' 128 anyway
    val = lambda v: "0xFFFFFFFFu" if v == NO_LIMIT else str(v)
    with open(INC, "w") as f:
        f.write(f"""// The MI355X (gfx950, 256 CUs) rows of the routing policies that choose
// between this build's batched kernels and its one-matrix-at-a-time blocked
// path.  Written by metal_linalg_amd/tuning/sweep.py from its measured
// sweep (metal_linalg_amd/tuning/gfx950_sweep.csv, {stamp}); rerun it to
// refresh.
#pragma once
#include <cstdint>

namespace mla::tuned {{
constexpr uint32_t kCholeskyBlockedMinN = {val(fits['cholesky'][0])};     // CholeskyPolicy.blocked_min_n
constexpr uint32_t kCholeskyBlockedMaxBatch = {val(fits['cholesky'][1])};   // CholeskyPolicy.blocked_max_batch (0: any batch)
constexpr uint32_t kLuBlockedMinN = {val(fits['lu'][0])};           // LuPolicy.gpu_min_n
constexpr uint32_t kLuBlockedMaxBatch = {val(fits['lu'][1])};         // LuPolicy.gpu_max_batch (0: any batch)
constexpr uint32_t kTrsmBlockedMinN = {val(fits['trsm'][0])};         // TrsmPolicy.gpu_min_n
constexpr uint32_t kTrsmBlockedMaxBatch = {val(fits['trsm'][1])};       // TrsmPolicy.gpu_max_batch (0: any batch)
constexpr const char* kSweep = "{stamp}";
}}  // namespace mla::tuned
""")
    return fits


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--quick", action="store_true", help="a smaller grid")
    ap.add_argument("--out-dir", default=None, help="write the .inc and .csv here instead of the package")
    args = ap.parse_args()
    global INC, CSV
    if args.out_dir:
        os.makedirs(args.out_dir, exist_ok=True)
        INC = os.path.join(args.out_dir, "tuned_gfx950.inc")
        CSV = os.path.join(args.out_dir, "gfx950_sweep.csv")
    rows = sweep(args.quick)
    from metal_linalg_amd import _lib

    stamp = f"{datetime.date.today().isoformat()} on {_lib.device_name().decode()} {_lib.hip_arch().decode()}"
    print(write(rows, stamp))


if __name__ == "__main__":
    main()
