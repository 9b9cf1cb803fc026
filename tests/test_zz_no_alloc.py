"""metal_linalg_hip_eigh_noalloc (include/metal_linalg/hip_ext.h), the
entry point that allocates nothing, against metal_linalg_eigh through the C
ABI on the same device buffers: eigenvalues, eigenvectors and info words
identical bit for bit (same kernels, same order), on two calls in a row, the
second with a smaller input.  The first call's batch is larger than one
chunk of the fixed device array (5405 matrices at n = 64 with vectors), so
the chunked path runs; the second, smaller, call finds the array holding the
first call's contents."""

import ctypes

import numpy as np
import pytest

from _util import config2_eigh, to_np

pytestmark = pytest.mark.gpu


def run(lib, fn, a, batch, n, lower, vectors, with_info, torch):
    w = torch.empty((batch, n), dtype=torch.float32, device="cuda")
    v = torch.empty((batch, n, n), dtype=torch.float32, device="cuda") if vectors else None
    info = torch.empty(batch, dtype=torch.int32, device="cuda") if with_info else None
    with lib.lock:
        rc = fn(a.data_ptr(), batch, n, int(lower), w.data_ptr(), v.data_ptr() if v is not None else None,
                info.data_ptr() if info is not None else None)
    torch.cuda.synchronize()
    assert rc == lib.OK, lib.last_error()
    return to_np(w), (to_np(v) if v is not None else None), (to_np(info) if info is not None else None)


def same(x, y):
    return x is None and y is None or np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("n,vectors,with_info", [(64, True, True), (64, True, False), (48, False, True),
                                                 (16, True, True)])
def test_noalloc_matches_eigh(cuda, lib, n, vectors, with_info):
    torch = cuda
    for batch, seed in ((6000 if n == 64 else 3000, 2), (37, 9)):   # second call smaller
        a = torch.from_numpy(config2_eigh(batch=batch, n=n, seed=seed)).to("cuda")
        print(f"[noalloc] n={n} vectors={vectors} info={with_info} batch={batch}", flush=True)
        ref = run(lib, lib.eigh, a, batch, n, True, vectors, with_info, torch)
        got = run(lib, lib.hip_eigh_noalloc, a, batch, n, True, vectors, with_info, torch)
        for x, y in zip(got, ref):
            assert same(x, y)


def test_noalloc_rejects(cuda, lib):
    torch = cuda
    a = torch.zeros((2, 65, 65), dtype=torch.float32, device="cuda")
    w = torch.empty((2, 65), dtype=torch.float32, device="cuda")
    assert lib.hip_eigh_noalloc(a.data_ptr(), 2, 65, 1, w.data_ptr(), None, None) == lib.INVALID_ARGUMENT
    assert b"n <= 64" in lib.last_error()
    host = np.zeros((2, 8, 8), np.float32)
    wh = torch.empty((2, 8), dtype=torch.float32, device="cuda")
    rc = lib.hip_eigh_noalloc(host.ctypes.data, 2, 8, 1, wh.data_ptr(), None, None)
    assert rc == lib.INVALID_ARGUMENT and b"device memory" in lib.last_error()
    assert lib.hip_eigh_noalloc(None, 0, 8, 1, None, None, None) == lib.OK
