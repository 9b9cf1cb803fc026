/* HIP-specific extensions of the MI355X build of metal_linalg.
 *
 * None of these has a counterpart in the reference library's C API; they
 * exist for measurement (per-kernel HIP-event timing, read by bench.py) and
 * for diagnostics.  Programs written against the reference never need them.
 */
#ifndef METAL_LINALG_HIP_EXT_H
#define METAL_LINALG_HIP_EXT_H

#include <stdint.h>

#include "c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Turn per-kernel timing on (1) or off (0).  While on, every kernel launch
 * is bracketed by HIP events on the stream it is launched on, and the elapsed
 * times are summed per kernel name when the call returns. */
void metal_linalg_hip_set_timing(int on);

/* Clear the per-kernel sums. */
void metal_linalg_hip_reset_timing(void);

/* Launch count and summed milliseconds of the kernel `name` since the last
 * reset; returns 0 (and zeros) if it has not run. */
int metal_linalg_hip_kernel_time(const char* name, uint64_t* launches, double* total_ms);

/* The names of the kernels timed since the last reset, one per line. */
const char* metal_linalg_hip_kernel_names(void);

/* The fp32 matrix-core GEMM the blocked factorisations use, on caller
 * buffers (host or device): C = alpha op(A) op(B) + beta C, row-major;
 * op(A) is A (M x K, stored with row stride lda) or, with transa, A^T (A
 * stored K x M); likewise B (K x N) or, with transb, B stored N x K; `batch`
 * products with element strides stride_a/b/c.  Returns a metal_linalg_status
 * value.  For tests and measurement. */
int metal_linalg_hip_sgemm(int transa, int transb, int M, int N, int K, float alpha, const float* A, int lda,
                           long long stride_a, const float* B, int ldb, long long stride_b, float beta, float* C,
                           int ldc, long long stride_c, int batch);

/* The tridiagonal form T = Q^T A Q of one symmetric n x n matrix (the lower
 * triangle read if `lower`, else the upper), as used by the large-matrix
 * eigh: d (n) and e (n - 1), host or device pointers.  Returns a
 * metal_linalg_status value.  For tests. */
int metal_linalg_hip_sytrd(const float* a, uint32_t n, int lower, float* d, float* e);

/* Orders the library's next calls after the work enqueued so far on
 * `stream` (a hipStream_t of the library's device, as void*; NULL is the null
 * stream) without blocking the host: an event recorded on `stream` that the
 * library's own stream waits for.  No counterpart in the reference, whose
 * calls take no stream: it is for frameworks whose kernels produce the
 * inputs on a stream of their own (the PyTorch binding calls it before every
 * operation on ROCm tensors).  The library's calls still return only when
 * their results are complete.  Returns a metal_linalg_status value. */
metal_linalg_status metal_linalg_hip_stream_wait(void* stream);

/* The device's gcnArchName ("" without a GPU). */
const char* metal_linalg_hip_arch(void);

/* metal_linalg_eigh for n <= 64 that allocates nothing.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory while
 * they run (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, results and info words as
 * metal_linalg_eigh, but every non-NULL pointer must be HIP device memory
 * (nothing is staged), and n must be at most 64 (else
 * METAL_LINALG_INVALID_ARGUMENT).  The batched kernel's workspace (and info
 * when `info` is NULL) lives in a fixed 8 MiB device array per GPU, found
 * once per device; a batch larger than it serves (5405 matrices at n = 64
 * with vectors) runs in chunks.  The array keeps the last call's contents
 * and is shared by every call on the GPU: calls that overlapped on one GPU
 * would race (the library serialises its own calls). */
metal_linalg_status metal_linalg_hip_eigh_noalloc(const float* a, uint32_t batch, uint32_t n, int lower,
                                                  float* w, float* v, uint32_t* info);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* METAL_LINALG_HIP_EXT_H */
