/* metal_linalg C ABI, MI355X (gfx950) build.
 *
 * The same entry points, status codes, enum values, info-word layout and
 * policy-struct layouts as the reference library's C API
 * (reference: include/metal_linalg/c_api.h:19-324), so that a program written
 * against the reference links against libmetal_linalg.so unchanged.  Each
 * declaration below names the reference line it stands in for.
 *
 * Data: float32, row-major, contiguous; a batch is its matrices back to back.
 * The caller owns every buffer.  A pointer may be host memory or HIP device
 * memory (classified per call with hipPointerGetAttributes): device memory is
 * read and written in place, host memory is staged through the device.
 * Every call is synchronous: it returns once its outputs are written.
 * A matrix holding a NaN or an infinity yields NaN output for that matrix
 * only (plus its info bits); it is not an error.
 */
#ifndef METAL_LINALG_C_API_H
#define METAL_LINALG_C_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference: c_api.h:19-24 */
typedef enum metal_linalg_status {
    METAL_LINALG_OK               = 0,
    METAL_LINALG_INVALID_ARGUMENT = 1,  /* NULL buffer with a nonzero count, or a shape no kernel takes */
    METAL_LINALG_RUNTIME_ERROR    = 2,  /* HIP failure, or a finite matrix that failed to converge */
    METAL_LINALG_OUT_OF_MEMORY    = 3
} metal_linalg_status;

/* Message of this thread's latest failure ("" if none); kept until the
 * thread's next failure.  reference: c_api.h:26-28 */
const char* metal_linalg_last_error(void);

/* ---- decompositions ---------------------------------------------------- */

/* Reduced QR, K = min(rows, cols): q [batch, rows, K], r [batch, K, cols].
 * reference: c_api.h:36-37 (core::qr, qr.mm:310-327) */
metal_linalg_status metal_linalg_qr(const float* a, uint32_t batch, uint32_t rows, uint32_t cols,
                                    float* q, float* r);

/* QR modes (numpy/torch naming).  reference: c_api.h:44-48 */
typedef enum metal_linalg_qr_mode {
    METAL_LINALG_QR_REDUCED  = 0,   /* q [b, rows, K],    r [b, K, cols]               */
    METAL_LINALG_QR_R        = 1,   /* r [b, K, cols] only; q may be NULL              */
    METAL_LINALG_QR_COMPLETE = 2,   /* q [b, rows, rows], r [b, rows, cols], zero rows below K */
} metal_linalg_qr_mode;

/* reference: c_api.h:49-50 */
metal_linalg_status metal_linalg_qr_with_mode(const float* a, uint32_t batch, uint32_t rows, uint32_t cols,
                                              metal_linalg_qr_mode mode, float* q, float* r);

/* Symmetric eigendecomposition A = V diag(w) V^T of n x n matrices.  Only the
 * lower triangle is read when `lower` != 0, else only the upper.  w [b, n]
 * ascending; v [b, n, n] eigenvectors as columns, or NULL for values only;
 * info [b] or NULL.  reference: c_api.h:56-57 */
metal_linalg_status metal_linalg_eigh(const float* a, uint32_t batch, uint32_t n, int lower,
                                      float* w, float* v, uint32_t* info);

/* Thin SVD A = U diag(s) Vt, K = min(rows, cols): u [b, rows, K], s [b, K]
 * descending, vt [b, K, cols]; u and vt both NULL for values only.
 * reference: c_api.h:62-63 */
metal_linalg_status metal_linalg_svd(const float* a, uint32_t batch, uint32_t rows, uint32_t cols,
                                     float* u, float* s, float* vt, uint32_t* info);

/* Cholesky A = L L^T reading the lower triangle (upper != 0: the upper, and
 * U = L^T is written).  The unwritten triangle of l is zero.  info [b] or
 * NULL: 0, or k when the leading minor of order k is not positive definite
 * (spotrf's convention; a non-finite pivot counts), and then l is all NaN.
 * reference: c_api.h:70-71 */
metal_linalg_status metal_linalg_cholesky(const float* a, uint32_t batch, uint32_t n, int upper,
                                          float* l, uint32_t* info);

/* P A = L U with partial pivoting (sgetrf's): lu [b, n, n] packed (U on and
 * above the diagonal, unit-L strictly below), pivots [b, n] 0-based
 * sequential row swaps, info [b] or NULL: 0, or k where U(k-1, k-1) == 0.
 * reference: c_api.h:77-78 */
metal_linalg_status metal_linalg_lu_factor(const float* a, uint32_t batch, uint32_t n, float* lu,
                                           uint32_t* pivots, uint32_t* info);

/* A X = B: b, x [b, n, nrhs]; a singular matrix's x is all NaN.
 * reference: c_api.h:82-83 */
metal_linalg_status metal_linalg_solve(const float* a, uint32_t batch, uint32_t n, const float* b,
                                       uint32_t nrhs, float* x, uint32_t* info);

/* A^-1: x [b, n, n]; a singular matrix's x is all NaN.  reference: c_api.h:87 */
metal_linalg_status metal_linalg_inv(const float* a, uint32_t batch, uint32_t n, float* x, uint32_t* info);

/* Triangular solve A X = B reading the lower triangle of a (upper != 0: the
 * upper; unit != 0: diagonal taken as 1 and not read); b, x [b, n, nrhs].
 * reference: c_api.h:92-93 */
metal_linalg_status metal_linalg_solve_triangular(const float* a, uint32_t batch, uint32_t n, const float* b,
                                                  uint32_t nrhs, int upper, int unit, float* x);

/* Info word of eigh / svd: bits 0-15 iterations, bit 16 converged, bit 17
 * non-finite input, bit 18 (svd) rank deficient.  reference: c_api.h:99-102 */
#define METAL_LINALG_INFO_SWEEPS(info)         ((info) & 0xFFFFu)
#define METAL_LINALG_INFO_CONVERGED(info)      (((info) >> 16) & 1u)
#define METAL_LINALG_INFO_NONFINITE(info)      (((info) >> 17) & 1u)
#define METAL_LINALG_INFO_RANK_DEFICIENT(info) (((info) >> 18) & 1u)

/* ---- Metal-buffer helpers ----------------------------------------------
 * Kept for link compatibility only: there are no Metal buffers on this
 * platform.  buffer_contents returns NULL, know_buffer 0, forget_buffer does
 * nothing.  HIP device pointers are accepted directly by every call above.
 * reference: c_api.h:118-130 */
void* metal_linalg_buffer_contents(const void* buffer, uint64_t offset, uint64_t bytes);
int   metal_linalg_know_buffer(const void* contents, const void* buffer);
void  metal_linalg_forget_buffer(const void* contents, const void* buffer);

/* ---- device and routing ------------------------------------------------ */

/* The HIP device's marketing name ("" without a GPU) and its compute-unit
 * count.  reference: c_api.h:138, 149 */
const char* metal_linalg_device_name(void);
uint32_t    metal_linalg_gpu_core_count(void);

/* Calibration notices (stderr, once per decomposition when the device has no
 * measured policy row).  reference: c_api.h:142-148 */
void        metal_linalg_set_calibration_notices(int enabled);
const char* metal_linalg_calibration_message(const char* decomposition);

/* Host threads: kept for API compatibility (the library computes on the GPU
 * only).  reference: c_api.h:154-155 */
void     metal_linalg_set_cpu_threads(uint32_t n);
uint32_t metal_linalg_cpu_threads(void);

/* Per-thread CPU-only flag.  This library has no CPU path: while the flag is
 * set on a thread, the routing queries answer "cpu" and the decompositions on
 * that thread fail with METAL_LINALG_RUNTIME_ERROR instead of using the GPU.
 * reference: c_api.h:160-161 */
void metal_linalg_set_cpu_only(int on);
int  metal_linalg_cpu_only(void);

/* The backend a call of that shape takes under the policy in effect (static
 * strings; the reference's names).  reference: c_api.h:172-179 */
const char* metal_linalg_qr_backend(uint32_t rows, uint32_t cols, uint32_t batch);
const char* metal_linalg_eigh_backend(uint32_t n, uint32_t batch);
const char* metal_linalg_eigvalsh_backend(uint32_t n, uint32_t batch);
const char* metal_linalg_svd_backend(uint32_t rows, uint32_t cols, uint32_t batch);
const char* metal_linalg_svdvals_backend(uint32_t rows, uint32_t cols, uint32_t batch);
const char* metal_linalg_cholesky_backend(uint32_t n, uint32_t batch);
const char* metal_linalg_lu_backend(uint32_t n, uint32_t batch);
const char* metal_linalg_trsm_backend(uint32_t n, uint32_t nrhs, uint32_t batch);

/* Routing policies: field order and meaning as the reference's
 * (reference: c_api.h:186-300).  gpu_cores and concurrent_matrices are
 * informational and ignored by the setters. */
#define METAL_LINALG_NO_LIMIT 0xFFFFFFFFu

typedef struct metal_linalg_qr_policy {
    uint32_t m_crossover_small_batch;
    uint32_t m_crossover_large_batch;
    uint32_t batch_threshold;
    uint32_t gpu_max_k;
    uint32_t gpu_min_batch_times_k;
    uint32_t gpu_min_batch;
    uint32_t gpu_cores;
    uint32_t concurrent_matrices;
    uint32_t gpu_large_min_k;
    uint32_t gpu_large_max_batch;
    uint32_t gpu_min_k;
    uint32_t share_min_batch;
} metal_linalg_qr_policy;

typedef struct metal_linalg_eigh_policy {
    uint32_t simd_max_n;
    uint32_t block_min_n;
    uint32_t block_min_n_batched;
    uint32_t block_min_batch;
    uint32_t gpu_max_n;
    uint32_t gpu_min_batch_times_n;
    uint32_t gpu_min_batch;
    uint32_t gpu_cores;
    uint32_t values_gpu_max_n;
    uint32_t values_gpu_min_batch_times_n;
    uint32_t values_gpu_min_batch;
    uint32_t tridiag_min_n;
    uint32_t values_tridiag_min_n;
    uint32_t ql_min_n;
    uint32_t ql_max_n;
    uint32_t tridiag_max_batch;
    uint32_t values_tridiag_max_batch;
    uint32_t share_min_batch;
    uint32_t gpu_big_batch_max_n;
    uint32_t gpu_big_batch_min;
    uint32_t values_band_min_n;
    uint32_t values_band_width;
    uint32_t band_min_n;
    uint32_t tridiag_batch_min_n;
    uint32_t tridiag_batch_max_n;
    uint32_t tridiag_batch_min_batch;
    uint32_t values_tridiag_batch_min_n;
    uint32_t values_tridiag_batch_max_n;
    uint32_t values_tridiag_batch_min_batch;
    uint32_t share_min_n;
} metal_linalg_eigh_policy;

typedef struct metal_linalg_svd_policy {
    uint32_t qr_min_rows;
    uint32_t qr_min_k;
    uint32_t block_min_k;
    uint32_t block_min_k_batched;
    uint32_t block_min_batch;
    uint32_t gpu_max_k;
    uint32_t gpu_min_batch_times_k;
    uint32_t gpu_min_batch;
    uint32_t gpu_cores;
    uint32_t bidiag_min_k;
    uint32_t values_bidiag_min_k;
    uint32_t bidiag_max_batch;
    uint32_t values_bidiag_max_batch;
    uint32_t gk_min_k;
    uint32_t gk_max_k;
    uint32_t gpu_max_l;
    uint32_t values_gpu_max_k;
    uint32_t values_gpu_min_batch_times_k;
    uint32_t values_gpu_min_batch;
    uint32_t values_gpu_max_l;
    uint32_t share_min_batch;
    uint32_t gpu_big_batch_max_k;
    uint32_t gpu_big_batch_min;
    uint32_t values_band_min_k;
    uint32_t values_band_width;
    uint32_t band_min_k;
    uint32_t bidiag_batch_min_k;
    uint32_t bidiag_batch_max_k;
    uint32_t bidiag_batch_min_batch;
    uint32_t bidiag_batch_max_l;
    uint32_t values_bidiag_batch_min_k;
    uint32_t values_bidiag_batch_max_k;
    uint32_t values_bidiag_batch_min_batch;
    uint32_t values_bidiag_batch_max_l;
    uint32_t share_min_k;
} metal_linalg_svd_policy;

typedef struct metal_linalg_cholesky_policy {
    uint32_t simd_max_n;
    uint32_t blocked_min_n;
    uint32_t blocked_max_batch;
    uint32_t gpu_max_n;
    uint32_t gpu_min_batch_times_n;
    uint32_t gpu_min_batch;
    uint32_t gpu_min_n;
    uint32_t gpu_large_min_n;
    uint32_t gpu_large_max_batch;
    uint32_t gpu_cores;
} metal_linalg_cholesky_policy;

typedef struct metal_linalg_lu_policy {
    uint32_t gpu_min_n;
    uint32_t gpu_max_batch;
    uint32_t gpu_solve_min_rhs;
    uint32_t gpu_cores;
} metal_linalg_lu_policy;

typedef struct metal_linalg_trsm_policy {
    uint32_t gpu_min_n;
    uint32_t gpu_min_rhs;
    uint32_t gpu_max_batch;
    uint32_t gpu_cores;
} metal_linalg_trsm_policy;

/* reference: c_api.h:302-307 */
metal_linalg_qr_policy       metal_linalg_qr_policy_get(void);
metal_linalg_eigh_policy     metal_linalg_eigh_policy_get(void);
metal_linalg_svd_policy      metal_linalg_svd_policy_get(void);
metal_linalg_cholesky_policy metal_linalg_cholesky_policy_get(void);
metal_linalg_lu_policy       metal_linalg_lu_policy_get(void);
metal_linalg_trsm_policy     metal_linalg_trsm_policy_get(void);

/* reference: c_api.h:309-314 */
void metal_linalg_qr_policy_set(const metal_linalg_qr_policy* p);
void metal_linalg_eigh_policy_set(const metal_linalg_eigh_policy* p);
void metal_linalg_svd_policy_set(const metal_linalg_svd_policy* p);
void metal_linalg_cholesky_policy_set(const metal_linalg_cholesky_policy* p);
void metal_linalg_lu_policy_set(const metal_linalg_lu_policy* p);
void metal_linalg_trsm_policy_set(const metal_linalg_trsm_policy* p);

/* "tuned:<device>", "env:<variables>", "user" or
 * "default:untuned-device (<device>)".  reference: c_api.h:316-324 */
const char* metal_linalg_qr_policy_source(void);
const char* metal_linalg_eigh_policy_source(void);
const char* metal_linalg_svd_policy_source(void);
const char* metal_linalg_cholesky_policy_source(void);
const char* metal_linalg_lu_policy_source(void);
const char* metal_linalg_trsm_policy_source(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* METAL_LINALG_C_API_H */
