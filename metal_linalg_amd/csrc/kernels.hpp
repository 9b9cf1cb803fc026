// Launchers of the HIP kernels, called by the buffer core (core.cpp).  Every
// pointer is device memory; every launcher only enqueues work on `s`.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mla {

// ---- QR ----
// Householder QR of `batch` m x n matrices, m, n <= 64: q [batch, m, qc]
// (qc = K, m or 0 for none), r [batch, rr, n] (rr = K or m).
bool qr_small_fits(uint32_t m, uint32_t n, uint32_t qc);
void qr_small(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
              hipStream_t s);

// ---- QR of tall matrices: n <= 64 columns, any m >= n rows, batched ----
// Reduced mode (q [batch, m, n]) or R alone (q NULL); r [batch, n, n].
// work = qr_tall_workspace(m, n, batch, q != NULL) bytes (none up to 128 rows).
bool qr_tall_fits(uint32_t m, uint32_t n, uint32_t qc);
size_t qr_tall_workspace(uint32_t m, uint32_t n, uint32_t batch, bool with_q);
void qr_tall(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, float* work,
             hipStream_t s);

// ---- QR of the mid-size window: m, n <= 128 (one above 64), batched ----
// Reduced mode (q [batch, m, min(m, n)]) or R alone (q NULL); r [batch, min(m, n), n].
bool qr_mid_fits(uint32_t m, uint32_t n, uint32_t qc);
void qr_mid(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, hipStream_t s);

// ---- QR for larger matrices (m <= 4096), one matrix at a time ----
// work = qr_blocked_workspace(m, n) bytes; q may be NULL when qc = 0.
bool qr_blocked_fits(uint32_t m, uint32_t n);
size_t qr_blocked_workspace(uint32_t m, uint32_t n);
void qr_blocked(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
                float* work, hipStream_t s);

// ---- QR of one matrix beyond the blocked QR's rows (m > 4096, n <= 2048), a tree of blocked QRs ----
// q (m x n) or NULL for R alone; r n x n; work = qr_tsqr_workspace(m, n, q != NULL) bytes.
bool qr_tsqr_fits(uint32_t m, uint32_t n, uint32_t qc);
size_t qr_tsqr_workspace(uint32_t m, uint32_t n, bool with_q);
void qr_tsqr_one(const float* a, float* q, float* r, uint32_t m, uint32_t n, float* work, hipStream_t s);

// ---- Cholesky, n <= 32 ----
bool chol_small_fits(uint32_t n);
void chol_small(const float* a, float* l, uint32_t* info, uint32_t batch, uint32_t n, bool upper, hipStream_t s);

// Blocked Cholesky, any n, one matrix at a time: work = chol_blocked_workspace(n)
// bytes (n x n working copy + the 128 x 128 triangular inverse).  `info` must
// be device memory (never NULL).
size_t chol_blocked_workspace(uint32_t n);
void chol_blocked(const float* a, float* l, uint32_t* info, float* work, float* xinv, uint32_t batch, uint32_t n,
                  bool upper, hipStream_t s);

// ---- LU, solve, inverse, triangular solve, n <= 32 ----
bool lu_small_fits(uint32_t n);
bool lu_small_factor_fits(uint32_t n);   // factor, solve, inverse, triangular solve: n <= 128
void lu_small_factor(const float* a, float* lu, uint32_t* pivots, uint32_t* info, uint32_t batch, uint32_t n,
                     hipStream_t s);
void lu_small_solve(const float* a, const float* b, uint32_t nrhs, float* x, uint32_t* info, uint32_t batch,
                    uint32_t n, hipStream_t s);
void lu_small_inv(const float* a, float* x, uint32_t* info, uint32_t batch, uint32_t n, hipStream_t s);
void trsm_small(const float* a, const float* b, float* x, uint32_t batch, uint32_t n, uint32_t nrhs, bool upper,
                bool unit, hipStream_t s);

// ---- LU and triangular solves for larger n (<= 16384), one matrix at a time ----
// `info` must be device memory (never NULL); work = lu_blocked_workspace(n) bytes.
bool lu_blocked_fits(uint32_t n);
size_t lu_blocked_workspace(uint32_t n);   // solve / inv
size_t lu_panel_workspace(uint32_t n);     // lu_factor
void lu_blocked_factor(const float* a, float* lu, uint32_t* pivots, uint32_t* info, float* work, uint32_t batch,
                       uint32_t n, hipStream_t s);
// X = A^-1 B (b == nullptr: X = A^-1), all NaN where info > 0
void lu_blocked_solve(const float* a, const float* b, uint32_t nrhs, float* x, uint32_t* info, float* work,
                      uint32_t batch, uint32_t n, hipStream_t s);
// B := T^-1 B in place for one n x n triangle T (row stride ldt), B n x nrhs
void trsm_blocked_one(const float* T, int ldt, float* B, int n, int nrhs, bool upper, bool unit, hipStream_t s);

// ---- symmetric eigendecomposition, n <= 64 ----
bool eigh_small_fits(uint32_t n);
// Bytes of device workspace eigh_small needs (0 without vectors or for n <= 32).
size_t eigh_small_workspace(uint32_t n, uint32_t batch, bool vectors);
void eigh_small(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
                hipStream_t s);

// ---- symmetric eigendecomposition, 65 <= n <= 128, batched ----
bool eigh_mid_fits(uint32_t n);
// Bytes of device workspace eigh_mid needs (0 without vectors).
size_t eigh_mid_workspace(uint32_t n, uint32_t batch, bool vectors);
void eigh_mid(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
              hipStream_t s);

// ---- symmetric eigendecomposition for larger n (<= 16384), one matrix at a time ----
struct EighWork {
    float *A, *V, *W, *abuf, *y, *partA, *partB, *d, *e, *tau;
    uint32_t* flags;   // [0] bits of max |a| over the read triangle, [1] non-finite
    float* rest;       // what follows stage 1's part of the workspace
};
bool eigh_blocked_fits(uint32_t n);
size_t eigh_sytrd_floats(uint32_t n);                 // stage 1's part of the workspace
EighWork eigh_carve(float* base, uint32_t n);
void sytrd_one(const float* a, uint32_t n, bool lower, const EighWork& w, hipStream_t s);
// y = x * 2^e (the scale stage 1 took out), or NaN for a non-finite matrix
void eigh_unscale(const float* x, float* y, uint32_t count, const uint32_t* flags, hipStream_t s);
// stages 2 and 3 after sytrd_one: eigenvalues (ascending, all n), the
// eigenvectors of eigenvalues il .. n-1 if v_out (n x (n - il), ascending),
// info; the workspace after stage 1's holds eigh_tridiag_floats(n)
size_t eigh_tridiag_floats(uint32_t n);
void eigh_tridiag_one(const EighWork& w, uint32_t n, float* w_out, float* v_out, uint32_t* info, hipStream_t s,
                      bool backtransform = true, uint32_t il = 0);
// Z (rows x cols, row-major) <- H_0 H_1 ... H_{nrefl-1} Z with H_j = I -
// tau_j v_j v_j^T, v_j row j of V (stride ldv, zero before its leading 1),
// in compact-WY panels on the MFMA GEMM; work = apply_reflectors_wy_floats.
size_t apply_reflectors_wy_floats(int rows, int cols);
void apply_reflectors_wy(const float* V, int ldv, const float* tau, int nrefl, int rows, float* Z, int cols,
                         float* work, hipStream_t s);

// Golub-Kahan bidiagonalisation of one tall matrix (m x k, m >= k), for the
// large SVD: T = Q B P^T, B upper bidiagonal (d, e), the reflectors of Q as
// the rows of VL (leading 1 at j) with tauq, those of P as the rows of VR
// (leading 1 at j + 1) with taup; B is T's scaled by 2^-e (flags[0] = bits
// of max |T|, flags[1] = a non-finite entry, which zeroes the work).
struct Bidiag {
    float *Ac, *VL, *VR, *tauq, *taup, *d, *e, *x, *rowbuf;
    uint32_t* flags;
};
size_t bidiag_floats(uint32_t m, uint32_t k);
Bidiag bidiag_carve(float* base, uint32_t m, uint32_t k);
void bidiag_one(const float* T, uint32_t m, uint32_t k, const Bidiag& b, hipStream_t s);
// the Golub-Kahan tridiagonal of B (2k x 2k, zero diagonal td, off-diagonal
// te = d_0, e_0, d_1, ..., d_{k-1})
void tgk_build(const Bidiag& b, uint32_t k, float* td, float* te, hipStream_t s);

// One m x n matrix beyond the batched windows (max(m, n) <= 4096):
// bidiagonalisation, the Golub-Kahan tridiagonal's eigenpairs, the
// reflectors' back-transforms; work = svd_large_workspace(m, n) bytes.
bool svd_large_fits(uint32_t m, uint32_t n);
size_t svd_large_workspace(uint32_t m, uint32_t n);
void svd_large_one(const float* a, float* u, float* s, float* vt, uint32_t* info, float* work, uint32_t m,
                   uint32_t n, hipStream_t st);

// ---- thin SVD, min(m, n) <= 64, max(m, n) <= 128, batched ----
bool svd_small_fits(uint32_t m, uint32_t n);
size_t svd_small_workspace(uint32_t m, uint32_t n, uint32_t batch);   // bytes
void svd_small(const float* a, float* u, float* s, float* vt, uint32_t* info, float* ws, uint32_t batch, uint32_t m,
               uint32_t n, hipStream_t st);

// ---- thin SVD, 65 <= min(m, n) <= 128 and max(m, n) <= 128, batched ----
// One-sided Jacobi in LDS; u and vt both or neither; no workspace.
bool svd_mid_fits(uint32_t m, uint32_t n);
void svd_mid(const float* a, float* u, float* s, float* vt, uint32_t* info, uint32_t batch, uint32_t m, uint32_t n,
             hipStream_t st);

// ---- fp32 MFMA GEMM: C = alpha op(A) op(B) + beta C, row-major, strided batches ----
// k_last >= 0: the last batch entry's K (a split-K batch whose tail is shorter)
void sgemm(bool ta, bool tb, int M, int N, int K, float alpha, const float* A, int lda, long long sa,
           const float* B, int ldb, long long sb, float beta, float* C, int ldc, long long sc, int batch,
           hipStream_t s, bool lower_only = false, int k_last = -1);

}  // namespace mla
