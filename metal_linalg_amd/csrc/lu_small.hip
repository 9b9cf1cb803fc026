// Batched LU with partial pivoting, solve, inverse and triangular solve for
// small matrices (n <= 64), one matrix per lane group of a wave64, in
// registers (a whole wave per matrix at 33 <= n <= 64).
//
// Role: the reference has no batched-small GPU LU or TRSM; its CPU path is
// the contract (reference: src/lu_cpu.mm:72-157, src/trsm.mm:193-206):
// sgetrf's partial pivoting (the first entry of largest magnitude, 0-based
// sequential swaps in `pivots`), info = k for the first exactly-zero U(k-1,
// k-1) with the factorization completed, and for solve/inv a singular
// matrix's x all NaN; strsm's substitution reading one triangle, with a unit
// diagonal not read.
//
// Layout: lane c of a group owns column c of [A | B], A's columns first
// (n padded to a power of two N with the identity), the right-hand sides
// after them (inv: the identity's columns).  At elimination step k lane k
// picks the pivot row from its own column, forms the multipliers and
// broadcasts both through LDS; every lane swaps the two rows in its column
// and updates it.  Back substitution then reads U from LDS.  Right-hand
// sides beyond one group's width are split over blockIdx.y.
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

enum Mode { kFactor = 0, kSolve = 1, kInv = 2 };

constexpr float kSfmin = 1.17549435e-38f;   // FLT_MIN: sgetf2 divides below it

// x[k] <-> x[p] for a runtime p >= k (a select chain: the row index must stay
// a compile-time register index).
template <int K, int N>
__device__ __forceinline__ void swap_rows(float (&x)[N], int p) {
    const float xk = x[K];
    float xp = xk;
#pragma unroll
    for (int r = K + 1; r < N; ++r) xp = (r == p) ? x[r] : xp;
#pragma unroll
    for (int r = K + 1; r < N; ++r) x[r] = (r == p) ? xk : x[r];
    x[K] = xp;
}

template <int K, int N>
__device__ __forceinline__ void lu_step(float (&x)[N], float* col, int* pivsh, int c, int n, int& info,
                                        int& mypiv) {
    if constexpr (K < N) {
        if (c == K) {
            float best = fabsf(x[K]);
            int p = K;
#pragma unroll
            for (int r = K + 1; r < N; ++r) {
                const float a = fabsf(x[r]);
                if (a > best) {
                    best = a;
                    p = r;
                }
            }
            swap_rows<K, N>(x, p);
            const float piv = x[K];
            if (piv != 0.0f) {
                if (fabsf(piv) >= kSfmin) {
                    const float inv = 1.0f / piv;
#pragma unroll
                    for (int r = K + 1; r < N; ++r) x[r] *= inv;
                } else {
#pragma unroll
                    for (int r = K + 1; r < N; ++r) x[r] /= piv;
                }
            }
#pragma unroll
            for (int r = K + 1; r < N; ++r) col[r] = x[r];
            pivsh[K] = p;
            pivsh[N + K] = piv == 0.0f ? 1 : 0;
            mypiv = p;
        }
        wave_lds_sync();
        const int p = pivsh[K];
        if (info == 0 && K < n && pivsh[N + K] != 0) info = K + 1;
        if (c != K) {
            swap_rows<K, N>(x, p);
            if (c > K) {
                const float f = x[K];
#pragma unroll
                for (int r = K + 1; r < N; ++r) x[r] = fmaf(-col[r], f, x[r]);
            }
        }
        wave_lds_sync();
        lu_step<K + 1, N>(x, col, pivsh, c, n, info, mypiv);
    }
}

// G = N lanes (factor) or 2N (A's N columns, then up to N right-hand sides).
template <int N, int MODE>
__global__ __launch_bounds__(64) void lu_small_kernel(const float* __restrict__ A, float* __restrict__ LU,
                                                      uint32_t* __restrict__ pivots, uint32_t* __restrict__ info_out,
                                                      const float* __restrict__ B, float* __restrict__ X,
                                                      uint32_t batch, uint32_t n, uint32_t nrhs) {
    constexpr int G = MODE == kFactor ? N : 2 * N;
    constexpr int MPW = 64 / G;
    __shared__ float col[MPW][N + 4];
    __shared__ int pivsh[MPW][2 * N];
    __shared__ float ush[MODE == kFactor ? 1 : MPW][MODE == kFactor ? 1 : N][N + 1];
    const int lane = threadIdx.x;
    const int c = lane % G;
    const int g = lane / G;
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;
    const int rc = c - N;                                   // right-hand-side column of this lane (if >= 0)
    const int col0 = (int)blockIdx.y * N;                   // first right-hand side of this block
    const int nr = MODE == kInv ? (int)n : (int)nrhs;
    const bool rhs_lane = MODE != kFactor && rc >= 0 && col0 + rc < nr;
    const size_t per = (size_t)n * n;

    float x[N];
    const float* src = A + mat * per;
#pragma unroll
    for (int r = 0; r < N; ++r) {
        float v = 0.0f;
        if (c < N) {
            v = (r == c) ? 1.0f : 0.0f;   // identity padding
            if (live && c < (int)n && r < (int)n) v = src[(size_t)r * n + c];
        } else if (rhs_lane && r < (int)n) {
            if (MODE == kInv) v = (r == col0 + rc) ? 1.0f : 0.0f;
            else if (live) v = B[mat * (size_t)n * nrhs + (size_t)r * nrhs + col0 + rc];
        }
        x[r] = v;
    }

    int info = 0, mypiv = 0;
    lu_step<0, N>(x, col[g], pivsh[g], c, (int)n, info, mypiv);

    if constexpr (MODE == kFactor) {
        if (!live) return;
        if (info_out && c == 0) info_out[mat] = (uint32_t)info;
        if (c >= (int)n) return;
        pivots[mat * n + c] = (uint32_t)mypiv;
        float* dst = LU + mat * per;
#pragma unroll
        for (int r = 0; r < N; ++r)
            if (r < (int)n) dst[(size_t)r * n + c] = x[r];
    } else {
        if (c < N) {
#pragma unroll
            for (int r = 0; r < N; ++r) ush[g][r][c] = x[r];
        }
        wave_lds_sync();
        if (rhs_lane) {
#pragma unroll
            for (int k = N - 1; k >= 0; --k) {
                const float y = x[k] / ush[g][k][k];
                x[k] = y;
#pragma unroll
                for (int r = 0; r < k; ++r) x[r] = fmaf(-ush[g][r][k], y, x[r]);
            }
        }
        if (!live) return;
        if (info_out && c == 0 && blockIdx.y == 0) info_out[mat] = (uint32_t)info;
        if (!rhs_lane) return;
        const int ld = MODE == kInv ? (int)n : (int)nrhs;
        float* dst = X + mat * (size_t)n * ld;
#pragma unroll
        for (int r = 0; r < N; ++r)
            if (r < (int)n) dst[(size_t)r * ld + col0 + rc] = info ? qnan() : x[r];
    }
}

// Triangular solve: lanes [0, N) hold the triangle's columns (identity
// padded, unit diagonal as 1, the other triangle never read), lanes
// [N, 2N) the right-hand sides.
template <int N>
__global__ __launch_bounds__(64) void trsm_small_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ X, uint32_t batch, uint32_t n,
                                                        uint32_t nrhs, int upper, int unit) {
    constexpr int G = 2 * N;
    constexpr int MPW = 64 / G;
    __shared__ float tsh[MPW][N][N + 1];
    const int lane = threadIdx.x;
    const int c = lane % G;
    const int g = lane / G;
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;
    const int rc = c - N;
    const int col0 = (int)blockIdx.y * N;
    const bool rhs_lane = rc >= 0 && col0 + rc < (int)nrhs;
    const size_t per = (size_t)n * n;

    if (c < N) {
        const float* src = A + mat * per;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            float v = (r == c) ? 1.0f : 0.0f;
            if (live && c < (int)n && r < (int)n) {
                const bool in = upper ? r < c : r > c;   // strictly inside the triangle
                if (in) v = src[(size_t)r * n + c];
                else if (r == c) v = unit ? 1.0f : src[(size_t)r * n + c];
                else v = 0.0f;
            }
            tsh[g][r][c] = v;
        }
    }
    float y[N];
#pragma unroll
    for (int r = 0; r < N; ++r)
        y[r] = (live && rhs_lane && r < (int)n) ? B[mat * (size_t)n * nrhs + (size_t)r * nrhs + col0 + rc] : 0.0f;
    wave_lds_sync();
    if (rhs_lane) {
        if (upper) {
#pragma unroll
            for (int k = N - 1; k >= 0; --k) {
                const float v = y[k] / tsh[g][k][k];
                y[k] = v;
#pragma unroll
                for (int r = 0; r < k; ++r) y[r] = fmaf(-tsh[g][r][k], v, y[r]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const float v = y[k] / tsh[g][k][k];
                y[k] = v;
#pragma unroll
                for (int r = k + 1; r < N; ++r) y[r] = fmaf(-tsh[g][r][k], v, y[r]);
            }
        }
    }
    if (!live || !rhs_lane) return;
    float* dst = X + mat * (size_t)n * nrhs;
#pragma unroll
    for (int r = 0; r < N; ++r)
        if (r < (int)n) dst[(size_t)r * nrhs + col0 + rc] = y[r];
}

// 33 <= n <= 64: one matrix per wave, the right-hand sides in LDS.
// ysh[r][j] holds row r of right-hand side j (lane j reads and writes only
// its own column, so the substitutions need no synchronisation); the
// triangle or factor is in LDS by columns (fac[k][r] = LU(r, k)), read as
// broadcasts.  The loops run to n at run time.  The arithmetic is that of
// the kernels above: the swaps composed and applied first, then the same
// multiply-adds and divisions in the same order.
template <int MODE>
__global__ __launch_bounds__(64) void lu_wide_kernel(const float* __restrict__ A, uint32_t* __restrict__ info_out,
                                                     const float* __restrict__ B, float* __restrict__ X,
                                                     uint32_t n, uint32_t nrhs) {
    constexpr int N = 64;
    __shared__ float col[N + 4];
    __shared__ int pivsh[2 * N];
    __shared__ int permsh[N];
    __shared__ float fac[N][N + 1];
    __shared__ float ysh[N][N + 1];
    const int c = threadIdx.x;
    const int nn = (int)n;
    const size_t mat = blockIdx.x;
    const int col0 = (int)blockIdx.y * N;
    const int nr = MODE == kInv ? nn : (int)nrhs;
    const bool rhs_lane = col0 + c < nr;
    const size_t per = (size_t)n * n;

    float x[N];
    const float* src = A + mat * per;
#pragma unroll
    for (int r = 0; r < N; ++r) {
        float v = (r == c) ? 1.0f : 0.0f;   // identity padding
        if (c < nn && r < nn) v = src[(size_t)r * n + c];
        x[r] = v;
    }
    int info = 0, mypiv = 0;
    lu_step<0, N>(x, col, pivsh, c, nn, info, mypiv);
#pragma unroll
    for (int r = 0; r < N; ++r) fac[c][r] = x[r];
    // lane r ends with the source row of position r: the swaps of the
    // pivots, in order, exchanged between lanes k and p
    int src_row = c;
    for (int k = 0; k < nn; ++k) {
        const int p = pivsh[k];
        const int from_p = __shfl(src_row, p, 64);
        const int from_k = __shfl(src_row, k, 64);
        src_row = c == k ? from_p : (c == p ? from_k : src_row);
    }
    permsh[c] = src_row;
    wave_lds_sync();
    const float* bsrc = MODE == kInv ? nullptr : B + mat * (size_t)n * nr;
    for (int r = 0; r < nn; ++r) {
        const int sr = permsh[r];
        float v = 0.0f;
        if (rhs_lane) v = MODE == kInv ? (sr == col0 + c ? 1.0f : 0.0f) : bsrc[(size_t)sr * nr + col0 + c];
        ysh[r][c] = v;
    }
    for (int k = 0; k < nn; ++k) {   // unit lower L
        const float yk = ysh[k][c];
        for (int r = k + 1; r < nn; ++r) ysh[r][c] = fmaf(-fac[k][r], yk, ysh[r][c]);
    }
    for (int k = nn - 1; k >= 0; --k) {   // U
        const float v = ysh[k][c] / fac[k][k];
        ysh[k][c] = v;
        for (int r = 0; r < k; ++r) ysh[r][c] = fmaf(-fac[k][r], v, ysh[r][c]);
    }
    if (info_out && c == 0 && blockIdx.y == 0) info_out[mat] = (uint32_t)info;
    if (!rhs_lane) return;
    float* dst = X + mat * (size_t)n * nr;
    for (int r = 0; r < nn; ++r) dst[(size_t)r * nr + col0 + c] = info ? qnan() : ysh[r][c];
}

// NMAX = 64 or 128 (the triangle's columns c and c + 64 loaded by lane c);
// 64 right-hand sides per workgroup either way.
template <int NMAX>
__global__ __launch_bounds__(64) void trsm_wide_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ X, uint32_t n, uint32_t nrhs, int upper,
                                                       int unit) {
    constexpr int N = 64;
    __shared__ float tsh[NMAX][NMAX + 1];   // tsh[k][r] = T(r, k)
    __shared__ float ysh[NMAX][N + 1];
    const int c = threadIdx.x;
    const int nn = (int)n;
    const size_t mat = blockIdx.x;
    const int col0 = (int)blockIdx.y * N;
    const bool rhs_lane = col0 + c < (int)nrhs;
    const float* src = A + mat * (size_t)n * n;
    const float* bsrc = B + mat * (size_t)n * nrhs;
    for (int r = 0; r < nn; ++r) {
#pragma unroll
        for (int h = 0; h < NMAX / N; ++h) {
            const int cc = c + h * N;
            float v = 0.0f;
            if (cc < nn) {
                const bool in = upper ? r < cc : r > cc;   // strictly inside the triangle
                if (in) v = src[(size_t)r * n + cc];
                else if (r == cc) v = unit ? 1.0f : src[(size_t)r * n + cc];
            }
            tsh[cc][r] = v;
        }
        ysh[r][c] = rhs_lane ? bsrc[(size_t)r * nrhs + col0 + c] : 0.0f;
    }
    wave_lds_sync();
    if (upper) {
        for (int k = nn - 1; k >= 0; --k) {
            const float v = ysh[k][c] / tsh[k][k];
            ysh[k][c] = v;
            for (int r = 0; r < k; ++r) ysh[r][c] = fmaf(-tsh[k][r], v, ysh[r][c]);
        }
    } else {
        for (int k = 0; k < nn; ++k) {
            const float v = ysh[k][c] / tsh[k][k];
            ysh[k][c] = v;
            for (int r = k + 1; r < nn; ++r) ysh[r][c] = fmaf(-tsh[k][r], v, ysh[r][c]);
        }
    }
    if (!rhs_lane) return;
    float* dst = X + mat * (size_t)n * nrhs;
    for (int r = 0; r < nn; ++r) dst[(size_t)r * nrhs + col0 + c] = ysh[r][c];
}

// 65 <= n <= 128, the factorization alone: one matrix per 256-thread
// workgroup, the matrix in LDS (row stride n + 1, 66 KB at n = 128: two
// workgroups per CU).  Per column: the pivot by a tree over the threads that
// keeps isamax's answer (the first row of largest magnitude, the diagonal
// row winning ties and when it holds NaN), the full-row swap, the
// multipliers and the rank-1 update, as in the kernels above.
constexpr int kMidN = 128;

__device__ __forceinline__ void piv_take(float& b, int& i, float ob, int oi, int k) {
    bool take;
    if (i == k) take = ob > b;           // the diagonal row keeps ties and NaN
    else if (oi == k) take = !(b > ob);  // unless strictly exceeded
    else take = ob > b || (ob == b && oi < i);
    if (take) {
        b = ob;
        i = oi;
    }
}

// Solve and inverse (MODE != kFactor) go on in the same workgroup, after
// the one factorization: the swaps composed into one row permutation, then
// the right-hand sides in passes of 4 * (64 / G) columns.  In a pass, each
// wave takes 64 / G columns with G lanes per column; lane q of a column holds
// rows q, q + G, q + 2G, ... in registers, so a substitution step is one
// broadcast of y_k within the column's lanes and up to 128 / G multiply-adds
// per lane, in the order of the kernels above.  Every read of A (into LDS)
// and of the pass's right-hand sides comes before any write of the same
// columns of X, so X may alias A (inv) or B (solve).
template <int MODE, int G>
__global__ __launch_bounds__(256) void lu_mid_kernel(const float* A, float* __restrict__ LU,
                                                     uint32_t* __restrict__ pivots, uint32_t* __restrict__ info_out,
                                                     const float* B, float* X, uint32_t n, uint32_t nrhs) {
    // row stride kLda at every n: a row's offset is a compile-time constant
    // in the unrolled substitutions (an immediate in the LDS instruction)
    constexpr int kLda = kMidN + 1;
    __shared__ float a[kMidN * kLda];
    __shared__ float wb[4];
    __shared__ int wi[4];
    __shared__ float wval[4];
    __shared__ int piv_sh[kMidN];
    __shared__ int perm[kMidN];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int nn = (int)n;
    constexpr int ld = kLda;
    const size_t mat = blockIdx.x;
    const float* src = A + mat * (size_t)n * n;
    for (int e = t; e < nn * nn; e += 256) {
        const int r = e / nn, c = e - r * nn;
        a[r * ld + c] = src[e];
    }
    __syncthreads();
    int info = 0;
    for (int k = 0; k < nn; ++k) {
        float b = -1.0f;
        int bi = 0x7fffffff;
        for (int r = k + t; r < nn; r += 256) {
            const float v = fabsf(a[r * ld + k]);
            if (r == k || v > b) {
                b = v;
                bi = r;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = __shfl_xor(b, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            piv_take(b, bi, ob, oi, k);
        }
        if (lane == 0) {   // each wave's candidate with its signed value, read before any write of this step
            wb[wv] = b;
            wi[wv] = bi;
            wval[wv] = a[(bi < nn ? bi : k) * ld + k];
        }
        __syncthreads();
        // every thread combines the four candidates in the same order
        b = wb[0];
        bi = wi[0];
        float piv = wval[0];
        for (int q = 1; q < 4; ++q) {
            const int before = bi;
            piv_take(b, bi, wb[q], wi[q], k);
            if (bi != before) piv = wval[q];
        }
        const int p = bi;
        if (t == 0) piv_sh[k] = p;
        // rows k and p swapped in every column but k; column k is swapped and
        // scaled by the threads that scale it, and its diagonal entry (the
        // pivot) is written in the update phase, which reads no diagonal
        if (p != k)
            for (int c = t; c < nn; c += 256)
                if (c != k) {
                    const float x = a[k * ld + c];
                    a[k * ld + c] = a[p * ld + c];
                    a[p * ld + c] = x;
                }
        const bool big = fabsf(piv) >= kSfmin;
        const float inv = 1.0f / piv;
        for (int r = k + 1 + t; r < nn; r += 256) {
            const float v = r == p ? a[k * ld + k] : a[r * ld + k];
            a[r * ld + k] = piv == 0.0f ? v : (big ? v * inv : v / piv);
        }
        if (piv == 0.0f && info == 0) info = k + 1;
        __syncthreads();
        if (t == 0) a[k * ld + k] = piv;
        // rows to the four waves in turn, columns to the lanes: a lane's (at
        // most two) columns are the same for every row, so their pivot-row
        // entries are read once, into registers
        {
            const int c0 = k + 1 + lane, c1 = c0 + 64;
            const bool in0 = c0 < nn, in1 = c1 < nn;
            const float u0 = in0 ? a[k * ld + c0] : 0.0f;
            const float u1 = in1 ? a[k * ld + c1] : 0.0f;
            for (int r = k + 1 + wv; r < nn; r += 4) {
                const float lr = a[r * ld + k];
                if (in0) a[r * ld + c0] = fmaf(-lr, u0, a[r * ld + c0]);
                if (in1) a[r * ld + c1] = fmaf(-lr, u1, a[r * ld + c1]);
            }
        }
        __syncthreads();
    }
    if constexpr (MODE == kFactor) {
        if (t == 0 && info_out) info_out[mat] = (uint32_t)info;
        for (int k = t; k < nn; k += 256) pivots[mat * n + k] = (uint32_t)piv_sh[k];
        float* dst = LU + mat * (size_t)n * n;
        for (int e = t; e < nn * nn; e += 256) {
            const int r = e / nn, c = e - r * nn;
            dst[e] = a[r * ld + c];
        }
    } else {
        constexpr int R = kMidN / G;        // rows per lane
        constexpr int CPW = 64 / G;         // columns per wave
        if (t == 0) {   // position r of P b is row perm[r] of b
            for (int r = 0; r < nn; ++r) perm[r] = r;
            for (int k = 0; k < nn; ++k) {
                const int p = piv_sh[k];
                const int x = perm[k];
                perm[k] = perm[p];
                perm[p] = x;
            }
            if (info_out) info_out[mat] = (uint32_t)info;
        }
        __syncthreads();
        const int q = lane % G;             // this lane's rows: q + G i
        const int base = lane - q;          // the column's first lane
        const int nr = MODE == kInv ? nn : (int)nrhs;
        const float* bsrc = MODE == kInv ? nullptr : B + mat * (size_t)n * nr;
        float* dst = X + mat * (size_t)n * nr;
        for (int col0 = 0; col0 < nr; col0 += 4 * CPW) {
            const int j = col0 + wv * CPW + lane / G;
            const bool live = j < nr;
            float y[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int r = G * i + q;
                float v = 0.0f;
                if (live && r < nn) {
                    const int sr = perm[r];
                    v = MODE == kInv ? (sr == j ? 1.0f : 0.0f) : bsrc[(size_t)sr * nr + j];
                }
                y[i] = v;
            }
            // unit lower L: y_r -= L(r, k) y_k for r > k
            // (rows at or past n take part and are never read: no bound per row)
#pragma clang loop unroll(full)
            for (int kk = 0; kk < R; ++kk) {
#pragma clang loop unroll(full)
                for (int s = 0; s < G; ++s) {
                    const int k = G * kk + s;
                    if (k < nn) {
                        const float yk = __shfl(y[kk], base + s, 64);
                        if (q > s) y[kk] = fmaf(-a[(G * kk + q) * ld + k], yk, y[kk]);
#pragma clang loop unroll(full)
                        for (int i = kk + 1; i < R; ++i) y[i] = fmaf(-a[(G * i + q) * ld + k], yk, y[i]);
                    }
                }
            }
            // U: y_k /= U(k, k), then y_r -= U(r, k) y_k for r < k
#pragma clang loop unroll(full)
            for (int kk = R - 1; kk >= 0; --kk) {
#pragma clang loop unroll(full)
                for (int s = G - 1; s >= 0; --s) {
                    const int k = G * kk + s;
                    if (k < nn) {
                        const float yk = __shfl(y[kk], base + s, 64) / a[k * ld + k];
                        if (q == s) y[kk] = yk;
                        if (q < s) y[kk] = fmaf(-a[(G * kk + q) * ld + k], yk, y[kk]);
#pragma clang loop unroll(full)
                        for (int i = 0; i < kk; ++i) y[i] = fmaf(-a[(G * i + q) * ld + k], yk, y[i]);
                    }
                }
            }
            if (live) {
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    const int r = G * i + q;
                    if (r < nn) dst[(size_t)r * nr + j] = info ? qnan() : y[i];
                }
            }
        }
    }
}

template <int N, int MODE>
void launch_lu(const float* a, float* lu, uint32_t* piv, uint32_t* info, const float* b, float* x, uint32_t batch,
               uint32_t n, uint32_t nrhs, hipStream_t s, const char* name) {
    constexpr int G = MODE == kFactor ? N : 2 * N;
    constexpr int MPW = 64 / G;
    const uint32_t chunks = MODE == kSolve ? (uint32_t)cdiv(nrhs, N) : 1;
    KernelTimer t(name, s);
    hipLaunchKernelGGL((lu_small_kernel<N, MODE>), dim3((uint32_t)cdiv(batch, MPW), chunks), dim3(64), 0, s, a, lu,
                       piv, info, b, x, batch, n, nrhs);
    t.stop();
}

template <int MODE>
void dispatch_lu(const float* a, float* lu, uint32_t* piv, uint32_t* info, const float* b, float* x, uint32_t batch,
                 uint32_t n, uint32_t nrhs, hipStream_t s, const char* name) {
    if (n <= 4) launch_lu<4, MODE>(a, lu, piv, info, b, x, batch, n, nrhs, s, name);
    else if (n <= 8) launch_lu<8, MODE>(a, lu, piv, info, b, x, batch, n, nrhs, s, name);
    else if (n <= 16) launch_lu<16, MODE>(a, lu, piv, info, b, x, batch, n, nrhs, s, name);
    else if (n <= 32) launch_lu<32, MODE>(a, lu, piv, info, b, x, batch, n, nrhs, s, name);
    else if constexpr (MODE == kFactor) launch_lu<64, MODE>(a, lu, piv, info, b, x, batch, n, nrhs, s, name);
    else if (n <= 64) {
        const uint32_t chunks = MODE == kSolve ? (uint32_t)cdiv(nrhs, 64) : 1;
        KernelTimer t(name, s);
        hipLaunchKernelGGL((lu_wide_kernel<MODE>), dim3(batch, chunks), dim3(64), 0, s, a, info, b, x, n, nrhs);
        t.stop();
    } else {
        // lanes per right-hand side: fewer columns, more lanes on each
        const uint32_t nr = MODE == kSolve ? nrhs : n;
        KernelTimer t(name, s);
        if (nr <= 16)
            hipLaunchKernelGGL((lu_mid_kernel<MODE, 16>), dim3(batch), dim3(256), 0, s, a, nullptr, nullptr, info, b,
                               x, n, nrhs);
        else if (nr <= 32)
            hipLaunchKernelGGL((lu_mid_kernel<MODE, 8>), dim3(batch), dim3(256), 0, s, a, nullptr, nullptr, info, b,
                               x, n, nrhs);
        else
            hipLaunchKernelGGL((lu_mid_kernel<MODE, 4>), dim3(batch), dim3(256), 0, s, a, nullptr, nullptr, info, b,
                               x, n, nrhs);
        t.stop();
    }
    MLA_HIP(hipGetLastError());
}

template <int N>
void launch_trsm(const float* a, const float* b, float* x, uint32_t batch, uint32_t n, uint32_t nrhs, bool upper,
                 bool unit, hipStream_t s) {
    constexpr int MPW = 64 / (2 * N);
    KernelTimer t("trsm_small", s);
    hipLaunchKernelGGL((trsm_small_kernel<N>), dim3((uint32_t)cdiv(batch, MPW), (uint32_t)cdiv(nrhs, N)), dim3(64),
                       0, s, a, b, x, batch, n, nrhs, upper ? 1 : 0, unit ? 1 : 0);
    t.stop();
}

constexpr uint32_t kMaxGridY = 65535;

}  // namespace

bool lu_small_fits(uint32_t n) { return n >= 1 && n <= 64; }
bool lu_small_factor_fits(uint32_t n) { return n >= 1 && n <= (uint32_t)kMidN; }

void lu_small_factor(const float* a, float* lu, uint32_t* pivots, uint32_t* info, uint32_t batch, uint32_t n,
                     hipStream_t s) {
    if (!lu_small_factor_fits(n)) invalid("[lu_factor] lu_small takes n <= 128");
    if (batch == 0) return;
    if (n > 64) {
        KernelTimer t("lu_small_factor", s);
        hipLaunchKernelGGL((lu_mid_kernel<kFactor, 4>), dim3(batch), dim3(256), 0, s, a, lu, pivots, info, nullptr,
                           nullptr, n, 0u);
        t.stop();
        MLA_HIP(hipGetLastError());
        return;
    }
    dispatch_lu<kFactor>(a, lu, pivots, info, nullptr, nullptr, batch, n, 0, s, "lu_small_factor");
}

void lu_small_solve(const float* a, const float* b, uint32_t nrhs, float* x, uint32_t* info, uint32_t batch,
                    uint32_t n, hipStream_t s) {
    if (!lu_small_factor_fits(n)) invalid("[solve] lu_small takes n <= 128");
    if (batch == 0 || nrhs == 0) return;
    const uint32_t N = n <= 4 ? 4 : n <= 8 ? 8 : n <= 16 ? 16 : n <= 32 ? 32 : 64;
    if (cdiv(nrhs, N) > kMaxGridY) invalid("[solve] too many right-hand sides for one call");
    dispatch_lu<kSolve>(a, nullptr, nullptr, info, b, x, batch, n, nrhs, s, "lu_small_solve");
}

void lu_small_inv(const float* a, float* x, uint32_t* info, uint32_t batch, uint32_t n, hipStream_t s) {
    if (!lu_small_factor_fits(n)) invalid("[inv] lu_small takes n <= 128");
    if (batch == 0) return;
    dispatch_lu<kInv>(a, nullptr, nullptr, info, nullptr, x, batch, n, n, s, "lu_small_inv");
}

void trsm_small(const float* a, const float* b, float* x, uint32_t batch, uint32_t n, uint32_t nrhs, bool upper,
                bool unit, hipStream_t s) {
    if (!lu_small_factor_fits(n)) invalid("[solve_triangular] trsm_small takes n <= 128");
    if (batch == 0 || nrhs == 0) return;
    const uint32_t N = n <= 4 ? 4 : n <= 8 ? 8 : n <= 16 ? 16 : n <= 32 ? 32 : 64;
    if (cdiv(nrhs, N) > kMaxGridY) invalid("[solve_triangular] too many right-hand sides for one call");
    if (n <= 4) launch_trsm<4>(a, b, x, batch, n, nrhs, upper, unit, s);
    else if (n <= 8) launch_trsm<8>(a, b, x, batch, n, nrhs, upper, unit, s);
    else if (n <= 16) launch_trsm<16>(a, b, x, batch, n, nrhs, upper, unit, s);
    else if (n <= 32) launch_trsm<32>(a, b, x, batch, n, nrhs, upper, unit, s);
    else {
        KernelTimer t("trsm_small", s);
        if (n <= 64)
            hipLaunchKernelGGL(trsm_wide_kernel<64>, dim3(batch, (uint32_t)cdiv(nrhs, 64)), dim3(64), 0, s, a, b, x,
                               n, nrhs, upper ? 1 : 0, unit ? 1 : 0);
        else
            hipLaunchKernelGGL(trsm_wide_kernel<kMidN>, dim3(batch, (uint32_t)cdiv(nrhs, 64)), dim3(64), 0, s, a, b,
                               x, n, nrhs, upper ? 1 : 0, unit ? 1 : 0);
        t.stop();
    }
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
