// LU with partial pivoting, and the triangular solves built on it, for
// matrices beyond the register kernels (n > 32; config 5's 4096 x 4096),
// one matrix at a time.
//
// Role: the MI355X counterpart of the reference's blocked LU (reference:
// src/lu_gpu.mm:146-441: panel LU with composed swap lists, L11^-1 A12 for
// the U12 block, trailing A22 -= L21 U12 as a matrix product, look-ahead),
// with the CPU path's contract (src/lu_cpu.mm:72-157): sgetrf's partial
// pivoting (the first entry of largest magnitude, 0-based sequential swaps,
// applied to whole rows), info = k for the first exactly-zero U(k-1, k-1)
// with the factorization completed; solve and inv give all-NaN x for
// info > 0.  Triangular solves (src/trsm.mm:193-206) read one triangle, a
// unit diagonal not at all.
//
// The reference factors its panels on the CPU; here everything stays on the
// GPU.  Per panel of NB = 128 columns (right-looking):
//   lu_leaf      one workgroup of 1024 threads factors a leaf of W columns
//                (rows pc..n-1 held in registers, RPT rows per thread) with
//                two barriers per column: a 64-bit (|pivot| bits, ~row) max
//                reduction picks the pivot, the pivot row and row k are
//                exchanged through LDS; then it applies its W swaps to the
//                rest of the panel and solves U rows of the panel's later
//                columns with its unit L11 (both through LDS staging)
//   sgemm        the rest of the panel: A -= L_leaf U_leaf (MFMA)
//   lu_swap      the panel's swaps on every column outside the panel
//   trsm_block   U12 = L11^-1 A12 (column-parallel, 16-row steps)
//   sgemm        A22 -= L21 U12 (MFMA)
#include <cstring>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NB = 128;                       // panel width
constexpr float kSfmin = 1.17549435e-38f;     // FLT_MIN: sgetf2 divides below it
constexpr uint32_t kMaxBlockedN = 16384;

// ---------------------------------------------------------------------------
// leaf factorization
// ---------------------------------------------------------------------------

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long shfl_xor64(unsigned long long v, int m) {
    const unsigned lo = __shfl_xor((unsigned)(v & 0xffffffffu), m);
    const unsigned hi = __shfl_xor((unsigned)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

// One elimination step of the leaf (column K), a template so that every
// register index is a compile-time constant.
struct LeafShared {
    unsigned long long cand[16];
    float urow[16], krow[16];
    int plist[16];
};

template <int K, int RPT, int W>
__device__ __forceinline__ void leaf_column(float (&a)[RPT][W], LeafShared& S, int t, int lane, int wv, int m,
                                            int& zero_at) {
    unsigned long long best = 0;
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = t + 1024 * q;
        if (li < m && li >= K) {
            const float av = fabsf(a[q][K]);
            const unsigned key = av == av ? __float_as_uint(av) : (li == K ? 0xffffffffu : 0u);
            best = umax64(best, ((unsigned long long)key << 32) | (unsigned)~li);
        }
    }
#pragma unroll
    for (int m2 = 32; m2 >= 1; m2 >>= 1) best = umax64(best, shfl_xor64(best, m2));
    if (lane == 0) S.cand[wv] = best;
    __syncthreads();
    best = S.cand[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) best = umax64(best, S.cand[i]);
    const int p = (int)~(unsigned)(best & 0xffffffffu);
#pragma unroll
    for (int q = 0; q < RPT; ++q)
        if (t + 1024 * q == p) {
#pragma unroll
            for (int c = 0; c < W; ++c) S.urow[c] = a[q][c];
        }
    if (t == K) {
#pragma unroll
        for (int c = 0; c < W; ++c) S.krow[c] = a[0][c];
    }
    __syncthreads();
    const float pv = S.urow[K];
    if (p != K) {
        if (t == K) {
#pragma unroll
            for (int c = 0; c < W; ++c) a[0][c] = S.urow[c];
        }
#pragma unroll
        for (int q = 0; q < RPT; ++q)
            if (t + 1024 * q == p) {
#pragma unroll
                for (int c = 0; c < W; ++c) a[q][c] = S.krow[c];
            }
    }
    if (pv == 0.0f && zero_at == 0) zero_at = K + 1;
    if (t == 0) S.plist[K] = p;
    const bool small = fabsf(pv) < kSfmin;
    const float inv = 1.0f / pv;
    float u[W];
#pragma unroll
    for (int c = K + 1; c < W; ++c) u[c] = S.urow[c];
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = t + 1024 * q;
        if (li < m && li > K) {
            if (pv != 0.0f) a[q][K] = small ? a[q][K] / pv : a[q][K] * inv;
#pragma unroll
            for (int c = K + 1; c < W; ++c) a[q][c] = fmaf(-a[q][K], u[c], a[q][c]);
        }
    }
}

template <int K, int RPT, int W>
struct LeafColumns {
    __device__ __forceinline__ static void run(float (&a)[RPT][W], LeafShared& S, int t, int lane, int wv, int m, int w,
                                               int& zero_at) {
        if constexpr (K < W) {
            if (K < w) {   // uniform
                leaf_column<K, RPT, W>(a, S, t, lane, wv, m, zero_at);
                LeafColumns<K + 1, RPT, W>::run(a, S, t, lane, wv, m, w, zero_at);
            }
        }
    }
};

// Leaf of W columns pc .. pc + w - 1 (w <= W) over rows pc .. n - 1 of the
// row-major n x n matrix A; the panel spans columns pj .. pe - 1.
// Pivot choice, as isamax on the column below the diagonal: the largest
// |a|, the first such row on ties; a NaN never wins, except a NaN in row k
// itself, which stays (the scan compares against it and every comparison
// fails).  Keys: (bits of |a|, ~row) as one 64-bit integer, NaN in row k
// -> all ones, NaN elsewhere -> 0.
template <int RPT, int W>
__global__ __launch_bounds__(1024) void lu_leaf_kernel(float* __restrict__ A, int n, int pc, int pj, int pe, int w,
                                                       uint32_t* __restrict__ piv, uint32_t* __restrict__ info) {
    __shared__ LeafShared S;
    __shared__ int edst[2 * W], esrc[2 * W];
    __shared__ int nent;
    __shared__ float stage[2 * W][NB];
    __shared__ float Ls[W][W + 1];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int m = n - pc;
    float a[RPT][W];
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = t + 1024 * q;
#pragma unroll
        for (int c = 0; c < W; ++c) a[q][c] = (li < m && c < w) ? A[(size_t)(pc + li) * n + pc + c] : 0.0f;
    }
    int zero_at = 0;
    LeafColumns<0, RPT, W>::run(a, S, t, lane, wv, m, w, zero_at);
    // the leaf back to A; pivots (global, 0-based) and info
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = t + 1024 * q;
        if (li < m) {
#pragma unroll
            for (int c = 0; c < W; ++c)
                if (c < w) A[(size_t)(pc + li) * n + pc + c] = a[q][c];
        }
    }
    __syncthreads();   // plist complete
    if (t < w) piv[pc + t] = (uint32_t)(pc + S.plist[t]);
    if (t == 0 && zero_at != 0 && *info == 0) *info = (uint32_t)(pc + zero_at);

    // the other columns of the panel: the leaf's swaps, then (right of the
    // leaf) the W rows of U:  U12 = L11^-1 A12
    const int ncl = pc - pj, ncr = pe - pc - w, nco = ncl + ncr;
    if (nco <= 0) return;   // uniform
    if (t == 0) {
        // compose the sequential swaps (k <-> plist[k]) into (row <- source row)
        int cnt = w;
        for (int e = 0; e < w; ++e) {
            edst[e] = e;
            esrc[e] = e;
        }
        for (int k = 0; k < w; ++k) {
            const int p = S.plist[k];
            if (p == k) continue;
            int ep = -1;
            for (int e = 0; e < cnt; ++e)
                if (edst[e] == p) ep = e;
            if (ep < 0) {
                ep = cnt++;
                edst[ep] = p;
                esrc[ep] = p;
            }
            const int s = esrc[k];
            esrc[k] = esrc[ep];
            esrc[ep] = s;
        }
        nent = cnt;
    }
    if (t < w) {
#pragma unroll
        for (int c = 0; c < W; ++c) Ls[t][c] = a[0][c];
    }
    __syncthreads();
    const int ne = nent;
    for (int idx = t; idx < ne * nco; idx += 1024) {
        const int e = idx / nco, cc = idx - e * nco;
        const int col = cc < ncl ? pj + cc : pc + w + (cc - ncl);
        stage[e][cc] = A[(size_t)(pc + esrc[e]) * n + col];
    }
    __syncthreads();
    if (t < ncr) {
        const int cc = ncl + t;
        float x[W];
#pragma unroll
        for (int i = 0; i < W; ++i) {
            if (i < w) {
                float s = stage[i][cc];
#pragma unroll
                for (int l = 0; l < i; ++l) s = fmaf(-Ls[i][l], x[l], s);
                x[i] = s;
                stage[i][cc] = s;
            }
        }
    }
    __syncthreads();
    for (int idx = t; idx < ne * nco; idx += 1024) {
        const int e = idx / nco, cc = idx - e * nco;
        const int col = cc < ncl ? pj + cc : pc + w + (cc - ncl);
        A[(size_t)(pc + edst[e]) * n + col] = stage[e][cc];
    }
}

// ---------------------------------------------------------------------------
// the panel's swaps (rows pj .. pe - 1, sequential) on the columns outside
// the panel; each workgroup composes them in LDS and moves a 32-column chunk
// ---------------------------------------------------------------------------

constexpr int kSwapCols = 32;

__global__ __launch_bounds__(256) void lu_swap_kernel(float* __restrict__ A, int n, int pj, int pe,
                                                      const uint32_t* __restrict__ piv) {
    __shared__ int src[kMaxBlockedN];   // src[r - pj] = source row of row r (r >= pj)
    __shared__ float stage[2 * NB][kSwapCols + 1];
    const int t = threadIdx.x;
    const int rows = n - pj, nbk = pe - pj;
    for (int i = t; i < rows; i += 256) src[i] = i;
    __syncthreads();
    if (t == 0) {
        for (int k = 0; k < nbk; ++k) {
            const int p = (int)piv[pj + k] - pj;
            const int s = src[k];
            src[k] = src[p];
            src[p] = s;
        }
    }
    __syncthreads();
    // entries: rows pj .. pe - 1, then each swap target below the panel
    // (duplicates rewrite the same value)
    const int nout = n - nbk;   // columns outside the panel
    const int c0 = blockIdx.x * kSwapCols;
    const int ne = 2 * nbk;
    for (int idx = t; idx < ne * kSwapCols; idx += 256) {
        const int e = idx / kSwapCols, cc = idx - e * kSwapCols;
        const int oc = c0 + cc;
        if (oc >= nout) continue;
        const int col = oc < pj ? oc : oc + nbk;
        int dst = e < nbk ? e : (int)piv[pj + e - nbk] - pj;
        if (e >= nbk && dst < nbk) continue;
        stage[e][cc] = A[(size_t)(pj + src[dst]) * n + col];
    }
    __syncthreads();
    for (int idx = t; idx < ne * kSwapCols; idx += 256) {
        const int e = idx / kSwapCols, cc = idx - e * kSwapCols;
        const int oc = c0 + cc;
        if (oc >= nout) continue;
        const int col = oc < pj ? oc : oc + nbk;
        int dst = e < nbk ? e : (int)piv[pj + e - nbk] - pj;
        if (e >= nbk && dst < nbk) continue;
        A[(size_t)(pj + dst) * n + col] = stage[e][cc];
    }
}

// ---------------------------------------------------------------------------
// T X = B for one diagonal block T (nbk <= 128 rows; lower or upper part
// read, the diagonal not read when UNIT), B nbk x ncols in place; a
// workgroup takes 64 columns.  Per 16-row step: 64 threads substitute down
// (or up) the 16 x 16 diagonal sub-block, one column each; then all 256
// threads remove the step's rows from the rest.  Division by the diagonal,
// as BLAS strsm.
// ---------------------------------------------------------------------------

constexpr int kTrsmCols = 64;

template <bool UPPER, bool UNIT>
__global__ __launch_bounds__(256) void trsm_block_kernel(const float* __restrict__ T, int ldt,
                                                         float* __restrict__ B, int ldb, int nbk, int ncols) {
    __shared__ float Ts[NB][NB + 4];
    __shared__ float Bs[NB][kTrsmCols + 1];
    const int t = threadIdx.x;
    const int c0 = blockIdx.x * kTrsmCols;
    const int nsb = (nbk + 15) >> 4, np = nsb * 16;
    for (int idx = t; idx < np * np; idx += 256) {
        const int i = idx / np, l = idx - i * np;
        float v = 0.0f;
        if (i < nbk && l < nbk) {
            const bool in = UPPER ? l >= i : l <= i;
            if (in && !(UNIT && l == i)) v = T[(size_t)i * ldt + l];
        }
        if (l == i && (UNIT || i >= nbk)) v = 1.0f;
        Ts[i][l] = v;
    }
    for (int idx = t; idx < np * kTrsmCols; idx += 256) {
        const int i = idx / kTrsmCols, c = idx - i * kTrsmCols;
        Bs[i][c] = (i < nbk && c0 + c < ncols) ? B[(size_t)i * ldb + c0 + c] : 0.0f;
    }
    __syncthreads();
    for (int s = 0; s < nsb; ++s) {
        const int sb = UPPER ? nsb - 1 - s : s;
        const int i0 = 16 * sb;
        if (t < kTrsmCols) {
            float x[16];
            if (!UPPER) {
#pragma unroll
                for (int ii = 0; ii < 16; ++ii) {
                    float v = Bs[i0 + ii][t];
#pragma unroll
                    for (int l = 0; l < ii; ++l) v = fmaf(-Ts[i0 + ii][i0 + l], x[l], v);
                    x[ii] = UNIT ? v : v / Ts[i0 + ii][i0 + ii];
                    Bs[i0 + ii][t] = x[ii];
                }
            } else {
#pragma unroll
                for (int ii = 15; ii >= 0; --ii) {
                    float v = Bs[i0 + ii][t];
#pragma unroll
                    for (int l = ii + 1; l < 16; ++l) v = fmaf(-Ts[i0 + ii][i0 + l], x[l], v);
                    x[ii] = UNIT ? v : v / Ts[i0 + ii][i0 + ii];
                    Bs[i0 + ii][t] = x[ii];
                }
            }
        }
        __syncthreads();
        const int c = t & (kTrsmCols - 1), rg = t >> 6;
        float xb[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) xb[l] = Bs[i0 + l][c];
        const int r_begin = UPPER ? 0 : i0 + 16;
        const int r_end = UPPER ? i0 : np;
        for (int i = r_begin + rg; i < r_end; i += 4) {
            float v = Bs[i][c];
#pragma unroll
            for (int l = 0; l < 16; l += 4) {
                const float4 tv = *reinterpret_cast<const float4*>(&Ts[i][i0 + l]);
                v = fmaf(-tv.x, xb[l], v);
                v = fmaf(-tv.y, xb[l + 1], v);
                v = fmaf(-tv.z, xb[l + 2], v);
                v = fmaf(-tv.w, xb[l + 3], v);
            }
            Bs[i][c] = v;
        }
        __syncthreads();
    }
    for (int idx = t; idx < nbk * kTrsmCols; idx += 256) {
        const int i = idx / kTrsmCols, c = idx - i * kTrsmCols;
        if (c0 + c < ncols) B[(size_t)i * ldb + c0 + c] = Bs[i][c];
    }
}

// x[i][:] = b[perm[i]][:]; all NaN where the matrix is singular
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ b, float* __restrict__ x,
                                                          const int* __restrict__ perm, int n, int ncols) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * ncols) return;
    const int i = (int)(idx / ncols), c = (int)(idx - (size_t)i * ncols);
    x[idx] = b[(size_t)perm[i] * ncols + c];
}

__global__ __launch_bounds__(256) void nan_if_singular_kernel(float* __restrict__ x, size_t count,
                                                              const uint32_t* __restrict__ info) {
    if (*info == 0) return;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) x[i] = qnan();
}

// x = P I: row i is e_{perm[i]}
__global__ __launch_bounds__(256) void perm_identity_kernel(float* __restrict__ x, const int* __restrict__ perm,
                                                            int n) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (size_t)i * n);
    x[idx] = j == perm[i] ? 1.0f : 0.0f;
}

__global__ void zero_info_kernel(uint32_t* p) { *p = 0; }

template <int RPT, int W>
void launch_leaf(float* A, int n, int pc, int pj, int pe, int w, uint32_t* piv, uint32_t* info, hipStream_t s) {
    hipLaunchKernelGGL((lu_leaf_kernel<RPT, W>), dim3(1), dim3(1024), 0, s, A, n, pc, pj, pe, w, piv, info);
}

// the leaf shape for an n x n factorization: rows per thread and width
void leaf(float* A, int n, int pc, int pj, int pe, uint32_t* piv, uint32_t* info, hipStream_t s, int& width) {
    if (n <= 1024) {
        width = 16;
        launch_leaf<1, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (n <= 2048) {
        width = 16;
        launch_leaf<2, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (n <= 4096) {
        width = 16;
        launch_leaf<4, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (n <= 8192) {
        width = 8;
        launch_leaf<8, 8>(A, n, pc, pj, pe, std::min(8, pe - pc), piv, info, s);
    } else {
        width = 4;
        launch_leaf<16, 4>(A, n, pc, pj, pe, std::min(4, pe - pc), piv, info, s);
    }
}

}  // namespace

bool lu_blocked_fits(uint32_t n) { return n <= kMaxBlockedN; }

// One n x n matrix: lu (in place over a copy of A), pivots, info.
void lu_blocked_one(float* lu, uint32_t* piv, uint32_t* info, int n, hipStream_t s) {
    hipLaunchKernelGGL(zero_info_kernel, dim3(1), dim3(1), 0, s, info);
    for (int pj = 0; pj < n; pj += NB) {
        const int pe = std::min(pj + NB, n);
        {
            KernelTimer tm("lu_leaf", s);
            for (int pc = pj; pc < pe;) {
                int width = 0;
                leaf(lu, n, pc, pj, pe, piv, info, s, width);
                const int w = std::min(width, pe - pc);
                const int mrest = n - pc - w, ncol = pe - pc - w;
                if (mrest > 0 && ncol > 0)
                    sgemm(false, false, mrest, ncol, w, -1.0f, lu + (size_t)(pc + w) * n + pc, n, 0,
                          lu + (size_t)pc * n + pc + w, n, 0, 1.0f, lu + (size_t)(pc + w) * n + pc + w, n, 0, 1, s);
                pc += w;
            }
            tm.stop();
        }
        const int nout = n - (pe - pj);
        if (nout > 0)
            hipLaunchKernelGGL(lu_swap_kernel, dim3((unsigned)cdiv(nout, kSwapCols)), dim3(256), 0, s, lu, n, pj, pe,
                               piv);
        if (pe < n) {
            const int nc = n - pe, nbk = pe - pj;
            hipLaunchKernelGGL((trsm_block_kernel<false, true>), dim3((unsigned)cdiv(nc, kTrsmCols)), dim3(256), 0, s,
                               lu + (size_t)pj * n + pj, n, lu + (size_t)pj * n + pe, n, nbk, nc);
            sgemm(false, false, nc, nc, nbk, -1.0f, lu + (size_t)pe * n + pj, n, 0, lu + (size_t)pj * n + pe, n, 0,
                  1.0f, lu + (size_t)pe * n + pe, n, 0, 1, s);
        }
    }
    MLA_HIP(hipGetLastError());
}

// The row permutation of the whole factorization (perm[i] = the source row
// of row i of P A), from the 0-based sequential swaps: one workgroup.
namespace {
__global__ __launch_bounds__(256) void compose_perm_kernel(const uint32_t* __restrict__ piv, int n,
                                                           int* __restrict__ perm) {
    __shared__ int src[kMaxBlockedN];
    const int t = threadIdx.x;
    for (int i = t; i < n; i += 256) src[i] = i;
    __syncthreads();
    if (t == 0)
        for (int k = 0; k < n; ++k) {
            const int p = (int)piv[k];
            const int s = src[k];
            src[k] = src[p];
            src[p] = s;
        }
    __syncthreads();
    for (int i = t; i < n; i += 256) perm[i] = src[i];
}
}  // namespace

// Triangular solve, one n x n matrix T (row stride ldt) and B (n x nrhs) in
// place: blocks of 128 rows, the diagonal block by trsm_block, the rest of
// the rows by the MFMA GEMM (reads only T's own triangle).
void trsm_blocked_one(const float* T, int ldt, float* B, int n, int nrhs, bool upper, bool unit, hipStream_t s) {
    const unsigned gx = (unsigned)cdiv(nrhs, kTrsmCols);
    KernelTimer tm("trsm_blocked", s);
    if (!upper) {
        for (int b0 = 0; b0 < n; b0 += NB) {
            const int nbk = std::min(NB, n - b0);
            if (unit)
                hipLaunchKernelGGL((trsm_block_kernel<false, true>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            else
                hipLaunchKernelGGL((trsm_block_kernel<false, false>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            const int below = n - b0 - nbk;
            if (below > 0)
                sgemm(false, false, below, nrhs, nbk, -1.0f, T + (size_t)(b0 + nbk) * ldt + b0, ldt, 0,
                      B + (size_t)b0 * nrhs, nrhs, 0, 1.0f, B + (size_t)(b0 + nbk) * nrhs, nrhs, 0, 1, s);
        }
    } else {
        const int nblk = cdiv(n, NB);
        for (int bi = nblk - 1; bi >= 0; --bi) {
            const int b0 = bi * NB, nbk = std::min(NB, n - b0);
            if (unit)
                hipLaunchKernelGGL((trsm_block_kernel<true, true>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            else
                hipLaunchKernelGGL((trsm_block_kernel<true, false>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            if (b0 > 0)
                sgemm(false, false, b0, nrhs, nbk, -1.0f, T + b0, ldt, 0, B + (size_t)b0 * nrhs, nrhs, 0, 1.0f, B,
                      nrhs, 0, 1, s);
        }
    }
    tm.stop();
    MLA_HIP(hipGetLastError());
}

size_t lu_blocked_workspace(uint32_t n) {
    // factor (n x n), pivots (n), permutation (n), info (1), padded
    return ((size_t)n * n + 3 * (size_t)n + 64) * sizeof(float);
}

void lu_blocked_factor(const float* a, float* lu, uint32_t* pivots, uint32_t* info, uint32_t batch, uint32_t n,
                       hipStream_t s) {
    const size_t per = (size_t)n * n;
    MLA_HIP(hipMemcpyAsync(lu, a, batch * per * sizeof(float), hipMemcpyDeviceToDevice, s));
    for (uint32_t b = 0; b < batch; ++b)
        lu_blocked_one(lu + b * per, pivots + (size_t)b * n, info + b, (int)n, s);
}

// X = A^-1 B through the factorization: P A = L U, X = U^-1 L^-1 P B;
// all NaN where info > 0.  b == nullptr: B = I (the inverse).
void lu_blocked_solve(const float* a, const float* b, uint32_t nrhs, float* x, uint32_t* info, float* work,
                      uint32_t batch, uint32_t n, hipStream_t s) {
    const size_t per = (size_t)n * n;
    float* lu = work;
    uint32_t* piv = reinterpret_cast<uint32_t*>(work + per);
    int* perm = reinterpret_cast<int*>(work + per + n);
    for (uint32_t bi = 0; bi < batch; ++bi) {
        MLA_HIP(hipMemcpyAsync(lu, a + bi * per, per * sizeof(float), hipMemcpyDeviceToDevice, s));
        uint32_t* inf = info + bi;
        lu_blocked_one(lu, piv, inf, (int)n, s);
        hipLaunchKernelGGL(compose_perm_kernel, dim3(1), dim3(256), 0, s, piv, (int)n, perm);
        float* xb = x + (size_t)bi * n * nrhs;
        const size_t cnt = (size_t)n * nrhs;
        if (b) {
            hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)cdiv(cnt, 256)), dim3(256), 0, s,
                               b + (size_t)bi * n * nrhs, xb, perm, (int)n, (int)nrhs);
        } else {
            hipLaunchKernelGGL(perm_identity_kernel, dim3((unsigned)cdiv(cnt, 256)), dim3(256), 0, s, xb, perm,
                               (int)n);
        }
        trsm_blocked_one(lu, (int)n, xb, (int)n, (int)nrhs, false, true, s);
        trsm_blocked_one(lu, (int)n, xb, (int)n, (int)nrhs, true, false, s);
        hipLaunchKernelGGL(nan_if_singular_kernel, dim3(256), dim3(256), 0, s, xb, cnt, inf);
    }
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
