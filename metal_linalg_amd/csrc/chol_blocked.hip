// Blocked Cholesky for large matrices (any n; the large-matrix regime, config
// 5's 4096 x 4096), right-looking in panels of 128 columns.
//
// Role: the MI355X counterpart of the reference's cholesky_blocked
// (reference: src/cholesky_gpu.mm:272-343, kernels shaders/Cholesky.metal:
// 170-208, 355-491, trailing update as MPS C -= A B^T in 512-column blocks,
// :184-198), with the CPU path's contract (src/cholesky_cpu.mm:93-151):
// only the requested triangle is read; info = k + 1 for the first pivot that
// is not positive and finite, and then the output is all NaN; the other
// triangle of the output is zero.
//
// Per panel j (columns j .. j+nb):
//   chol_diag    one workgroup: the nb x nb diagonal block in LDS, factored,
//                and its triangular inverse X = L11^-1 (forward substitution
//                on the identity, rows in parallel)
//   TRSM         L21 = A21 X^T as one MFMA GEMM, in place (one column tile
//                of 128, so each workgroup reads its rows before writing them)
//   SYRK         A22 -= L21 L21^T as an MFMA GEMM over the tiles that reach
//                the lower triangle
// The matrix is first copied (transposed for `upper`) into a working lower
// triangle, and written out at the end with the other triangle zeroed.
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NB = 128;

// dst (n x n) = src or src^T, through 32 x 32 LDS tiles (both sides coalesced).
__global__ __launch_bounds__(256) void copy_transpose_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                             int n, int trans) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
    if (!trans) {
        for (int r = ty; r < 32; r += 8) {
            const int i = by + r, jx = bx + tx;
            if (i < n && jx < n) dst[(size_t)i * n + jx] = src[(size_t)i * n + jx];
        }
        return;
    }
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, jx = bx + tx;
        if (i < n && jx < n) tile[r][tx] = src[(size_t)i * n + jx];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int i = bx + r, jx = by + tx;   // dst row i = src column
        if (i < n && jx < n) dst[(size_t)i * n + jx] = tile[tx][r];
    }
}

// One workgroup factors the nb x nb diagonal block (nb <= 128, padded to 128
// with the identity) and forms the inverse X = L^-1 of its factor in the same
// sweep.  Thread t owns the 8 x 8 blocks at block row bi = t >> 4 and block
// column bj = t & 15 of both A (a[i][j] = A[8 bi + i][8 bj + j]) and X.
//
// Step k: the threads of block column k / 8 publish their A blocks to LDS
// transposed (so column k is contiguous), the threads of block row k / 8
// their X blocks (so row k is contiguous).  With d = A[k][k],
// inv = 1 / sqrt(d) and g = inv^2, every thread then applies
//   a[i][j] -= A[r][k] * lc(c),      x[i][j] -= lc(r) * X[k][c],
//   lc(q) = A[q][k] g (q > k),  1 - inv (q = k),  0 (q < k)
// (r = 8 bi + i, c = 8 bj + j; A[r][k] taken as 0 for r < k).  For the
// columns right of k this is the right-looking update
// A[r][c] -= L[r][k] L[c][k]; on column k it scales to L[r][k] = A[r][k] inv;
// on X it scales row k by inv and performs the forward substitution
// X[r] -= L[r][k] X[k] for the rows below.  Entries above the diagonal of A
// pick up one finite value each (row k, from A[k][k]) that is never read
// again: the output takes the lower triangle, the diagonal from the saved
// pivots.  X stays exactly lower triangular.  The published blocks alternate between two LDS slots, so one
// barrier per step suffices: a slot is rewritten two steps later, after
// every thread has passed the barrier that follows its reads.
//
// The first pivot that is not positive and finite sets info = j0 + k + 1
// (unless an earlier block already set it); the block carries on with NaN,
// which the final extract turns into the all-NaN output.
struct DiagSlot {
    float a[8][NB];   // a[j][r] = A[r][8 kb + j]: block column kb, transposed
    float x[8][NB];   // x[i][c] = X[8 kb + i][c]: block row kb
};

__global__ __launch_bounds__(256) void chol_diag_kernel(float* __restrict__ W, int ld, int j0, int nb,
                                                        float* __restrict__ X, uint32_t* __restrict__ info) {
    __shared__ DiagSlot slot[2];
    __shared__ float piv[NB];
    const int t = threadIdx.x;
    const int bi = t >> 4, bj = t & 15;
    const int r0 = 8 * bi, c0 = 8 * bj;
    float a[8][8], x[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = r0 + i, c = c0 + j;
            // unconditional load from a clamped address, then masked: all 64
            // loads are in flight before the first wait
            const bool in = r < nb && c < nb && c <= r;
            const float v = W[in ? (size_t)(j0 + r) * ld + j0 + c : (size_t)j0 * ld + j0];
            a[i][j] = in ? v : (r == c && (r >= nb || c >= nb) ? 1.0f : 0.0f);
            x[i][j] = r == c ? 1.0f : 0.0f;
        }
    int fail = 0;
    for (int k = 0; k < NB; ++k) {
        DiagSlot& S = slot[k & 1];
        const int kb = k >> 3, kk = k & 7;
        if (bj == kb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                *reinterpret_cast<float4*>(&S.a[j][r0]) = make_float4(a[0][j], a[1][j], a[2][j], a[3][j]);
                *reinterpret_cast<float4*>(&S.a[j][r0 + 4]) = make_float4(a[4][j], a[5][j], a[6][j], a[7][j]);
            }
        }
        if (bi == kb) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                *reinterpret_cast<float4*>(&S.x[i][c0]) = make_float4(x[i][0], x[i][1], x[i][2], x[i][3]);
                *reinterpret_cast<float4*>(&S.x[i][c0 + 4]) = make_float4(x[i][4], x[i][5], x[i][6], x[i][7]);
            }
        }
        __syncthreads();
        const float* colk = S.a[kk];   // column k of A
        const float* rowk = S.x[kk];   // row k of X
        const float d = colk[k];
        if (fail == 0 && !(d > 0.0f && d <= FLT_MAX)) fail = k + 1;
        const float p = sqrtf(d);
        const float inv = 1.0f / p;
        const float g = inv * inv, one = 1.0f - inv;
        if (t == 0) piv[k] = p;
        const float4 cr0 = *reinterpret_cast<const float4*>(&colk[r0]);
        const float4 cr1 = *reinterpret_cast<const float4*>(&colk[r0 + 4]);
        const float4 cc0 = *reinterpret_cast<const float4*>(&colk[c0]);
        const float4 cc1 = *reinterpret_cast<const float4*>(&colk[c0 + 4]);
        const float4 xr0 = *reinterpret_cast<const float4*>(&rowk[c0]);
        const float4 xr1 = *reinterpret_cast<const float4*>(&rowk[c0 + 4]);
        float cr[8] = {cr0.x, cr0.y, cr0.z, cr0.w, cr1.x, cr1.y, cr1.z, cr1.w};
        const float cc[8] = {cc0.x, cc0.y, cc0.z, cc0.w, cc1.x, cc1.y, cc1.z, cc1.w};
        const float xk[8] = {xr0.x, xr0.y, xr0.z, xr0.w, xr1.x, xr1.y, xr1.z, xr1.w};
        float lr[8], lcol[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            lr[q] = r0 + q > k ? cr[q] * g : (r0 + q == k ? one : 0.0f);
            lcol[q] = c0 + q > k ? cc[q] * g : (c0 + q == k ? one : 0.0f);
            cr[q] = r0 + q < k ? 0.0f : cr[q];   // above the diagonal: not an entry of L
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                a[i][j] = fmaf(-cr[i], lcol[j], a[i][j]);
                x[i][j] = fmaf(-lr[i], xk[j], x[i][j]);
            }
    }
    __syncthreads();   // piv complete
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = r0 + i;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = c0 + j;
            if (r < nb && c <= r) W[(size_t)(j0 + r) * ld + j0 + c] = r == c ? piv[r] : a[i][j];
            if (r < nb && c < nb) X[(size_t)r * nb + c] = x[i][j];
        }
    }
    if (t == 0 && fail != 0 && *info == 0) *info = (uint32_t)(j0 + fail);
}

// out = the working lower triangle (or its transpose for `upper`), the
// other triangle zero; all NaN when a pivot failed.
__global__ __launch_bounds__(256) void chol_extract_kernel(const float* __restrict__ W, float* __restrict__ out,
                                                           int n, int upper, const uint32_t* __restrict__ info) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const bool failed = *info != 0;
    if (!upper) {
        for (int r = ty; r < 32; r += 8) {
            const int i = by + r, c = bx + tx;
            if (i < n && c < n) out[(size_t)i * n + c] = failed ? qnan() : (c <= i ? W[(size_t)i * n + c] : 0.0f);
        }
        return;
    }
    // U[i][c] = L[c][i] for c >= i
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, c = bx + tx;   // source element L[i][c]
        if (i < n && c < n) tile[r][tx] = W[(size_t)i * n + c];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int i = bx + r, c = by + tx;   // out[i][c] = L[c][i]
        if (i < n && c < n) out[(size_t)i * n + c] = failed ? qnan() : (c >= i ? tile[tx][r] : 0.0f);
    }
}

__global__ void zero_u32_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

void chol_blocked(const float* a, float* l, uint32_t* info, float* work, float* xinv, uint32_t batch, uint32_t n,
                  bool upper, hipStream_t s) {
    const int nn = (int)n;
    const size_t per = (size_t)n * n;
    const dim3 tiles((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32));
    for (uint32_t b = 0; b < batch; ++b) {
        float* W = work;
        uint32_t* inf = info + b;
        hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, s, inf, 1);
        hipLaunchKernelGGL(copy_transpose_kernel, tiles, dim3(256), 0, s, a + b * per, W, nn, upper ? 1 : 0);
        for (int j = 0; j < nn; j += NB) {
            const int nb = nn - j < NB ? nn - j : NB;
            {
                KernelTimer t("chol_diag", s);
                hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(256), 0, s, W, nn, j, nb, xinv, inf);
                t.stop();
            }
            const int m2 = nn - j - nb;
            if (m2 <= 0) break;
            float* A21 = W + (size_t)(j + nb) * n + j;
            float* A22 = W + (size_t)(j + nb) * n + j + nb;
            // L21 = A21 X^T (in place: one column tile)
            sgemm(false, true, m2, nb, nb, 1.0f, A21, nn, 0, xinv, nb, 0, 0.0f, A21, nn, 0, 1, s);
            // A22 -= L21 L21^T, lower tiles
            sgemm(false, true, m2, m2, nb, -1.0f, A21, nn, 0, A21, nn, 0, 1.0f, A22, nn, 0, 1, s, true);
        }
        hipLaunchKernelGGL(chol_extract_kernel, tiles, dim3(256), 0, s, W, l + b * per, nn, upper ? 1 : 0, inf);
    }
    MLA_HIP(hipGetLastError());
}

size_t chol_blocked_workspace(uint32_t n) { return ((size_t)n * n + (size_t)NB * NB) * sizeof(float); }

}  // namespace mla
