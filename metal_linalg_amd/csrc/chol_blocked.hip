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

__global__ __launch_bounds__(256) void chol_diag_kernel(float* __restrict__ W, int ld, int j0, int nb,
                                                        float* __restrict__ X, uint32_t* __restrict__ info) {
    __shared__ float L[NB][NB + 1];
    __shared__ float Xs[NB][NB + 1];
    __shared__ int fail;
    const int t = threadIdx.x;
    for (int idx = t; idx < nb * nb; idx += 256) {
        const int r = idx / nb, c = idx - r * nb;
        L[r][c] = c <= r ? W[(size_t)(j0 + r) * ld + j0 + c] : 0.0f;
        Xs[r][c] = r == c ? 1.0f : 0.0f;
    }
    if (t == 0) fail = 0;
    __syncthreads();
    for (int k = 0; k < nb; ++k) {
        if (t == 0) {
            const float d = L[k][k];
            if (!(d > 0.0f && d <= FLT_MAX) && fail == 0) fail = k + 1;
            L[k][k] = sqrtf(d);
        }
        __syncthreads();
        const float inv = 1.0f / L[k][k];
        for (int r = k + 1 + t; r < nb; r += 256) L[r][k] *= inv;
        __syncthreads();
        const int w = nb - k - 1;
        for (int p = t; p < w * w; p += 256) {
            const int r = k + 1 + p / w, c = k + 1 + p % w;
            if (c <= r) L[r][c] = fmaf(-L[r][k], L[c][k], L[r][c]);
        }
        __syncthreads();
    }
    // X = L^-1: forward substitution on the identity, row k then the rows below
    for (int k = 0; k < nb; ++k) {
        const float inv = 1.0f / L[k][k];
        for (int c = t; c <= k; c += 256) Xs[k][c] *= inv;
        __syncthreads();
        const int w = nb - k - 1, h = k + 1;
        for (int p = t; p < w * h; p += 256) {
            const int i = k + 1 + p / h, c = p % h;
            Xs[i][c] = fmaf(-L[i][k], Xs[k][c], Xs[i][c]);
        }
        __syncthreads();
    }
    for (int idx = t; idx < nb * nb; idx += 256) {
        const int r = idx / nb, c = idx - r * nb;
        if (c <= r) W[(size_t)(j0 + r) * ld + j0 + c] = L[r][c];
        X[(size_t)r * nb + c] = Xs[r][c];
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
