// Thin SVD of a single larger matrix (min(M, N) > 64, max(M, N) <= 4096),
// through the symmetric eigensolver of this build.
//
// Role: the MI355X counterpart of the reference's large-matrix SVD routes
// (reference: src/svd.mm:902-1026 routing, src/svd_bidiag.mm for the band /
// bidiagonal regimes), with the contract of core::svd (src/svd.mm:1058-1106):
// s descending and non-negative, U (M x K) and V^T (K x N) with orthonormal
// columns / rows, a non-finite input gives all-NaN outputs and info bit 17,
// otherwise info = 1 | bit 16 (converged) | bit 18 when s_min <= 32
// FLT_EPSILON s_max (the batched kernels' rank-deficient rule).
//
// Method: the tall problem T (m x k, m >= k; a wide A is solved as A^T) is
// embedded in the symmetric (m + k) x (m + k) matrix H = [0 T^T; T 0], whose
// eigenvalues are +-s_i and m - k zeros, with eigenvectors (v_i; u_i) / sqrt 2
// for +s_i (Jordan-Wielandt).  H goes through the blocked tridiagonalisation,
// bisection and inverse iteration of the large eigh path; the k largest
// eigenpairs give s, U and V.  Where the smallest s_i come within the
// solver's grouping distance of zero, +-s_i and the zeros form one close
// group, in which the solver returns some orthonormal basis of the invariant
// subspace: the u and v parts of those columns are not singular vectors.
// They are rebuilt (see svd_large_one): orthonormal completions of the
// well-separated columns, rotated by a small SVD (Rayleigh-Ritz).
#include <algorithm>
#include <cmath>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

// H = [0 T^T; T 0] (n2 = k + m), T row-major m x k
__global__ __launch_bounds__(256) void jw_build_kernel(const float* __restrict__ T, int m, int k,
                                                       float* __restrict__ H) {
    const int n2 = m + k;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n2 * n2) return;
    const int i = (int)(idx / n2), j = (int)(idx - (size_t)i * n2);
    float v = 0.0f;
    if (i >= k && j < k) v = T[(size_t)(i - k) * k + j];
    else if (i < k && j >= k) v = T[(size_t)(j - k) * k + i];
    H[idx] = v;
}

// s_i = max(w[n2-1-i], 0); U[r][i] = sqrt2 Z[k + r][n2-1-i]; V[c][i] (as
// Vt[i][c]) = sqrt2 Z[c][n2-1-i]
__global__ __launch_bounds__(256) void jw_extract_kernel(const float* __restrict__ Z, const float* __restrict__ w,
                                                         int m, int k, float* __restrict__ U, float* __restrict__ Vt,
                                                         float* __restrict__ s) {
    const int n2 = m + k;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const float r2 = 1.41421356237309515f;
    if (idx < (size_t)k) {
        const float x = w[n2 - 1 - (int)idx];
        s[idx] = x != x ? x : fmaxf(x, 0.0f);   // NaN stays NaN
    }
    if (!U) return;
    if (idx < (size_t)m * k) {
        const int r = (int)(idx / k), i = (int)(idx - (size_t)r * k);
        U[idx] = r2 * Z[(size_t)(k + r) * n2 + (n2 - 1 - i)];
    }
    if (idx < (size_t)k * k) {
        const int i = (int)(idx / k), c = (int)(idx - (size_t)i * k);
        Vt[idx] = r2 * Z[(size_t)c * n2 + (n2 - 1 - i)];
    }
}

// Each column of X (rows x cols, row-major) scaled to unit length: an
// eigenvector of H can carry a little of its -s partner, which moves weight
// between its u and v parts without turning either.  One thread per column;
// the loop walks rows, so a wave reads consecutive columns of one row.
__global__ __launch_bounds__(256) void normalize_cols_kernel(float* __restrict__ X, int rows, int cols) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    float ss = 0.0f;
    for (int r = 0; r < rows; ++r) ss = fmaf(X[(size_t)r * cols + c], X[(size_t)r * cols + c], ss);
    const float inv = ss > 0.0f ? 1.0f / sqrtf(ss) : 0.0f;
    for (int r = 0; r < rows; ++r) X[(size_t)r * cols + c] *= inv;
}

// dst[r][c] = src[r][c] for a rows x cols block (row strides lds, ldd)
__global__ __launch_bounds__(256) void copy_block_kernel(const float* __restrict__ src, int lds, float* __restrict__ dst,
                                                         int ldd, int rows, int cols) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rows * cols) return;
    const int r = (int)(idx / cols), c = (int)(idx - (size_t)r * cols);
    dst[(size_t)r * ldd + c] = src[(size_t)r * lds + c];
}

// dst (cols x rows) = src^T (rows x cols)
__global__ __launch_bounds__(256) void transpose_full_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                             int rows, int cols) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = src[(size_t)(r0 + r) * cols + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 32; c += 8)
        if (c0 + c < cols && r0 + tx < rows) dst[(size_t)(c0 + c) * rows + r0 + tx] = tile[tx][c];
}

void transpose_full(const float* src, float* dst, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(transpose_full_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32)), dim3(256), 0,
                       s, src, dst, rows, cols);
}

unsigned blocks(size_t count) { return (unsigned)cdiv(count, 256); }

void copy_block(const float* src, int lds, float* dst, int ldd, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(copy_block_kernel, dim3(blocks((size_t)rows * cols)), dim3(256), 0, s, src, lds, dst, ldd, rows,
                       cols);
}

}  // namespace

bool svd_large_fits(uint32_t m, uint32_t n) {
    const uint32_t l = std::max(m, n), k = std::min(m, n);
    return k >= 1 && qr_blocked_fits(l, k) && eigh_blocked_fits(l + k);
}

size_t svd_large_workspace(uint32_t m, uint32_t n) {
    const size_t l = std::max(m, n), k = std::min(m, n), n2 = l + k;
    size_t floats = eigh_sytrd_floats((uint32_t)n2) + eigh_tridiag_floats((uint32_t)n2);
    floats += 2 * n2 * n2 + n2 + 64;            // H, Z, w
    floats += 4 * l * k + 3 * k * k + 3 * 64 * 64;   // T, U, Q, C, V, Vt', R
    floats += svd_small_workspace(64, 64, 1) / sizeof(float) + 64;
    const size_t qw = qr_blocked_workspace((uint32_t)l, (uint32_t)k) / sizeof(float) + 64;
    return (floats + qw + 16 * 64) * sizeof(float);   // + the 64-float rounding of each piece
}

void svd_large_one(const float* a, float* u, float* s, float* vt, uint32_t* info, float* work, uint32_t M,
                   uint32_t N, hipStream_t st) {
    const bool wide = M < N;
    const int m = (int)(wide ? N : M), k = (int)(wide ? M : N), n2 = m + k;
    const bool vec = u != nullptr;
    float* p = work;
    auto take = [&](size_t floats) {
        float* q = p;
        p += (floats + 63) / 64 * 64;
        return q;
    };
    const EighWork ew = eigh_carve(take(eigh_sytrd_floats((uint32_t)n2) + eigh_tridiag_floats((uint32_t)n2)),
                                   (uint32_t)n2);
    float* H = take((size_t)n2 * n2);
    float* Z = vec ? take((size_t)n2 * n2) : nullptr;
    float* w = take((size_t)n2);
    float* T = take((size_t)m * k);
    float* Ut = take((size_t)m * k);    // the tall problem's U (m x k)
    float* Q = take((size_t)m * k);
    float* Vtt = take((size_t)k * k);   // the tall problem's V^T (k x k)
    float* V = take((size_t)k * k);
    float* R = take((size_t)k * k + 3 * 64 * 64);
    float* C = take((size_t)m * k);
    float* sws = take(svd_small_workspace(64, 64, 1) / sizeof(float) + 64);
    float* qw = take(qr_blocked_workspace((uint32_t)m, (uint32_t)k) / sizeof(float) + 64);
    uint32_t* dinfo = reinterpret_cast<uint32_t*>(take(64));

    const float* tall = a;
    if (wide) {
        transpose_full(a, T, (int)M, (int)N, st);
        tall = T;
    }
    hipLaunchKernelGGL(jw_build_kernel, dim3(blocks((size_t)n2 * n2)), dim3(256), 0, st, tall, m, k, H);
    sytrd_one(H, (uint32_t)n2, true, ew, st);
    eigh_tridiag_one(ew, (uint32_t)n2, w, Z, dinfo, st);
    hipLaunchKernelGGL(jw_extract_kernel, dim3(blocks(std::max((size_t)m * k, (size_t)k * k))), dim3(256), 0, st, Z,
                       w, m, k, vec ? Ut : nullptr, Vtt, s);

    if (vec) {
        hipLaunchKernelGGL(normalize_cols_kernel, dim3(blocks((size_t)k)), dim3(256), 0, st, Ut, m, k);
        transpose_full(Vtt, V, k, k, st);
        hipLaunchKernelGGL(normalize_cols_kernel, dim3(blocks((size_t)k)), dim3(256), 0, st, V, k, k);
    }
    // the host decides: non-finite input, the rank rule, the completion
    uint32_t hinfo = 0;
    std::vector<float> hs((size_t)k);
    MLA_HIP(hipMemcpyAsync(&hinfo, dinfo, sizeof(hinfo), hipMemcpyDeviceToHost, st));
    MLA_HIP(hipMemcpyAsync(hs.data(), s, (size_t)k * sizeof(float), hipMemcpyDeviceToHost, st));
    MLA_HIP(hipStreamSynchronize(st));
    const bool bad = (hinfo >> 17) & 1;
    uint32_t out_info = 1u << 17;
    if (!bad) {
        const float smax = hs[0], smin = hs[(size_t)k - 1];
        out_info = 1u | (1u << 16) | (!(smin > 32.0f * FLT_EPSILON * smax) ? (1u << 18) : 0u);
        // The close group around zero: -s_i, the m - k zeros and +s_i share
        // one group in the eigensolver (which returns some orthonormal basis
        // of it) from the smallest s upwards while the gaps stay below the
        // solver's grouping distance (taken generously, 4e-5 s_max).  Those
        // columns, J = g .. k-1, are rebuilt: V_J and U_J as the orthonormal
        // completions of the other columns' (V_J from the Q of [V_good,
        // V_rest], U_J from the Q of [U_good, A V_J]), then, for up to 64 of
        // them, rotated by the SVD of U_J^T A V_J (Rayleigh-Ritz), which also
        // gives their singular values.
        const float thr = 4e-5f * smax;
        int g = k;
        if (((m > k) ? hs[(size_t)k - 1] : 2.0f * hs[(size_t)k - 1]) <= thr) {
            g = k - 1;
            while (g > 0 && hs[(size_t)g - 1] - hs[(size_t)g] <= thr) --g;
        }
        const int nj = k - g;
        if (vec && nj > 0) {
            qr_blocked(V, Q, R, 1, (uint32_t)k, (uint32_t)k, (uint32_t)k, (uint32_t)k, qw, st);
            copy_block(Q + g, k, V + g, k, k, nj, st);
            sgemm(false, false, m, nj, k, 1.0f, tall, k, 0, V + g, k, 0, 0.0f, C, nj, 0, 1, st);   // A V_J
            copy_block(C, nj, Ut + g, k, m, nj, st);
            qr_blocked(Ut, Q, R, 1, (uint32_t)m, (uint32_t)k, (uint32_t)k, (uint32_t)k, qw, st);
            copy_block(Q + g, k, Ut + g, k, m, nj, st);
            if (nj <= 64) {
                float* Bm = R;                     // nj x nj
                float* P = R + (size_t)nj * nj;    // nj x nj
                float* Pt = P + (size_t)nj * nj;   // nj x nj
                sgemm(true, false, nj, nj, m, 1.0f, Ut + g, k, 0, C, nj, 0, 0.0f, Bm, nj, 0, 1, st);   // U_J^T A V_J
                svd_small(Bm, P, s + g, Pt, dinfo + 1, sws, 1, (uint32_t)nj, (uint32_t)nj, st);
                sgemm(false, false, m, nj, nj, 1.0f, Ut + g, k, 0, P, nj, 0, 0.0f, C, nj, 0, 1, st);
                copy_block(C, nj, Ut + g, k, m, nj, st);
                sgemm(false, true, k, nj, nj, 1.0f, V + g, k, 0, Pt, nj, 0, 0.0f, C, nj, 0, 1, st);
                copy_block(C, nj, V + g, k, k, nj, st);
            }
        }
    }
    if (vec) transpose_full(V, Vtt, k, k, st);
    if (vec) {
        if (wide) {
            transpose_full(Vtt, u, k, k, st);   // A's U (M x k) = V'
            transpose_full(Ut, vt, m, k, st);   // A's V^T (k x N) = U'^T
        } else {
            MLA_HIP(hipMemcpyAsync(u, Ut, (size_t)m * k * sizeof(float), hipMemcpyDeviceToDevice, st));
            MLA_HIP(hipMemcpyAsync(vt, Vtt, (size_t)k * k * sizeof(float), hipMemcpyDeviceToDevice, st));
        }
    }
    MLA_HIP(hipMemcpyAsync(info, &out_info, sizeof(out_info), hipMemcpyHostToDevice, st));
    MLA_HIP(hipStreamSynchronize(st));   // out_info is a host local
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
