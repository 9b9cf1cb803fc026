// Thin SVD of a single larger matrix (beyond the batched windows, max(M, N)
// <= 4096), by bidiagonalisation and the symmetric tridiagonal eigensolver of
// this build.
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
// bidiagonalised, T = Q B P^T (svd_bidiag.hip).  B's singular triplets are
// the eigenpairs of its Golub-Kahan tridiagonal (2k x 2k, zero diagonal,
// off-diagonal d_0, e_0, d_1, ...): eigenvalues +-s_i, eigenvectors
// (v_1, u_1, v_2, u_2, ...) / sqrt 2 for +s_i, computed by the large eigh
// path's bisection and inverse iteration.  U = Q U_B and V = P V_B by the
// reflectors in compact-WY panels on the MFMA GEMM.  Where the smallest s_i
// come within the solver's grouping distance of zero, +-s_i form one close
// group, in which the solver returns some orthonormal basis of the invariant
// subspace: the u and v parts of those columns are not singular vectors.
// They are rebuilt (see svd_large_one): orthonormal completions of the
// well-separated columns, rotated by a small SVD (Rayleigh-Ritz).  The
// earlier route embedded T in the (m + k)-square Jordan-Wielandt matrix
// and tridiagonalised that: eight times the reduction's work at m = k.
#include <algorithm>
#include <cmath>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

// From the Golub-Kahan tridiagonal's eigenpairs (w ascending, all 2k; Z
// 2k x k, the eigenvectors of w[k .. 2k-1]): s_i = max(w[2k-1-i], 0) (NaN
// kept); U[r][i] = sqrt2 Z[2r+1][k-1-i] for r < k (rows k .. m-1 of U zero:
// Q's reflectors fill them); V[c][i] (as Vt[i][c]) = sqrt2 Z[2c][k-1-i]
__global__ __launch_bounds__(256) void tgk_extract_kernel(const float* __restrict__ Z, const float* __restrict__ w,
                                                          int m, int k, float* __restrict__ U, float* __restrict__ Vt,
                                                          float* __restrict__ s) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int n2 = 2 * k;
    const float sq2 = 1.41421356237f;
    if (idx < (size_t)k) {
        const float x = w[n2 - 1 - idx];
        s[idx] = x != x ? x : fmaxf(x, 0.0f);   // a NaN (non-finite input) stays NaN
    }
    if (Z == nullptr) return;
    // Z (2k x k) holds the eigenvectors of w[k .. 2k-1], ascending: that of
    // s_i = w[2k-1-i] is column k-1-i
    if (U && idx < (size_t)m * k) {
        const int r = (int)(idx / k), i = (int)(idx - (size_t)r * k);
        U[idx] = r < k ? sq2 * Z[(size_t)(2 * r + 1) * k + (k - 1 - i)] : 0.0f;
    }
    if (idx < (size_t)k * k) {
        const int i = (int)(idx / k), c = (int)(idx - (size_t)i * k);
        Vt[idx] = sq2 * Z[(size_t)(2 * c) * k + (k - 1 - i)];
    }
}

// Each column of X (rows x cols, row-major) scaled to unit length: an
// eigenvector of the tridiagonal can carry a little of its -s partner, which moves weight
// between its u and v parts without turning either.  One thread per column;
// the loop walks rows, so a wave reads consecutive columns of one row.
// Columns of X (rows x cols, row-major) to unit length (a zero column stays
// zero): a 1024-thread workgroup per 64 columns, 16 row groups of 64 lanes
// (each row of the group read coalesced), the groups' sums of squares added
// in LDS in a fixed order.
__global__ __launch_bounds__(1024) void normalize_cols_kernel(float* __restrict__ X, int rows, int cols) {
    __shared__ float part[16][64];
    __shared__ float inv_s[64];
    const int t = threadIdx.x, cl = t & 63, rg = t >> 6;
    const int c = blockIdx.x * 64 + cl;
    const bool live = c < cols;
    const int cc = live ? c : 0;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int r = rg;
    for (; r + 48 < rows; r += 64) {
        const float a = X[(size_t)r * cols + cc], b = X[(size_t)(r + 16) * cols + cc];
        const float d = X[(size_t)(r + 32) * cols + cc], e = X[(size_t)(r + 48) * cols + cc];
        s0 = fmaf(a, a, s0);
        s1 = fmaf(b, b, s1);
        s2 = fmaf(d, d, s2);
        s3 = fmaf(e, e, s3);
    }
    for (; r < rows; r += 16) {
        const float a = X[(size_t)r * cols + cc];
        s0 = fmaf(a, a, s0);
    }
    part[rg][cl] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (rg == 0) {
        float ss = 0.0f;
#pragma unroll
        for (int g = 0; g < 16; ++g) ss += part[g][cl];
        inv_s[cl] = ss > 0.0f ? 1.0f / sqrtf(ss) : 0.0f;
    }
    __syncthreads();
    if (!live) return;
    const float inv = inv_s[cl];
    for (int rr = rg; rr < rows; rr += 16) X[(size_t)rr * cols + c] *= inv;
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

namespace {

// The fix-up's QR of the tall factor (l x k): blocked to 4096 rows, a tree
// of blocked QRs beyond
bool tall_qr_fits(uint32_t l, uint32_t k) { return qr_blocked_fits(l, k) || qr_tsqr_fits(l, k, k); }

size_t tall_qr_floats(uint32_t l, uint32_t k) {
    const size_t tall = qr_blocked_fits(l, k) ? qr_blocked_workspace(l, k) : qr_tsqr_workspace(l, k, true);
    return std::max(tall, qr_blocked_workspace(k, k)) / sizeof(float) + 64;
}

void tall_qr(const float* a, float* q, float* r, uint32_t l, uint32_t k, float* work, hipStream_t s) {
    if (qr_blocked_fits(l, k)) qr_blocked(a, q, r, 1, l, k, k, k, work, s);
    else qr_tsqr_one(a, q, r, l, k, work, s);
}

}  // namespace

bool svd_large_fits(uint32_t m, uint32_t n) {
    const uint32_t l = std::max(m, n), k = std::min(m, n);
    return k >= 1 && qr_blocked_fits(k, k) && tall_qr_fits(l, k) && eigh_blocked_fits(2 * k);
}

size_t svd_large_workspace(uint32_t m, uint32_t n) {
    const size_t l = std::max(m, n), k = std::min(m, n), n2 = 2 * k;
    size_t floats = bidiag_floats((uint32_t)l, (uint32_t)k) + eigh_tridiag_floats((uint32_t)n2);
    floats += 2 * n2 + n2 * k + n2 + 64;             // the tridiagonal, Z, w
    floats += 4 * l * k + 3 * k * k + 3 * 64 * 64;   // T, U, Q, C, V, Vt', R
    floats += svd_small_workspace(64, 64, 1) / sizeof(float) + 64;
    floats += apply_reflectors_wy_floats((int)l, (int)k) + 64;
    const size_t qw = tall_qr_floats((uint32_t)l, (uint32_t)k);
    return (floats + qw + 20 * 64) * sizeof(float);   // + the 64-float rounding of each piece
}

void svd_large_one(const float* a, float* u, float* s, float* vt, uint32_t* info, float* work, uint32_t M,
                   uint32_t N, hipStream_t st) {
    const bool wide = M < N;
    const int m = (int)(wide ? N : M), k = (int)(wide ? M : N), n2 = 2 * k;
    const bool vec = u != nullptr;
    float* p = work;
    auto take = [&](size_t floats) {
        float* q = p;
        p += (floats + 63) / 64 * 64;
        return q;
    };
    const Bidiag bd = bidiag_carve(take(bidiag_floats((uint32_t)m, (uint32_t)k)), (uint32_t)m, (uint32_t)k);
    EighWork ew{};
    ew.d = take((size_t)n2);
    ew.e = take((size_t)n2);
    ew.flags = bd.flags;
    ew.rest = take(eigh_tridiag_floats((uint32_t)n2));
    float* Z = vec ? take((size_t)n2 * k) : nullptr;
    float* w = take((size_t)n2);
    float* T = take((size_t)m * k);
    float* Ut = take((size_t)m * k);    // the tall problem's U (m x k)
    float* Q = take((size_t)m * k);
    float* Vtt = take((size_t)k * k);   // the tall problem's V^T (k x k)
    float* V = take((size_t)k * k);
    float* R = take((size_t)k * k + 3 * 64 * 64);
    float* C = take((size_t)m * k);
    float* sws = take(svd_small_workspace(64, 64, 1) / sizeof(float) + 64);
    float* wyw = take(apply_reflectors_wy_floats(m, k));
    float* qw = take(tall_qr_floats((uint32_t)m, (uint32_t)k));
    uint32_t* dinfo = reinterpret_cast<uint32_t*>(take(64));

    const float* tall = a;
    if (wide) {
        transpose_full(a, T, (int)M, (int)N, st);
        tall = T;
    }
    bidiag_one(tall, (uint32_t)m, (uint32_t)k, bd, st);
    tgk_build(bd, (uint32_t)k, ew.d, ew.e, st);
    eigh_tridiag_one(ew, (uint32_t)n2, w, Z, dinfo, st, false, (uint32_t)k);   // the k eigenvectors of +s
    hipLaunchKernelGGL(tgk_extract_kernel, dim3(blocks(std::max((size_t)m * k, (size_t)k * k))), dim3(256), 0, st, Z,
                       w, m, k, vec ? Ut : nullptr, Vtt, s);

    if (vec) {
        // B's vectors to unit length (an eigenvector of the tridiagonal can
        // carry a little of its -s partner), then U = Q U_B, V = P V_B
        // (U's rows k .. m-1 are still zero: its first k rows hold the norms)
        hipLaunchKernelGGL(normalize_cols_kernel, dim3((unsigned)cdiv(k, 64)), dim3(1024), 0, st, Ut, k, k);
        transpose_full(Vtt, V, k, k, st);
        hipLaunchKernelGGL(normalize_cols_kernel, dim3((unsigned)cdiv(k, 64)), dim3(1024), 0, st, V, k, k);
        apply_reflectors_wy(bd.VL, m, bd.tauq, k, m, Ut, k, wyw, st);
        apply_reflectors_wy(bd.VR, k, bd.taup, k - 1, k, V, k, wyw, st);
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
        // The close group around zero: -s_i and +s_i share one group in the
        // eigensolver (which returns some orthonormal basis
        // of it) from the smallest s upwards while the gaps stay below the
        // solver's grouping distance (taken generously, 4e-5 s_max).  Those
        // columns, J = g .. k-1, are rebuilt: V_J and U_J as the orthonormal
        // completions of the other columns' (V_J from the Q of [V_good,
        // V_rest], U_J from the Q of [U_good, A V_J]), then, for up to 64 of
        // them, rotated by the SVD of U_J^T A V_J (Rayleigh-Ritz), which also
        // gives their singular values.
        const float thr = 4e-5f * smax;
        int g = k;
        if (2.0f * hs[(size_t)k - 1] <= thr) {
            g = k - 1;
            while (g > 0 && hs[(size_t)g - 1] - hs[(size_t)g] <= thr) --g;
        }
        const int nj = k - g;
        if (vec && nj > 0) {
            qr_blocked(V, Q, R, 1, (uint32_t)k, (uint32_t)k, (uint32_t)k, (uint32_t)k, qw, st);
            copy_block(Q + g, k, V + g, k, k, nj, st);
            sgemm(false, false, m, nj, k, 1.0f, tall, k, 0, V + g, k, 0, 0.0f, C, nj, 0, 1, st);   // A V_J
            copy_block(C, nj, Ut + g, k, m, nj, st);
            tall_qr(Ut, Q, R, (uint32_t)m, (uint32_t)k, qw, st);
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
