// Golub-Kahan bidiagonalisation of one tall matrix on the GPU, for the large
// SVD: T (m x k, m >= k) = Q B P^T with B upper bidiagonal (d on the
// diagonal, e above it), Q = H_0 ... H_{k-1} and P = G_0 ... G_{k-2} products
// of Householder reflectors (LAPACK sgebd2, column by column).
//
// Role: the MI355X counterpart of the reference's bidiagonal stage of its
// large SVD (reference: src/svd_bidiag.mm, shaders/Svd_Bidiag.metal:530-1290,
// which reduce to a band and chase it to bidiagonal form); here a one-stage
// reduction whose per-column matrix-vector products are the HBM-bound part.
//
// Working layout: T's columns contiguous (column-major copy scaled by a
// power of two into [0.5, 1)), so that a column is a coalesced vector and a
// product A v walks rows across the threads.  Per column j, four launches:
//   bd_col      one workgroup: column j (with the previous step's right
//               update applied) -> the left reflector u_j (kept as row j of
//               VL), tau_q, d_j
//   bd_left     a wave per trailing column: the previous right update, then
//               H_j, in one pass; row j's entries after H_j go to rowbuf
//   bd_row      one workgroup: the right reflector v_j from rowbuf (row j of
//               VR, leading 1 at j + 1), tau_p, e_j
//   bd_matvec   x = A v_j over rows j+1 .. m-1 (a thread per row, v_j in
//               LDS); the update A -= tau_p x v_j^T is folded into the next
//               column's bd_col and bd_left, which read every entry anyway
// Reflectors with a tail whose sum of squares is below 2^-80 are the
// identity (the batched kernels' cut-off).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80
constexpr int kColThreads = 1024;

__device__ __forceinline__ float block_sum_1024(float v, float* red) {
    v = wave_sum_f(v);
    const int t = threadIdx.x;
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kColThreads / 64; ++w) s += red[w];
    __syncthreads();
    return s;
}

// flags[0] = bits of max |x| (non-negative floats order as their bits),
// flags[1] = any non-finite entry
__global__ __launch_bounds__(256) void bd_scan_kernel(const float* __restrict__ x, size_t count,
                                                      uint32_t* __restrict__ flags) {
    float m = 0.0f;
    int bad = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) {
        const float v = x[i];
        bad |= !finite_f(v);
        m = fmaxf(m, finite_f(v) ? fabsf(v) : 0.0f);
    }
    m = group_max<64>(m);
    bad = group_or<64>(bad);
    if ((threadIdx.x & 63) == 0) {
        if (m > 0.0f) atomicMax(&flags[0], __float_as_uint(m));
        if (bad) atomicOr(&flags[1], 1u);
    }
}

__global__ void bd_zero_flags_kernel(uint32_t* f) {
    f[0] = 0;
    f[1] = 0;
}

// Ac[c m + r] = T[r k + c] 2^-e (zero for a bad matrix), through 32 x 32 tiles
__global__ __launch_bounds__(256) void bd_load_kernel(const float* __restrict__ T, int m, int k,
                                                      float* __restrict__ Ac, const uint32_t* __restrict__ flags) {
    __shared__ float tile[32][33];
    const bool bad = flags[1] != 0;
    const int e = bad ? 0 : scale_exponent(__uint_as_float(flags[0]));
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8)
        if (r0 + i < m && c0 + tx < k) tile[i][tx] = T[(size_t)(r0 + i) * k + c0 + tx];
    __syncthreads();
    for (int i = ty; i < 32; i += 8)
        if (c0 + i < k && r0 + tx < m) Ac[(size_t)(c0 + i) * m + r0 + tx] = bad ? 0.0f : ldexpf(tile[tx][i], -e);
}

// Column j: the previous right update (a -= tau_p[j-1] x, v_{j-1}[j] = 1),
// then the left reflector over rows j .. m-1.
__global__ __launch_bounds__(kColThreads) void bd_col_kernel(float* __restrict__ Ac, int m, int j,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ taup,
                                                             float* __restrict__ VL, float* __restrict__ tauq,
                                                             float* __restrict__ d) {
    __shared__ float red[kColThreads / 64];
    __shared__ float alpha_s;
    const int t = threadIdx.x;
    float* a = Ac + (size_t)j * m;
    const float tp = j > 0 ? taup[j - 1] : 0.0f;
    float ss = 0.0f;
    for (int r = j + t; r < m; r += kColThreads) {
        float v = a[r];
        if (j > 0) v = fmaf(-tp, x[r], v);
        a[r] = v;
        if (r == j) alpha_s = v;
        else ss = fmaf(v, v, ss);
    }
    ss = block_sum_1024(ss, red);   // its barriers also publish alpha_s
    const float alpha = alpha_s;
    float beta = alpha, tau = 0.0f, scale = 1.0f;
    if (ss >= kTinySumsq) {
        beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
        tau = (beta - alpha) / beta;
        scale = 1.0f / (alpha - beta);
    }
    float* u = VL + (size_t)j * m;
    for (int r = t; r < m; r += kColThreads) u[r] = r < j ? 0.0f : (r == j ? 1.0f : a[r] * scale);
    if (t == 0) {
        tauq[j] = tau;
        d[j] = beta;
    }
}

// Trailing columns c = j+1 .. k-1, a wave each: the previous right update,
// then H_j = I - tau_q u u^T; row j of the result goes to rowbuf.
__global__ __launch_bounds__(256) void bd_left_kernel(float* __restrict__ Ac, int m, int k, int j,
                                                      const float* __restrict__ x, const float* __restrict__ taup,
                                                      const float* __restrict__ VR, const float* __restrict__ VL,
                                                      const float* __restrict__ tauq, float* __restrict__ rowbuf) {
    const int lane = threadIdx.x & 63;
    const int c = j + 1 + blockIdx.x * 4 + (threadIdx.x >> 6);
    if (c >= k) return;
    float* a = Ac + (size_t)c * m;
    const float* u = VL + (size_t)j * m;
    const float tpv = j > 0 ? taup[j - 1] * VR[(size_t)(j - 1) * k + c] : 0.0f;
    float dot = 0.0f;
    for (int r = j + lane; r < m; r += 64) {
        float v = a[r];
        if (j > 0) v = fmaf(-tpv, x[r], v);
        a[r] = v;
        dot = fmaf(u[r], v, dot);
    }
    dot = wave_sum_f(dot);
    const float g = tauq[j] * dot;
    for (int r = j + lane; r < m; r += 64) {
        const float v = fmaf(-g, u[r], a[r]);
        a[r] = v;
        if (r == j) rowbuf[c] = v;
    }
}

// The right reflector from rowbuf[j+1 .. k-1] (row j of the left-updated
// matrix): v_j with its leading 1 at j + 1, tau_p, e_j.
__global__ __launch_bounds__(kColThreads) void bd_row_kernel(const float* __restrict__ rowbuf, int k, int j,
                                                             float* __restrict__ VR, float* __restrict__ taup,
                                                             float* __restrict__ e) {
    __shared__ float red[kColThreads / 64];
    const int t = threadIdx.x;
    float ss = 0.0f;
    for (int c = j + 2 + t; c < k; c += kColThreads) ss = fmaf(rowbuf[c], rowbuf[c], ss);
    ss = block_sum_1024(ss, red);
    const float alpha = rowbuf[j + 1];
    float beta = alpha, tau = 0.0f, scale = 1.0f;
    if (ss >= kTinySumsq) {
        beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
        tau = (beta - alpha) / beta;
        scale = 1.0f / (alpha - beta);
    }
    float* v = VR + (size_t)j * k;
    for (int c = t; c < k; c += kColThreads) v[c] = c <= j ? 0.0f : (c == j + 1 ? 1.0f : rowbuf[c] * scale);
    if (t == 0) {
        taup[j] = tau;
        e[j] = beta;
    }
}

// x[r] = sum_{c > j} A[r][c] v_j[c] for rows r = j+1 .. m-1: a thread per row,
// v_j in LDS, the columns read coalesced across the threads.
__global__ __launch_bounds__(256) void bd_matvec_kernel(const float* __restrict__ Ac, int m, int k, int j,
                                                        const float* __restrict__ VR, float* __restrict__ x) {
    extern __shared__ float vs[];
    const float* v = VR + (size_t)j * k;
    for (int c = threadIdx.x; c < k; c += 256) vs[c] = v[c];
    __syncthreads();
    const int r = j + 1 + blockIdx.x * 256 + threadIdx.x;
    if (r >= m) return;
    float s0 = 0.0f, s1 = 0.0f;
    int c = j + 1;
    for (; c + 1 < k; c += 2) {
        s0 = fmaf(Ac[(size_t)c * m + r], vs[c], s0);
        s1 = fmaf(Ac[(size_t)(c + 1) * m + r], vs[c + 1], s1);
    }
    if (c < k) s0 = fmaf(Ac[(size_t)c * m + r], vs[c], s0);
    x[r] = s0 + s1;
}

// The Golub-Kahan tridiagonal of B (size 2k, zero diagonal): off-diagonal
// d_0, e_0, d_1, e_1, ..., d_{k-1}
__global__ __launch_bounds__(256) void tgk_build_kernel(const float* __restrict__ d, const float* __restrict__ e, int k,
                                                        float* __restrict__ td, float* __restrict__ te) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < 2 * k) td[i] = 0.0f;
    if (i < 2 * k - 1) te[i] = (i & 1) ? e[i >> 1] : d[i >> 1];
}

}  // namespace

size_t bidiag_floats(uint32_t m, uint32_t k) {
    const size_t M = m, K = k;
    // Ac, VL, VR, tau_q, tau_p, d, e, x, rowbuf, flags (each rounded to 64)
    return (M * K + 64) + (K * M + 64) + (K * K + 64) + 4 * (K + 64) + (M + 64) + (K + 64) + 64;
}

Bidiag bidiag_carve(float* base, uint32_t m, uint32_t k) {
    float* p = base;
    auto take = [&](size_t c) {
        float* r = p;
        p += (c + 63) / 64 * 64;
        return r;
    };
    Bidiag b;
    b.Ac = take((size_t)m * k);
    b.VL = take((size_t)k * m);
    b.VR = take((size_t)k * k);
    b.tauq = take(k);
    b.taup = take(k);
    b.d = take(k);
    b.e = take(k);
    b.x = take(m);
    b.rowbuf = take(k);
    b.flags = reinterpret_cast<uint32_t*>(take(64));
    return b;
}

void bidiag_one(const float* T, uint32_t mm, uint32_t kk, const Bidiag& b, hipStream_t s) {
    const int m = (int)mm, k = (int)kk;
    KernelTimer t("svd_bidiag_large", s);
    hipLaunchKernelGGL(bd_zero_flags_kernel, dim3(1), dim3(1), 0, s, b.flags);
    hipLaunchKernelGGL(bd_scan_kernel, dim3((unsigned)std::min<uint64_t>(cdiv((uint64_t)m * k, 256), 2048)),
                       dim3(256), 0, s, T, (size_t)m * k, b.flags);
    hipLaunchKernelGGL(bd_load_kernel, dim3((unsigned)cdiv(k, 32), (unsigned)cdiv(m, 32)), dim3(256), 0, s, T, m, k,
                       b.Ac, b.flags);
    for (int j = 0; j < k; ++j) {
        hipLaunchKernelGGL(bd_col_kernel, dim3(1), dim3(kColThreads), 0, s, b.Ac, m, j, b.x, b.taup, b.VL, b.tauq,
                           b.d);
        if (j + 1 >= k) break;
        hipLaunchKernelGGL(bd_left_kernel, dim3((unsigned)cdiv(k - j - 1, 4)), dim3(256), 0, s, b.Ac, m, k, j, b.x,
                           b.taup, b.VR, b.VL, b.tauq, b.rowbuf);
        hipLaunchKernelGGL(bd_row_kernel, dim3(1), dim3(kColThreads), 0, s, b.rowbuf, k, j, b.VR, b.taup, b.e);
        if (m - j - 1 > 0)
            hipLaunchKernelGGL(bd_matvec_kernel, dim3((unsigned)cdiv(m - j - 1, 256)), dim3(256),
                               (size_t)k * sizeof(float), s, b.Ac, m, k, j, b.VR, b.x);
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

void tgk_build(const Bidiag& b, uint32_t k, float* td, float* te, hipStream_t s) {
    hipLaunchKernelGGL(tgk_build_kernel, dim3((unsigned)cdiv(2 * k, 256)), dim3(256), 0, s, b.d, b.e, (int)k, td, te);
}

}  // namespace mla
