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
// product A v walks rows across the threads.  Per column j, three launches:
//   bd_col      one workgroup: column j (with the previous step's right
//               update applied) -> the left reflector u_j (kept as row j of
//               VL), tau_q, d_j
//   bd_left     a workgroup per trailing column, held in registers: the
//               previous right update, then H_j; row j's entries after H_j
//               go to rowbuf
//   bd_matvec   the right reflector v_j from rowbuf (every workgroup forms
//               it; the first records it as row j of VR with tau_p, e_j),
//               then x = A v_j over rows j+1 .. m-1 (a workgroup per 32-row
//               tile, all columns); the update A -= tau_p x v_j^T is folded
//               into the next column's bd_col and bd_left, which read every
//               entry anyway
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
constexpr int kMvBatch = 8;   // loads in flight per lane in the matrix-vector product

// the working copy's column stride: m rounded up to an odd number of 64-row
// blocks (16-byte loads; columns a power of two apart share memory channels)
size_t bidiag_ld(uint32_t m) { return (cdiv(m, 64) | 1) * 64; }

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

// Ac[c ld + r] = T[r k + c] 2^-e (zero for a bad matrix, and in the pad rows
// m .. ld-1), through 32 x 32 tiles
__global__ __launch_bounds__(256) void bd_load_kernel(const float* __restrict__ T, int m, int k, int ld,
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
        if (c0 + i < k && r0 + tx < ld)
            Ac[(size_t)(c0 + i) * ld + r0 + tx] = bad || r0 + tx >= m ? 0.0f : ldexpf(tile[tx][i], -e);
}

// Column j: the previous right update (a -= tau_p[j-1] x, v_{j-1}[j] = 1),
// then the left reflector over rows j .. m-1.
__global__ __launch_bounds__(kColThreads) void bd_col_kernel(float* __restrict__ Ac, int m, int ld, int j,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ taup,
                                                             float* __restrict__ VL, float* __restrict__ tauq,
                                                             float* __restrict__ d) {
    __shared__ float red[kColThreads / 64];
    __shared__ float alpha_s;
    const int t = threadIdx.x;
    float* a = Ac + (size_t)j * ld;
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

// Trailing column c = j + 1 + blockIdx.x, a workgroup each, rows j .. m-1
// in registers (R per thread, row j + t + 256 i): the previous right update,
// then H_j = I - tau_q u u^T, one read and one write of each entry; row j of
// the result goes to rowbuf.
template <int R>
__global__ __launch_bounds__(256) void bd_left_kernel(float* __restrict__ Ac, int m, int ld, int k, int j,
                                                      const float* __restrict__ x, const float* __restrict__ taup,
                                                      const float* __restrict__ VR, const float* __restrict__ VL,
                                                      const float* __restrict__ tauq, float* __restrict__ rowbuf) {
    __shared__ float red[4];
    const int t = threadIdx.x;
    const int c = j + 1 + blockIdx.x;
    float* a = Ac + (size_t)c * ld;
    const float* u = VL + (size_t)j * m;
    const float tpv = j > 0 ? taup[j - 1] * VR[(size_t)(j - 1) * k + c] : 0.0f;
    float av[R], uv[R];
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int r = j + t + 256 * i;
        float v = 0.0f, uu = 0.0f;
        if (r < m) {
            v = a[r];
            uu = u[r];
            if (j > 0) v = fmaf(-tpv, x[r], v);
        }
        av[i] = v;
        uv[i] = uu;
        dot = fmaf(uu, v, dot);
    }
    dot = wave_sum_f(dot);
    if ((t & 63) == 0) red[t >> 6] = dot;
    __syncthreads();
    const float g = tauq[j] * ((red[0] + red[1]) + (red[2] + red[3]));
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int r = j + t + 256 * i;
        if (r < m) {
            const float v = fmaf(-g, uv[i], av[i]);
            a[r] = v;
            if (i == 0 && t == 0) rowbuf[c] = v;
        }
    }
}

// The same for columns longer than 16 * 256 rows: a wave per column, two
// passes over it.
__global__ __launch_bounds__(256) void bd_left_long_kernel(float* __restrict__ Ac, int m, int ld, int k, int j,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ taup,
                                                           const float* __restrict__ VR,
                                                           const float* __restrict__ VL,
                                                           const float* __restrict__ tauq,
                                                           float* __restrict__ rowbuf) {
    const int lane = threadIdx.x & 63;
    const int c = j + 1 + blockIdx.x * 4 + (threadIdx.x >> 6);
    if (c >= k) return;
    float* a = Ac + (size_t)c * ld;
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

// The right reflector v_j from rowbuf[j+1 .. k-1] (row j of the
// left-updated matrix; its leading 1 at j + 1), then x[r] = sum_{c > j}
// A[r][c] v_j[c] for rows r = j+1 .. m-1.  Every workgroup forms v_j (the
// same sum of squares in the same order, so the same bits) and workgroup 0
// records it (row j of VR, tau_p, e_j), which saves a launch per column.
// The product in one pass: a 1024-thread workgroup per tile of 32 rows from
// r0 = (j + 1) & ~3 (rows below j + 1 come along and are dropped; the pad
// rows are zero).  A lane holds 4 rows (16-byte loads): 8 lanes cover the
// tile, and the 128 column lanes of the workgroup take every 128th column,
// kMvBatch loads in flight before the first product; the 128 sums per row
// meet in LDS in a fixed order.  (Splitting the columns over workgroups
// instead needs a device-scope fence per workgroup to combine them, which
// costs more than the product on this chip.)
__global__ __launch_bounds__(kColThreads) void bd_matvec_kernel(const float* __restrict__ Ac, int m, int ld, int k,
                                                                int j, const float* __restrict__ rowbuf,
                                                                float* __restrict__ VR, float* __restrict__ taup,
                                                                float* __restrict__ e, float* __restrict__ x) {
    __shared__ float red[128][33];
    __shared__ float red2[32][33];
    __shared__ float rsum[kColThreads / 64];
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    float scale;
    {
        float ss = 0.0f;
        for (int c = j + 2 + t; c < k; c += kColThreads) ss = fmaf(rowbuf[c], rowbuf[c], ss);
        ss = block_sum_1024(ss, rsum);
        const float alpha = rowbuf[j + 1];
        float beta = alpha, tau = 0.0f;
        scale = 1.0f;
        if (ss >= kTinySumsq) {
            beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
            tau = (beta - alpha) / beta;
            scale = 1.0f / (alpha - beta);
        }
        if (blockIdx.x == 0) {
            float* v = VR + (size_t)j * k;
            for (int c = t; c < k; c += kColThreads) v[c] = c <= j ? 0.0f : (c == j + 1 ? 1.0f : rowbuf[c] * scale);
            if (t == 0) {
                taup[j] = tau;
                e[j] = beta;
            }
        }
    }
    const int rl = l & 7, cl = (w << 3) | (l >> 3);
    const int r0 = ((j + 1) & ~3) + blockIdx.x * 32;
    const int rq = min(r0 + 4 * rl, ld - 4);   // in the allocation; rows beyond m are dropped below
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int cb = j + 1 + cl; cb < k; cb += 128 * kMvBatch) {
        float4 av[kMvBatch];
        float vv[kMvBatch];
#pragma unroll
        for (int i = 0; i < kMvBatch; ++i) {
            const int c = cb + 128 * i;
            const int cc = min(c, k - 1);
            av[i] = *reinterpret_cast<const float4*>(Ac + (size_t)cc * ld + rq);
            vv[i] = (cc == j + 1 ? 1.0f : rowbuf[cc] * scale) * (c < k ? 1.0f : 0.0f);
        }
#pragma unroll
        for (int i = 0; i < kMvBatch; ++i) {
            acc.x = fmaf(av[i].x, vv[i], acc.x);
            acc.y = fmaf(av[i].y, vv[i], acc.y);
            acc.z = fmaf(av[i].z, vv[i], acc.z);
            acc.w = fmaf(av[i].w, vv[i], acc.w);
        }
    }
    red[cl][4 * rl] = acc.x;
    red[cl][4 * rl + 1] = acc.y;
    red[cl][4 * rl + 2] = acc.z;
    red[cl][4 * rl + 3] = acc.w;
    __syncthreads();
    {
        const int row = t & 31, part = t >> 5;
        red2[part][row] = (red[4 * part][row] + red[4 * part + 1][row]) + (red[4 * part + 2][row] + red[4 * part + 3][row]);
    }
    __syncthreads();
    if (t < 32) {
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 32; ++q) sum += red2[q][t];
        const int rr = r0 + t;
        if (rr < m && rr > j) x[rr] = sum;
    }
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
    const size_t L = bidiag_ld(m);
    return (L * K + 64) + (K * M + 64) + (K * K + 64) + 4 * (K + 64) + (L + 64) + (K + 64) + 64;
}

Bidiag bidiag_carve(float* base, uint32_t m, uint32_t k) {
    float* p = base;
    auto take = [&](size_t c) {
        float* r = p;
        p += (c + 63) / 64 * 64;
        return r;
    };
    Bidiag b;
    b.Ac = take((size_t)bidiag_ld(m) * k);
    b.VL = take((size_t)k * m);
    b.VR = take((size_t)k * k);
    b.tauq = take(k);
    b.taup = take(k);
    b.d = take(k);
    b.e = take(k);
    b.x = take(bidiag_ld(m));
    b.rowbuf = take(k);
    b.flags = reinterpret_cast<uint32_t*>(take(64));
    return b;
}

void bidiag_one(const float* T, uint32_t mm, uint32_t kk, const Bidiag& b, hipStream_t s) {
    const int m = (int)mm, k = (int)kk, ld = (int)bidiag_ld(mm);
    KernelTimer t("svd_bidiag_large", s);
    hipLaunchKernelGGL(bd_zero_flags_kernel, dim3(1), dim3(1), 0, s, b.flags);
    hipLaunchKernelGGL(bd_scan_kernel, dim3((unsigned)std::min<uint64_t>(cdiv((uint64_t)m * k, 256), 2048)),
                       dim3(256), 0, s, T, (size_t)m * k, b.flags);
    hipLaunchKernelGGL(bd_load_kernel, dim3((unsigned)cdiv(k, 32), (unsigned)cdiv(ld, 32)), dim3(256), 0, s, T, m, k,
                       ld, b.Ac, b.flags);
    for (int j = 0; j < k; ++j) {
        hipLaunchKernelGGL(bd_col_kernel, dim3(1), dim3(kColThreads), 0, s, b.Ac, m, ld, j, b.x, b.taup, b.VL,
                           b.tauq, b.d);
        if (j + 1 >= k) break;
        const int cols = k - j - 1, rows_here = (int)cdiv(m - j, 256);
        const dim3 lg((unsigned)cols);
#define MLA_BD_LEFT(R) \
    hipLaunchKernelGGL(bd_left_kernel<R>, lg, dim3(256), 0, s, b.Ac, m, ld, k, j, b.x, b.taup, b.VR, b.VL, b.tauq, \
                       b.rowbuf)
        if (rows_here <= 1) MLA_BD_LEFT(1);
        else if (rows_here <= 2) MLA_BD_LEFT(2);
        else if (rows_here <= 4) MLA_BD_LEFT(4);
        else if (rows_here <= 8) MLA_BD_LEFT(8);
        else if (rows_here <= 16) MLA_BD_LEFT(16);
        else
            hipLaunchKernelGGL(bd_left_long_kernel, dim3((unsigned)cdiv(cols, 4)), dim3(256), 0, s, b.Ac, m, ld, k, j,
                               b.x, b.taup, b.VR, b.VL, b.tauq, b.rowbuf);
#undef MLA_BD_LEFT
        // rows j+1 .. m-1 (m > j + 1 since m >= k > j + 1)
        const int r0 = (j + 1) & ~3;
        hipLaunchKernelGGL(bd_matvec_kernel, dim3((unsigned)cdiv(m - r0, 32)), dim3(kColThreads), 0, s, b.Ac, m, ld,
                           k, j, b.rowbuf, b.VR, b.taup, b.e, b.x);
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

void tgk_build(const Bidiag& b, uint32_t k, float* td, float* te, hipStream_t s) {
    hipLaunchKernelGGL(tgk_build_kernel, dim3((unsigned)cdiv(2 * k, 256)), dim3(256), 0, s, b.d, b.e, (int)k, td, te);
}

}  // namespace mla
