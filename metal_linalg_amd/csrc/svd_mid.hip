// Batched thin SVD of mid-size matrices: 65 <= min(m, n) <= 128 and
// max(m, n) <= 128, one matrix per workgroup of eight waves, by one-sided
// Jacobi.
//
// Role: the MI355X counterpart of the reference's golub_kahan kernel past
// the 64-column window of svd_small (reference: src/svd_golub_kahan.mm:
// 205-211, which takes K up to about 83 on its threadgroup memory;
// shaders/Svd_GolubKahan.metal), so that a batch of such matrices is one
// launch instead of one large-matrix SVD per matrix.  Contract of core::svd
// (src/svd.mm:1058-1106) as the batched kernels keep it: A scaled by a power
// of two into [0.5, 1) and the values unscaled after; a matrix holding a NaN
// or an infinity gives all-NaN s, U, Vt and info bit 17; otherwise info
// counts the sweeps (bits 0-15), bit 16 converged, bit 18 rank-deficient
// unless s_min > 32 FLT_EPSILON s_max; s descending and non-negative; U and
// V^T with orthonormal columns and rows.
//
// Method (Hestenes; Demmel & Veselic, SIAM J. Matrix Anal. Appl. 13 (1992)
// 1204-1245): the tall problem T (L x K, L >= K; a wide A is solved as A^T)
// is orthogonalised column against column by plane rotations, T J_1 J_2 ...
// = U S, the rotations accumulated into V; a sweep visits every pair of
// columns once, in the round-robin order of a tournament (K / 2 disjoint
// pairs per round, all rotated at once).  A pair is rotated while
// |a_i . a_j| > tol |a_i| |a_j| with tol = 4 sqrt(L) eps; the sweeps stop
// when one rotates nothing.  Then s_c = |a_c|, u_c = a_c / s_c, and a column
// that is exactly zero gets an orthonormal completion (Gram-Schmidt of unit
// vectors against the others), so that U is orthonormal whatever the rank.
// One-sided Jacobi gives the singular values to high relative accuracy; the
// rotations are applied in Rutishauser's form, which keeps the column norms
// from drifting over the sweeps.
//
// MI355X layout: T's columns and V's columns live in LDS (each column
// contiguous, stride 132 floats: 135 KB at K = 128), eight threads per
// pair, each taking sixteen consecutive rows of both columns into VGPRs
// (four 16-byte reads a column); the pair's
// three inner products are DPP sums over the eight lanes, every lane forms
// the same rotation, and the rotated rows go back to LDS.  One barrier per
// round.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int kMaxK = 128;
constexpr int kMinK = 65;
constexpr int kMaxL = 128;
constexpr int kLd = kMaxL + 4;   // column stride in LDS (16-byte aligned columns)
constexpr int kSub = 8;          // threads per pair
constexpr int kThreads = (kMaxK / 2) * kSub;
constexpr int kRowsPer = kMaxL / kSub;   // rows per thread of a column
constexpr int kMaxSweeps = 30;
constexpr float kEps = 5.9604645e-08f;   // 2^-24

struct alignas(16) JacobiLds {
    float a[kMaxK * kLd];   // T's columns (rows past L zero)
    float v[kMaxK * kLd];   // V's columns (rows past K zero)
    float sig[kMaxK];
    int rank[kMaxK];
    int colof[kMaxK];       // the column of each rank
    float red[kThreads / 64];
    float u[kMaxL];         // the completion's working vector
    float dcoef[kMaxK];
};

// Sum over the aligned group of eight lanes, on every lane of the group.
__device__ __forceinline__ float sum8(float v) { return half_row_sum(v); }

__device__ __forceinline__ float block_sum(float v, float* red, int t) {
    v = wave_sum_f(v);
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    __syncthreads();
    return s;
}

__device__ __forceinline__ float block_max(float v, float* red, int t) {
    v = group_max<64>(v);
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s = fmaxf(s, red[w]);
    __syncthreads();
    return s;
}

// The pair of round r (0 <= r < P - 1) for slot k of P players (P even):
// player P - 1 stays, the others turn around it.
__device__ __forceinline__ void tournament_pair(int P, int r, int k, int& i, int& j) {
    if (k == 0) {
        i = r;
        j = P - 1;
    } else {
        i = (r + k) % (P - 1);
        j = (r - k + (P - 1)) % (P - 1);
    }
}

__global__ __launch_bounds__(kThreads) void svd_jacobi_kernel(const float* __restrict__ A, float* __restrict__ U,
                                                              float* __restrict__ S, float* __restrict__ Vt,
                                                              uint32_t* __restrict__ info, uint32_t m_, uint32_t n_) {
    __shared__ JacobiLds s;
    const int t = threadIdx.x;
    const size_t mat = blockIdx.x;
    const int m = (int)m_, n = (int)n_;
    const bool trans = m < n;
    const int L = trans ? n : m, K = trans ? m : n;   // the tall problem T, L x K
    const int P = K + (K & 1);                         // players (an odd K gets an idle one)

    // 1. T into LDS (A read contiguously), scanned and scaled; V = I
    float amax = 0.0f;
    int bad = 0;
    const float* src = A + mat * (size_t)m * n;
    for (int g = t; g < kMaxK * kLd; g += kThreads) {
        s.a[g] = 0.0f;
        const int c = g / kLd, r = g - c * kLd;
        s.v[g] = r == c ? 1.0f : 0.0f;
    }
    __syncthreads();
    for (int g = t; g < m * n; g += kThreads) {
        const int i = g / n, j = g - i * n;   // A[i][j]
        const float x = src[g];
        amax = fmaxf(amax, fabsf(x));
        bad |= !finite_f(x);
        const int r = trans ? j : i, c = trans ? i : j;   // T[r][c]
        s.a[c * kLd + r] = x;
    }
    amax = block_max(amax, s.red, t);
    bad = __syncthreads_or(bad);
    const int ex = bad ? 0 : scale_exponent(amax);
    for (int g = t; g < K * kLd; g += kThreads) s.a[g] = bad ? 0.0f : ldexpf(s.a[g], -ex);
    __syncthreads();

    // 2. sweeps
    const int p = t / kSub, q = t % kSub;
    const float tol = 4.0f * sqrtf((float)L) * kEps;
    int sweeps = 0;
    bool converged = bad != 0;
    while (!converged && sweeps < kMaxSweeps) {
        int rotated = 0;
        for (int r = 0; r < P - 1; ++r) {
            int i = 0, j = 0;
            if (p < P / 2) tournament_pair(P, r, p, i, j);
            const bool live = p < P / 2 && i < K && j < K;
            if (live) {
                // rows 16 q .. 16 q + 15 of both columns, as 16-byte reads
                float4* ai = reinterpret_cast<float4*>(s.a + i * kLd + kRowsPer * q);
                float4* aj = reinterpret_cast<float4*>(s.a + j * kLd + kRowsPer * q);
                float4 xi[kRowsPer / 4], xj[kRowsPer / 4];
                float al = 0.0f, be = 0.0f, ga = 0.0f;
#pragma unroll
                for (int k = 0; k < kRowsPer / 4; ++k) {
                    xi[k] = ai[k];
                    xj[k] = aj[k];
                    al = fmaf(xi[k].x, xi[k].x, fmaf(xi[k].y, xi[k].y, fmaf(xi[k].z, xi[k].z, fmaf(xi[k].w, xi[k].w, al))));
                    be = fmaf(xj[k].x, xj[k].x, fmaf(xj[k].y, xj[k].y, fmaf(xj[k].z, xj[k].z, fmaf(xj[k].w, xj[k].w, be))));
                    ga = fmaf(xi[k].x, xj[k].x, fmaf(xi[k].y, xj[k].y, fmaf(xi[k].z, xj[k].z, fmaf(xi[k].w, xj[k].w, ga))));
                }
                al = sum8(al);
                be = sum8(be);
                ga = sum8(ga);
                if (fabsf(ga) > tol * __builtin_amdgcn_sqrtf(al) * __builtin_amdgcn_sqrtf(be)) {
                    // the same on the pair's eight lanes; hardware
                    // reciprocal and square root estimates (about an ulp):
                    // only the rotation's orthogonality matters, which the
                    // form below keeps to the rounding of tau
                    const float zeta = (be - al) * rcp_refined(2.0f * ga);
                    const float az = fabsf(zeta);
                    const float tt = az > 1e18f ? 0.5f * rcp_refined(zeta)
                                                : copysignf(rcp_refined(az + __builtin_amdgcn_sqrtf(fmaf(az, az, 1.0f))), zeta);
                    const float cs = rcp_refined(__builtin_amdgcn_sqrtf(fmaf(tt, tt, 1.0f)));
                    const float sn = cs * tt;
                    // Rutishauser's form: x_i - s (x_j + tau x_i) and
                    // x_j + s (x_i - tau x_j), tau = s / (1 + c), is
                    // (c x_i - s x_j, s x_i + c x_j) with each update a
                    // correction of the size of s; written with c and s
                    // directly the rounding of c^2 + s^2 = 1 scales the
                    // columns by about an ulp per rotation, a drift of
                    // 1e-5 of the largest value after the ~1000 rotations
                    // a column sees
                    const float tau = sn * rcp_refined(1.0f + cs);
                    auto rot = [&](float4 x, float4 y, float4& xo, float4& yo) {
                        xo = make_float4(fmaf(-sn, fmaf(tau, x.x, y.x), x.x), fmaf(-sn, fmaf(tau, x.y, y.y), x.y),
                                         fmaf(-sn, fmaf(tau, x.z, y.z), x.z), fmaf(-sn, fmaf(tau, x.w, y.w), x.w));
                        yo = make_float4(fmaf(sn, fmaf(-tau, y.x, x.x), y.x), fmaf(sn, fmaf(-tau, y.y, x.y), y.y),
                                         fmaf(sn, fmaf(-tau, y.z, x.z), y.z), fmaf(sn, fmaf(-tau, y.w, x.w), y.w));
                    };
#pragma unroll
                    for (int k = 0; k < kRowsPer / 4; ++k) rot(xi[k], xj[k], ai[k], aj[k]);
                    float4* vi = reinterpret_cast<float4*>(s.v + i * kLd + kRowsPer * q);
                    float4* vj = reinterpret_cast<float4*>(s.v + j * kLd + kRowsPer * q);
                    float4 yi[kRowsPer / 4], yj[kRowsPer / 4];
#pragma unroll
                    for (int k = 0; k < kRowsPer / 4; ++k) {
                        yi[k] = vi[k];
                        yj[k] = vj[k];
                    }
#pragma unroll
                    for (int k = 0; k < kRowsPer / 4; ++k) rot(yi[k], yj[k], vi[k], vj[k]);
                    rotated = 1;
                }
            }
            __syncthreads();
        }
        ++sweeps;
        converged = __syncthreads_or(rotated) == 0;
    }

    // 3. s, ranks (descending, ties by column), u_c = a_c / s_c
    if (t < K) {
        const float* ac = s.a + t * kLd;
        float nrm = 0.0f;
        for (int r = 0; r < L; ++r) nrm = fmaf(ac[r], ac[r], nrm);
        s.sig[t] = sqrtf(nrm);
    }
    __syncthreads();
    if (t < K) {
        const float sc = s.sig[t];
        int rk = 0;
        for (int i = 0; i < K; ++i) {
            const float si = s.sig[i];
            rk += (si > sc) || (si == sc && i < t);
        }
        s.rank[t] = rk;
        s.colof[rk] = t;
        float* ac = s.a + t * kLd;
        const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
        for (int r = 0; r < L; ++r) ac[r] *= inv;
    }
    __syncthreads();
    // a zero column (bad matrices aside: their outputs are NaN) gets a unit
    // vector e_j made orthogonal to every finished column (two Gram-Schmidt
    // passes), trying j = 0, 1, ... until one keeps a squared length above
    // 1 / (2 L): the squared lengths left of e_0 .. e_{L-1} sum to L minus
    // the finished columns, at least 1, so one of them is at least 1 / L
    if (!bad && U) {
        for (int z = 0; z < K; ++z) {
            if (s.sig[z] > 0.0f) continue;   // uniform: s.sig is shared
            for (int jc = 0; jc < L; ++jc) {
                if (t < L) s.u[t] = t == jc ? 1.0f : 0.0f;
                __syncthreads();
                for (int pass = 0; pass < 2; ++pass) {
                    // coefficients against the finished columns (nonzero, or
                    // completed before z)
                    if (t < K) {
                        float d = 0.0f;
                        const bool done = s.sig[t] > 0.0f || t < z;
                        if (done && t != z) {
                            const float* ac = s.a + t * kLd;
                            for (int r = 0; r < L; ++r) d = fmaf(ac[r], s.u[r], d);
                        }
                        s.dcoef[t] = d;
                    }
                    __syncthreads();
                    if (t < L) {
                        float x = s.u[t];
                        for (int i = 0; i < K; ++i) x = fmaf(-s.dcoef[i], s.a[i * kLd + t], x);
                        s.u[t] = x;
                    }
                    __syncthreads();
                }
                const float nrm2 = block_sum(t < L ? s.u[t] * s.u[t] : 0.0f, s.red, t);
                if (nrm2 > 0.5f / (float)L) {
                    const float inv = 1.0f / sqrtf(nrm2);
                    if (t < L) s.a[z * kLd + t] = s.u[t] * inv;
                    __syncthreads();
                    break;
                }
            }
        }
    }

    // 4. outputs: s[rank] = s_c 2^e; T's U and V become A's (swapped for a
    // wide A)
    float smax = 0.0f, smin = FLT_MAX;
    for (int c = 0; c < K; ++c) {
        smax = fmaxf(smax, s.sig[c]);
        smin = fminf(smin, s.sig[c]);
    }
    if (t < K) S[mat * K + s.rank[t]] = bad ? qnan() : ldexpf(s.sig[t], ex);
    if (U) {
        float* Ua = U + mat * (size_t)m * K;
        float* Va = Vt + mat * (size_t)K * n;
        // A's U (m x K): T's U (non-wide) or T's V (wide); A's V^T (K x n):
        // T's V^T, or T's U^T
        for (int g = t; g < m * K; g += kThreads) {
            const int r = g / K, col = g - r * K;   // U[r][col], col = a rank
            const int c = s.colof[col];
            Ua[g] = bad ? qnan() : (trans ? s.v[c * kLd + r] : s.a[c * kLd + r]);
        }
        for (int g = t; g < K * n; g += kThreads) {
            const int row = g / n, col = g - row * n;   // Vt[row][col], row = a rank
            const int c = s.colof[row];
            const float x = trans ? s.a[c * kLd + col] : s.v[c * kLd + col];
            Va[g] = bad ? qnan() : x;
        }
    }
    if (info && t == 0) {
        uint32_t w = bad ? (1u << 17) : ((uint32_t)sweeps | (converged ? (1u << 16) : 0u));
        if (!bad && !(smin > 32.0f * FLT_EPSILON * smax)) w |= 1u << 18;
        info[mat] = w;
    }
}

}  // namespace

bool svd_mid_fits(uint32_t m, uint32_t n) {
    const uint32_t k = m < n ? m : n, l = m < n ? n : m;
    return k >= (uint32_t)kMinK && k <= (uint32_t)kMaxK && l <= (uint32_t)kMaxL;
}

void svd_mid(const float* a, float* u, float* s, float* vt, uint32_t* info, uint32_t batch, uint32_t m, uint32_t n,
             hipStream_t st) {
    if (!svd_mid_fits(m, n)) invalid("[svd] svd_mid takes 65 <= min(m, n) <= 128 and max(m, n) <= 128");
    if (batch == 0) return;
    if ((u == nullptr) != (vt == nullptr)) invalid("[svd] svd_mid takes both U and Vt or neither");
    KernelTimer t("svd_jacobi", st);
    for (uint32_t b0 = 0; b0 < batch; b0 += 1u << 20) {
        const uint32_t nb = std::min<uint32_t>(batch - b0, 1u << 20);
        const uint32_t k = m < n ? m : n;
        hipLaunchKernelGGL(svd_jacobi_kernel, dim3(nb), dim3(kThreads), 0, st, a + (size_t)b0 * m * n,
                           u ? u + (size_t)b0 * m * k : nullptr, s + (size_t)b0 * k,
                           vt ? vt + (size_t)b0 * k * n : nullptr, info ? info + b0 : nullptr, m, n);
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
