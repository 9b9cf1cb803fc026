// Batched symmetric eigendecomposition of small matrices (n <= 64), one
// matrix per lane group of a wave64 (a whole wave at n = 64), in registers.
//
// Role: the MI355X counterpart of the reference's eigh_ql kernel
// (reference: shaders/Eigh_QL.metal:229-485, driver src/eigh_ql.mm:169-266),
// LAPACK's method per matrix: Householder tridiagonalisation (ssytd2),
// the orthogonal factor, implicit QL iterations with a Wilkinson-type shift
// on the tridiagonal (the method of EISPACK tql2 / LAPACK ssteqr) with the
// rotations applied to the eigenvectors, and an ascending sort.  Conventions
// of the reference's contract: only the requested triangle is read; the
// matrix is scaled by a power of two into [0.5, 1) before and the values
// unscaled after; a matrix holding a NaN or an infinity in the read triangle
// gives all-NaN w and V with info bit 17; info otherwise counts the QL
// iterations in bits 0-15 with bit 16 set once every eigenvalue converged
// (at most 30 n iterations, ssteqr's budget).
//
// MI355X layout: lane c of an N-lane group owns column c of the (symmetric)
// working matrix, so the tridiagonalisation's products A v are lane-local
// FMA chains and only v and w are broadcast through LDS.  The orthogonal
// factor is accumulated as Q^T = H_{n-3} ... H_0 in the same layout, which
// leaves lane r holding row r of Q: a QL rotation of columns (i, i+1) is
// then two registers of every lane.  The QL recurrence runs redundantly on
// every lane of the group with d and e in registers (the sweep loop is
// unrolled so every index is compile-time; inactive positions are skipped
// by a group-uniform branch), mirrored in LDS for the split search, which
// the group's lanes do in parallel (one candidate position each, then a
// ballot).
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr float kEps = 5.9604645e-08f;        // 2^-24, fp32 unit roundoff
constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80: a reflector below it is the identity
constexpr float kSafeMin = 1.17549435e-38f;   // FLT_MIN

template <int N>
struct EighLds {
    float vs[N][N + 1];   // staging of the read triangle, then the reflectors v_k (row k)
    float bc[N + 4];      // per-step broadcast (v, then w)
    float d[N + 1];
    float e[N + 1];
    float tau[N];
    int perm[N];
};

// sum of x[r] * y[r] over r in [LO, N), four partial sums
template <int LO, int N>
__device__ __forceinline__ float dot_tail(const float* x, const float* y) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int r = LO; r < N; r += 4) {
        s0 = fmaf(x[r], y[r], s0);
        if (r + 1 < N) s1 = fmaf(x[r + 1], y[r + 1], s1);
        if (r + 2 < N) s2 = fmaf(x[r + 2], y[r + 2], s2);
        if (r + 3 < N) s3 = fmaf(x[r + 3], y[r + 3], s3);
    }
    return (s0 + s1) + (s2 + s3);
}

// ssytd2 (lower) step K: reflector from column K below the subdiagonal, then
// the symmetric rank-2 update of the trailing block.
template <int K, int N>
__device__ __forceinline__ void tridiag_step(float (&x)[N], EighLds<N>& s, int c, int n) {
    if constexpr (K + 2 < N) {
        if (K + 2 < n) {
            if (c == K) {
                const float alpha = x[K + 1];
                const float ss = dot_tail<K + 2, N>(x, x);
                float beta = alpha, tau = 0.0f, scale = 1.0f;
                if (ss >= kTinySumsq) {
                    beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
                    tau = (beta - alpha) / beta;
                    scale = 1.0f / (alpha - beta);
                }
                s.d[K] = x[K];
                s.e[K] = beta;
                s.tau[K] = tau;
                x[K + 1] = 1.0f;
                s.bc[K + 1] = 1.0f;
#pragma unroll
                for (int r = K + 2; r < N; ++r) {
                    x[r] *= scale;
                    s.bc[r] = x[r];
                }
            }
            wave_lds_sync();
            const float tau = s.tau[K];
            float v[N];
#pragma unroll
            for (int r = K + 1; r < N; ++r) v[r] = s.bc[r];
            const bool act = c > K && c < n;
            float p = 0.0f, vc = 0.0f;
            if (act) {
                vc = s.bc[c];
                p = tau * dot_tail<K + 1, N>(v, x);
            }
            const float half = 0.5f * tau * group_sum<N>(p * vc);
            const float w = fmaf(-half, vc, p);
            wave_lds_sync();
            if (act) s.bc[c] = w;
            wave_lds_sync();
            if (act) {
#pragma unroll
                for (int r = K + 1; r < N; ++r) x[r] = fmaf(-v[r], w, fmaf(-s.bc[r], vc, x[r]));
            }
            wave_lds_sync();
        }
        tridiag_step<K + 1, N>(x, s, c, n);
    }
}

// Q^T <- H_K Q^T (forward accumulation; lane r holds column r of Q^T).
template <int K, int N>
__device__ __forceinline__ void accumulate_step(float (&x)[N], EighLds<N>& s, int n) {
    if constexpr (K + 2 < N) {
        if (K + 2 < n) {
            const float tau = s.tau[K];
            float v[N];
#pragma unroll
            for (int r = K + 1; r < N; ++r) v[r] = s.vs[K][r];
            const float d = tau * dot_tail<K + 1, N>(v, x);
#pragma unroll
            for (int r = K + 1; r < N; ++r) x[r] = fmaf(-d, v[r], x[r]);
        }
        accumulate_step<K + 1, N>(x, s, n);
    }
}

template <int N, bool VEC>
__global__ __launch_bounds__(64) void eigh_small_kernel(const float* __restrict__ A, float* __restrict__ W,
                                                        float* __restrict__ V, uint32_t* __restrict__ info,
                                                        uint32_t batch, uint32_t n, int lower) {
    constexpr int MPW = 64 / N;
    __shared__ EighLds<N> lds[MPW];
    const int lane = threadIdx.x;
    const int c = lane % N;
    const int g = lane / N;
    EighLds<N>& s = lds[g];
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;
    const int nn = (int)n;
    const size_t per = (size_t)n * n;

    // 1. the read triangle, mirrored into a full symmetric matrix
    float x[N];
    float amax = 0.0f;
    int bad = 0;
    const float* src = A + mat * per;
#pragma unroll
    for (int r = 0; r < N; ++r) {
        float v = 0.0f;
        const bool take = lower ? r >= c : r <= c;
        if (live && r < nn && c < nn && take) {
            v = src[(size_t)r * n + c];
            amax = fmaxf(amax, fabsf(v));
            bad |= !finite_f(v);
            s.vs[r][c] = v;
        }
        x[r] = v;
    }
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < N; ++r) {
        const bool take = lower ? r >= c : r <= c;
        if (live && r < nn && c < nn && !take) x[r] = s.vs[c][r];
    }
    amax = group_max<N>(amax);
    bad = group_or<N>(bad);
    const int ex = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -ex);
    wave_lds_sync();

    // 2. tridiagonalise: d, e, tau, and v_k in lane k's column
    tridiag_step<0, N>(x, s, c, nn);
    {
        float diag = 0.0f, sub = 0.0f;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            diag = r == c ? x[r] : diag;
            sub = r == c + 1 ? x[r] : sub;
        }
        if (c == nn - 2) {
            s.d[c] = diag;
            s.e[c] = sub;
        }
        if (c == nn - 1) {
            s.d[c] = diag;
            s.e[c] = 0.0f;
        }
    }
    if (VEC) {
        if (c + 2 < nn) {
#pragma unroll
            for (int r = 0; r < N; ++r)
                if (r > c) s.vs[c][r] = x[r];
        }
    }
    wave_lds_sync();

    // 3. Q^T = H_{n-3} ... H_0 I, lane r ends holding row r of Q
    if (VEC) {
#pragma unroll
        for (int r = 0; r < N; ++r) x[r] = r == c ? 1.0f : 0.0f;
        accumulate_step<0, N>(x, s, nn);
    }

    // 4. implicit QL on (d, e), rotations applied to the rows of Q
    float dd[N], ee[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        dd[i] = s.d[i];
        ee[i] = s.e[i];
    }
    int iters = 0;
    bool converged = true;
    const int budget = 30 * nn;
    for (int l = 0; l < nn && converged; ++l) {
        while (true) {
            // split search: lane i tests e[i] for i in [l, n-1)
            const float di = s.d[c], di1 = s.d[c + 1 < N ? c + 1 : c], ei = s.e[c];
            const bool small = c >= l && c + 1 < nn &&
                               (fabsf(ei) <= kEps * (fabsf(di) + fabsf(di1)) || fabsf(ei) < kSafeMin);
            uint64_t mask = __ballot(small);
            if (N < 64) mask = (mask >> (g * N)) & ((1ull << N) - 1);
            const int m = mask ? __ffsll((unsigned long long)mask) - 1 : nn - 1;
            if (m == l) break;
            if (iters >= budget) {
                converged = false;
                break;
            }
            ++iters;
            // the shift, from the 2x2 at the block's top
            const float dl = s.d[l], dl1 = s.d[l + 1], el = s.e[l], dm = s.d[m];
            float gg = (dl1 - dl) / (2.0f * el);
            float rr = sqrtf(fmaf(gg, gg, 1.0f));
            gg = dm - dl + el / (gg + copysignf(rr, gg));
            float cs = 1.0f, sn = 1.0f, p = 0.0f;
            bool stop = false;
#pragma unroll
            for (int i = N - 2; i >= 0; --i) {
                if (i >= l && i < m && !stop) {
                    float f = sn * ee[i];
                    const float b = cs * ee[i];
                    // (c, s) from (g, f) as a plane rotation.  Tiny pairs are
                    // scaled by a power of two first (group-uniform, rare), so
                    // that f^2 + g^2 is never subnormal: rsqrt of a subnormal
                    // is not accurate.
                    float ga = gg, up = 1.0f;
                    const float mx = fmaxf(fabsf(f), fabsf(gg));
                    if (mx < 0x1p-50f && mx > 0.0f) {
                        int eb = 0;
                        (void)frexpf(mx, &eb);
                        f = ldexpf(f, -eb);
                        ga = ldexpf(gg, -eb);
                        up = ldexpf(1.0f, eb);
                    }
                    const float h = fmaf(f, f, ga * ga);
                    if (h == 0.0f) {
                        // underflow: d[i+1] -= p and restart (e[m] already zero)
                        dd[i + 1] -= p;
                        ee[i + 1] = 0.0f;
                        s.d[i + 1] = dd[i + 1];
                        s.e[i + 1] = 0.0f;
                        stop = true;
                    } else {
                        const float rinv = rsqrtf(h);
                        const float ri = rinv * fmaf(-0.5f * h * rinv, rinv, 1.5f);   // one Newton step
                        const float r = h * ri * up;
                        ee[i + 1] = (i == m - 1) ? 0.0f : r;
                        s.e[i + 1] = ee[i + 1];
                        sn = f * ri;
                        cs = ga * ri;
                        gg = dd[i + 1] - p;
                        const float t = fmaf(dd[i] - gg, sn, 2.0f * cs * b);
                        p = sn * t;
                        dd[i + 1] = gg + p;
                        s.d[i + 1] = dd[i + 1];
                        gg = fmaf(cs, t, -b);
                        if (VEC) {
                            const float z1 = x[i + 1];
                            x[i + 1] = fmaf(sn, x[i], cs * z1);
                            x[i] = fmaf(cs, x[i], -sn * z1);
                        }
                        if (i == l) {
                            dd[i] -= p;
                            ee[i] = gg;
                            s.d[i] = dd[i];
                            s.e[i] = gg;
                        }
                    }
                }
            }
            wave_lds_sync();
        }
    }

    // 5. ascending order: rank of each value (ties by index)
    if (c < nn) {
        const float dc = s.d[c];
        int rank = 0;
        for (int i = 0; i < nn; ++i) {
            const float di = s.d[i];
            rank += (di < dc) || (di == dc && i < c);
        }
        s.perm[rank] = c;
        if (live) W[mat * n + rank] = bad ? qnan() : ldexpf(dc, ex);
    }
    if (live && info && c == 0) {
        info[mat] = bad ? (1u << 17) : ((uint32_t)(iters < 0xFFFF ? iters : 0xFFFF) | (converged ? 1u << 16 : 0u));
    }
    if (VEC) {
        wave_lds_sync();
        // rows of Q through LDS, so that each lane writes one output column
#pragma unroll
        for (int j = 0; j < N; ++j) s.vs[c][j] = x[j];
        wave_lds_sync();
        if (live && c < nn) {
            const int j = s.perm[c];
            float* dst = V + mat * per;
#pragma unroll
            for (int r = 0; r < N; ++r)
                if (r < nn) dst[(size_t)r * n + c] = bad ? qnan() : s.vs[r][j];
        }
    }
}

template <int N, bool VEC>
void launch(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower,
            hipStream_t s) {
    constexpr int MPW = 64 / N;
    KernelTimer t("eigh_small", s);
    hipLaunchKernelGGL((eigh_small_kernel<N, VEC>), dim3((uint32_t)cdiv(batch, MPW)), dim3(64), 0, s, a, w, v, info,
                       batch, n, lower ? 1 : 0);
    t.stop();
}

template <bool VEC>
void dispatch(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower,
              hipStream_t s) {
    if (n <= 8) launch<8, VEC>(a, w, v, info, batch, n, lower, s);
    else if (n <= 16) launch<16, VEC>(a, w, v, info, batch, n, lower, s);
    else if (n <= 32) launch<32, VEC>(a, w, v, info, batch, n, lower, s);
    else launch<64, VEC>(a, w, v, info, batch, n, lower, s);
}

}  // namespace

bool eigh_small_fits(uint32_t n) { return n >= 1 && n <= 64; }

void eigh_small(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower,
                hipStream_t s) {
    if (!eigh_small_fits(n)) invalid("[eigh] eigh_small takes n <= 64");
    if (batch == 0) return;
    if (v) dispatch<true>(a, w, v, info, batch, n, lower, s);
    else dispatch<false>(a, w, nullptr, info, batch, n, lower, s);
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
