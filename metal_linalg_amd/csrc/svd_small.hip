// Batched thin SVD of matrices with min(m, n) <= 64 and max(m, n) <= 128,
// one matrix per wave64, in three kernels joined by an HBM workspace.
//
// Role: the MI355X counterpart of the reference's golub_kahan backend
// (reference: src/svd_golub_kahan.mm:232-367, shaders/Svd_GolubKahan.metal:425-799;
// config 3 routes there after a QR, src/svd.mm:902-914): Householder
// bidiagonalisation (LAPACK sgebd2), implicit shifted QR on the bidiagonal
// (Golub & Reinsch, Numer. Math. 14 (1970) 403-420) with the rotations
// accumulated into the bidiagonal's singular vectors, then the
// back-transformation by the reflectors.  The contract is the reference's:
// A scaled by a power of two into [0.5, 1) and the values unscaled after;
// a matrix holding a NaN or an infinity gives all-NaN s, U, Vt and info bit
// 17; otherwise info counts the QR sweeps (bits 0-15), bit 16 converged,
// bit 18 rank-deficient unless s_min > 32 FLT_EPSILON s_max
// (Svd_GolubKahan.metal:795-797); s descending and non-negative.
//
// A wide matrix (m < n) is solved as its transpose, the roles of U and Vt
// swapped.  Below, "the problem" is the tall M x N (M >= N) one.
//
//   svd_bidiag     the problem in LDS (M x 65 floats); a wave works it,
//                  lanes over columns for the left reflectors' products and
//                  over rows for the right ones, so every product is a
//                  lane-local loop over LDS (no cross-lane reductions beyond
//                  two norms per step).  Writes d, e, the reflectors
//                  (column-contiguous) and their tau.
//   svd_bdsqr      lane r holds row r of the bidiagonal's U and V in VGPRs;
//                  the Golub-Reinsch recurrence runs on every lane with d
//                  and e in registers (unrolled sweep, wave-uniform guards),
//                  mirrored in LDS for the lane-parallel split test; then
//                  sign fix, descending sort.
//   svd_backtransform  lane c forms column c of U = Q [U_B; 0] and of
//                  V = P V_B from the reflectors (wave-uniform loads).
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int kMaxM = 128;
constexpr int kMaxN = 64;
constexpr int kPitch = kMaxN + 1;
constexpr float kEps = 5.9604645e-08f;        // 2^-24
constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80

// Per-matrix workspace, in floats.
struct SvdWs {
    uint32_t M, N;
    __host__ __device__ size_t refl() const { return 0; }                        // [N][M]  v_k, contiguous per k
    __host__ __device__ size_t refr() const { return (size_t)N * M; }            // [N][N]  u_k, contiguous per k
    __host__ __device__ size_t tq() const { return refr() + (size_t)N * N; }     // [N]
    __host__ __device__ size_t tp() const { return tq() + N; }                   // [N]
    __host__ __device__ size_t d() const { return tp() + N; }                    // [N]
    __host__ __device__ size_t e() const { return d() + N; }                     // [N] e[k] couples (k, k+1)
    __host__ __device__ size_t ub() const { return e() + N; }                    // [N][N] U_B, sorted columns
    __host__ __device__ size_t vb() const { return ub() + (size_t)N * N; }       // [N][N] V_B, sorted columns
    __host__ __device__ size_t meta() const { return vb() + (size_t)N * N; }     // [2] exponent, bad
    __host__ __device__ size_t per() const { return meta() + 2; }
};

// ---------------------------------------------------------------- bidiag
__global__ __launch_bounds__(64) void svd_bidiag_kernel(const float* __restrict__ A, float* __restrict__ ws,
                                                        uint32_t batch, uint32_t rows, uint32_t cols, int trans,
                                                        int vectors) {
    __shared__ float a[kMaxM][kPitch];
    const int t = threadIdx.x;
    const size_t mat = blockIdx.x;
    if (mat >= batch) return;   // whole wave: uniform
    const int M = trans ? (int)cols : (int)rows;
    const int N = trans ? (int)rows : (int)cols;
    const SvdWs W{(uint32_t)M, (uint32_t)N};
    float* w = ws + mat * W.per();
    const float* src = A + mat * (size_t)rows * cols;

    // load (transposed for a wide input), scan
    float amax = 0.0f;
    int bad = 0;
    for (int r = 0; r < M; ++r) {
        if (t < N) {
            const float v = trans ? src[(size_t)t * cols + r] : src[(size_t)r * cols + t];
            amax = fmaxf(amax, fabsf(v));
            bad |= !finite_f(v);
            a[r][t] = v;
        }
    }
    amax = group_max<64>(amax);
    bad = group_or<64>(bad);
    const int ex = bad ? 0 : scale_exponent(amax);
    for (int r = 0; r < M; ++r)
        if (t < N) a[r][t] = bad ? 0.0f : ldexpf(a[r][t], -ex);
    wave_lds_sync();

    for (int k = 0; k < N; ++k) {
        // ---- left reflector on column k, rows k.. ----
        float part = 0.0f;
        for (int r = k + 1 + t; r < M; r += 64) part = fmaf(a[r][k], a[r][k], part);
        const float ss = group_sum<64>(part);
        const float alpha = a[k][k];
        float beta = alpha, tau = 0.0f, scale = 1.0f;
        if (ss >= kTinySumsq) {
            beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
            tau = (beta - alpha) / beta;
            scale = 1.0f / (alpha - beta);
        }
        wave_lds_sync();
        for (int r = k + 1 + t; r < M; r += 64) a[r][k] *= scale;
        wave_lds_sync();
        if (t > k && t < N && tau != 0.0f) {
            float dot = a[k][t];
            for (int r = k + 1; r < M; ++r) dot = fmaf(a[r][k], a[r][t], dot);
            dot *= tau;
            a[k][t] -= dot;
            for (int r = k + 1; r < M; ++r) a[r][t] = fmaf(-dot, a[r][k], a[r][t]);
        }
        if (t == 0) {
            w[W.d() + k] = beta;
            w[W.tq() + k] = tau;
        }
        if (vectors) {   // v_k, contiguous: [k] = 1, below from the column
            for (int r = t; r < M; r += 64)
                w[W.refl() + (size_t)k * M + r] = r < k ? 0.0f : (r == k ? 1.0f : a[r][k]);
        }
        wave_lds_sync();
        if (k + 1 >= N) break;
        // ---- right reflector on row k, columns k+1.. ----
        const float x = (t > k + 1 && t < N) ? a[k][t] : 0.0f;
        const float ssr = group_sum<64>(x * x);
        const float alr = a[k][k + 1];
        float br = alr, taur = 0.0f, scr = 1.0f;
        if (ssr >= kTinySumsq) {
            br = -copysignf(sqrtf(fmaf(alr, alr, ssr)), alr);
            taur = (br - alr) / br;
            scr = 1.0f / (alr - br);
        }
        wave_lds_sync();
        if (t > k + 1 && t < N) a[k][t] *= scr;
        wave_lds_sync();
        if (taur != 0.0f) {
            for (int r = k + 1 + t; r < M; r += 64) {
                float dot = a[r][k + 1];
                for (int c = k + 2; c < N; ++c) dot = fmaf(a[r][c], a[k][c], dot);
                dot *= taur;
                a[r][k + 1] -= dot;
                for (int c = k + 2; c < N; ++c) a[r][c] = fmaf(-dot, a[k][c], a[r][c]);
            }
        }
        if (t == 0) {
            w[W.e() + k] = br;
            w[W.tp() + k] = taur;
        }
        if (vectors && t < N)   // u_k: [k+1] = 1, then the row
            w[W.refr() + (size_t)k * N + t] = t <= k ? 0.0f : (t == k + 1 ? 1.0f : a[k][t]);
        wave_lds_sync();
    }
    if (t == 0) {
        w[W.e() + N - 1] = 0.0f;
        w[W.tp() + N - 1] = 0.0f;
        w[W.meta()] = __int_as_float(ex);
        w[W.meta() + 1] = __int_as_float(bad);
    }
    if (vectors && t < N) w[W.refr() + (size_t)(N - 1) * N + t] = 0.0f;
}

// ---------------------------------------------------------------- bdsqr
struct BdLds {
    float q[kMaxN + 1];
    float e[kMaxN + 1];   // Golub-Reinsch convention: e[i] couples (i-1, i), e[0] = 0
    float st[kMaxN][kMaxN + 1];
    int perm[kMaxN];
};

// (c, s, r) of the rotation taking (f, h) to (r, 0), robust to tiny pairs
// (rescaled by a power of two so that f^2 + h^2 is never subnormal).
__device__ __forceinline__ float rot(float f, float h, float& c, float& s) {
    float up = 1.0f;
    const float mx = fmaxf(fabsf(f), fabsf(h));
    if (mx < 0x1p-50f && mx > 0.0f) {
        int eb = 0;
        (void)frexpf(mx, &eb);
        f = ldexpf(f, -eb);
        h = ldexpf(h, -eb);
        up = ldexpf(1.0f, eb);
    }
    const float sq = fmaf(f, f, h * h);
    if (sq == 0.0f) {
        c = 1.0f;
        s = 0.0f;
        return 0.0f;
    }
    const float y = rsqrtf(sq);
    const float ri = y * fmaf(-0.5f * sq * y, y, 1.5f);
    c = f * ri;
    s = h * ri;
    return sq * ri * up;
}

template <bool VEC>
__global__ __launch_bounds__(64) void svd_bdsqr_kernel(float* __restrict__ ws, float* __restrict__ S,
                                                       uint32_t* __restrict__ info, uint32_t batch, uint32_t Mp,
                                                       uint32_t Np) {
    constexpr int NN = kMaxN;
    __shared__ BdLds s;
    const int lane = threadIdx.x;
    const size_t mat = blockIdx.x;
    if (mat >= batch) return;
    const int n = (int)Np;
    const SvdWs W{Mp, Np};
    float* w = ws + mat * W.per();
    const int ex = __float_as_int(w[W.meta()]);
    const int bad = __float_as_int(w[W.meta() + 1]);

    float qq[NN], ee[NN];
    float xu[VEC ? NN : 1], xv[VEC ? NN : 1];
#pragma unroll
    for (int i = 0; i < NN; ++i) {
        qq[i] = i < n ? w[W.d() + i] : 0.0f;
        ee[i] = (i >= 1 && i < n) ? w[W.e() + i - 1] : 0.0f;
        if (VEC) {
            xu[i] = i == lane ? 1.0f : 0.0f;
            xv[i] = i == lane ? 1.0f : 0.0f;
        }
    }
    float anorm = 0.0f;
#pragma unroll
    for (int i = 0; i < NN; ++i) anorm = fmaxf(anorm, fabsf(qq[i]) + fabsf(ee[i]));
    if (lane < n) {
        float qv = 0.0f, ev = 0.0f;
#pragma unroll
        for (int i = 0; i < NN; ++i) {
            qv = i == lane ? qq[i] : qv;
            ev = i == lane ? ee[i] : ev;
        }
        s.q[lane] = qv;
        s.e[lane] = ev;
    }
    wave_lds_sync();
    const float tol = kEps * anorm;

    int sweeps = 0;
    bool converged = true;
    const int budget = 30 * n;
    for (int k = n - 1; k >= 0 && converged; --k) {
        while (true) {
            // split test: l = the largest i <= k with e[i] or q[i-1] negligible
            const float ei = s.e[lane < NN ? lane : 0];
            const float qm = s.q[lane >= 1 && lane <= NN ? lane - 1 : 0];
            const bool se = lane <= k && (lane == 0 || fabsf(ei) <= tol);
            const bool sq = lane <= k && lane >= 1 && fabsf(qm) <= tol;
            const uint64_t any = __ballot(se || sq);
            const int l = 63 - __clzll((long long)any);
            const bool cancel = !((__ballot(se) >> l) & 1ull);
            if (cancel) {
                // e[l] is cancelled by rotations of rows (l-1, i), i = l..k
                const int nm = l - 1;
                float cc = 0.0f, sn = 1.0f;
                float unm = 0.0f;
                if (VEC) {
#pragma unroll
                    for (int j = 0; j < NN; ++j) unm = j == nm ? xu[j] : unm;
                }
                bool done = false;
#pragma unroll
                for (int i = 0; i < NN; ++i) {
                    if (i >= l && i <= k && !done) {
                        const float f = sn * ee[i];
                        ee[i] = cc * ee[i];
                        s.e[i] = ee[i];
                        if (fabsf(f) <= tol) {
                            done = true;
                        } else {
                            const float g = qq[i];
                            float c2, s2;
                            const float h = rot(g, f, c2, s2);
                            qq[i] = h;
                            s.q[i] = h;
                            cc = c2;
                            sn = -s2;
                            if (VEC) {
                                const float y = unm, z = xu[i];
                                unm = fmaf(y, cc, z * sn);
                                xu[i] = fmaf(z, cc, -y * sn);
                            }
                        }
                    }
                }
                if (VEC) {
#pragma unroll
                    for (int j = 0; j < NN; ++j) xu[j] = j == nm ? unm : xu[j];
                }
                wave_lds_sync();
            }
            if (l == k) break;   // q[k] converged (its sign is fixed at the end)
            if (sweeps >= budget) {
                converged = false;
                break;
            }
            ++sweeps;
            // shift from the bottom 2x2
            const float x0 = s.q[l], y0 = s.q[k - 1], g0 = s.e[k - 1], h0 = s.e[k], z0 = s.q[k];
            float f = ((y0 - z0) * (y0 + z0) + (g0 - h0) * (g0 + h0)) / (2.0f * h0 * y0);
            const float gq = sqrtf(fmaf(f, f, 1.0f));
            f = ((x0 - z0) * (x0 + z0) + h0 * ((y0 / (f + copysignf(gq, f))) - h0)) / x0;
            float c = 1.0f, sn = 1.0f, x = x0;
#pragma unroll
            for (int j = 0; j < NN - 1; ++j) {
                if (j >= l && j < k) {
                    const int i = j + 1;
                    float g = ee[i];
                    float y = qq[i];
                    float h = sn * g;
                    g = c * g;
                    float cz, sz;
                    const float z1 = rot(f, h, cz, sz);
                    ee[j] = (j == l) ? 0.0f : z1;
                    s.e[j] = ee[j];
                    c = cz;
                    sn = sz;
                    f = fmaf(x, c, g * sn);
                    g = fmaf(g, c, -x * sn);
                    h = y * sn;
                    y *= c;
                    if (VEC) {
                        const float vx = xv[j], vz = xv[i];
                        xv[j] = fmaf(vx, c, vz * sn);
                        xv[i] = fmaf(vz, c, -vx * sn);
                    }
                    float c2, s2;
                    const float z2 = rot(f, h, c2, s2);
                    qq[j] = z2;
                    s.q[j] = z2;
                    if (z2 != 0.0f) {
                        c = c2;
                        sn = s2;
                    }
                    f = fmaf(c, g, sn * y);
                    x = fmaf(c, y, -sn * g);
                    if (VEC) {
                        const float uy = xu[j], uz = xu[i];
                        xu[j] = fmaf(uy, c, uz * sn);
                        xu[i] = fmaf(uz, c, -uy * sn);
                    }
                    if (i == k) {
                        ee[i] = f;
                        qq[i] = x;
                        s.e[i] = f;
                        s.q[i] = x;
                    }
                }
            }
            wave_lds_sync();
        }
    }

    // signs: non-negative values, the matching V columns negated
#pragma unroll
    for (int j = 0; j < NN; ++j) {
        if (j < n && qq[j] < 0.0f) {
            qq[j] = -qq[j];
            if (VEC) xv[j] = -xv[j];
        }
    }
    wave_lds_sync();
    if (lane < n) {
        float qv = 0.0f;
#pragma unroll
        for (int i = 0; i < NN; ++i) qv = i == lane ? qq[i] : qv;
        s.q[lane] = qv;
    }
    wave_lds_sync();
    float smax = 0.0f, smin = 3.0e38f;
    int rank = 0;
    if (lane < n) {
        const float mine = s.q[lane];
        for (int i = 0; i < n; ++i) {
            const float o = s.q[i];
            rank += (o > mine) || (o == mine && i < lane);
            smax = fmaxf(smax, o);
            smin = fminf(smin, o);
        }
        s.perm[rank] = lane;
        S[mat * n + rank] = bad ? qnan() : ldexpf(mine, ex);
    }
    if (info && lane == 0) {
        uint32_t word;
        if (bad) {
            word = 1u << 17;
        } else {
            word = (uint32_t)(sweeps < 0xFFFF ? sweeps : 0xFFFF) | (converged ? 1u << 16 : 0u);
            if (n > 0 && !(smin > 32.0f * FLT_EPSILON * smax)) word |= 1u << 18;
        }
        info[mat] = word;
    }
    if (!VEC) return;
    // sorted columns of U_B, then V_B, through LDS (lane r holds row r)
    wave_lds_sync();
    if (lane < n) {
#pragma unroll
        for (int j = 0; j < NN; ++j) s.st[lane][j] = xu[j];
    }
    wave_lds_sync();
    if (lane < n) {
        const int j = s.perm[lane];
        for (int r = 0; r < n; ++r) w[W.ub() + (size_t)r * n + lane] = s.st[r][j];
    }
    wave_lds_sync();
    if (lane < n) {
#pragma unroll
        for (int j = 0; j < NN; ++j) s.st[lane][j] = xv[j];
    }
    wave_lds_sync();
    if (lane < n) {
        const int j = s.perm[lane];
        for (int r = 0; r < n; ++r) w[W.vb() + (size_t)r * n + lane] = s.st[r][j];
    }
}

// ---------------------------------------------------------- back-transform
__global__ __launch_bounds__(64) void svd_backtransform_kernel(const float* __restrict__ ws, float* __restrict__ U,
                                                               float* __restrict__ Vt, uint32_t batch, uint32_t rows,
                                                               uint32_t cols, int trans) {
    __shared__ float tr[kMaxN][kMaxN + 1];
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    if (mat >= batch) return;
    const int M = trans ? (int)cols : (int)rows;
    const int N = trans ? (int)rows : (int)cols;
    const SvdWs W{(uint32_t)M, (uint32_t)N};
    const float* w = ws + mat * W.per();
    const int bad = __float_as_int(w[W.meta() + 1]);
    const float nanv = qnan();

    // U_p = H_0 ... H_{N-1} [U_B; 0], lane c its column c
    float x[kMaxM];
#pragma unroll
    for (int r = 0; r < kMaxM; ++r) x[r] = (c < N && r < N) ? w[W.ub() + (size_t)r * N + c] : 0.0f;
    for (int k = N - 1; k >= 0; --k) {
        const float tau = w[W.tq() + k];
        if (tau == 0.0f) continue;   // uniform
        const float* v = w + W.refl() + (size_t)k * M;
        float d = 0.0f;
#pragma unroll
        for (int r = 0; r < kMaxM; ++r)
            if (r < M) d = fmaf(v[r], x[r], d);   // v[r] = 0 above k
        d *= tau;
#pragma unroll
        for (int r = 0; r < kMaxM; ++r)
            if (r < M) x[r] = fmaf(-d, v[r], x[r]);
    }
    // V_p = G_0 ... G_{N-2} V_B, lane c its column c
    float y[kMaxN];
#pragma unroll
    for (int j = 0; j < kMaxN; ++j) y[j] = (c < N && j < N) ? w[W.vb() + (size_t)j * N + c] : 0.0f;
    for (int k = N - 2; k >= 0; --k) {
        const float tau = w[W.tp() + k];
        if (tau == 0.0f) continue;
        const float* u = w + W.refr() + (size_t)k * N;
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxN; ++j)
            if (j < N) d = fmaf(u[j], y[j], d);
        d *= tau;
#pragma unroll
        for (int j = 0; j < kMaxN; ++j)
            if (j < N) y[j] = fmaf(-d, u[j], y[j]);
    }
    // outputs: tall: U = U_p (M x N), Vt = V_p^T (N x N).
    //          wide: U = V_p (rows x rows), Vt = U_p^T (rows x cols).
    if (!trans) {
        float* uo = U + mat * (size_t)M * N;
        if (c < N) {
#pragma unroll
            for (int r = 0; r < kMaxM; ++r)
                if (r < M) uo[(size_t)r * N + c] = bad ? nanv : x[r];
        }
        if (c < N) {
#pragma unroll
            for (int j = 0; j < kMaxN; ++j) tr[c][j] = y[j];
        }
        wave_lds_sync();
        float* vo = Vt + mat * (size_t)N * N;
        if (c < N)
            for (int i = 0; i < N; ++i) vo[(size_t)i * N + c] = bad ? nanv : tr[i][c];
    } else {
        // U (rows x rows) = V_p: lane c writes its column
        float* uo = U + mat * (size_t)N * N;
        if (c < N) {
#pragma unroll
            for (int j = 0; j < kMaxN; ++j)
                if (j < N) uo[(size_t)j * N + c] = bad ? nanv : y[j];
        }
        // Vt (rows x cols) = U_p^T: row c of Vt is lane c's column
        float* vo = Vt + mat * (size_t)N * M;
        if (c < N) {
#pragma unroll
            for (int r = 0; r < kMaxM; ++r)
                if (r < M) vo[(size_t)c * M + r] = bad ? nanv : x[r];
        }
    }
}

}  // namespace

bool svd_small_fits(uint32_t m, uint32_t n) {
    const uint32_t k = m < n ? m : n, l = m < n ? n : m;
    return k >= 1 && k <= (uint32_t)kMaxN && l <= (uint32_t)kMaxM;
}

size_t svd_small_workspace(uint32_t m, uint32_t n, uint32_t batch) {
    const uint32_t K = m < n ? m : n, L = m < n ? n : m;
    const SvdWs W{L, K};
    return W.per() * batch * sizeof(float);
}

void svd_small(const float* a, float* u, float* s, float* vt, uint32_t* info, float* ws, uint32_t batch, uint32_t m,
               uint32_t n, hipStream_t st) {
    if (!svd_small_fits(m, n)) invalid("[svd] svd_small takes min(m, n) <= 64 and max(m, n) <= 128");
    if (batch == 0) return;
    const bool trans = m < n;
    const bool vec = u != nullptr;
    const uint32_t Mp = trans ? n : m, Np = trans ? m : n;
    {
        KernelTimer t("svd_bidiag", st);
        hipLaunchKernelGGL(svd_bidiag_kernel, dim3(batch), dim3(64), 0, st, a, ws, batch, m, n, trans ? 1 : 0,
                           vec ? 1 : 0);
        t.stop();
    }
    {
        KernelTimer t("svd_bdsqr", st);
        if (vec)
            hipLaunchKernelGGL((svd_bdsqr_kernel<true>), dim3(batch), dim3(64), 0, st, ws, s, info, batch, Mp, Np);
        else
            hipLaunchKernelGGL((svd_bdsqr_kernel<false>), dim3(batch), dim3(64), 0, st, ws, s, info, batch, Mp, Np);
        t.stop();
    }
    if (vec) {
        KernelTimer t("svd_backtransform", st);
        hipLaunchKernelGGL(svd_backtransform_kernel, dim3(batch), dim3(64), 0, st, ws, u, vt, batch, m, n,
                           trans ? 1 : 0);
        t.stop();
    }
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
