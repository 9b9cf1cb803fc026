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
//   svd_bidiag     lane c holds column c of the problem in VGPRs (rows and
//                  columns beyond the shape zero); left reflectors are
//                  applied lane-locally from LDS broadcasts, right ones
//                  through a transposed reduction in LDS.  Writes d, e, the
//                  reflectors (column-contiguous) and their tau.
//   svd_bdsqr      lane r holds row r of the bidiagonal's U and V in VGPRs;
//                  the Golub-Reinsch recurrence runs on every lane with d
//                  and e in LDS (unrolled sweep, wave-uniform guards), the
//                  lane-parallel split test on the same arrays; then sign
//                  fix, descending sort.
//   svd_backtransform  lane c forms column c of U = Q [U_B; 0] and of
//                  V = P V_B from the reflectors, staged through LDS in
//                  blocks of eight.
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
constexpr int kChunks = kMaxM / 4;   // 4-row chunks of a lane's column

struct BidiagLds {
    float v[kMaxM];       // the left reflector: 0 above row k, 1 at row k
    float w[kMaxM];       // A u for the right reflector u
    float p[64][68];      // products x_c[r] u_c of one half of the rows, [c][r]
};

// Lane c holds column c of the problem in VGPRs (rows >= M and columns >= N
// zero, which every reflector leaves zero).  Step k: lane k publishes its
// column; the norm comes from a wave sum; the reflector goes back to LDS and
// every lane forms v^T x_c and its update from 16-byte broadcasts.  The
// right reflector is row k (element k of every lane's column, read by a
// wave-uniform select), its norm a wave sum; A u is a transposed reduction
// through LDS (lanes store x_c[r] u_c for 64 rows, then lane t sums row t),
// and the update again reads A u as broadcasts.  Row chunks above row k are
// skipped by wave-uniform branches; the rows above k that a chunk still
// covers are finished and never read with a non-zero coefficient.
__global__ __launch_bounds__(64) void svd_bidiag_kernel(const float* __restrict__ A, float* __restrict__ ws,
                                                        uint32_t batch, uint32_t rows, uint32_t cols, int trans,
                                                        int vectors) {
    __shared__ __align__(16) BidiagLds s;
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    if (mat >= batch) return;   // whole wave: uniform
    const int M = trans ? (int)cols : (int)rows;
    const int N = trans ? (int)rows : (int)cols;
    const SvdWs W{(uint32_t)M, (uint32_t)N};
    float* w = ws + mat * W.per();
    const float* src = A + mat * (size_t)rows * cols;

    // load (transposed for a wide input) with clamped indices, scan
    float x[kMaxM];
    const int cc = c < N ? c : N - 1;
#pragma unroll
    for (int r = 0; r < kMaxM; ++r) {
        const int rr = r < M ? r : M - 1;
        const float v = trans ? src[(size_t)cc * cols + rr] : src[(size_t)rr * cols + cc];
        x[r] = (r < M && c < N) ? v : 0.0f;
    }
    float amax = 0.0f, chk = 0.0f;   // chk becomes NaN at a NaN or an infinity
#pragma unroll
    for (int r = 0; r < kMaxM; ++r) {
        amax = fmaxf(amax, fabsf(x[r]));
        chk = fmaf(x[r], 0.0f, chk);
    }
    amax = group_max<64>(amax);
    const int bad = group_or<64>(chk != chk ? 1 : 0);
    const int ex = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < kMaxM; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -ex);

    for (int k = 0; k < N; ++k) {
        const int j0 = k >> 2;   // the chunk holding row k
        // ---- left reflector on column k, rows k.. ----
        if (c == k) {
#pragma unroll
            for (int j = 0; j < kChunks; ++j)
                if (j >= j0)
                    *reinterpret_cast<float4*>(&s.v[4 * j]) = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2],
                                                                          x[4 * j + 3]);
        }
        __syncthreads();
        const float a0 = s.v[c], a1 = s.v[c + 64];   // rows c and c + 64 (> k)
        const float alpha = s.v[k];
        const float l0 = c > k ? a0 : 0.0f;
        const float ss = wave_sum_f(fmaf(l0, l0, a1 * a1));
        float beta = alpha, tau = 0.0f, scale = 1.0f;
        if (ss >= kTinySumsq) {
            // hardware square root, refined reciprocals (about 1 ulp)
            beta = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alpha, alpha, ss)), alpha);
            tau = (beta - alpha) * rcp_refined(beta);
            scale = rcp_refined(alpha - beta);
        }
        __syncthreads();   // every read of column k before the reflector replaces it
        const float v0 = c < k ? 0.0f : (c == k ? 1.0f : a0 * scale);
        const float v1 = a1 * scale;
        s.v[c] = v0;
        s.v[c + 64] = v1;
        if (vectors) {   // v_k, contiguous
            if (c < M) w[W.refl() + (size_t)k * M + c] = v0;
            if (c + 64 < M) w[W.refl() + (size_t)k * M + c + 64] = v1;
        }
        if (c == 0) {
            w[W.d() + k] = beta;
            w[W.tq() + k] = tau;
        }
        __syncthreads();
        if (tau != 0.0f) {   // uniform
            float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
            for (int g8 = 0; g8 < kChunks / 8; ++g8) {
                if (8 * g8 + 7 >= j0) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                    for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                        const float4 vv = *reinterpret_cast<const float4*>(&s.v[4 * j]);
                        d0 = fmaf(vv.x, x[4 * j], d0);
                        d1 = fmaf(vv.y, x[4 * j + 1], d1);
                        d2 = fmaf(vv.z, x[4 * j + 2], d2);
                        d3 = fmaf(vv.w, x[4 * j + 3], d3);
                    }
                }
            }
            const float g = c > k ? tau * ((d0 + d1) + (d2 + d3)) : 0.0f;
#pragma unroll
            for (int g8 = 0; g8 < kChunks / 8; ++g8) {
                if (8 * g8 + 7 >= j0) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                    for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                        const float4 vv = *reinterpret_cast<const float4*>(&s.v[4 * j]);
                        x[4 * j] = fmaf(-g, vv.x, x[4 * j]);
                        x[4 * j + 1] = fmaf(-g, vv.y, x[4 * j + 1]);
                        x[4 * j + 2] = fmaf(-g, vv.z, x[4 * j + 2]);
                        x[4 * j + 3] = fmaf(-g, vv.w, x[4 * j + 3]);
                    }
                }
            }
        }
        if (k + 1 >= N) break;
        // ---- right reflector on row k, columns k+1.. ----
        float xk = 0.0f;   // element k of this lane's column (k < 64)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j == j0) {
                const int q = k & 3;
                xk = q == 0 ? x[4 * j] : (q == 1 ? x[4 * j + 1] : (q == 2 ? x[4 * j + 2] : x[4 * j + 3]));
            }
        }
        const float alr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xk), k + 1));
        const float ur = c > k + 1 ? xk : 0.0f;
        const float ssr = wave_sum_f(ur * ur);
        float br = alr, taur = 0.0f, scr = 1.0f;
        if (ssr >= kTinySumsq) {
            br = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alr, alr, ssr)), alr);
            taur = (br - alr) * rcp_refined(br);
            scr = rcp_refined(alr - br);
        }
        const float up = c == k + 1 ? 1.0f : ur * scr;   // u_c, 0 for c <= k
        if (vectors && c < N) w[W.refr() + (size_t)k * N + c] = up;
        if (c == 0) {
            w[W.e() + k] = br;
            w[W.tp() + k] = taur;
        }
        if (taur != 0.0f) {   // uniform
            // A u, 64 rows at a time
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (h == 1 && M <= 64) break;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int r = 64 * h + 4 * j;
                    *reinterpret_cast<float4*>(&s.p[c][4 * j]) =
                        make_float4(x[r] * up, x[r + 1] * up, x[r + 2] * up, x[r + 3] * up);
                }
                __syncthreads();
                float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int g8 = 0; g8 < 8; ++g8) {
                    if (8 * g8 + 7 > k) {   // columns <= k have u = 0
#pragma unroll
                        for (int q = 0; q < 8; ++q) acc[q] += s.p[8 * g8 + q][c];
                    }
                }
                s.w[64 * h + c] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
                __syncthreads();
            }
            const float gr = taur * up;
#pragma unroll
            for (int g8 = 0; g8 < kChunks / 8; ++g8) {
                if (8 * g8 + 7 >= j0 && 32 * g8 < M) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                    for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                        const float4 ww = *reinterpret_cast<const float4*>(&s.w[4 * j]);
                        x[4 * j] = fmaf(-gr, ww.x, x[4 * j]);
                        x[4 * j + 1] = fmaf(-gr, ww.y, x[4 * j + 1]);
                        x[4 * j + 2] = fmaf(-gr, ww.z, x[4 * j + 2]);
                        x[4 * j + 3] = fmaf(-gr, ww.w, x[4 * j + 3]);
                    }
                }
            }
        }
    }
    if (c == 0) {
        w[W.e() + N - 1] = 0.0f;
        w[W.tp() + N - 1] = 0.0f;
        w[W.meta()] = __int_as_float(ex);
        w[W.meta() + 1] = __int_as_float(bad);
    }
    if (vectors && c < N) w[W.refr() + (size_t)(N - 1) * N + c] = 0.0f;
}

// ---------------------------------------------------------------- bdsqr
struct BdLds {
    float q[kMaxN + 1];
    float e[kMaxN + 1];   // Golub-Reinsch convention: e[i] couples (i-1, i), e[0] = 0
    float st[kMaxN][kMaxN + 1];
    int perm[kMaxN];
};

// (c, s, r) of the rotation taking (f, h) to (r, 0).  A pair with
// f^2 + h^2 below 2^-100 (entries below 2^-50, far under the convergence
// tolerance of a matrix scaled into [0.5, 1)) gives the identity and r = 0:
// an orthogonal rotation either way, off by less than 2^-50 in what it
// leaves behind, and never a rotation built from a subnormal sum of squares.
// Branch-free; 1/sqrt(f^2 + h^2) is the hardware's (v_rsq_f32, about one
// ulp: a Newton step on it measured no gain in the orthogonality of U and V
// at config 3, 1.3e-5 with it against 8.7e-6 without).
__device__ __forceinline__ float rot(float f, float h, float& c, float& s) {
    const float sq = fmaf(f, f, h * h);
    const bool ok = sq >= 0x1p-100f;
    const float ri = ok ? __builtin_amdgcn_rsqf(sq) : 0.0f;
    c = ok ? f * ri : 1.0f;
    s = h * ri;
    return sq * ri;
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

    // q and e live in LDS only (every lane reads the same entries); the
    // VGPRs hold this lane's rows of U_B and V_B
    float xu[VEC ? NN : 1], xv[VEC ? NN : 1];
    if (VEC) {
#pragma unroll
        for (int i = 0; i < NN; ++i) {
            xu[i] = i == lane ? 1.0f : 0.0f;
            xv[i] = i == lane ? 1.0f : 0.0f;
        }
    }
    {
        const float qv = lane < n ? w[W.d() + (lane < n ? lane : 0)] : 0.0f;
        const float ev = (lane >= 1 && lane < n) ? w[W.e() + (lane >= 1 ? lane - 1 : 0)] : 0.0f;
        s.q[lane] = qv;
        s.e[lane] = ev;
        if (lane == 0) {
            s.q[NN] = 0.0f;
            s.e[NN] = 0.0f;
        }
    }
    const float anorm = group_max<64>(fabsf(s.q[lane]) + fabsf(s.e[lane]));
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
            int l = 63 - __clzll((long long)any);
            // opaque to the optimiser: otherwise every unrolled test j >= l
            // becomes a 64-bit compare of the ballot with 2^j, and the 64
            // constants stay live in VGPRs
            asm volatile("" : "+s"(l));
            const bool cancel = !((__ballot(se) >> l) & 1ull);
            if (cancel) {
                // e[l] is cancelled by rotations of rows (l-1, i), i = l..k
                const int nm = l - 1;
                float cc = 0.0f, sn = 1.0f;
                float unm = 0.0f;
                // xu[nm] by wave-uniform branches (the asm keeps them branches:
                // selects here would hold 64 lane masks live across the loop)
                if (VEC) {
#pragma unroll
                    for (int j = 0; j < NN; ++j)
                        if (j == nm) {
                            asm volatile("");
                            unm = xu[j];
                        }
                }
                bool done = false;
#pragma unroll
                for (int i = 0; i < NN; ++i) {
                    if (i >= l && i <= k && !done) {
                        const float ei = s.e[i];
                        const float f = sn * ei;
                        s.e[i] = cc * ei;
                        if (fabsf(f) <= tol) {
                            done = true;
                        } else {
                            const float g = s.q[i];
                            float c2, s2;
                            const float h = rot(g, f, c2, s2);
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
                    for (int j = 0; j < NN; ++j)
                        if (j == nm) {
                            asm volatile("");
                            xu[j] = unm;
                        }
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
            // e[j+1] and q[j+1] are read one rotation ahead: step j writes
            // only e[j] and q[j], so step j+1's entries are final when step
            // j starts, and their LDS latency hides behind step j's chain
            float gn = s.e[l + 1], yn = s.q[l + 1];
#pragma unroll
            for (int j = 0; j < NN - 1; ++j) {
                // l and k laundered per step: two scalar compares here,
                // instead of the 63 compares precomputed at the sweep's start
                // and spilled to VGPR lanes
                int lj = l, kj = k;
                asm volatile("" : "+s"(lj), "+s"(kj));
                if (j >= lj && j < kj) {
                    const int i = j + 1;
                    float g = gn;
                    float y = yn;
                    gn = s.e[j + 2 <= NN ? j + 2 : NN];
                    yn = s.q[j + 2 <= NN ? j + 2 : NN];
                    float h = sn * g;
                    g = c * g;
                    float cz, sz;
                    const float z1 = rot(f, h, cz, sz);
                    s.e[j] = z1;   // e[l] becomes 0 after the sweep
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
                }
            }
            s.e[l] = 0.0f;
            s.e[k] = f;
            s.q[k] = x;
            wave_lds_sync();
        }
    }

    // signs: non-negative values, the matching V columns negated
    wave_lds_sync();
    {
        const float qv = s.q[lane];
        const uint64_t neg = __ballot(lane < n && qv < 0.0f);
        if (VEC) {
#pragma unroll
            for (int j = 0; j < NN; ++j) xv[j] = ((neg >> j) & 1ull) ? -xv[j] : xv[j];
        }
        wave_lds_sync();
        if (lane < n) s.q[lane] = fabsf(qv);
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
constexpr int kRB = 8;   // reflectors staged per block

union BackLds {
    struct {
        float v[2][kRB][kMaxM];   // two blocks of reflectors
        float tau[2][kRB];
    };
    float tr[kMaxN][kMaxN + 1];   // V_p, transposed on the way out
};

// Lane c holds column c of U_B (then V_B) in VGPRs.  Reflectors move in
// blocks of kRB: the wave loads the next block (two rows per lane and
// reflector) while it applies the current one from LDS, read back as
// 16-byte broadcasts; chunks above a reflector's first non-zero row are
// skipped (wave-uniform).
__global__ __launch_bounds__(64) void svd_backtransform_kernel(const float* __restrict__ ws, float* __restrict__ U,
                                                               float* __restrict__ Vt, uint32_t batch, uint32_t rows,
                                                               uint32_t cols, int trans) {
    __shared__ __align__(16) BackLds sb;
    auto& tr = sb.tr;
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    if (mat >= batch) return;
    const int M = trans ? (int)cols : (int)rows;
    const int N = trans ? (int)rows : (int)cols;
    const SvdWs W{(uint32_t)M, (uint32_t)N};
    const float* w = ws + mat * W.per();
    const int bad = __float_as_int(w[W.meta() + 1]);
    const float nanv = qnan();
    const int cc = c < N ? c : N - 1;

    // U_p = H_0 ... H_{N-1} [U_B; 0]
    float x[kMaxM];
#pragma unroll
    for (int r = 0; r < kMaxN; ++r) {
        const float v = w[W.ub() + (size_t)(r < N ? r : N - 1) * N + cc];
        x[r] = (c < N && r < N) ? v : 0.0f;
    }
#pragma unroll
    for (int r = kMaxN; r < kMaxM; ++r) x[r] = 0.0f;
    {
        const int c0 = c < M ? c : M - 1, c1 = c + 64 < M ? c + 64 : M - 1;
        float n0[kRB], n1[kRB], tn = 0.0f;
        // reflectors kb, kb - 1, .., kb - kRB + 1 (those below 0 clamped, unused)
        auto fetch = [&](int kb) {
#pragma unroll
            for (int i = 0; i < kRB; ++i) {
                const float* v = w + W.refl() + (size_t)max(kb - i, 0) * M;
                // raw values: masked when staged, a block later (a select
                // here would wait for the loads at once)
                n0[i] = v[c0];
                n1[i] = v[c1];
            }
            tn = w[W.tq() + max(kb - min(c, kRB - 1), 0)];   // stored by lanes c < kRB only
        };
        fetch(N - 1);
        for (int kb = N - 1, blk = 0; kb >= 0; kb -= kRB, ++blk) {
            float(*vk)[kMaxM] = sb.v[blk & 1];
#pragma unroll
            for (int i = 0; i < kRB; ++i) {
                vk[i][c] = c < M ? n0[i] : 0.0f;
                vk[i][c + 64] = c + 64 < M ? n1[i] : 0.0f;
            }
            if (c < kRB) sb.tau[blk & 1][c] = tn;
            if (kb - kRB >= 0) fetch(kb - kRB);
            __syncthreads();
#pragma unroll 1
            for (int i = 0; i < kRB && kb - i >= 0; ++i) {
                const int k = kb - i;
                const float tau = sb.tau[blk & 1][i];
                if (tau == 0.0f) continue;   // uniform
                const float* vr = vk[i];
                const int j0 = k >> 2;       // v_k is zero above row k
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
                for (int g8 = 0; g8 < kChunks / 8; ++g8) {
                    if (8 * g8 + 7 >= j0 && 32 * g8 < M) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                        for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                            const float4 vv = *reinterpret_cast<const float4*>(&vr[4 * j]);
                            d0 = fmaf(vv.x, x[4 * j], d0);
                            d1 = fmaf(vv.y, x[4 * j + 1], d1);
                            d2 = fmaf(vv.z, x[4 * j + 2], d2);
                            d3 = fmaf(vv.w, x[4 * j + 3], d3);
                        }
                    }
                }
                const float g = tau * ((d0 + d1) + (d2 + d3));
#pragma unroll
                for (int g8 = 0; g8 < kChunks / 8; ++g8) {
                    if (8 * g8 + 7 >= j0 && 32 * g8 < M) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                        for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                            const float4 vv = *reinterpret_cast<const float4*>(&vr[4 * j]);
                            x[4 * j] = fmaf(-g, vv.x, x[4 * j]);
                            x[4 * j + 1] = fmaf(-g, vv.y, x[4 * j + 1]);
                            x[4 * j + 2] = fmaf(-g, vv.z, x[4 * j + 2]);
                            x[4 * j + 3] = fmaf(-g, vv.w, x[4 * j + 3]);
                        }
                    }
                }
            }
        }
    }
    // V_p = G_0 ... G_{N-2} V_B
    float y[kMaxN];
#pragma unroll
    for (int j = 0; j < kMaxN; ++j) {
        const float v = w[W.vb() + (size_t)(j < N ? j : N - 1) * N + cc];
        y[j] = (c < N && j < N) ? v : 0.0f;
    }
    __syncthreads();   // the last U block's reads before the buffers are reused
    if (N >= 2) {
        float n0[kRB], tn = 0.0f;
        auto fetch = [&](int kb) {
#pragma unroll
            for (int i = 0; i < kRB; ++i) {
                n0[i] = w[W.refr() + (size_t)max(kb - i, 0) * N + cc];   // masked when staged
            }
            tn = w[W.tp() + max(kb - min(c, kRB - 1), 0)];
        };
        fetch(N - 2);
        for (int kb = N - 2, blk = 0; kb >= 0; kb -= kRB, ++blk) {
            float(*uk)[kMaxM] = sb.v[blk & 1];
#pragma unroll
            for (int i = 0; i < kRB; ++i) uk[i][c] = c < N ? n0[i] : 0.0f;
            if (c < kRB) sb.tau[blk & 1][c] = tn;
            if (kb - kRB >= 0) fetch(kb - kRB);
            __syncthreads();
#pragma unroll 1
            for (int i = 0; i < kRB && kb - i >= 0; ++i) {
                const int k = kb - i;
                const float tau = sb.tau[blk & 1][i];
                if (tau == 0.0f) continue;
                const float* ur = uk[i];
                const int j0 = (k + 1) >> 2;   // u_k is zero above entry k + 1
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
                for (int g8 = 0; g8 < kMaxN / 32; ++g8) {
                    if (8 * g8 + 7 >= j0 && 32 * g8 < N) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                        for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                            const float4 uu = *reinterpret_cast<const float4*>(&ur[4 * j]);
                            d0 = fmaf(uu.x, y[4 * j], d0);
                            d1 = fmaf(uu.y, y[4 * j + 1], d1);
                            d2 = fmaf(uu.z, y[4 * j + 2], d2);
                            d3 = fmaf(uu.w, y[4 * j + 3], d3);
                        }
                    }
                }
                const float g = tau * ((d0 + d1) + (d2 + d3));
#pragma unroll
                for (int g8 = 0; g8 < kMaxN / 32; ++g8) {
                    if (8 * g8 + 7 >= j0 && 32 * g8 < N) {   // 8 chunks at a time: one LDS wait per group
#pragma unroll
                        for (int j = 8 * g8; j < 8 * g8 + 8; ++j) {
                            const float4 uu = *reinterpret_cast<const float4*>(&ur[4 * j]);
                            y[4 * j] = fmaf(-g, uu.x, y[4 * j]);
                            y[4 * j + 1] = fmaf(-g, uu.y, y[4 * j + 1]);
                            y[4 * j + 2] = fmaf(-g, uu.z, y[4 * j + 2]);
                            y[4 * j + 3] = fmaf(-g, uu.w, y[4 * j + 3]);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();   // the last V block's reads before the transpose buffer
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
        __syncthreads();
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
