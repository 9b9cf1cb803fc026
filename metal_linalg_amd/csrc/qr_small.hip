// Batched Householder QR of small matrices (rows <= 64, columns <= 64), one
// matrix per lane group of a wave64, held in registers.
//
// Role: the MI355X counterpart of the reference's qr_householder_simd
// (reference: shaders/QR_Householder.metal:189-300, driver
// src/qr_householder.mm:293-381): LAPACK's sgeqr2 + sorg2r per matrix, with
// the reference GPU kernel's conventions -- the matrix scaled by a power of
// two so that its largest entry lies in [0.5, 1), a reflector whose tail has
// a sum of squares below 2^-80 taken as the identity, R unscaled on output,
// and a matrix holding a NaN or an infinity written as all quiet NaN.
//
// Layout (MI355X-first, not the reference's): lane c of a G-lane group owns
// column c of its matrix, all of its rows in VGPRs, so a column's dot
// product with a reflector is a lane-local FMA chain and no cross-lane
// reduction is needed; the reflector itself is broadcast through LDS.  A
// row-major matrix read this way is coalesced: for a fixed row the group's
// lanes read consecutive floats.  64/G matrices share a wave; one wave per
// workgroup, so the LDS hand-offs need no s_barrier.
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80

template <int G, int R>
__global__ __launch_bounds__(64) void qr_small_kernel(const float* __restrict__ A, float* __restrict__ Q,
                                                      float* __restrict__ Rout, uint32_t batch, uint32_t m,
                                                      uint32_t n, uint32_t qc, uint32_t rr) {
    constexpr int MPW = 64 / G;
    __shared__ float vsh[MPW][R];
    __shared__ float tsh[MPW][64];
    const int lane = threadIdx.x;
    const int c = lane % G;
    const int g = lane / G;
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;
    const int K = (int)(m < n ? m : n);

    float x[R];
    float amax = 0.0f;
    int bad = 0;
    const float* src = A + mat * m * n;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = 0.0f;
        if (live && r < (int)m && c < (int)n) v = src[(size_t)r * n + c];
        x[r] = v;
        amax = fmaxf(amax, fabsf(v));
        bad |= !finite_f(v);
    }
    amax = group_max<G>(amax);
    bad = group_or<G>(bad);
    const int e = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < R; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -e);

    // sgeqr2: column j's reflector H_j = I - tau v v^T, v(j) = 1
    for (int j = 0; j < K; ++j) {
        float ss = 0.0f, alpha = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ss = r > j ? fmaf(x[r], x[r], ss) : ss;
            alpha = r == j ? x[r] : alpha;
        }
        float beta = alpha, tau = 0.0f, scale = 1.0f;
        if (ss >= kTinySumsq) {
            beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
            tau = (beta - alpha) / beta;
            scale = 1.0f / (alpha - beta);
        }
        if (c == j) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = r < j ? 0.0f : (r == j ? 1.0f : x[r] * scale);
                vsh[g][r] = v;
                x[r] = r == j ? beta : (r > j ? v : x[r]);
            }
            tsh[g][j] = tau;
        }
        wave_lds_sync();
        if (c > j) {
            const float t = tsh[g][j];
            float d = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) d = r >= j ? fmaf(vsh[g][r], x[r], d) : d;
            d *= t;
#pragma unroll
            for (int r = 0; r < R; ++r) x[r] = r >= j ? fmaf(-d, vsh[g][r], x[r]) : x[r];
        }
        wave_lds_sync();
    }

    // R: rows below K are zero (complete mode), the strict lower part zero
    if (live) {
        float* out_r = Rout + mat * rr * n;
        const float unscale = ldexpf(1.0f, e);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r < (int)rr && c < (int)n) {
                float v = (r < K && c >= r) ? x[r] * unscale : 0.0f;
                out_r[(size_t)r * n + c] = bad ? qnan() : v;
            }
        }
    }
    if (qc == 0) return;

    // sorg2r backward: columns >= K of a square Q start as the identity's
    if (c >= K) {
#pragma unroll
        for (int r = 0; r < R; ++r) x[r] = r == c ? 1.0f : 0.0f;
    }
    for (int j = K - 1; j >= 0; --j) {
        if (c == j) {
#pragma unroll
            for (int r = 0; r < R; ++r) vsh[g][r] = r < j ? 0.0f : (r == j ? 1.0f : x[r]);
        }
        wave_lds_sync();
        const float t = tsh[g][j];
        if (c > j && c < (int)qc) {
            float d = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) d = r >= j ? fmaf(vsh[g][r], x[r], d) : d;
            d *= t;
#pragma unroll
            for (int r = 0; r < R; ++r) x[r] = r >= j ? fmaf(-d, vsh[g][r], x[r]) : x[r];
        } else if (c == j) {
#pragma unroll
            for (int r = 0; r < R; ++r) x[r] = r < j ? 0.0f : (r == j ? 1.0f - t : -t * x[r]);
        }
        wave_lds_sync();
    }
    if (live && c < (int)qc) {
        float* out_q = Q + mat * m * qc;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < (int)m) out_q[(size_t)r * qc + c] = bad ? qnan() : x[r];
    }
}

// Sum of x[r] * y[r] for r in [lo, M), four partial sums to shorten the
// dependent FMA chain; everything compile-time.
template <int LO, int M>
__device__ __forceinline__ float dot_from(const float* x, const float* y) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int r = LO; r < M; r += 4) {
        s0 = fmaf(x[r], y[r], s0);
        if (r + 1 < M) s1 = fmaf(x[r + 1], y[r + 1], s1);
        if (r + 2 < M) s2 = fmaf(x[r + 2], y[r + 2], s2);
        if (r + 3 < M) s3 = fmaf(x[r + 3], y[r + 3], s3);
    }
    return (s0 + s1) + (s2 + s3);
}

// The value of lane j of this lane's G-lane group, on every lane.
template <int G>
__device__ __forceinline__ float group_lane(float v, int j, int lane) {
    if constexpr (G == 64) {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
    } else if constexpr (G == 32) {
        // five VALU instructions (the SGPR results go back to VGPRs for the
        // half-select), but off LDS: an LDS permute here put its round trip
        // on every step's critical path (config 1: 71.5 -> 73.9 us)
        const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
        const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j + 32));
        return lane >= 32 ? hi : lo;
    } else {
        return __shfl(v, (lane & ~(G - 1)) + j, 64);
    }
}

// Rows LO .. M-1 of a column between registers and LDS as 16-byte pieces,
// from the aligned row at or before LO (the rows before LO that this moves
// are ignored by the reader).
template <int LO, int M, int LD>
__device__ __forceinline__ void put_rows(float (&vsh)[LD], const float (&x)[M]) {
#pragma unroll
    for (int r = LO / 4 * 4; r < M; r += 4)
        *reinterpret_cast<float4*>(&vsh[r]) = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
}
template <int LO, int M, int LD>
__device__ __forceinline__ void get_rows(float (&v)[M], const float (&vsh)[LD]) {
#pragma unroll
    for (int r = LO / 4 * 4; r < M; r += 4) {
        const float4 q = *reinterpret_cast<const float4*>(&vsh[r]);
        v[r] = q.x;
        v[r + 1] = q.y;
        v[r + 2] = q.z;
        v[r + 3] = q.w;
    }
}

// Factorization step J of the fixed-shape kernel (compile-time J, so every
// row predicate folds away and only rows >= J are touched).  Every lane
// forms the reflector from lane J's column (alpha and the tail's sum of
// squares read across lanes) with the hardware square root and refined
// reciprocals; lane J publishes its column unscaled, the other lanes fold
// the scale into their products, and each lane keeps the scale of its own
// reflector to apply once after the last step.  Every lane runs the same
// instructions, its part selected by a coefficient (zero for lanes at or
// left of J): a divergent branch here would make the compiler copy the
// column at every merge, as many moves as the step has multiply-adds.  The
// lane index is laundered per step, or the compiler precomputes the lane
// masks of every step at entry and spills them.
template <int J, int M, int N, int G, int LD>
__device__ __forceinline__ void qr_fixed_step(float (&x)[M], float (&vsh)[LD], float* tsh, int c, int lane,
                                              float& myscale) {
    if constexpr (J < (M < N ? M : N)) {
        int cl = c;
        __asm__ volatile("" : "+v"(cl));
        const float alpha = group_lane<G>(x[J], J, lane);
        const float ss = group_lane<G>(dot_from<J + 1, M>(x, x), J, lane);
        const bool nz = ss >= kTinySumsq;
        const float b = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alpha, alpha, ss)), alpha);
        const float beta = nz ? b : alpha;
        const float tau = nz ? (b - alpha) * rcp_refined(b) : 0.0f;
        const float sc = nz ? rcp_refined(alpha - b) : 1.0f;
        if (cl == J) {   // stores only: no register changes inside
            put_rows<J + 1, M, LD>(vsh, x);
            tsh[J] = tau;
        }
        myscale = cl == J ? sc : myscale;
        wave_lds_sync();
        float v[M];
        get_rows<J + 1, M, LD>(v, vsh);
        const float d0 = tau * fmaf(sc, dot_from<J + 1, M>(v, x), x[J]);
        const float d = cl > J ? d0 : 0.0f;
        const float ds = d * sc;
        x[J] = cl == J ? beta : x[J] - d;
#pragma unroll
        for (int r = J + 1; r < M; ++r) x[r] = fmaf(-ds, v[r], x[r]);
        wave_lds_sync();
        qr_fixed_step<J + 1, M, N, G, LD>(x, vsh, tsh, c, lane, myscale);
    }
}

// Q formation step J (backward, sorg2r), for J = K-1 down to 0.  Lane J
// holds its reflector v (1 at row J, zero above, set before the first step)
// and becomes e_J - tau v; lanes right of J lose tau (v . x) v; the others
// keep their column.  In one form for every lane: x - beta v, plus 1 at row
// J in lane J, with beta = tau + 1 in lane J (x = v there), tau (v . x)
// right of J and 0 left of it.
template <int J, int M, int K, int LD>
__device__ __forceinline__ void qr_fixed_qstep(float (&x)[M], float (&vsh)[LD], const float* tsh, int c, int qc) {
    if constexpr (J >= 0) {
        int cl = c;
        __asm__ volatile("" : "+v"(cl));
        if (cl == J) put_rows<J, M, LD>(vsh, x);
        wave_lds_sync();
        const float t = tsh[J];
        float v[M];
        get_rows<J, M, LD>(v, vsh);
        const float dot = t * dot_from<J, M>(v, x);
        const float beta = cl == J ? t + 1.0f : (cl > J && cl < qc ? dot : 0.0f);
#pragma unroll
        for (int r = J; r < M; ++r) x[r] = fmaf(-beta, v[r], x[r]);
        x[J] += cl == J ? 1.0f : 0.0f;
        wave_lds_sync();
        qr_fixed_qstep<J - 1, M, K, LD>(x, vsh, tsh, c, qc);
    }
}

// Fixed-shape variant for M >= N known at compile time (the hot batched
// shapes): the column loop is unrolled, so row predicates vanish and step j
// touches rows j.. only.  qc is 0 (R alone) or N.  (Two groups of matrices
// per wave, the second's loads in flight during the first's arithmetic, ran
// slower at config 1: 82.9 against 71.2 us, the lower occupancy costing more
// than the overlap gained.)
template <int M, int N, int G>
__global__ __launch_bounds__(64) void qr_fixed_kernel(const float* __restrict__ A, float* __restrict__ Q,
                                                      float* __restrict__ Rout, uint32_t batch, uint32_t qc) {
    constexpr int MPW = 64 / G;
    constexpr int LD = M + 4;   // per-group stride (16-byte multiple), off the other group's banks
    __shared__ float vsh[MPW][LD];
    __shared__ float tsh[MPW][N];
    const int lane = threadIdx.x;
    const int c = lane % G;
    const int g = lane / G;
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;

    float x[M];
    float amax = 0.0f;
    int bad = 0;
    const float* src = A + mat * M * N;
#pragma unroll
    for (int r = 0; r < M; ++r) {
        float v = 0.0f;
        if (live && c < N) v = src[(size_t)r * N + c];
        x[r] = v;
        amax = fmaxf(amax, fabsf(v));
        bad |= !finite_f(v);
    }
    amax = group_max<G>(amax);
    bad = group_or<G>(bad);
    const int e = bad ? 0 : scale_exponent(amax);
    // a matrix with a NaN or an infinity is factored as it is (the non-finite
    // values stay inside its lane group: every exchange, LDS rows, readlanes
    // and shuffles, is within the group) and written as NaN below
#pragma unroll
    for (int r = 0; r < M; ++r) x[r] = ldexpf(x[r], -e);

    float myscale = 1.0f;
    qr_fixed_step<0, M, N, G, LD>(x, vsh[g], tsh[g], c, lane, myscale);

    if (live && c < N) {
        float* out_r = Rout + mat * N * N;
        const float unscale = bad ? qnan() : ldexpf(1.0f, e);   // 0 * NaN: the zeros below too
#pragma unroll
        for (int r = 0; r < N; ++r) out_r[(size_t)r * N + c] = (c >= r ? x[r] : 0.0f) * unscale;
    }
    if (qc == 0) return;
    // lane c's column becomes its reflector, scaled now: 1 at row c, zero
    // above (the columns of a square Q past K do not exist here: M >= N = K)
#pragma unroll
    for (int r = 0; r < M; ++r) x[r] = r < c ? 0.0f : (r == c ? 1.0f : x[r] * myscale);
    qr_fixed_qstep<N - 1, M, N, LD>(x, vsh[g], tsh[g], c, (int)qc);
    if (live && c < N) {
        float* out_q = Q + mat * M * N;
        if (__ballot(bad) == 0) {   // uniform: no select per entry
#pragma unroll
            for (int r = 0; r < M; ++r) out_q[(size_t)r * N + c] = x[r];
        } else {
#pragma unroll
            for (int r = 0; r < M; ++r) out_q[(size_t)r * N + c] = bad ? qnan() : x[r];
        }
    }
}

template <int M, int N, int G>
void launch_fixed(const float* a, float* q, float* r, uint32_t batch, uint32_t qc, hipStream_t s) {
    constexpr int MPW = 64 / G;
    KernelTimer t("qr_small", s);
    hipLaunchKernelGGL((qr_fixed_kernel<M, N, G>), dim3((uint32_t)cdiv(batch, MPW)), dim3(64), 0, s, a, q, r, batch,
                       qc);
    t.stop();
}

template <int G, int R>
void launch_g_r(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
                hipStream_t s) {
    constexpr int MPW = 64 / G;
    const uint64_t blocks = cdiv(batch, MPW);
    KernelTimer t("qr_small", s);
    hipLaunchKernelGGL((qr_small_kernel<G, R>), dim3((uint32_t)blocks), dim3(64), 0, s, a, q, r, batch, m, n, qc, rr);
    t.stop();
}

template <int G>
void launch_g(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
              hipStream_t s) {
    if (m <= 8) launch_g_r<G, 8>(a, q, r, batch, m, n, qc, rr, s);
    else if (m <= 16) launch_g_r<G, 16>(a, q, r, batch, m, n, qc, rr, s);
    else if (m <= 32) launch_g_r<G, 32>(a, q, r, batch, m, n, qc, rr, s);
    else launch_g_r<G, 64>(a, q, r, batch, m, n, qc, rr, s);
}

}  // namespace

bool qr_small_fits(uint32_t m, uint32_t n, uint32_t qc) {
    return m <= 64 && n <= 64 && qc <= 64 && m >= 1 && n >= 1;
}

void qr_small(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
              hipStream_t s) {
    if (!qr_small_fits(m, n, qc)) invalid("[qr] qr_small takes at most 64 rows and 64 columns");
    if (batch == 0) return;
    if (m == n && (qc == 0 || qc == n) && rr == n) {
        switch (n) {
            case 8: launch_fixed<8, 8, 8>(a, q, r, batch, qc, s); MLA_HIP(hipGetLastError()); return;
            case 16: launch_fixed<16, 16, 16>(a, q, r, batch, qc, s); MLA_HIP(hipGetLastError()); return;
            case 32: launch_fixed<32, 32, 32>(a, q, r, batch, qc, s); MLA_HIP(hipGetLastError()); return;
            case 64: launch_fixed<64, 64, 64>(a, q, r, batch, qc, s); MLA_HIP(hipGetLastError()); return;
            default: break;
        }
    }
    const uint32_t w = n > qc ? n : qc;
    if (w <= 8) launch_g<8>(a, q, r, batch, m, n, qc, rr, s);
    else if (w <= 16) launch_g<16>(a, q, r, batch, m, n, qc, rr, s);
    else if (w <= 32) launch_g<32>(a, q, r, batch, m, n, qc, rr, s);
    else launch_g<64>(a, q, r, batch, m, n, qc, rr, s);
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
