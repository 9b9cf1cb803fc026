// Batched symmetric eigendecomposition of mid-size matrices (65 <= n <= 128),
// one matrix per workgroup of two waves, in registers.
//
// Role: the MI355X counterpart of the reference's eigh_ql kernel past the
// 64-column window of eigh_small (reference: shaders/Eigh_QL.metal:229-485,
// driver src/eigh_ql.mm:151-266, which takes n up to about 87 on its
// threadgroup memory), so that a batch of such matrices is one launch
// instead of one blocked factorisation per matrix.  The method and contract
// are eigh_small's (eigh_small.hip): Householder tridiagonalisation
// (ssytd2), every eigenvalue by bisection on Sturm counts (sstebz's rule)
// after one multisection pass, every eigenvector by inverse iteration with
// partial pivoting (slagtf / slagts as in sstein) in two steps from a
// pseudo-random start, modified Gram-Schmidt inside groups of eigenvalues
// closer than 1e-3 |T|, and the back-transformation by the reflectors.  The
// read triangle only; the matrix scaled by a power of two into [0.5, 1) and
// the values unscaled after; a NaN or an infinity in the read triangle gives
// all-NaN w and V with info bit 17; otherwise info = bisection steps | bit 16.
//
// MI355X layout: thread c of 128 owns column c of the working matrix (rows
// past n zero), N = 16 MC rows in VGPRs (MC = ceil(n / 16)).  The steps run
// as loops over row chunks of 16 whose ranges are compile-time per phase
// (the chunk holding the step's row), so the register arrays are never
// indexed at run time.  Block-wide sums go through DPP wave sums and two
// LDS words; the reflector and w of the rank-2 update are broadcast through
// LDS.  Where T splits, each unreduced block is bisected and solved on its
// own rows (sstebz / sstein per block) and the pairs are ranked after.  Two
// launches: the first tridiagonalises, bisects and writes w (and, with
// vectors, the state the second needs: d, e, 1/e, tau, and per thread the
// eigenvalue, its block and its rank); the second solves for the
// vectors, keeping the pivoted factor's upper entries in a per-matrix
// scratch laid out [row][thread] (coalesced: 128 VGPRs more would halve the
// waves per SIMD), and back-transforms by the reflectors that the first
// left packed in V's storage.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int kMax = 128;       // the largest order
constexpr int kMin = 65;        // the smallest (below: eigh_small)
constexpr int kC = 16;          // rows per chunk
constexpr int kThreads = 128;   // two waves
constexpr float kEps = 5.9604645e-08f;        // 2^-24, fp32 unit roundoff
constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80: a reflector below it is the identity
constexpr float kSafeMin = 1.17549435e-38f;   // FLT_MIN
constexpr float kPad = 0x1p100f;              // the diagonal of padding rows: never counted
constexpr float kOrtol = 1e-3f;               // close eigenvalues: gap <= kOrtol |T| (sstein's ORTOL)
constexpr int kMaxBisect = 64;
constexpr int kBT = 8;                        // reflectors staged per back-transform block
// per matrix, between the launches: d, e, 1/e, tau, the eigenvalue, its
// block's rows [bs, be) and its rank of each thread, then tnorm, the
// all-blocks-of-one-row flag and bad
constexpr int kStateFloats = 8 * kMax + 4;

struct alignas(16) MidLds {
    float vr[2][kMax + 4];   // the current reflector (v_K[K+1] = 1), alternate steps
    float bc[2][kMax + 4];   // w of the rank-2 update, alternate steps
    float d[kMax + 4];       // the tridiagonal, rows >= n padded with kPad
    float e[kMax + 4];       // e[k] couples rows k and k+1; zero at splits and from row n - 1 on
    float f[kMax + 4];       // f[k] = e[k-1]^2, f[0] = 0
    float re[kMax + 4];      // 1 / e[k] (0 where e[k] = 0)
    float tau[kMax];
    float lamv[kMax];
    int cnt[kMax];
    float red[16];           // per-wave partial sums and maxima
    float bcast[4];
    unsigned long long brk[2];   // per-wave masks of cluster starts
    float bt[2][kBT][kMax + 4];  // back-transform: two blocks of reflectors
};

__device__ __forceinline__ int wave_of(int c) { return c >> 6; }

// max over the block, on every thread; `slot` two words not in use
__device__ __forceinline__ float block_max(float v, float* slot, int c) {
    v = group_max<64>(v);
    if ((c & 63) == 0) slot[wave_of(c)] = v;
    __syncthreads();
    return fmaxf(slot[0], slot[1]);
}

// Where v_K's entries K+1 .. n-1 start in the packed reflector storage:
// after v_0 .. v_{K-1}.  The whole set, n(n-1)/2 - 1 floats, fits in V.
__device__ __forceinline__ int refl_offset(int K, int n) { return K * (n - 1) - K * (K - 1) / 2; }

// Sixteen rows of an LDS vector, as four 16-byte reads.
struct Rows16 {
    float4 q[4];
};
__device__ __forceinline__ Rows16 rows16(const float* p) {
    const float4* v = reinterpret_cast<const float4*>(p);
    return {{v[0], v[1], v[2], v[3]}};
}
__device__ __forceinline__ float at16(const Rows16& k, int i) {
    const float4& q = k.q[i >> 2];
    const int j = i & 3;
    return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}

// v . x over rows R0 .. N-1 with v in LDS, read one chunk ahead of the
// arithmetic; each chunk's read offset passes through an empty asm
// statement that takes the running sum, so the reads are not all hoisted
// to the top (all of v in VGPRs beside the column).
template <int R0, int N>
__device__ __forceinline__ float dot_lds(const float* v, const float (&x)[N]) {
    float d0 = 0.0f, d1 = 0.0f;
    Rows16 cur = rows16(v + R0);
#pragma unroll
    for (int r0 = R0; r0 < N; r0 += kC) {
        Rows16 nxt = cur;
        if (r0 + kC < N) {
            int off = r0 + kC;
            __asm__ volatile("" : "+v"(off) : "v"(d0));
            nxt = rows16(v + off);
        }
#pragma unroll
        for (int i = 0; i < kC; i += 2) {
            d0 = fmaf(at16(cur, i), x[r0 + i], d0);
            d1 = fmaf(at16(cur, i + 1), x[r0 + i + 1], d1);
        }
        cur = nxt;
    }
    return d0 + d1;
}

// x -= b v over rows R0 .. N-1, v in LDS (as dot_lds)
template <int R0, int N>
__device__ __forceinline__ void axpy_lds(float (&x)[N], const float* v, float b) {
    Rows16 cur = rows16(v + R0);
#pragma unroll
    for (int r0 = R0; r0 < N; r0 += kC) {
        Rows16 nxt = cur;
        if (r0 + kC < N) {
            int off = r0 + kC;
            __asm__ volatile("" : "+v"(off) : "v"(x[r0 > R0 ? r0 - 1 : r0]));
            nxt = rows16(v + off);
        }
#pragma unroll
        for (int i = 0; i < kC; ++i) x[r0 + i] = fmaf(-b, at16(cur, i), x[r0 + i]);
        cur = nxt;
    }
}

// x -= v w + b vc over rows R0 .. N-1 (the symmetric rank-2 update), v and
// b in LDS, eight rows of each read one block ahead (as dot_lds)
struct Rows8 {
    float4 v0, v1, b0, b1;
};
__device__ __forceinline__ Rows8 rows8(const float* v, const float* b, int off) {
    return {*reinterpret_cast<const float4*>(v + off), *reinterpret_cast<const float4*>(v + off + 4),
            *reinterpret_cast<const float4*>(b + off), *reinterpret_cast<const float4*>(b + off + 4)};
}

template <int R0, int N>
__device__ __forceinline__ void rank2_lds(float (&x)[N], const float* v, const float* b, float w, float vc) {
    Rows8 cur = rows8(v, b, R0);
#pragma unroll
    for (int r0 = R0; r0 < N; r0 += 8) {
        Rows8 nxt = cur;
        if (r0 + 8 < N) {
            int off = r0 + 8;
            __asm__ volatile("" : "+v"(off) : "v"(x[r0 > R0 ? r0 - 1 : r0]));
            nxt = rows8(v, b, off);
        }
        const float vv[8] = {cur.v0.x, cur.v0.y, cur.v0.z, cur.v0.w, cur.v1.x, cur.v1.y, cur.v1.z, cur.v1.w};
        const float bb[8] = {cur.b0.x, cur.b0.y, cur.b0.z, cur.b0.w, cur.b1.x, cur.b1.y, cur.b1.z, cur.b1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) x[r0 + i] = fmaf(-vv[i], w, fmaf(-bb[i], vc, x[r0 + i]));
        cur = nxt;
    }
}

// ssytd2 (lower) step K, K in chunk P.  Thread c holds column c, so by
// symmetry row K of the trailing block is x[K] across the threads: the
// reflector's entries are formed thread-parallel, written to LDS (and, for
// the back-transform, to V's storage), and read back as broadcasts.  Rows
// at and above K hold v = w = 0, so the products and the update leave them
// as they are with no row test.
template <int P, int MC>
__device__ __forceinline__ void trid_step(float (&x)[kC * MC], MidLds& s, int c, int n, int K, float* vg) {
    constexpr int N = kC * MC, R0 = kC * P;
    int cl = c;
    __asm__ volatile("" : "+v"(cl));
    float xk = 0.0f;
#pragma unroll
    for (int i = 0; i < kC; ++i) xk = R0 + i == K ? x[R0 + i] : xk;
    const int par = K & 1;
    const float sq = wave_sum_f(cl > K + 1 && cl < n ? xk * xk : 0.0f);
    if ((cl & 63) == 0) s.red[2 * par + wave_of(cl)] = sq;
    if (cl == K + 1) s.bcast[par] = xk;
    __syncthreads();
    const float ss = s.red[2 * par] + s.red[2 * par + 1];
    const float alpha = s.bcast[par];
    float beta = alpha, tau = 0.0f, scale = 1.0f;
    if (ss >= kTinySumsq) {   // hardware square root, refined reciprocals
        beta = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alpha, alpha, ss)), alpha);
        tau = (beta - alpha) * rcp_refined(beta);
        scale = rcp_refined(alpha - beta);
    }
    const bool act = cl > K && cl < n;
    const float vc = cl == K + 1 ? 1.0f : (act ? xk * scale : 0.0f);
    s.vr[par][c] = vc;
    if (vg && act) vg[refl_offset(K, n) + c - K - 1] = vc;
    if (cl == K) {
        s.d[K] = xk;
        s.e[K] = beta;
        s.tau[K] = tau;
    }
    __syncthreads();
    // p = tau A v (the lane mask as a factor: a select would become a
    // branch around the product)
    const float p = tau * dot_lds<R0, N>(s.vr[par], x) * (act ? 1.0f : 0.0f);
    const float pv = wave_sum_f(p * vc);
    if ((cl & 63) == 0) s.red[4 + 2 * par + wave_of(cl)] = pv;
    __syncthreads();
    const float half = 0.5f * tau * (s.red[4 + 2 * par] + s.red[4 + 2 * par + 1]);
    const float w = fmaf(-half, vc, p);
    s.bc[par][c] = w;
    __syncthreads();
    rank2_lds<R0, N>(x, s.vr[par], s.bc[par], w, vc);
    // the next step uses the other buffers and slots; the one after, these,
    // only past the next step's barriers
}

template <int P, int MC>
__device__ __forceinline__ void trid_phases(float (&x)[kC * MC], MidLds& s, int c, int n, float* vg) {
    if constexpr (P < MC) {
        const int ke = min(kC * P + kC, n - 2);   // steps K with K + 2 < n
        for (int K = kC * P; K < ke; ++K) trid_step<P, MC>(x, s, c, n, K, vg);
        trid_phases<P + 1, MC>(x, s, c, n, vg);
    }
}

// Number of eigenvalues of the (split) tridiagonal below x: the signs of
// the LDL^T pivots t of T - x I (slaebz's count), each reciprocal 1/t
// clamped to [-rbig, rbig], rbig = 1/pivmin: a pivot smaller than pivmin in
// magnitude (zero included) acts as pivmin with its own sign, where slaebz
// replaces it by -pivmin (one median instruction instead of a compare and a
// select; either count is the exact one of a shift within a few pivmin of
// x).  t stays finite (|f r| <= 2^126): no NaN, also across a split (f = 0).
// d and f = e^2 (shifted by one row) are read four rows at a time from LDS;
// rows past n carry kPad and count nothing.
template <int N>
__device__ __forceinline__ int sturm_count(const MidLds& s, float x, float rbig) {
    int cnt = 0;
    float r = 1.0f;   // 1 / t of the row above (t = 1 before row 0)
#pragma unroll
    for (int k0 = 0; k0 < N; k0 += 4) {
        const float4 dv = *reinterpret_cast<const float4*>(&s.d[k0]);
        const float4 fv = *reinterpret_cast<const float4*>(&s.f[k0]);
        const float dk[4] = {dv.x, dv.y, dv.z, dv.w};
        const float fk[4] = {fv.x, fv.y, fv.z, fv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float t = fmaf(-fk[j], r, dk[j] - x);
            cnt += (int)(__float_as_uint(t) >> 31);
            r = __builtin_amdgcn_fmed3f(__builtin_amdgcn_rcpf(t), -rbig, rbig);
        }
    }
    return cnt;
}

// The same count over the rows [lo_row, hi_row) of one block only (the
// recurrence restarts at the block's first row by itself: e = 0 above it).
template <int N>
__device__ __forceinline__ int sturm_count_in(const MidLds& s, float x, float rbig, int lo_row, int hi_row) {
    int cnt = 0;
    float r = 1.0f;
    const unsigned span = (unsigned)(hi_row - lo_row);
#pragma unroll
    for (int k0 = 0; k0 < N; k0 += 4) {
        const float4 dv = *reinterpret_cast<const float4*>(&s.d[k0]);
        const float4 fv = *reinterpret_cast<const float4*>(&s.f[k0]);
        const float dk[4] = {dv.x, dv.y, dv.z, dv.w};
        const float fk[4] = {fv.x, fv.y, fv.z, fv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float t = fmaf(-fk[j], r, dk[j] - x);
            r = __builtin_amdgcn_fmed3f(__builtin_amdgcn_rcpf(t), -rbig, rbig);
            const int neg = (int)(__float_as_uint(t) >> 31);
            cnt += (unsigned)(k0 + j - lo_row) < span ? neg : 0;
        }
    }
    return cnt;
}

// Split masks over the rows (bit i: rows i and i + 1 decoupled), two words:
// the largest split below row c (-1 for none) and the smallest at or above
// row c (-1 for none).
__device__ __forceinline__ int last_split_below(unsigned long long m0, unsigned long long m1, int c) {
    if (c > 64) {
        const int k = c - 64;
        const unsigned long long mm = k >= 64 ? m1 : (m1 & ((1ull << k) - 1));
        if (mm) return 64 + 63 - __clzll(mm);
        return m0 ? 63 - __clzll(m0) : -1;
    }
    const unsigned long long mm = c >= 64 ? m0 : (m0 & ((1ull << c) - 1));
    return mm ? 63 - __clzll(mm) : -1;
}
__device__ __forceinline__ int first_split_from(unsigned long long m0, unsigned long long m1, int c) {
    if (c < 64) {
        const unsigned long long mm = m0 & (~0ull << c);
        if (mm) return __ffsll((long long)mm) - 1;
        return m1 ? 64 + __ffsll((long long)m1) - 1 : -1;
    }
    const unsigned long long mm = m1 & (~0ull << (c - 64));
    return mm ? 64 + __ffsll((long long)mm) - 1 : -1;
}

// x <- x / |x|_2, scaled by its largest entry first.
template <int N>
__device__ __forceinline__ void normalize(float (&x)[N]) {
    float xm = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k) xm = fmaxf(xm, fabsf(x[k]));
    const float sc = xm > 0.0f ? 1.0f / xm : 0.0f;
    float nrm = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        x[k] *= sc;
        nrm = fmaf(x[k], x[k], nrm);
    }
    const float inv = nrm > 0.0f ? 1.0f / sqrtf(nrm) : 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k) x[k] *= inv;
}

// ---- launch 1: tridiagonalisation, bisection ----

template <int MC, bool VEC>
__global__ __launch_bounds__(kThreads) void eigh_mid_values_kernel(const float* __restrict__ A, float* __restrict__ W,
                                                                   float* __restrict__ V, uint32_t* __restrict__ info,
                                                                   uint32_t n_, int lower, float* __restrict__ Sv) {
    constexpr int N = kC * MC;
    __shared__ MidLds s;
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    const int n = (int)n_;
    const size_t per = (size_t)n * n;

    // 1. the read triangle, mirrored: entry r of thread c's column from the
    // column (coalesced across threads) in the read triangle and from row c
    // outside it.  Every load unconditional (clamped into the matrix), the
    // mask applied after; fences every 16 rows bound the live addresses.
    float x[N];
    float amax = 0.0f;
    int bad = 0;
    {
        const int cc = c < n ? c : n - 1;
        const float* src = A + mat * per;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            const int rr = r < n ? r : n - 1;
            const bool take = lower ? r >= c : r <= c;
            x[r] = src[take ? rr * n + cc : cc * n + rr];
            if ((r & 15) == 15) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int r = 0; r < N; ++r) {
            const bool in = r < n && c < n;
            const bool take = lower ? r >= c : r <= c;
            const float v = in ? x[r] : 0.0f;
            amax = fmaxf(amax, fabsf(v));
            bad |= in && take && !finite_f(v);
            x[r] = v;
        }
    }
    amax = block_max(amax, s.red + 8, c);
    bad = __syncthreads_or(bad);
    const int ex = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -ex);

    // 2. tridiagonalise: d, e, tau; v_K to V's storage (packed)
    float* vg = VEC ? V + mat * per : nullptr;
    trid_phases<0, MC>(x, s, c, n, vg);
    {
        float diag = 0.0f, sub = 0.0f;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            diag = r == c ? x[r] : diag;
            sub = r == c + 1 ? x[r] : sub;
        }
        if (c == n - 2) {
            s.d[c] = diag;
            s.e[c] = sub;
        }
        if (c == n - 1) {
            s.d[c] = diag;
            s.e[c] = 0.0f;
        }
    }
    __syncthreads();

    // 3. splits (sstebz's test), e^2, padding, Gershgorin bounds
    float ei = 0.0f;
    if (c < n - 1) {
        ei = s.e[c];
        const float di = s.d[c], di1 = s.d[c + 1];
        if (fabsf(ei) <= kEps * (fabsf(di) + fabsf(di1)) || fabsf(ei) < kSafeMin) ei = 0.0f;
    }
    const bool split = c < n - 1 && ei == 0.0f;
    __syncthreads();   // every e read before it is overwritten
    s.e[c] = ei;       // zero from row n - 1 on
    s.f[c + 1] = ei * ei;
    s.re[c] = ei != 0.0f ? __builtin_amdgcn_rcpf(ei) : 0.0f;
    if (c == 0) s.f[0] = 0.0f;
    if (c >= n) s.d[c] = kPad;
    if (c < 4) {
        s.d[kMax + c] = kPad;
        s.e[kMax + c] = 0.0f;
        if (c > 0) s.f[kMax + c] = 0.0f;
        s.re[kMax + c] = 0.0f;
    }
    // T's unreduced blocks: thread c's row lies in [bs, be).  As sstebz and
    // sstein, each block has its own eigenvalues and eigenvectors (whose
    // supports are the block's rows, so that vectors of different blocks
    // are orthogonal whatever their eigenvalues); a block of one row is the
    // exact pair (d_c, e_c).
    const unsigned long long sw = __ballot(split);
    if ((c & 63) == 0) s.brk[wave_of(c)] = sw;
    const bool one_block = __syncthreads_and(c >= n - 1 || !split) != 0;
    int bs = 0, be = n;
    if (!one_block) {
        const unsigned long long m0 = s.brk[0], m1 = s.brk[1];
        bs = last_split_below(m0, m1, c) + 1;
        const int fs = first_split_from(m0, m1, c);
        be = fs < 0 || fs + 1 > n ? n : fs + 1;
    }
    const bool mine = c < n;
    const bool single = be - bs <= 1;
    const bool all_single = __syncthreads_and(!mine || single) != 0;
    float glo = FLT_MAX, ghi = -FLT_MAX;
    if (c < n) {
        const float r = fabsf(ei) + (c > 0 ? fabsf(s.e[c - 1]) : 0.0f);
        const float dc = s.d[c];
        glo = dc - r;
        ghi = dc + r;
    }
    glo = -block_max(-glo, s.red + 10, c);
    ghi = block_max(ghi, s.red + 12, c);
    const float e2max = block_max(ei * ei, s.red + 14, c);
    const float tnorm = fmaxf(fabsf(glo), fabsf(ghi));
    const float pivmin = kSafeMin * fmaxf(1.0f, e2max);
    const float slack = 2.1f * 2.0f * kEps * tnorm * (float)n + 4.2f * pivmin;
    const float atol = fmaxf(kEps * tnorm, 2.0f * pivmin);
    const float rbig = 1.0f / pivmin;

    // 4. bisection: thread c brackets the (c - bs)-th smallest eigenvalue
    // of its block
    const float g0 = glo - slack, g1 = ghi + slack;
    float lo = g0, hi = g1;
    int steps = 0;
    float lam;
    int rank = c;
    if (one_block) {
        // one multisection pass first: thread i counts at the i-th of N + 1
        // equal divisions of the Gershgorin interval, and every thread takes
        // its bracket from those counts
        const float gh = (g1 - g0) / (float)(N + 1);
        if (c < N) s.cnt[c] = sturm_count<N>(s, fmaf((float)(c + 1), gh, g0), rbig);
        __syncthreads();
#pragma unroll 4
        for (int i = 0; i < N; ++i) {
            const float xi = fmaf((float)(i + 1), gh, g0);
            if (s.cnt[i] <= c) lo = fmaxf(lo, xi);
            else hi = fminf(hi, xi);
        }
        if (!(lo < hi)) {   // counts not monotone in floating point: the whole interval
            lo = g0;
            hi = g1;
        }
        steps = 1;
        while (steps < kMaxBisect) {
            const float mid = 0.5f * (lo + hi);
            const int cm = sturm_count<N>(s, mid, rbig);
            if (cm > c) hi = mid;
            else lo = mid;
            ++steps;
            const bool done = !mine || hi - lo <= fmaxf(atol, 2.0f * kEps * fmaxf(fabsf(lo), fabsf(hi)));
            if (!__syncthreads_or(!done)) break;
        }
        // ascending even where brackets of equal eigenvalues overlap: prefix max
        lam = 0.5f * (lo + hi);
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float up = __shfl_up(lam, off, 64);
            if ((c & 63) >= off) lam = fmaxf(lam, up);
        }
        if (c == 63) s.bcast[2] = lam;
        __syncthreads();
        if (c >= 64) lam = fmaxf(lam, s.bcast[2]);
    } else {
        const int j = c - bs;
        if (!all_single) {
            while (steps < kMaxBisect) {
                const bool done = !mine || single || hi - lo <= fmaxf(atol, 2.0f * kEps * fmaxf(fabsf(lo), fabsf(hi)));
                if (!__syncthreads_or(!done)) break;
                const float mid = 0.5f * (lo + hi);
                const int cm = sturm_count_in<N>(s, mid, rbig, bs, be);
                if (cm > j) hi = mid;
                else lo = mid;
                ++steps;
            }
        }
        lam = single ? s.d[c] : 0.5f * (lo + hi);
        // the rank among all the eigenvalues (ties by row)
        s.lamv[c] = mine ? lam : FLT_MAX;
        __syncthreads();
        rank = 0;
        for (int i = 0; i < n; ++i) {
            const float li = s.lamv[i];
            rank += (li < lam) || (li == lam && i < c);
        }
    }

    if (VEC) {
        float* st = Sv + mat * kStateFloats;
        st[c] = s.d[c];
        st[kMax + c] = s.e[c];
        st[2 * kMax + c] = s.re[c];
        st[3 * kMax + c] = c < kMax - 2 ? s.tau[c] : 0.0f;
        st[4 * kMax + c] = lam;
        st[5 * kMax + c] = __int_as_float(bs);
        st[6 * kMax + c] = __int_as_float(be);
        st[7 * kMax + c] = __int_as_float(rank);
        if (c == 0) {
            st[8 * kMax] = tnorm;
            st[8 * kMax + 1] = __int_as_float(all_single ? 1 : 0);
            st[8 * kMax + 2] = __int_as_float(bad);
        }
    }
    if (mine) W[mat * n + rank] = bad ? qnan() : ldexpf(lam, ex);
    if (info && c == 0) info[mat] = bad ? (1u << 17) : ((uint32_t)steps | (1u << 16));
}

// ---- launch 2: the vectors ----

// Back-transform step K (K + 1 in chunk P): x <- H_K x.  Reflectors come
// from V's storage in blocks of kBT (thread c loads element c of each, one
// block ahead), staged in LDS and read as broadcasts; entries at and above
// row K are zero.
// The loads are masked only when the block is staged, a block later: a
// select right after them would wait for them.
__device__ __forceinline__ int bt_k(int kb, int i, int n) {
    const int kmax = n - 3;
    return kb - i < 0 ? 0 : (kb - i > kmax ? kmax : kb - i);
}
__device__ __forceinline__ void bt_fetch(float (&nx)[kBT], const float* vg, int kb, int c, int n) {
#pragma unroll
    for (int i = 0; i < kBT; ++i) {
        const int k = bt_k(kb, i, n);
        const bool in = c > k && c < n;
        const int off = refl_offset(k, n);
        nx[i] = vg[in ? off + c - k - 1 : off];
    }
}

template <int P, int MC>
__device__ __forceinline__ void bt_phase(float (&x)[kC * MC], MidLds& s, int c, int n, const float* vg,
                                         float (&nx)[kBT]) {
    constexpr int N = kC * MC, R0 = kC * P;
    // K + 1 in chunk P: K from min(R0 + kC - 2, n - 3) down to R0 - 1
    const int khi = min(R0 + kC - 2, n - 3), klo = R0 - 1 > 0 ? R0 - 1 : 0;
    for (int K = khi; K >= klo; --K) {
        const int q = (n - 3) - K;
        const int blk = q / kBT, i = q - blk * kBT;
        if (i == 0) {   // a new block: store the fetched one, fetch the next
#pragma unroll
            for (int j = 0; j < kBT; ++j) {
                const int k = bt_k(K, j, n);
                s.bt[blk & 1][j][c] = (c > k && c < n) ? nx[j] : 0.0f;
            }
            if (K - kBT >= 0) bt_fetch(nx, vg, K - kBT, c, n);
            __syncthreads();
        }
        const float* v = s.bt[blk & 1][i];
        const float d = s.tau[K] * dot_lds<R0, N>(v, x);
        axpy_lds<R0, N>(x, v, d);
    }
}

template <int P, int MC>
__device__ __forceinline__ void bt_phases(float (&x)[kC * MC], MidLds& s, int c, int n, const float* vg,
                                          float (&nx)[kBT]) {
    if constexpr (P >= 0) {
        bt_phase<P, MC>(x, s, c, n, vg, nx);
        bt_phases<P - 1, MC>(x, s, c, n, vg, nx);
    }
}

// Thread c: inverse iteration for the eigenvector of its eigenvalue, MGS
// inside close groups, back-transform, column c of V.  U: this matrix's
// scratch, N rows x kThreads.
template <int MC>
__global__ __launch_bounds__(kThreads) void eigh_mid_vectors_kernel(const float* __restrict__ Sv,
                                                                    float* __restrict__ V, uint32_t n_,
                                                                    float* __restrict__ Uall) {
    constexpr int N = kC * MC;
    __shared__ MidLds s;
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    const int n = (int)n_;
    const size_t per = (size_t)n * n;
    const float* st = Sv + mat * kStateFloats;
    float* U = Uall + mat * (size_t)N * kThreads;
    s.d[c] = st[c];
    s.e[c] = st[kMax + c];
    s.re[c] = st[2 * kMax + c];
    s.tau[c] = st[3 * kMax + c];
    if (c < 4) {
        s.d[kMax + c] = kPad;
        s.e[kMax + c] = 0.0f;
        s.re[kMax + c] = 0.0f;
    }
    const float lam = st[4 * kMax + c];
    const int bs = __float_as_int(st[5 * kMax + c]);
    const int be = __float_as_int(st[6 * kMax + c]);
    const int rank = __float_as_int(st[7 * kMax + c]);
    const float tnorm = st[8 * kMax];
    const bool all_single = __float_as_int(st[8 * kMax + 1]) != 0;
    const int bad = __float_as_int(st[8 * kMax + 2]);
    const bool mine = c < n;
    const bool single = be - bs <= 1;
    __syncthreads();

    float x[N];
    // 5. inverse iteration: T - sigma I = P L U with partial pivoting
    // (slagtf), the right-hand side carried along: x[k] holds the
    // right-hand side, then row k of U scaled by its pivot, then the
    // solution; the superdiagonal entry where row k kept its place goes to
    // U (NaN where rows k and k+1 were swapped: U's row is then (e_k,
    // d_{k+1} - sigma, e_{k+1}), rebuilt from LDS on the way back; sigma is
    // the eigenvalue, set apart from its group's below).
    const float tol = fmaxf(kEps * tnorm, kSafeMin);   // smaller pivots become +-tol
    // the start: pseudo-random on the block's rows (the same for every
    // matrix: a matrix's result does not depend on where it sits in the
    // batch), zero elsewhere, so that the solution stays on the block
#pragma unroll
    for (int k = 0; k < N; ++k) x[k] = k >= bs && k < be ? hash_uniform((uint32_t)c, (uint32_t)k) : 0.0f;
    // close eigenvalues of one block: threads cs .. c with gaps <= kOrtol |T|
    float prev = __shfl_up(lam, 1, 64);
    if (c == 63) s.bcast[0] = lam;
    __syncthreads();
    if (c == 64) prev = s.bcast[0];
    const bool brk = c == bs || !mine || single || lam - prev > kOrtol * tnorm;
    const unsigned long long bw = __ballot(brk);
    if ((c & 63) == 0) s.brk[wave_of(c)] = bw;
    __syncthreads();
    int cs;
    {
        const unsigned long long b0 = s.brk[0], b1 = s.brk[1];
        if (c >= 64) {
            const unsigned long long m1 = b1 & ((2ull << (c - 64)) - 1);
            cs = m1 ? 64 + 63 - __clzll(m1) : 63 - __clzll(b0);
        } else {
            cs = 63 - __clzll(b0 & ((2ull << c) - 1));
        }
    }
    const int pos = c - cs;
    const int rounds = (int)block_max((float)pos, s.red, c);
    // inside a group, shifts at least 10 eps |T| apart (sstein's PERTOL):
    // with equal shifts every member's solve would be drawn to the same
    // vector of the group, and the Gram-Schmidt rounds would leave noise
    s.lamv[c] = lam;
    __syncthreads();
    float sigma = lam;
    if (pos > 0) {
        const float pertol = 10.0f * kEps * tnorm;
        sigma = s.lamv[cs];
        for (int i = cs + 1; i <= c; ++i) sigma = fmaxf(s.lamv[i], sigma + pertol);
    }
    for (int pass = 0; pass < (all_single ? 0 : 2); ++pass) {
        float a = s.d[0] - sigma, cc = s.e[0], b0 = x[0];
        float enow = s.e[0], dnx = s.d[1], enx = s.e[1];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            if (k + 1 < N) {
                const float ek = enow;
                const float an = dnx - sigma, cn = enx, b1 = x[k + 1];
                enow = enx;
                if (k + 2 < N) {
                    dnx = s.d[k + 2];
                    enx = s.e[k + 2];
                }
                const bool keep = fabsf(a) >= fabsf(ek);
                const float piv = keep ? a : ek;
                const float r0 = __builtin_amdgcn_rcpf(fabsf(piv) < tol ? copysignf(tol, piv) : piv);
                const float l = (keep ? ek : a) * r0;
                x[k] = (keep ? b0 : b1) * r0;
                U[(size_t)k * kThreads + c] = keep ? cc * r0 : qnan();   // NaN marks a swap
                const float na = keep ? fmaf(-l, cc, an) : fmaf(-l, an, cc);
                cc = keep ? cn : -l * cn;
                b0 = keep ? fmaf(-l, b0, b1) : fmaf(-l, b1, b0);
                a = na;
            } else {
                x[k] = b0 * __builtin_amdgcn_rcpf(fabsf(a) < tol ? copysignf(tol, a) : a);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // back substitution; U's entries loaded a chunk of 16 rows ahead
        float x1 = 0.0f, x2 = 0.0f;
        float ub[kC];
#pragma unroll
        for (int i = 0; i < kC; ++i) {
            const int k = N - kC + i;
            ub[i] = k + 1 < N ? U[(size_t)k * kThreads + c] : 0.0f;
        }
#pragma unroll
        for (int k0 = N - kC; k0 >= 0; k0 -= kC) {
            float un[kC];
            if (k0 > 0) {
#pragma unroll
                for (int i = 0; i < kC; ++i) un[i] = U[(size_t)(k0 - kC + i) * kThreads + c];
            }
#pragma unroll
            for (int i = kC - 1; i >= 0; --i) {
                const int k = k0 + i;
                float xv = x[k];
                if (k + 1 < N) {
                    const float rk = s.re[k], dk1 = s.d[k + 1], ek1 = s.e[k + 1];
                    const bool swapped = ub[i] != ub[i];
                    const float q1 = swapped ? (dk1 - sigma) * rk : ub[i];
                    const float q2 = swapped ? ek1 * rk : 0.0f;
                    xv = fmaf(-q2, x2, fmaf(-q1, x1, xv));
                }
                x[k] = xv;
                x2 = x1;
                x1 = xv;
            }
            if (k0 > 0) {
#pragma unroll
                for (int i = 0; i < kC; ++i) ub[i] = un[i];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        normalize<N>(x);
        // modified Gram-Schmidt within each close group, one member per
        // round: the member at position t is final when round t begins and
        // publishes its vector in its own column of U (every thread's loads
        // of U for the solve are done: a thread reads only its own column
        // there, and a barrier separates the rounds)
        for (int t = 0; t < rounds; ++t) {
            if (pos == t) {
                normalize<N>(x);
#pragma unroll
                for (int k = 0; k < N; ++k) U[(size_t)k * kThreads + c] = x[k];
            }
            __syncthreads();
            if (pos > t) {
                const int src = cs + t;
                float dot = 0.0f;
#pragma unroll
                for (int k = 0; k < N; ++k) dot = fmaf(U[(size_t)k * kThreads + src], x[k], dot);
#pragma unroll
                for (int k = 0; k < N; ++k) x[k] = fmaf(-dot, U[(size_t)k * kThreads + src], x[k]);
            }
            __syncthreads();
        }
        normalize<N>(x);
    }
    if (single) {
#pragma unroll
        for (int k = 0; k < N; ++k) x[k] = k == c ? 1.0f : 0.0f;
    }

    // 6. back to A's basis; thread c writes column `rank` of V over the
    // reflectors once every thread's loads of them have returned
    {
        float nx[kBT];
        const float* vsrc = V + mat * per;
        bt_fetch(nx, vsrc, n - 3, c, n);
        bt_phases<MC - 1, MC>(x, s, c, n, vsrc, nx);
    }
    __syncthreads();
    if (mine) {
        float* dst = V + mat * per;
#pragma unroll
        for (int r = 0; r < N; ++r)
            if (r < n) dst[(size_t)r * n + rank] = bad ? qnan() : x[r];
    }
}

template <int MC>
void launch(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
            hipStream_t s) {
    if (v) {
        float* U = ws + (size_t)batch * kStateFloats;
        hipLaunchKernelGGL((eigh_mid_values_kernel<MC, true>), dim3(batch), dim3(kThreads), 0, s, a, w, v, info, n,
                           lower ? 1 : 0, ws);
        hipLaunchKernelGGL((eigh_mid_vectors_kernel<MC>), dim3(batch), dim3(kThreads), 0, s, ws, v, n, U);
    } else {
        hipLaunchKernelGGL((eigh_mid_values_kernel<MC, false>), dim3(batch), dim3(kThreads), 0, s, a, w, nullptr,
                           info, n, lower ? 1 : 0, nullptr);
    }
}

}  // namespace

bool eigh_mid_fits(uint32_t n) { return n >= (uint32_t)kMin && n <= (uint32_t)kMax; }

size_t eigh_mid_workspace(uint32_t n, uint32_t batch, bool vectors) {
    if (!vectors) return 0;
    const size_t rows = (n + kC - 1) / kC * kC;
    return (size_t)batch * (kStateFloats + rows * kThreads) * sizeof(float);
}

void eigh_mid(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
              hipStream_t s) {
    if (!eigh_mid_fits(n)) invalid("[eigh] eigh_mid takes 65 <= n <= 128");
    if (batch == 0) return;
    if (v && !ws) invalid("[eigh] eigh_mid needs its workspace with vectors");
    KernelTimer t("eigh_mid", s);
    // launches of at most 2^20 matrices, one after another on the stream
    // (the workspace is sized for the batch and reused from its start)
    for (uint32_t b0 = 0; b0 < batch; b0 += 1u << 20) {
        const uint32_t nb = std::min<uint32_t>(batch - b0, 1u << 20);
        const size_t off = (size_t)b0 * n * n;
        switch ((n + kC - 1) / kC) {
        case 5: launch<5>(a + off, w + (size_t)b0 * n, v ? v + off : nullptr, info ? info + b0 : nullptr, nb, n, lower, ws, s); break;
        case 6: launch<6>(a + off, w + (size_t)b0 * n, v ? v + off : nullptr, info ? info + b0 : nullptr, nb, n, lower, ws, s); break;
        case 7: launch<7>(a + off, w + (size_t)b0 * n, v ? v + off : nullptr, info ? info + b0 : nullptr, nb, n, lower, ws, s); break;
        default: launch<8>(a + off, w + (size_t)b0 * n, v ? v + off : nullptr, info ? info + b0 : nullptr, nb, n, lower, ws, s); break;
        }
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
