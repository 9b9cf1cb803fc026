// Batched symmetric eigendecomposition of small matrices (n <= 64), one
// matrix per lane group of a wave64 (a whole wave at n = 64), in registers.
//
// Role: the MI355X counterpart of the reference's eigh_ql kernel
// (reference: shaders/Eigh_QL.metal:229-485, driver src/eigh_ql.mm:169-266).
// Same contract, different method for the tridiagonal stage: Householder
// tridiagonalisation (LAPACK ssytd2), then every eigenvalue by bisection on
// Sturm counts (LAPACK sstebz's rule) and every eigenvector by inverse
// iteration with partial pivoting (LAPACK slagtf/slagts, as in sstein), two
// steps from a pseudo-random start, with modified Gram-Schmidt inside groups
// of eigenvalues closer than 1e-3 |T| (sstein's ORTOL), and finally the
// back-transformation by the reflectors.  Conventions of the reference's
// contract: only the requested triangle is read; the matrix is scaled by a
// power of two into [0.5, 1) before and the values unscaled after; a matrix
// holding a NaN or an infinity in the read triangle gives all-NaN w and V
// with info bit 17; otherwise info holds the number of bisection steps in
// bits 0-15 with bit 16 (converged) set; values ascending.
//
// MI355X layout: lane c of an N-lane group owns column c of the (symmetric)
// working matrix, so the tridiagonalisation's products A v are lane-local
// FMA chains and only v and w are broadcast through LDS.  The tridiagonal
// stage is lane-parallel: lane c bisects for the c-th smallest eigenvalue
// (each Sturm count a register-resident recurrence over d and e^2 read from
// LDS as float4 broadcasts), then solves for its own eigenvector with the
// pivoted factor, right-hand side and back substitution in VGPRs.  Lanes of
// a close group exchange vectors with cross-lane permutes, one member per
// round.  The reflectors wait in V's own storage (packed lower parts) and come
// back through LDS eight at a time; lane c applies them to its vector and
// writes column c of V over them; lanes write consecutive addresses.  LDS
// holds only the current reflector, w, the tridiagonal and a staging block
// (7.3 KB at n = 64).  With vectors at n = 64 the work runs in two launches:
// the tridiagonalisation and the bisection fit 128 VGPRs (four waves per
// SIMD, so a 4096-matrix batch is resident at once), the inverse iteration
// needs ~150 (three); the first saves the tridiagonal, the eigenvalues and
// tau for the second (1.5 KB per matrix).  The previous design ran
// implicit QL on every lane redundantly: a serial rotation chain that kept
// 63 of 64 lanes idle (the bisection and the solves need ~30x fewer issue
// slots per matrix).
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr float kEps = 5.9604645e-08f;        // 2^-24, fp32 unit roundoff
constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80: a reflector below it is the identity
constexpr float kSafeMin = 1.17549435e-38f;   // FLT_MIN

constexpr float kPad = 0x1p100f;             // the diagonal of padding rows: never counted
constexpr float kOrtol = 1e-3f;               // close eigenvalues: gap <= kOrtol |T| (sstein's ORTOL)
constexpr int kMaxBisect = 64;
constexpr int kBT = 8;                       // reflectors staged per back-transform block
// float4 chunks of the reflector (and of w) read ahead of their use in the
// tridiagonalisation's dot product and rank-2 update (2/1 to 6/3 measured
// within 3 us of each other on config 2)
constexpr int kDotAhead = 4;
constexpr int kRank2Ahead = 2;

// n = 64 with vectors runs in two launches (the first fits four waves per
// SIMD, the vectors need more VGPRs): per matrix the first leaves d, e, 1/e,
// tau, the eigenvalue and the diagonal-path row of each lane, and three
// scalars for the second
constexpr int kSplitN = 64;
constexpr int kSplitFloats = 6 * kSplitN + 4;

template <int N>
struct alignas(16) EighLds {
    // the arrays read every step first: their offsets then fit the LDS
    // instructions' immediate fields (no address register per read)
    float vr[2][N + 4];          // the current reflector (v_k[k+1] = 1), alternate steps
    float bc[2][N + 4];          // w of the rank-2 update, alternate steps
    float d[N + 4];       // the tridiagonal, rows >= n padded with kPad
    float e[N + 4];       // e[k] couples rows k and k+1; zero at splits and from row n - 1 on
    float f[N + 4];       // f[k] = e[k-1]^2, f[0] = 0
    float re[N + 4];      // 1 / e[k] (0 where e[k] = 0)
    float tau[N];
    int perm[N];
    int cnt[N];
    float bt[2][kBT][N + 4];     // back-transform: two blocks of reflectors
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

// Rows A0 .. N-1 (A0 a multiple of 4) of an LDS vector as float4 chunks,
// each read D chunks before its use: the reads of later chunks are in
// flight while the current one is consumed, instead of a full LDS round
// trip every few rows.  The schedule barrier after each chunk keeps the
// compiler from hoisting every read to the top (which would hold the whole
// vector in VGPRs beside the column).
template <int A0, int N>
__device__ __forceinline__ float4 lds_chunk(const float* a, int q) {
    return *reinterpret_cast<const float4*>(a + A0 + 4 * q);
}

// sum of v[r] x[r] over rows A0 .. N-1 into four partial sums by r mod 4
template <int A0, int N, int D>
__device__ __forceinline__ float lds_dot(const float* v, const float (&x)[N]) {
    constexpr int NC = (N - A0) / 4;
    float4 b[NC];
    float dp0 = 0.0f, dp1 = 0.0f, dp2 = 0.0f, dp3 = 0.0f;
#pragma unroll
    for (int q = 0; q < (D < NC ? D : NC); ++q) b[q] = lds_chunk<A0, N>(v, q);
#pragma unroll
    for (int q = 0; q < NC; ++q) {
        if (q + D < NC) b[q + D] = lds_chunk<A0, N>(v, q + D);
        const int r = A0 + 4 * q;
        dp0 = fmaf(b[q].x, x[r], dp0);
        dp1 = fmaf(b[q].y, x[r + 1], dp1);
        dp2 = fmaf(b[q].z, x[r + 2], dp2);
        dp3 = fmaf(b[q].w, x[r + 3], dp3);
        __builtin_amdgcn_sched_barrier(0);
    }
    return (dp0 + dp1) + (dp2 + dp3);
}

// x[r] -= v[r] w + b[r] u over rows A0 .. N-1
template <int A0, int N, int D>
__device__ __forceinline__ void lds_rank2(float (&x)[N], const float* v, const float* bw, float w, float u) {
    constexpr int NC = (N - A0) / 4;
    float4 p[NC], q4[NC];
#pragma unroll
    for (int q = 0; q < (D < NC ? D : NC); ++q) {
        p[q] = lds_chunk<A0, N>(v, q);
        q4[q] = lds_chunk<A0, N>(bw, q);
    }
#pragma unroll
    for (int q = 0; q < NC; ++q) {
        if (q + D < NC) {
            p[q + D] = lds_chunk<A0, N>(v, q + D);
            q4[q + D] = lds_chunk<A0, N>(bw, q + D);
        }
        const int r = A0 + 4 * q;
        x[r] = fmaf(-p[q].x, w, fmaf(-q4[q].x, u, x[r]));
        x[r + 1] = fmaf(-p[q].y, w, fmaf(-q4[q].y, u, x[r + 1]));
        x[r + 2] = fmaf(-p[q].z, w, fmaf(-q4[q].z, u, x[r + 2]));
        x[r + 3] = fmaf(-p[q].w, w, fmaf(-q4[q].w, u, x[r + 3]));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Global memory as the compiler's address space 1: stores through such a
// pointer are global_store (a generic pointer gives flat_store, which also
// counts against the LDS wait counter).
typedef __attribute__((address_space(1))) float gfloat;

// A pointer that is the same on every lane, moved to SGPRs (otherwise a
// 64-bit VGPR pair that the register allocator spills and reloads), as a
// global pointer.
__device__ __forceinline__ gfloat* uniform_gptr(float* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (gfloat*)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ gfloat* global_ptr(float* p) { return (gfloat*)reinterpret_cast<uint64_t>(p); }

// Where v_K's entries K+1 .. n-1 start in the packed reflector storage:
// after v_0 .. v_{K-1} (n-1, n-2, ... entries).  The whole set, n(n-1)/2 - 1
// floats, fits in V's n x n.
__device__ __forceinline__ int refl_offset(int K, int n) { return K * (n - 1) - K * (K - 1) / 2; }

// ssytd2 (lower) step K: reflector from column K below the subdiagonal, then
// the symmetric rank-2 update of the trailing block.
// The value of lane `src` of the group, on every lane of the group.
template <int N>
__device__ __forceinline__ float group_bcast(float v, int src) {
    if constexpr (N == 64) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
    else return __shfl(v, src, N);
}

// ssytd2 (lower) step K.  Lane c holds column c of the working matrix, so
// by symmetry row K of the trailing block is x[K] across the lanes: the
// reflector's entries are formed lane-parallel (lane c scales its own
// x[K]), written as row K of vs (which keeps them for the
// back-transformation), and read back as a broadcast for the products.
// Then the symmetric rank-2 update of the trailing block, w through bc.
template <int K, int N>
__device__ __forceinline__ void tridiag_step(float (&x)[N], EighLds<N>& s, int c, int n, gfloat* vg) {
    if constexpr (K + 2 < N) {
        if (K + 2 < n) {
            // c laundered: otherwise the compiler precomputes the lane masks
            // below for every step at kernel entry and spills the SGPR pairs
            int cl = c;
            __asm__ volatile("" : "+v"(cl));
            const float xk = x[K];
            const float alpha = group_bcast<N>(xk, K + 1);
            const float ss = group_sum_dpp<N>(cl > K + 1 && cl < n ? xk * xk : 0.0f);
            float beta = alpha, tau = 0.0f, scale = 1.0f;
            if (ss >= kTinySumsq) {   // hardware square root, refined reciprocals
                beta = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alpha, alpha, ss)), alpha);
                tau = (beta - alpha) * rcp_refined(beta);
                scale = rcp_refined(alpha - beta);
            }
            const bool act = cl > K && cl < n;
            const float vc = cl == K + 1 ? 1.0f : (act ? xk * scale : 0.0f);
            s.vr[K & 1][c] = vc;
            // entries K+1 .. n-1 of v_K, packed after those of v_0 .. v_{K-1}
            // in V's storage, for the back-transform
            if (vg && cl > K && c < n) vg[refl_offset(K, n) + c - K - 1] = vc;
            if (cl == K) {
                s.d[K] = xk;
                s.e[K] = beta;
                s.tau[K] = tau;
            }
            // v^T x_c from the aligned row at or before K+1: v is zero in
            // the rows up to K (every lane wrote its entry, zero at and left
            // of K), so those rows add exact zeros
            constexpr int A0 = (K + 1) / 4 * 4;
            wave_lds_sync();
            float dv = lds_dot<A0, N, kDotAhead>(s.vr[K & 1], x);
            __asm__ volatile("" : "+v"(dv));   // computed by every lane: no branch around the reads
            const float p = act ? tau * dv : 0.0f;
            const float half = 0.5f * tau * group_sum_dpp<N>(p * vc);
            const float w = fmaf(-half, vc, p);
            float* bc = s.bc[K & 1];
            bc[c] = w;
            wave_lds_sync();
            // every lane: outside the trailing block vc = w = 0, so the
            // update leaves x as it is (no divergent branch, whose merge
            // would copy the column); v and w are zero in the rows up to K,
            // which are left as they are.  v is read again from LDS: holding
            // it across the barrier would keep N more VGPRs live.
            lds_rank2<A0, N, kRank2Ahead>(x, s.vr[K & 1], bc, w, vc);
        }
        tridiag_step<K + 1, N>(x, s, c, n, vg);
    }
}

// Number of eigenvalues of the (split) tridiagonal below x: the signs of
// the LDL^T pivots t of T - x I (LAPACK slaebz's count), where each
// reciprocal 1/t is clamped to [-rbig, rbig], rbig = 1/pivmin: a pivot
// smaller than pivmin in magnitude (zero included) acts as pivmin with its
// own sign, where slaebz replaces it by -pivmin (one median instruction here
// instead of a compare and a select; either count is the exact one of a
// shift within a few pivmin of x).  t stays finite (|f r| <= 2^126), so no
// NaN can arise, also across a split (f = 0).  d and f = e^2 (shifted by one
// row) are read four rows at a time from LDS; rows past n carry kPad and
// count nothing.
template <int N>
__device__ __forceinline__ int sturm_count(const EighLds<N>& s, float x, float rbig) {
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

// Column c of the symmetric matrix whose LOWER (or upper) triangle is read,
// for lane c of its N-lane group.  Every row is read whole across the lanes
// (lane c: entry (r, c), coalesced); the entries outside the read triangle
// are then replaced by their mirror images, which other lanes hold: lanes
// stage their columns in LDS, CH at a time, and lane c takes entry c of
// column r from there.  The values read outside the triangle are never used
// (a NaN there changes nothing).  Reads stay inside the n x n matrix; rows
// and columns past n are zero.
template <int N, bool LOWER>
__device__ __forceinline__ void load_symmetric(float (&x)[N], EighLds<N>& s, const float* src, int c, int nn) {
    if (nn == N) {   // the whole group's shape: row offsets are constants
        // a lane outside the read triangle reads row r's diagonal entry in
        // place of its own (the value is replaced below): only the read
        // triangle's cache lines are fetched
        if constexpr (N == 64) {
            // one matrix per wave: a buffer resource over it (SGPR base,
            // 32-bit offsets per lane, the row's offset an immediate)
            // (the base made uniform explicitly: otherwise the compiler
            // wraps every load in a loop over the distinct bases)
            const uint64_t pv = reinterpret_cast<uint64_t>(src);
            const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)pv);
            const uint32_t phi = __builtin_amdgcn_readfirstlane((uint32_t)(pv >> 32));
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                reinterpret_cast<float*>(((uint64_t)phi << 32) | plo), (short)0, N * N * 4, 0x00020000);
            const int cb = 4 * c;
#pragma unroll
            for (int r = 0; r < N; ++r) {
                const int vo = 4 * N * r + (LOWER ? min(cb, 4 * r) : max(cb, 4 * r));
                x[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vo, 0, 0));
                if ((r & 15) == 15) __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // several matrices per wave: the base differs between lane
            // groups (a buffer resource must be uniform), so global loads
#pragma unroll
            for (int r = 0; r < N; ++r) {
                x[r] = src[r * N + (LOWER ? min(c, r) : max(c, r))];
                if ((r & 15) == 15) __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        const int cc = c < nn ? c : nn - 1;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            const int rr = r < nn ? r : nn - 1;
            x[r] = src[rr * nn + cc];   // 32-bit offsets: n <= 64
            if ((r & 15) == 15) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int r = 0; r < N; ++r) x[r] = (r < nn && c < nn) ? x[r] : 0.0f;
    }
    constexpr int CH = N < 16 ? N : 16;
    constexpr int LD = N + 4;
    float* stg = &s.bt[0][0][0];   // CH x LD floats, free until the back-transform
    static_assert(CH * LD <= 2 * kBT * (N + 4), "mirror staging fits the back-transform block");
#pragma unroll
    for (int j = 0; j < N / CH; ++j) {
        if (c >= j * CH && c < (j + 1) * CH) {   // stores only
#pragma unroll
            for (int r = 0; r < N; r += 4)
                *reinterpret_cast<float4*>(&stg[(c - j * CH) * LD + r]) = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
        }
        wave_lds_sync();
#pragma unroll
        for (int r = j * CH; r < (j + 1) * CH; ++r) {
            const bool take = LOWER ? r >= c : r <= c;
            const float m = stg[(r - j * CH) * LD + c];
            x[r] = take ? x[r] : m;
        }
        wave_lds_sync();
    }
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

// x <- H_K x for K = K0, K0-1, ..., 0: the eigenvector of T in lane c
// becomes that of A (Q = H_0 H_1 ... H_{n-3}).  The reflectors come back
// from V's storage (packed: entries K+1 .. n-1 of v_K from
// refl_offset(K, n)) in blocks of kBT: a block is loaded (element c of each
// reflector by lane c) one block ahead, stored to LDS and read as
// broadcasts.  Reflectors past n - 3 are clamped into range and never used.
// The loads are masked (zero at and above row k) only when the block is
// staged, a block later: a select right after them would wait for them.
__device__ __forceinline__ int bt_k(int kb, int i, int n) {
    const int kmax = n - 3 > 0 ? n - 3 : 0;
    return kb - i < 0 ? 0 : (kb - i > kmax ? kmax : kb - i);
}
template <int N>
__device__ __forceinline__ void bt_fetch(float (&nx)[kBT], const float* vg, int kb, int c, int n) {
#pragma unroll
    for (int i = 0; i < kBT; ++i) {
        const int k = bt_k(kb, i, n);
        const bool in = c > k && c < n;   // v_k is zero at and above row k
        const int off = refl_offset(k, n);
        nx[i] = vg[in ? off + c - k - 1 : off];
    }
}

template <int K, int N>
__device__ __forceinline__ void backtransform_step(float (&x)[N], EighLds<N>& s, int c, int n, const float* vg,
                                                   float (&nx)[kBT]) {
    if constexpr (K >= 0) {
        constexpr int B = ((N - 3) - K) / kBT;   // block of K
        constexpr int I = ((N - 3) - K) % kBT;   // position in the block
        if constexpr (I == 0) {
#pragma unroll
            for (int i = 0; i < kBT; ++i) {
                const int k = bt_k(K, i, n);
                s.bt[B & 1][i][c] = (c > k && c < n) ? nx[i] : 0.0f;
            }
            if constexpr (K - kBT >= 0) bt_fetch<N>(nx, vg, K - kBT, c, n);
            wave_lds_sync();
        }
        if (K + 2 < n) {
            const float tau = s.tau[K];
            float v[N];
#pragma unroll
            for (int r = K + 1; r < N; ++r) v[r] = s.bt[B & 1][I][r];
            const float d = tau * dot_tail<K + 1, N>(v, x);
#pragma unroll
            for (int r = K + 1; r < N; ++r) x[r] = fmaf(-d, v[r], x[r]);
        }
        backtransform_step<K - 1, N>(x, s, c, n, vg, nx);
    }
}

// Stage 5-7 for lane c of group g: inverse iteration for the eigenvector
// of lam, MGS inside close groups, back-transform by the reflectors kept in
// V's storage, and column c of V written.  s holds d, e, 1/e and tau.
template <int N>
__device__ __forceinline__ void eigh_vectors(EighLds<N>& s, float (&x)[N], float* __restrict__ V, int c, int g,
                                             size_t mat, bool live, int nn, uint32_t n, size_t per, float lam,
                                             bool mine, bool diag, int row, bool all_diag, float tnorm, int bad) {
    // 5. inverse iteration: T - lam I = P L U with partial pivoting
    // (slagtf), the right-hand side carried along.  x[k] holds the
    // right-hand side, then row k of U scaled by its pivot (x, and u =
    // the superdiagonal entry where row k kept its place), then the
    // solution.  Where rows k and k+1 were swapped (u = NaN), U's row is
    // (e_k, d_{k+1} - lam, e_{k+1}), rebuilt from LDS on the way back.
    // The whole tridiagonal is solved: at a split (e = 0) the
    // elimination decouples, and rows past n (kPad, e = 0) carry zeros.
    // Eigenvectors of other blocks with an eigenvalue as close as this
    // one's fall into its close group below.
    const float tol = fmaxf(kEps * tnorm, kSafeMin);   // smaller pivots become +-tol
    float u[N];
    // the same start for every matrix: a matrix's result does not depend on
    // where it sits in the batch
#pragma unroll
    for (int k = 0; k < N; ++k) x[k] = k < nn ? hash_uniform((uint32_t)c, (uint32_t)k) : 0.0f;
    // close eigenvalues: lanes cs .. c with gaps <= kOrtol |T|
    const float prev = __shfl_up(lam, 1, N);
    const bool brk = c == 0 || !mine || diag || lam - prev > kOrtol * tnorm;
    uint64_t brks = __ballot(brk);
    if (N < 64) brks = (brks >> (g * N)) & ((1ull << N) - 1);
    const int cs = 63 - __clzll((unsigned long long)(brks & ((2ull << c) - 1)));
    const int pos = c - cs;
    int rounds = pos;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) rounds = max(rounds, __shfl_xor(rounds, off, 64));
    // inside a group, shifts at least 10 eps |T| apart (sstein's PERTOL):
    // with equal shifts every member's solve would be drawn to the same
    // vector of the group, and the Gram-Schmidt rounds would leave noise.
    // Member t of the group takes max(lam_t, shift_{t-1} + pertol), the
    // lanes reading the members' values in uniform rounds.
    float sigma = lam;
    {
        const float pertol = 10.0f * kEps * tnorm;
        float sp = __shfl(lam, g * N + cs, 64);
        for (int t = 1; t <= rounds; ++t) {
            const float lt = __shfl(lam, g * N + min(cs + t, N - 1), 64);
            if (t <= pos) sp = fmaxf(lt, sp + pertol);
        }
        if (pos > 0) sigma = sp;
    }
    for (int pass = 0; pass < (all_diag ? 0 : 2); ++pass) {
        float a = s.d[0] - sigma, cc = s.e[0], b0 = x[0];
        // d and e of the next row are read one step ahead (their LDS
        // latency hides behind this step's recurrence)
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
                u[k] = keep ? cc * r0 : qnan();   // NaN marks a swap
                // pinned: computed here, not sunk into the backward loop
                // with their factors kept live instead
                __asm__ volatile("" : "+v"(x[k]), "+v"(u[k]));
                const float na = keep ? fmaf(-l, cc, an) : fmaf(-l, an, cc);
                cc = keep ? cn : -l * cn;
                b0 = keep ? fmaf(-l, b0, b1) : fmaf(-l, b1, b0);
                a = na;
            } else {
                x[k] = b0 * __builtin_amdgcn_rcpf(fabsf(a) < tol ? copysignf(tol, a) : a);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // reload d, e from LDS below rather than keep the forward
        // loop's copies live across it
        __asm__ volatile("" ::: "memory");
        float x1 = 0.0f, x2 = 0.0f;
        float rnx = s.re[N - 2], dnx2 = s.d[N - 1], enx2 = s.e[N - 1];   // one step ahead
#pragma unroll
        for (int k = N - 1; k >= 0; --k) {
            float xv = x[k];
            if (k + 1 < N) {
                const float rk = rnx, dk1 = dnx2, ek1 = enx2;
                if (k > 0) {
                    rnx = s.re[k - 1];
                    dnx2 = s.d[k];
                    enx2 = s.e[k];
                }
                const bool swapped = u[k] != u[k];
                const float q1 = swapped ? (dk1 - sigma) * rk : u[k];
                const float q2 = swapped ? ek1 * rk : 0.0f;
                xv = fmaf(-q2, x2, fmaf(-q1, x1, xv));
            }
            x[k] = xv;
            __asm__ volatile("" : "+v"(x[k]));
            x2 = x1;
            x1 = xv;
            __builtin_amdgcn_sched_barrier(0);
        }
        normalize<N>(x);
        // modified Gram-Schmidt within each close group, one member per
        // round: the member at position t is final when round t begins
        for (int t = 0; t < rounds; ++t) {
            if (pos == t) normalize<N>(x);
            const int src = g * N + min(cs + t, N - 1);
            float dot = 0.0f;
#pragma unroll
            for (int k = 0; k < N; ++k) {
                u[k] = __shfl(x[k], src, 64);
                dot = fmaf(u[k], x[k], dot);
            }
            if (pos > t) {
#pragma unroll
                for (int k = 0; k < N; ++k) x[k] = fmaf(-dot, u[k], x[k]);
            }
        }
        normalize<N>(x);
    }

    if (diag) {
#pragma unroll
        for (int k = 0; k < N; ++k) x[k] = k == row ? 1.0f : 0.0f;
    }

    // 7. back to A's basis; lane c writes column c of V (over the
    // reflectors: every lane's loads of them have returned by the last
    // barrier of the back-transform)
    {
        float nx[kBT];
        const float* vsrc = V + (live ? mat : 0) * per;
        bt_fetch<N>(nx, vsrc, N - 3, c, nn);
        backtransform_step<N - 3, N>(x, s, c, nn, vsrc, nx);
    }
    if (live && mine) {
        float* dst = V + mat * per;
#pragma unroll
        for (int r = 0; r < N; ++r)
            if (r < nn) dst[(size_t)r * n + c] = bad ? qnan() : x[r];
    }
}

template <int N, bool VEC, bool SPLIT = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(SPLIT ? 4 : 1))) void eigh_small_kernel(const float* __restrict__ A, float* __restrict__ W,
                                                        float* __restrict__ V, uint32_t* __restrict__ info,
                                                        uint32_t batch, uint32_t n, int lower,
                                                        float* __restrict__ Sv) {
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
    {
        const float* src = A + (live ? mat : 0) * per;
        if (lower) load_symmetric<N, true>(x, s, src, c, nn);
        else load_symmetric<N, false>(x, s, src, c, nn);
        // every entry now comes from the read triangle (or is a zero pad):
        // the largest magnitude, and a NaN or infinity anywhere (v * 0 is
        // NaN exactly for those)
        float nz = 0.0f;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            amax = fmaxf(amax, fabsf(x[r]));
            nz = fmaf(x[r], 0.0f, nz);
        }
        bad = (live && nz != 0.0f) ? 1 : 0;   // nz is 0 or NaN
    }
    amax = group_max<N>(amax);
    bad = group_or<N>(bad);
    const int ex = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -ex);

    // 2. tridiagonalise: d, e, tau; v_k goes to V's storage (packed)
    // one matrix per wave: the base in SGPRs
    gfloat* vg = MPW == 1 ? uniform_gptr((VEC && live) ? V + mat * per : nullptr)
                          : global_ptr((VEC && live) ? V + mat * per : nullptr);
    tridiag_step<0, N>(x, s, c, nn, vg);
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
    wave_lds_sync();

    // 3. splits (sstebz's test, as ssteqr's), e^2, padding, Gershgorin bounds
    float ei = 0.0f;
    if (c < nn - 1) {
        ei = s.e[c];
        const float di = s.d[c], di1 = s.d[c + 1];
        if (fabsf(ei) <= kEps * (fabsf(di) + fabsf(di1)) || fabsf(ei) < kSafeMin) ei = 0.0f;
    }
    const bool split = c < nn - 1 && ei == 0.0f;
    uint64_t splits = __ballot(split);
    if (N < 64) splits = (splits >> (g * N)) & ((1ull << N) - 1);
    s.e[c] = ei;               // zero from row n - 1 on
    s.f[c + 1] = ei * ei;
    s.re[c] = ei != 0.0f ? __builtin_amdgcn_rcpf(ei) : 0.0f;
    if (c == 0) s.f[0] = 0.0f;
    if (c >= nn) s.d[c] = kPad;
    if (c < 4) {
        s.d[N + c] = kPad;
        s.e[N + c] = 0.0f;
        if (c > 0) s.f[N + c] = 0.0f;
        s.re[N + c] = 0.0f;
    }
    wave_lds_sync();
    float glo = FLT_MAX, ghi = -FLT_MAX;
    if (c < nn) {
        const float r = fabsf(ei) + (c > 0 ? fabsf(s.e[c - 1]) : 0.0f);
        const float dc = s.d[c];
        glo = dc - r;
        ghi = dc + r;
    }
    glo = -group_max<N>(-glo);
    ghi = group_max<N>(ghi);
    const float e2max = group_max<N>(ei * ei);
    const float tnorm = fmaxf(fabsf(glo), fabsf(ghi));
    const float pivmin = kSafeMin * fmaxf(1.0f, e2max);
    const float slack = 2.1f * 2.0f * kEps * tnorm * (float)nn + 4.2f * pivmin;
    const float atol = fmaxf(kEps * tnorm, 2.0f * pivmin);
    const float rbig = 1.0f / pivmin;

    // A diagonal T (every coupling split, e.g. A = a multiple of I, or the
    // zero matrix of a non-finite input): its eigenpairs are (d_j, e_j)
    // with j ranked by d (ties by index), exactly.  Waves holding only such
    // groups skip the bisection and the inverse iteration.
    const bool diag = nn == 1 || splits == ((1ull << (nn - 1)) - 1);
    const bool all_diag = __ballot(!diag) == 0;
    int row = c;
    if (diag && c < nn) {
        const float dc = s.d[c];
        int rank = 0;
        for (int i = 0; i < nn; ++i) {
            const float di = s.d[i];
            rank += (di < dc) || (di == dc && i < c);
        }
        s.perm[rank] = c;
    }
    wave_lds_sync();
    if (diag && c < nn) row = s.perm[c];

    // 4. bisection: lane c brackets the c-th smallest eigenvalue.  First
    // one multisection pass: lane i counts at the i-th of N + 1 equal
    // divisions of the Gershgorin interval, and every lane takes its bracket
    // from those counts (the points with at most c, and more than c,
    // eigenvalues below them); this replaces the first bisection steps, in
    // which the lanes would all count at the same few points.
    const bool mine = c < nn;
    const float g0 = glo - slack, g1 = ghi + slack, gh = (g1 - g0) / (float)(N + 1);
    float lo = g0, hi = g1;
    int steps = 0;
    if (!all_diag) {
        s.cnt[c] = sturm_count<N>(s, fmaf((float)(c + 1), gh, g0), rbig);
        wave_lds_sync();
#pragma unroll
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
    }
    while (!all_diag && steps < kMaxBisect) {
        const float mid = 0.5f * (lo + hi);
        const int cm = sturm_count<N>(s, mid, rbig);
        if (cm > c) {
            hi = mid;
        } else {
            lo = mid;
        }
        ++steps;
        const bool done = !mine || hi - lo <= fmaxf(atol, 2.0f * kEps * fmaxf(fabsf(lo), fabsf(hi)));
        if (__ballot(!done) == 0) break;
    }
    // ascending even where brackets of equal eigenvalues overlap: prefix max
    float lam = 0.5f * (lo + hi);
#pragma unroll
    for (int off = 1; off < N; off <<= 1) {
        const float up = __shfl_up(lam, off, N);
        if (c >= off) lam = fmaxf(lam, up);
    }
    if (diag) lam = s.d[row];

    if (VEC) {
        if (SPLIT) {
            // phase A of the split launch: what the vectors need, saved
            float* st = Sv + mat * kSplitFloats;
            if (live) {
                st[c] = s.d[c];
                st[N + c] = s.e[c];
                st[2 * N + c] = s.re[c];
                st[3 * N + c] = c < N - 2 ? s.tau[c] : 0.0f;
                st[4 * N + c] = lam;
                st[5 * N + c] = __int_as_float(diag ? row : -1);
                if (c == 0) {
                    st[6 * N] = tnorm;
                    st[6 * N + 1] = __int_as_float(all_diag ? 1 : 0);
                    st[6 * N + 2] = __int_as_float(bad);
                }
            }
        } else {
            eigh_vectors<N>(s, x, V, c, g, mat, live, nn, n, per, lam, mine, diag, row, all_diag, tnorm, bad);
        }
    }
    if (live && mine) W[mat * n + c] = bad ? qnan() : ldexpf(lam, ex);
    if (live && info && c == 0)
        info[mat] = bad ? (1u << 17) : ((uint32_t)steps | (1u << 16));
}

// Phase B of the split launch (n = 64 with vectors): stages 5-7 from the
// state phase A left.
__global__ __launch_bounds__(64) void eigh_vectors_kernel(const float* __restrict__ Sv, float* __restrict__ V,
                                                          uint32_t batch, uint32_t n) {
    constexpr int N = kSplitN;
    __shared__ EighLds<N> lds[1];
    EighLds<N>& s = lds[0];
    const int c = threadIdx.x;
    const size_t mat = blockIdx.x;
    const bool live = mat < batch;
    const int nn = (int)n;
    const size_t per = (size_t)n * n;
    const float* st = Sv + (live ? mat : 0) * kSplitFloats;
    s.d[c] = st[c];
    s.e[c] = st[N + c];
    s.re[c] = st[2 * N + c];
    s.tau[c] = st[3 * N + c];
    if (c < 4) {
        s.d[N + c] = kPad;
        s.e[N + c] = 0.0f;
        s.re[N + c] = 0.0f;
    }
    const float lam = st[4 * N + c];
    const int rw = __float_as_int(st[5 * N + c]);
    const float tnorm = st[6 * N];
    const bool all_diag = __float_as_int(st[6 * N + 1]) != 0;
    const int bad = __float_as_int(st[6 * N + 2]);
    wave_lds_sync();
    float x[N];
    eigh_vectors<N>(s, x, V, c, 0, mat, live, nn, n, per, lam, c < nn, rw >= 0, rw >= 0 ? rw : c, all_diag, tnorm,
                    bad);
}

template <int N, bool VEC>
void launch(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
            hipStream_t s) {
    constexpr int MPW = 64 / N;
    KernelTimer t("eigh_small", s);
    if constexpr (N == kSplitN && VEC) {
        hipLaunchKernelGGL((eigh_small_kernel<N, true, true>), dim3(batch), dim3(64), 0, s, a, w, v, info, batch, n,
                           lower ? 1 : 0, ws);
        hipLaunchKernelGGL(eigh_vectors_kernel, dim3(batch), dim3(64), 0, s, ws, v, batch, n);
    } else {
        hipLaunchKernelGGL((eigh_small_kernel<N, VEC>), dim3((uint32_t)cdiv(batch, MPW)), dim3(64), 0, s, a, w, v,
                           info, batch, n, lower ? 1 : 0, ws);
    }
    t.stop();
}

template <bool VEC>
void dispatch(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
              hipStream_t s) {
    if (n <= 8) launch<8, VEC>(a, w, v, info, batch, n, lower, ws, s);
    else if (n <= 16) launch<16, VEC>(a, w, v, info, batch, n, lower, ws, s);
    else if (n <= 32) launch<32, VEC>(a, w, v, info, batch, n, lower, ws, s);
    else launch<64, VEC>(a, w, v, info, batch, n, lower, ws, s);
}

}  // namespace

bool eigh_small_fits(uint32_t n) { return n >= 1 && n <= 64; }

size_t eigh_small_workspace(uint32_t n, uint32_t batch, bool vectors) {
    return (vectors && n > 32) ? (size_t)batch * kSplitFloats * sizeof(float) : 0;
}

void eigh_small(const float* a, float* w, float* v, uint32_t* info, uint32_t batch, uint32_t n, bool lower, float* ws,
                hipStream_t s) {
    if (!eigh_small_fits(n)) invalid("[eigh] eigh_small takes n <= 64");
    if (batch == 0) return;
    if (v && n > 32 && !ws) invalid("[eigh] eigh_small needs its workspace for n > 32 with vectors");
    if (v) dispatch<true>(a, w, v, info, batch, n, lower, ws, s);
    else dispatch<false>(a, w, nullptr, info, batch, n, lower, ws, s);
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
