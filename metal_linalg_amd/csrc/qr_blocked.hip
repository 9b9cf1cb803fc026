// Householder QR for matrices beyond the register kernel (more than 64 rows
// or columns; config 5's 4096 x 4096), one matrix at a time: sgeqrf's
// blocked factorization and sorgqr's blocked formation of Q.
//
// Role: the MI355X counterpart of the reference's qr_blocked (reference:
// src/qr_blocked.mm:153-302, src/band_reduce.mm:342-451: panels of
// reflectors, aggregated into compact WY form, trailing Z = Y^T C,
// W = Ta^T Z, C -= Y W; Q accumulated backward), with the conventions of
// the register kernel (shaders/QR_Householder.metal:189-300): the matrix
// scaled by a power of two so that its largest entry lies in [0.5, 1) (R
// unscaled on output), a reflector whose tail has a sum of squares below
// 2^-80 taken as the identity, and a matrix holding a NaN or an infinity
// written as all quiet NaN.  R is exactly zero below the diagonal.
//
// Per panel of NB = 128 columns (rows pj .. m - 1):
//   transpose     the panel into P (column-major: a column is contiguous)
//   qr_leaf       one workgroup of 512 threads per 16 columns: per column
//                 a sum of squares (DPP + LDS), the reflector, the dot
//                 products of the reflector with the leaf's other columns
//                 (an LDS transpose-reduction), the update, and the leaf's
//                 T (T[0:k, k] = -tau_k T[0:k, 0:k] V^T v_k) on the way
//   gram          Y = V^T C for the panel's later columns, split over rows
//   qr_apply      C -= V (T^T Y), one thread per row
//   qr_panel_t    the panel's 128 x 128 T from the leaves' T and V^T V (gram)
//   sgemm         W = V^T A2 (split over rows), summed, W = T^T W,
//                 A2 -= V W: the trailing matrix (MFMA)
// Q: [I; 0], then per panel from the last: Q2 -= V (T (V^T Q2)).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NB = 128;                        // panel width
constexpr int LW = 16;                         // leaf width
constexpr int LT = 512;                        // leaf threads
constexpr int kChunk = 512;                    // rows per split of a product over rows
constexpr int kPanelTThreads = 1024;           // the panel T kernel's workgroup (its block merges are thread-parallel)
constexpr float kTinySumsq = 8.271806e-25f;    // 2^-80

// ---- wave reductions through DPP ----

__device__ __forceinline__ float dpp_add_rows(float v) {
    // every lane of each row of 16 ends with the row's sum
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
    return v;
}

// lanes 31 and 63 end with the sums of lanes 0-31 and 32-63
__device__ __forceinline__ float dpp_add_halves(float v) {
    v = dpp_add_rows(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));   // row_bcast15
    return v;
}

// the wave's sum, in every lane (lane 63's value broadcast)
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add_halves(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));   // row_bcast31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---- scan and scale ----

__global__ __launch_bounds__(256) void scan_kernel(const float* __restrict__ a, size_t count,
                                                   uint32_t* __restrict__ flags) {
    // flags[0] = bits of max |a| (non-negative floats order as integers),
    // flags[1] = 1 if any entry is not finite
    unsigned m = 0, bad = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) {
        const float v = fabsf(a[i]);
        bad |= !(v <= FLT_MAX);
        m = v <= FLT_MAX ? max(m, __float_as_uint(v)) : m;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        m = max(m, (unsigned)__shfl_xor((int)m, o));
        bad |= (unsigned)__shfl_xor((int)bad, o);
    }
    if ((threadIdx.x & 63) == 0) {
        if (m) atomicMax(&flags[0], m);
        if (bad) atomicOr(&flags[1], 1u);
    }
}

__global__ void zero_flags_kernel(uint32_t* f) {
    f[0] = 0;
    f[1] = 0;
}

// dst = src * 2^-e (exact), e from the scanned maximum; 0 for a bad matrix
__global__ __launch_bounds__(256) void scale_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                         size_t count, const uint32_t* __restrict__ flags) {
    const bool bad = flags[1] != 0;
    const int e = bad ? 0 : scale_exponent(__uint_as_float(flags[0]));
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256)
        dst[i] = bad ? 0.0f : ldexpf(src[i], -e);
}

// ---- the leaf ----

template <int RPT>
struct LeafRows {
    static constexpr int G = RPT < 4 ? RPT : 4;
    __device__ static constexpr int row(int t, int q) { return (q / G) * (G * LT) + G * t + (q % G); }
};

struct QrLeafShared {
    float part[LT / 64];        // per-wave sums of squares
    float alpha;
    float red[LW][LT];          // per-thread partial dot products, by column
    float dot[LW];
    float tau[LW];
    float T[LW][LW + 1];
};

// Column K of the leaf.  Rows below the leaf's top hold the leaf's rows
// (row K of the leaf = the panel row of its diagonal).
template <int K, int RPT>
__device__ __forceinline__ void qr_leaf_column(float (&a)[RPT][LW], QrLeafShared& S, int t, int lane, int wv) {
    using R = LeafRows<RPT>;
    constexpr int G = R::G;
    constexpr int tk = K / G, qk = K % G;   // the thread and slot of row K
    // phase A: the tail's sum of squares and the head
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < RPT; ++q)
        if (q >= G || R::row(t, q) > K) ss = fmaf(a[q][K], a[q][K], ss);
    ss = wave_sum(ss);
    if (lane == 0) S.part[wv] = ss;
    if (t == tk) S.alpha = a[qk][K];
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < LT / 64; ++i) tot += S.part[i];
    const float alpha = S.alpha;
    float beta = alpha, tau = 0.0f, scal = 1.0f;
    if (tot >= kTinySumsq) {
        beta = -copysignf(sqrtf(fmaf(alpha, alpha, tot)), alpha);
        tau = (beta - alpha) / beta;
        scal = 1.0f / (alpha - beta);
    }
    // v: the tail scaled, 1 at row K (implicit); row K now holds beta
#pragma unroll
    for (int q = 0; q < RPT; ++q)
        if (q >= G || R::row(t, q) > K) a[q][K] *= scal;
    float v[RPT];
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = R::row(t, q);
        v[q] = (q >= G || li > K) ? a[q][K] : (li == K ? 1.0f : 0.0f);
    }
    if (t == tk) a[qk][K] = beta;
    // phase B: v^T a_c for every other column: for c > K the update's
    // coefficient, for c < K the entry (V^T v_K)_c of the leaf's T
#pragma unroll
    for (int c = 0; c < LW; ++c) {
        float p = 0.0f;
        if (c != K) {
#pragma unroll
            for (int q = 0; q < RPT; ++q) p = fmaf(v[q], a[q][c], p);
        }
        S.red[c][t] = p;
    }
    __syncthreads();
    {
        const int c = t >> 5, j = t & 31;   // 32 threads per column, 16 partials each
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < LT / 32; ++i) s += S.red[c][i * 32 + j];   // lanes on consecutive banks
        s = dpp_add_halves(s);
        if (lane == 31 || lane == 63) S.dot[c] = s;
    }
    if (t == 0) S.tau[K] = tau;
    __syncthreads();
    // phase C: the update of the later columns, and T's column K
#pragma unroll
    for (int c = K + 1; c < LW; ++c) {
        const float d = tau * S.dot[c];
#pragma unroll
        for (int q = 0; q < RPT; ++q) a[q][c] = fmaf(-d, v[q], a[q][c]);
    }
    if (t < K) {
        float s = 0.0f;
#pragma unroll
        for (int l = 0; l < K; ++l)
            if (l >= t) s = fmaf(S.T[t][l], S.dot[l], s);
        S.T[t][K] = -tau * s;
    }
    if (t == K) S.T[K][K] = tau;
}

template <int K, int RPT>
struct QrLeafColumns {
    __device__ __forceinline__ static void run(float (&a)[RPT][LW], QrLeafShared& S, int t, int lane, int wv, int w) {
        if constexpr (K < LW) {
            if (K < w) {   // uniform
                qr_leaf_column<K, RPT>(a, S, t, lane, wv);
                QrLeafColumns<K + 1, RPT>::run(a, S, t, lane, wv, w);
            }
        }
    }
};

// The leaf: panel columns cl .. cl + w - 1 (w <= 16), panel rows cl .. ldp - 1
// of P (column c of the panel at P + c * ldp).  Writes the factored columns
// back to P (R on and above the diagonal, V below), V^T's rows into Vt
// (row c at Vt + c * ldv: zeros left of the diagonal, then 1, then V), tau
// and the leaf's w x w T (row-major, stride LW).
template <int RPT>
__global__ __launch_bounds__(LT) void qr_leaf_kernel(float* __restrict__ P, int ldp, int cl, int w,
                                                     float* __restrict__ Vt, int ldv, float* __restrict__ tau_out,
                                                     float* __restrict__ Tleaf) {
    __shared__ QrLeafShared S;
    using R = LeafRows<RPT>;
    constexpr int G = R::G;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int m = ldp - cl;   // rows of the leaf
    float a[RPT][LW];
    const bool vec = G == 4 && (ldp & 3) == 0 && (cl & 3) == 0 && w == LW;
    if (vec) {
#pragma unroll
        for (int c = 0; c < LW; ++c) {
            const float* col = P + (size_t)(cl + c) * ldp + cl;
#pragma unroll
            for (int q0 = 0; q0 < RPT; q0 += G) {
                const int li = R::row(t, q0);
                const bool in = li + 3 < m;
                const float4 x = *reinterpret_cast<const float4*>(col + (in ? li : 0));
                a[q0][c] = in ? x.x : 0.0f;
                a[q0 + 1][c] = in ? x.y : 0.0f;
                a[q0 + 2][c] = in ? x.z : 0.0f;
                a[q0 + 3][c] = in ? x.w : 0.0f;
            }
        }
        if ((m & 3) != 0) {
#pragma unroll
            for (int q0 = 0; q0 < RPT; q0 += G) {
                const int li = R::row(t, q0);
                if (li < m && li + 3 >= m) {
#pragma unroll
                    for (int c = 0; c < LW; ++c)
#pragma unroll
                        for (int g = 0; g < G; ++g)
                            a[q0 + g][c] = li + g < m ? P[(size_t)(cl + c) * ldp + cl + li + g] : 0.0f;
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < LW; ++c)
#pragma unroll
            for (int q = 0; q < RPT; ++q) {
                const int li = R::row(t, q);
                const bool in = li < m && c < w;
                const float x = P[(size_t)(in ? cl + c : cl) * ldp + cl + (in ? li : 0)];
                a[q][c] = in ? x : 0.0f;
            }
    }
    QrLeafColumns<0, RPT>::run(a, S, t, lane, wv, w);

    // back to P, and V^T's rows; a thread's G consecutive rows move as one
    // 16-byte store where aligned and inside the leaf
    const bool vst = vec && (ldv & 3) == 0;
#pragma unroll
    for (int c = 0; c < LW; ++c) {
        if (c >= w) continue;
        float* col = P + (size_t)(cl + c) * ldp + cl;
        float* vrow = Vt + (size_t)(cl + c) * ldv + cl;
#pragma unroll
        for (int q0 = 0; q0 < RPT; q0 += G) {
            const int li = R::row(t, q0);
            float vv[G];
#pragma unroll
            for (int g = 0; g < G; ++g) vv[g] = li + g < c ? 0.0f : (li + g == c ? 1.0f : a[q0 + g][c]);
            if constexpr (G == 4) {
                if (vst && li + 3 < m) {
                    *reinterpret_cast<float4*>(col + li) = make_float4(a[q0][c], a[q0 + 1][c], a[q0 + 2][c], a[q0 + 3][c]);
                    *reinterpret_cast<float4*>(vrow + li) = make_float4(vv[0], vv[1], vv[2], vv[3]);
                    continue;
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g)
                if (li + g < m) {
                    col[li + g] = a[q0 + g][c];
                    vrow[li + g] = vv[g];
                }
        }
    }
    for (int idx = t; idx < w * cl; idx += LT) {   // V^T left of the leaf: zero
        const int c = idx / cl, r = idx - c * cl;
        Vt[(size_t)(cl + c) * ldv + r] = 0.0f;
    }
    __syncthreads();
    if (t < w) tau_out[cl + t] = S.tau[t];
    for (int idx = t; idx < LW * LW; idx += LT) {
        const int i = idx / LW, j = idx - i * LW;
        Tleaf[idx] = (i < w && j < w && j >= i) ? S.T[i][j] : 0.0f;
    }
}

// ---- the rest of the panel after a leaf: C -= V (T^T Y), Y = V^T C ----
//
// C^T is stored in P: panel column cl + w + c, panel row r at
// P[(cl + w + c) * ldp + r].  Y arrives as nsplit partial sums
// (w x ncol each, stride w * ncol).  One thread per row r (>= cl) and 16
// columns: V[r][k] = Vt[(cl + k) * ldv + r].
constexpr int kApplyCols = 16;

__global__ __launch_bounds__(256) void qr_leaf_apply_kernel(float* __restrict__ P, int ldp, int cl, int w, int ncol,
                                                            const float* __restrict__ Vt, int ldv,
                                                            const float* __restrict__ Ypart, int nsplit,
                                                            const float* __restrict__ Tleaf) {
    __shared__ float Tl[LW][LW];
    __shared__ float Y[LW][kApplyCols];
    __shared__ float Y2[LW][kApplyCols];
    const int t = threadIdx.x;
    const int c0 = blockIdx.y * kApplyCols;
    {
        const int k = t >> 4, c = t & 15;   // 256 = LW x kApplyCols
        Tl[k][c] = Tleaf[k * LW + c];
        float s = 0.0f;
        if (c0 + c < ncol && k < w)
            for (int b = 0; b < nsplit; ++b) s += Ypart[(size_t)b * w * ncol + (size_t)k * ncol + c0 + c];
        Y[k][c] = s;
    }
    __syncthreads();
    {
        // Y2 = T^T Y: Y2[k][c] = sum_{l <= k} T[l][k] Y[l][c]
        const int k = t >> 4, c = t & 15;
        float s = 0.0f;
#pragma unroll
        for (int l = 0; l < LW; ++l) s = l <= k ? fmaf(Tl[l][k], Y[l][c], s) : s;
        Y2[k][c] = s;
    }
    __syncthreads();
    const int r = cl + blockIdx.x * 256 + t;
    const int rr = r < ldp ? r : cl;
    float v[LW], cv[kApplyCols];
#pragma unroll
    for (int k = 0; k < LW; ++k) {
        const float x = Vt[(size_t)(cl + (k < w ? k : 0)) * ldv + rr];
        v[k] = k < w ? x : 0.0f;
    }
#pragma unroll
    for (int c = 0; c < kApplyCols; ++c) cv[c] = P[(size_t)(cl + w + (c0 + c < ncol ? c0 + c : 0)) * ldp + rr];
    if (r >= ldp) return;
#pragma unroll
    for (int c = 0; c < kApplyCols; ++c) {
        float s = cv[c];
#pragma unroll
        for (int k = 0; k < LW; ++k) s = fmaf(-v[k], Y2[k][c], s);
        if (c0 + c < ncol) P[(size_t)(cl + w + c0 + c) * ldp + r] = s;
    }
}

// ---- the panel's T (nbk x nbk, upper triangular, row-major) ----
//
// Diagonal 16 x 16 blocks are the leaves' T; block column j above them is
// T[0:16j, Bj] = -T[0:16j, 0:16j] (S[0:16j, Bj] T_jj), S = V^T V
// (nbk x nbk, row-major).
__global__ __launch_bounds__(kPanelTThreads) void qr_panel_t_kernel(const float* __restrict__ Ssum,
                                                         const float* __restrict__ Tleaves, int nbk,
                                                         float* __restrict__ Tout) {
    __shared__ float S[NB][NB + 1];
    __shared__ float T[NB][NB + 1];
    __shared__ float X[NB][LW + 1];
    const int t = threadIdx.x;
    for (int idx0 = 0; idx0 < NB * NB; idx0 += kPanelTThreads * 4) {
        float sv[4], tv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = idx0 + u * kPanelTThreads + t, i = idx >> 7, j = idx & (NB - 1);
            const bool in = i < nbk && j < nbk && j > i;
            const float sx = Ssum[in ? (size_t)i * nbk + j : 0];
            sv[u] = in ? sx : 0.0f;
            // diagonal blocks from the leaves
            const int bi = i / LW, bj = j / LW;
            const bool din = bi == bj && i < nbk && j < nbk;
            const float x = Tleaves[din ? (size_t)bi * LW * LW + (i % LW) * LW + (j % LW) : 0];
            tv[u] = din ? x : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = idx0 + u * kPanelTThreads + t;
            S[idx >> 7][idx & (NB - 1)] = sv[u];
            T[idx >> 7][idx & (NB - 1)] = tv[u];
        }
    }
    __syncthreads();
    const int nblk = (nbk + LW - 1) / LW;
    for (int jb = 1; jb < nblk; ++jb) {
        const int j0 = jb * LW, rows = j0;   // block column jb, rows 0 .. j0 - 1
        // X = S[0:j0, Bj] T_jj
        for (int idx = t; idx < rows * LW; idx += kPanelTThreads) {
            const int r = idx / LW, c = idx % LW;
            float s = 0.0f;
#pragma unroll
            for (int l = 0; l < LW; ++l) s = fmaf(S[r][j0 + l], T[j0 + l][j0 + c], s);
            X[r][c] = s;
        }
        __syncthreads();
        // T[0:j0, Bj] = -T[0:j0, 0:j0] X
        for (int idx = t; idx < rows * LW; idx += kPanelTThreads) {
            const int r = idx / LW, c = idx % LW;
            float s = 0.0f;
            for (int l = r; l < rows; ++l) s = fmaf(T[r][l], X[l][c], s);
            T[r][j0 + c] = -s;
        }
        __syncthreads();
    }
    for (int idx = t; idx < nbk * nbk; idx += kPanelTThreads) {
        const int i = idx / nbk, j = idx - i * nbk;
        Tout[idx] = T[i][j];
    }
}

// ---- helpers ----

__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ src, int lds, float* __restrict__ dst,
                                                        int ldd, int rows, int cols) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = src[(size_t)(r0 + r) * lds + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 32; c += 8)
        if (c0 + c < cols && r0 + tx < rows) dst[(size_t)(c0 + c) * ldd + r0 + tx] = tile[tx][c];
}

void transpose(const float* src, int lds, float* dst, int ldd, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32)), dim3(256), 0, s, src,
                       lds, dst, ldd, rows, cols);
}

// Products of row vectors over a split of their length:
//   part[b][i][j] = sum_{r in chunk b} X[i][r] Y[j][r]
// (X: M rows, Y: N rows, both with row stride ld, entries 0 .. K - 1;
// chunks of kChunk).  For the thin products of the panel -- V^T C with 16
// reflectors, V^T V -- whose outputs are too few for matrix-core tiles:
// a workgroup takes 16 x 16 outputs of one chunk, both operands' slices
// staged in LDS, one output per thread, four entries per LDS read.
constexpr int kGramTile = 16;

__global__ __launch_bounds__(256) void gram_kernel(const float* __restrict__ X, const float* __restrict__ Y, int ld,
                                                   int M, int N, int K, float* __restrict__ part) {
    __shared__ float xs[kGramTile][kChunk + 4];
    __shared__ float ys[kGramTile][kChunk + 4];
    const int t = threadIdx.x;
    const int i0 = blockIdx.x * kGramTile, j0 = blockIdx.y * kGramTile, b = blockIdx.z;
    const int r0 = b * kChunk;
    const int len = min(kChunk, K - r0);
    // stage: 16 rows x kChunk of each operand; 4-float groups, clamped loads
    const bool vec = (ld & 3) == 0 && (((uintptr_t)X | (uintptr_t)Y) & 15) == 0;
    constexpr int groups = kGramTile * kChunk / 4;   // 2048 per operand
#pragma unroll
    for (int g0 = 0; g0 < groups; g0 += 256 * 4) {
        float4 xv[4], yv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int g = g0 + u * 256 + t, row = g / (kChunk / 4), c4 = (g % (kChunk / 4)) * 4;
            const bool xin = i0 + row < M, yin = j0 + row < N;
            const size_t xo = (size_t)(xin ? i0 + row : 0) * ld + r0 + c4;
            const size_t yo = (size_t)(yin ? j0 + row : 0) * ld + r0 + c4;
            if (vec && c4 + 3 < len) {
                xv[u] = *reinterpret_cast<const float4*>(X + xo);
                yv[u] = *reinterpret_cast<const float4*>(Y + yo);
            } else {
                float xx[4], yy[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool in = c4 + e < len;
                    xx[e] = X[in ? xo + e : 0];
                    yy[e] = Y[in ? yo + e : 0];
                    xx[e] = in ? xx[e] : 0.0f;
                    yy[e] = in ? yy[e] : 0.0f;
                }
                xv[u] = make_float4(xx[0], xx[1], xx[2], xx[3]);
                yv[u] = make_float4(yy[0], yy[1], yy[2], yy[3]);
            }
            if (!xin) xv[u] = make_float4(0, 0, 0, 0);
            if (!yin) yv[u] = make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int g = g0 + u * 256 + t, row = g / (kChunk / 4), c4 = (g % (kChunk / 4)) * 4;
            *reinterpret_cast<float4*>(&xs[row][c4]) = xv[u];
            *reinterpret_cast<float4*>(&ys[row][c4]) = yv[u];
        }
    }
    __syncthreads();
    const int i = t >> 4, j = t & 15;
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int r = 0; r < kChunk; r += 8) {
        const float4 a0 = *reinterpret_cast<const float4*>(&xs[i][r]);
        const float4 b0 = *reinterpret_cast<const float4*>(&ys[j][r]);
        const float4 a1 = *reinterpret_cast<const float4*>(&xs[i][r + 4]);
        const float4 b1 = *reinterpret_cast<const float4*>(&ys[j][r + 4]);
        acc0 = fmaf(a0.x, b0.x, acc0);
        acc1 = fmaf(a1.x, b1.x, acc1);
        acc0 = fmaf(a0.y, b0.y, acc0);
        acc1 = fmaf(a1.y, b1.y, acc1);
        acc0 = fmaf(a0.z, b0.z, acc0);
        acc1 = fmaf(a1.z, b1.z, acc1);
        acc0 = fmaf(a0.w, b0.w, acc0);
        acc1 = fmaf(a1.w, b1.w, acc1);
    }
    if (i0 + i < M && j0 + j < N) part[(size_t)b * M * N + (size_t)(i0 + i) * N + j0 + j] = acc0 + acc1;
}

int gram(const float* X, const float* Y, int ld, int M, int N, int K, float* part, hipStream_t s) {
    const int nsplit = cdiv(K, kChunk);
    hipLaunchKernelGGL(gram_kernel, dim3((unsigned)cdiv(M, kGramTile), (unsigned)cdiv(N, kGramTile), (unsigned)nsplit),
                       dim3(256), 0, s, X, Y, ld, M, N, K, part);
    return nsplit;
}

// out[i] = sum_b part[b][i], in order of b; eight partials in flight at a
// time (indices past the last read it again and add zero)
__global__ __launch_bounds__(256) void sum_parts_kernel(const float* __restrict__ part, int nsplit, size_t count,
                                                        float* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) {
        float s = 0.0f;
        for (int b0 = 0; b0 < nsplit; b0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = part[(size_t)min(b0 + j, nsplit - 1) * count + i];
#pragma unroll
            for (int j = 0; j < 8; ++j) s += v[j] * (b0 + j < nsplit ? 1.0f : 0.0f);
        }
        out[i] = s;
    }
}

__global__ __launch_bounds__(256) void identity_kernel(float* __restrict__ q, int m, int qc) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)m * qc) return;
    const int i = (int)(idx / qc), j = (int)(idx - (size_t)i * qc);
    q[idx] = i == j ? 1.0f : 0.0f;
}

// R (rr x n) from the factored matrix: the upper trapezoid unscaled, zero
// below; all NaN for a bad matrix
__global__ __launch_bounds__(256) void extract_r_kernel(const float* __restrict__ A, int m, int n, int rr,
                                                        float* __restrict__ R, const uint32_t* __restrict__ flags) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rr * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (size_t)i * n);
    const bool bad = flags[1] != 0;
    const int e = bad ? 0 : scale_exponent(__uint_as_float(flags[0]));
    const int k = m < n ? m : n;
    R[idx] = bad ? qnan() : ((i < k && j >= i) ? ldexpf(A[(size_t)i * n + j], e) : 0.0f);
}

__global__ __launch_bounds__(256) void nan_if_bad_kernel(float* __restrict__ x, size_t count,
                                                         const uint32_t* __restrict__ flags) {
    if (flags[1] == 0) return;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) x[i] = qnan();
}

unsigned grid_for(size_t count) { return (unsigned)std::min<size_t>(cdiv(count, 256), 4096); }

// C = alpha A B (+ beta C) split over K in chunks of kChunk: part[b] gets the
// chunk b product (A: M x K with K-stride 1 per column, lda; B: K x N rows
// ldb, or with tb B stored N x K).  Returns the number of parts.
int split_k_gemm(bool tb, int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* part,
                 hipStream_t s) {
    // one batched launch, the last chunk shorter
    const int nsplit = cdiv(K, kChunk), last = K - (nsplit - 1) * kChunk;
    const long long sb = tb ? kChunk : (long long)kChunk * ldb;
    sgemm(false, tb, M, N, kChunk, 1.0f, A, lda, kChunk, B, ldb, sb, 0.0f, part, N, (long long)M * N, nsplit, s,
          false, last);
    return nsplit;
}

template <int RPT>
void launch_leaf(float* P, int ldp, int cl, int w, float* Vt, int ldv, float* tau, float* Tleaf, hipStream_t s) {
    hipLaunchKernelGGL((qr_leaf_kernel<RPT>), dim3(1), dim3(LT), 0, s, P, ldp, cl, w, Vt, ldv, tau, Tleaf);
}

void leaf(int m_rows, float* P, int ldp, int cl, int w, float* Vt, int ldv, float* tau, float* Tleaf, hipStream_t s) {
    if (m_rows <= LT) launch_leaf<1>(P, ldp, cl, w, Vt, ldv, tau, Tleaf, s);
    else if (m_rows <= 2 * LT) launch_leaf<2>(P, ldp, cl, w, Vt, ldv, tau, Tleaf, s);
    else if (m_rows <= 4 * LT) launch_leaf<4>(P, ldp, cl, w, Vt, ldv, tau, Tleaf, s);
    else launch_leaf<8>(P, ldp, cl, w, Vt, ldv, tau, Tleaf, s);
}

struct QrWork {
    float *A, *P, *Vt, *T, *tau, *Tleaves, *part, *W, *W2;
    uint32_t* flags;
};

QrWork carve(float* base, int m, int n) {
    const int k = std::min(m, n);
    const int npan = cdiv(k, NB);
    const int nsplit = cdiv(m, kChunk);
    const int wide = std::max(m, n);
    QrWork w{};
    float* p = base;
    auto take = [&](size_t count) {
        float* r = p;
        p += (count + 63) / 64 * 64;
        return r;
    };
    w.A = take((size_t)m * n);
    w.P = take((size_t)NB * m);
    w.Vt = take((size_t)npan * NB * m);
    w.T = take((size_t)npan * NB * NB);
    w.tau = take((size_t)k);
    w.Tleaves = take((size_t)(NB / LW) * LW * LW);
    w.part = take((size_t)nsplit * NB * wide);
    w.W = take((size_t)NB * wide);
    w.W2 = take((size_t)NB * wide);
    w.flags = reinterpret_cast<uint32_t*>(take(64));
    return w;
}

}  // namespace

// the leaf holds up to 8 rows per thread: m <= 4096
bool qr_blocked_fits(uint32_t m, uint32_t n) { return m <= 8 * (uint32_t)LT && n <= 65536; }

size_t qr_blocked_workspace(uint32_t m, uint32_t n) {
    const int k = (int)std::min(m, n);
    const int npan = cdiv(k, NB);
    const int nsplit = cdiv((int)m, kChunk);
    const size_t wide = std::max(m, n);
    const size_t floats = (size_t)m * n + (size_t)NB * m + (size_t)npan * NB * m + (size_t)npan * NB * NB + k +
                          (size_t)(NB / LW) * LW * LW + (size_t)nsplit * NB * wide + 2 * (size_t)NB * wide + 64;
    return (floats + 64 * 12) * sizeof(float);
}

// One m x n matrix a -> q (m x qc, row-major; qc = 0: none) and r (rr x n).
void qr_blocked_one(const float* a, float* q, float* r, int m, int n, int qc, int rr, float* work, hipStream_t s) {
    const int k = std::min(m, n);
    QrWork w = carve(work, m, n);
    const size_t count = (size_t)m * n;
    hipLaunchKernelGGL(zero_flags_kernel, dim3(1), dim3(1), 0, s, w.flags);
    hipLaunchKernelGGL(scan_kernel, dim3(grid_for(count)), dim3(256), 0, s, a, count, w.flags);
    hipLaunchKernelGGL(scale_copy_kernel, dim3(grid_for(count)), dim3(256), 0, s, a, w.A, count, w.flags);

    int pi = 0;
    for (int pj = 0; pj < k; pj += NB, ++pi) {
        const int pe = std::min(pj + NB, k), nbk = pe - pj, ldp = m - pj;
        float* panel = w.A + (size_t)pj * n + pj;
        float* Vt = w.Vt + (size_t)pi * NB * m;   // nbk rows of length ldp (ld = ldp)
        const int ldv = ldp;
        transpose(panel, n, w.P, ldp, ldp, nbk, s);
        {
            KernelTimer tm("qr_panel", s);
            for (int cl = 0; cl < nbk; cl += LW) {
                const int lw = std::min(LW, nbk - cl);
                leaf(ldp - cl, w.P, ldp, cl, lw, Vt, ldv, w.tau + pj, w.Tleaves + (size_t)(cl / LW) * LW * LW, s);
                const int ncol = nbk - cl - lw;
                if (ncol > 0) {
                    // Y = V^T C over the leaf's rows, then C -= V (T^T Y)
                    const int rows = ldp - cl;
                    const int nsplit = gram(Vt + (size_t)cl * ldv + cl, w.P + (size_t)(cl + lw) * ldp + cl, ldp, lw,
                                            ncol, rows, w.part, s);
                    hipLaunchKernelGGL(qr_leaf_apply_kernel,
                                       dim3((unsigned)cdiv(rows, 256), (unsigned)cdiv(ncol, kApplyCols)), dim3(256),
                                       0, s, w.P, ldp, cl, lw, ncol, Vt, ldv, w.part, nsplit,
                                       w.Tleaves + (size_t)(cl / LW) * LW * LW);
                }
            }
            tm.stop();
        }
        transpose(w.P, ldp, panel, n, nbk, ldp, s);
        // the panel's T from the leaves' T and S = V^T V
        float* T = w.T + (size_t)pi * NB * NB;
        {
            const int nsplit = gram(Vt, Vt, ldv, nbk, nbk, ldp, w.part, s);
            hipLaunchKernelGGL(sum_parts_kernel, dim3(grid_for((size_t)nbk * nbk)), dim3(256), 0, s, w.part, nsplit,
                               (size_t)nbk * nbk, w.W);
            hipLaunchKernelGGL(qr_panel_t_kernel, dim3(1), dim3(kPanelTThreads), 0, s, w.W, w.Tleaves, nbk, T);
        }
        // trailing matrix: A2 -= V (T^T (V^T A2))
        const int n2 = n - pe;
        if (n2 > 0) {
            float* A2 = w.A + (size_t)pj * n + pe;
            const int nsplit = split_k_gemm(false, nbk, n2, ldp, Vt, ldv, A2, n, w.part, s);
            hipLaunchKernelGGL(sum_parts_kernel, dim3(grid_for((size_t)nbk * n2)), dim3(256), 0, s, w.part, nsplit,
                               (size_t)nbk * n2, w.W);
            sgemm(true, false, nbk, n2, nbk, 1.0f, T, nbk, 0, w.W, n2, 0, 0.0f, w.W2, n2, 0, 1, s);
            sgemm(true, false, ldp, n2, nbk, -1.0f, Vt, ldv, 0, w.W2, n2, 0, 1.0f, A2, n, 0, 1, s);
        }
    }

    hipLaunchKernelGGL(extract_r_kernel, dim3((unsigned)cdiv((size_t)rr * n, 256)), dim3(256), 0, s, w.A, m, n, rr, r,
                       w.flags);
    if (qc > 0) {
        KernelTimer tq("qr_form_q", s);
        hipLaunchKernelGGL(identity_kernel, dim3((unsigned)cdiv((size_t)m * qc, 256)), dim3(256), 0, s, q, m, qc);
        for (int pj = (k - 1) / NB * NB, pi2 = (k - 1) / NB; pj >= 0; pj -= NB, --pi2) {
            const int pe = std::min(pj + NB, k), nbk = pe - pj, ldp = m - pj;
            const float* Vt = w.Vt + (size_t)pi2 * NB * m;
            const float* T = w.T + (size_t)pi2 * NB * NB;
            const int nq = qc - pj;
            float* Q2 = q + (size_t)pj * qc + pj;
            const int nsplit = split_k_gemm(false, nbk, nq, ldp, Vt, ldp, Q2, qc, w.part, s);
            hipLaunchKernelGGL(sum_parts_kernel, dim3(grid_for((size_t)nbk * nq)), dim3(256), 0, s, w.part, nsplit,
                               (size_t)nbk * nq, w.W);
            sgemm(false, false, nbk, nq, nbk, 1.0f, T, nbk, 0, w.W, nq, 0, 0.0f, w.W2, nq, 0, 1, s);
            sgemm(true, false, ldp, nq, nbk, -1.0f, Vt, ldp, 0, w.W2, nq, 0, 1.0f, Q2, qc, 0, 1, s);
        }
        tq.stop();
        hipLaunchKernelGGL(nan_if_bad_kernel, dim3(grid_for((size_t)m * qc)), dim3(256), 0, s, q, (size_t)m * qc,
                           w.flags);
    }
    MLA_HIP(hipGetLastError());
}

void qr_blocked(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
                float* work, hipStream_t s) {
    for (uint32_t b = 0; b < batch; ++b)
        qr_blocked_one(a + (size_t)b * m * n, q ? q + (size_t)b * m * qc : nullptr, r + (size_t)b * rr * n, (int)m,
                       (int)n, (int)qc, (int)rr, work, s);
}

}  // namespace mla
