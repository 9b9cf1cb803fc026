// LU with partial pivoting, and the triangular solves built on it, for
// matrices beyond the register kernels (n > 32; config 5's 4096 x 4096),
// one matrix at a time.
//
// Role: the MI355X counterpart of the reference's blocked LU (reference:
// src/lu_gpu.mm:146-441: panel LU with composed swap lists, L11^-1 A12 for
// the U12 block, trailing A22 -= L21 U12 as a matrix product, look-ahead),
// with the CPU path's contract (src/lu_cpu.mm:72-157): sgetrf's partial
// pivoting (the first entry of largest magnitude, 0-based sequential swaps,
// applied to whole rows), info = k for the first exactly-zero U(k-1, k-1)
// with the factorization completed; solve and inv give all-NaN x for
// info > 0.  Triangular solves (src/trsm.mm:193-206) read one triangle, a
// unit diagonal not at all.
//
// The reference factors its panels on the CPU; here everything stays on the
// GPU.  Per panel of NB = 128 columns (right-looking):
//   lu_leaf      one workgroup of 512 threads factors a leaf of W columns
//                (rows pc..n-1 held in registers, RPT rows per thread) with
//                one barrier per column: a 64-bit (|pivot| bits, ~row) max
//                reduction picks the pivot, each wave publishing its best
//                candidate row alongside; then it applies its W swaps to the
//                rest of the panel and solves U rows of the panel's later
//                columns with its unit L11 (both through LDS staging)
//   panel_update the rest of the panel: A -= L_leaf U_leaf (a thin rank-W
//                update, coalesced VALU)
//   lu_swap      the panel's swaps on every column outside the panel
//   trsm_block   U12 = L11^-1 A12 (column-parallel, 16-row steps)
//   sgemm        A22 -= L21 U12 (MFMA)
#include <cstring>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NB = 128;                       // panel width
constexpr float kSfmin = 1.17549435e-38f;     // FLT_MIN: sgetf2 divides below it
constexpr uint32_t kMaxBlockedN = 16384;

// ---------------------------------------------------------------------------
// leaf factorization
// ---------------------------------------------------------------------------

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long shfl_xor64(unsigned long long v, int m) {
    const unsigned lo = __shfl_xor((unsigned)(v & 0xffffffffu), m);
    const unsigned hi = __shfl_xor((unsigned)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

constexpr int LT = 512;   // leaf threads (8 waves)

// Wave-wide maximum of an unsigned value through DPP (row-local swaps and
// mirrors, then the row broadcasts), the result read from lane 63: a few
// cycles per step, against an LDS round trip per step for a shuffle.
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));    // quad_perm 1,0,3,2
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));    // quad_perm 2,3,0,1
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));   // row_half_mirror
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));   // row_mirror
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));   // row_bcast15
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));   // row_bcast31
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

// LDS of the leaf.  Per column, slots alternate by column parity so that one
// barrier per column suffices (a slot is rewritten two columns later, after
// every thread has passed the barrier that follows its reads).
struct LeafShared {
    unsigned long long cand[2][LT / 64];   // each wave's best pivot: key << 32 | ~row
    float crow[2][LT / 64][16];            // and that candidate's row
    float krow[2][16];                     // row k before the exchange
    int plist[16];
};

// Rows of a leaf thread: groups of G = min(RPT, 4) consecutive rows, so that
// a column's rows move as float4s; group j of thread t starts at row
// j * G * LT + G * t.  Rows below 16 all lie in group 0.
template <int RPT>
struct LeafRows {
    static constexpr int G = RPT < 4 ? RPT : 4;
    __device__ static constexpr int row(int t, int q) { return (q / G) * (G * LT) + G * t + (q % G); }
};

// One elimination step of the leaf (column K), a template so that every
// register index is a compile-time constant.  Every wave publishes its best
// candidate key and that row; after the barrier every thread picks the
// winner, so the pivot row arrives with the choice.
// The source row of row x under the sequential swaps k <-> pl[k] for k =
// 0 .. m-1, found by undoing them from the last; pl is read 8 entries at a
// time so that the LDS reads overlap instead of one round trip per swap.
__device__ __forceinline__ int undo_swaps(const int* pl, int m, int x) {
    for (int k1 = m; k1 > 0;) {
        const int k0 = k1 >= 8 ? k1 - 8 : 0;
        int p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = pl[k0 + i < k1 ? k0 + i : k0];
#pragma unroll
        for (int i = 7; i >= 0; --i) {
            const int k = k0 + i;
            if (k < k1) x = x == k ? p[i] : (x == p[i] ? k : x);
        }
        k1 = k0;
    }
    return x;
}

template <int K, int RPT, int W>
__device__ __forceinline__ void leaf_column(float (&a)[RPT][W], LeafShared& S, int t, int lane, int wv,
                                            int& zero_at) {
    using R = LeafRows<RPT>;
    constexpr int G = R::G;
    constexpr int sl = K & 1;
    // this thread's candidate: rows in ascending order, strictly larger wins
    // (the first of equal values); NaN never wins, except in row K itself,
    // which then outranks everything (key all ones).  Rows past the matrix
    // hold zeros and come after every real row: they never win.
    unsigned key = 0, nrow = 0;   // nrow = ~row (larger for earlier rows)
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        const int li = R::row(t, q);
        const bool ok = q >= G || li >= K;
        const float av = fabsf(a[q][K]);
        const unsigned kq = av != av ? (li == K ? 0xffffffffu : 0u) : __float_as_uint(av);
        const bool take = ok && (kq > key || nrow == 0);
        key = take ? kq : key;
        nrow = take ? ~(unsigned)li : nrow;
    }
    // the wave's best: the largest key, then the first row with it
    const unsigned wkey = wave_max_u32(key);
    const unsigned wrow = wave_max_u32(key == wkey ? nrow : 0u);
    const int lw = (int)~wrow;
    if (wrow != 0) {
        if (lane == 0) S.cand[sl][wv] = ((unsigned long long)wkey << 32) | wrow;
#pragma unroll
        for (int q = 0; q < RPT; ++q)
            if (R::row(t, q) == lw) {   // one lane, one q: the other blocks are skipped
#pragma unroll
                for (int c = 0; c < W; ++c) S.crow[sl][wv][c] = a[q][c];
            }
    } else if (lane == 0) {
        S.cand[sl][wv] = 0;
    }
    constexpr int tk = K / G, qk = K % G;   // the thread and slot of row K
    if (t == tk) {
#pragma unroll
        for (int c = 0; c < W; ++c) S.krow[sl][c] = a[qk][c];
    }
    __syncthreads();
    // the winner among the waves (pairwise: the earlier wave wins ties; keys
    // are distinct anyway, since they carry the row)
    unsigned long long c8[LT / 64];
#pragma unroll
    for (int i = 0; i < LT / 64; ++i) c8[i] = S.cand[sl][i];
    int gi[LT / 64];
#pragma unroll
    for (int i = 0; i < LT / 64; ++i) gi[i] = i;
#pragma unroll
    for (int span = 1; span < LT / 64; span *= 2)
#pragma unroll
        for (int i = 0; i + span < LT / 64; i += 2 * span)
            if (c8[i + span] > c8[i]) {
                c8[i] = c8[i + span];
                gi[i] = gi[i + span];
            }
    const int p = __builtin_amdgcn_readfirstlane((int)~(unsigned)(c8[0] & 0xffffffffu));
    const int gw = __builtin_amdgcn_readfirstlane(gi[0]);
    float u[W];
#pragma unroll
    for (int c = 0; c < W; ++c) u[c] = S.crow[sl][gw][c];   // the new row K
    const float pv = u[K];
    if (p != K) {   // uniform
        if (t == tk) {
#pragma unroll
            for (int c = 0; c < W; ++c) a[qk][c] = u[c];
        }
#pragma unroll
        for (int q = 0; q < RPT; ++q)
            if (R::row(t, q) == p) {
#pragma unroll
                for (int c = 0; c < W; ++c) a[q][c] = S.krow[sl][c];
            }
    }
    if (pv == 0.0f && zero_at == 0) zero_at = K + 1;
    if (t == 0) S.plist[K] = p;
    // multipliers (rows below K) and the rank-1 update of the rows below K
    // only (rows <= K are not touched, as sger's: no 0 * NaN from a
    // non-finite pivot row)
    if (pv != 0.0f) {   // uniform
        if (fabsf(pv) >= kSfmin) {
            const float inv = 1.0f / pv;
#pragma unroll
            for (int q = 0; q < RPT; ++q)
                if (q >= G || R::row(t, q) > K) a[q][K] *= inv;
        } else {
#pragma unroll
            for (int q = 0; q < RPT; ++q)
                if (q >= G || R::row(t, q) > K) a[q][K] /= pv;
        }
    }
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        if (q >= G || R::row(t, q) > K) {   // rows past group 0 are all below K
            const float l = a[q][K];
#pragma unroll
            for (int c = K + 1; c < W; ++c) a[q][c] = fmaf(-l, u[c], a[q][c]);
        }
    }
}

template <int K, int RPT, int W>
struct LeafColumns {
    __device__ __forceinline__ static void run(float (&a)[RPT][W], LeafShared& S, int t, int lane, int wv, int w,
                                               int& zero_at) {
        if constexpr (K < W) {
            if (K < w) {   // uniform
                leaf_column<K, RPT, W>(a, S, t, lane, wv, zero_at);
                LeafColumns<K + 1, RPT, W>::run(a, S, t, lane, wv, w, zero_at);
            }
        }
    }
};

// Leaf of W columns pc .. pc + w - 1 (w <= W) over rows pc .. n - 1 of the
// n x n matrix, whose panel (columns pj .. pe - 1, rows pj .. n - 1) is held
// transposed in P: panel column c, row r at P[(c - pj) * ldp + r - pj],
// ldp = n - pj, so that a column is contiguous and the leaf's loads coalesce.
// Pivot choice, as isamax on the column below the diagonal: the largest
// |a|, the first such row on ties; a NaN never wins, except a NaN in row k
// itself, which stays (the scan compares against it and every comparison
// fails).  Keys: (bits of |a|, ~row) as one 64-bit integer, NaN in row k
// -> all ones, NaN elsewhere -> 0.
template <int RPT, int W>
__global__ __launch_bounds__(LT) void lu_leaf_kernel(float* __restrict__ P, int n, int pc, int pj, int pe, int w,
                                                       uint32_t* __restrict__ piv, uint32_t* __restrict__ info) {
    __shared__ LeafShared S;
    __shared__ int edst[2 * W], esrc[2 * W];
    __shared__ float stage[2 * W][NB];
    __shared__ float Ls[W][W + 1];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int m = n - pc;
    float a[RPT][W];
    const int ldp = n - pj, r0 = pc - pj, cl = pc - pj;   // the leaf's first row and column in P
    using R = LeafRows<RPT>;
    constexpr int G = R::G;
    // A column's G consecutive rows of a thread move together when aligned.
    // Every load is issued unconditionally (from a clamped address, the value
    // then masked) so that all of them are in flight before the first wait.
    const bool vec = G == 4 && (ldp & 3) == 0 && w == W;
    if (vec) {
#pragma unroll
        for (int c = 0; c < W; ++c) {
            const float* col = P + (size_t)(cl + c) * ldp + r0;
#pragma unroll
            for (int q0 = 0; q0 < RPT; q0 += G) {
                const int li = R::row(t, q0);
                const bool in = li + 3 < m;
                const float4 v = *reinterpret_cast<const float4*>(col + (in ? li : 0));
                a[q0][c] = in ? v.x : 0.0f;
                a[q0 + 1][c] = in ? v.y : 0.0f;
                a[q0 + 2][c] = in ? v.z : 0.0f;
                a[q0 + 3][c] = in ? v.w : 0.0f;
            }
        }
        // the last, partial group of rows (m not a multiple of 4)
        if ((m & 3) != 0) {
#pragma unroll
            for (int q0 = 0; q0 < RPT; q0 += G) {
                const int li = R::row(t, q0);
                if (li < m && li + 3 >= m) {
#pragma unroll
                    for (int c = 0; c < W; ++c)
#pragma unroll
                        for (int g = 0; g < G; ++g)
                            a[q0 + g][c] = li + g < m ? P[(size_t)(cl + c) * ldp + r0 + li + g] : 0.0f;
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < W; ++c)
#pragma unroll
            for (int q = 0; q < RPT; ++q) {
                const int li = R::row(t, q);
                const bool in = li < m && c < w;
                const float v = P[(size_t)(in ? cl + c : cl) * ldp + r0 + (in ? li : 0)];
                a[q][c] = in ? v : 0.0f;
            }
    }
    int zero_at = 0;
    LeafColumns<0, RPT, W>::run(a, S, t, lane, wv, w, zero_at);
    // the leaf back to P; pivots (global, 0-based) and info
#pragma unroll
    for (int c = 0; c < W; ++c) {
        float* col = P + (size_t)(cl + c) * ldp + r0;
#pragma unroll
        for (int q0 = 0; q0 < RPT; q0 += G) {
            const int li = R::row(t, q0);
            if (c >= w) continue;
            if (vec && li + 3 < m) {
                *reinterpret_cast<float4*>(col + li) = make_float4(a[q0][c], a[q0 + 1][c], a[q0 + 2][c], a[q0 + 3][c]);
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    if (li + g < m) col[li + g] = a[q0 + g][c];
            }
        }
    }
    __syncthreads();   // plist complete
    if (t < w) piv[pc + t] = (uint32_t)(pc + S.plist[t]);
    if (t == 0 && zero_at != 0 && *info == 0) *info = (uint32_t)(pc + zero_at);

    // the other columns of the panel: the leaf's swaps, then (right of the
    // leaf) the W rows of U:  U12 = L11^-1 A12
    const int ncl = pc - pj, ncr = pe - pc - w, nco = ncl + ncr;
    if (nco <= 0) return;   // uniform
    // compose the sequential swaps (k <-> plist[k]) into (row <- source row)
    // for rows 0 .. w-1 and each target below them; the source of a row is
    // found by undoing the swaps from the last back
    if (t < 2 * w) {
        int d = t;
        if (t >= w) {
            d = S.plist[t - w];
            if (d < w) d = -1;   // already an entry
        }
        const int x = d >= 0 ? undo_swaps(S.plist, w, d) : d;
        edst[t] = d;
        esrc[t] = x;
    }
#pragma unroll
    for (int q = 0; q < G; ++q) {
        const int li = R::row(t, q);
        if (li < w) {
#pragma unroll
            for (int c = 0; c < W; ++c) Ls[li][c] = a[q][c];
        }
    }
    __syncthreads();
    const int ne = 2 * w, tot = ne * nco;   // <= 2 W x NB, a few per thread
    constexpr int kStageIters = (2 * W * NB + LT - 1) / LT;
    float sv[kStageIters];
#pragma unroll
    for (int j = 0; j < kStageIters; ++j) {
        const int idx = t + LT * j;
        const int e = idx / nco, cc = idx - e * nco;
        const bool in = idx < tot && edst[e < ne ? e : 0] >= 0;
        const int col = cc < ncl ? cc : cl + w + (cc - ncl);   // panel column
        sv[j] = P[in ? (size_t)col * ldp + r0 + esrc[e] : 0];
    }
#pragma unroll
    for (int j = 0; j < kStageIters; ++j) {
        const int idx = t + LT * j;
        const int e = idx / nco, cc = idx - e * nco;
        if (idx < tot) stage[e][cc] = sv[j];
    }
    __syncthreads();
    if (t < ncr) {
        const int cc = ncl + t;
        float x[W];
        if (w == W) {   // uniform; the usual case: no branch per row, so the
                        // LDS reads of all rows can be in flight together
#pragma unroll
            for (int i = 0; i < W; ++i) {
                float s = stage[i][cc];
#pragma unroll
                for (int l = 0; l < i; ++l) s = fmaf(-Ls[i][l], x[l], s);
                x[i] = s;
                stage[i][cc] = s;
            }
        } else {
#pragma unroll
            for (int i = 0; i < W; ++i) {
                if (i < w) {
                    float s = stage[i][cc];
#pragma unroll
                    for (int l = 0; l < i; ++l) s = fmaf(-Ls[i][l], x[l], s);
                    x[i] = s;
                    stage[i][cc] = s;
                }
            }
        }
    }
    __syncthreads();
    for (int idx = t; idx < ne * nco; idx += LT) {
        const int e = idx / nco, cc = idx - e * nco;
        if (edst[e] < 0) continue;
        const int col = cc < ncl ? cc : cl + w + (cc - ncl);
        P[(size_t)col * ldp + r0 + edst[e]] = stage[e][cc];
    }
}

// ---------------------------------------------------------------------------
// the panel's swaps (rows pj .. pe - 1, sequential) on the columns outside
// the panel; each workgroup composes them in LDS and moves a 32-column chunk
// ---------------------------------------------------------------------------

constexpr int kSwapCols = 32;

__global__ __launch_bounds__(256) void lu_swap_kernel(float* __restrict__ A, int n, int pj, int pe,
                                                      const uint32_t* __restrict__ piv, int oc0, int oc1) {
    __shared__ int pl[NB];              // the panel's swap targets, relative to pj
    __shared__ int edst[2 * NB], esrc[2 * NB];
    __shared__ float stage[2 * NB][kSwapCols + 1];
    const int t = threadIdx.x;
    const int nbk = pe - pj;
    if (t < nbk) pl[t] = (int)piv[pj + t] - pj;
    __syncthreads();
    // entries: rows pj .. pe - 1, then each swap target below the panel
    // (duplicates carry the same source); sources by undoing the swaps
    {
        const int e = t;   // 256 threads = 2 NB entries
        int d = -1;
        if (e < nbk) d = e;
        else if (e >= NB && e - NB < nbk && pl[e - NB] >= nbk) d = pl[e - NB];
        const int x = d >= 0 ? undo_swaps(pl, nbk, d) : d;
        edst[e] = d;
        esrc[e] = x;
    }
    __syncthreads();
    // columns outside the panel, numbered oc = 0 .. n - nbk - 1 left to
    // right; this launch moves oc0 .. oc1 - 1
    const int nout = oc1;
    const int c0 = oc0 + blockIdx.x * kSwapCols;
    // all loads first (clamped addresses), then the LDS writes
    constexpr int kIters = 2 * NB * kSwapCols / 256;
    float sv[kIters];
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        const int idx = t + 256 * j;
        const int e = idx / kSwapCols, cc = idx - e * kSwapCols;
        const int oc = c0 + cc;
        const bool in = oc < nout && edst[e] >= 0;
        const int col = oc < pj ? oc : oc + nbk;
        sv[j] = A[in ? (size_t)(pj + esrc[e]) * n + col : 0];
    }
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        const int idx = t + 256 * j;
        stage[idx / kSwapCols][idx % kSwapCols] = sv[j];
    }
    __syncthreads();
    for (int idx = t; idx < 2 * NB * kSwapCols; idx += 256) {
        const int e = idx / kSwapCols, cc = idx - e * kSwapCols;
        const int oc = c0 + cc;
        if (oc >= nout || edst[e] < 0) continue;
        const int col = oc < pj ? oc : oc + nbk;
        A[(size_t)(pj + edst[e]) * n + col] = stage[e][cc];
    }
}

// ---------------------------------------------------------------------------
// T X = B for one diagonal block T (nbk <= 128 rows; lower or upper part
// read, the diagonal not read when UNIT), B nbk x ncols in place; a
// workgroup takes 64 columns.  Per 16-row step: 64 threads substitute down
// (or up) the 16 x 16 diagonal sub-block, one column each; then all 256
// threads remove the step's rows from the rest.  Division by the diagonal,
// as BLAS strsm.
// ---------------------------------------------------------------------------

constexpr int kTrsmCols = 64;

template <bool UPPER, bool UNIT>
__global__ __launch_bounds__(256) void trsm_block_kernel(const float* __restrict__ T, int ldt,
                                                         float* __restrict__ B, int ldb, int nbk, int ncols) {
    __shared__ float Ts[NB][NB + 4];
    __shared__ float Bs[NB][kTrsmCols + 1];
    const int t = threadIdx.x;
    const int c0 = blockIdx.x * kTrsmCols;
    const int nsb = (nbk + 15) >> 4, np = nsb * 16;
    // T's triangle and the B tile: loads issued in batches of 16 from
    // clamped addresses, so that they overlap instead of waiting one by one
    for (int base = 0; base < NB * NB; base += 16 * 256) {
        float tv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = base + t + 256 * j, i = idx >> 7, l = idx & (NB - 1);
            const bool in = i < nbk && l < nbk && (UPPER ? l >= i : l <= i) && !(UNIT && l == i);
            tv[j] = T[in ? (size_t)i * ldt + l : 0];
            tv[j] = in ? tv[j] : ((l == i && (UNIT || i >= nbk)) ? 1.0f : 0.0f);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = base + t + 256 * j;
            Ts[idx >> 7][idx & (NB - 1)] = tv[j];
        }
    }
    {
        float bv[NB * kTrsmCols / 256];
#pragma unroll
        for (int j = 0; j < NB * kTrsmCols / 256; ++j) {
            const int idx = t + 256 * j, i = idx / kTrsmCols, c = idx % kTrsmCols;
            const bool in = i < nbk && c0 + c < ncols;
            bv[j] = B[in ? (size_t)i * ldb + c0 + c : 0];
            bv[j] = in ? bv[j] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < NB * kTrsmCols / 256; ++j) {
            const int idx = t + 256 * j;
            Bs[idx / kTrsmCols][idx % kTrsmCols] = bv[j];
        }
    }
    __syncthreads();
    for (int s = 0; s < nsb; ++s) {
        const int sb = UPPER ? nsb - 1 - s : s;
        const int i0 = 16 * sb;
        if (t < kTrsmCols) {
            float x[16];
            if (!UPPER) {
#pragma unroll
                for (int ii = 0; ii < 16; ++ii) {
                    float v = Bs[i0 + ii][t];
#pragma unroll
                    for (int l = 0; l < ii; ++l) v = fmaf(-Ts[i0 + ii][i0 + l], x[l], v);
                    x[ii] = UNIT ? v : v / Ts[i0 + ii][i0 + ii];
                    Bs[i0 + ii][t] = x[ii];
                }
            } else {
#pragma unroll
                for (int ii = 15; ii >= 0; --ii) {
                    float v = Bs[i0 + ii][t];
#pragma unroll
                    for (int l = ii + 1; l < 16; ++l) v = fmaf(-Ts[i0 + ii][i0 + l], x[l], v);
                    x[ii] = UNIT ? v : v / Ts[i0 + ii][i0 + ii];
                    Bs[i0 + ii][t] = x[ii];
                }
            }
        }
        __syncthreads();
        const int c = t & (kTrsmCols - 1), rg = t >> 6;
        float xb[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) xb[l] = Bs[i0 + l][c];
        const int r_begin = UPPER ? 0 : i0 + 16;
        const int r_end = UPPER ? i0 : np;
        for (int i = r_begin + rg; i < r_end; i += 4) {
            float v = Bs[i][c];
#pragma unroll
            for (int l = 0; l < 16; l += 4) {
                const float4 tv = *reinterpret_cast<const float4*>(&Ts[i][i0 + l]);
                v = fmaf(-tv.x, xb[l], v);
                v = fmaf(-tv.y, xb[l + 1], v);
                v = fmaf(-tv.z, xb[l + 2], v);
                v = fmaf(-tv.w, xb[l + 3], v);
            }
            Bs[i][c] = v;
        }
        __syncthreads();
    }
    for (int idx = t; idx < nbk * kTrsmCols; idx += 256) {
        const int i = idx / kTrsmCols, c = idx - i * kTrsmCols;
        if (c0 + c < ncols) B[(size_t)i * ldb + c0 + c] = Bs[i][c];
    }
}

// The panel's later columns after a leaf, on the transposed panel:
//   C'[c][r] -= sum_k U'[c][k] L'[k][r]   (c < ncol, r < mrest, k < w <= 16)
// (C' = columns right of the leaf, rows below it; U' = the leaf's U rows,
// transposed; L' = the leaf's multipliers, transposed).  A rank-w update
// this thin is bound by moving C', not by arithmetic: one thread per row r
// and 16 columns, coalesced along r, instead of matrix-core tiles.
constexpr int kUpdCols = 16;

__global__ __launch_bounds__(256) void panel_update_kernel(float* __restrict__ C, const float* __restrict__ U,
                                                           const float* __restrict__ L, int ldp, int ncol, int mrest,
                                                           int w) {
    __shared__ float us[kUpdCols][16];
    const int t = threadIdx.x;
    const int c0 = blockIdx.y * kUpdCols;
    {
        const int c = t >> 4, k = t & 15;
        us[c][k] = (c0 + c < ncol && k < w) ? U[(size_t)(c0 + c) * ldp + k] : 0.0f;
    }
    const int r = blockIdx.x * 256 + t;
    const int rr = r < mrest ? r : 0;   // clamped: every load is issued unconditionally
    float l[16], cv[kUpdCols];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        l[k] = L[(size_t)(k < w ? k : 0) * ldp + rr];
        l[k] = k < w ? l[k] : 0.0f;
    }
#pragma unroll
    for (int c = 0; c < kUpdCols; ++c) cv[c] = C[(size_t)(c0 + c < ncol ? c0 + c : 0) * ldp + rr];
    __syncthreads();
    if (r >= mrest) return;
#pragma unroll
    for (int c = 0; c < kUpdCols; ++c) {
        float acc = cv[c];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(-us[c][k], l[k], acc);
        if (c0 + c < ncol) C[(size_t)(c0 + c) * ldp + r] = acc;
    }
}

// dst (cols x rows, row stride ldd) = src^T (src rows x cols, row stride lds),
// through 32 x 32 LDS tiles
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

// x[i][:] = b[perm[i]][:]; all NaN where the matrix is singular
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ b, float* __restrict__ x,
                                                          const int* __restrict__ perm, int n, int ncols) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * ncols) return;
    const int i = (int)(idx / ncols), c = (int)(idx - (size_t)i * ncols);
    x[idx] = b[(size_t)perm[i] * ncols + c];
}

__global__ __launch_bounds__(256) void nan_if_singular_kernel(float* __restrict__ x, size_t count,
                                                              const uint32_t* __restrict__ info) {
    if (*info == 0) return;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) x[i] = qnan();
}

// x = P I: row i is e_{perm[i]}
__global__ __launch_bounds__(256) void perm_identity_kernel(float* __restrict__ x, const int* __restrict__ perm,
                                                            int n) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (size_t)i * n);
    x[idx] = j == perm[i] ? 1.0f : 0.0f;
}

__global__ void zero_info_kernel(uint32_t* p) { *p = 0; }

template <int RPT, int W>
void launch_leaf(float* A, int n, int pc, int pj, int pe, int w, uint32_t* piv, uint32_t* info, hipStream_t s) {
    hipLaunchKernelGGL((lu_leaf_kernel<RPT, W>), dim3(1), dim3(LT), 0, s, A, n, pc, pj, pe, w, piv, info);
}

// the leaf shape for the rows it holds (pc .. n - 1): rows per thread and
// width; later leaves hold fewer rows and get fewer rows per thread
void leaf(float* A, int n, int pc, int pj, int pe, uint32_t* piv, uint32_t* info, hipStream_t s, int& width) {
    const int m = n - pc;
    if (m <= LT) {
        width = 16;
        launch_leaf<1, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (m <= 2 * LT) {
        width = 16;
        launch_leaf<2, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (m <= 4 * LT) {
        width = 16;
        launch_leaf<4, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (m <= 8 * LT) {
        width = 16;
        launch_leaf<8, 16>(A, n, pc, pj, pe, std::min(16, pe - pc), piv, info, s);
    } else if (m <= 16 * LT) {
        width = 8;
        launch_leaf<16, 8>(A, n, pc, pj, pe, std::min(8, pe - pc), piv, info, s);
    } else {
        width = 4;
        launch_leaf<32, 4>(A, n, pc, pj, pe, std::min(4, pe - pc), piv, info, s);
    }
}

}  // namespace

bool lu_blocked_fits(uint32_t n) { return n <= kMaxBlockedN; }

// One n x n matrix: lu (in place over a copy of A), pivots, info; P = a
// 128 x n panel buffer.
void lu_blocked_one(float* lu, uint32_t* piv, uint32_t* info, float* P, int n, hipStream_t s) {
    hipLaunchKernelGGL(zero_info_kernel, dim3(1), dim3(1), 0, s, info);
    for (int pj = 0; pj < n; pj += NB) {
        const int pe = std::min(pj + NB, n), nbk = pe - pj, ldp = n - pj;
        float* panel = lu + (size_t)pj * n + pj;
        transpose(panel, n, P, ldp, ldp, nbk, s);
        {
            KernelTimer tm("lu_panel", s);
            for (int pc = pj; pc < pe;) {
                int width = 0;
                leaf(P, n, pc, pj, pe, piv, info, s, width);
                const int w = std::min(width, pe - pc);
                const int mrest = n - pc - w, ncol = pe - pc - w, cl = pc - pj;
                // the panel's later columns: C^T -= U^T L^T on the transposed panel
                if (mrest > 0 && ncol > 0)
                    hipLaunchKernelGGL(panel_update_kernel, dim3((unsigned)cdiv(mrest, 256), (unsigned)cdiv(ncol, kUpdCols)),
                                       dim3(256), 0, s, P + (size_t)(cl + w) * ldp + cl + w, P + (size_t)(cl + w) * ldp + cl,
                                       P + (size_t)cl * ldp + cl + w, ldp, ncol, mrest, w);
                pc += w;
            }
            tm.stop();
        }
        transpose(P, ldp, panel, n, nbk, ldp, s);
        const int nout = n - nbk;
        if (nout > 0)
            hipLaunchKernelGGL(lu_swap_kernel, dim3((unsigned)cdiv(nout, kSwapCols)), dim3(256), 0, s, lu, n, pj, pe,
                               piv, 0, nout);
        if (pe < n) {
            const int nc = n - pe;
            hipLaunchKernelGGL((trsm_block_kernel<false, true>), dim3((unsigned)cdiv(nc, kTrsmCols)), dim3(256), 0, s,
                               lu + (size_t)pj * n + pj, n, lu + (size_t)pj * n + pe, n, nbk, nc);
            sgemm(false, false, nc, nc, nbk, -1.0f, lu + (size_t)pe * n + pj, n, 0, lu + (size_t)pj * n + pe, n, 0,
                  1.0f, lu + (size_t)pe * n + pe, n, 0, 1, s);
        }
    }
    MLA_HIP(hipGetLastError());
}

// The row permutation of the whole factorization (perm[i] = the source row
// of row i of P A), from the 0-based sequential swaps: one workgroup.
namespace {
__global__ __launch_bounds__(256) void compose_perm_kernel(const uint32_t* __restrict__ piv, int n,
                                                           int* __restrict__ perm) {
    __shared__ int src[kMaxBlockedN];
    __shared__ int pl[NB];
    const int t = threadIdx.x;
    for (int i = t; i < n; i += 256) src[i] = i;
    // panel by panel: the panel's swaps composed (as in lu_swap_kernel),
    // then applied to the running permutation in one gather
    for (int pj = 0; pj < n; pj += NB) {
        const int nbk = min(NB, n - pj);
        __syncthreads();
        if (t < nbk) pl[t] = (int)piv[pj + t] - pj;
        __syncthreads();
        int d = -1;
        if (t < nbk) d = t;
        else if (t >= NB && t - NB < nbk && pl[t - NB] >= nbk) d = pl[t - NB];
        const int x = d >= 0 ? undo_swaps(pl, nbk, d) : d;
        const int v = d >= 0 ? src[pj + x] : 0;
        __syncthreads();
        if (d >= 0) src[pj + d] = v;
    }
    __syncthreads();
    for (int i = t; i < n; i += 256) perm[i] = src[i];
}
}  // namespace

// Triangular solve, one n x n matrix T (row stride ldt) and B (n x nrhs) in
// place: blocks of 128 rows, the diagonal block by trsm_block, the rest of
// the rows by the MFMA GEMM (reads only T's own triangle).
void trsm_blocked_one(const float* T, int ldt, float* B, int n, int nrhs, bool upper, bool unit, hipStream_t s) {
    const unsigned gx = (unsigned)cdiv(nrhs, kTrsmCols);
    KernelTimer tm("trsm_blocked", s);
    if (!upper) {
        for (int b0 = 0; b0 < n; b0 += NB) {
            const int nbk = std::min(NB, n - b0);
            if (unit)
                hipLaunchKernelGGL((trsm_block_kernel<false, true>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            else
                hipLaunchKernelGGL((trsm_block_kernel<false, false>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            const int below = n - b0 - nbk;
            if (below > 0)
                sgemm(false, false, below, nrhs, nbk, -1.0f, T + (size_t)(b0 + nbk) * ldt + b0, ldt, 0,
                      B + (size_t)b0 * nrhs, nrhs, 0, 1.0f, B + (size_t)(b0 + nbk) * nrhs, nrhs, 0, 1, s);
        }
    } else {
        const int nblk = cdiv(n, NB);
        for (int bi = nblk - 1; bi >= 0; --bi) {
            const int b0 = bi * NB, nbk = std::min(NB, n - b0);
            if (unit)
                hipLaunchKernelGGL((trsm_block_kernel<true, true>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            else
                hipLaunchKernelGGL((trsm_block_kernel<true, false>), dim3(gx), dim3(256), 0, s,
                                   T + (size_t)b0 * ldt + b0, ldt, B + (size_t)b0 * nrhs, nrhs, nbk, nrhs);
            if (b0 > 0)
                sgemm(false, false, b0, nrhs, nbk, -1.0f, T + b0, ldt, 0, B + (size_t)b0 * nrhs, nrhs, 0, 1.0f, B,
                      nrhs, 0, 1, s);
        }
    }
    tm.stop();
    MLA_HIP(hipGetLastError());
}

size_t lu_panel_workspace(uint32_t n) { return (size_t)NB * n * sizeof(float); }

size_t lu_blocked_workspace(uint32_t n) {
    // factor (n x n), pivots (n), permutation (n), padding, panel buffer
    return ((size_t)n * n + 2 * (size_t)n + 64) * sizeof(float) + lu_panel_workspace(n);
}

void lu_blocked_factor(const float* a, float* lu, uint32_t* pivots, uint32_t* info, float* work, uint32_t batch,
                       uint32_t n, hipStream_t s) {
    const size_t per = (size_t)n * n;
    MLA_HIP(hipMemcpyAsync(lu, a, batch * per * sizeof(float), hipMemcpyDeviceToDevice, s));
    for (uint32_t b = 0; b < batch; ++b)
        lu_blocked_one(lu + b * per, pivots + (size_t)b * n, info + b, work, (int)n, s);
}

// X = A^-1 B through the factorization: P A = L U, X = U^-1 L^-1 P B;
// all NaN where info > 0.  b == nullptr: B = I (the inverse).
void lu_blocked_solve(const float* a, const float* b, uint32_t nrhs, float* x, uint32_t* info, float* work,
                      uint32_t batch, uint32_t n, hipStream_t s) {
    const size_t per = (size_t)n * n;
    float* lu = work;
    uint32_t* piv = reinterpret_cast<uint32_t*>(work + per);
    int* perm = reinterpret_cast<int*>(work + per + n);
    float* P = work + per + 2 * (size_t)n + 64;
    for (uint32_t bi = 0; bi < batch; ++bi) {
        MLA_HIP(hipMemcpyAsync(lu, a + bi * per, per * sizeof(float), hipMemcpyDeviceToDevice, s));
        uint32_t* inf = info + bi;
        lu_blocked_one(lu, piv, inf, P, (int)n, s);
        hipLaunchKernelGGL(compose_perm_kernel, dim3(1), dim3(256), 0, s, piv, (int)n, perm);
        float* xb = x + (size_t)bi * n * nrhs;
        const size_t cnt = (size_t)n * nrhs;
        if (b) {
            hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)cdiv(cnt, 256)), dim3(256), 0, s,
                               b + (size_t)bi * n * nrhs, xb, perm, (int)n, (int)nrhs);
        } else {
            hipLaunchKernelGGL(perm_identity_kernel, dim3((unsigned)cdiv(cnt, 256)), dim3(256), 0, s, xb, perm,
                               (int)n);
        }
        trsm_blocked_one(lu, (int)n, xb, (int)n, (int)nrhs, false, true, s);
        trsm_blocked_one(lu, (int)n, xb, (int)n, (int)nrhs, true, false, s);
        hipLaunchKernelGGL(nan_if_singular_kernel, dim3(256), dim3(256), 0, s, xb, cnt, inf);
    }
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
