// Blocked Cholesky for large matrices (any n; the large-matrix regime, config
// 5's 4096 x 4096), right-looking in panels of 128 columns.
//
// Role: the MI355X counterpart of the reference's cholesky_blocked
// (reference: src/cholesky_gpu.mm:272-343, kernels shaders/Cholesky.metal:
// 170-208, 355-491, trailing update as MPS C -= A B^T in 512-column blocks,
// :184-198), with the CPU path's contract (src/cholesky_cpu.mm:93-151):
// only the requested triangle is read; info = k + 1 for the first pivot that
// is not positive and finite, and then the output is all NaN; the other
// triangle of the output is zero.
//
// Per panel j (columns j .. j+nb):
//   chol_diag    one 1024-thread workgroup: the nb x nb diagonal block in LDS, factored,
//                and its triangular inverse X = L11^-1 (forward substitution
//                on the identity, rows in parallel)
//   TRSM         L21 = A21 X^T as one MFMA GEMM, in place (one column tile
//                of 128, so each workgroup reads its rows before writing them)
//   SYRK         A22 -= L21 L21^T as an MFMA GEMM over the tiles that reach
//                the lower triangle
// The matrix is first copied (transposed for `upper`) into a working lower
// triangle, and written out at the end with the other triangle zeroed.
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NB = 128;

// dst (n x n) = src or src^T, through 32 x 32 LDS tiles (both sides coalesced).
__global__ __launch_bounds__(256) void copy_transpose_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                             int n, int trans) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
    if (!trans) {
        for (int r = ty; r < 32; r += 8) {
            const int i = by + r, jx = bx + tx;
            if (i < n && jx < n) dst[(size_t)i * n + jx] = src[(size_t)i * n + jx];
        }
        return;
    }
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, jx = bx + tx;
        if (i < n && jx < n) tile[r][tx] = src[(size_t)i * n + jx];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int i = bx + r, jx = by + tx;   // dst row i = src column
        if (i < n && jx < n) dst[(size_t)i * n + jx] = tile[tx][r];
    }
}

// One workgroup of 1024 threads factors the nb x nb diagonal block (nb <=
// 128, padded to 128 with the identity) in LDS and forms the inverse X = L^-1
// of its factor, in four sub-panels of 32 columns (right-looking within the
// block):
//   1. wave 0 factors the 32 x 32 diagonal sub-block, lane r holding row r:
//      per column k the pivot and the scaled column are read across lanes
//      (readlane, so no LDS round trip or barrier per column), and the same
//      column values drive, in lanes 32..63, the forward substitution that
//      builds the sub-block's inverse Y (lane 32 + c holding column c);
//   2. the rows below, within the block: L = A Y^T;
//   3. the trailing lower triangle of the block: A -= L L^T;
// then the off-diagonal 32 x 32 blocks of X, by block forward substitution:
// X_ip = -Y_i sum_{k=p}^{i-1} L_ik X_kp, in rounds of i - p = 1, 2, 3.  The
// products of 2, 3 and the rounds run on the matrix cores, a wave per 32 x 32
// block (4 x 4 VALU tiles read LDS with 4-way bank conflicts: the trailing
// update alone took 10 us); the load and store use all sixteen waves.
//
// The first pivot that is not positive and finite sets info = j0 + k + 1
// (unless an earlier block already set it); the factorisation carries on with
// NaN, which the final extract turns into the all-NaN output.
constexpr int SB = 32;           // sub-panel width
constexpr int DT = 1024;         // threads of the diagonal-block kernel
constexpr int LDA = NB + 4;      // LDS row stride: rows 16-byte aligned

struct DiagLds {
    float A[NB][LDA];            // the block, then its factor L (lower)
    float X[NB][LDA];            // X = L^-1 (lower), zero above
    float S[3][SB][SB + 4];      // block products of one round
    int fail;
};

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// acc (a 32 x 32 MFMA block: lane l holds column l % 32, rows 8 (e / 4) +
// 4 (l / 32) + e % 4) += P Q over K = 16 kt, P = rows of `prow` (32 rows,
// k contiguous, stride LDA) and Q given either as rows of `qcol` with k
// contiguous (QKM false: Q[k][c] = qcol[c LDA + k]) or k-major (QKM true:
// Q[k][c] = qcol[k ldq + c]).  As in the GEMM kernel, lanes 0-31 supply k
// = 0..7 and lanes 32-63 k = 8..15 of each 16-k step (16-byte P reads).
template <bool QKM>
__device__ __forceinline__ void mfma_block(floatx16& acc, const float* prow, const float* qcol, int ldq, int kt,
                                           int lane) {
    const int lr = lane & 31, kh = (lane >> 5) * 8;
    for (int t16 = 0; t16 < kt; ++t16) {
        const int k = t16 * 16 + kh;
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(prow + lr * LDA + k);
        const floatx4 a1 = *reinterpret_cast<const floatx4*>(prow + lr * LDA + k + 4);
        float b[8];
        if (QKM) {
#pragma unroll
            for (int s = 0; s < 8; ++s) b[s] = qcol[(k + s) * ldq + lr];
        } else {
            const floatx4 b0 = *reinterpret_cast<const floatx4*>(qcol + lr * LDA + k);
            const floatx4 b1 = *reinterpret_cast<const floatx4*>(qcol + lr * LDA + k + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                b[s] = b0[s];
                b[s + 4] = b1[s];
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b[s], acc, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s], b[s + 4], acc, 0, 0, 0);
    }
}

__device__ __forceinline__ int mfma_row(int e, int lane) { return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); }

__global__ __launch_bounds__(DT) void chol_diag_kernel(float* __restrict__ W, int ld, int j0, int nb,
                                                       float* __restrict__ Xout, uint32_t* __restrict__ info) {
    __shared__ DiagLds D;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // the lower triangle, padded with the identity.  Thread t takes column
    // c = t % 128 of rows t / 128 + 8 i; every load is issued unconditionally
    // from a clamped address (then masked), all 16 in flight together.
    const int cc = t & (NB - 1), rb = t >> 7;
    constexpr int RSTEP = DT / NB, RPT = NB / RSTEP;   // 8 rows apart, 16 per thread
    {
        const float* src = W + (size_t)j0 * ld + j0 + (cc < nb ? cc : nb - 1);
        float v[RPT];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int r = rb + RSTEP * i;
            v[i] = src[(size_t)(r < nb ? r : nb - 1) * ld];
        }
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int r = rb + RSTEP * i;
            const bool in = r < nb && cc < nb && cc <= r;
            D.A[r][cc] = in ? v[i] : (r == cc ? 1.0f : 0.0f);
            D.X[r][cc] = 0.0f;
        }
    }
    if (t == 0) D.fail = 0;
    __syncthreads();

    for (int s0 = 0; s0 < NB; s0 += SB) {
        // 1. the 32 x 32 diagonal sub-block and its inverse (wave 0).  Lane
        // r < 32 holds row r of the sub-block (becoming row r of L), lane
        // 32 + r column r of the identity (becoming column r of Y = L^-1):
        // both take the same update, z[c] -= z[k] L[c][k], with L[c][k] read
        // from lane c.
        if (wv == 0) {
            const int r = lane & (SB - 1);
            const bool lrow = lane < SB;
            float z[SB];
#pragma unroll
            for (int j = 0; j < SB; ++j) {
                const float av = D.A[s0 + r][s0 + j];
                z[j] = lrow ? (j <= r ? av : 0.0f) : (j == r ? 1.0f : 0.0f);
            }
            int failk = 0;
#pragma unroll
            for (int k = 0; k < SB; ++k) {
                const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(z[k]), k));
                if (failk == 0 && !(d > 0.0f && d <= FLT_MAX)) failk = k + 1;
                // 1 / sqrt(d) by the hardware estimate and one Newton step
                // (the critical path of the column chain), sqrt(d) = d / sqrt(d)
                const float e0 = __builtin_amdgcn_rsqf(d);
                const float ik = e0 * fmaf(-0.5f * d * e0, e0, 1.5f);
                const float pk = d * ik;
                // L[r][k] = A[r][k] / L[k][k] (r > k), L[k][k]; Y[k][.] final
                z[k] = lrow && r == k ? pk : z[k] * ik;
#pragma unroll
                for (int c = k + 1; c < SB; ++c) {
                    const float lck = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(z[k]), c));
                    z[c] = fmaf(-z[k], lck, z[c]);
                }
            }
            if (lrow) {
#pragma unroll
                for (int j = 0; j < SB; ++j)
                    if (j <= r) D.A[s0 + r][s0 + j] = z[j];
            } else {
#pragma unroll
                for (int j = 0; j < SB; ++j) D.X[s0 + j][s0 + r] = z[j];   // Y[j][r], zero for j < r
            }
            if (lane == 0 && failk != 0 && D.fail == 0) D.fail = s0 + failk;
        }
        __syncthreads();
        const int mi = NB - s0 - SB;   // rows below the sub-block, within the block
        if (mi <= 0) break;
        // 2. L = A Y^T for the rows below, in place: wave w < mi / 32 takes
        // rows s0 + 32 (w + 1) .. + 31 (its reads of them all precede its
        // writes; no other wave touches them)
        const int nrt = mi / SB;
        if (wv < nrt) {
            const int r0 = s0 + SB * (wv + 1);
            floatx16 acc = {};
            mfma_block<false>(acc, &D.A[r0][s0], &D.X[s0][s0], LDA, SB / 16, lane);
#pragma unroll
            for (int e = 0; e < 16; ++e) D.A[r0 + mfma_row(e, lane)][s0 + (lane & 31)] = acc[e];
        }
        __syncthreads();
        // 3. the trailing lower triangle: A[i][c] -= sum_k L[i][k] L[c][k],
        // a wave per 32 x 32 tile (ti >= tj) of the mi x mi block
        if (wv < nrt * (nrt + 1) / 2) {
            int ti = 0, rem = wv;
            while (rem > ti) rem -= ++ti;
            const int tj = rem;
            const int r0 = s0 + SB * (ti + 1), c0 = s0 + SB * (tj + 1);
            floatx16 acc = {};
            mfma_block<false>(acc, &D.A[r0][s0], &D.A[c0][s0], LDA, SB / 16, lane);
            const int col = c0 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = r0 + mfma_row(e, lane);
                if (col <= row) D.A[row][col] -= acc[e];
            }
        }
        __syncthreads();
    }

    // X's off-diagonal blocks: round dd computes X_ip for i - p = dd, a wave
    // per block: S = sum_{k=p}^{i-1} L_ik X_kp (one 32 dd long sum), then
    // X_ip = -Y_i S
#pragma unroll
    for (int dd = 1; dd < NB / SB; ++dd) {
        const int nblk = NB / SB - dd;   // blocks this round (<= 3)
        const int p = wv, i = p + dd;
        if (wv < nblk) {
            floatx16 acc = {};
            mfma_block<true>(acc, &D.A[i * SB][p * SB], &D.X[p * SB][p * SB], LDA, 2 * dd, lane);
#pragma unroll
            for (int e = 0; e < 16; ++e) D.S[wv][mfma_row(e, lane)][lane & 31] = acc[e];
        }
        __syncthreads();
        if (wv < nblk) {
            floatx16 acc = {};
            mfma_block<true>(acc, &D.X[i * SB][i * SB], &D.S[wv][0][0], SB + 4, SB / 16, lane);
#pragma unroll
            for (int e = 0; e < 16; ++e) D.X[i * SB + mfma_row(e, lane)][p * SB + (lane & 31)] = -acc[e];
        }
        __syncthreads();
    }

    // L (lower, diagonal included) back to W; X out (nb x nb)
    if (cc < nb) {
        float* dst = W + (size_t)j0 * ld + j0 + cc;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int r = rb + RSTEP * i;
            if (r < nb) {
                if (cc <= r) dst[(size_t)r * ld] = D.A[r][cc];
                Xout[(size_t)r * nb + cc] = D.X[r][cc];
            }
        }
    }
    if (t == 0 && D.fail != 0 && *info == 0) *info = (uint32_t)(j0 + D.fail);
}

// out = the working lower triangle (or its transpose for `upper`), the
// other triangle zero; all NaN when a pivot failed.
__global__ __launch_bounds__(256) void chol_extract_kernel(const float* __restrict__ W, float* __restrict__ out,
                                                           int n, int upper, const uint32_t* __restrict__ info) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const bool failed = *info != 0;
    if (!upper) {
        for (int r = ty; r < 32; r += 8) {
            const int i = by + r, c = bx + tx;
            if (i < n && c < n) out[(size_t)i * n + c] = failed ? qnan() : (c <= i ? W[(size_t)i * n + c] : 0.0f);
        }
        return;
    }
    // U[i][c] = L[c][i] for c >= i
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, c = bx + tx;   // source element L[i][c]
        if (i < n && c < n) tile[r][tx] = W[(size_t)i * n + c];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int i = bx + r, c = by + tx;   // out[i][c] = L[c][i]
        if (i < n && c < n) out[(size_t)i * n + c] = failed ? qnan() : (c >= i ? tile[tx][r] : 0.0f);
    }
}

__global__ void zero_u32_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

void chol_blocked(const float* a, float* l, uint32_t* info, float* work, float* xinv, uint32_t batch, uint32_t n,
                  bool upper, hipStream_t s) {
    const int nn = (int)n;
    const size_t per = (size_t)n * n;
    const dim3 tiles((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32));
    for (uint32_t b = 0; b < batch; ++b) {
        float* W = work;
        uint32_t* inf = info + b;
        hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, s, inf, 1);
        hipLaunchKernelGGL(copy_transpose_kernel, tiles, dim3(256), 0, s, a + b * per, W, nn, upper ? 1 : 0);
        for (int j = 0; j < nn; j += NB) {
            const int nb = nn - j < NB ? nn - j : NB;
            {
                KernelTimer t("chol_diag", s);
                hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(DT), 0, s, W, nn, j, nb, xinv, inf);
                t.stop();
            }
            const int m2 = nn - j - nb;
            if (m2 <= 0) break;
            float* A21 = W + (size_t)(j + nb) * n + j;
            float* A22 = W + (size_t)(j + nb) * n + j + nb;
            // L21 = A21 X^T (in place: one column tile)
            sgemm(false, true, m2, nb, nb, 1.0f, A21, nn, 0, xinv, nb, 0, 0.0f, A21, nn, 0, 1, s);
            // A22 -= L21 L21^T, lower tiles
            sgemm(false, true, m2, m2, nb, -1.0f, A21, nn, 0, A21, nn, 0, 1.0f, A22, nn, 0, 1, s, true);
        }
        hipLaunchKernelGGL(chol_extract_kernel, tiles, dim3(256), 0, s, W, l + b * per, nn, upper ? 1 : 0, inf);
    }
    MLA_HIP(hipGetLastError());
}

size_t chol_blocked_workspace(uint32_t n) { return ((size_t)n * n + (size_t)NB * NB) * sizeof(float); }

}  // namespace mla
