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
//   chol_diag    one workgroup: the nb x nb diagonal block in LDS, factored,
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

// One workgroup factors the nb x nb diagonal block (nb <= 128, padded to 128
// with the identity) in LDS and forms the inverse X = L^-1 of its factor, in
// four sub-panels of 32 columns (right-looking within the block):
//   1. wave 0 factors the 32 x 32 diagonal sub-block, lane r holding row r:
//      per column k the pivot and the scaled column are read across lanes
//      (readlane, so no LDS round trip or barrier per column), and the same
//      column values drive, in lanes 32..63, the forward substitution that
//      builds the sub-block's inverse Y (lane 32 + c holding column c);
//   2. the rows below, within the block: L = A Y^T (all threads);
//   3. the trailing lower triangle of the block: A -= L L^T (4 x 4 tiles);
// then the off-diagonal 32 x 32 blocks of X, by block forward substitution:
// X_ip = -Y_i sum_{k=p}^{i-1} L_ik X_kp, in rounds of i - p = 1, 2, 3.
// Barriers: a handful per sub-panel instead of one per column.
//
// The first pivot that is not positive and finite sets info = j0 + k + 1
// (unless an earlier block already set it); the factorisation carries on with
// NaN, which the final extract turns into the all-NaN output.
constexpr int SB = 32;           // sub-panel width
constexpr int DT = 256;          // threads of the diagonal-block kernel
constexpr int LDA = NB + 4;      // LDS row stride: rows 16-byte aligned

struct DiagLds {
    float A[NB][LDA];            // the block, then its factor L (lower)
    float X[NB][LDA];            // X = L^-1 (lower), zero above
    float S[3][SB][SB + 4];      // block products of one round
    int fail;
};

// acc (4 x 4) += P[r0 .. r0+3][0 .. 31] Q[0 .. 31][c0 .. c0+3]: P and Q are
// 32 x 32 blocks with row strides ldp and ldq.
__device__ __forceinline__ void tile_mm(float (&acc)[4][4], const float* P, int ldp, const float* Q, int ldq, int r0,
                                        int c0) {
#pragma unroll
    for (int q0 = 0; q0 < SB; q0 += 4) {
        float pr[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(P + (r0 + i) * ldp + q0);
            pr[i][0] = v.x;
            pr[i][1] = v.y;
            pr[i][2] = v.z;
            pr[i][3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 qv = *reinterpret_cast<const float4*>(Q + (q0 + q) * ldq + c0);
            const float qq[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(pr[i][q], qq[j], acc[i][j]);
        }
    }
}

__global__ __launch_bounds__(DT) void chol_diag_kernel(float* __restrict__ W, int ld, int j0, int nb,
                                                       float* __restrict__ Xout, uint32_t* __restrict__ info) {
    __shared__ DiagLds D;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // the lower triangle, padded with the identity.  Thread t takes column
    // c = t % 128 of rows t / 128 + 2 i; every load is issued unconditionally
    // from a clamped address (then masked), 16 in flight per batch.
    const int cc = t & (NB - 1), rb = t >> 7;
    const float* src = W + (size_t)j0 * ld + j0 + (cc < nb ? cc : nb - 1);
#pragma unroll
    for (int i0 = 0; i0 < NB / 2; i0 += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = rb + 2 * (i0 + i);
            v[i] = src[(size_t)(r < nb ? r : nb - 1) * ld];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = rb + 2 * (i0 + i);
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
        // 2. L[i][s0 ..] = A[i][s0 ..] Y^T for the rows below: thread -> (row,
        // 8 columns), at most two passes; results held over the barrier
        float out[2][8];
        int orow[2], ocol[2];
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const int idx = t + pass * DT;
            const int i = s0 + SB + (idx >> 2), cg = (idx & 3) * 8;
            orow[pass] = idx < mi * 4 ? i : -1;
            ocol[pass] = cg;
            const int ii = idx < mi * 4 ? i : s0 + SB;
            float ar[SB];
#pragma unroll
            for (int k0 = 0; k0 < SB; k0 += 4) {
                const float4 v = *reinterpret_cast<const float4*>(&D.A[ii][s0 + k0]);
                ar[k0] = v.x;
                ar[k0 + 1] = v.y;
                ar[k0 + 2] = v.z;
                ar[k0 + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float* yr = &D.X[s0 + cg + j][s0];
                float acc = 0.0f;
#pragma unroll
                for (int k0 = 0; k0 < SB; k0 += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(yr + k0);
                    acc = fmaf(ar[k0], v.x, acc);
                    acc = fmaf(ar[k0 + 1], v.y, acc);
                    acc = fmaf(ar[k0 + 2], v.z, acc);
                    acc = fmaf(ar[k0 + 3], v.w, acc);
                }
                out[pass][j] = acc;
            }
        }
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < 2; ++pass)
            if (orow[pass] >= 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) D.A[orow[pass]][s0 + ocol[pass] + j] = out[pass][j];
            }
        __syncthreads();
        // 3. the trailing lower triangle: A[i][c] -= sum_k L[i][k] L[c][k],
        // 4 x 4 tiles (tr >= tc) of the mi x mi block
        const int tn = mi / 4, ntiles = tn * (tn + 1) / 2;
        for (int idx = t; idx < ntiles; idx += DT) {
            int tr = (int)((sqrtf(8.0f * (float)idx + 1.0f) - 1.0f) * 0.5f);
            while ((tr + 1) * (tr + 2) / 2 <= idx) ++tr;
            while (tr * (tr + 1) / 2 > idx) --tr;
            const int tc = idx - tr * (tr + 1) / 2;
            const int i0 = s0 + SB + 4 * tr, c0 = s0 + SB + 4 * tc;
            float acc[4][4] = {};
#pragma unroll
            for (int k0 = 0; k0 < SB; k0 += 4) {
                float li[4][4], lc[4][4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 u = *reinterpret_cast<const float4*>(&D.A[i0 + q][s0 + k0]);
                    const float4 v = *reinterpret_cast<const float4*>(&D.A[c0 + q][s0 + k0]);
                    li[q][0] = u.x; li[q][1] = u.y; li[q][2] = u.z; li[q][3] = u.w;
                    lc[q][0] = v.x; lc[q][1] = v.y; lc[q][2] = v.z; lc[q][3] = v.w;
                }
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(li[i][kk], lc[j][kk], acc[i][j]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (c0 + j <= i0 + i) D.A[i0 + i][c0 + j] -= acc[i][j];
        }
        __syncthreads();
    }

    // X's off-diagonal blocks: round dd computes X_ip for i - p = dd
#pragma unroll
    for (int dd = 1; dd < NB / SB; ++dd) {
        const int nblk = NB / SB - dd;   // blocks this round (<= 3)
        // S_b = sum_{k=p}^{i-1} L_ik X_kp; thread -> one 4 x 4 tile of one block
        if (t < nblk * 64) {
            const int bidx = t >> 6, tile = t & 63;
            const int p = bidx, i = p + dd;
            const int r0 = (tile >> 3) * 4, c0 = (tile & 7) * 4;
            float acc[4][4] = {};
            for (int k = p; k < i; ++k)
                tile_mm(acc, &D.A[i * SB][k * SB], LDA, &D.X[k * SB][p * SB], LDA, r0, c0);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) D.S[bidx][r0 + q][c0 + j] = acc[q][j];
        }
        __syncthreads();
        // X_ip = -Y_i S_b
        if (t < nblk * 64) {
            const int bidx = t >> 6, tile = t & 63;
            const int p = bidx, i = p + dd;
            const int r0 = (tile >> 3) * 4, c0 = (tile & 7) * 4;
            float acc[4][4] = {};
            tile_mm(acc, &D.X[i * SB][i * SB], LDA, &D.S[bidx][0][0], SB + 4, r0, c0);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) D.X[i * SB + r0 + q][p * SB + c0 + j] = -acc[q][j];
        }
        __syncthreads();
    }

    // L (lower, diagonal included) back to W; X out (nb x nb)
    if (cc < nb) {
        float* dst = W + (size_t)j0 * ld + j0 + cc;
#pragma unroll 8
        for (int i = 0; i < NB / 2; ++i) {
            const int r = rb + 2 * i;
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
                hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(256), 0, s, W, nn, j, nb, xinv, inf);
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
