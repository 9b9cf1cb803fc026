// fp32 GEMM on the MI355X's matrix cores (v_mfma_f32_32x32x2f32), for the
// trailing-matrix updates of the blocked factorisations:
//
//     C = alpha * op(A) * op(B) + beta * C,   all row-major, strided batches
//
// op(A) is A (M x K, lda) or A^T (A stored K x M); op(B) is B (K x N) or B^T
// (B stored N x K).  Takes the place of the reference's MPS products
// (reference: src/band_reduce.mm:159-174, src/cholesky_gpu.mm:184-198,
// src/lu_gpu.mm:99-112).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of C; each of its
// four waves a 64 x 64 quarter as 2 x 2 blocks of 32 x 32 MFMA accumulators
// (16 floats per lane each).  K advances 16 at a time through LDS, double
// buffered: the next tile is loaded into registers while the current one
// feeds the matrix cores.  Both operands sit in LDS k-contiguous ([row][k],
// pitch 20 floats), and the K index of the 2-wide MFMA steps is permuted so
// that a lane's eight k values for one tile are contiguous: lanes 0-31
// supply k = 0..7 and lanes 32-63 k = 8..15 of the tile, read with two
// conflict-free ds_read_b128.  (A permutation of the summation index applied
// to both operands leaves the product unchanged.)
#include <new>
#include <stdexcept>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int LP = BK + 4;   // LDS pitch (floats): conflict-free b128 reads
// below this many 128 x 128 tiles per batch entry a K <= 128 product takes
// the 64 x 64 kernel
constexpr uint64_t kSmallTiles = 512;

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    int lda, ldb, ldc;
    long long sa, sb, sc;   // batch strides (floats)
    float alpha, beta;
    int lower;   // 1: only tiles that reach the lower triangle (row >= col) of C
    int K_last;  // K of the last batch entry (a split-K batch's shorter tail)
};

// Loads this thread's share of a 128 x 16 operand tile (rows r0.., k0..) into
// registers: 2048 floats = 256 threads x 8.  TRANS = the operand is stored
// k-major (element (row, k) at p[k * ld + row]): op(A) = A^T, and op(B) = B
// (whose tile rows are B's columns).  VEC: 16-byte aligned rows and a
// contiguous extent that is a multiple of 4, so a float4 is wholly inside
// or wholly outside.  Every load is issued unconditionally (outside the
// operand: from its first element, then masked to zero), so that no branch
// join forces a wait on the prefetch.
template <bool TRANS, bool VEC>
__device__ __forceinline__ void load_tile(const float* __restrict__ p, int ld, int rows, int K, int r0, int k0,
                                          float (&reg)[8]) {
    const int t = threadIdx.x;
    if (!TRANS) {
        // 4 consecutive threads cover 16 k of one row: 64 B contiguous
        const int kq = (t & 3) * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = r0 + (t >> 2) + h * 64;
            const int k = k0 + kq;
            if (VEC) {
                const bool in = r < rows && k < K;
                const floatx4 v = *reinterpret_cast<const floatx4*>(p + (in ? (size_t)r * ld + k : 0));
#pragma unroll
                for (int i = 0; i < 4; ++i) reg[h * 4 + i] = in ? v[i] : 0.0f;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool in = r < rows && k + i < K;
                    const float x = p[in ? (size_t)r * ld + k + i : 0];
                    reg[h * 4 + i] = in ? x : 0.0f;
                }
            }
        }
    } else {
        // stored [k][row]: thread t takes row t % 128 of the tile at k =
        // kb .. kb+3 and kb+8 .. kb+11 (kb = 4 (t / 128)).  Each load is a
        // wave's 64 consecutive rows of one k (coalesced), and the thread
        // ends with 4 consecutive k of one row: one conflict-free 16-byte
        // LDS store each (a row-strided store of single floats would hit
        // two banks only).
        const int rr = t & (BM - 1), kb = (t >> 7) * 4;
        const int r = r0 + rr;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = k0 + kb + h * 8 + i;
                const bool in = k < K && r < rows;
                const float x = p[in ? (size_t)k * ld + r : 0];
                reg[h * 4 + i] = in ? x : 0.0f;
            }
    }
}

// Registers of load_tile into the LDS tile s[row][k].
template <bool TRANS>
__device__ __forceinline__ void store_tile(float (*s)[LP], const float (&reg)[8]) {
    const int t = threadIdx.x;
    if (!TRANS) {
        const int kq = (t & 3) * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = (t >> 2) + h * 64;
            floatx4 v = {reg[h * 4 + 0], reg[h * 4 + 1], reg[h * 4 + 2], reg[h * 4 + 3]};
            *reinterpret_cast<floatx4*>(&s[r][kq]) = v;
        }
    } else {
        const int rr = t & (BM - 1), kb = (t >> 7) * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            floatx4 v = {reg[h * 4 + 0], reg[h * 4 + 1], reg[h * 4 + 2], reg[h * 4 + 3]};
            *reinterpret_cast<floatx4*>(&s[rr][kb + h * 8]) = v;
        }
    }
}

template <bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
    __shared__ float As[2][BM][LP];
    __shared__ float Bs[2][BN][LP];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    // Tile order: workgroups are dispatched round-robin over the eight XCDs,
    // each with its own L2, so consecutive workgroup ids go to different
    // XCDs.  Renumber so that each XCD takes a contiguous range of tiles,
    // and walk that range in bands of 8 tile rows (a band's tiles share A's
    // row panels and, band by band, B's column panels in that XCD's L2).
    int ty = blockIdx.y, tx = blockIdx.x;
    {
        const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
        const int bid = blockIdx.y * gx + blockIdx.x;
        const int lin = (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid;
        constexpr int GM = 8;
        const int in_group = GM * gx;
        const int first = (lin / in_group) * GM;
        const int gm = min(gy - first, GM);
        const int r = lin - (lin / in_group) * in_group;
        ty = first + r % gm;
        tx = r / gm;
    }
    const int m0 = ty * BM, n0 = tx * BN;
    if (g.lower && n0 >= m0 + BM) return;   // tile strictly above the diagonal (uniform)
    const size_t bz = blockIdx.z;
    const float* A = g.A + bz * g.sa;
    const float* B = g.B + bz * g.sb;
    float* C = g.C + bz * g.sc;
    const int K = blockIdx.z + 1 == gridDim.z ? g.K_last : g.K;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    float ra[8], rb[8];
    load_tile<TA, VEC>(A, g.lda, g.M, K, m0, 0, ra);
    load_tile<!TB, VEC>(B, g.ldb, g.N, K, n0, 0, rb);
    store_tile<TA>(As[0], ra);
    store_tile<!TB>(Bs[0], rb);
    __syncthreads();

    const int ktiles = (K + BK - 1) / BK;
    const int lr = lane & 31;         // row (A) / column (B) within a 32-block
    const int kh = (lane >> 5) * 8;   // this lane's 8 k values of the tile
    for (int kt = 0; kt < ktiles; ++kt) {
        const int cur = kt & 1;
        // the next tile (past the end: all masked, no branch)
        load_tile<TA, VEC>(A, g.lda, g.M, K, m0, (kt + 1) * BK, ra);
        load_tile<!TB, VEC>(B, g.ldb, g.N, K, n0, (kt + 1) * BK, rb);
        floatx4 a0[2][2], b0[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a0[i][0] = *reinterpret_cast<const floatx4*>(&As[cur][wm + i * 32 + lr][kh]);
            a0[i][1] = *reinterpret_cast<const floatx4*>(&As[cur][wm + i * 32 + lr][kh + 4]);
            b0[i][0] = *reinterpret_cast<const floatx4*>(&Bs[cur][wn + i * 32 + lr][kh]);
            b0[i][1] = *reinterpret_cast<const floatx4*>(&Bs[cur][wn + i * 32 + lr][kh + 4]);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[i][s >> 2][s & 3], b0[j][s >> 2][s & 3],
                                                                     acc[i][j], 0, 0, 0);
        }
        store_tile<TA>(As[cur ^ 1], ra);   // (after the last tile: zeros, never read)
        store_tile<!TB>(Bs[cur ^ 1], rb);
        __syncthreads();
    }

    // epilogue: lane holds column (lane & 31) of each 32 x 32 block, rows
    // 8 * (e / 4) + 4 * (lane / 32) + (e % 4).  Per block, the 16 loads of C
    // (clamped addresses) are all issued before the first use, so that their
    // latencies overlap instead of adding up.
    const bool keep = g.beta != 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + j * 32 + lr;
            const bool cin = col < g.N;
            float cv[16];
            if (keep) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                    const bool in = cin && row < g.M;
                    cv[e] = C[in ? (size_t)row * g.ldc + col : 0];
                }
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (cin && row < g.M) {
                    const float v = g.alpha * acc[i][j][e];
                    C[(size_t)row * g.ldc + col] = keep ? fmaf(g.beta, cv[e], v) : v;
                }
            }
        }
}

// Small-K products (K <= 128: the rank-nb trailing updates and TRSMs of the
// blocked factorisations), where the 128 x 128 kernel's K loop is a chain of
// global-load latencies and its tiles too few to fill the chip.  A
// 256-thread workgroup computes a TM x TN tile of C (64 x 64, or 32 x 128
// for an in-place product with N <= 128), a wave per 32 x 32 MFMA block; the whole
// K extent of both operands is loaded at once (every load in flight
// together) into LDS, [row][k] with pitch KP, then fed to the matrix cores
// with the same permuted-k reads as above.  With a tile as wide as N, a
// workgroup has read its rows of A whole before it writes C, so C may be A
// itself (an in-place product).
constexpr int SM = 64, SK = 128, KP = SK + 4;

template <bool TRANS, bool VEC, int ROWS>
__device__ __forceinline__ void load_panel(const float* __restrict__ p, int ld, int rows, int K, int r0,
                                           float (*s)[KP]) {
    constexpr int IT = ROWS / 8;   // float4 per thread: ROWS x 128 floats over 256 threads
    static_assert(IT >= 1 && ROWS % 32 == 0, "panel rows");
    const int t = threadIdx.x;
    float v[IT][4];
    if (!TRANS) {
        // 32 float4 per row (k = 4q): thread t takes (row, q) = (idx / 32, idx % 32)
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int idx = t + 256 * i, r = r0 + (idx >> 5), k = (idx & 31) * 4;
            if (VEC) {
                const bool in = r < rows && k < K;
                const floatx4 x = *reinterpret_cast<const floatx4*>(p + (in ? (size_t)r * ld + k : 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = in ? x[e] : 0.0f;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool in = r < rows && k + e < K;
                    const float x = p[in ? (size_t)r * ld + k + e : 0];
                    v[i][e] = in ? x : 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int idx = t + 256 * i;
            floatx4 x = {v[i][0], v[i][1], v[i][2], v[i][3]};
            *reinterpret_cast<floatx4*>(&s[idx >> 5][(idx & 31) * 4]) = x;
        }
    } else {
        // stored [k][row]: thread t takes rows 4q .. 4q+3 of one k, (k, q) =
        // (idx / (ROWS / 4), idx % (ROWS / 4)): consecutive threads read
        // consecutive rows of one k
        constexpr int QR = ROWS / 4;
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int idx = t + 256 * i, k = idx / QR, r = r0 + (idx % QR) * 4;
            if (VEC) {
                const bool in = k < K && r < rows;
                const floatx4 x = *reinterpret_cast<const floatx4*>(p + (in ? (size_t)k * ld + r : 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = in ? x[e] : 0.0f;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool in = k < K && r + e < rows;
                    const float x = p[in ? (size_t)k * ld + r + e : 0];
                    v[i][e] = in ? x : 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int idx = t + 256 * i, k = idx / QR, rq = (idx % QR) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) s[rq + e][k] = v[i][e];
        }
    }
}

template <bool TA, bool TB, bool VEC, int TM, int TN>
__global__ __launch_bounds__(256) void gemm_k128_kernel(GemmArgs g) {
    constexpr int WM = TM / 32, WN = 4 / WM;   // the four waves as WM x WN
    constexpr int NBW = TN / WN / 32;          // 32 x 32 blocks per wave along N
    static_assert(NBW >= 1 && WM * WN == 4, "tile shape");
    __shared__ float As[TM][KP];
    __shared__ float Bs[TN][KP];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = (wave % WM) * 32, wn = (wave / WM) * (TN / WN);
    const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    if (g.lower && n0 >= m0 + TM) return;   // tile strictly above the diagonal (uniform)
    const size_t bz = blockIdx.z;
    const float* A = g.A + bz * g.sa;
    const float* B = g.B + bz * g.sb;
    float* C = g.C + bz * g.sc;
    const int K = blockIdx.z + 1 == gridDim.z ? g.K_last : g.K;

    load_panel<TA, VEC, TM>(A, g.lda, g.M, K, m0, As);
    load_panel<!TB, VEC, TN>(B, g.ldb, g.N, K, n0, Bs);
    __syncthreads();

    floatx16 acc[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    const int lr = lane & 31;
    const int kh = (lane >> 5) * 8;
    const int ktiles = (K + 15) / 16;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int kb = kt * 16 + kh;
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(&As[wm + lr][kb]);
        const floatx4 a1 = *reinterpret_cast<const floatx4*>(&As[wm + lr][kb + 4]);
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
            const floatx4 b0 = *reinterpret_cast<const floatx4*>(&Bs[wn + 32 * j + lr][kb]);
            const floatx4 b1 = *reinterpret_cast<const floatx4*>(&Bs[wn + 32 * j + lr][kb + 4]);
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b0[s], acc[j], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s], b1[s], acc[j], 0, 0, 0);
        }
    }

    const bool keep = g.beta != 0.0f;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const int col = n0 + wn + 32 * j + lr;
        const bool cin = col < g.N;
        float cv[16];
        if (keep) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                const bool in = cin && row < g.M;
                cv[e] = C[in ? (size_t)row * g.ldc + col : 0];
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (cin && row < g.M) {
                const float v = g.alpha * acc[j][e];
                C[(size_t)row * g.ldc + col] = keep ? fmaf(g.beta, cv[e], v) : v;
            }
        }
    }
}

// Whether two strided row-major blocks (rows x cols, leading dimension ld,
// `nb` of them `stride` floats apart) share an element.  With one block each
// and equal leading dimensions the test is exact (two rectangles of the same
// row grid, the second's columns possibly wrapping into the next row), so
// that neighbouring blocks of one matrix (a panel and its trailing block)
// are told apart; otherwise the address ranges are compared.
bool blocks_overlap(const float* p, long long rows, long long cols, int ld, long long stride, const float* q,
                    long long qrows, long long qcols, int qld, long long qstride, int nb) {
    if (rows <= 0 || cols <= 0 || qrows <= 0 || qcols <= 0) return false;
    if (nb == 1 && ld == qld && cols <= ld && qcols <= ld) {
        const long long d = (long long)(q - p);   // q's first element on p's grid
        long long dr = d / ld, dc = d % ld;
        if (dc < 0) {
            dc += ld;
            --dr;
        }
        auto hit = [&](long long r0, long long r1, long long c0, long long c1) {   // [r0, r1) x [c0, c1)
            return r0 < rows && 0 < r1 && c0 < cols && 0 < c1;
        };
        if (dc + qcols <= ld) return hit(dr, dr + qrows, dc, dc + qcols);
        return hit(dr, dr + qrows, dc, ld) || hit(dr + 1, dr + qrows + 1, 0, dc + qcols - ld);
    }
    const uintptr_t p0 = (uintptr_t)p, q0 = (uintptr_t)q;
    const uintptr_t p1 = (uintptr_t)(p + (nb - 1) * stride + (rows - 1) * ld + cols);
    const uintptr_t q1 = (uintptr_t)(q + (nb - 1) * qstride + (qrows - 1) * qld + qcols);
    return p0 < q1 && q0 < p1;
}

}  // namespace

void sgemm(bool ta, bool tb, int M, int N, int K, float alpha, const float* A, int lda, long long sa,
           const float* B, int ldb, long long sb, float beta, float* C, int ldc, long long sc, int batch,
           hipStream_t s, bool lower_only, int k_last) {
    if (M <= 0 || N <= 0 || batch <= 0) return;
    GemmArgs g{A, B, C, M, N, K, lda, ldb, ldc, sa, sb, sc, alpha, beta, lower_only ? 1 : 0,
               k_last >= 0 ? k_last : K};
    const dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, BM), (unsigned)batch);
    KernelTimer t("gemm_mfma", s);
    // K <= 128 with fewer than kSmallTiles 128 x 128 tiles per entry: the 64 x 64
    // whole-K kernel (four times the workgroups, one load latency) -- unless
    // C overlaps an operand (an in-place product such as the blocked
    // Cholesky's L21 = A21 X^T): its 64-column tiles would let one
    // workgroup overwrite rows of A that another still reads, whereas a
    // single 128-column tile reads its rows whole before writing them
    auto over_a_or_b = [&](const float* p, long long rows, long long cols, int ld, long long stride) {
        return blocks_overlap(p, rows, cols, ld, stride, C, M, N, ldc, sc, batch);
    };
    const bool over_a = over_a_or_b(A, ta ? K : M, ta ? M : K, lda, sa);
    const bool over_b = over_a_or_b(B, tb ? N : K, tb ? K : N, ldb, sb);
    // C = A itself, row for row, with N <= 128: tiles as wide as N (32 x
    // 128, or 64 x 64 for N <= 64) read each row of A whole before writing
    // it, and no other workgroup touches it
    const bool same_rows = over_a && !over_b && C == A && !ta && ldc == lda && sc == sa && N <= 128;
    const bool small = K <= SK && (!(over_a || over_b) || same_rows) && (uint64_t)grid.x * grid.y < kSmallTiles;
    const bool wide = same_rows && N > SM;   // the 32 x 128 tiles
    const int tm = wide ? 32 : SM, tn = wide ? 128 : SM;
    const dim3 sgrid((unsigned)cdiv(N, tn), (unsigned)cdiv(M, tm), (unsigned)batch);
    // float4 operand loads: 16-byte aligned bases, strides and leading
    // dimensions, and the contiguous extent of each operand a multiple of 4
    auto al = [](const void* p) { return (((uintptr_t)p) & 15) == 0; };
    const bool vec = al(A) && al(B) && (lda & 3) == 0 && (ldb & 3) == 0 && (sa & 3) == 0 && (sb & 3) == 0 &&
                     ((ta ? M : K) & 3) == 0 && ((tb ? K : N) & 3) == 0 && ((ta ? M : g.K_last) & 3) == 0 &&
                     ((tb ? g.K_last : N) & 3) == 0;
#define MLA_GEMM_LAUNCH(TA_, TB_)                                                                       \
    do {                                                                                                \
        if (small && wide && vec)                                                                       \
            hipLaunchKernelGGL((gemm_k128_kernel<TA_, TB_, true, 32, 128>), sgrid, dim3(256), 0, s, g); \
        else if (small && wide)                                                                         \
            hipLaunchKernelGGL((gemm_k128_kernel<TA_, TB_, false, 32, 128>), sgrid, dim3(256), 0, s, g);\
        else if (small && vec)                                                                          \
            hipLaunchKernelGGL((gemm_k128_kernel<TA_, TB_, true, 64, 64>), sgrid, dim3(256), 0, s, g);  \
        else if (small)                                                                                 \
            hipLaunchKernelGGL((gemm_k128_kernel<TA_, TB_, false, 64, 64>), sgrid, dim3(256), 0, s, g); \
        else if (vec) hipLaunchKernelGGL((gemm_kernel<TA_, TB_, true>), grid, dim3(256), 0, s, g);      \
        else hipLaunchKernelGGL((gemm_kernel<TA_, TB_, false>), grid, dim3(256), 0, s, g);              \
    } while (0)
    if (!ta && !tb) MLA_GEMM_LAUNCH(false, false);
    else if (!ta && tb) MLA_GEMM_LAUNCH(false, true);
    else if (ta && !tb) MLA_GEMM_LAUNCH(true, false);
    else MLA_GEMM_LAUNCH(true, true);
#undef MLA_GEMM_LAUNCH
    t.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla

// Test and measurement hook (include/metal_linalg/hip_ext.h): the MFMA GEMM
// on caller buffers (host or device), row-major, strided batches.
extern "C" int metal_linalg_hip_sgemm(int transa, int transb, int M, int N, int K, float alpha, const float* A,
                                      int lda, long long stride_a, const float* B, int ldb, long long stride_b,
                                      float beta, float* C, int ldc, long long stride_c, int batch) {
    try {
        if (M < 0 || N < 0 || K < 0 || batch < 0) return 1;
        if (!M || !N || !batch) return 0;
        mla::Call call;
        const long long ra = transa ? K : M, ca = transa ? M : K;
        const long long rb = transb ? N : K, cb = transb ? K : N;
        const size_t na = (size_t)((batch - 1) * stride_a + (ra - 1) * lda + ca);
        const size_t nb = (size_t)((batch - 1) * stride_b + (rb - 1) * ldb + cb);
        const size_t nc = (size_t)((batch - 1) * stride_c + (long long)(M - 1) * ldc + N);
        const float* dA = K ? call.in(A, na) : nullptr;
        const float* dB = K ? call.in(B, nb) : nullptr;
        float* dC = call.out(C, nc);
        if (beta != 0.0f) {
            // C is also an input: a host C must be copied in first
            const float* cin = call.in(C, nc);
            if (cin != dC) MLA_HIP(hipMemcpyAsync(dC, cin, nc * sizeof(float), hipMemcpyDeviceToDevice, call.stream()));
        }
        mla::sgemm(transa != 0, transb != 0, M, N, K, alpha, dA, lda, stride_a, dB, ldb, stride_b, beta, dC, ldc,
                   stride_c, batch, call.stream());
        call.finish();
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    } catch (const std::bad_alloc&) {
        return 3;
    } catch (...) {
        return 2;
    }
}
