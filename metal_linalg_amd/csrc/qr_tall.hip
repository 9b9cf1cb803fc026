// Batched Householder QR of tall matrices with at most 64 columns and any
// number of rows: one block of up to 128 rows per wave, and beyond 128 rows a
// reduction tree of such block QRs.
//
// Role: the MI355X counterpart of the reference's batched QR for matrices
// past its register kernel (reference: shaders/QR_Householder.metal:665-847,
// driver src/qr_householder.mm:100-164: one threadgroup per matrix, panels of
// reflectors, up to 4096 rows), with the register kernel's conventions (the
// block scaled by a power of two into [0.5, 1), a reflector whose tail has a
// sum of squares below 2^-80 taken as the identity, R unscaled and exactly
// upper triangular, a matrix holding a NaN or an infinity written as all
// quiet NaN).  Reduced mode (Q m x n, R n x n) and R alone.
//
// qr_tall_kernel: lane c owns column c of the block, its rows in VGPRs.  Step
// J forms the reflector u = x - beta e_J of lane J's column (u_J = alpha -
// beta, H = I - u u^T / (beta (beta - alpha))), publishes u to LDS, and every
// lane right of J takes its dot product with u and its update.  The steps run
// as a loop (unrolling 64 steps of 128 rows would be a quarter megabyte of
// code, four times the instruction cache); the rows are handled in eight
// chunks of 16 held in registers, each chunk behind a wave-uniform test of
// the step against its rows, so that step J touches rows J.. only and the
// per-row masks are paid in the one chunk that holds row J.  Q is formed
// backwards from the reflectors kept in the lanes (sorg2r).
//
// Beyond 128 rows, a reduction tree of QRs (TSQR): the rows are split into
// blocks of 64 to 128 rows (balanced, so every block has at least n rows and
// an orthonormal Q), each block is factored, and the blocks' R factors,
// stacked in row order, form the next level's matrix, until one block is
// left; its R is the matrix's R.  Q is formed from the top: each block's Q
// times the n x n slice of the level above that belongs to its R, in place.
// Every level is one batched launch over all the batch's blocks.
#include <algorithm>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr float kTinySumsq = 8.271806e-25f;   // 2^-80
constexpr int kTallRows = 128;                // rows of a block, at most
constexpr int kTallCols = 64;                 // columns, at most
constexpr int kChunk = 16;
constexpr uint64_t kMaxGrid = uint64_t(1) << 22;   // workgroups per launch, at most

__device__ __forceinline__ float lane_value(float v, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// Rows of a level of `rows_total` rows split into `blocks` balanced blocks:
// the first `rows_total % blocks` blocks have one row more.
struct BlockRows {
    int start, rows;
};
__host__ __device__ inline BlockRows block_rows(int rows_total, int blocks, int i) {
    const int base = rows_total / blocks, extra = rows_total - base * blocks;
    return {i * base + (i < extra ? i : extra), base + (i < extra ? 1 : 0)};
}

// Sixteen rows of u to LDS.
__device__ __forceinline__ void write_chunk(float* dst, const float (&v)[kChunk]) {
#pragma unroll
    for (int i = 0; i < kChunk; i += 4)
        *reinterpret_cast<float4*>(dst + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}

// u . x over rows R0 .. RE-1 and x -= b u over the same rows, u read from
// LDS one chunk ahead of the arithmetic.  The offset of each chunk's reads
// passes through an empty asm statement that takes the previous chunk's
// result as an input, so the reads cannot all be hoisted to the top (which
// would hold all of u in registers next to the column and halve the waves
// per SIMD): at most two chunks of u are live, and each chunk's reads are in
// flight during the previous chunk's multiply-adds.
struct Chunk {
    float4 a, b, c, d;
};
__device__ __forceinline__ Chunk load_chunk(const float* u) {
    const float4* p = reinterpret_cast<const float4*>(u);
    return {p[0], p[1], p[2], p[3]};
}
__device__ __forceinline__ float chunk_at(const Chunk& k, int i) {
    const float4& q = i < 4 ? k.a : i < 8 ? k.b : i < 12 ? k.c : k.d;
    const int j = i & 3;
    return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}

template <int R0, int RE, int N>
__device__ __forceinline__ float dot_u(const float* u, const float (&x)[N]) {
    float d0 = 0.0f, d1 = 0.0f;
    Chunk cur = load_chunk(u + R0);
#pragma unroll
    for (int r0 = R0; r0 < RE; r0 += kChunk) {
        Chunk nxt = cur;
        if (r0 + kChunk < RE) {
            int off = r0 + kChunk;
            __asm__ volatile("" : "+v"(off) : "v"(d0));
            nxt = load_chunk(u + off);
        }
#pragma unroll
        for (int i = 0; i < kChunk; i += 2) {
            d0 = fmaf(chunk_at(cur, i), x[r0 + i], d0);
            d1 = fmaf(chunk_at(cur, i + 1), x[r0 + i + 1], d1);
        }
        cur = nxt;
    }
    return d0 + d1;
}

// x -= b u; with ONE, lane value `one` added at row j of chunk R0 (the
// formation of Q)
template <int R0, int RE, bool ONE, int N>
__device__ __forceinline__ void axpy_u(float (&x)[N], const float* u, float b, int j, float one) {
    Chunk cur = load_chunk(u + R0);
#pragma unroll
    for (int r0 = R0; r0 < RE; r0 += kChunk) {
        Chunk nxt = cur;
        if (r0 + kChunk < RE) {
            int off = r0 + kChunk;
            if (r0 > R0) __asm__ volatile("" : "+v"(off) : "v"(x[r0 - 1]));
            else __asm__ volatile("" : "+v"(off) : "v"(b));
            nxt = load_chunk(u + off);
        }
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const float y = fmaf(-b, chunk_at(cur, i), x[r0 + i]);
            x[r0 + i] = ONE && r0 == R0 ? y + (r0 + i == j ? one : 0.0f) : y;
        }
        cur = nxt;
    }
}

// Step J of sgeqr2, J in chunk P (16 P <= J < 16 P + 16): rows of chunks
// P .. MC-1 (compile-time, so the LDS reads of u can be issued ahead of the
// arithmetic), chunk P partial (rows above J untouched, row J the diagonal).
template <int P, int MC>
__device__ __forceinline__ void factor_step(float (&x)[MC * kChunk], float* u, float* csh, float* ujsh, float* bsh,
                                            int c, int J) {
    constexpr int R0 = P * kChunk, RE = MC * kChunk;
    int cl = c;
    __asm__ volatile("" : "+v"(cl));
    // x_J and the sum of squares below it, in every lane (lane J's used)
    float al = 0.0f, s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int r = R0 + i;
        al = r == J ? x[r] : al;
        s0 = fmaf(r > J ? x[r] : 0.0f, x[r], s0);
    }
#pragma unroll
    for (int r = R0 + kChunk; r < RE; r += 2) {
        s0 = fmaf(x[r], x[r], s0);
        s1 = fmaf(x[r + 1], x[r + 1], s1);
    }
    const float alpha = lane_value(al, J);
    const float ss = lane_value(s0 + s1, J);
    const bool nz = ss >= kTinySumsq;
    const float b = -copysignf(__builtin_amdgcn_sqrtf(fmaf(alpha, alpha, ss)), alpha);
    const float beta = nz ? b : alpha;
    const float uj = nz ? alpha - b : 1.0f;
    const float coef = nz ? rcp_refined(b * (b - alpha)) : 0.0f;
    if (cl == J) {   // stores only: u, zero above row J
        float v[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int r = R0 + i;
            v[i] = r < J ? 0.0f : (r == J ? uj : x[r]);
        }
        write_chunk(u + R0, v);
#pragma unroll
        for (int r = R0 + kChunk; r < RE; r += 4)
            *reinterpret_cast<float4*>(u + r) = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
        csh[J] = coef;
        ujsh[J] = uj;
        bsh[J] = beta;
    }
    wave_lds_sync();
    // the lane masks as factors (a select would become a branch around the
    // product and the update, and a copy of the column at its end)
    const float right = cl > J ? 1.0f : 0.0f;
    const float d = coef * dot_u<R0, RE>(u, x) * right;
    axpy_u<R0, RE, false>(x, u, d, J, 0.0f);
    // the next step writes the other buffer, and the one after writes this
    // one only past the next step's barrier
}

template <int P, int MC>
__device__ __forceinline__ void factor_phases(float (&x)[MC * kChunk], float* ush, float* csh, float* ujsh,
                                              float* bsh, int c, int n) {
    if constexpr (P < MC) {
        const int je = min(P * kChunk + kChunk, n);
        for (int J = P * kChunk; J < je; ++J) factor_step<P, MC>(x, ush + (J & 1) * kTallRows, csh, ujsh, bsh, c, J);
        factor_phases<P + 1, MC>(x, ush, csh, ujsh, bsh, c, n);
    }
}

// Step J of sorg2r's backward accumulation, J in chunk P: lane J (holding its
// reflector u, zero above row J) becomes e_J - coef u_J u = x - (1 + coef u_J)
// u + e_J, lanes right of J lose coef (u . x) u, lanes left of J keep theirs.
template <int P, int MC>
__device__ __forceinline__ void q_step(float (&x)[MC * kChunk], float* u, const float* csh, const float* ujsh,
                                       int c, int J) {
    constexpr int R0 = P * kChunk, RE = MC * kChunk;
    int cl = c;
    __asm__ volatile("" : "+v"(cl));
    if (cl == J) {
#pragma unroll
        for (int r = R0; r < RE; r += 4)
            *reinterpret_cast<float4*>(u + r) = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
    }
    wave_lds_sync();
    const float coef = csh[J];
    const float uj = ujsh[J];
    const float dot = dot_u<R0, RE>(u, x);
    const float self = cl == J ? 1.0f : 0.0f;
    const float right = cl > J ? 1.0f : 0.0f;
    const float bq = fmaf(self, fmaf(coef, uj, 1.0f), coef * dot * right);
    axpy_u<R0, RE, true>(x, u, bq, J, self);
}

template <int P, int MC>
__device__ __forceinline__ void q_phases(float (&x)[MC * kChunk], float* ush, const float* csh, const float* ujsh,
                                         int c, int n) {
    if constexpr (P >= 0) {
        for (int J = min(P * kChunk + kChunk, n) - 1; J >= P * kChunk; --J)
            q_step<P, MC>(x, ush + (J & 1) * kTallRows, csh, ujsh, c, J);
        q_phases<P - 1, MC>(x, ush, csh, ujsh, c, n);
    }
}

// One block per workgroup of one wave: block `blk % blocks` of matrix
// `blk / blocks`, whose H x n rows (row-major, contiguous per matrix) start
// at X; the level's blocks have at most 16 MC rows.  Writes the block's Q
// rows into Q at the same row positions (Q NULL for none) and its n x n R at
// R + blk n n.
template <int MC>
__global__ __launch_bounds__(64) void qr_tall_kernel(const float* __restrict__ X, float* __restrict__ Q,
                                                     float* __restrict__ R, uint32_t count, int H, int n,
                                                     int blocks) {
    constexpr int RE = MC * kChunk;
    __shared__ __align__(16) float ush[2 * kTallRows];
    __shared__ float csh[kTallCols];    // the reflectors' coefficients 1 / (beta (beta - alpha))
    __shared__ float ujsh[kTallCols];   // u_J
    __shared__ float bsh[kTallCols];    // beta: R's diagonal
    const uint32_t blk = blockIdx.x;
    if (blk >= count) return;
    const uint32_t mat = blk / (uint32_t)blocks;
    const BlockRows br = block_rows(H, blocks, (int)(blk - mat * (uint32_t)blocks));
    const int m = br.rows;   // n <= m <= 16 MC
    const int c = threadIdx.x;
    const bool col = c < n;
    const size_t row0 = (size_t)mat * H + br.start;

    // every lane loads (lanes past n read column 0, rows past m row m - 1)
    // and multiplies by 0 or 1: a select on a load would become a branch
    // around each load, with a wait inside it; a non-finite value read for a
    // lane or row outside makes no difference, the block holding it anyway.
    // Every block of a level has at least 16 (MC - 1) rows, so only the last
    // chunk's rows need the row test.  Fences every 32 rows bound the
    // addresses live at once.
    float x[RE];
    const float* src = X + row0 * n + (col ? c : 0);
    const float keep = col ? 1.0f : 0.0f;
#pragma unroll
    for (int r = 0; r < RE - kChunk; ++r) {
        x[r] = src[(size_t)r * n] * keep;
        if ((r & 31) == 31) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = RE - kChunk; r < RE; ++r) x[r] = src[(size_t)(r < m ? r : m - 1) * n] * (r < m ? keep : 0.0f);
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int r = 0; r < RE; ++r) {
        amax = fmaxf(amax, fabsf(x[r]));
        bad |= !finite_f(x[r]);
    }
    amax = group_max<64>(amax);
    bad = group_or<64>(bad);
    const int e = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < RE; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -e);

    factor_phases<0, MC>(x, ush, csh, ujsh, bsh, c, n);

    // R: rows above the diagonal from the lanes, the diagonal from beta
    if (col) {
        float* out_r = R + (size_t)blk * n * n;
        const float unscale = ldexpf(1.0f, e);
        const float diag = bsh[c];
        constexpr int RR = RE < kTallCols ? RE : kTallCols;
#pragma unroll
        for (int r = 0; r < RR; ++r)
            if (r < n) out_r[(size_t)r * n + c] = bad ? qnan() : (r < c ? x[r] : (r == c ? diag : 0.0f)) * unscale;
    }
    if (!Q) return;

    // lane c's column becomes its reflector u: zero above row c, u_c at row c
    {
        const float ujc = col ? ujsh[c] : 0.0f;
#pragma unroll
        for (int r = 0; r < RE; ++r) x[r] = r < c ? 0.0f : (r == c ? ujc : x[r]);
    }
    q_phases<MC - 1, MC>(x, ush, csh, ujsh, c, n);
    float* out_q = Q + row0 * n + c;
#pragma unroll
    for (int r = 0; r < RE; ++r)
        if (col && r < m) out_q[(size_t)r * n] = bad ? qnan() : x[r];
}

// G = Q_l U in place, per block of level l: the block's Q rows (in Q at its
// row positions) times the n x n slice of the level above's Q that belongs
// to the block's R (rows bi n .. bi n + n - 1 of the matrix above, Gup).  A
// NaN result is written as the quiet NaN 0x7FC00000.
__global__ __launch_bounds__(256) void tsqr_down_kernel(float* __restrict__ Q, const float* __restrict__ Gup,
                                                        uint32_t count, int H, int n, int blocks) {
    __shared__ float u[kTallCols * kTallCols];
    __shared__ float qs[kTallRows * (kTallCols + 1)];
    const uint32_t blk = blockIdx.x;
    if (blk >= count) return;
    const uint32_t mat = blk / (uint32_t)blocks;
    const int bi = (int)(blk - mat * (uint32_t)blocks);
    const BlockRows br = block_rows(H, blocks, bi);
    const int nn = n * n, ld = n + 1;
    const float* us = Gup + ((size_t)mat * blocks + bi) * nn;
    for (int i = threadIdx.x; i < nn; i += 256) u[i] = us[i];
    float* q = Q + ((size_t)mat * H + br.start) * n;
    for (int i = threadIdx.x; i < br.rows * n; i += 256) {
        const int r = i / n;
        qs[r * ld + (i - r * n)] = q[i];
    }
    __syncthreads();
    const int cc = threadIdx.x & 63;
    if (cc >= n) return;
    for (int r = threadIdx.x >> 6; r < br.rows; r += 4) {
        float s0 = 0.0f, s1 = 0.0f;
        int k = 0;
        for (; k + 1 < n; k += 2) {
            s0 = fmaf(qs[r * ld + k], u[k * n + cc], s0);
            s1 = fmaf(qs[r * ld + k + 1], u[(k + 1) * n + cc], s1);
        }
        if (k < n) s0 = fmaf(qs[r * ld + k], u[k * n + cc], s0);
        const float s = s0 + s1;
        q[(size_t)r * n + cc] = s != s ? qnan() : s;
    }
}

// The tree's levels: the rows of each level's matrix and its block count.
struct Level {
    int H, blocks;
};

std::vector<Level> tsqr_levels(int m, int n) {
    std::vector<Level> lv;
    int H = m;
    for (;;) {
        const int blocks = (H + kTallRows - 1) / kTallRows;
        lv.push_back({H, blocks});
        if (blocks == 1) break;
        H = blocks * n;
    }
    return lv;
}

// One launch of a level's blocks, the kernel instance chosen by the level's
// largest block (ceil(H / blocks) rows).
void launch_level(const float* x, float* q, float* r, uint32_t cnt, const Level& v, int n, hipStream_t s) {
    const int rows = (v.H + v.blocks - 1) / v.blocks;
    const int mc = (rows + kChunk - 1) / kChunk;
    void (*k)(const float*, float*, float*, uint32_t, int, int, int) = nullptr;
    switch (mc) {
    case 1: k = qr_tall_kernel<1>; break;
    case 2: k = qr_tall_kernel<2>; break;
    case 3: k = qr_tall_kernel<3>; break;
    case 4: k = qr_tall_kernel<4>; break;
    case 5: k = qr_tall_kernel<5>; break;
    case 6: k = qr_tall_kernel<6>; break;
    case 7: k = qr_tall_kernel<7>; break;
    case 8: k = qr_tall_kernel<8>; break;
    default: invalid("[qr] qr_tall: a block of " + std::to_string(rows) + " rows");
    }
    hipLaunchKernelGGL(k, dim3(cnt), dim3(64), 0, s, x, q, r, cnt, v.H, n, v.blocks);
}

// Matrices per launch so that a launch stays within kMaxGrid workgroups.
uint64_t mats_per_launch(const Level& l) { return std::max<uint64_t>(1, kMaxGrid / (uint64_t)l.blocks); }

// ---- the mid-size window: up to 128 rows and 128 columns, two waves ----
//
// qr_mid_kernel: the same steps over a workgroup of two waves, thread c
// owning column c (c < n <= 128), rows in VGPRs (m <= 16 MC <= 128).  Step
// J's reflector is formed by thread J alone from its own column and
// published in LDS (u, coef, u_J, beta) before the step's one barrier: the
// other wave cannot read lane J's registers.  K = min(m, n) steps (a wide
// matrix's later columns only take the updates); Q is m x K (reduced, or R
// alone), R is K x n.
constexpr int kMidCols = 128;

template <int P, int MC>
__device__ __forceinline__ void mid_factor_step(float (&x)[MC * kChunk], float* u, float* csh, float* ujsh,
                                                float* bsh, int c, int J) {
    constexpr int R0 = P * kChunk, RE = MC * kChunk;
    int cl = c;
    __asm__ volatile("" : "+v"(cl));
    if (cl == J) {
        float al = 0.0f, s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int r = R0 + i;
            al = r == J ? x[r] : al;
            s0 = fmaf(r > J ? x[r] : 0.0f, x[r], s0);
        }
#pragma unroll
        for (int r = R0 + kChunk; r < RE; r += 2) {
            s0 = fmaf(x[r], x[r], s0);
            s1 = fmaf(x[r + 1], x[r + 1], s1);
        }
        const float ss = s0 + s1;
        const bool nz = ss >= kTinySumsq;
        const float b = -copysignf(__builtin_amdgcn_sqrtf(fmaf(al, al, ss)), al);
        const float uj = nz ? al - b : 1.0f;
        float v[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int r = R0 + i;
            v[i] = r < J ? 0.0f : (r == J ? uj : x[r]);
        }
        write_chunk(u + R0, v);
#pragma unroll
        for (int r = R0 + kChunk; r < RE; r += 4)
            *reinterpret_cast<float4*>(u + r) = make_float4(x[r], x[r + 1], x[r + 2], x[r + 3]);
        csh[J] = nz ? rcp_refined(b * (b - al)) : 0.0f;
        ujsh[J] = uj;
        bsh[J] = nz ? b : al;
    }
    __syncthreads();
    const float right = cl > J ? 1.0f : 0.0f;
    const float d = csh[J] * dot_u<R0, RE>(u, x) * right;
    axpy_u<R0, RE, false>(x, u, d, J, 0.0f);
}

template <int P, int MC>
__device__ __forceinline__ void mid_factor_phases(float (&x)[MC * kChunk], float* ush, float* csh, float* ujsh,
                                                  float* bsh, int c, int K) {
    if constexpr (P < MC) {
        const int je = min(P * kChunk + kChunk, K);
        for (int J = P * kChunk; J < je; ++J)
            mid_factor_step<P, MC>(x, ush + (J & 1) * kTallRows, csh, ujsh, bsh, c, J);
        mid_factor_phases<P + 1, MC>(x, ush, csh, ujsh, bsh, c, K);
    }
}

template <int MC>
__global__ __launch_bounds__(kMidCols) void qr_mid_kernel(const float* __restrict__ A, float* __restrict__ Q,
                                                          float* __restrict__ R, uint32_t batch, int m, int n) {
    constexpr int RE = MC * kChunk;
    __shared__ __align__(16) float ush[2 * kTallRows];
    __shared__ float csh[kMidCols], ujsh[kMidCols], bsh[kMidCols];
    __shared__ float red[2];
    __shared__ int redb[2];
    const uint32_t mat = blockIdx.x;
    if (mat >= batch) return;
    const int c = threadIdx.x, lane = c & 63, wv = c >> 6;
    const int K = min(m, n);
    const bool col = c < n;
    const float* src = A + (size_t)mat * m * n + (col ? c : 0);
    const float keep = col ? 1.0f : 0.0f;
    // every thread loads (clamped: threads past n read column 0, rows past m
    // row m - 1) and multiplies by 0 or 1, as in the tall kernel
    float x[RE];
#pragma unroll
    for (int r = 0; r < RE; ++r) {
        x[r] = src[(size_t)(r < m ? r : m - 1) * n] * (r < m ? keep : 0.0f);
        if ((r & 31) == 31) __builtin_amdgcn_sched_barrier(0);
    }
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int r = 0; r < RE; ++r) {
        amax = fmaxf(amax, fabsf(x[r]));
        bad |= !finite_f(x[r]);
    }
    amax = group_max<64>(amax);
    bad = group_or<64>(bad);
    if (lane == 0) {
        red[wv] = amax;
        redb[wv] = bad;
    }
    __syncthreads();
    amax = fmaxf(red[0], red[1]);
    bad = redb[0] | redb[1];
    const int e = bad ? 0 : scale_exponent(amax);
#pragma unroll
    for (int r = 0; r < RE; ++r) x[r] = bad ? 0.0f : ldexpf(x[r], -e);

    mid_factor_phases<0, MC>(x, ush, csh, ujsh, bsh, c, K);

    // R (K x n): above the diagonal from the threads, the diagonal from beta
    if (col) {
        float* out_r = R + (size_t)mat * K * n;
        const float unscale = ldexpf(1.0f, e);
        const float diag = c < K ? bsh[c] : 0.0f;
#pragma unroll
        for (int r = 0; r < RE; ++r)
            if (r < K) out_r[(size_t)r * n + c] = bad ? qnan() : (r < c ? x[r] : (r == c ? diag : 0.0f)) * unscale;
    }
    if (!Q) return;
    // Q (m x K) backwards from the reflectors: thread c < K holds u_c
    {
        const float ujc = c < K ? ujsh[c] : 0.0f;
#pragma unroll
        for (int r = 0; r < RE; ++r) x[r] = c < K ? (r < c ? 0.0f : (r == c ? ujc : x[r])) : 0.0f;
    }
    q_phases<MC - 1, MC>(x, ush, csh, ujsh, c, K);
    if (c < K) {
        float* out_q = Q + (size_t)mat * m * K + c;
#pragma unroll
        for (int r = 0; r < RE; ++r)
            if (r < m) out_q[(size_t)r * K] = bad ? qnan() : x[r];
    }
}

}  // namespace

bool qr_tall_fits(uint32_t m, uint32_t n, uint32_t qc) {
    return n >= 1 && n <= (uint32_t)kTallCols && m >= n && (qc == 0 || qc == n);
}

size_t qr_tall_workspace(uint32_t m, uint32_t n, uint32_t batch, bool with_q) {
    const auto lv = tsqr_levels((int)m, (int)n);
    size_t floats = 0;
    // level l's R factors (level l+1's matrix) and level l+1's Q
    for (size_t l = 0; l + 1 < lv.size(); ++l) floats += (size_t)batch * lv[l + 1].H * n * (with_q ? 2 : 1);
    return floats * sizeof(float);
}

bool qr_mid_fits(uint32_t m, uint32_t n, uint32_t qc) {
    const uint32_t K = std::min(m, n);
    return m >= 1 && n >= 1 && m <= (uint32_t)kMidCols && n <= (uint32_t)kMidCols && std::max(m, n) > 64 &&
           (qc == 0 || qc == K);
}

void qr_mid(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, hipStream_t s) {
    if (!qr_mid_fits(m, n, q ? std::min(m, n) : 0)) invalid("[qr] qr_mid takes m, n <= 128");
    if (batch == 0) return;
    KernelTimer t("qr_mid", s);
    const int mc = (int)cdiv(m, kChunk);
    for (uint64_t b0 = 0; b0 < batch; b0 += kMaxGrid) {
        const uint32_t nb = (uint32_t)std::min<uint64_t>(kMaxGrid, batch - b0);
        const float* ab = a + b0 * m * n;
        float* qb = q ? q + b0 * m * std::min(m, n) : nullptr;
        float* rb = r + b0 * std::min(m, n) * n;
#define MLA_QR_MID(MC)                                                                                         \
    hipLaunchKernelGGL(qr_mid_kernel<MC>, dim3(nb), dim3(kMidCols), 0, s, ab, qb, rb, nb, (int)m, (int)n)
        switch (mc) {
            case 1: MLA_QR_MID(1); break;
            case 2: MLA_QR_MID(2); break;
            case 3: MLA_QR_MID(3); break;
            case 4: MLA_QR_MID(4); break;
            case 5: MLA_QR_MID(5); break;
            case 6: MLA_QR_MID(6); break;
            case 7: MLA_QR_MID(7); break;
            default: MLA_QR_MID(8); break;
        }
#undef MLA_QR_MID
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

void qr_tall(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, float* work,
             hipStream_t s) {
    if (!qr_tall_fits(m, n, q ? n : 0)) invalid("[qr] qr_tall takes n <= 64 columns and m >= n rows");
    if (batch == 0) return;
    KernelTimer t("qr_tall", s);
    const int N = (int)n;
    const auto lv = tsqr_levels((int)m, N);
    const size_t L = lv.size();
    // level l's matrix X_l (level 0: a), its Q (level 0: q) and its blocks' R
    // factors (the top level's: r)
    std::vector<const float*> X(L);
    std::vector<float*> Qs(L, nullptr), Rs(L);
    X[0] = a;
    Qs[0] = q;
    float* p = work;
    for (size_t l = 0; l + 1 < L; ++l) {
        const size_t above = (size_t)batch * lv[l + 1].H * N;
        Rs[l] = p;
        X[l + 1] = p;
        p += above;
        if (q) {
            Qs[l + 1] = p;
            p += above;
        }
    }
    Rs[L - 1] = r;
    for (size_t l = 0; l < L; ++l) {
        const Level& v = lv[l];
        const uint64_t per = mats_per_launch(v);
        for (uint64_t m0 = 0; m0 < batch; m0 += per) {
            const uint64_t nm = std::min<uint64_t>(per, batch - m0);
            const uint32_t cnt = (uint32_t)(nm * v.blocks);
            launch_level(X[l] + m0 * v.H * N, q ? Qs[l] + m0 * v.H * N : nullptr, Rs[l] + m0 * v.blocks * N * N,
                         cnt, v, N, s);
        }
    }
    if (q) {
        for (size_t l = L - 1; l-- > 0;) {
            const Level& v = lv[l];
            const uint64_t per = mats_per_launch(v);
            for (uint64_t m0 = 0; m0 < batch; m0 += per) {
                const uint64_t nm = std::min<uint64_t>(per, batch - m0);
                const uint32_t cnt = (uint32_t)(nm * v.blocks);
                hipLaunchKernelGGL(tsqr_down_kernel, dim3(cnt), dim3(256), 0, s, Qs[l] + m0 * v.H * N,
                                   Qs[l + 1] + m0 * lv[l + 1].H * N, cnt, v.H, N, v.blocks);
            }
        }
    }
    t.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
