// Symmetric eigendecomposition for matrices beyond the register kernel
// (n > 64; config 5's 4096 x 4096), one matrix at a time:
//   1. reduction to tridiagonal form, Q^T A Q = T (ssytrd, lower, blocked
//      as slatrd: panels of NB columns, trailing update A -= V W^T + W V^T)
//   2. the tridiagonal eigenproblem (tridiag_solver: divide and conquer for
//      vectors, bisection for values only)
//   3. back-transformation V = Q Z with the reflectors in compact WY form
//
// Role: the MI355X counterpart of the reference's large-matrix eigh
// (reference: src/svd_bidiag.mm eigh_band_vectors and
// src/band_reduce.mm:610-711 band_reduce_symmetric, src/band_chase.cpp:431,
// src/divide_conquer.cpp:934), with the CPU path's contract
// (src/eigh.mm:664-758): only the `lower` (or upper) triangle is read;
// eigenvalues ascending, eigenvectors as columns; a non-finite entry in the
// read triangle gives all-NaN w and V and info = 1 << 17; otherwise
// info = 1 | 1 << 16.  The reference reduces to a band on the GPU and
// finishes on the CPU; here every stage runs on the GPU.
//
// Stage 1, per column j (panel column i = j - j0), two launches over row
// blocks, with W materialised one column late so that each reduction folds
// into the next launch:
//   sytrd_col   W[:, i-1] = tau (y - W qV - V qW) + alpha' v from the
//               previous column's partial dot products (each workgroup sums
//               them itself), then the column update
//               a = A[:, j] - V W[j, :]^T - W V[j, :]^T and partial sums of
//               squares of its tail
//   sytrd_symv  the reflector (every workgroup forms the whole v from a),
//               y = A[j+1:, j+1:] v for its rows (the bandwidth-bound symv:
//               16 rows per workgroup, float4 loads, DPP row sums) and the
//               partial dot products V^T v, W^T v, y^T v
// and per panel two MFMA products for the trailing update.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NBT = 64;                        // panel width of the reduction
constexpr int kColRows = 64;                   // rows per workgroup in sytrd_col (4 threads per row)
constexpr int kSymvRows = 16;                  // rows per workgroup in sytrd_symv (16 lanes per row)
constexpr float kTinySumsq = 8.271806e-25f;    // 2^-80

// ---- scan of the read triangle, scaled symmetric copy ----

__global__ __launch_bounds__(256) void sym_scan_kernel(const float* __restrict__ a, int n, int lower,
                                                       uint32_t* __restrict__ flags) {
    unsigned m = 0, bad = 0;
    const size_t count = (size_t)n * n;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) {
        const int r = (int)(i / n), c = (int)(i - (size_t)r * n);
        if (lower ? c > r : c < r) continue;
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

__global__ void sym_zero_flags_kernel(uint32_t* f) {
    f[0] = 0;
    f[1] = 0;
}

// W (full, symmetric) = the read triangle mirrored, times 2^-e
__global__ __launch_bounds__(256) void sym_copy_kernel(const float* __restrict__ a, float* __restrict__ W, int n,
                                                       int lower, const uint32_t* __restrict__ flags) {
    __shared__ float tile[32][33];
    const bool bad = flags[1] != 0;
    const int e = bad ? 0 : scale_exponent(__uint_as_float(flags[0]));
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;   // output tile: rows by.., columns bx..
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    // the transposed source tile (rows bx.., columns by..)
    for (int r = ty; r < 32; r += 8) {
        const int i = bx + r, c = by + tx;
        tile[r][tx] = (i < n && c < n) ? a[(size_t)i * n + c] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, c = bx + tx;
        if (i >= n || c >= n) continue;
        const bool own = lower ? c <= i : c >= i;   // (i, c) in the read triangle
        const float v = own ? a[(size_t)i * n + c] : tile[tx][r];
        W[(size_t)i * n + c] = bad ? 0.0f : ldexpf(v, -e);
    }
}

// ---- stage 1: the two per-column launches ----

struct SytrdArgs {
    float* A;          // n x n working matrix (row-major)
    int n;
    int j0, i;         // panel start and panel column: column j = j0 + i
    float* Vp;         // the panel's reflectors: V_k[r] at Vp[k * n + r] (also the record for stage 3)
    float* Wp;         // W_k[r] at Wp[k * n + r]
    float* abuf;       // the updated column j (n)
    float* y;          // A22 v of the previous column (n)
    float* partA;      // per-workgroup sums of squares (sytrd_col)
    float* partB;      // per-workgroup partial dots (sytrd_symv): [slot][wg], 2 * NBT + 1 slots
    int nwgB;          // workgroups of sytrd_symv
    float* d;
    float* e;
    float* tau;
    int update;        // 0: only materialise W[:, i-1] (end of a panel)
};



// 64 rows per workgroup, 4 threads per row; thread `sub` of a row takes the
// panel columns k = sub, sub + 4, ...  Every global load of a thread is
// issued before the first use (clamped addresses), so their latencies
// overlap.
__global__ __launch_bounds__(256) void sytrd_col_kernel(SytrdArgs g) {
    __shared__ float q[2 * NBT + 1];   // qV (k < i-1), qW, y^T v of the previous column
    __shared__ float rowj[2 * NBT];    // V[j, k], W[j, k] for k < i
    __shared__ float red[256 / 64];
    __shared__ float wj;               // W[j, i-1]
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int n = g.n, j = g.j0 + g.i, i = g.i;
    const int row = blockIdx.x * kColRows + (t >> 2), sub = t & 3;
    const int rr = row < n ? row : n - 1;
    const int ip = i - 1;   // the column whose W is materialised
    // this thread's share of row `row` of V and W (the columns k = sub + 4u)
    float vk[NBT / 4], wk[NBT / 4];
#pragma unroll
    for (int u = 0; u < NBT / 4; ++u) {
        const int k = sub + 4 * u;
        const float x = g.Vp[(size_t)(k < i ? k : 0) * n + rr];
        const float y = g.Wp[(size_t)(k < ip ? k : 0) * n + rr];
        vk[u] = k < i ? x : 0.0f;
        wk[u] = k < ip ? y : 0.0f;
    }
    const float yr = g.y[rr], vipr = g.Vp[(size_t)(ip >= 0 ? ip : 0) * n + rr];
    const float arj = g.A[(size_t)rr * n + j];
    // row j of V and W (W[j, ip] comes from its own dot below)
    if (g.update && t < i) {
        rowj[t] = g.Vp[(size_t)t * n + j];
        rowj[NBT + t] = t < ip ? g.Wp[(size_t)t * n + j] : 0.0f;
    }
    float tp = 0.0f, alpha2 = 0.0f;
    if (ip >= 0) {
        // the previous column's partial dots: qV[k], qW[k] (k < ip), y^T v.
        // Two threads per slot (nv <= 2 NBT - 1 <= 127 slots: one pass of
        // 256 threads), each summing half of the workgroups' partials, so
        // that one round of loads (32 float4 each at n <= 4096) covers it
        const int nv = 2 * ip + 1;
        const int hn = ((g.nwgB + 7) >> 3) << 2;   // half of nwgB, rounded up to a multiple of 4
        const bool vec4 = (g.nwgB & 3) == 0;
        for (int x0 = 0; x0 < nv; x0 += 128) {
            const int x = x0 + (t >> 1), hf = t & 1;
            const bool live = x < nv;
            const int xs = live ? x : 0;
            const int slot = xs < ip ? xs : (xs < 2 * ip ? NBT + (xs - ip) : 2 * NBT);
            const float* ps = g.partB + (size_t)slot * g.nwgB;
            const int bb = hf * hn, be = min(g.nwgB, bb + hn);
            float acc = 0.0f;
            if (vec4) {
                for (int b0 = bb; b0 < be; b0 += 128) {
                    float4 pv[32];
#pragma unroll
                    for (int u = 0; u < 32; ++u) {
                        const int b = b0 + 4 * u;
                        pv[u] = *reinterpret_cast<const float4*>(ps + (b < be ? b : 0));
                    }
                    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int u = 0; u < 32; ++u)
                        if (b0 + 4 * u < be) {
                            s4[0] += pv[u].x;
                            s4[1] += pv[u].y;
                            s4[2] += pv[u].z;
                            s4[3] += pv[u].w;
                        }
                    acc += (s4[0] + s4[1]) + (s4[2] + s4[3]);
                }
            } else {
                for (int b = bb; b < be; ++b) acc += ps[b];
            }
            acc += __shfl_xor(acc, 1, 64);
            if (live && hf == 0) q[x] = acc;
        }
        __syncthreads();
        tp = g.tau[g.j0 + ip];
        // w^T v before the correction = tau (y^T v - 2 qV . qW); ip < 64,
        // so one lane per k and a wave sum
        const float qq = wave_sum_f(lane < ip ? q[lane] * q[ip + (lane < ip ? lane : 0)] : 0.0f);
        alpha2 = -0.5f * tp * (tp * (q[2 * ip] - 2.0f * qq));
    }
    // W[row, ip] = tau (y - W qV - V qW) + alpha' v  (rows >= j)
    float wnew = 0.0f;
    if (ip >= 0) {
        float sp = 0.0f;
#pragma unroll
        for (int u = 0; u < NBT / 4; ++u) {
            const int k = sub + 4 * u;
            if (k < ip) sp = fmaf(wk[u], q[k], fmaf(vk[u], q[ip + k], sp));
        }
        sp = quad_sum(sp);
        wnew = row >= j ? fmaf(tp, yr - sp, alpha2 * vipr) : 0.0f;
        if (sub == 0 && row < n) g.Wp[(size_t)ip * n + row] = wnew;
    }
    if (!g.update) return;
    __syncthreads();   // rowj
    if (t < 64) {   // wave 0: one lane per k
        float wv0 = 0.0f;
        if (ip >= 0) {
            const int k = lane < ip ? lane : 0;
            const float sp = wave_sum_f(lane < ip ? fmaf(rowj[NBT + k], q[k], rowj[k] * q[ip + k]) : 0.0f);
            wv0 = fmaf(tp, g.y[j] - sp, alpha2 * rowj[ip]);
        }
        if (t == 0) wj = wv0;
    }
    __syncthreads();
    // a = A[:, j] - V W[j, :]^T - W V[j, :]^T on rows >= j
    float sa = 0.0f;
#pragma unroll
    for (int u = 0; u < NBT / 4; ++u) {
        const int k = sub + 4 * u;
        if (k < i) {
            const float wkk = k == ip ? wnew : wk[u];
            const float wjk = k == ip ? wj : rowj[NBT + k];
            sa = fmaf(vk[u], wjk, fmaf(wkk, rowj[k], sa));
        }
    }
    sa = quad_sum(sa);
    const float av = arj - sa;
    float ss = 0.0f;
    if (sub == 0 && row < n && row >= j) {
        g.abuf[row] = av;
        if (row == j) g.d[j] = av;
        if (row >= j + 2) ss = av * av;
    }
    ss = wave_sum_f(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    if (t == 0) g.partA[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// 16 rows per workgroup: the reflector (every workgroup forms all of v in
// LDS), y = A22 v, and the partial dot products for the next column.
__global__ __launch_bounds__(256) void sytrd_symv_kernel(SytrdArgs g, int nwgA) {
    extern __shared__ float v[];   // the reflector, whole (n floats)
    __shared__ float sc[2];
    __shared__ float yrow[kSymvRows];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int n = g.n, j = g.j0 + g.i, i = g.i;
    if (wv == 0) {
        float ss = 0.0f;
        for (int b = lane; b < nwgA; b += 64) ss += g.partA[b];
        ss = wave_sum_f(ss);
        if (lane == 0) {
            const float alpha = j + 1 < n ? g.abuf[j + 1] : 0.0f;
            float beta = alpha, tau = 0.0f, scal = 1.0f;
            if (ss >= kTinySumsq) {
                beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
                tau = (beta - alpha) / beta;
                scal = 1.0f / (alpha - beta);
            }
            sc[0] = tau;
            sc[1] = scal;
            if (blockIdx.x == 0) {
                g.e[j] = beta;
                g.tau[j] = tau;
            }
        }
    }
    __syncthreads();
    const float scal = sc[1];
    // v from the updated column (16 loads in flight per round)
    for (int r0 = 0; r0 < n; r0 += 256 * 16) {
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int r = r0 + t + 256 * u;
            x[u] = g.abuf[r < n ? r : 0];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int r = r0 + t + 256 * u;
            if (r < n) v[r] = r < j + 1 ? 0.0f : (r == j + 1 ? 1.0f : x[u] * scal);
        }
    }
    __syncthreads();
    const int rb = blockIdx.x * kSymvRows;
    for (int r = rb + t; r < min(n, rb + kSymvRows); r += 256) g.Vp[(size_t)i * n + r] = v[r];
    // y = A22 v: 16 lanes per row; a row's columns as float4s from the
    // aligned column at or before j + 1 (v is zero left of j + 1), 16 loads
    // in flight per lane
    const int c0 = (j + 1) & ~3;
    const bool vec = (n & 3) == 0;
    const int sub = t & 15;
    {
        const int row = rb + (t >> 4);
        float acc = 0.0f;
        if (row < n && row >= j + 1) {
            const float* ar = g.A + (size_t)row * n;
            if (vec) {
                for (int cb = c0 + sub * 4; cb < n; cb += 64 * 16) {
                    float4 xs[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        const int c = cb + 64 * u;
                        xs[u] = *reinterpret_cast<const float4*>(ar + (c < n ? c : c0));
                    }
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        const int c = cb + 64 * u;
                        if (c < n)
                            acc = fmaf(xs[u].x, v[c],
                                       fmaf(xs[u].y, v[c + 1], fmaf(xs[u].z, v[c + 2], fmaf(xs[u].w, v[c + 3], acc))));
                    }
                }
            } else {
                for (int c = j + 1 + sub; c < n; c += 16) acc = fmaf(ar[c], v[c], acc);
            }
        }
        acc = dpp_row_sum(acc);
        if (sub == 0 && row < n) {
            const float yv = row >= j + 1 ? acc : 0.0f;
            g.y[row] = yv;
            yrow[t >> 4] = yv;
        }
    }
    __syncthreads();
    // partial dots over this block's rows: V_k^T v, W_k^T v (k < i), y^T v;
    // a thread per value, its 64 rows as float4s
    const int nwg = gridDim.x;
    for (int x = t; x < 2 * i + 1; x += 256) {
        const float* src = x < i ? g.Vp + (size_t)x * n : (x < 2 * i ? g.Wp + (size_t)(x - i) * n : nullptr);
        float s = 0.0f;
        if (src && vec && rb + kSymvRows <= n) {
            float4 o[kSymvRows / 4];
#pragma unroll
            for (int u = 0; u < kSymvRows / 4; ++u) o[u] = *reinterpret_cast<const float4*>(src + rb + 4 * u);
#pragma unroll
            for (int u = 0; u < kSymvRows / 4; ++u) {
                const int r = rb + 4 * u;
                s = fmaf(o[u].x, v[r], fmaf(o[u].y, v[r + 1], fmaf(o[u].z, v[r + 2], fmaf(o[u].w, v[r + 3], s))));
            }
        } else {
            for (int rr = 0; rr < kSymvRows; ++rr) {
                const int r = rb + rr;
                if (r < n) s = fmaf(src ? src[r] : yrow[rr], v[r], s);
            }
        }
        const int slot = x < i ? x : (x < 2 * i ? NBT + (x - i) : 2 * NBT);
        g.partB[(size_t)slot * nwg + blockIdx.x] = s;
    }
}

// 2^e x (the scale taken out by sym_copy), or NaN for a bad matrix
__global__ __launch_bounds__(256) void eigh_unscale_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                           int count, const uint32_t* __restrict__ flags) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const bool bad = flags[1] != 0;
    const int e = bad ? 0 : scale_exponent(__uint_as_float(flags[0]));
    y[i] = bad ? qnan() : ldexpf(x[i], e);
}

}  // namespace

EighWork eigh_carve(float* base, uint32_t n) {
    const size_t N = n;
    const int nwgA = cdiv((int)n, kColRows), nwgB = cdiv((int)n, kSymvRows);
    float* p = base;
    auto take = [&](size_t c) {
        float* r = p;
        p += (c + 63) / 64 * 64;
        return r;
    };
    EighWork w{};
    w.A = take(N * N);
    w.V = take(N * N);
    w.W = take((size_t)NBT * N);
    w.abuf = take(N);
    w.y = take(N);
    w.partA = take(nwgA);
    w.partB = take((size_t)nwgB * (2 * NBT + 1));
    w.d = take(N);
    w.e = take(N);
    w.tau = take(N);
    w.flags = reinterpret_cast<uint32_t*>(take(64));
    w.rest = p;
    return w;
}

size_t eigh_sytrd_floats(uint32_t n) {
    const size_t N = n;
    const int nwgA = cdiv((int)n, kColRows), nwgB = cdiv((int)n, kSymvRows);
    auto r = [](size_t c) { return (c + 63) / 64 * 64; };
    return r(N * N) * 2 + r((size_t)NBT * N) + r(N) * 2 + r(nwgA) + r((size_t)nwgB * (2 * NBT + 1)) + r(N) * 3 + 64;
}

bool eigh_blocked_fits(uint32_t n) { return n >= 2 && n <= 16384; }

void eigh_unscale(const float* x, float* y, uint32_t count, const uint32_t* flags, hipStream_t s) {
    hipLaunchKernelGGL(eigh_unscale_kernel, dim3((unsigned)cdiv((int)count, 256)), dim3(256), 0, s, x, y, (int)count,
                       flags);
}

// Stage 1 on one matrix: a (n x n, the `lower` or upper triangle read) ->
// w.d, w.e (T's diagonal and subdiagonal, scaled by 2^-e), the reflectors
// (w.V[j * n + r], r > j, v_j[j + 1] = 1) and w.tau; flags[0] = bits of
// max |a|, flags[1] = non-finite.
void sytrd_one(const float* a, uint32_t nn, bool lower, const EighWork& w, hipStream_t s) {
    const int n = (int)nn;
    const size_t N = nn;
    const int nwgA = cdiv(n, kColRows), nwgB = cdiv(n, kSymvRows);
    hipLaunchKernelGGL(sym_zero_flags_kernel, dim3(1), dim3(1), 0, s, w.flags);
    hipLaunchKernelGGL(sym_scan_kernel, dim3((unsigned)std::min<size_t>(cdiv(N * N, 256), 4096)), dim3(256), 0, s, a,
                       n, lower ? 1 : 0, w.flags);
    hipLaunchKernelGGL(sym_copy_kernel, dim3((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32)), dim3(256), 0, s, a, w.A, n,
                       lower ? 1 : 0, w.flags);
    KernelTimer tm("sytrd", s);
    for (int j0 = 0; j0 < n; j0 += NBT) {
        const int nb = std::min(NBT, n - j0);
        float* Vp = w.V + (size_t)j0 * N;
        SytrdArgs g{w.A, n, j0, 0, Vp, w.W, w.abuf, w.y, w.partA, w.partB, nwgB, w.d, w.e, w.tau, 1};
        for (int i = 0; i < nb; ++i) {
            g.i = i;
            g.update = 1;
            hipLaunchKernelGGL(sytrd_col_kernel, dim3((unsigned)nwgA), dim3(256), 0, s, g);
            if (j0 + i < n - 1)
                hipLaunchKernelGGL(sytrd_symv_kernel, dim3((unsigned)nwgB), dim3(256), N * sizeof(float), s, g, nwgA);
        }
        const int pe = j0 + nb;
        if (pe < n) {
            // W[:, nb-1], then A22 -= V W^T + W V^T on rows and columns >= pe
            g.i = nb;
            g.update = 0;
            hipLaunchKernelGGL(sytrd_col_kernel, dim3((unsigned)nwgA), dim3(256), 0, s, g);
            const int n2 = n - pe;
            float* A22 = w.A + (size_t)pe * n + pe;
            sgemm(true, false, n2, n2, nb, -1.0f, Vp + pe, n, 0, w.W + pe, n, 0, 1.0f, A22, n, 0, 1, s);
            sgemm(true, false, n2, n2, nb, -1.0f, w.W + pe, n, 0, Vp + pe, n, 0, 1.0f, A22, n, 0, 1, s);
        }
    }
    tm.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla

// Diagnostic hook (include/metal_linalg/hip_ext.h): the tridiagonal form of
// one symmetric matrix (device or host pointers), d and e scaled back.
extern "C" int metal_linalg_hip_sytrd(const float* a, uint32_t n, int lower, float* d, float* e) {
    try {
        if (n < 2) return 1;
        mla::Call call;
        const float* da = call.in(a, (size_t)n * n);
        float* dd = call.out(d, n);
        float* de = call.out(e, n - 1);
        float* work = static_cast<float*>(call.scratch(mla::eigh_sytrd_floats(n) * sizeof(float)));
        const mla::EighWork w = mla::eigh_carve(work, n);
        mla::sytrd_one(da, n, lower != 0, w, call.stream());
        mla::eigh_unscale(w.d, dd, n, w.flags, call.stream());
        mla::eigh_unscale(w.e, de, n - 1, w.flags, call.stream());
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
