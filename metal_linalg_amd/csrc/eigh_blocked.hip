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
constexpr int kColRows = 256;                  // rows per workgroup in sytrd_col
constexpr int kSymvRows = 16;                  // rows per workgroup in sytrd_symv
constexpr float kTinySumsq = 8.271806e-25f;    // 2^-80

__device__ __forceinline__ float dpp_row_sum(float v) {
    // every lane of each row of 16 ends with the row's sum
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
    return v;
}

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
    float* partB;      // per-workgroup partial dots (sytrd_symv): [wg][2 * NBT + 1]
    int nwgB;          // workgroups of sytrd_symv
    float* d;
    float* e;
    float* tau;
    int update;        // 0: only materialise W[:, i-1] (end of a panel)
};

__global__ __launch_bounds__(256) void sytrd_col_kernel(SytrdArgs g) {
    __shared__ float q[2 * NBT + 1];   // qV (k < i-1), qW, y^T v of the previous column
    __shared__ float rowj[2 * NBT];    // V[j, k], W[j, k] for k < i
    __shared__ float red[256 / 64];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int n = g.n, j = g.j0 + g.i, i = g.i;
    const int r0 = blockIdx.x * kColRows;
    const int ip = i - 1;   // the column whose W is materialised
    float tp = 0.0f, alpha2 = 0.0f;
    if (ip >= 0) {
        // sum the previous column's partial dots: qV[k], qW[k] (k < ip), y^T v
        const int nv = 2 * ip + 1;
        for (int x = t; x < nv; x += 256) {
            const int slot = x < ip ? x : (x < 2 * ip ? NBT + (x - ip) : 2 * NBT);
            float s = 0.0f;
#pragma unroll 8
            for (int b = 0; b < g.nwgB; ++b) s += g.partB[(size_t)b * (2 * NBT + 1) + slot];
            q[x] = s;
        }
        __syncthreads();
        tp = g.tau[g.j0 + ip];
        // w^T v before the correction = tau (y^T v - 2 qV . qW)
        float qq = 0.0f;
        for (int k = 0; k < ip; ++k) qq = fmaf(q[k], q[ip + k], qq);
        alpha2 = -0.5f * tp * (tp * (q[2 * ip] - 2.0f * qq));
    }
    // W[:, ip] for this block's rows (defined on rows >= j), and row j of V, W
    const float* vp = g.Vp + (size_t)ip * n;
    auto wval = [&](int r) {
        float s = g.y[r];
#pragma unroll 4
        for (int k = 0; k < ip; ++k) s = fmaf(-g.Wp[(size_t)k * n + r], q[k], fmaf(-g.Vp[(size_t)k * n + r], q[ip + k], s));
        return fmaf(tp, s, alpha2 * vp[r]);
    };
    if (ip >= 0) {
        for (int r = r0 + t; r < min(n, r0 + kColRows); r += 256)
            g.Wp[(size_t)ip * n + r] = r >= j ? wval(r) : 0.0f;
    }
    if (!g.update) return;
    for (int k = t; k < i; k += 256) {
        rowj[k] = g.Vp[(size_t)k * n + j];
        rowj[NBT + k] = k == ip ? wval(j) : g.Wp[(size_t)k * n + j];
    }
    __syncthreads();
    // a = A[:, j] - V W[j, :]^T - W V[j, :]^T on rows >= j; partial tail sums of squares
    float ss = 0.0f;
    for (int r = r0 + t; r < min(n, r0 + kColRows); r += 256) {
        if (r < j) continue;
        float s = g.A[(size_t)r * n + j];
        // (W[:, ip] of this row was written just above by this thread)
#pragma unroll 4
        for (int k = 0; k < i; ++k)
            s = fmaf(-g.Vp[(size_t)k * n + r], rowj[NBT + k], fmaf(-g.Wp[(size_t)k * n + r], rowj[k], s));
        g.abuf[r] = s;
        if (r == j) g.d[j] = s;
        if (r >= j + 2) ss = fmaf(s, s, ss);
    }
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    if (t == 0) g.partA[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void sytrd_symv_kernel(SytrdArgs g, int nwgA) {
    extern __shared__ float v[];   // the reflector, whole (n floats)
    __shared__ float sc[4];
    __shared__ float yrow[kSymvRows];
    const int t = threadIdx.x;
    const int n = g.n, j = g.j0 + g.i, i = g.i;
    if (t == 0) {
        float ss = 0.0f;
        for (int b = 0; b < nwgA; ++b) ss += g.partA[b];
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
    __syncthreads();
    const float scal = sc[1];
    for (int r = t; r < n; r += 256) v[r] = r < j + 1 ? 0.0f : (r == j + 1 ? 1.0f : g.abuf[r] * scal);
    __syncthreads();
    const int r0 = blockIdx.x * kSymvRows;
    for (int r = r0 + t; r < min(n, r0 + kSymvRows); r += 256) g.Vp[(size_t)i * n + r] = v[r];
    // y = A22 v for rows r0 .. r0 + 15 (16 lanes per row, float4 columns from
    // the aligned column at or before j + 1; v is zero left of j + 1)
    const int row = r0 + (t >> 4), sub = t & 15;
    const int c0 = (j + 1) & ~3;
    float acc = 0.0f;
    if (row < n && row >= j + 1) {
        const float* ar = g.A + (size_t)row * n;
        if ((n & 3) == 0) {
            for (int c = c0 + sub * 4; c < n; c += 64) {
                const float4 x = *reinterpret_cast<const float4*>(ar + c);
                acc = fmaf(x.x, v[c], fmaf(x.y, v[c + 1], fmaf(x.z, v[c + 2], fmaf(x.w, v[c + 3], acc))));
            }
        } else {
            for (int c = j + 1 + sub; c < n; c += 16) acc = fmaf(ar[c], v[c], acc);
        }
    }
    acc = dpp_row_sum(acc);
    if (sub == 0 && row < n) {
        const float yr = row >= j + 1 ? acc : 0.0f;
        g.y[row] = yr;
        yrow[t >> 4] = yr;
    }
    __syncthreads();
    // partial dots over this block's rows: V_k^T v, W_k^T v (k < i), y^T v
    float* out = g.partB + (size_t)blockIdx.x * (2 * NBT + 1);
    for (int x = t; x < 2 * i + 1; x += 256) {
        const float* src = x < i ? g.Vp + (size_t)x * n : (x < 2 * i ? g.Wp + (size_t)(x - i) * n : nullptr);
        float o[kSymvRows];
#pragma unroll
        for (int rr = 0; rr < kSymvRows; ++rr) {
            const int r = min(r0 + rr, n - 1);
            o[rr] = src ? src[r] : yrow[rr];
        }
        float s = 0.0f;
#pragma unroll
        for (int rr = 0; rr < kSymvRows; ++rr)
            if (r0 + rr < n) s = fmaf(o[rr], v[r0 + rr], s);
        const int slot = x < i ? x : (x < 2 * i ? NBT + (x - i) : 2 * NBT);
        out[slot] = s;
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
