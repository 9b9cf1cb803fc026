// Stages 2 and 3 of the large-matrix eigh: the tridiagonal eigenproblem
// T = Z diag(w) Z^T, and the back-transformation V = Q Z.
//
// Role: the MI355X counterpart of the reference's tridiagonal solver and
// back-transform (reference: src/divide_conquer.cpp:934
// tridiagonal_eigensystem, src/svd_bidiag.mm eigh_band_vectors V = Q1 Q2 Z);
// LAPACK's contract for the result (ssyevd: ascending eigenvalues,
// orthonormal eigenvectors).  The method is LAPACK's other route, sstebz +
// sstein, shaped for a GPU:
//   - T splits where |e_i| <= eps sqrt(|d_i d_{i+1}|) into unreduced blocks
//     (their eigenvectors have disjoint supports);
//   - eigenvalues by multisection of the Sturm count: 16 lanes per
//     eigenvalue evaluate 16 points at once, so an iteration narrows the
//     interval 17-fold (sstebz bisects);
//   - eigenvectors by inverse iteration from a pseudo-random start, two
//     solves with (T - lambda I) factored with partial pivoting (slagtf /
//     slagts), one thread per cluster of eigenvalues closer than
//     1e-5 ||T||, modified Gram-Schmidt inside a cluster (sstein);
//   - the remaining loss of orthogonality (of order eps ||T|| / gap) removed
//     by one Newton-Schulz step Z <- Z (3 I - Z^T Z) / 2 on the matrix
//     cores: the columns move by a skew-symmetric correction of the same
//     order, which changes the residual A Z - Z W only at the eps ||T||
//     level;
//   - V = Q Z with Q's reflectors in compact WY form per panel of 64:
//     Z2 -= V (T (V^T Z2)), MFMA products.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr int NBT = 64;        // the reduction's panel width (reflectors per block)
constexpr int kMS = 16;        // multisection points per eigenvalue
constexpr int kIters = 2;      // inverse-iteration solves
constexpr int CH = 16;         // rows per chunk of the inverse iteration's passes

struct Slot {            // one eigenvalue: its block and its place in it
    int start, size, local, pad;
    float lo, hi;        // the block's Gershgorin interval
};

// ---- eigenvalues: multisection of the Sturm count ----
//
// count(x) = the number of eigenvalues of the block below x, from the signs
// of the pivots of T - x I = L D L^T (q_i = d_i - x - e_{i-1}^2 / q_{i-1});
// a pivot smaller than pivmin in magnitude is taken as -pivmin.
__device__ __forceinline__ int sturm_count(const float* __restrict__ d, const float* __restrict__ e2, int s, int m,
                                           float x, float pivmin) {
    float q = d[s] - x;
    q = fabsf(q) <= pivmin ? -pivmin : q;
    int c = q < 0.0f;
    for (int i = 1; i < m; ++i) {
        q = (d[s + i] - x) - e2[s + i - 1] * __builtin_amdgcn_rcpf(q);
        q = fabsf(q) <= pivmin ? -pivmin : q;
        c += q < 0.0f;
    }
    return c;
}

__global__ __launch_bounds__(256) void multisection_kernel(const float* __restrict__ d, const float* __restrict__ e2,
                                                           const Slot* __restrict__ slots, int nslots, float pivmin,
                                                           float* __restrict__ lam) {
    const int t = threadIdx.x, lane = t & 63;
    const int sidx = blockIdx.x * (256 / kMS) + (t / kMS);
    const int j = t % kMS;   // this lane's point
    const bool live = sidx < nslots;
    const Slot sl = slots[live ? sidx : 0];
    float lo = sl.lo, hi = sl.hi;
    for (int it = 0; it < 12; ++it) {
        const float x = lo + (hi - lo) * (float)(j + 1) / (float)(kMS + 1);
        const bool above = live && sturm_count(d, e2, sl.start, sl.size, x, pivmin) > sl.local;
        // the first point (of this eigenvalue's 16) with more than `local`
        // eigenvalues below it bounds the eigenvalue from above
        const unsigned long long b = __ballot(above);
        const unsigned row = (unsigned)(b >> ((lane / kMS) * kMS)) & ((1u << kMS) - 1u);
        const int first = row ? __ffs(row) - 1 : kMS;
        const float nlo = first == 0 ? lo : lo + (hi - lo) * (float)first / (float)(kMS + 1);
        const float nhi = first == kMS ? hi : lo + (hi - lo) * (float)(first + 1) / (float)(kMS + 1);
        lo = nlo;
        hi = nhi;
        if (hi - lo <= 2.0f * FLT_EPSILON * fmaxf(fabsf(lo), fabsf(hi)) + pivmin) break;   // uniform per 16 lanes
    }
    if (live && j == 0) lam[sidx] = 0.5f * (lo + hi);
}

// ---- eigenvectors: inverse iteration ----

struct Cluster {         // consecutive slots of one block, close together
    int start, size;     // the block
    int first, count;    // slots first .. first + count - 1
};


// One thread per cluster.  Z[r * ldz + slot] holds the vectors (rows of
// the block; the thread also zeroes the rest of its columns).  U is scratch
// for the factor: 3 floats per row, [3 * row][thread] (coalesced).
__global__ __launch_bounds__(64) void inverse_iteration_kernel(const float* __restrict__ d,
                                                                const float* __restrict__ e,
                                                                const Cluster* __restrict__ cl, int ncl,
                                                                const float* __restrict__ lam, float tnorm,
                                                                float* __restrict__ Z, int ldz, int n,
                                                                float* __restrict__ U) {
    const int tid = blockIdx.x * 64 + threadIdx.x;
    if (tid >= ncl) return;
    const Cluster c = cl[tid];
    const int s = c.start, m = c.size;
    float* u0 = U + tid;            // U[(3 r + 0) * ncl + tid]
    const size_t us = (size_t)ncl;
    const float tol = FLT_EPSILON * tnorm;   // a zero pivot becomes this
    for (int q = 0; q < c.count; ++q) {
        const int slot = c.first + q;
        float* z = Z + slot;        // z[r * ldz]
        // zero outside the block
        for (int r = 0; r < s; ++r) z[(size_t)r * ldz] = 0.0f;
        for (int r = s + m; r < n; ++r) z[(size_t)r * ldz] = 0.0f;
        if (m == 1) {
            z[(size_t)s * ldz] = 1.0f;
            continue;
        }
        const float lambda = lam[slot];
        for (int r = 0; r < m; ++r) z[(size_t)(s + r) * ldz] = hash_uniform((unsigned)slot, (unsigned)r);
        for (int it = 0; it < kIters; ++it) {
            // forward: factor (T - lambda I) = P L U on the fly, apply P, L to
            // z.  Rows move in chunks of CH: all of a chunk's loads are issued
            // before its recurrence runs.
            float a = d[s] - lambda;         // the running diagonal entry of row k
            float cc = e[s];                 // row k's superdiagonal
            float b0 = z[(size_t)s * ldz];   // the running right-hand side of row k
            // chunk loads run one chunk ahead of the recurrence (the next
            // chunk's rows are never the ones this chunk writes)
            float zb[CH], db[CH], eb[CH], en[CH];
            auto load_fwd = [&](int k0, float (&zl)[CH], float (&dl)[CH], float (&el)[CH], float (&nl)[CH]) {
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    const int k = min(k0 + j, m - 2);
                    zl[j] = z[(size_t)(s + k + 1) * ldz];
                    dl[j] = d[s + k + 1];
                    el[j] = e[s + k];
                    nl[j] = k + 1 < m - 1 ? e[s + k + 1] : 0.0f;
                }
            };
            load_fwd(0, zb, db, eb, en);
            for (int k0 = 0; k0 < m - 1; k0 += CH) {
                float zn[CH], dn[CH], ebn[CH], enn[CH];
                load_fwd(k0 + CH < m - 1 ? k0 + CH : k0, zn, dn, ebn, enn);
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const int k = k0 + c;
                    if (k >= m - 1) break;
                    const float bk = eb[c];
                    const float an = db[c] - lambda;
                    const float cn = en[c];
                    const float b1 = zb[c];
                    const bool keep = fabsf(a) >= fabsf(bk);
                    float p0 = keep ? a : bk;
                    // pivots below tol (zero, or subnormal) become +-tol
                    p0 = fabsf(p0) < tol ? copysignf(tol, p0) : p0;
                    const float r0 = __builtin_amdgcn_rcpf(p0);
                    const float l = (keep ? bk : a) * r0;
                    const float p1 = keep ? cc : an;
                    const float p2 = keep ? 0.0f : cn;
                    const float rhs = keep ? b0 : b1;
                    const float na = keep ? fmaf(-l, cc, an) : fmaf(-l, an, cc);
                    const float nc = keep ? cn : -l * cn;
                    const float nb0 = keep ? fmaf(-l, b0, b1) : fmaf(-l, b1, b0);
                    u0[(3 * (size_t)k + 0) * us] = r0;   // the backward pass multiplies
                    u0[(3 * (size_t)k + 1) * us] = p1;
                    u0[(3 * (size_t)k + 2) * us] = p2;
                    z[(size_t)(s + k) * ldz] = rhs;
                    a = na;
                    cc = nc;
                    b0 = nb0;
                }
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    zb[c] = zn[c];
                    db[c] = dn[c];
                    eb[c] = ebn[c];
                    en[c] = enn[c];
                }
            }
            a = fabsf(a) < tol ? copysignf(tol, a) : a;
            // backward: U x = rhs, and |x|^2, in chunks from the bottom
            float x2 = 0.0f, x1 = 0.0f, nrm = 0.0f;
            {
                const float x = b0 / a;
                z[(size_t)(s + m - 1) * ldz] = x;
                x1 = x;
                nrm = x * x;
            }
            for (int k1 = m - 2; k1 >= 0; k1 -= CH) {
                float r0[CH], r1[CH], r2[CH], rz[CH];
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const int k = max(k1 - c, 0);
                    r0[c] = u0[(3 * (size_t)k + 0) * us];
                    r1[c] = u0[(3 * (size_t)k + 1) * us];
                    r2[c] = u0[(3 * (size_t)k + 2) * us];
                    rz[c] = z[(size_t)(s + k) * ldz];
                }
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const int k = k1 - c;
                    if (k < 0) break;
                    const float x = (rz[c] - r1[c] * x1 - r2[c] * x2) * r0[c];
                    z[(size_t)(s + k) * ldz] = x;
                    x2 = x1;
                    x1 = x;
                    nrm = fmaf(x, x, nrm);
                }
            }
            // against the cluster's earlier vectors (modified Gram-Schmidt)
            for (int p = 0; p < q; ++p) {
                const float* zp = Z + c.first + p;
                float dot = 0.0f;
                for (int r = 0; r < m; ++r) dot = fmaf(zp[(size_t)(s + r) * ldz], z[(size_t)(s + r) * ldz], dot);
                nrm = 0.0f;
                for (int r = 0; r < m; ++r) {
                    const float x = fmaf(-dot, zp[(size_t)(s + r) * ldz], z[(size_t)(s + r) * ldz]);
                    z[(size_t)(s + r) * ldz] = x;
                    nrm = fmaf(x, x, nrm);
                }
            }
            const float inv = nrm > 0.0f ? 1.0f / sqrtf(nrm) : 0.0f;
            for (int r0 = 0; r0 < m; r0 += CH) {
                float x[CH];
#pragma unroll
                for (int c = 0; c < CH; ++c) x[c] = z[(size_t)(s + min(r0 + c, m - 1)) * ldz];
#pragma unroll
                for (int c = 0; c < CH; ++c)
                    if (r0 + c < m) z[(size_t)(s + r0 + c) * ldz] = x[c] * inv;
            }
        }
    }
}

// M = (3 I - G) / 2
__global__ __launch_bounds__(256) void newton_schulz_kernel(float* __restrict__ G, int n) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (size_t)i * n);
    G[idx] = (i == j ? 1.5f : 0.0f) - 0.5f * G[idx];
}

// T (nb x nb, upper, row-major) of the compact WY form of nb reflectors
// from S = V^T V (nb x nb, symmetric) and tau: T[k][k] = tau_k,
// T[0:k, k] = -tau_k T[0:k, 0:k] S[0:k, k].  Row t of T depends only on row
// t's earlier entries and on S, so each of the 64 threads builds its own row
// in registers (every index compile-time, no barrier between columns),
// reading S's rows (= columns) as float4 broadcasts from LDS.
__global__ __launch_bounds__(64) void wy_t_kernel(const float* __restrict__ S, const float* __restrict__ tau, int nb,
                                                  float* __restrict__ T) {
    __shared__ float Ss[NBT][NBT + 4];
    __shared__ float ts[NBT];
    const int t = threadIdx.x;
    for (int i0 = 0; i0 < NBT; i0 += 16) {
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = i0 + u;
            const bool in = i < nb && t < nb;
            x[u] = S[in ? i * nb + t : 0];
            x[u] = in ? x[u] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) Ss[i0 + u][t] = x[u];
    }
    ts[t] = t < nb ? tau[t] : 0.0f;
    __syncthreads();
    float tr[NBT];   // row t of T; entries left of the diagonal stay 0
#pragma unroll
    for (int k = 0; k < NBT; ++k) {
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int l0 = 0; l0 < k; l0 += 4) {
            const float4 sv = *reinterpret_cast<const float4*>(&Ss[k][l0]);
            s0 = fmaf(tr[l0], sv.x, s0);
            if (l0 + 1 < k) s1 = fmaf(tr[l0 + 1], sv.y, s1);
            if (l0 + 2 < k) s2 = fmaf(tr[l0 + 2], sv.z, s2);
            if (l0 + 3 < k) s3 = fmaf(tr[l0 + 3], sv.w, s3);
        }
        const float tk = ts[k];
        tr[k] = t < k ? -tk * ((s0 + s1) + (s2 + s3)) : (t == k ? tk : 0.0f);
    }
    if (t < nb) {
#pragma unroll
        for (int k = 0; k < NBT; ++k)
            if (k < nb) T[t * nb + k] = tr[k];
    }
}

// out[i][j] = Z[i][perm[j]]; w[j] = lam[perm[j]] 2^e
// V (n x cols) column j = Z (n x n) column perm[j]
__global__ __launch_bounds__(256) void permute_columns_kernel(const float* __restrict__ Z, float* __restrict__ V,
                                                              const int* __restrict__ perm, int n, int cols) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n * cols) return;
    const int i = (int)(idx / cols), j = (int)(idx - (size_t)i * cols);
    V[idx] = Z[(size_t)i * n + perm[j]];
}

__global__ __launch_bounds__(256) void permute_values_kernel(const float* __restrict__ lam, float* __restrict__ w,
                                                             const int* __restrict__ perm, int n,
                                                             const uint32_t* __restrict__ flags) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const int e = scale_exponent(__uint_as_float(flags[0]));
    w[j] = ldexpf(lam[perm[j]], e);
}

__global__ __launch_bounds__(256) void fill_nan_kernel(float* __restrict__ x, size_t count) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) x[i] = qnan();
}

// out[i] = sum over b of part[b count + i], in order of b; eight partials in
// flight at a time (indices past the last read it again and add zero)
__global__ __launch_bounds__(256) void sum_parts2_kernel(const float* __restrict__ part, int nsplit, size_t count,
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

__global__ void set_info_kernel(uint32_t* info, const uint32_t* flags) {
    *info = flags[1] ? (1u << 17) : (1u | (1u << 16));
}

unsigned grid_of(size_t count) { return (unsigned)std::min<size_t>(cdiv(count, 256), 4096); }

constexpr int kRowChunk = 128;   // rows of a split-K chunk: the small-K GEMM's whole K

// C (M x N) = A B over a long K, split in chunks summed afterwards (the
// products with V^T over many rows): A M x K (row-major, lda); B K x N
// (ldb), or with tb stored N x K
void split_rows_gemm(bool tb, int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* part,
                     float* C, hipStream_t s) {
    // one batched launch over chunks of kRowChunk rows of the sum (the last
    // one shorter), then the partials added in order
    const int nsplit = (K + kRowChunk - 1) / kRowChunk;
    const int last = K - (nsplit - 1) * kRowChunk;
    const long long sb = tb ? kRowChunk : (long long)kRowChunk * ldb;
    sgemm(false, tb, M, N, kRowChunk, 1.0f, A, lda, kRowChunk, B, ldb, sb, 0.0f, part, N, (long long)M * N, nsplit, s,
          false, last);
    hipLaunchKernelGGL(sum_parts2_kernel, dim3(grid_of((size_t)M * N)), dim3(256), 0, s, part, nsplit, (size_t)M * N,
                       C);
}

}  // namespace

size_t apply_reflectors_wy_floats(int rows, int cols) {
    const size_t nsplit = (rows + kRowChunk - 1) / kRowChunk;
    const size_t wide = std::max(cols, NBT);
    return nsplit * NBT * wide + 2 * (size_t)NBT * wide + 2 * (size_t)NBT * NBT + 4 * 64;
}

// Z (rows x cols, row-major) <- H_0 H_1 ... H_{nrefl-1} Z, H_j = I - tau_j v_j
// v_j^T, v_j stored as row j of V (stride ldv, `rows` entries, zero before
// its leading 1); panels of NBT reflectors from the last, each in compact WY
// form: S = V^T V, T from S and tau (wy_t_kernel), Z2 -= V (T (V^T Z2)),
// the products on the MFMA GEMM.  Rows before the panel's first reflector
// are zero in all of its reflectors and are left out.
void apply_reflectors_wy(const float* V, int ldv, const float* tau, int nrefl, int rows, float* Z, int cols,
                         float* work, hipStream_t s) {
    if (nrefl <= 0 || cols <= 0) return;
    const size_t nsplit = (rows + kRowChunk - 1) / kRowChunk;
    const size_t wide = std::max(cols, NBT);
    float* part = work;
    float* Wb = part + nsplit * NBT * wide;
    float* W2 = Wb + (size_t)NBT * wide;
    float* Sg = W2 + (size_t)NBT * wide;
    float* Tg = Sg + (size_t)NBT * NBT;
    for (int j0 = (nrefl - 1) / NBT * NBT; j0 >= 0; j0 -= NBT) {
        const int nb = std::min(NBT, nrefl - j0);
        const int r = rows - j0;
        const float* Vp = V + (size_t)j0 * ldv + j0;   // reflector k: Vp[k * ldv + i], i = row - j0
        float* Z2 = Z + (size_t)j0 * cols;
        split_rows_gemm(true, nb, nb, r, Vp, ldv, Vp, ldv, part, Sg, s);
        hipLaunchKernelGGL(wy_t_kernel, dim3(1), dim3(64), 0, s, Sg, tau + j0, nb, Tg);
        split_rows_gemm(false, nb, cols, r, Vp, ldv, Z2, cols, part, Wb, s);
        sgemm(false, false, nb, cols, nb, 1.0f, Tg, nb, 0, Wb, cols, 0, 0.0f, W2, cols, 0, 1, s);
        sgemm(true, false, r, cols, nb, -1.0f, Vp, ldv, 0, W2, cols, 0, 1.0f, Z2, cols, 0, 1, s);
    }
}

size_t eigh_tridiag_floats(uint32_t n) {
    const size_t N = n;
    // lam, e2, slots/clusters (as floats), perm; Z; scratch (G, inverse
    // iteration's factor: 3 N per cluster); the back-transform's partials
    return 4 * N + 12 * N + N * N + N + 3 * N * N + apply_reflectors_wy_floats((int)N, (int)N) + 64 * 16;
}

// Stages 2 and 3 on one matrix after sytrd_one: w_out (n), and if v_out
// V (n x n) with the eigenvectors as columns; info.
void eigh_tridiag_one(const EighWork& w, uint32_t nn, float* w_out, float* v_out, uint32_t* info, hipStream_t s,
                      bool backtransform, uint32_t il) {
    const int n = (int)nn;
    const size_t N = nn;
    const int nw = n - (int)il;   // eigenvectors wanted: those of eigenvalues il .. n-1
    float* p = w.rest;
    auto take = [&](size_t c) {
        float* r = p;
        p += (c + 63) / 64 * 64;
        return r;
    };
    float* lam = take(N);
    float* e2 = take(N);
    Slot* slots = reinterpret_cast<Slot*>(take(6 * N));
    Cluster* clusters = reinterpret_cast<Cluster*>(take(4 * N));
    int* perm = reinterpret_cast<int*>(take(N));
    float* Z = take(N * N);
    float* dE = take(N);                 // e with the splits zeroed
    float* scratch = take(3 * N * N);    // inverse iteration's factor, then Z^T Z
    float* part = take(apply_reflectors_wy_floats(n, n));   // the back-transform's products

    hipLaunchKernelGGL(set_info_kernel, dim3(1), dim3(1), 0, s, info, w.flags);
    // the small host-side bookkeeping: T's entries, the splits and Gershgorin
    // intervals, the clusters and the final order
    std::vector<float> hd(N), he(N > 1 ? N - 1 : 1);
    uint32_t hflags[2];
    MLA_HIP(hipMemcpyAsync(hd.data(), w.d, N * sizeof(float), hipMemcpyDeviceToHost, s));
    if (n > 1) MLA_HIP(hipMemcpyAsync(he.data(), w.e, (N - 1) * sizeof(float), hipMemcpyDeviceToHost, s));
    MLA_HIP(hipMemcpyAsync(hflags, w.flags, sizeof(hflags), hipMemcpyDeviceToHost, s));
    MLA_HIP(hipStreamSynchronize(s));
    if (hflags[1]) {   // a non-finite entry: all NaN
        hipLaunchKernelGGL(fill_nan_kernel, dim3(grid_of(N)), dim3(256), 0, s, w_out, N);
        if (v_out) hipLaunchKernelGGL(fill_nan_kernel, dim3(grid_of(N * nw)), dim3(256), 0, s, v_out, N * nw);
        MLA_HIP(hipGetLastError());
        return;
    }
    std::vector<float> he2(N, 0.0f);
    float tnorm = 0.0f, emax2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float off = (i > 0 ? std::fabs(he[i - 1]) : 0.0f) + (i + 1 < n ? std::fabs(he[i]) : 0.0f);
        tnorm = std::max(tnorm, std::fabs(hd[i]) + off);
    }
    // splits (sstebz): e_i^2 <= eps^2 |d_i d_{i+1}|
    std::vector<int> bstart;
    bstart.push_back(0);
    for (int i = 0; i + 1 < n; ++i) {
        const float ee = he[i] * he[i];
        const bool split = ee <= FLT_EPSILON * FLT_EPSILON * std::fabs(hd[i] * hd[i + 1]) || he[i] == 0.0f;
        he2[i] = split ? 0.0f : ee;
        if (split) {
            he[i] = 0.0f;
            bstart.push_back(i + 1);
        }
        emax2 = std::max(emax2, he2[i]);
    }
    bstart.push_back(n);
    const float pivmin = FLT_MIN * std::max(1.0f, emax2);
    std::vector<Slot> hs(N);
    for (size_t b = 0; b + 1 < bstart.size(); ++b) {
        const int s0 = bstart[b], m = bstart[b + 1] - s0;
        float gl = FLT_MAX, gu = -FLT_MAX;
        for (int i = s0; i < s0 + m; ++i) {
            const float off = (i > s0 ? std::fabs(he[i - 1]) : 0.0f) + (i + 1 < s0 + m ? std::fabs(he[i]) : 0.0f);
            gl = std::min(gl, hd[i] - off);
            gu = std::max(gu, hd[i] + off);
        }
        const float pad = 2.0f * FLT_EPSILON * std::max(std::fabs(gl), std::fabs(gu)) * m + 2.0f * pivmin;
        for (int k = 0; k < m; ++k) hs[s0 + k] = Slot{s0, m, k, 0, gl - pad, gu + pad};
    }
    MLA_HIP(hipMemcpyAsync(e2, he2.data(), N * sizeof(float), hipMemcpyHostToDevice, s));
    MLA_HIP(hipMemcpyAsync(slots, hs.data(), N * sizeof(Slot), hipMemcpyHostToDevice, s));
    {
        KernelTimer tm("tridiag_values", s);
        hipLaunchKernelGGL(multisection_kernel, dim3((unsigned)cdiv(n, 256 / kMS)), dim3(256), 0, s, w.d, e2, slots,
                           n, pivmin, lam);
        tm.stop();
    }
    std::vector<float> hl(N);
    MLA_HIP(hipMemcpyAsync(hl.data(), lam, N * sizeof(float), hipMemcpyDeviceToHost, s));
    MLA_HIP(hipStreamSynchronize(s));
    std::vector<int> hp(N);
    std::iota(hp.begin(), hp.end(), 0);
    std::stable_sort(hp.begin(), hp.end(), [&](int a, int b) { return hl[a] < hl[b]; });
    MLA_HIP(hipMemcpyAsync(perm, hp.data(), N * sizeof(int), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(permute_values_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, lam, w_out, perm, n,
                       w.flags);
    if (!v_out) {
        MLA_HIP(hipStreamSynchronize(s));   // the host vectors above must outlive the copies
        MLA_HIP(hipGetLastError());
        return;
    }

    // clusters: consecutive eigenvalues of a block within 1e-5 ||T||; only
    // those holding a wanted eigenvalue (rank il or above) are solved, each
    // whole (its members are orthogonalised together)
    std::vector<int> rank(N);
    for (int r = 0; r < n; ++r) rank[hp[r]] = r;
    std::vector<Cluster> hc;
    const float ctol = 1e-5f * tnorm;
    for (size_t b = 0; b + 1 < bstart.size(); ++b) {
        const int s0 = bstart[b], m = bstart[b + 1] - s0;
        int k = 0;
        while (k < m) {
            int c = 1;
            while (k + c < m && hl[s0 + k + c] - hl[s0 + k + c - 1] <= ctol) ++c;
            bool want = false;
            for (int q = 0; q < c; ++q) want |= rank[s0 + k + q] >= (int)il;
            if (want) hc.push_back(Cluster{s0, m, s0 + k, c});
            k += c;
        }
    }
    const int ncl = (int)hc.size();
    MLA_HIP(hipMemcpyAsync(clusters, hc.data(), ncl * sizeof(Cluster), hipMemcpyHostToDevice, s));
    MLA_HIP(hipMemcpyAsync(dE, he.data(), (N - 1) * sizeof(float), hipMemcpyHostToDevice, s));
    float* U = scratch;
    {
        KernelTimer tm("tridiag_vectors", s);
        if (ncl > 0)
            hipLaunchKernelGGL(inverse_iteration_kernel, dim3((unsigned)cdiv(ncl, 64)), dim3(64), 0, s, w.d, dE,
                               clusters, ncl, lam, tnorm, Z, n, n, U);
        // the wanted columns in ascending order, Zs = Z[:, perm[il ..]]
        // (n x nw), then one Newton-Schulz step Zs <- Zs (3 I - Zs^T Zs) / 2
        // into v_out
        float* Zs = scratch;
        float* G = scratch + N * nw;
        hipLaunchKernelGGL(permute_columns_kernel, dim3((unsigned)cdiv(N * nw, 256)), dim3(256), 0, s, Z, Zs,
                           perm + il, n, nw);
        sgemm(true, false, nw, nw, n, 1.0f, Zs, nw, 0, Zs, nw, 0, 0.0f, G, nw, 0, 1, s);
        hipLaunchKernelGGL(newton_schulz_kernel, dim3((unsigned)cdiv((size_t)nw * nw, 256)), dim3(256), 0, s, G, nw);
        sgemm(false, false, n, nw, nw, 1.0f, Zs, nw, 0, G, nw, 0, 0.0f, v_out, nw, 0, 1, s);
        tm.stop();
    }
    // V = Q Z: panels from the last, Z2 = Z[j0 + 1 :, :] -= V (T (V^T Z2))
    // (row j0 is zero in every reflector of the panel, kept so that the
    // operands stay 16-byte aligned)
    if (backtransform) {
        KernelTimer tm("eigh_backtransform", s);
        apply_reflectors_wy(w.V, n, w.tau, n - 1, n, v_out, nw, part, s);
        tm.stop();
    }
    MLA_HIP(hipStreamSynchronize(s));   // the host vectors above must outlive the copies
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
