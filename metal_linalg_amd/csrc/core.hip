// The buffer core: argument shapes to kernels.  Every decomposition runs on
// the GPU; host buffers are staged by mla::Call.
#include "core.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "policy.hpp"
#include "runtime.hpp"

namespace mla {

namespace {
thread_local bool tls_cpu_only = false;
}

bool cpu_only() { return tls_cpu_only; }
void set_cpu_only(bool on) { tls_cpu_only = on; }

void require_gpu_allowed(const char* what) {
    if (tls_cpu_only)
        throw std::runtime_error(std::string("[") + what +
                                 "] CPU-only is set on this thread, and this build of metal_linalg has no CPU path");
}

}  // namespace mla

namespace mla::core {

namespace {

float* f32(void* p) { return static_cast<float*>(p); }
uint32_t* u32p(void* p) { return static_cast<uint32_t*>(p); }

__global__ void fill_identity_kernel(float* q, uint64_t batch, uint32_t m) {
    const uint64_t per = (uint64_t)m * m;
    const uint64_t total = batch * per;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t k = i % per;
        q[i] = (k / m == k % m) ? 1.0f : 0.0f;
    }
}

}  // namespace

// reference: src/qr.mm:310-327 (core::qr) with the kernel choice by shape
void qr(const Matrices& a, float* q, float* r, QrMode mode) {
    require_gpu_allowed("qr");
    const uint32_t M = a.rows, N = a.cols, K = std::min(M, N), B = a.batch;
    const uint32_t QC = qr_q_cols(mode, M, N), RR = qr_r_rows(mode, M, N);
    if (mode == QrMode::complete && N == 0 && q && B && M) {   // nothing to factor: Q = I (qr.mm:312-317)
        Call call;
        float* dq = call.out(q, (size_t)B * M * M);
        const uint64_t total = (uint64_t)B * M * M;
        const uint32_t blocks = (uint32_t)std::min<uint64_t>(cdiv(total, 256), 65536);
        hipLaunchKernelGGL(fill_identity_kernel, dim3(blocks), dim3(256), 0, call.stream(), dq, (uint64_t)B, M);
        call.finish();
        return;
    }
    if (K == 0 || B == 0) return;
    const bool small = qr_small_fits(M, N, QC);
    // tall matrices of at most 64 columns: the batched tall kernel (a tree
    // of 128-row blocks past 128 rows)
    const bool tall = !small && qr_tall_fits(M, N, QC);
    // up to 128 rows and columns (one of them above 64): two waves a matrix
    const bool mid = !small && !tall && qr_mid_fits(M, N, QC);
    // beyond the blocked QR's 4096 rows: a tree of blocked QRs, to 2048 columns
    const bool tree = !small && !tall && !mid && !qr_blocked_fits(M, N) && qr_tsqr_fits(M, N, QC);
    if (!small && !tall && !mid && !tree && !qr_blocked_fits(M, N))
        invalid("[qr] " + std::to_string(M) + "x" + std::to_string(N) + (mode == QrMode::complete ? " complete" : "") +
                ": this build's QR kernels take at most 4096 rows beyond 64 columns, or any number of rows "
                "with at most 2048 columns (reduced or R only)");
    Call call;
    if (tree) {
        const size_t per = (size_t)M * N;
        const float* da = call.in(a.data, (size_t)B * per);
        float* dq = QC ? call.out(q, (size_t)B * per) : nullptr;
        float* dr = call.out(r, (size_t)B * N * N);
        float* work = static_cast<float*>(call.scratch(qr_tsqr_workspace(M, N, QC != 0)));
        for (uint32_t b = 0; b < B; ++b)
            qr_tsqr_one(da + b * per, dq ? dq + b * per : nullptr, dr + (size_t)b * N * N, M, N, work, call.stream());
        call.finish();
        return;
    }
    if (small || tall || mid) {
        const std::vector<Call::Slice> sl = {{a.data, nullptr, (size_t)M * N * 4},
                                             {nullptr, QC ? q : nullptr, (size_t)M * QC * 4},
                                             {nullptr, r, (size_t)RR * N * 4}};
        const size_t wsb = tall ? qr_tall_workspace(M, N, call.chunk_size(B, sl), QC != 0) : 0;
        float* ws = wsb ? static_cast<float*>(call.scratch(wsb)) : nullptr;
        call.batched(B, sl, [&](void* const* d, uint32_t nb, hipStream_t s) {
            if (small) qr_small(f32(d[0]), f32(d[1]), f32(d[2]), nb, M, N, QC, RR, s);
            else if (tall) qr_tall(f32(d[0]), f32(d[1]), f32(d[2]), nb, M, N, ws, s);
            else qr_mid(f32(d[0]), f32(d[1]), f32(d[2]), nb, M, N, s);
        });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * M * N);
    float* dq = QC ? call.out(q, (size_t)B * M * QC) : nullptr;
    float* dr = call.out(r, (size_t)B * RR * N);
    float* work = static_cast<float*>(call.scratch(qr_blocked_workspace(M, N)));
    qr_blocked(da, dq, dr, B, M, N, QC, RR, work, call.stream());
    call.finish();
}

namespace {

// A finite matrix that did not converge is an error (reference:
// src/eigh_ql.mm:254-262, src/svd_golub_kahan.mm:349-362): the info words
// are read back and checked.
void check_converged_host(const uint32_t* h, uint32_t batch, const char* what) {
    for (uint32_t b = 0; b < batch; ++b) {
        const uint32_t i = h[b];
        if (!((i >> 17) & 1u) && !((i >> 16) & 1u))
            throw std::runtime_error(std::string("[") + what + "] matrix " + std::to_string(b) + " of " +
                                     std::to_string(batch) + " did not converge (" + std::to_string(i & 0xFFFFu) +
                                     " iterations).");
    }
}

void check_converged(const uint32_t* dinfo, uint32_t batch, hipStream_t s, const char* what) {
    std::vector<uint32_t> h(batch);
    MLA_HIP(hipMemcpyAsync(h.data(), dinfo, (size_t)batch * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    MLA_HIP(hipStreamSynchronize(s));
    check_converged_host(h.data(), batch, what);
}

}  // namespace

// reference: src/eigh.mm:911-958 (core::eigh)
void eigh(const Matrices& a, bool lower, float* w, float* v, uint32_t* info) {
    require_gpu_allowed("eigh");
    if (a.rows != a.cols) invalid("[eigh] Input matrices must be square.");
    const uint32_t n = a.cols, B = a.batch;
    if (B == 0) return;
    if (n == 0) {
        if (info) {
            Call call;
            uint32_t* di = call.out(info, B);
            MLA_HIP(hipMemsetAsync(di, 0, (size_t)B * sizeof(uint32_t), call.stream()));
            call.finish();
        }
        return;
    }
    const bool small = eigh_small_fits(n);
    const bool mid = eigh_mid_fits(n);
    if (!small && !mid && !eigh_blocked_fits(n))
        invalid("[eigh] n = " + std::to_string(n) + ": this build's eigh kernels take n <= 16384");
    Call call;
    if (small || mid) {
        // no convergence read-back: bisection always ends (every info word
        // carries bit 16, or bit 17 for a non-finite matrix), so the
        // reference's non-convergence error cannot arise on this path
        const std::vector<Call::Slice> sl = {{a.data, nullptr, (size_t)n * n * 4},
                                             {nullptr, w, (size_t)n * 4},
                                             {nullptr, v, v ? (size_t)n * n * 4 : 0},
                                             {nullptr, info, 4}};
        const uint32_t chunk = call.chunk_size(B, sl);
        const size_t wsb = small ? eigh_small_workspace(n, chunk, v != nullptr) : eigh_mid_workspace(n, chunk, v != nullptr);
        float* ws = wsb ? static_cast<float*>(call.scratch(wsb)) : nullptr;
        call.batched(B, sl, [&](void* const* d, uint32_t nb, hipStream_t s) {
            if (small) eigh_small(f32(d[0]), f32(d[1]), f32(d[2]), u32p(d[3]), nb, n, lower, ws, s);
            else eigh_mid(f32(d[0]), f32(d[1]), f32(d[2]), u32p(d[3]), nb, n, lower, ws, s);
        });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    float* dw = call.out(w, (size_t)B * n);
    float* dv = v ? call.out(v, (size_t)B * n * n) : nullptr;
    uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
    {
        const size_t floats = eigh_sytrd_floats(n) + eigh_tridiag_floats(n);
        float* work = static_cast<float*>(call.scratch(floats * sizeof(float)));
        const EighWork ew = eigh_carve(work, n);
        const size_t per = (size_t)n * n;
        for (uint32_t b = 0; b < B; ++b) {
            sytrd_one(da + b * per, n, lower, ew, call.stream());
            eigh_tridiag_one(ew, n, dw + (size_t)b * n, dv ? dv + b * per : nullptr, di + b, call.stream());
        }
    }
    call.finish();
}

namespace {

// dst[b] (cols x rows) = src[b]^T (rows x cols), through 32 x 32 LDS tiles
__global__ __launch_bounds__(256) void batch_transpose_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                              int rows, int cols) {
    __shared__ float tile[32][33];
    const size_t per = (size_t)rows * cols;
    const float* S = src + blockIdx.z * per;
    float* D = dst + blockIdx.z * per;
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = S[(size_t)(r0 + r) * cols + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 32; c += 8)
        if (c0 + c < cols && r0 + tx < rows) D[(size_t)(c0 + c) * rows + r0 + tx] = tile[tx][c];
}

void batch_transpose(const float* src, float* dst, uint32_t batch, uint32_t rows, uint32_t cols, hipStream_t s) {
    for (uint32_t b0 = 0; b0 < batch; b0 += 65535) {
        const uint32_t nb = std::min<uint32_t>(65535, batch - b0);
        const size_t off = (size_t)b0 * rows * cols;
        hipLaunchKernelGGL(batch_transpose_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32), nb),
                           dim3(256), 0, s, src + off, dst + off, (int)rows, (int)cols);
    }
}

// Thin SVD of matrices with min(M, N) = K <= 64 beyond the batched kernel's
// 128 rows: the tall problem A = Q R (the batched tall QR), the SVD of the
// K x K factor R = U_R S V^T (batched kernel), then U = Q U_R (MFMA GEMM).
// A wide matrix is solved as its transpose.  Non-finite input reaches R as
// NaN and gives NaN outputs with info bit 17; the flag bits and sweep counts
// are those of R's SVD, which has A's singular values and right vectors.
// The reference's tall route is the same factorisation on its CPU path
// (src/svd.mm:772-890: sgeqrf, sgesdd on R, U = Q U_R).
void svd_tall(const Matrices& a, float* u, float* s, float* vt, uint32_t* info) {
    const uint32_t M = a.rows, N = a.cols, B = a.batch;
    const bool wide = M < N;
    const uint32_t m = wide ? N : M, k = wide ? M : N;   // the tall problem: m x k
    const bool vec = u != nullptr;
    Call call;
    hipStream_t st = call.stream();
    const float* da = call.in(a.data, (size_t)B * M * N);
    float* ds = call.out(s, (size_t)B * k);
    float* du = vec ? call.out(u, (size_t)B * M * k) : nullptr;
    float* dvt = vec ? call.out(vt, (size_t)B * k * N) : nullptr;
    uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
    const float* tall = da;
    if (wide) {
        float* at = call.tmp<float>((size_t)B * m * k);
        batch_transpose(da, at, B, M, N, st);
        tall = at;
    }
    float* q = vec ? call.tmp<float>((size_t)B * m * k) : nullptr;
    float* r = call.tmp<float>((size_t)B * k * k);
    const size_t qwb = qr_tall_workspace(m, k, B, vec);
    float* qw = qwb ? static_cast<float*>(call.scratch(qwb)) : nullptr;
    qr_tall(tall, q, r, B, m, k, qw, st);
    float* ur = vec ? call.tmp<float>((size_t)B * k * k) : nullptr;
    // right vectors of the tall problem: A's V^T, or (wide) A's U transposed
    float* vtt = !vec ? nullptr : wide ? call.tmp<float>((size_t)B * k * k) : dvt;
    float* ws = static_cast<float*>(call.scratch(svd_small_workspace(k, k, B)));
    svd_small(r, ur, ds, vtt, di, ws, B, k, k, st);
    if (vec) {
        // left vectors of the tall problem, m x k: Q U_R
        float* ut = wide ? call.tmp<float>((size_t)B * m * k) : du;
        sgemm(false, false, (int)m, (int)k, (int)k, 1.0f, q, (int)k, (long long)m * k, ur, (int)k, (long long)k * k,
              0.0f, ut, (int)k, (long long)m * k, (int)B, st);
        if (wide) {
            batch_transpose(ut, dvt, B, m, k, st);    // A's V^T (k x N) = (Q U_R)^T
            batch_transpose(vtt, du, B, k, k, st);    // A's U (M x k) = V_R
        }
    }
    check_converged(di, B, st, "svd");
    call.finish();
}

}  // namespace

// reference: src/svd.mm:1058-1106 (core::svd)
void svd(const Matrices& a, float* u, float* s, float* vt, uint32_t* info) {
    require_gpu_allowed("svd");
    const uint32_t M = a.rows, N = a.cols, K = std::min(M, N), B = a.batch;
    if (B == 0) return;
    if (K == 0) {
        if (info) {
            Call call;
            uint32_t* di = call.out(info, B);
            MLA_HIP(hipMemsetAsync(di, 0, (size_t)B * sizeof(uint32_t), call.stream()));
            call.finish();
        }
        return;
    }
    if (!svd_small_fits(M, N) && svd_mid_fits(M, N)) {
        Call call;
        uint32_t* ibuf = info ? info : call.tmp<uint32_t>(B);
        const std::vector<Call::Slice> sl = {{a.data, nullptr, (size_t)M * N * 4},
                                             {nullptr, u, u ? (size_t)M * K * 4 : 0},
                                             {nullptr, s, (size_t)K * 4},
                                             {nullptr, vt, vt ? (size_t)K * N * 4 : 0},
                                             {nullptr, ibuf, 4}};
        call.batched(B, sl, [&](void* const* d, uint32_t nb, hipStream_t st) {
            svd_mid(f32(d[0]), f32(d[1]), f32(d[2]), f32(d[3]), u32p(d[4]), nb, M, N, st);
        });
        if (is_device_memory(ibuf)) check_converged(ibuf, B, call.stream(), "svd");
        else check_converged_host(ibuf, B, "svd");
        call.finish();
        return;
    }
    if (!svd_small_fits(M, N)) {
        if (K <= 64) {
            svd_tall(a, u, s, vt, info);
            return;
        }
        if (!svd_large_fits(M, N))
            invalid("[svd] " + std::to_string(M) + "x" + std::to_string(N) +
                    ": this build's SVD kernels take min(M, N) <= 64 at any length, max(M, N) <= 4096, or "
                    "min(M, N) <= 2048 beyond");
        Call call;
        const size_t per = (size_t)M * N;
        const float* da = call.in(a.data, (size_t)B * per);
        float* ds = call.out(s, (size_t)B * K);
        float* du = u ? call.out(u, (size_t)B * M * K) : nullptr;
        float* dvt = vt ? call.out(vt, (size_t)B * K * N) : nullptr;
        uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
        float* work = static_cast<float*>(call.scratch(svd_large_workspace(M, N)));
        for (uint32_t b = 0; b < B; ++b)
            svd_large_one(da + b * per, du ? du + (size_t)b * M * K : nullptr, ds + (size_t)b * K,
                          dvt ? dvt + (size_t)b * K * N : nullptr, di + b, work, M, N, call.stream());
        call.finish();
        return;
    }
    Call call;
    // the info words are read back for the convergence check: the caller's
    // array (host or device) or a device one
    uint32_t* ibuf = info ? info : call.tmp<uint32_t>(B);
    const std::vector<Call::Slice> sl = {{a.data, nullptr, (size_t)M * N * 4},
                                         {nullptr, u, u ? (size_t)M * K * 4 : 0},
                                         {nullptr, s, (size_t)K * 4},
                                         {nullptr, vt, vt ? (size_t)K * N * 4 : 0},
                                         {nullptr, ibuf, 4}};
    float* ws = static_cast<float*>(call.scratch(svd_small_workspace(M, N, call.chunk_size(B, sl))));
    call.batched(B, sl, [&](void* const* d, uint32_t nb, hipStream_t st) {
        svd_small(f32(d[0]), f32(d[1]), f32(d[2]), f32(d[3]), u32p(d[4]), ws, nb, M, N, st);
    });
    if (is_device_memory(ibuf)) check_converged(ibuf, B, call.stream(), "svd");
    else check_converged_host(ibuf, B, "svd");
    call.finish();
}

namespace {

// LU, solve and inverse: the batched kernels unless the route is the
// blocked path (the reference's "cpu" route is its batch path, which is the
// batched kernels here)
bool lu_batched(uint32_t n, uint32_t batch) {
    return lu_small_factor_fits(n) && std::strcmp(lu_backend_name(n, batch), "blocked") != 0;
}

void require_square(const Matrices& a, const char* what) {
    if (a.rows != a.cols)
        invalid(std::string("[") + what + "] The matrices must be square, got " + std::to_string(a.rows) + "x" +
                std::to_string(a.cols) + ".");
}

[[noreturn]] void too_large(const char* what, uint32_t n, uint32_t limit) {
    invalid(std::string("[") + what + "] n = " + std::to_string(n) + ": this build's kernels take n <= " +
            std::to_string(limit));
}

}  // namespace

// reference: src/cholesky.mm:178-189 (core::cholesky)
void cholesky(const Matrices& a, bool upper, float* l, uint32_t* info) {
    require_gpu_allowed("cholesky");
    require_square(a, "cholesky");
    const uint32_t n = a.cols, B = a.batch;
    if (n == 0 || B == 0) return;
    Call call;
    // the routed backend: the batched kernels ("simd", "threadgroup"; also a
    // "cpu" route, this build's batch path) or the blocked path
    if (chol_small_fits(n) && std::strcmp(cholesky_backend_name(n, B), "blocked") != 0) {
        call.batched(B, {{a.data, nullptr, (size_t)n * n * 4}, {nullptr, l, (size_t)n * n * 4}, {nullptr, info, 4}},
                     [&](void* const* d, uint32_t nb, hipStream_t s) {
                         chol_small(f32(d[0]), f32(d[1]), u32p(d[2]), nb, n, upper, s);
                     });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    float* dl = call.out(l, (size_t)B * n * n);
    {
        uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
        float* work = static_cast<float*>(call.scratch(chol_blocked_workspace(n)));
        chol_blocked(da, dl, di, work, work + (size_t)n * n, B, n, upper, call.stream());
    }
    call.finish();
}

// reference: src/lu.mm:148-166 (core::lu_factor, solve, inv)
void lu_factor(const Matrices& a, float* lu, uint32_t* pivots, uint32_t* info) {
    require_gpu_allowed("lu_factor");
    require_square(a, "lu_factor");
    const uint32_t n = a.cols, B = a.batch;
    if (n == 0 || B == 0) return;
    if (!lu_blocked_fits(n)) too_large("lu_factor", n, 16384);
    Call call;
    if (lu_batched(n, B)) {
        call.batched(B, {{a.data, nullptr, (size_t)n * n * 4}, {nullptr, lu, (size_t)n * n * 4},
                         {nullptr, pivots, (size_t)n * 4}, {nullptr, info, 4}},
                     [&](void* const* d, uint32_t nb, hipStream_t s) {
                         lu_small_factor(f32(d[0]), f32(d[1]), u32p(d[2]), u32p(d[3]), nb, n, s);
                     });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    float* dlu = call.out(lu, (size_t)B * n * n);
    uint32_t* dp = call.out(pivots, (size_t)B * n);
    {
        uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
        float* work = static_cast<float*>(call.scratch(lu_panel_workspace(n)));
        lu_blocked_factor(da, dlu, dp, di, work, B, n, call.stream());
    }
    call.finish();
}

void solve(const Matrices& a, const float* b, uint32_t nrhs, float* x, uint32_t* info) {
    require_gpu_allowed("solve");
    require_square(a, "solve");
    const uint32_t n = a.cols, B = a.batch;
    if (n == 0 || B == 0 || nrhs == 0) {
        if (info && B) {   // reference: lu_cpu.mm:108-111 (info zeroed)
            Call call;
            uint32_t* di = call.out(info, B);
            MLA_HIP(hipMemsetAsync(di, 0, (size_t)B * sizeof(uint32_t), call.stream()));
            call.finish();
        }
        return;
    }
    if (!lu_blocked_fits(n)) too_large("solve", n, 16384);
    Call call;
    if (lu_batched(n, B)) {
        call.batched(B, {{a.data, nullptr, (size_t)n * n * 4}, {b, nullptr, (size_t)n * nrhs * 4},
                         {nullptr, x, (size_t)n * nrhs * 4}, {nullptr, info, 4}},
                     [&](void* const* d, uint32_t nb, hipStream_t s) {
                         lu_small_solve(f32(d[0]), f32(d[1]), nrhs, f32(d[2]), u32p(d[3]), nb, n, s);
                     });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    const float* db = call.in(b, (size_t)B * n * nrhs);
    float* dx = call.out(x, (size_t)B * n * nrhs);
    {
        uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
        float* work = static_cast<float*>(call.scratch(lu_blocked_workspace(n)));
        // the blocked path gathers b's rows into x: an x that overlaps b
        // (a solve in place) reads a copy of b instead
        const size_t bytes = (size_t)B * n * nrhs * sizeof(float);
        const char *xb = reinterpret_cast<const char*>(dx), *bb = reinterpret_cast<const char*>(db);
        if (xb < bb + bytes && bb < xb + bytes) {
            float* copy = call.tmp<float>((size_t)B * n * nrhs);
            MLA_HIP(hipMemcpyAsync(copy, db, bytes, hipMemcpyDeviceToDevice, call.stream()));
            db = copy;
        }
        lu_blocked_solve(da, db, nrhs, dx, di, work, B, n, call.stream());
    }
    call.finish();
}

void inv(const Matrices& a, float* x, uint32_t* info) {
    require_gpu_allowed("inv");
    require_square(a, "inv");
    const uint32_t n = a.cols, B = a.batch;
    if (n == 0 || B == 0) return;
    if (!lu_blocked_fits(n)) too_large("inv", n, 16384);
    Call call;
    if (lu_batched(n, B)) {
        call.batched(B, {{a.data, nullptr, (size_t)n * n * 4}, {nullptr, x, (size_t)n * n * 4}, {nullptr, info, 4}},
                     [&](void* const* d, uint32_t nb, hipStream_t s) {
                         lu_small_inv(f32(d[0]), f32(d[1]), u32p(d[2]), nb, n, s);
                     });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    float* dx = call.out(x, (size_t)B * n * n);
    {
        uint32_t* di = info ? call.out(info, B) : call.tmp<uint32_t>(B);
        float* work = static_cast<float*>(call.scratch(lu_blocked_workspace(n)));
        lu_blocked_solve(da, nullptr, n, dx, di, work, B, n, call.stream());
    }
    call.finish();
}

// reference: src/trsm.mm:288-294 (core::solve_triangular)
void solve_triangular(const Matrices& a, const float* b, uint32_t nrhs, bool upper, bool unit, float* x) {
    require_gpu_allowed("solve_triangular");
    require_square(a, "solve_triangular");
    const uint32_t n = a.cols, B = a.batch;
    if (n == 0 || B == 0 || nrhs == 0) return;
    Call call;
    // the triangular solve takes the same n; the routed backend as LU's
    if (lu_small_factor_fits(n) && std::strcmp(trsm_backend_name(n, nrhs, B), "blocked") != 0) {
        call.batched(B, {{a.data, nullptr, (size_t)n * n * 4}, {b, nullptr, (size_t)n * nrhs * 4},
                         {nullptr, x, (size_t)n * nrhs * 4}},
                     [&](void* const* d, uint32_t nb, hipStream_t s) {
                         trsm_small(f32(d[0]), f32(d[1]), f32(d[2]), nb, n, nrhs, upper, unit, s);
                     });
        call.finish();
        return;
    }
    const float* da = call.in(a.data, (size_t)B * n * n);
    const float* db = call.in(b, (size_t)B * n * nrhs);
    float* dx = call.out(x, (size_t)B * n * nrhs);
    {
        if (dx != db)
            MLA_HIP(hipMemcpyAsync(dx, db, (size_t)B * n * nrhs * sizeof(float), hipMemcpyDeviceToDevice,
                                   call.stream()));
        for (uint32_t i = 0; i < B; ++i)
            trsm_blocked_one(da + (size_t)i * n * n, (int)n, dx + (size_t)i * n * nrhs, (int)n, (int)nrhs, upper,
                             unit, call.stream());
    }
    call.finish();
}

}  // namespace mla::core
