// The buffer core: argument shapes to kernels.  Every decomposition runs on
// the GPU; host buffers are staged by mla::Call.
#include "core.hpp"

#include <algorithm>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernels.hpp"
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
    if (!qr_small_fits(M, N, QC))
        invalid("[qr] " + std::to_string(M) + "x" + std::to_string(N) +
                ": this build's QR kernels take at most 64 rows and 64 columns so far");
    Call call;
    const float* da = call.in(a.data, (size_t)B * M * N);
    float* dq = QC ? call.out(q, (size_t)B * M * QC) : nullptr;
    float* dr = call.out(r, (size_t)B * RR * N);
    qr_small(da, dq, dr, B, M, N, QC, RR, call.stream());
    call.finish();
}

void eigh(const Matrices&, bool, float*, float*, uint32_t*) {
    require_gpu_allowed("eigh");
    invalid("[eigh] not available in this build yet");
}

void svd(const Matrices&, float*, float*, float*, uint32_t*) {
    require_gpu_allowed("svd");
    invalid("[svd] not available in this build yet");
}

void cholesky(const Matrices&, bool, float*, uint32_t*) {
    require_gpu_allowed("cholesky");
    invalid("[cholesky] not available in this build yet");
}

void lu_factor(const Matrices&, float*, uint32_t*, uint32_t*) {
    require_gpu_allowed("lu_factor");
    invalid("[lu_factor] not available in this build yet");
}

void solve(const Matrices&, const float*, uint32_t, float*, uint32_t*) {
    require_gpu_allowed("solve");
    invalid("[solve] not available in this build yet");
}

void inv(const Matrices&, float*, uint32_t*) {
    require_gpu_allowed("inv");
    invalid("[inv] not available in this build yet");
}

void solve_triangular(const Matrices&, const float*, uint32_t, bool, bool, float*) {
    require_gpu_allowed("solve_triangular");
    invalid("[solve_triangular] not available in this build yet");
}

}  // namespace mla::core
