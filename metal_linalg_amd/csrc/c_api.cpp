// The C ABI (include/metal_linalg/c_api.h) over the buffer core: argument
// checks, exceptions turned into status codes, the message kept per thread.
// Behaviour follows the reference's src/c_api.cpp:17-401 (guarded(),
// present(), the per-call checks and the policy get/set field copies).
#include <metal_linalg/c_api.h>

#include <algorithm>
#include <new>
#include <stdexcept>
#include <string>

#include "core.hpp"
#include "policy.hpp"
#include "runtime.hpp"

using mla::core::Matrices;
using mla::core::QrMode;

namespace {

thread_local std::string g_last_error;

template <class F>
metal_linalg_status guarded(F&& f) {
    try {
        f();
        return METAL_LINALG_OK;
    } catch (const std::invalid_argument& e) {
        g_last_error = e.what();
        return METAL_LINALG_INVALID_ARGUMENT;
    } catch (const std::bad_alloc&) {
        g_last_error = "out of memory";
        return METAL_LINALG_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return METAL_LINALG_RUNTIME_ERROR;
    } catch (...) {
        g_last_error = "unknown error";
        return METAL_LINALG_RUNTIME_ERROR;
    }
}

void require(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(what);
}

// A buffer may be NULL only when it holds nothing.
bool present(const void* p, uint64_t count) { return p != nullptr || count == 0; }

}  // namespace

extern "C" {

const char* metal_linalg_last_error(void) { return g_last_error.c_str(); }

metal_linalg_status metal_linalg_qr(const float* a, uint32_t batch, uint32_t rows, uint32_t cols, float* q,
                                    float* r) {
    return guarded([&] {
        const uint64_t k = std::min(rows, cols);
        require(present(a, (uint64_t)batch * rows * cols), "[qr] a is NULL");
        require(present(q, (uint64_t)batch * rows * k), "[qr] q is NULL");
        require(present(r, (uint64_t)batch * k * cols), "[qr] r is NULL");
        mla::core::qr({a, batch, rows, cols}, q, r, QrMode::reduced);
    });
}

metal_linalg_status metal_linalg_qr_with_mode(const float* a, uint32_t batch, uint32_t rows, uint32_t cols,
                                              metal_linalg_qr_mode mode, float* q, float* r) {
    return guarded([&] {
        require(mode == METAL_LINALG_QR_REDUCED || mode == METAL_LINALG_QR_R || mode == METAL_LINALG_QR_COMPLETE,
                "[qr] mode must be METAL_LINALG_QR_REDUCED, _R or _COMPLETE");
        const QrMode m = mode == METAL_LINALG_QR_R          ? QrMode::r
                         : mode == METAL_LINALG_QR_COMPLETE ? QrMode::complete
                                                            : QrMode::reduced;
        const uint64_t qc = mla::core::qr_q_cols(m, rows, cols), rr = mla::core::qr_r_rows(m, rows, cols);
        require(present(a, (uint64_t)batch * rows * cols), "[qr] a is NULL");
        if (qc) require(present(q, (uint64_t)batch * rows * qc), "[qr] q is NULL");
        require(present(r, (uint64_t)batch * rr * cols), "[qr] r is NULL");
        mla::core::qr({a, batch, rows, cols}, qc ? q : nullptr, r, m);
    });
}

metal_linalg_status metal_linalg_eigh(const float* a, uint32_t batch, uint32_t n, int lower, float* w, float* v,
                                      uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[eigh] a is NULL");
        require(present(w, (uint64_t)batch * n), "[eigh] w is NULL");
        mla::core::eigh({a, batch, n, n}, lower != 0, w, v, info);
    });
}

metal_linalg_status metal_linalg_svd(const float* a, uint32_t batch, uint32_t rows, uint32_t cols, float* u,
                                     float* s, float* vt, uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * rows * cols), "[svd] a is NULL");
        require(present(s, (uint64_t)batch * std::min(rows, cols)), "[svd] s is NULL");
        require((u == nullptr) == (vt == nullptr), "[svd] u and vt must both be given or both be NULL");
        mla::core::svd({a, batch, rows, cols}, u, s, vt, info);
    });
}

metal_linalg_status metal_linalg_cholesky(const float* a, uint32_t batch, uint32_t n, int upper, float* l,
                                          uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[cholesky] a is NULL");
        require(present(l, (uint64_t)batch * n * n), "[cholesky] l is NULL");
        mla::core::cholesky({a, batch, n, n}, upper != 0, l, info);
    });
}

metal_linalg_status metal_linalg_lu_factor(const float* a, uint32_t batch, uint32_t n, float* lu, uint32_t* pivots,
                                           uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[lu_factor] a is NULL");
        require(present(lu, (uint64_t)batch * n * n), "[lu_factor] lu is NULL");
        require(present(pivots, (uint64_t)batch * n), "[lu_factor] pivots is NULL");
        mla::core::lu_factor({a, batch, n, n}, lu, pivots, info);
    });
}

metal_linalg_status metal_linalg_solve(const float* a, uint32_t batch, uint32_t n, const float* b, uint32_t nrhs,
                                       float* x, uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[solve] a is NULL");
        require(present(b, (uint64_t)batch * n * nrhs), "[solve] b is NULL");
        require(present(x, (uint64_t)batch * n * nrhs), "[solve] x is NULL");
        mla::core::solve({a, batch, n, n}, b, nrhs, x, info);
    });
}

metal_linalg_status metal_linalg_inv(const float* a, uint32_t batch, uint32_t n, float* x, uint32_t* info) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[inv] a is NULL");
        require(present(x, (uint64_t)batch * n * n), "[inv] x is NULL");
        mla::core::inv({a, batch, n, n}, x, info);
    });
}

metal_linalg_status metal_linalg_solve_triangular(const float* a, uint32_t batch, uint32_t n, const float* b,
                                                  uint32_t nrhs, int upper, int unit, float* x) {
    return guarded([&] {
        require(present(a, (uint64_t)batch * n * n), "[solve_triangular] a is NULL");
        require(present(b, (uint64_t)batch * n * nrhs), "[solve_triangular] b is NULL");
        require(present(x, (uint64_t)batch * n * nrhs), "[solve_triangular] x is NULL");
        mla::core::solve_triangular({a, batch, n, n}, b, nrhs, upper != 0, unit != 0, x);
    });
}

// ---- Metal buffers: no such thing on this platform ----
void* metal_linalg_buffer_contents(const void*, uint64_t, uint64_t) { return nullptr; }
int metal_linalg_know_buffer(const void*, const void*) { return 0; }
void metal_linalg_forget_buffer(const void*, const void*) {}

// ---- device and routing ----
const char* metal_linalg_device_name(void) {
    static std::string name;
    name = mla::have_device() ? mla::device().name : std::string();
    return name.c_str();
}
uint32_t metal_linalg_gpu_core_count(void) { return mla::have_device() ? mla::device().cus : 0u; }
void metal_linalg_set_calibration_notices(int enabled) { mla::set_calibration_notices(enabled != 0); }
const char* metal_linalg_calibration_message(const char* decomposition) {
    return mla::calibration_message(decomposition);
}
void metal_linalg_set_cpu_threads(uint32_t n) { mla::set_cpu_threads(n); }
uint32_t metal_linalg_cpu_threads(void) { return mla::cpu_threads(); }
void metal_linalg_set_cpu_only(int on) { mla::set_cpu_only(on != 0); }
int metal_linalg_cpu_only(void) { return mla::cpu_only() ? 1 : 0; }

const char* metal_linalg_qr_backend(uint32_t rows, uint32_t cols, uint32_t batch) {
    return mla::qr_backend_name(rows, cols, batch);
}
const char* metal_linalg_eigh_backend(uint32_t n, uint32_t batch) { return mla::eigh_backend_name(n, batch, true); }
const char* metal_linalg_eigvalsh_backend(uint32_t n, uint32_t batch) {
    return mla::eigh_backend_name(n, batch, false);
}
const char* metal_linalg_svd_backend(uint32_t rows, uint32_t cols, uint32_t batch) {
    return mla::svd_backend_name(rows, cols, batch, true);
}
const char* metal_linalg_svdvals_backend(uint32_t rows, uint32_t cols, uint32_t batch) {
    return mla::svd_backend_name(rows, cols, batch, false);
}
const char* metal_linalg_cholesky_backend(uint32_t n, uint32_t batch) { return mla::cholesky_backend_name(n, batch); }
const char* metal_linalg_lu_backend(uint32_t n, uint32_t batch) { return mla::lu_backend_name(n, batch); }
const char* metal_linalg_trsm_backend(uint32_t n, uint32_t nrhs, uint32_t batch) {
    return mla::trsm_backend_name(n, nrhs, batch);
}

// ---- policies: informational fields keep the detected values on set ----
metal_linalg_qr_policy metal_linalg_qr_policy_get(void) { return mla::qr_policy(); }
metal_linalg_eigh_policy metal_linalg_eigh_policy_get(void) { return mla::eigh_policy(); }
metal_linalg_svd_policy metal_linalg_svd_policy_get(void) { return mla::svd_policy(); }
metal_linalg_cholesky_policy metal_linalg_cholesky_policy_get(void) { return mla::cholesky_policy(); }
metal_linalg_lu_policy metal_linalg_lu_policy_get(void) { return mla::lu_policy(); }
metal_linalg_trsm_policy metal_linalg_trsm_policy_get(void) { return mla::trsm_policy(); }

void metal_linalg_qr_policy_set(const metal_linalg_qr_policy* c) {
    if (!c) return;
    metal_linalg_qr_policy& p = mla::qr_policy();
    const uint32_t cores = p.gpu_cores, conc = p.concurrent_matrices;
    p = *c;
    p.gpu_cores = cores;
    p.concurrent_matrices = conc;
    mla::mark_user_policy("qr");
}

void metal_linalg_eigh_policy_set(const metal_linalg_eigh_policy* c) {
    if (!c) return;
    metal_linalg_eigh_policy& p = mla::eigh_policy();
    const uint32_t cores = p.gpu_cores;
    p = *c;
    p.gpu_cores = cores;
    mla::mark_user_policy("eigh");
}

void metal_linalg_svd_policy_set(const metal_linalg_svd_policy* c) {
    if (!c) return;
    metal_linalg_svd_policy& p = mla::svd_policy();
    const uint32_t cores = p.gpu_cores;
    p = *c;
    p.gpu_cores = cores;
    mla::mark_user_policy("svd");
}

void metal_linalg_cholesky_policy_set(const metal_linalg_cholesky_policy* c) {
    if (!c) return;
    metal_linalg_cholesky_policy& p = mla::cholesky_policy();
    const uint32_t cores = p.gpu_cores;
    p = *c;
    p.gpu_cores = cores;
    mla::mark_user_policy("cholesky");
}

void metal_linalg_lu_policy_set(const metal_linalg_lu_policy* c) {
    if (!c) return;
    metal_linalg_lu_policy& p = mla::lu_policy();
    const uint32_t cores = p.gpu_cores;
    p = *c;
    p.gpu_cores = cores;
    mla::mark_user_policy("lu");
}

void metal_linalg_trsm_policy_set(const metal_linalg_trsm_policy* c) {
    if (!c) return;
    metal_linalg_trsm_policy& p = mla::trsm_policy();
    const uint32_t cores = p.gpu_cores;
    p = *c;
    p.gpu_cores = cores;
    mla::mark_user_policy("trsm");
}

const char* metal_linalg_qr_policy_source(void) { return mla::policy_source("qr"); }
const char* metal_linalg_eigh_policy_source(void) { return mla::policy_source("eigh"); }
const char* metal_linalg_svd_policy_source(void) { return mla::policy_source("svd"); }
const char* metal_linalg_cholesky_policy_source(void) { return mla::policy_source("cholesky"); }
const char* metal_linalg_lu_policy_source(void) { return mla::policy_source("lu"); }
const char* metal_linalg_trsm_policy_source(void) { return mla::policy_source("trsm"); }

}  // extern "C"
