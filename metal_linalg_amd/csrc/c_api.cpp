// The C ABI (include/metal_linalg/c_api.h) over the buffer core.
//
// Each decomposition entry point is one row of the same shape: the caller's
// buffers listed with their element counts (a buffer may be NULL only when
// it holds nothing), then the core call.  enter() applies the buffer rule in
// the listed order; run_entry (entry.hpp) turns whatever the core throws
// into a status code, keeping the message for metal_linalg_last_error() on
// the calling thread.
// Observable behaviour (statuses, messages, which check reports first)
// follows the reference's src/c_api.cpp:17-190.
#include <metal_linalg/c_api.h>

#include <algorithm>
#include <exception>
#include <initializer_list>
#include <new>
#include <stdexcept>
#include <string>

#include "core.hpp"
#include "entry.hpp"
#include "policy.hpp"
#include "runtime.hpp"

using mla::core::Matrices;
using mla::core::QrMode;

namespace {

// A caller buffer as the buffer rule sees it.
struct Buf {
    const char* name;   // the argument's name in the message
    const void* ptr;
    uint64_t count;     // elements it holds for this call
};

template <class Work>
metal_linalg_status enter(const char* op, std::initializer_list<Buf> bufs, Work&& work) noexcept {
    return mla::run_entry([&] {
        for (const Buf& b : bufs)
            if (b.ptr == nullptr && b.count != 0)
                throw std::invalid_argument(std::string("[") + op + "] " + b.name + " is NULL");
        work();
    });
}

metal_linalg_status reject(const char* message) noexcept {
    mla::last_error_message() = message;
    return METAL_LINALG_INVALID_ARGUMENT;
}

uint64_t elems(uint64_t batch, uint64_t rows, uint64_t cols) { return batch * rows * cols; }

}  // namespace

extern "C" {

const char* metal_linalg_last_error(void) { return mla::last_error_message().c_str(); }

metal_linalg_status metal_linalg_qr(const float* a, uint32_t batch, uint32_t rows, uint32_t cols, float* q,
                                    float* r) {
    const uint64_t k = std::min(rows, cols);
    return enter("qr", {{"a", a, elems(batch, rows, cols)}, {"q", q, elems(batch, rows, k)},
                        {"r", r, elems(batch, k, cols)}},
                 [&] { mla::core::qr({a, batch, rows, cols}, q, r, QrMode::reduced); });
}

metal_linalg_status metal_linalg_qr_with_mode(const float* a, uint32_t batch, uint32_t rows, uint32_t cols,
                                              metal_linalg_qr_mode mode, float* q, float* r) {
    QrMode m;
    switch (mode) {
        case METAL_LINALG_QR_REDUCED: m = QrMode::reduced; break;
        case METAL_LINALG_QR_R: m = QrMode::r; break;
        case METAL_LINALG_QR_COMPLETE: m = QrMode::complete; break;
        default: return reject("[qr] mode must be METAL_LINALG_QR_REDUCED, _R or _COMPLETE");
    }
    const uint64_t qc = mla::core::qr_q_cols(m, rows, cols), rr = mla::core::qr_r_rows(m, rows, cols);
    // q is not read when the mode forms no Q (its count is then zero)
    return enter("qr", {{"a", a, elems(batch, rows, cols)}, {"q", q, elems(batch, rows, qc)},
                        {"r", r, elems(batch, rr, cols)}},
                 [&] { mla::core::qr({a, batch, rows, cols}, qc ? q : nullptr, r, m); });
}

metal_linalg_status metal_linalg_eigh(const float* a, uint32_t batch, uint32_t n, int lower, float* w, float* v,
                                      uint32_t* info) {
    return enter("eigh", {{"a", a, elems(batch, n, n)}, {"w", w, elems(batch, n, 1)}},
                 [&] { mla::core::eigh({a, batch, n, n}, lower != 0, w, v, info); });
}

metal_linalg_status metal_linalg_svd(const float* a, uint32_t batch, uint32_t rows, uint32_t cols, float* u,
                                     float* s, float* vt, uint32_t* info) {
    return enter("svd", {{"a", a, elems(batch, rows, cols)}, {"s", s, elems(batch, std::min(rows, cols), 1)}}, [&] {
        if ((u == nullptr) != (vt == nullptr))
            throw std::invalid_argument("[svd] u and vt must both be given or both be NULL");
        mla::core::svd({a, batch, rows, cols}, u, s, vt, info);
    });
}

metal_linalg_status metal_linalg_cholesky(const float* a, uint32_t batch, uint32_t n, int upper, float* l,
                                          uint32_t* info) {
    return enter("cholesky", {{"a", a, elems(batch, n, n)}, {"l", l, elems(batch, n, n)}},
                 [&] { mla::core::cholesky({a, batch, n, n}, upper != 0, l, info); });
}

metal_linalg_status metal_linalg_lu_factor(const float* a, uint32_t batch, uint32_t n, float* lu, uint32_t* pivots,
                                           uint32_t* info) {
    return enter("lu_factor",
                 {{"a", a, elems(batch, n, n)}, {"lu", lu, elems(batch, n, n)}, {"pivots", pivots, elems(batch, n, 1)}},
                 [&] { mla::core::lu_factor({a, batch, n, n}, lu, pivots, info); });
}

metal_linalg_status metal_linalg_solve(const float* a, uint32_t batch, uint32_t n, const float* b, uint32_t nrhs,
                                       float* x, uint32_t* info) {
    return enter("solve",
                 {{"a", a, elems(batch, n, n)}, {"b", b, elems(batch, n, nrhs)}, {"x", x, elems(batch, n, nrhs)}},
                 [&] { mla::core::solve({a, batch, n, n}, b, nrhs, x, info); });
}

metal_linalg_status metal_linalg_inv(const float* a, uint32_t batch, uint32_t n, float* x, uint32_t* info) {
    return enter("inv", {{"a", a, elems(batch, n, n)}, {"x", x, elems(batch, n, n)}},
                 [&] { mla::core::inv({a, batch, n, n}, x, info); });
}

metal_linalg_status metal_linalg_solve_triangular(const float* a, uint32_t batch, uint32_t n, const float* b,
                                                  uint32_t nrhs, int upper, int unit, float* x) {
    return enter("solve_triangular",
                 {{"a", a, elems(batch, n, n)}, {"b", b, elems(batch, n, nrhs)}, {"x", x, elems(batch, n, nrhs)}},
                 [&] { mla::core::solve_triangular({a, batch, n, n}, b, nrhs, upper != 0, unit != 0, x); });
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
