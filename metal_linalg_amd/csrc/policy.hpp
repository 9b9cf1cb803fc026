// Routing policies and the backend each call shape takes.
//
// The policy structs, their resolution order (a tuned row for this device,
// else the defaults; then environment overrides; set_*_policy replacing
// both), and the routing rules are the reference's
// (reference: src/qr.mm:114-286, src/eigh.mm:274-880, src/svd.mm:130-1026,
// src/cholesky.mm:81-176, src/lu.mm:100-138, src/trsm.mm:100-140), so that
// the *_backend queries answer as the reference's do under the same policy.
// The tuned rows are the MI355X's own (its CUs, its kernels' limits).
//
// What executes is the GPU kernel family for the shape: this build has no
// CPU path, and a route the reference would have sent to the CPU runs on the
// GPU here too (the cpu_only flag instead makes a call fail).
#pragma once

#include <metal_linalg/c_api.h>

#include <cstdint>

namespace mla {

// The largest n of the batched eigh kernel ("ql") and the largest k of the
// batched Golub-Kahan SVD kernel on this device.
constexpr uint32_t kEighQlMaxN = 64;
constexpr uint32_t kSvdGkMaxK = 64;
bool svd_gk_fits(uint32_t m, uint32_t n);

const char* qr_backend_name(uint32_t m, uint32_t n, uint32_t batch);
const char* eigh_backend_name(uint32_t n, uint32_t batch, bool vectors);
const char* svd_backend_name(uint32_t m, uint32_t n, uint32_t batch, bool vectors);
const char* cholesky_backend_name(uint32_t n, uint32_t batch);
const char* lu_backend_name(uint32_t n, uint32_t batch);
const char* trsm_backend_name(uint32_t n, uint32_t nrhs, uint32_t batch);

metal_linalg_qr_policy& qr_policy();
metal_linalg_eigh_policy& eigh_policy();
metal_linalg_svd_policy& svd_policy();
metal_linalg_cholesky_policy& cholesky_policy();
metal_linalg_lu_policy& lu_policy();
metal_linalg_trsm_policy& trsm_policy();

const char* policy_source(const char* which);   // "qr", "eigh", "svd", "cholesky", "lu", "trsm"
void mark_user_policy(const char* which);

void set_calibration_notices(bool on);
const char* calibration_message(const char* decomposition);

uint32_t cpu_threads();
void set_cpu_threads(uint32_t n);

}  // namespace mla
