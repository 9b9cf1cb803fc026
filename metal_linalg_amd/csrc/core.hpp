// The buffer core: the decompositions on caller buffers (host or device
// memory), each picking its GPU kernels by shape.  Mirrors the reference's
// core:: layer (reference: include/metal_linalg/core.h:777-1049).  Errors are
// thrown: std::invalid_argument for a shape no kernel takes,
// std::runtime_error for a HIP failure or a finite matrix that did not
// converge, std::bad_alloc for device memory.
#pragma once

#include <cstdint>

namespace mla::core {

struct Matrices {   // reference: core.h:777-782
    const float* data;
    uint32_t batch;
    uint32_t rows;
    uint32_t cols;
};

enum class QrMode { reduced, r, complete };   // reference: core.h:786-790

inline uint32_t qr_q_cols(QrMode mode, uint32_t m, uint32_t n) {   // reference: core.h:792-794
    return mode == QrMode::r ? 0 : mode == QrMode::complete ? m : (m < n ? m : n);
}
inline uint32_t qr_r_rows(QrMode mode, uint32_t m, uint32_t n) {   // reference: core.h:795-797
    return mode == QrMode::complete ? m : (m < n ? m : n);
}

void qr(const Matrices& a, float* q, float* r, QrMode mode);
void eigh(const Matrices& a, bool lower, float* w, float* v, uint32_t* info);
void svd(const Matrices& a, float* u, float* s, float* vt, uint32_t* info);
void cholesky(const Matrices& a, bool upper, float* l, uint32_t* info);
void lu_factor(const Matrices& a, float* lu, uint32_t* pivots, uint32_t* info);
void solve(const Matrices& a, const float* b, uint32_t nrhs, float* x, uint32_t* info);
void inv(const Matrices& a, float* x, uint32_t* info);
void solve_triangular(const Matrices& a, const float* b, uint32_t nrhs, bool upper, bool unit, float* x);

}  // namespace mla::core

namespace mla {

// Per-thread CPU-only flag (reference: device.h, device.mm:93-98).  This
// build has no CPU path: with the flag set the decompositions throw.
bool cpu_only();
void set_cpu_only(bool on);
void require_gpu_allowed(const char* what);

}  // namespace mla
