// Launchers of the HIP kernels, called by the buffer core (core.cpp).  Every
// pointer is device memory; every launcher only enqueues work on `s`.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mla {

// ---- QR ----
// Householder QR of `batch` m x n matrices, m, n <= 64: q [batch, m, qc]
// (qc = K, m or 0 for none), r [batch, rr, n] (rr = K or m).
bool qr_small_fits(uint32_t m, uint32_t n, uint32_t qc);
void qr_small(const float* a, float* q, float* r, uint32_t batch, uint32_t m, uint32_t n, uint32_t qc, uint32_t rr,
              hipStream_t s);

}  // namespace mla
