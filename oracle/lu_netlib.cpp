// ORACLE -- test infrastructure, not product code.
//
// LU, solve and inverse restated from netlib LAPACK 3.x's unblocked
// routines, for the parity of non-finite inputs.  The reference calls
// Accelerate's sgetrf / sgetrs / sgetri (src/lu_cpu.mm:72-157) with no scan
// of the input, so a NaN or an infinity in a read entry travels through the
// factorization and the pivot search decides where it lands.  LAPACK fixes
// that search in ISAMAX: the first entry of largest magnitude, compared with
// a strict '>', so a NaN is never taken over a number and a NaN in the first
// (diagonal) position is kept.  The OpenBLAS build that stands in for
// Accelerate in lapack_batch.cpp departs from that rule when a NaN is present
// (its vectorised isamax skips a leading NaN and returns the last of an
// all-NaN column), so the non-finite cases are pinned to this restatement of
// LAPACK's published algorithm instead.
//
// Every product is formed (no skipping of zero multipliers): IEEE semantics,
// so 0 * Inf and 0 * NaN give NaN where the algorithm multiplies them.
//
//   lu_netlib_factor   sgetf2 (LAPACK 3.x; sgetrf2's recursion performs the
//                      same eliminations, associated differently)
//   lu_netlib_solve    sgetf2 + sgetrs: slaswp, strsm(L, unit), strsm(U)
//   lu_netlib_inv      sgetf2 + sgetri: strti2 on U, the unblocked column
//                      loop for inv(A) L = inv(U), the column interchanges
// A matrix whose factorization meets an exactly-zero pivot (info > 0) gives
// an all-NaN solve / inverse, as src/lu_cpu.mm:119-122,146-149 does.
//
// Compiled with -ffp-contract=off: no fused multiply-adds, as LAPACK's
// Fortran on a target without FMA.

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

namespace {

constexpr float kQNaN = std::numeric_limits<float>::quiet_NaN();

// ISAMAX over x[0], x[stride], ..., x[(len-1)*stride]: 0-based index.
uint32_t isamax(const float* x, uint32_t len, size_t stride) {
    uint32_t best = 0;
    float smax = std::fabs(x[0]);
    for (uint32_t i = 1; i < len; ++i) {
        const float v = std::fabs(x[i * stride]);
        if (v > smax) {
            best = i;
            smax = v;
        }
    }
    return best;
}

// sgetf2 on the row-major n x n matrix w in place; ipiv 0-based.  Returns
// info (k + 1 for the first exactly-zero pivot U(k, k)).
uint32_t getf2(float* w, uint32_t n, uint32_t* ipiv) {
    uint32_t info = 0;
    for (uint32_t j = 0; j < n; ++j) {
        const uint32_t p = j + isamax(w + (size_t)j * n + j, n - j, n);
        ipiv[j] = p;
        if (w[(size_t)p * n + j] != 0.0f) {
            if (p != j)
                for (uint32_t c = 0; c < n; ++c) std::swap(w[(size_t)j * n + c], w[(size_t)p * n + c]);
            const float piv = w[(size_t)j * n + j];
            if (std::fabs(piv) >= FLT_MIN) {
                const float r = 1.0f / piv;
                for (uint32_t i = j + 1; i < n; ++i) w[(size_t)i * n + j] *= r;
            } else {
                for (uint32_t i = j + 1; i < n; ++i) w[(size_t)i * n + j] /= piv;
            }
        } else if (info == 0) {
            info = j + 1;
        }
        for (uint32_t i = j + 1; i < n; ++i) {   // sger: A22 -= l u^T
            const float l = w[(size_t)i * n + j];
            for (uint32_t c = j + 1; c < n; ++c) w[(size_t)i * n + c] -= l * w[(size_t)j * n + c];
        }
    }
    return info;
}

// sgetrs('N') on row-major B (n x nrhs) in place, from getf2's factors.
void getrs(const float* lu, const uint32_t* ipiv, uint32_t n, float* b, uint32_t nrhs) {
    for (uint32_t k = 0; k < n; ++k)   // slaswp, k = 1..n
        if (ipiv[k] != k)
            for (uint32_t j = 0; j < nrhs; ++j) std::swap(b[(size_t)k * nrhs + j], b[(size_t)ipiv[k] * nrhs + j]);
    for (uint32_t j = 0; j < nrhs; ++j) {
        for (uint32_t k = 0; k < n; ++k) {   // strsm Left Lower NoTrans Unit
            const float bk = b[(size_t)k * nrhs + j];
            for (uint32_t i = k + 1; i < n; ++i) b[(size_t)i * nrhs + j] -= bk * lu[(size_t)i * n + k];
        }
        for (uint32_t k = n; k-- > 0;) {   // strsm Left Upper NoTrans NonUnit
            const float bk = b[(size_t)k * nrhs + j] / lu[(size_t)k * n + k];
            b[(size_t)k * nrhs + j] = bk;
            for (uint32_t i = 0; i < k; ++i) b[(size_t)i * nrhs + j] -= bk * lu[(size_t)i * n + k];
        }
    }
}

// sgetri on getf2's factors (row-major, in place), for a matrix with info 0.
void getri(float* w, const uint32_t* ipiv, uint32_t n) {
    auto A = [&](uint32_t r, uint32_t c) -> float& { return w[(size_t)r * n + c]; };
    std::vector<float> x(n), work(n);
    // strti2('Upper', 'Non-unit'): column j of inv(U) from the columns before it
    for (uint32_t j = 0; j < n; ++j) {
        A(j, j) = 1.0f / A(j, j);
        const float ajj = -A(j, j);
        // strmv('Upper', 'No transpose', 'Non-unit', j, A, A(0:j, j)): x := T x
        for (uint32_t i = 0; i < j; ++i) x[i] = A(i, j);
        for (uint32_t c = 0; c < j; ++c) {
            const float t = x[c];
            for (uint32_t i = 0; i < c; ++i) x[i] += t * A(i, c);
            x[c] = t * A(c, c);
        }
        for (uint32_t i = 0; i < j; ++i) A(i, j) = x[i] * ajj;   // sscal
    }
    // inv(A) L = inv(U), one column at a time from the last
    for (uint32_t j = n; j-- > 0;) {
        for (uint32_t i = j + 1; i < n; ++i) {
            work[i] = A(i, j);
            A(i, j) = 0.0f;
        }
        if (j + 1 < n) {   // sgemv('N'): A(:, j) -= A(:, j+1:n) work(j+1:n)
            for (uint32_t c = j + 1; c < n; ++c) {
                const float t = -work[c];
                for (uint32_t i = 0; i < n; ++i) A(i, j) += t * A(i, c);
            }
        }
    }
    // the column interchanges, in reverse order
    for (uint32_t j = n - 1; j-- > 0;)
        if (ipiv[j] != j)
            for (uint32_t i = 0; i < n; ++i) std::swap(A(i, j), A(i, ipiv[j]));
}

}  // namespace

extern "C" {

void oracle_lu_netlib_factor(const float* a, uint32_t batch, uint32_t n, float* lu, uint32_t* pivots,
                             uint32_t* info) {
    const size_t per = (size_t)n * n;
    for (uint32_t b = 0; b < batch; ++b) {
        std::memcpy(lu + b * per, a + b * per, per * sizeof(float));
        const uint32_t i = getf2(lu + b * per, n, pivots + (size_t)b * n);
        if (info) info[b] = i;
    }
}

void oracle_lu_netlib_solve(const float* a, uint32_t batch, uint32_t n, const float* rhs, uint32_t nrhs, float* x,
                            uint32_t* info) {
    const size_t per = (size_t)n * n, bper = (size_t)n * nrhs;
    std::vector<float> w(per);
    std::vector<uint32_t> ipiv(n);
    for (uint32_t b = 0; b < batch; ++b) {
        std::memcpy(w.data(), a + b * per, per * sizeof(float));
        const uint32_t i = getf2(w.data(), n, ipiv.data());
        if (info) info[b] = i;
        float* out = x + b * bper;
        if (i > 0) {
            for (size_t e = 0; e < bper; ++e) out[e] = kQNaN;
            continue;
        }
        std::memcpy(out, rhs + b * bper, bper * sizeof(float));
        getrs(w.data(), ipiv.data(), n, out, nrhs);
    }
}

void oracle_lu_netlib_inv(const float* a, uint32_t batch, uint32_t n, float* x, uint32_t* info) {
    const size_t per = (size_t)n * n;
    std::vector<uint32_t> ipiv(n);
    for (uint32_t b = 0; b < batch; ++b) {
        float* w = x + b * per;
        std::memcpy(w, a + b * per, per * sizeof(float));
        const uint32_t i = getf2(w, n, ipiv.data());
        if (info) info[b] = i;
        if (i > 0) {
            for (size_t e = 0; e < per; ++e) w[e] = kQNaN;
            continue;
        }
        getri(w, ipiv.data(), n);
    }
}

}  // extern "C"
