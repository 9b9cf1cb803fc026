// QR of one matrix taller than the blocked QR's panels take (more than 4096
// rows) with at most 2048 columns: a tree of blocked QRs (TSQR).
//
// Role: the MI355X counterpart of the reference's TSQR panels for tall
// matrices (reference: src/band_reduce.mm:309-313, a tree of up to 2^15
// leaves under qr_blocked, src/qr_blocked.mm:276), here at the level of the
// whole matrix: the rows are cut into nb balanced blocks of at most 4096,
// each factored by the blocked QR (Q_b R_b = A_b), the R_b stacked (nb n x n,
// at most half the rows when n <= 2048) and factored the same way (by the
// blocked QR, or again as a tree while taller than 4096), and Q = diag(Q_b)
// Q_S formed top-down, one MFMA product per block.  Householder blocks at
// every level keep Q orthogonal to working precision whatever the rank.  R
// is unique up to the signs of its rows: they are those of the stack's
// factorisation, not of one Householder sweep over A.
#include <algorithm>

#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

constexpr uint32_t kLeafRows = 4096;   // the blocked QR's row limit
constexpr uint32_t kMaxCols = 2048;    // a stack of two blocks' R stays within kLeafRows

struct Split {
    uint32_t nb, rb;   // blocks, rows per block (the last one fewer)
};

Split split(uint32_t rows) {
    const uint32_t nb = (uint32_t)cdiv(rows, kLeafRows);
    return {nb, (uint32_t)cdiv(rows, nb)};
}

size_t round64(size_t c) { return (c + 63) / 64 * 64; }

// floats of one level (and those under it) for rows x n, Q formed or not
size_t level_floats(uint32_t rows, uint32_t n, bool with_q) {
    if (rows <= kLeafRows) return round64(qr_blocked_workspace(rows, n) / sizeof(float) + 64);
    const Split sp = split(rows);
    const size_t srows = (size_t)sp.nb * n;
    size_t f = round64(srows * n);                                  // S, the stacked R
    if (with_q) f += round64((size_t)rows * n) + round64(srows * n);   // the blocks' Q, the stack's Q
    return f + std::max(level_floats((uint32_t)srows, n, with_q),
                        round64(qr_blocked_workspace(kLeafRows, n) / sizeof(float) + 64));
}

// A (rows x n, contiguous) = Q R: Q rows x n (contiguous; NULL: R alone),
// R n x n upper triangular
void tsqr(const float* A, uint32_t rows, uint32_t n, float* Q, float* R, float* work, hipStream_t s) {
    if (rows <= kLeafRows) {
        qr_blocked(A, Q, R, 1, rows, n, Q ? n : 0, n, work, s);
        return;
    }
    const Split sp = split(rows);
    const uint32_t srows = sp.nb * n;
    float* p = work;
    float* S = p;
    p += round64((size_t)srows * n);
    float* Qb = nullptr;
    float* Qs = nullptr;
    if (Q) {
        Qb = p;
        p += round64((size_t)rows * n);
        Qs = p;
        p += round64((size_t)srows * n);
    }
    for (uint32_t b = 0; b < sp.nb; ++b) {
        const uint32_t r0 = b * sp.rb, rb = std::min(sp.rb, rows - r0);
        qr_blocked(A + (size_t)r0 * n, Q ? Qb + (size_t)r0 * n : nullptr, S + (size_t)b * n * n, 1, rb, n, Q ? n : 0,
                   n, p, s);
    }
    tsqr(S, srows, n, Qs, R, p, s);
    if (!Q) return;
    for (uint32_t b = 0; b < sp.nb; ++b) {
        const uint32_t r0 = b * sp.rb, rb = std::min(sp.rb, rows - r0);
        sgemm(false, false, (int)rb, (int)n, (int)n, 1.0f, Qb + (size_t)r0 * n, (int)n, 0, Qs + (size_t)b * n * n,
              (int)n, 0, 0.0f, Q + (size_t)r0 * n, (int)n, 0, 1, s);
    }
}

}  // namespace

bool qr_tsqr_fits(uint32_t m, uint32_t n, uint32_t qc) {
    if (m <= kLeafRows || n < 1 || n > kMaxCols || m < n || !(qc == 0 || qc == n)) return false;
    // every block holds at least n rows, so that its R is n x n
    const Split sp = split(m);
    return m - (sp.nb - 1) * sp.rb >= n;
}

size_t qr_tsqr_workspace(uint32_t m, uint32_t n, bool with_q) { return level_floats(m, n, with_q) * sizeof(float); }

void qr_tsqr_one(const float* a, float* q, float* r, uint32_t m, uint32_t n, float* work, hipStream_t s) {
    KernelTimer t("qr_tsqr", s);
    tsqr(a, m, n, q, r, work, s);
    t.stop();
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
