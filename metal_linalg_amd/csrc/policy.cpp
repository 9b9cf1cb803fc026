// Routing policies: resolution, environment overrides, and the routing rules
// behind the *_backend queries.  The rules restate the reference's (the
// functions below cite the lines they follow); the tuned rows are this
// device's.
#include "policy.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <thread>

#include "core.hpp"
#include "runtime.hpp"
#include "tuned_gfx950.inc"

namespace mla {
namespace {

constexpr uint32_t kNoLimit = METAL_LINALG_NO_LIMIT;

struct DeviceId {
    std::string name, arch;
    uint32_t cus = 0;
    bool mi355x = false;   // gfx950 with 256 CUs: the device the rows were measured for
};

const DeviceId& device_id() {
    static const DeviceId d = [] {
        DeviceId r;
        if (have_device()) {
            const Device& dev = device();
            r.name = dev.name;
            r.arch = dev.arch;
            r.cus = dev.cus;
            r.mi355x = r.arch.rfind("gfx950", 0) == 0 && r.cus == 256;
        }
        return r;
    }();
    return d;
}

std::string tuned_label() { return "tuned:" + device_id().name + " (" + device_id().arch + ", " +
                                   std::to_string(device_id().cus) + " CUs)"; }
std::string untuned_label() {
    const DeviceId& d = device_id();
    return "default:untuned-device" + (d.name.empty() ? std::string() : " (" + d.name + ")");
}

// A non-negative integer from the environment; 0 is a value (reference:
// src/qr.mm:98-106).
bool env_value(const char* name, uint32_t& out) {
    const char* s = std::getenv(name);
    if (!s || !*s) return false;
    char* end = nullptr;
    const long long v = std::strtoll(s, &end, 10);
    if (end == s || v < 0) return false;
    out = v > 0xFFFFFFFFll ? kNoLimit : (uint32_t)v;
    return true;
}

struct EnvList {
    std::string names;
    void over(const char* name, uint32_t& field) {
        if (env_value(name, field)) names += (names.empty() ? "" : ",") + std::string(name);
    }
};

std::atomic<bool> g_notices{true};
std::mutex g_notice_mutex;
std::map<std::string, bool> g_tuned;   // decomposition -> tuned row applied

void notice(const char* what, bool tuned) {
    {
        std::lock_guard<std::mutex> lock(g_notice_mutex);
        g_tuned[what] = tuned;
    }
    if (tuned || !g_notices) return;
    if (const char* e = std::getenv("METAL_LINALG_NO_CALIBRATION_NOTICE"))
        if (*e && std::string(e) != "0") return;
    if (device_id().name.empty()) return;
    static std::set<std::string> shown;
    {
        std::lock_guard<std::mutex> lock(g_notice_mutex);
        if (!shown.insert(what).second) return;
    }
    std::fprintf(stderr, "%s\n", calibration_message(what));
}

template <class P>
struct State {
    P policy{};
    std::string source;
};

// ---------------------------------------------------------------- QR ----
State<metal_linalg_qr_policy>& qr_state() {
    static State<metal_linalg_qr_policy> s = [] {
        State<metal_linalg_qr_policy> r;
        metal_linalg_qr_policy& p = r.policy;
        // reference defaults (core.h QrPolicy)
        p = {384, 384, 16, kNoLimit, 1024, 1, 0, 0, 0, 0, 0, 0};
        p.gpu_cores = device_id().cus;
        p.concurrent_matrices = device_id().cus * 32;   // one matrix-wave per wave slot
        if (device_id().mi355x) {
            // qr_small ("unblocked") up to k = 64, the blocked path beyond;
            // every shape on the GPU
            p.m_crossover_small_batch = 65;
            p.m_crossover_large_batch = 65;
            p.batch_threshold = 16;
            p.gpu_max_k = kNoLimit;
            p.gpu_min_batch_times_k = 0;
            p.gpu_min_batch = 1;
            p.gpu_min_k = 0;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("QR", device_id().mi355x);
        EnvList env;
        uint32_t crossover = 0;
        if (env_value("QR_M_CROSSOVER", crossover) && crossover > 0) {
            p.m_crossover_small_batch = p.m_crossover_large_batch = crossover;
            env.names = "QR_M_CROSSOVER";
        }
        env.over("QR_GPU_MAX_K", p.gpu_max_k);
        env.over("QR_GPU_MIN_BATCH_TIMES_K", p.gpu_min_batch_times_k);
        env.over("QR_GPU_MIN_BATCH", p.gpu_min_batch);
        env.over("QR_GPU_MIN_K", p.gpu_min_k);
        env.over("QR_GPU_LARGE_MIN_K", p.gpu_large_min_k);
        env.over("QR_GPU_LARGE_MAX_BATCH", p.gpu_large_max_batch);
        env.over("QR_SHARE_MIN_BATCH", p.share_min_batch);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

// floor(sqrt(m k)) exactly (reference: src/qr.mm:240-247)
uint32_t qr_work_side(uint32_t m, uint32_t k) {
    const unsigned long long p = (unsigned long long)m * k;
    unsigned long long w = (unsigned long long)std::sqrt((double)p);
    while (w * w > p) --w;
    while ((w + 1) * (w + 1) <= p) ++w;
    return (uint32_t)w;
}

// reference: src/qr.mm:253-277
bool qr_uses_gpu(uint32_t m, uint32_t n, uint32_t batch) {
    if (cpu_only()) return false;
    if (const char* e = std::getenv("QR_DEVICE")) {
        if (!std::strcmp(e, "gpu")) return true;
        if (!std::strcmp(e, "cpu")) return false;
    }
    const metal_linalg_qr_policy& p = qr_state().policy;
    const uint32_t k = std::min(m, n);
    const unsigned long long L = p.gpu_large_min_k;
    if (p.gpu_large_min_k && (unsigned long long)m * k >= L * L &&
        (p.gpu_large_max_batch == 0 || batch <= p.gpu_large_max_batch))
        return true;
    const uint32_t w = qr_work_side(m, k);
    return w >= p.gpu_min_k && w <= p.gpu_max_k && (unsigned long long)batch * w >= p.gpu_min_batch_times_k &&
           batch >= p.gpu_min_batch;
}

// ---------------------------------------------------------------- eigh ----
State<metal_linalg_eigh_policy>& eigh_state() {
    static State<metal_linalg_eigh_policy> s = [] {
        State<metal_linalg_eigh_policy> r;
        metal_linalg_eigh_policy& p = r.policy;
        std::memset(&p, 0, sizeof(p));
        // reference defaults (core.h EighPolicy)
        p.simd_max_n = 8;
        p.block_min_n = 96;
        p.gpu_max_n = 64;
        p.gpu_min_batch_times_n = 1024;
        p.gpu_min_batch = 1;
        p.gpu_cores = device_id().cus;
        if (device_id().mi355x) {
            // the batched kernel ("ql") for every n it takes, at any batch;
            // larger n to the blocked path ("tridiag")
            p.simd_max_n = 0;
            p.block_min_n = kNoLimit;
            p.gpu_max_n = kEighQlMaxN;
            p.gpu_min_batch_times_n = 0;
            p.gpu_min_batch = 1;
            p.ql_min_n = 1;
            p.ql_max_n = kEighQlMaxN;
            p.tridiag_min_n = kEighQlMaxN + 1;
            p.values_tridiag_min_n = kEighQlMaxN + 1;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("eigh", device_id().mi355x);
        EnvList env;
        env.over("EIGH_SIMD_MAX_N", p.simd_max_n);
        env.over("EIGH_BLOCK_MIN_N", p.block_min_n);
        env.over("EIGH_BLOCK_MIN_N_BATCHED", p.block_min_n_batched);
        env.over("EIGH_BLOCK_MIN_BATCH", p.block_min_batch);
        env.over("EIGH_GPU_MAX_N", p.gpu_max_n);
        env.over("EIGH_GPU_MIN_BATCH_TIMES_N", p.gpu_min_batch_times_n);
        env.over("EIGH_GPU_MIN_BATCH", p.gpu_min_batch);
        env.over("EIGH_VALUES_GPU_MAX_N", p.values_gpu_max_n);
        env.over("EIGH_VALUES_GPU_MIN_BATCH_TIMES_N", p.values_gpu_min_batch_times_n);
        env.over("EIGH_VALUES_GPU_MIN_BATCH", p.values_gpu_min_batch);
        env.over("EIGH_TRIDIAG_MIN_N", p.tridiag_min_n);
        env.over("EIGH_VALUES_TRIDIAG_MIN_N", p.values_tridiag_min_n);
        env.over("EIGH_TRIDIAG_MAX_BATCH", p.tridiag_max_batch);
        env.over("EIGH_VALUES_TRIDIAG_MAX_BATCH", p.values_tridiag_max_batch);
        env.over("EIGH_QL_MIN_N", p.ql_min_n);
        env.over("EIGH_QL_MAX_N", p.ql_max_n);
        env.over("EIGH_SHARE_MIN_BATCH", p.share_min_batch);
        env.over("EIGH_GPU_BIG_BATCH_MAX_N", p.gpu_big_batch_max_n);
        env.over("EIGH_GPU_BIG_BATCH_MIN", p.gpu_big_batch_min);
        env.over("EIGH_VALUES_BAND_MIN_N", p.values_band_min_n);
        env.over("EIGH_VALUES_BAND_WIDTH", p.values_band_width);
        env.over("EIGH_BAND_MIN_N", p.band_min_n);
        env.over("EIGH_TRIDIAG_BATCH_MIN_N", p.tridiag_batch_min_n);
        env.over("EIGH_TRIDIAG_BATCH_MAX_N", p.tridiag_batch_max_n);
        env.over("EIGH_TRIDIAG_BATCH_MIN_BATCH", p.tridiag_batch_min_batch);
        env.over("EIGH_VALUES_TRIDIAG_BATCH_MIN_N", p.values_tridiag_batch_min_n);
        env.over("EIGH_VALUES_TRIDIAG_BATCH_MAX_N", p.values_tridiag_batch_max_n);
        env.over("EIGH_VALUES_TRIDIAG_BATCH_MIN_BATCH", p.values_tridiag_batch_min_batch);
        env.over("EIGH_SHARE_MIN_N", p.share_min_n);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

bool env_is(const char* var, const char* value) {
    const char* e = std::getenv(var);
    return e && !std::strcmp(e, value);
}

// reference: src/eigh.mm:763-775
const char* eigh_gpu_backend(uint32_t n, uint32_t batch) {
    const metal_linalg_eigh_policy& p = eigh_state().policy;
    if (p.ql_max_n && n >= p.ql_min_n && n <= std::min(p.ql_max_n, kEighQlMaxN)) return "ql";
    if (n >= p.block_min_n) return "block";
    if (p.block_min_batch && n >= p.block_min_n_batched && batch >= p.block_min_batch) return "block";
    return n <= p.simd_max_n ? "simd" : "threadgroup";
}

// reference: src/eigh.mm:779-788
bool eigh_gpu_rule(uint32_t n, uint32_t batch, uint32_t max_n, uint32_t min_bn, uint32_t min_batch) {
    if (env_is("EIGH_DEVICE", "gpu")) return true;
    if (env_is("EIGH_DEVICE", "cpu")) return false;
    return n <= max_n && (unsigned long long)batch * n >= min_bn && batch >= min_batch;
}

// reference: src/eigh.mm:790-810
bool eigh_uses_gpu(uint32_t n, uint32_t batch, bool vectors) {
    if (cpu_only()) return false;
    const metal_linalg_eigh_policy& p = eigh_state().policy;
    if (!vectors && p.values_gpu_min_batch != 0)
        return eigh_gpu_rule(n, batch, p.values_gpu_max_n, p.values_gpu_min_batch_times_n, p.values_gpu_min_batch);
    if (!std::getenv("EIGH_DEVICE") && p.gpu_big_batch_min && p.gpu_max_n && n > p.gpu_max_n &&
        n <= p.gpu_big_batch_max_n && batch >= p.gpu_big_batch_min)
        return true;
    return eigh_gpu_rule(n, batch, p.gpu_max_n, p.gpu_min_batch_times_n, p.gpu_min_batch);
}

// reference: src/eigh.mm:816-850
const char* eigh_cpu_side(uint32_t n, uint32_t batch, bool vectors) {
    if (env_is("EIGH_DEVICE", "cpu")) return "cpu";
    if (env_is("EIGH_DEVICE", "tridiag")) return "tridiag";
    const metal_linalg_eigh_policy& p = eigh_state().policy;
    const uint32_t bmin = vectors ? p.tridiag_batch_min_n : p.values_tridiag_batch_min_n;
    const uint32_t bmax = vectors ? p.tridiag_batch_max_n : p.values_tridiag_batch_max_n;
    const uint32_t bbat = vectors ? p.tridiag_batch_min_batch : p.values_tridiag_batch_min_batch;
    if (bmax != 0 && n >= bmin && n <= std::min(bmax, 1024u) && batch >= std::max(bbat, 1u)) return "tridiag_batch";
    const uint32_t cap = vectors ? p.tridiag_max_batch : p.values_tridiag_max_batch;
    if (cap != 0 && batch > cap) return "cpu";
    if (!vectors && p.values_band_min_n != 0 && n >= p.values_band_min_n) return "band";
    if (vectors && p.band_min_n != 0 && n >= p.band_min_n) return "band";
    const uint32_t from = vectors ? p.tridiag_min_n : p.values_tridiag_min_n;
    return from != 0 && n >= from ? "tridiag" : "cpu";
}

// ---------------------------------------------------------------- SVD ----
State<metal_linalg_svd_policy>& svd_state() {
    static State<metal_linalg_svd_policy> s = [] {
        State<metal_linalg_svd_policy> r;
        metal_linalg_svd_policy& p = r.policy;
        std::memset(&p, 0, sizeof(p));
        // reference defaults (core.h SvdPolicy)
        p.qr_min_rows = 512;
        p.qr_min_k = 64;
        p.block_min_k = 192;
        p.gpu_max_k = 64;
        p.gpu_min_batch_times_k = 1024;
        p.gpu_min_batch = 1;
        p.gpu_max_l = kNoLimit;
        p.values_gpu_max_l = kNoLimit;
        p.bidiag_batch_max_l = kNoLimit;
        p.values_bidiag_batch_max_l = kNoLimit;
        p.gpu_cores = device_id().cus;
        if (device_id().mi355x) {
            // the batched Golub-Kahan kernel for k up to 64 (after a QR when
            // the matrix is taller than it takes), at any batch; larger k to
            // the blocked path ("bidiag")
            p.gpu_max_k = kSvdGkMaxK;
            p.gpu_min_batch_times_k = 0;
            p.gpu_min_batch = 1;
            p.gk_min_k = 1;
            p.gk_max_k = kSvdGkMaxK;
            p.bidiag_min_k = kSvdGkMaxK + 1;
            p.values_bidiag_min_k = kSvdGkMaxK + 1;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("SVD", device_id().mi355x);
        EnvList env;
        env.over("SVD_QR_MIN_ROWS", p.qr_min_rows);
        env.over("SVD_QR_MIN_K", p.qr_min_k);
        env.over("SVD_BLOCK_MIN_K", p.block_min_k);
        env.over("SVD_BLOCK_MIN_K_BATCHED", p.block_min_k_batched);
        env.over("SVD_BLOCK_MIN_BATCH", p.block_min_batch);
        env.over("SVD_GPU_MAX_K", p.gpu_max_k);
        env.over("SVD_GPU_MIN_BATCH_TIMES_K", p.gpu_min_batch_times_k);
        env.over("SVD_GPU_MIN_BATCH", p.gpu_min_batch);
        env.over("SVD_GPU_MAX_L", p.gpu_max_l);
        env.over("SVD_VALUES_GPU_MAX_K", p.values_gpu_max_k);
        env.over("SVD_VALUES_GPU_MIN_BATCH_TIMES_K", p.values_gpu_min_batch_times_k);
        env.over("SVD_VALUES_GPU_MIN_BATCH", p.values_gpu_min_batch);
        env.over("SVD_VALUES_GPU_MAX_L", p.values_gpu_max_l);
        env.over("SVD_BIDIAG_MIN_K", p.bidiag_min_k);
        env.over("SVD_VALUES_BIDIAG_MIN_K", p.values_bidiag_min_k);
        env.over("SVD_BIDIAG_MAX_BATCH", p.bidiag_max_batch);
        env.over("SVD_VALUES_BIDIAG_MAX_BATCH", p.values_bidiag_max_batch);
        env.over("SVD_GK_MIN_K", p.gk_min_k);
        env.over("SVD_GK_MAX_K", p.gk_max_k);
        env.over("SVD_SHARE_MIN_BATCH", p.share_min_batch);
        env.over("SVD_GPU_BIG_BATCH_MAX_K", p.gpu_big_batch_max_k);
        env.over("SVD_GPU_BIG_BATCH_MIN", p.gpu_big_batch_min);
        env.over("SVD_VALUES_BAND_MIN_K", p.values_band_min_k);
        env.over("SVD_VALUES_BAND_WIDTH", p.values_band_width);
        env.over("SVD_BAND_MIN_K", p.band_min_k);
        env.over("SVD_BIDIAG_BATCH_MIN_K", p.bidiag_batch_min_k);
        env.over("SVD_BIDIAG_BATCH_MAX_K", p.bidiag_batch_max_k);
        env.over("SVD_BIDIAG_BATCH_MIN_BATCH", p.bidiag_batch_min_batch);
        env.over("SVD_BIDIAG_BATCH_MAX_L", p.bidiag_batch_max_l);
        env.over("SVD_VALUES_BIDIAG_BATCH_MIN_K", p.values_bidiag_batch_min_k);
        env.over("SVD_VALUES_BIDIAG_BATCH_MAX_K", p.values_bidiag_batch_max_k);
        env.over("SVD_VALUES_BIDIAG_BATCH_MIN_BATCH", p.values_bidiag_batch_min_batch);
        env.over("SVD_VALUES_BIDIAG_BATCH_MAX_L", p.values_bidiag_batch_max_l);
        env.over("SVD_SHARE_MIN_K", p.share_min_k);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

// reference: src/svd.mm:400-404
bool svd_wants_block(uint32_t k, uint32_t batch) {
    const metal_linalg_svd_policy& p = svd_state().policy;
    if (k >= p.block_min_k) return true;
    return p.block_min_batch && k >= p.block_min_k_batched && batch >= p.block_min_batch;
}

// reference: src/svd.mm:902-914
const char* svd_gpu_backend(uint32_t m, uint32_t n, uint32_t batch) {
    const metal_linalg_svd_policy& p = svd_state().policy;
    const unsigned long long k = std::min(m, n), l = std::max(m, n);
    if (p.gk_max_k != 0 && k >= p.gk_min_k && k <= std::min<unsigned long long>(p.gk_max_k, kSvdGkMaxK))
        return svd_gk_fits(m, n) ? "golub_kahan" : "qr_golub_kahan";
    const bool precondition = l >= p.qr_min_rows && k >= p.qr_min_k && l >= 2 * k;
    const bool block = svd_wants_block((uint32_t)k, batch);
    if (precondition) return block ? "qr_block_jacobi" : "qr_jacobi";
    return block ? "block_jacobi" : "jacobi";
}

int svd_forced_device() {
    if (env_is("SVD_DEVICE", "gpu")) return 1;
    if (env_is("SVD_DEVICE", "cpu")) return 0;
    return -1;
}

bool svd_gpu_rule(uint32_t m, uint32_t n, uint32_t batch, uint32_t max_k, uint32_t min_bk, uint32_t min_batch,
                  uint32_t max_l) {
    const uint32_t k = std::min(m, n), l = std::max(m, n);
    return k <= max_k && l <= max_l && (unsigned long long)batch * k >= min_bk && batch >= min_batch;
}

// reference: src/svd.mm:936-958
bool svd_uses_gpu(uint32_t m, uint32_t n, uint32_t batch, bool vectors) {
    if (cpu_only()) return false;
    if (const int f = svd_forced_device(); f >= 0) return f == 1;
    const metal_linalg_svd_policy& p = svd_state().policy;
    if (!vectors && p.values_gpu_min_batch != 0)
        return svd_gpu_rule(m, n, batch, p.values_gpu_max_k, p.values_gpu_min_batch_times_k, p.values_gpu_min_batch,
                            p.values_gpu_max_l);
    const uint32_t k = std::min(m, n);
    if (p.gpu_big_batch_min && p.gpu_max_k && k > p.gpu_max_k && k <= p.gpu_big_batch_max_k &&
        std::max(m, n) <= p.gpu_max_l && batch >= p.gpu_big_batch_min)
        return true;
    return svd_gpu_rule(m, n, batch, p.gpu_max_k, p.gpu_min_batch_times_k, p.gpu_min_batch, p.gpu_max_l);
}

// ------------------------------------------------------------ Cholesky ----
State<metal_linalg_cholesky_policy>& cholesky_state() {
    static State<metal_linalg_cholesky_policy> s = [] {
        State<metal_linalg_cholesky_policy> r;
        metal_linalg_cholesky_policy& p = r.policy;
        p = {32, 256, 0, 0, 0, 1, 0, 2048, 0, 0};   // reference defaults (core.h CholeskyPolicy)
        p.gpu_cores = device_id().cus;
        if (device_id().mi355x) {
            p.gpu_max_n = kNoLimit;   // every shape on the GPU
            p.gpu_min_batch_times_n = 0;
            p.gpu_min_batch = 1;
            p.gpu_min_n = 0;
            p.gpu_large_min_n = 0;
            // batched kernels ("simd", "threadgroup") against the blocked path
            p.blocked_min_n = tuned::kCholeskyBlockedMinN;
            p.blocked_max_batch = tuned::kCholeskyBlockedMaxBatch;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("Cholesky", device_id().mi355x);
        EnvList env;
        env.over("CHOLESKY_SIMD_MAX_N", p.simd_max_n);
        env.over("CHOLESKY_BLOCKED_MIN_N", p.blocked_min_n);
        env.over("CHOLESKY_BLOCKED_MAX_BATCH", p.blocked_max_batch);
        env.over("CHOLESKY_GPU_MAX_N", p.gpu_max_n);
        env.over("CHOLESKY_GPU_MIN_BATCH_TIMES_N", p.gpu_min_batch_times_n);
        env.over("CHOLESKY_GPU_MIN_BATCH", p.gpu_min_batch);
        env.over("CHOLESKY_GPU_MIN_N", p.gpu_min_n);
        env.over("CHOLESKY_GPU_LARGE_MIN_N", p.gpu_large_min_n);
        env.over("CHOLESKY_GPU_LARGE_MAX_BATCH", p.gpu_large_max_batch);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

// ------------------------------------------------------------------ LU ----
State<metal_linalg_lu_policy>& lu_state() {
    static State<metal_linalg_lu_policy> s = [] {
        State<metal_linalg_lu_policy> r;
        metal_linalg_lu_policy& p = r.policy;
        p = {2048, 0, 16, 0};   // reference defaults (core.h LuPolicy)
        p.gpu_cores = device_id().cus;
        if (device_id().mi355x) {
            // "blocked": the one-matrix-at-a-time blocked path; "cpu": the
            // batch path, which on this device is the batched GPU kernels
            p.gpu_min_n = tuned::kLuBlockedMinN;
            p.gpu_max_batch = tuned::kLuBlockedMaxBatch;
            p.gpu_solve_min_rhs = 1;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("LU", device_id().mi355x);
        EnvList env;
        env.over("LU_GPU_MIN_N", p.gpu_min_n);
        env.over("LU_GPU_MAX_BATCH", p.gpu_max_batch);
        env.over("LU_GPU_SOLVE_MIN_RHS", p.gpu_solve_min_rhs);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

// ---------------------------------------------------------------- TRSM ----
State<metal_linalg_trsm_policy>& trsm_state() {
    static State<metal_linalg_trsm_policy> s = [] {
        State<metal_linalg_trsm_policy> r;
        metal_linalg_trsm_policy& p = r.policy;
        p = {1024, 256, 0, 0};   // reference defaults (core.h TrsmPolicy)
        p.gpu_cores = device_id().cus;
        if (device_id().mi355x) {
            // as LU's: "blocked" the blocked path, "cpu" the batched kernels
            p.gpu_min_n = tuned::kTrsmBlockedMinN;
            p.gpu_min_rhs = 0;
            p.gpu_max_batch = tuned::kTrsmBlockedMaxBatch;
            r.source = tuned_label();
        } else {
            r.source = untuned_label();
        }
        notice("triangular solve", device_id().mi355x);
        EnvList env;
        env.over("TRSM_GPU_MIN_N", p.gpu_min_n);
        env.over("TRSM_GPU_MIN_RHS", p.gpu_min_rhs);
        env.over("TRSM_GPU_MAX_BATCH", p.gpu_max_batch);
        if (!env.names.empty()) r.source = "env:" + env.names;
        return r;
    }();
    return s;
}

std::atomic<uint32_t> g_cpu_threads{0};

}  // namespace

bool svd_gk_fits(uint32_t m, uint32_t n) { return std::min(m, n) <= kSvdGkMaxK && std::max(m, n) <= kSvdGkMaxK; }

const char* qr_backend_name(uint32_t m, uint32_t n, uint32_t batch) {
    if (!qr_uses_gpu(m, n, batch)) return "cpu";
    // reference: src/qr.mm:231-236
    const metal_linalg_qr_policy& p = qr_state().policy;
    const uint32_t crossover = batch < p.batch_threshold ? p.m_crossover_small_batch : p.m_crossover_large_batch;
    return std::min(m, n) >= crossover ? "streaming_reduced" : "unblocked";
}

// reference: src/eigh.mm:852-870
const char* eigh_backend_name(uint32_t n, uint32_t batch, bool vectors) {
    if (cpu_only()) return "cpu";
    if (env_is("EIGH_DEVICE", "tridiag")) return "tridiag";
    if (env_is("EIGH_DEVICE", "band")) return "band";
    if (env_is("EIGH_DEVICE", "tridiag_batch")) return "tridiag_batch";
    return eigh_uses_gpu(n, batch, vectors) ? eigh_gpu_backend(n, batch) : eigh_cpu_side(n, batch, vectors);
}

// reference: src/svd.mm:966-995
const char* svd_backend_name(uint32_t m, uint32_t n, uint32_t batch, bool vectors) {
    if (cpu_only()) return "cpu";
    if (env_is("SVD_DEVICE", "bidiag")) return "bidiag";
    if (env_is("SVD_DEVICE", "band")) return "band";
    if (env_is("SVD_DEVICE", "bidiag_batch")) return "bidiag_batch";
    if (svd_uses_gpu(m, n, batch, vectors)) return svd_gpu_backend(m, n, batch);
    if (env_is("SVD_DEVICE", "cpu")) return "cpu";
    const metal_linalg_svd_policy& p = svd_state().policy;
    const uint32_t k = std::min(m, n), l = std::max(m, n);
    {
        const uint32_t lo = vectors ? p.bidiag_batch_min_k : p.values_bidiag_batch_min_k;
        const uint32_t hi = vectors ? p.bidiag_batch_max_k : p.values_bidiag_batch_max_k;
        const uint32_t mb = vectors ? p.bidiag_batch_min_batch : p.values_bidiag_batch_min_batch;
        const uint32_t ml = vectors ? p.bidiag_batch_max_l : p.values_bidiag_batch_max_l;
        const bool fits = (l >= 2 * k && k <= 1024) || l <= 1024;
        if (hi != 0 && k >= lo && k <= hi && l <= ml && fits && batch >= std::max(mb, 1u)) return "bidiag_batch";
    }
    const uint32_t cap = vectors ? p.bidiag_max_batch : p.values_bidiag_max_batch;
    if (cap != 0 && batch > cap) return "cpu";
    const uint32_t band = vectors ? p.band_min_k : p.values_band_min_k;
    if (band != 0 && k >= band) return "band";
    const uint32_t from = vectors ? p.bidiag_min_k : p.values_bidiag_min_k;
    return from != 0 && k >= from ? "bidiag" : "cpu";
}

// reference: src/cholesky.mm:134-176
const char* cholesky_backend_name(uint32_t n, uint32_t batch) {
    if (cpu_only()) return "cpu";
    const metal_linalg_cholesky_policy& p = cholesky_state().policy;
    auto kernel = [&]() -> const char* {
        if (const char* e = std::getenv("CHOLESKY_DEVICE")) {
            if (!std::strcmp(e, "simd") && n <= 32) return "simd";
            if (!std::strcmp(e, "threadgroup")) return "threadgroup";
            if (!std::strcmp(e, "blocked")) return "blocked";
        }
        if (n <= std::min(32u, p.simd_max_n)) return "simd";
        if (n >= p.blocked_min_n && (!p.blocked_max_batch || batch <= p.blocked_max_batch)) return "blocked";
        return "threadgroup";
    };
    if (const char* e = std::getenv("CHOLESKY_DEVICE")) {
        if (!std::strcmp(e, "cpu")) return "cpu";
        if (!std::strcmp(e, "gpu") || !std::strcmp(e, "simd") || !std::strcmp(e, "threadgroup") ||
            !std::strcmp(e, "blocked"))
            return kernel();
    }
    bool gpu;
    if (p.gpu_large_min_n && n >= p.gpu_large_min_n && (!p.gpu_large_max_batch || batch <= p.gpu_large_max_batch))
        gpu = true;
    else
        gpu = n >= p.gpu_min_n && n <= p.gpu_max_n && (uint64_t)batch * n >= p.gpu_min_batch_times_n &&
              batch >= std::max(1u, p.gpu_min_batch);
    return gpu ? kernel() : "cpu";
}

// reference: src/lu.mm:116-138
const char* lu_backend_name(uint32_t n, uint32_t batch) {
    if (cpu_only()) return "cpu";
    if (const char* e = std::getenv("LU_DEVICE")) {
        if (!std::strcmp(e, "cpu")) return "cpu";
        if (!std::strcmp(e, "gpu") || !std::strcmp(e, "blocked")) return "blocked";
    }
    const metal_linalg_lu_policy& p = lu_state().policy;
    return p.gpu_min_n && n >= p.gpu_min_n && (!p.gpu_max_batch || batch <= p.gpu_max_batch) ? "blocked" : "cpu";
}

// reference: src/trsm.mm:136-138, 278-286
const char* trsm_backend_name(uint32_t n, uint32_t k, uint32_t batch) {
    if (cpu_only()) return "cpu";
    if (const char* e = std::getenv("TRSM_DEVICE")) {
        if (!std::strcmp(e, "cpu")) return "cpu";
        if (!std::strcmp(e, "gpu") || !std::strcmp(e, "blocked")) return "blocked";
    }
    const metal_linalg_trsm_policy& p = trsm_state().policy;
    return p.gpu_min_n && n >= p.gpu_min_n && k >= p.gpu_min_rhs && (!p.gpu_max_batch || batch <= p.gpu_max_batch)
               ? "blocked"
               : "cpu";
}

metal_linalg_qr_policy& qr_policy() { return qr_state().policy; }
metal_linalg_eigh_policy& eigh_policy() { return eigh_state().policy; }
metal_linalg_svd_policy& svd_policy() { return svd_state().policy; }
metal_linalg_cholesky_policy& cholesky_policy() { return cholesky_state().policy; }
metal_linalg_lu_policy& lu_policy() { return lu_state().policy; }
metal_linalg_trsm_policy& trsm_policy() { return trsm_state().policy; }

const char* policy_source(const char* which) {
    const std::string w = which;
    if (w == "qr") return qr_state().source.c_str();
    if (w == "eigh") return eigh_state().source.c_str();
    if (w == "svd") return svd_state().source.c_str();
    if (w == "cholesky") return cholesky_state().source.c_str();
    if (w == "lu") return lu_state().source.c_str();
    return trsm_state().source.c_str();
}

void mark_user_policy(const char* which) {
    const std::string w = which;
    if (w == "qr") qr_state().source = "user";
    else if (w == "eigh") eigh_state().source = "user";
    else if (w == "svd") svd_state().source = "user";
    else if (w == "cholesky") cholesky_state().source = "user";
    else if (w == "lu") lu_state().source = "user";
    else trsm_state().source = "user";
}

void set_calibration_notices(bool on) { g_notices = on; }

const char* calibration_message(const char* decomposition) {
    thread_local std::string msg;
    msg.clear();
    if (!decomposition) return msg.c_str();
    bool known = false, tuned = false;
    {
        std::lock_guard<std::mutex> lock(g_notice_mutex);
        auto it = g_tuned.find(decomposition);
        if (it != g_tuned.end()) {
            known = true;
            tuned = it->second;
        }
    }
    const DeviceId& d = device_id();
    if (!known || tuned || d.name.empty()) return msg.c_str();
    msg = std::string("metal-linalg: ") + decomposition + " has no routing policy measured on this GPU (" + d.name +
          ", " + d.arch + ", " + std::to_string(d.cus) +
          " CUs); it routes with the library defaults, which may leave speed unused"
          " (METAL_LINALG_NO_CALIBRATION_NOTICE=1 hides this)";
    return msg.c_str();
}

// reference: src/device.mm:72-91
uint32_t cpu_threads() {
    const uint32_t n = g_cpu_threads;
    if (n) return n;
    static const uint32_t def = [] {
        if (const char* s = std::getenv("METAL_LINALG_CPU_THREADS")) {
            const long v = std::strtol(s, nullptr, 10);
            if (v > 0) return (uint32_t)v;
        }
        return std::max(1u, std::thread::hardware_concurrency());
    }();
    return def;
}

void set_cpu_threads(uint32_t n) { g_cpu_threads = n; }

}  // namespace mla
