// ORACLE -- test infrastructure, not product code.
//
// A CPU restatement of the reference library's LAPACK-batched CPU path: the
// same LAPACK routines, called in the same sequence, with the same non-finite
// scan, NaN fills, info words and batch-over-cores scheduling.  It is used
// only by tests/ (as the parity checker), by __graft_entry__.smoke() and by
// bench.py's cpu_baseline leg (as the timed host baseline).  Nothing in
// metal_linalg_amd/ links, loads or calls it.
//
// The reference calls Apple Accelerate, which is absent on Linux.  The same
// LAPACK routines are taken here from the OpenBLAS 0.3.28 build bundled with
// scipy 1.15.3 (exports prefixed "scipy_"), or an unprefixed system LAPACK,
// resolved at run time by oracle_init().  Bit-level agreement with
// Accelerate is therefore not claimed; agreement is pinned by the reference
// tests' known answers and by invariants (tests/test_oracle.py).
//
// Functions and the reference code each restates:
//   scan_matrices      src/metal_runtime.mm:140-177 (Part, |v| <= FLT_MAX)
//   lapack_batches     src/metal_runtime.mm:376-432 (threads, 4 chunks/thread)
//   oracle_qr          src/qr_cpu.mm:32-121
//   oracle_eigh        src/eigh.mm:664-758 (ssyevd, uplo flipped; values-only
//                      two-stage from n = 128, eigh.mm:555,685)
//   oracle_svd         src/svd.mm:772-890
//   oracle_cholesky    src/cholesky_cpu.mm:93-151
//   oracle_lu_factor   src/lu_cpu.mm:87-102
//   oracle_solve       src/lu_cpu.mm:104-133
//   oracle_inv         src/lu_cpu.mm:135-157
//   oracle_solve_triangular  src/trsm.mm:193-206
// Deviation: for eigh/SVD with vectors at n >= 192 on idle cores the
// reference splits ssyevd/sgesdd into their steps around its own divide and
// conquer (eigh.mm:607-660, svd.mm:660-770); this restatement calls the
// LAPACK drivers whole, which run the same steps inside.

#include <dlfcn.h>
#include <link.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <memory>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

using lint = int;   // LP64 LAPACK
using flen = size_t;   // hidden Fortran character-length arguments

// ---- the LAPACK/BLAS entry points, resolved at run time ----
struct Lapack {
    void (*sgeqrf)(const lint*, const lint*, float*, const lint*, float*, float*, const lint*, lint*);
    void (*sorgqr)(const lint*, const lint*, const lint*, float*, const lint*, const float*, float*, const lint*, lint*);
    void (*ssyevd)(const char*, const char*, const lint*, float*, const lint*, float*, float*, const lint*, lint*,
                   const lint*, lint*, flen, flen);
    void (*ssyevd_2stage)(const char*, const char*, const lint*, float*, const lint*, float*, float*, const lint*,
                          lint*, const lint*, lint*, flen, flen);
    void (*sgesdd)(const char*, const lint*, const lint*, float*, const lint*, float*, float*, const lint*, float*,
                   const lint*, float*, const lint*, lint*, lint*, flen);
    void (*spotrf)(const char*, const lint*, float*, const lint*, lint*, flen);
    void (*sgetrf)(const lint*, const lint*, float*, const lint*, lint*, lint*);
    void (*sgetrs)(const char*, const lint*, const lint*, const float*, const lint*, const lint*, float*, const lint*,
                   lint*, flen);
    void (*sgetri)(const lint*, float*, const lint*, const lint*, float*, const lint*, lint*);
    // CBLAS (enum arguments as int: RowMajor 101, ColMajor 102, NoTrans 111,
    // Trans 112, Upper 121, Lower 122, NonUnit 131, Unit 132, Left 141)
    void (*cblas_sgemm)(int, int, int, lint, lint, lint, float, const float*, lint, const float*, lint, float, float*,
                        lint);
    void (*cblas_strsm)(int, int, int, int, int, lint, lint, float, const float*, lint, float*, lint);
    void (*set_num_threads)(int);
    char* (*get_config)();
    std::string name;
};

Lapack g_lapack{};
bool g_ready = false;
thread_local std::string g_error;

enum : int { RowMajor = 101, ColMajor = 102, NoTrans = 111, Trans = 112, Upper = 121, Lower = 122,
             NonUnit = 131, Unit = 132, Left = 141 };

template <class F>
bool resolve(void* h, const char* prefix, const char* name, F& out) {
    std::string s = std::string(prefix) + name;
    out = reinterpret_cast<F>(dlsym(h, s.c_str()));
    return out != nullptr;
}

// ---- the reference's scan (metal_runtime.mm:140-177) ----
enum class Part { all, lower, upper };

void scan_matrices(const float* a, uint32_t batch, uint32_t rows, uint32_t cols, Part part, float* amax,
                   char* finite) {
    const size_t per = (size_t)rows * cols;
    for (uint32_t b = 0; b < batch; ++b) {
        const float* d = a + b * per;
        float m = 0.0f;
        unsigned ok = 1;
        for (uint32_t i = 0; i < rows; ++i) {
            uint32_t j0 = 0, j1 = cols;
            if (part == Part::lower) j1 = std::min(cols, i + 1);
            if (part == Part::upper) j0 = std::min(cols, i);
            for (uint32_t j = j0; j < j1; ++j) {
                const float v = std::fabs(d[(size_t)i * cols + j]);
                ok &= (unsigned)(v <= FLT_MAX);
                m = v > m ? v : m;
            }
        }
        amax[b] = m;
        finite[b] = ok ? 1 : 0;
    }
}

// ---- the reference's batch loop (metal_runtime.mm:402-432) ----
//
// A persistent pool of workers, one per host thread; a call cuts the batch
// into 4 chunks per worker (kChunksPerThread) taken in turn.  Each worker
// calls its own copy of the LAPACK library, loaded into a separate link
// namespace (dlmopen): OpenBLAS serialises concurrent small calls from
// different threads on its buffer-pool lock, which flattened the batch loop
// at about 4 threads when every worker shared one copy.  Worker 0 uses the
// copy oracle_init loaded; a copy that cannot be loaded falls back to it.
uint32_t g_threads = 0;   // 0: every hardware thread

uint32_t thread_count() {
    if (g_threads) return g_threads;
    const unsigned h = std::thread::hardware_concurrency();
    return h ? h : 1;
}

std::string g_path;                              // the library oracle_init loaded
bool resolve_all(void* h, Lapack& L, const std::string& path);   // below
// Copies are loaded into their own link namespaces (dlmopen; each brings its
// own C runtime, so they share nothing), which glibc limits to 16 and static
// TLS space to about 10: 8 copies, two workers sharing one at 16 threads
// (measured: one copy per two workers scales as well as one per worker).
constexpr uint32_t kMaxCopies = 8;
std::vector<std::unique_ptr<Lapack>> g_copies;   // one per worker
thread_local const Lapack* tls_lapack = nullptr;

// The LAPACK of the calling thread (inside a batch: its worker's copy).
const Lapack& lap();

const Lapack* load_copy() {
    const char* old = std::getenv("OPENBLAS_NUM_THREADS");
    const std::string keep = old ? old : "";
    setenv("OPENBLAS_NUM_THREADS", "1", 1);
    void* h = dlmopen(LM_ID_NEWLM, g_path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (old) setenv("OPENBLAS_NUM_THREADS", keep.c_str(), 1);
    else unsetenv("OPENBLAS_NUM_THREADS");
    if (!h) return nullptr;
    auto L = std::make_unique<Lapack>();
    if (!resolve_all(h, *L, g_path)) return nullptr;
    if (L->set_num_threads) L->set_num_threads(1);
    g_copies.push_back(std::move(L));
    return g_copies.back().get();
}

class Pool {
public:
    // Runs job(b0, b1) over `chunks` contiguous pieces of [0, batch) on
    // `workers` workers; rethrows the first exception.
    void run(uint32_t workers, uint32_t batch, uint32_t chunks, const std::function<void(uint32_t, uint32_t)>& job) {
        grow(workers);
        std::unique_lock<std::mutex> lock(m_);
        job_ = &job;
        batch_ = batch;
        chunks_ = chunks;
        next_ = 0;
        active_ = workers;
        pending_ = workers;
        error_ = nullptr;
        ++generation_;
        wake_.notify_all();
        done_.wait(lock, [&] { return pending_ == 0; });
        job_ = nullptr;
        if (error_) std::rethrow_exception(error_);
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lock(m_);
            stop_ = true;
            ++generation_;
        }
        wake_.notify_all();
        for (auto& t : threads_) t.join();
    }

private:
    void grow(uint32_t workers) {
        while (threads_.size() < workers) {
            const uint32_t w = (uint32_t)threads_.size();
            const Lapack* L = &g_lapack;
            const uint32_t slot = w % kMaxCopies;
            while (g_copies.size() <= slot && load_copy()) {}
            if (g_copies.size() > slot) L = g_copies[slot].get();
            threads_.emplace_back([this, w, L] { loop(w, L); });
        }
    }
    void loop(uint32_t w, const Lapack* L) {
        tls_lapack = L;
        uint64_t seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lock(m_);
            wake_.wait(lock, [&] { return generation_ != seen; });
            seen = generation_;
            if (stop_) return;
            if (w >= active_) continue;
            const auto* job = job_;
            lock.unlock();
            for (uint32_t c; !failed_ && (c = next_.fetch_add(1)) < chunks_;) {
                const uint32_t b0 = (uint32_t)((uint64_t)batch_ * c / chunks_);
                const uint32_t b1 = (uint32_t)((uint64_t)batch_ * (c + 1) / chunks_);
                try {
                    (*job)(b0, b1);
                } catch (...) {
                    std::lock_guard<std::mutex> g(m_);
                    if (!error_) error_ = std::current_exception();
                    failed_ = true;
                }
            }
            lock.lock();
            if (--pending_ == 0) {
                failed_ = false;
                done_.notify_all();
            }
        }
    }
    std::mutex m_;
    std::condition_variable wake_, done_;
    std::vector<std::thread> threads_;
    const std::function<void(uint32_t, uint32_t)>* job_ = nullptr;
    uint32_t batch_ = 0, chunks_ = 0, active_ = 0, pending_ = 0;
    std::atomic<uint32_t> next_{0};
    std::atomic<bool> failed_{false};
    std::exception_ptr error_;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

Pool& pool() {
    static Pool* p = new Pool();   // never destroyed: workers outlive static teardown order
    return *p;
}

const Lapack& lap() { return tls_lapack ? *tls_lapack : g_lapack; }

template <class F>
void lapack_batches(uint32_t batch, const F& f) {
    const uint32_t threads = std::min<uint32_t>(thread_count(), batch);
    if (batch <= 1) {
        // one matrix: LAPACK's own threads, as the reference leaves
        // Accelerate threaded there (metal_runtime.mm:413-416)
        if (g_lapack.set_num_threads) g_lapack.set_num_threads((int)thread_count());
        try {
            f(0u, batch);
        } catch (...) {
            if (g_lapack.set_num_threads) g_lapack.set_num_threads(1);
            throw;
        }
        if (g_lapack.set_num_threads) g_lapack.set_num_threads(1);
        return;
    }
    const uint32_t chunks = std::min<uint32_t>(batch, threads * 4);   // kChunksPerThread
    pool().run(threads, batch, chunks, std::function<void(uint32_t, uint32_t)>(f));
}

void transpose(const float* in, size_t ldi, float* out, size_t ldo, uint32_t rows, uint32_t cols) {
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < cols; ++c) out[(size_t)c * ldo + r] = in[(size_t)r * ldi + c];
}

// transpose.h:35
uint32_t padded_ld(uint32_t n) { return n >= 128 ? (n + 15) / 16 * 16 + 16 : std::max(n, 1u); }

void need_ready() {
    if (!g_ready) throw std::runtime_error("oracle: LAPACK not loaded (call oracle_init first)");
}

template <class F>
int guarded(F&& f) {
    try {
        need_ready();
        f();
        return 0;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return 1;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 2;
    }
}

constexpr float kNaN = std::numeric_limits<float>::quiet_NaN();

bool resolve_all(void* h, Lapack& L, const std::string& path) {
    const char* prefixes[] = {"scipy_", ""};
    for (const char* p : prefixes) {
        const bool ok = resolve(h, p, "sgeqrf_", L.sgeqrf) && resolve(h, p, "sorgqr_", L.sorgqr) &&
                        resolve(h, p, "ssyevd_", L.ssyevd) && resolve(h, p, "sgesdd_", L.sgesdd) &&
                        resolve(h, p, "spotrf_", L.spotrf) && resolve(h, p, "sgetrf_", L.sgetrf) &&
                        resolve(h, p, "sgetrs_", L.sgetrs) && resolve(h, p, "sgetri_", L.sgetri) &&
                        resolve(h, p, "cblas_sgemm", L.cblas_sgemm) && resolve(h, p, "cblas_strsm", L.cblas_strsm);
        if (ok) {
            resolve(h, p, "ssyevd_2stage_", L.ssyevd_2stage);
            if (!resolve(h, p, "openblas_set_num_threads", L.set_num_threads)) L.set_num_threads = nullptr;
            if (!resolve(h, p, "openblas_get_config", L.get_config)) L.get_config = nullptr;
            L.name = path + " (prefix '" + p + "')";
            return true;
        }
    }
    return false;
}

}  // namespace

extern "C" {

const char* oracle_last_error(void) { return g_error.c_str(); }

// Loads LAPACK from `path` (scipy's OpenBLAS, or a system LAPACK/OpenBLAS)
// and makes BLAS single-threaded: the batch is spread over this file's own
// workers, one matrix per call, as SingleThreadedBlas does
// (src/blas_threading.h:20-42).  Returns 0 on success.
int oracle_init(const char* path) {
    void* h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        g_error = std::string("oracle: dlopen failed: ") + dlerror();
        return 2;
    }
    Lapack L{};
    if (!resolve_all(h, L, path)) {
        g_error = "oracle: the library lacks the LAPACK routines needed";
        return 2;
    }
    if (L.set_num_threads) L.set_num_threads(1);
    g_lapack = L;
    g_path = path;
    g_ready = true;
    return 0;
}

const char* oracle_lapack_config(void) {
    static std::string s;
    s = g_lapack.name;
    if (g_lapack.get_config) s += std::string(": ") + g_lapack.get_config();
    return s.c_str();
}

void oracle_set_threads(uint32_t n) { g_threads = n; }
uint32_t oracle_threads(void) { return thread_count(); }

// Copies of the LAPACK library loaded for the workers (0 until a batch has
// run on more than one thread).
uint32_t oracle_lapack_copies(void) { return (uint32_t)g_copies.size(); }

// mode: 0 reduced, 1 R alone, 2 complete.  src/qr_cpu.mm:32-121
int oracle_qr(const float* a, uint32_t batch, uint32_t M, uint32_t N, int mode, float* q_out, float* r_out) {
    return guarded([&] {
        const uint32_t K = std::min(M, N);
        const uint32_t QC = mode == 1 ? 0 : mode == 2 ? M : K;   // core.h qr_q_cols
        const uint32_t RR = mode == 2 ? M : K;                  // core.h qr_r_rows
        if (mode == 2 && N == 0 && q_out) {                     // qr.mm:312-317
            std::fill(q_out, q_out + (size_t)batch * M * M, 0.0f);
            for (size_t i = 0; i < (size_t)batch * M; ++i) q_out[i * M + i % M] = 1.0f;
            return;
        }
        if (K == 0 || batch == 0) return;
        const Lapack& L = g_lapack;
        const bool wide = M < N;
        const uint32_t lcols = wide ? K : N;
        const uint32_t wcols = std::max(lcols, QC);
        const lint lm = (lint)M, ln = (lint)lcols, lk = (lint)K, lq = (lint)std::max(QC, K);
        const size_t per = (size_t)M * N;
        lint lwork = 1, query = -1, err = 0;
        float wq = 0.0f, scratch = 0.0f;
        L.sgeqrf(&lm, &ln, &scratch, &lm, &scratch, &wq, &query, &err);
        lwork = std::max<lint>(lwork, (lint)std::ceil(wq));
        L.sorgqr(&lm, &lq, &lk, &scratch, &lm, &scratch, &wq, &query, &err);
        lwork = std::max<lint>(lwork, (lint)std::ceil(wq));

        std::vector<float> amax(batch);
        std::vector<char> finite(batch);
        scan_matrices(a, batch, M, N, Part::all, amax.data(), finite.data());

        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            lint lw = lwork, err = 0;
            std::vector<float> wa((size_t)M * wcols), tau(K), work(lwork);
            for (uint32_t b = b0; b < b1; ++b) {
                float* qb = QC ? q_out + (size_t)b * M * QC : nullptr;
                float* rb = r_out + (size_t)b * RR * N;
                if (!finite[b]) {
                    if (qb) std::fill(qb, qb + (size_t)M * QC, kNaN);
                    std::fill(rb, rb + (size_t)RR * N, kNaN);
                    continue;
                }
                const float* ab = a + b * per;
                transpose(ab, N, wa.data(), M, M, lcols);   // column-major A (A1 if wide)
                L.sgeqrf(&lm, &ln, wa.data(), &lm, tau.data(), work.data(), &lw, &err);
                if (err != 0) throw std::runtime_error("oracle qr: sgeqrf info " + std::to_string(err));
                for (uint32_t i = 0; i < K; ++i)
                    for (uint32_t j = 0; j < lcols; ++j) rb[(size_t)i * N + j] = j >= i ? wa[i + (size_t)j * M] : 0.0f;
                std::fill(rb + (size_t)K * N, rb + (size_t)RR * N, 0.0f);
                if (!qb) {
                    if (wide) {
                        L.sorgqr(&lm, &lk, &lk, wa.data(), &lm, tau.data(), work.data(), &lw, &err);
                        L.cblas_sgemm(RowMajor, NoTrans, NoTrans, (lint)K, (lint)(N - K), (lint)K, 1.0f, wa.data(),
                                      (lint)M, ab + K, (lint)N, 0.0f, rb + K, (lint)N);
                    }
                    continue;
                }
                L.sorgqr(&lm, &lq, &lk, wa.data(), &lm, tau.data(), work.data(), &lw, &err);
                if (err != 0) throw std::runtime_error("oracle qr: sorgqr info " + std::to_string(err));
                transpose(wa.data(), M, qb, QC, QC, M);   // row-major Q, M x QC
                if (wide)
                    L.cblas_sgemm(RowMajor, NoTrans, NoTrans, (lint)K, (lint)(N - K), (lint)K, 1.0f, wa.data(),
                                  (lint)M, ab + K, (lint)N, 0.0f, rb + K, (lint)N);
            }
        });
    });
}

// src/eigh.mm:664-758.  v_out may be NULL (values only), info may be NULL.
int oracle_eigh(const float* a, uint32_t batch, uint32_t n, int lower, float* w_out, float* v_out, uint32_t* info) {
    return guarded([&] {
        if (n == 0 || batch == 0) {
            if (info) std::fill(info, info + batch, 0u);
            return;
        }
        const Lapack& L = g_lapack;
        char jobz = v_out ? 'V' : 'N';
        char uplo = lower ? 'U' : 'L';   // LAPACK sees the row-major matrix transposed
        const bool two_stage = !v_out && n >= 128 && L.ssyevd_2stage != nullptr;
        const bool transpose_in = two_stage && lower;
        if (two_stage) uplo = 'L';
        const size_t per = (size_t)n * n;
        std::vector<float> amax(batch);
        std::vector<char> finite(batch);
        scan_matrices(a, batch, n, n, lower ? Part::lower : Part::upper, amax.data(), finite.data());
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            auto syevd = two_stage ? L.ssyevd_2stage : L.ssyevd;
            char jz = jobz, ul = uplo;
            std::vector<float> wa(per);
            lint N = (lint)n, lwork = -1, liwork = -1, err = 0, liq = 0;
            float lq = 0.0f;
            std::vector<float> wtmp(n);
            syevd(&jz, &ul, &N, wa.data(), &N, wtmp.data(), &lq, &lwork, &liq, &liwork, &err, 1, 1);
            lwork = std::max<lint>(1, (lint)std::ceil(lq));
            liwork = std::max<lint>(1, liq);
            std::vector<float> work(lwork);
            std::vector<lint> iwork(liwork);
            for (uint32_t b = b0; b < b1; ++b) {
                float* w = w_out + (size_t)b * n;
                if (!finite[b]) {
                    std::fill(w, w + n, kNaN);
                    if (v_out) std::fill(v_out + b * per, v_out + (b + 1) * per, kNaN);
                    if (info) info[b] = 1u << 17;
                    continue;
                }
                if (transpose_in) transpose(a + b * per, n, wa.data(), n, n, n);
                else std::memcpy(wa.data(), a + b * per, per * sizeof(float));
                syevd(&jz, &ul, &N, wa.data(), &N, w, work.data(), &lwork, iwork.data(), &liwork, &err, 1, 1);
                if (err != 0) throw std::runtime_error("oracle eigh: ssyevd info " + std::to_string(err));
                if (v_out) transpose(wa.data(), n, v_out + b * per, n, n, n);
                if (info) info[b] = 1u | (1u << 16);
            }
        });
    });
}

// src/svd.mm:772-890.  u/vt both NULL for values only.
int oracle_svd(const float* a, uint32_t batch, uint32_t M, uint32_t N, float* u_out, float* s_out, float* vt_out,
               uint32_t* info) {
    return guarded([&] {
        const uint32_t K = std::min(M, N);
        if (K == 0 || batch == 0) {
            if (info) std::fill(info, info + batch, 0u);
            return;
        }
        const Lapack& L = g_lapack;
        const bool compute_uv = u_out || vt_out;
        const size_t per = (size_t)M * N;
        const bool tall = M >= 2 * N;
        char jobz = compute_uv ? 'S' : 'N';
        const lint lm = (lint)N, ln = (lint)M, lk = (lint)K;
        lint lwork = 1, query = -1, err = 0;
        {
            std::vector<lint> iq(8 * (size_t)K);
            float scratch = 0.0f, q = 0.0f, sdummy[1];
            auto grow = [&](float v) { lwork = std::max<lint>(lwork, (lint)std::ceil(v)); };
            if (tall) {
                L.sgeqrf(&ln, &lk, &scratch, &ln, &scratch, &q, &query, &err);
                grow(q);
                if (compute_uv) {
                    L.sorgqr(&ln, &lk, &lk, &scratch, &ln, &scratch, &q, &query, &err);
                    grow(q);
                }
                L.sgesdd(&jobz, &lk, &lk, &scratch, &lk, sdummy, &scratch, &lk, &scratch, &lk, &q, &query, iq.data(),
                         &err, 1);
                grow(q);
            } else {
                L.sgesdd(&jobz, &lm, &ln, &scratch, &lm, sdummy, &scratch, &lm, &scratch, &lk, &q, &query, iq.data(),
                         &err, 1);
                grow(q);
            }
        }
        std::vector<float> amax(batch);
        std::vector<char> finite(batch);
        scan_matrices(a, batch, M, N, Part::all, amax.data(), finite.data());
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            char jz = jobz;
            lint lw = lwork, err = 0;
            std::vector<float> wa(per), tau(K), r(tall ? (size_t)K * K : 1), work(lwork);
            std::vector<float> spare_u(compute_uv ? (size_t)M * K : 1), spare_vt(compute_uv ? (size_t)K * N : 1);
            std::vector<float> r_u(tall && compute_uv ? (size_t)K * K : 1), r_vt(tall && compute_uv ? (size_t)K * K : 1);
            std::vector<lint> iwork(8 * (size_t)K);
            auto check = [&](const char* routine) {
                if (err != 0) throw std::runtime_error(std::string("oracle svd: ") + routine + " info " + std::to_string(err));
            };
            for (uint32_t b = b0; b < b1; ++b) {
                float* s = s_out + (size_t)b * K;
                float* u = u_out ? u_out + (size_t)b * M * K : spare_u.data();
                float* vt = vt_out ? vt_out + (size_t)b * K * N : spare_vt.data();
                if (!finite[b]) {
                    std::fill(s, s + K, kNaN);
                    if (u_out) std::fill(u, u + (size_t)M * K, kNaN);
                    if (vt_out) std::fill(vt, vt + (size_t)K * N, kNaN);
                    if (info) info[b] = 1u << 17;
                    continue;
                }
                if (!tall) {
                    std::memcpy(wa.data(), a + b * per, per * sizeof(float));
                    L.sgesdd(&jz, &lm, &ln, wa.data(), &lm, s, vt, &lm, u, &lk, work.data(), &lw, iwork.data(), &err, 1);
                    check("sgesdd");
                } else {
                    transpose(a + b * per, N, wa.data(), M, M, N);
                    L.sgeqrf(&ln, &lk, wa.data(), &ln, tau.data(), work.data(), &lw, &err);
                    check("sgeqrf");
                    for (uint32_t j = 0; j < K; ++j)
                        for (uint32_t i = 0; i < K; ++i) r[i + (size_t)j * K] = i <= j ? wa[i + (size_t)j * M] : 0.0f;
                    L.sgesdd(&jz, &lk, &lk, r.data(), &lk, s, r_u.data(), &lk, r_vt.data(), &lk, work.data(), &lw,
                             iwork.data(), &err, 1);
                    check("sgesdd");
                    if (compute_uv) {
                        L.sorgqr(&ln, &lk, &lk, wa.data(), &ln, tau.data(), work.data(), &lw, &err);
                        check("sorgqr");
                        L.cblas_sgemm(RowMajor, Trans, Trans, (lint)M, lk, lk, 1.0f, wa.data(), (lint)M, r_u.data(), lk,
                                      0.0f, u, lk);
                        transpose(r_vt.data(), K, vt, K, K, K);
                    }
                }
                if (info) info[b] = 1u | (1u << 16);
            }
        });
    });
}

// src/cholesky_cpu.mm:93-151
int oracle_cholesky(const float* a, uint32_t batch, uint32_t n, int upper, float* l, uint32_t* info) {
    return guarded([&] {
        if (n == 0 || batch == 0) return;
        const Lapack& L = g_lapack;
        const size_t per = (size_t)n * n;
        const uint32_t ld = n >= 128 ? (n + 15) / 16 * 16 + 16 : n;
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            std::vector<float> w((size_t)n * ld, 0.0f);
            for (uint32_t b = b0; b < b1; ++b) {
                const float* src = a + b * per;
                float* dst = l + b * per;
                // column-major lower triangle: column j of w holds rows j..n-1
                for (uint32_t j = 0; j < n; ++j)
                    for (uint32_t i = j; i < n; ++i)
                        w[(size_t)j * ld + i] = upper ? src[(size_t)j * n + i] : src[(size_t)i * n + j];
                lint ln = (lint)n, lld = (lint)ld, err = 0;
                char uplo = 'L';
                L.spotrf(&uplo, &ln, w.data(), &lld, &err, 1);
                if (err < 0) throw std::runtime_error("oracle cholesky: spotrf argument " + std::to_string(-err));
                if (err == 0)
                    for (uint32_t k = 0; k < n; ++k)
                        if (!std::isfinite(w[(size_t)k * ld + k])) {
                            err = (lint)k + 1;
                            break;
                        }
                if (err > 0) {
                    std::fill(dst, dst + per, kNaN);
                } else {
                    for (uint32_t i = 0; i < n; ++i)
                        for (uint32_t j = 0; j < n; ++j) {
                            // L(i, j) = w[j * ld + i] for i >= j
                            const bool in = upper ? j >= i : i >= j;
                            const float v = upper ? w[(size_t)i * ld + j] : w[(size_t)j * ld + i];
                            dst[(size_t)i * n + j] = in ? v : 0.0f;
                        }
                }
                if (info) info[b] = (uint32_t)err;
            }
        });
    });
}

// src/lu_cpu.mm:87-102
int oracle_lu_factor(const float* a, uint32_t batch, uint32_t n, float* lu, uint32_t* pivots, uint32_t* info) {
    return guarded([&] {
        if (n == 0 || batch == 0) return;
        const Lapack& L = g_lapack;
        const size_t per = (size_t)n * n;
        const uint32_t ld = padded_ld(n);
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            std::vector<float> w((size_t)n * ld);
            std::vector<lint> ipiv(n);
            for (uint32_t b = b0; b < b1; ++b) {
                transpose(a + b * per, n, w.data(), ld, n, n);
                lint ln = (lint)n, lld = (lint)ld, err = 0;
                L.sgetrf(&ln, &ln, w.data(), &lld, ipiv.data(), &err);
                if (err < 0) throw std::runtime_error("oracle lu: sgetrf argument " + std::to_string(-err));
                transpose(w.data(), ld, lu + b * per, n, n, n);
                for (uint32_t k = 0; k < n; ++k) pivots[(size_t)b * n + k] = (uint32_t)(ipiv[k] - 1);
                if (info) info[b] = (uint32_t)err;
            }
        });
    });
}

// src/lu_cpu.mm:104-133
int oracle_solve(const float* a, uint32_t batch, uint32_t n, const float* bm, uint32_t nrhs, float* x,
                 uint32_t* info) {
    return guarded([&] {
        if (n == 0 || batch == 0 || nrhs == 0) {
            if (info) std::fill(info, info + batch, 0u);
            return;
        }
        const Lapack& L = g_lapack;
        const size_t per = (size_t)n * n, bper = (size_t)n * nrhs;
        const uint32_t ld = padded_ld(n);
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            std::vector<float> w((size_t)n * ld), bw((size_t)nrhs * ld);
            std::vector<lint> ipiv(n);
            for (uint32_t b = b0; b < b1; ++b) {
                transpose(a + b * per, n, w.data(), ld, n, n);
                lint ln = (lint)n, lld = (lint)ld, err = 0;
                L.sgetrf(&ln, &ln, w.data(), &lld, ipiv.data(), &err);
                if (err < 0) throw std::runtime_error("oracle solve: sgetrf argument " + std::to_string(-err));
                float* out = x + b * bper;
                if (info) info[b] = (uint32_t)err;
                if (err > 0) {
                    std::fill(out, out + bper, kNaN);
                    continue;
                }
                transpose(bm + b * bper, nrhs, bw.data(), ld, n, nrhs);
                char trans = 'N';
                lint lr = (lint)nrhs, e2 = 0;
                L.sgetrs(&trans, &ln, &lr, w.data(), &lld, ipiv.data(), bw.data(), &lld, &e2, 1);
                transpose(bw.data(), ld, out, nrhs, nrhs, n);
            }
        });
    });
}

// src/lu_cpu.mm:135-157
int oracle_inv(const float* a, uint32_t batch, uint32_t n, float* x, uint32_t* info) {
    return guarded([&] {
        if (n == 0 || batch == 0) return;
        const Lapack& L = g_lapack;
        const size_t per = (size_t)n * n;
        const uint32_t ld = padded_ld(n);
        const size_t lwork = (size_t)n * 64;
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            std::vector<float> w((size_t)n * ld), work(lwork);
            std::vector<lint> ipiv(n);
            for (uint32_t b = b0; b < b1; ++b) {
                transpose(a + b * per, n, w.data(), ld, n, n);
                lint ln = (lint)n, lld = (lint)ld, err = 0;
                L.sgetrf(&ln, &ln, w.data(), &lld, ipiv.data(), &err);
                float* out = x + b * per;
                if (info) info[b] = (uint32_t)err;
                if (err > 0) {
                    std::fill(out, out + per, kNaN);
                    continue;
                }
                lint lw = (lint)lwork, e2 = 0;
                L.sgetri(&ln, w.data(), &lld, ipiv.data(), work.data(), &lw, &e2);
                transpose(w.data(), ld, out, n, n, n);
            }
        });
    });
}

// src/trsm.mm:193-206
int oracle_solve_triangular(const float* a, uint32_t batch, uint32_t n, const float* b, uint32_t nrhs, int upper,
                            int unit, float* x) {
    return guarded([&] {
        if (n == 0 || batch == 0 || nrhs == 0) return;
        const Lapack& L = g_lapack;
        const size_t per = (size_t)n * n, bper = (size_t)n * nrhs;
        lapack_batches(batch, [&](uint32_t b0, uint32_t b1) {
            const Lapack& L = lap();
            for (uint32_t m = b0; m < b1; ++m) {
                std::copy(b + m * bper, b + (m + 1) * bper, x + m * bper);
                L.cblas_strsm(RowMajor, Left, upper ? Upper : Lower, NoTrans, unit ? Unit : NonUnit, (lint)n,
                              (lint)nrhs, 1.0f, a + m * per, (lint)n, x + m * bper, (lint)nrhs);
            }
        });
    });
}

}  // extern "C"
