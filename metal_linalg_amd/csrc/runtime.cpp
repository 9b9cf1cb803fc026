// Runtime implementation: device, per-call staging, workspace, kernel timing.
#include "runtime.hpp"

#include "entry.hpp"

#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <map>
#include <thread>
#include <utility>

namespace mla {

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory) throw std::bad_alloc();
    throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

void invalid(const std::string& what) { throw std::invalid_argument(what); }

namespace {

std::mutex g_call_mutex;

struct DeviceState {
    Device dev;
    bool ok = false;
    std::string error;
};

DeviceState& state() {
    static DeviceState s = [] {
        DeviceState st;
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            st.error = "no HIP device is available";
            return st;
        }
        int id = 0;
        if (hipGetDevice(&id) != hipSuccess) id = 0;
        hipDeviceProp_t p{};
        if (hipGetDeviceProperties(&p, id) != hipSuccess) {
            (void)hipGetLastError();
            st.error = "hipGetDeviceProperties failed";
            return st;
        }
        st.dev.id = id;
        st.dev.name = p.name;
        st.dev.arch = p.gcnArchName;
        st.dev.cus = (uint32_t)p.multiProcessorCount;
        st.dev.lds_per_block = p.sharedMemPerBlock;
        // A blocking stream at default priority: ordered after work the
        // caller queued on the null stream (torch's default stream).
        if (hipStreamCreate(&st.dev.stream) != hipSuccess) {
            (void)hipGetLastError();
            st.error = "hipStreamCreate failed";
            return st;
        }
        st.ok = true;
        return st;
    }();
    return s;
}

// Grow-only device allocations, reused across calls (calls are serialised).
struct Workspace {
    std::vector<std::pair<void*, size_t>> slots;
};
Workspace& workspace() {
    static Workspace w;
    return w;
}

// ---- timing ----
bool g_timing = false;
struct Pending { const char* name; hipEvent_t a, b; };
std::vector<Pending>& pending() {
    static std::vector<Pending> p;
    return p;
}
std::map<std::string, std::pair<uint64_t, double>>& totals() {
    static std::map<std::string, std::pair<uint64_t, double>> t;
    return t;
}
std::vector<hipEvent_t>& event_pool() {
    static std::vector<hipEvent_t> p;
    return p;
}
hipEvent_t get_event() {
    auto& pool = event_pool();
    if (!pool.empty()) {
        hipEvent_t e = pool.back();
        pool.pop_back();
        return e;
    }
    hipEvent_t e;
    MLA_HIP(hipEventCreate(&e));
    return e;
}

}  // namespace

namespace {

// 0: pageable host memory (or unknown to HIP), 1: pinned host memory,
// 2: device (or managed) memory
int memory_kind(const void* p) {
    if (!p) return 0;
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged || attr.type == hipMemoryTypeUnified)
        return 2;
    return attr.type == hipMemoryTypeHost ? 1 : 0;
}

}  // namespace

bool is_device_memory(const void* p) { return memory_kind(p) == 2; }

std::string& last_error_message() {
    thread_local std::string message;
    return message;
}

metal_linalg_status status_of_current_exception() noexcept {
    try {
        throw;
    } catch (const std::invalid_argument& e) {
        last_error_message() = e.what();
        return METAL_LINALG_INVALID_ARGUMENT;
    } catch (const std::bad_alloc&) {
        last_error_message() = "out of memory";
        return METAL_LINALG_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        last_error_message() = e.what();
        return METAL_LINALG_RUNTIME_ERROR;
    } catch (...) {
        last_error_message() = "unknown error";
        return METAL_LINALG_RUNTIME_ERROR;
    }
}

bool have_device() { return state().ok; }

Device& device() {
    DeviceState& s = state();
    if (!s.ok) throw std::runtime_error("metal_linalg: " + s.error);
    return s.dev;
}

bool timing_enabled() { return g_timing; }

void timing_collect() {
    for (auto& p : pending()) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& t = totals()[p.name];
            t.first += 1;
            t.second += ms;
        } else {
            (void)hipGetLastError();
        }
        event_pool().push_back(p.a);
        event_pool().push_back(p.b);
    }
    pending().clear();
}

KernelTimer::KernelTimer(const char* name, hipStream_t s) : name_(name), s_(s), on_(g_timing) {
    if (!on_) return;
    a_ = get_event();
    b_ = get_event();
    MLA_HIP(hipEventRecord(a_, s_));
}

void KernelTimer::stop() {
    if (!on_ || stopped_) return;
    stopped_ = true;
    MLA_HIP(hipEventRecord(b_, s_));
    pending().push_back({name_, a_, b_});
}

KernelTimer::~KernelTimer() {
    if (on_ && !stopped_) {
        if (hipEventRecord(b_, s_) == hipSuccess) pending().push_back({name_, a_, b_});
        else (void)hipGetLastError();
    }
}

Call::Call() : lock_(g_call_mutex), dev_(device()) { MLA_HIP(hipSetDevice(dev_.id)); }

void sync_copy_stream();   // below

Call::~Call() {
    // On an exception the streams may still hold work on our buffers.
    if (!back_.empty() || slot_ != 0) {
        (void)hipStreamSynchronize(dev_.stream);
        sync_copy_stream();
    }
}

void* Call::take(size_t bytes) {
    auto& ws = workspace().slots;
    const size_t need = std::max<size_t>(bytes, 256);
    if (slot_ == ws.size()) ws.push_back({nullptr, 0});
    auto& s = ws[slot_++];
    if (s.second < need) {
        if (s.first) {
            MLA_HIP(hipStreamSynchronize(dev_.stream));
            MLA_HIP(hipFree(s.first));
            s.first = nullptr;
            s.second = 0;
        }
        const size_t round = size_t(2) << 20;
        const size_t sz = (need + round - 1) / round * round;
        MLA_HIP(hipMalloc(&s.first, sz));
        s.second = sz;
    }
    return s.first;
}

const void* Call::input(const void* p, size_t bytes) {
    if (bytes == 0) return p;
    if (is_device_memory(p)) return p;
    void* d = take(bytes);
    MLA_HIP(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, dev_.stream));
    return d;
}

void* Call::output(void* p, size_t bytes) {
    if (!p) return nullptr;
    if (bytes == 0) return p;
    if (is_device_memory(p)) return p;
    void* d = take(bytes);
    back_.push_back({p, d, bytes});
    return d;
}

void* Call::scratch(size_t bytes) { return take(bytes); }

// ---- batched calls through pinned staging ----

namespace {

// Host traffic per chunk, and the fewest matrices per chunk: the batched
// kernels give each matrix a wave (or a few lanes), so a chunk smaller than
// the device's width takes as long as a full one (the SVD's 204-matrix
// chunks of 16 MB each ran at the latency of a full batch: 13.3 ms for the
// 2048-matrix config against 0.37 ms of kernels).
constexpr size_t kChunkBytes = size_t(32) << 20;
constexpr uint64_t kMinChunk = 1024;

// Pinned host memory, grow-only, two slots (hipHostMalloc: the memory is
// allocated pinned, never registered after the fact).
struct PinnedSlots {
    void* p[2] = {nullptr, nullptr};
    size_t bytes = 0;
    void* get(int slot, size_t need) {
        if (need > bytes) {
            for (auto& q : p)
                if (q) {
                    (void)hipHostFree(q);
                    q = nullptr;
                }
            bytes = 0;
            const size_t round = size_t(4) << 20;
            const size_t sz = (need + round - 1) / round * round;
            for (auto& q : p) MLA_HIP(hipHostMalloc(&q, sz, hipHostMallocDefault));
            bytes = sz;
        }
        return p[slot];
    }
};

// Device slots of the all-pinned path: every chunk is queued at once, and
// chunk k reuses slot k mod kSlots after chunk k - kSlots's download.
constexpr int kSlots = 4;

struct Staging {
    PinnedSlots pinned;
    hipStream_t copy = nullptr, down = nullptr;   // host-to-device, device-to-host (the link is full duplex)
    hipEvent_t ev_in[kSlots] = {}, ev_kern[kSlots] = {}, ev_out[kSlots] = {};
    bool ready = false;
    void init() {
        if (ready) return;
        MLA_HIP(hipStreamCreate(&copy));   // default priority
        MLA_HIP(hipStreamCreate(&down));
        for (int i = 0; i < kSlots; ++i) {
            MLA_HIP(hipEventCreateWithFlags(&ev_in[i], hipEventDisableTiming));
            MLA_HIP(hipEventCreateWithFlags(&ev_kern[i], hipEventDisableTiming));
            MLA_HIP(hipEventCreateWithFlags(&ev_out[i], hipEventDisableTiming));
        }
        ready = true;
    }
};

Staging& staging() {
    static Staging s;
    return s;
}

// memcpy over a few threads for large pieces (one thread's copy does not
// reach the host's memory bandwidth); small ones on the calling thread.
class CopyPool {
public:
    void copy(void* dst, const void* src, size_t bytes) {
        const size_t kMinPiece = size_t(256) << 10;
        const unsigned n = (unsigned)std::min<size_t>(threads(), bytes / kMinPiece);
        if (n <= 1) {
            std::memcpy(dst, src, bytes);
            return;
        }
        std::unique_lock<std::mutex> lock(m_);
        dst_ = static_cast<char*>(dst);
        src_ = static_cast<const char*>(src);
        bytes_ = bytes;
        parts_ = n;
        pending_ = n - 1;
        ++gen_;
        wake_.notify_all();
        lock.unlock();
        piece(0);   // the caller copies piece 0
        lock.lock();
        done_.wait(lock, [&] { return pending_ == 0; });
    }

private:
    unsigned threads() {
        if (pool_.empty()) {
            const unsigned hw = std::thread::hardware_concurrency();
            const unsigned t = std::max(1u, std::min(16u, hw ? hw : 1u));
            for (unsigned i = 1; i < t; ++i) pool_.emplace_back([this, i] { loop(i); });
            size_ = t;
        }
        return size_;
    }
    void piece(unsigned i) {
        const size_t per = (bytes_ + parts_ - 1) / parts_;
        const size_t b0 = std::min(bytes_, per * i), b1 = std::min(bytes_, b0 + per);
        if (b1 > b0) std::memcpy(dst_ + b0, src_ + b0, b1 - b0);
    }
    void loop(unsigned i) {
        uint64_t seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lock(m_);
            wake_.wait(lock, [&] { return gen_ != seen; });
            seen = gen_;
            if (i >= parts_) continue;
            lock.unlock();
            piece(i);
            lock.lock();
            if (--pending_ == 0) done_.notify_all();
        }
    }
    std::mutex m_;
    std::condition_variable wake_, done_;
    std::vector<std::thread> pool_;
    unsigned size_ = 1, parts_ = 0, pending_ = 0;
    uint64_t gen_ = 0;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t bytes_ = 0;
};

CopyPool& copy_pool() {
    static CopyPool* p = new CopyPool();   // threads live as long as the process
    return *p;
}

bool all_device(const std::vector<Call::Slice>& slices) {
    for (const auto& sl : slices) {
        if (sl.in && !is_device_memory(sl.in)) return false;
        if (sl.out && !is_device_memory(sl.out)) return false;
    }
    return true;
}

}  // namespace

void sync_copy_stream() {
    if (staging().ready) {
        (void)hipStreamSynchronize(staging().copy);
        (void)hipStreamSynchronize(staging().down);
    }
}

uint32_t Call::chunk_size(uint32_t batch, const std::vector<Slice>& slices) const {
    if (batch == 0 || all_device(slices)) return batch;
    size_t host = 0;
    for (const auto& sl : slices)
        if ((sl.in && !is_device_memory(sl.in)) || (sl.out && !is_device_memory(sl.out))) host += sl.per;
    const uint64_t c = host ? std::max<uint64_t>(kMinChunk, kChunkBytes / host) : batch;
    return (uint32_t)std::min<uint64_t>(c, batch);
}

void Call::batched(uint32_t batch, const std::vector<Slice>& slices, const ChunkLaunch& launch) {
    if (batch == 0) return;
    const size_t ns = slices.size();
    std::vector<void*> dev(ns);
    if (all_device(slices)) {
        for (size_t i = 0; i < ns; ++i) dev[i] = slices[i].in ? const_cast<void*>(slices[i].in) : slices[i].out;
        launch(dev.data(), batch, dev_.stream);
        return;
    }
    const uint32_t chunk = chunk_size(batch, slices);
    // per slice: host-staged (1 in, 2 out) or in place, its offset in a
    // slot's buffers, and whether the host side is the caller's own pinned
    // memory (then the transfers use it directly: no host copy)
    std::vector<char> staged(ns, 0), pinned(ns, 0);
    std::vector<size_t> off(ns, 0);
    size_t in_bytes = 0, out_bytes = 0;
    for (size_t i = 0; i < ns; ++i) {
        const auto& sl = slices[i];
        const int kind = memory_kind(sl.in ? sl.in : sl.out);
        if (kind == 2 || (!sl.in && !sl.out)) continue;
        pinned[i] = kind == 1;
        if (sl.in) {
            staged[i] = 1;
            off[i] = in_bytes;
            in_bytes += sl.per * chunk;
        } else {
            staged[i] = 2;
            off[i] = out_bytes;
            out_bytes += sl.per * chunk;
        }
    }
    Staging& st = staging();
    st.init();
    const size_t slot_bytes = in_bytes + out_bytes;
    bool all_pinned = true;
    for (size_t i = 0; i < ns; ++i)
        if (staged[i] && !pinned[i]) all_pinned = false;
    if (all_pinned) {
        pinned_chunks(batch, chunk, slices, staged, off, in_bytes, slot_bytes, launch);
        return;
    }
    char* dslot[2] = {static_cast<char*>(take(slot_bytes)), static_cast<char*>(take(slot_bytes))};
    char* hslot[2] = {static_cast<char*>(st.pinned.get(0, slot_bytes)), static_cast<char*>(st.pinned.get(1, slot_bytes))};
    const uint32_t nchunks = (uint32_t)((batch + chunk - 1) / chunk);
    auto range = [&](uint32_t k, uint32_t& b0, uint32_t& nb) {
        b0 = k * chunk;
        nb = std::min(chunk, batch - b0);
    };
    // the host side of chunk k's outputs, once its transfers are done
    auto drain = [&](uint32_t k) {
        const int s = (int)(k & 1);
        MLA_HIP(hipEventSynchronize(st.ev_out[s]));
        uint32_t b0, nb;
        range(k, b0, nb);
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 2 && !pinned[i])
                copy_pool().copy(static_cast<char*>(slices[i].out) + (size_t)b0 * slices[i].per,
                                 hslot[s] + in_bytes + off[i], (size_t)nb * slices[i].per);
    };
    // the host end of a staged slice's transfer for chunk b0: the caller's
    // pinned buffer itself, or the pinned slot
    auto host_end = [&](size_t i, int s, uint32_t b0) -> char* {
        if (pinned[i]) {
            const auto& sl = slices[i];
            return (sl.in ? const_cast<char*>(static_cast<const char*>(sl.in)) : static_cast<char*>(sl.out)) +
                   (size_t)b0 * sl.per;
        }
        return hslot[s] + (staged[i] == 2 ? in_bytes : 0) + off[i];
    };
    for (uint32_t k = 0; k < nchunks; ++k) {
        const int s = (int)(k & 1);
        uint32_t b0, nb;
        range(k, b0, nb);
        // chunk k - 2 used this slot: drained at step k - 1 (its kernel and
        // both transfers are complete)
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 1 && !pinned[i])
                copy_pool().copy(hslot[s] + off[i], static_cast<const char*>(slices[i].in) + (size_t)b0 * slices[i].per,
                                 (size_t)nb * slices[i].per);
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 1)
                MLA_HIP(hipMemcpyAsync(dslot[s] + off[i], host_end(i, s, b0), (size_t)nb * slices[i].per,
                                       hipMemcpyHostToDevice, st.copy));
        MLA_HIP(hipEventRecord(st.ev_in[s], st.copy));
        MLA_HIP(hipStreamWaitEvent(dev_.stream, st.ev_in[s], 0));
        for (size_t i = 0; i < ns; ++i) {
            const auto& sl = slices[i];
            if (staged[i] == 1) dev[i] = dslot[s] + off[i];
            else if (staged[i] == 2) dev[i] = dslot[s] + in_bytes + off[i];
            else if (sl.in) dev[i] = const_cast<char*>(static_cast<const char*>(sl.in)) + (size_t)b0 * sl.per;
            else dev[i] = sl.out ? static_cast<char*>(sl.out) + (size_t)b0 * sl.per : nullptr;
        }
        launch(dev.data(), nb, dev_.stream);
        MLA_HIP(hipEventRecord(st.ev_kern[s], dev_.stream));
        MLA_HIP(hipStreamWaitEvent(st.down, st.ev_kern[s], 0));
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 2)
                MLA_HIP(hipMemcpyAsync(host_end(i, s, b0), dslot[s] + in_bytes + off[i], (size_t)nb * slices[i].per,
                                       hipMemcpyDeviceToHost, st.down));
        MLA_HIP(hipEventRecord(st.ev_out[s], st.down));
        if (k > 0) drain(k - 1);
    }
    drain(nchunks - 1);
}

// Every host buffer is the caller's pinned memory: no host copies, so the
// host only queues.  Uploads run back to back on the copy stream, each
// chunk's kernel waits for its upload, its download for its kernel, and an
// upload into a reused slot for that slot's previous download; the host
// waits once, for the last download.
void Call::pinned_chunks(uint32_t batch, uint32_t chunk, const std::vector<Slice>& slices,
                         const std::vector<char>& staged, const std::vector<size_t>& off, size_t in_bytes,
                         size_t slot_bytes, const ChunkLaunch& launch) {
    Staging& st = staging();
    const size_t ns = slices.size();
    const uint32_t nchunks = (uint32_t)((batch + chunk - 1) / chunk);
    const int nslots = (int)std::min<uint32_t>(kSlots, nchunks);
    char* dslot[kSlots] = {};
    for (int s = 0; s < nslots; ++s) dslot[s] = static_cast<char*>(take(slot_bytes));
    std::vector<void*> dev(ns);
    for (uint32_t k = 0; k < nchunks; ++k) {
        const int s = (int)(k % kSlots);
        const uint32_t b0 = k * chunk, nb = std::min(chunk, batch - b0);
        if (k >= (uint32_t)kSlots) MLA_HIP(hipStreamWaitEvent(st.copy, st.ev_out[s], 0));
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 1)
                MLA_HIP(hipMemcpyAsync(dslot[s] + off[i], static_cast<const char*>(slices[i].in) + (size_t)b0 * slices[i].per,
                                       (size_t)nb * slices[i].per, hipMemcpyHostToDevice, st.copy));
        MLA_HIP(hipEventRecord(st.ev_in[s], st.copy));
        MLA_HIP(hipStreamWaitEvent(dev_.stream, st.ev_in[s], 0));
        for (size_t i = 0; i < ns; ++i) {
            const auto& sl = slices[i];
            if (staged[i] == 1) dev[i] = dslot[s] + off[i];
            else if (staged[i] == 2) dev[i] = dslot[s] + in_bytes + off[i];
            else if (sl.in) dev[i] = const_cast<char*>(static_cast<const char*>(sl.in)) + (size_t)b0 * sl.per;
            else dev[i] = sl.out ? static_cast<char*>(sl.out) + (size_t)b0 * sl.per : nullptr;
        }
        launch(dev.data(), nb, dev_.stream);
        MLA_HIP(hipEventRecord(st.ev_kern[s], dev_.stream));
        MLA_HIP(hipStreamWaitEvent(st.down, st.ev_kern[s], 0));
        for (size_t i = 0; i < ns; ++i)
            if (staged[i] == 2)
                MLA_HIP(hipMemcpyAsync(static_cast<char*>(slices[i].out) + (size_t)b0 * slices[i].per,
                                       dslot[s] + in_bytes + off[i], (size_t)nb * slices[i].per, hipMemcpyDeviceToHost,
                                       st.down));
        MLA_HIP(hipEventRecord(st.ev_out[s], st.down));
    }
    MLA_HIP(hipEventSynchronize(st.ev_out[(nchunks - 1) % kSlots]));
}

void Call::finish() {
    MLA_HIP(hipGetLastError());
    for (auto& b : back_) MLA_HIP(hipMemcpyAsync(b.host, b.dev, b.bytes, hipMemcpyDeviceToHost, dev_.stream));
    MLA_HIP(hipStreamSynchronize(dev_.stream));
    back_.clear();
    slot_ = 0;
    if (g_timing) timing_collect();
}

}  // namespace mla

// ---- HIP-specific extensions (no counterpart in the reference) ----
extern "C" {

void metal_linalg_hip_set_timing(int on) {
    std::lock_guard<std::mutex> lock(mla::g_call_mutex);
    mla::g_timing = on != 0;
}

void metal_linalg_hip_reset_timing(void) {
    std::lock_guard<std::mutex> lock(mla::g_call_mutex);
    mla::totals().clear();
}

int metal_linalg_hip_kernel_time(const char* name, uint64_t* launches, double* total_ms) {
    std::lock_guard<std::mutex> lock(mla::g_call_mutex);
    auto it = mla::totals().find(name ? name : "");
    if (it == mla::totals().end()) {
        if (launches) *launches = 0;
        if (total_ms) *total_ms = 0.0;
        return 0;
    }
    if (launches) *launches = it->second.first;
    if (total_ms) *total_ms = it->second.second;
    return 1;
}

// Names of the timed kernels, separated by '\n' (valid until the next call).
const char* metal_linalg_hip_kernel_names(void) {
    static std::string s;
    std::lock_guard<std::mutex> lock(mla::g_call_mutex);
    s.clear();
    for (auto& kv : mla::totals()) {
        s += kv.first;
        s += '\n';
    }
    return s.c_str();
}

metal_linalg_status metal_linalg_hip_stream_wait(void* stream) {
    return mla::run_entry([&] {
        std::lock_guard<std::mutex> lock(mla::g_call_mutex);
        mla::Device& d = mla::device();
        MLA_HIP(hipSetDevice(d.id));
        static hipEvent_t ev = nullptr;   // re-recorded each time; a wait takes the record current when made
        if (!ev) MLA_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        MLA_HIP(hipEventRecord(ev, static_cast<hipStream_t>(stream)));
        MLA_HIP(hipStreamWaitEvent(d.stream, ev, 0));
    });
}

const char* metal_linalg_hip_arch(void) {
    static std::string s;
    s = mla::have_device() ? mla::device().arch : std::string();
    return s.c_str();
}

}  // extern "C"
