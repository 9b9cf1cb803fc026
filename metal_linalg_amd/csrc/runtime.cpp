// Runtime implementation: device, per-call staging, workspace, kernel timing.
#include "runtime.hpp"

#include "entry.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
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

bool is_device_memory(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
           attr.type == hipMemoryTypeUnified;
}

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

Call::~Call() {
    // On an exception the stream may still hold work reading our buffers.
    if (!back_.empty() || slot_ != 0) (void)hipStreamSynchronize(dev_.stream);
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

const char* metal_linalg_hip_arch(void) {
    static std::string s;
    s = mla::have_device() ? mla::device().arch : std::string();
    return s.c_str();
}

}  // extern "C"
