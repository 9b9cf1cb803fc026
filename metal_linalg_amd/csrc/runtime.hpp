// Runtime for the MI355X build: the HIP device and the library's stream,
// per-call staging of caller buffers (host or device), a grow-only device
// workspace cache, and optional per-kernel HIP-event timing.
//
// Takes the place of the reference's MetalRuntime / input_buffer / wrap_host /
// copy_out (src/metal_runtime.h:36-215): on Apple unified memory the reference
// wraps host memory in place; on a discrete GPU a host pointer is copied to
// HBM and back, and a device pointer is used in place.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace mla {

// Throws std::runtime_error naming the failed HIP call.
void hip_check(hipError_t e, const char* what);
#define MLA_HIP(call) ::mla::hip_check((call), #call)

struct Device {
    int id = 0;
    hipStream_t stream = nullptr;
    std::string name;       // marketing name
    std::string arch;       // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    uint32_t cus = 0;       // compute units
    size_t lds_per_block = 0;
};

// The device the library computes on (HIP's current device at first use),
// initialised once.  Throws if there is no usable GPU.
Device& device();
// True when a GPU is present; never throws.
bool have_device();

// One decomposition call: classifies the caller's pointers, stages host
// buffers through device memory, and makes the call synchronous.  Calls are
// serialised by a process-wide lock held for the object's lifetime (the
// workspace cache is shared).
class Call {
public:
    Call();
    ~Call();
    Call(const Call&) = delete;
    Call& operator=(const Call&) = delete;

    hipStream_t stream() const { return dev_.stream; }

    // A device pointer to `bytes` of input: `p` itself when it is device
    // memory, else a staged copy.
    const void* input(const void* p, size_t bytes);
    template <class T> const T* in(const T* p, size_t count) {
        return static_cast<const T*>(input(p, count * sizeof(T)));
    }
    // A device pointer to `bytes` of output: `p` itself when it is device
    // memory, else scratch copied back to `p` by finish().  NULL stays NULL.
    void* output(void* p, size_t bytes);
    template <class T> T* out(T* p, size_t count) { return static_cast<T*>(output(p, count * sizeof(T))); }
    // Device scratch that lives until the call ends.
    void* scratch(size_t bytes);
    template <class T> T* tmp(size_t count) { return static_cast<T*>(scratch(count * sizeof(T))); }

    // Waits for the kernels, copies host outputs back, checks for errors.
    void finish();

    // ---- batched calls of independent matrices ----
    // One caller buffer of a batched call: an input (`in`) or an output
    // (`out`, NULL allowed), `per` bytes per matrix.
    struct Slice {
        const void* in = nullptr;
        void* out = nullptr;
        size_t per = 0;
    };
    // Device pointers of a chunk's slices (in the order given), the chunk's
    // matrix count and the stream to launch on.
    using ChunkLaunch = std::function<void(void* const* dev, uint32_t count, hipStream_t s)>;
    // Matrices per launch that batched() will use: the whole batch when
    // every buffer is device memory, else a chunk of about kChunkBytes of
    // host traffic.  Size per-launch scratch with it.
    uint32_t chunk_size(uint32_t batch, const std::vector<Slice>& slices) const;
    // Runs a batched call.  Device buffers are used in place and the whole
    // batch is one launch.  When any buffer is host memory the batch runs in
    // chunks (uploads and downloads on two more streams, ordered by events).
    // Pageable buffers go through pinned staging, two chunks in flight: the
    // host copies of one chunk, the transfers of another and the kernels of
    // a third overlap.  When every host buffer is the caller's pinned memory
    // the chunks are all queued at once over four device slots.  Every host
    // output is written when this returns; finish() still follows.
    void batched(uint32_t batch, const std::vector<Slice>& slices, const ChunkLaunch& launch);

private:
    std::unique_lock<std::mutex> lock_;
    Device& dev_;
    size_t slot_ = 0;   // next workspace slot
    struct Back { void* host; void* dev; size_t bytes; };
    std::vector<Back> back_;
    void* take(size_t bytes);
    void pinned_chunks(uint32_t batch, uint32_t chunk, const std::vector<Slice>& slices,
                       const std::vector<char>& staged, const std::vector<size_t>& off, size_t in_bytes,
                       size_t slot_bytes, const ChunkLaunch& launch);
};

// Kernel timing for measurement (bench.py): when enabled, launch sites
// bracket their kernels with HIP events on the launch stream and the elapsed
// times are summed per kernel name when the call finishes.
class KernelTimer {
public:
    KernelTimer(const char* name, hipStream_t s);
    ~KernelTimer();
    void stop();
private:
    const char* name_;
    hipStream_t s_;
    hipEvent_t a_ = nullptr, b_ = nullptr;
    bool on_ = false, stopped_ = false;
};
bool timing_enabled();
void timing_collect();   // after a stream synchronisation

// True for HIP device (or managed) memory; false for host memory and NULL.
bool is_device_memory(const void* p);

// ceil(a / b)
inline uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Throws std::invalid_argument with the message.
[[noreturn]] void invalid(const std::string& what);

}  // namespace mla
