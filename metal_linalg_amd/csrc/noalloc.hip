// An entry point that allocates nothing: the batched symmetric
// eigendecomposition (n <= 64) of metal_linalg_eigh, for callers that cannot
// allocate device memory while they run (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  It has no counterpart in
// the reference.
//
// metal_linalg_eigh takes the batched kernel's workspace (the tridiagonal,
// eigenvalues and reflector scalars handed from the first launch to the
// second, kSplitFloats per matrix, needed with vectors at n > 32) and, when
// the caller passes no info array, a per-matrix info buffer from the
// library's grow-only device cache, and stages host pointers through device
// memory.  Here both buffers live in `scratch`, a file-scope device array of
// fixed size, and only device pointers are accepted.  A batch larger than
// the array serves is run in chunks, one after another on the library's
// stream.
//
// The array is per process and per GPU (each device holds its own copy, at
// its own address, found once per device with hipGetSymbolAddress; host code
// uses that address, never the array's name).  It keeps the last call's
// contents; nothing in it needs to start at zero (the first kernel of a chunk
// writes every word the second reads).  The library serialises its own calls
// with one process-wide lock and waits for each call's kernels before it
// returns, so two calls of this process never share the array at once; two
// calls that overlapped on one GPU would race on it.
#include <metal_linalg/c_api.h>
#include <metal_linalg/hip_ext.h>

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>

#include "core.hpp"
#include "entry.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace {

constexpr size_t kScratchBytes = size_t(8) << 20;   // 8 MiB per GPU
constexpr size_t kScratchFloats = kScratchBytes / sizeof(float);
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_symbol_mutex;
float* g_scratch[kMaxDevices] = {};   // the array's device address, per device

// The address of `scratch` on the current device, looked up once.
float* scratch_on(int device) {
    if (device < 0 || device >= kMaxDevices) throw std::runtime_error("[eigh_noalloc] device index out of range");
    std::lock_guard<std::mutex> lock(g_symbol_mutex);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            throw std::runtime_error(std::string("[eigh_noalloc] hipGetSymbolAddress failed: ") +
                                     hipGetErrorString(e));
        }
        g_scratch[device] = static_cast<float*>(p);
    }
    return g_scratch[device];
}

__global__ void fill_info_kernel(uint32_t* info, uint32_t count) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < count) info[i] = 0u;
}

void require_device(const void* p, const char* name) {
    if (p && !mla::is_device_memory(p))
        throw std::invalid_argument(std::string("[eigh_noalloc] ") + name +
                                    " must be device memory (this entry point stages nothing)");
}

}  // namespace

extern "C" {

metal_linalg_status metal_linalg_hip_eigh_noalloc(const float* a, uint32_t batch, uint32_t n, int lower, float* w,
                                                  float* v, uint32_t* info) {
    return mla::run_entry([&] {
        const uint64_t per = (uint64_t)n * n;
        if (!a && batch * per) throw std::invalid_argument("[eigh_noalloc] a is NULL");
        if (!w && (uint64_t)batch * n) throw std::invalid_argument("[eigh_noalloc] w is NULL");
        if (n > 64)
            throw std::invalid_argument("[eigh_noalloc] n = " + std::to_string(n) +
                                        ": this entry point takes n <= 64 (the batched kernel's window)");
        mla::require_gpu_allowed("eigh_noalloc");
        if (batch == 0) return;
        require_device(a, "a");
        require_device(w, "w");
        require_device(v, "v");
        require_device(info, "info");
        mla::Call call;
        if (n == 0) {   // nothing to decompose: info 0
            if (info)
                hipLaunchKernelGGL(fill_info_kernel, dim3((unsigned)mla::cdiv(batch, 256)), dim3(256), 0,
                                   call.stream(), info, batch);
            call.finish();
            return;
        }
        float* base = scratch_on(mla::device().id);
        // per matrix: the kernel's workspace, and an info word when the caller gives none
        const size_t ws_floats = mla::eigh_small_workspace(n, 1, v != nullptr) / sizeof(float);
        const size_t per_matrix = ws_floats + (info ? 0 : 1);
        const uint64_t chunk = per_matrix ? kScratchFloats / per_matrix : batch;
        for (uint64_t b0 = 0; b0 < batch; b0 += chunk) {
            const uint32_t cb = (uint32_t)std::min<uint64_t>(chunk, batch - b0);
            float* ws = ws_floats ? base : nullptr;
            uint32_t* di = info ? info + b0 : reinterpret_cast<uint32_t*>(base + (size_t)cb * ws_floats);
            mla::eigh_small(a + b0 * per, w + b0 * n, v ? v + b0 * per : nullptr, di, cb, n, lower != 0, ws,
                            call.stream());
        }
        call.finish();
    });
}

}  // extern "C"
