// Batched Cholesky of small matrices (n <= 64), one matrix per lane group of
// a wave64 (a whole wave at 33 <= n <= 64), held in registers; 65 <= n <= 128
// one matrix per workgroup in LDS.
//
// Role: the MI355X counterpart of the reference's chol_simd
// (reference: shaders/Cholesky.metal:61-146, driver src/cholesky_gpu.mm:216-244)
// with the contract of its CPU path (src/cholesky_cpu.mm:93-151): only the
// requested triangle is read; info = k + 1 for the first pivot that is not
// positive and finite (spotrf's info, a NaN or infinite pivot included), and
// then that matrix's output is all quiet NaN; the other triangle of the
// output is exactly zero.
//
// Layout: lane c of an N-lane group owns column c of the lower triangle
// (row c of the upper one), N = n rounded up to a power of two and padded
// with the identity, 64/N matrices per wave.  Right-looking: at step k lane
// k forms column k of L, broadcasts it through LDS together with its
// pivot's verdict, and lanes c > k apply the rank-1 update to their columns.
#include "device_common.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace mla {
namespace {

template <int K, int N>
__device__ __forceinline__ void chol_step(float (&x)[N], float* col, int c, int& fail) {
    if constexpr (K < N) {
        if (c == K) {
            const float d = x[K];
            const bool good = d > 0.0f && d <= FLT_MAX;
            const float lkk = sqrtf(d);
            const float inv = 1.0f / lkk;
            x[K] = lkk;
#pragma unroll
            for (int r = K + 1; r < N; ++r) {
                x[r] *= inv;
                col[r] = x[r];
            }
            col[N] = good ? 0.0f : 1.0f;
        }
        wave_lds_sync();
        if (!fail && col[N] != 0.0f) fail = K + 1;
        if (c > K) {
            const float lc = col[c];
#pragma unroll
            for (int r = K + 1; r < N; ++r) x[r] = fmaf(-col[r], lc, x[r]);
        }
        wave_lds_sync();
        chol_step<K + 1, N>(x, col, c, fail);
    }
}

template <int N>
__global__ __launch_bounds__(64) void chol_small_kernel(const float* __restrict__ A, float* __restrict__ L,
                                                        uint32_t* __restrict__ info, uint32_t batch, uint32_t n,
                                                        int upper) {
    constexpr int MPW = 64 / N;
    __shared__ float col[MPW][N + 4];
    const int lane = threadIdx.x;
    const int c = lane % N;
    const int g = lane / N;
    const size_t mat = (size_t)blockIdx.x * MPW + g;
    const bool live = mat < batch;
    const size_t per = (size_t)n * n;
    const float* src = A + mat * per;

    float x[N];
#pragma unroll
    for (int r = 0; r < N; ++r) {
        float v = (r == c) ? 1.0f : 0.0f;   // identity padding
        if (live && c < (int)n && r < (int)n) {
            v = 0.0f;
            if (r >= c) v = upper ? src[(size_t)c * n + r] : src[(size_t)r * n + c];
        }
        x[r] = v;
    }

    int fail = 0;
    chol_step<0, N>(x, col[g], c, fail);

    if (!live) return;
    if (info && c == 0) info[mat] = (uint32_t)fail;
    if (c >= (int)n) return;
    float* dst = L + mat * per;
#pragma unroll
    for (int r = 0; r < N; ++r) {
        if (r < (int)n) {
            const float v = fail ? qnan() : (r >= c ? x[r] : 0.0f);
            if (upper) dst[(size_t)c * n + r] = v;   // U = L^T: row c of U is column c of L
            else dst[(size_t)r * n + c] = v;
        }
    }
}

// 65 <= n <= 128: one matrix per 256-thread workgroup, the lower triangle in
// LDS (row stride n + 1, 66 KB at n = 128: two workgroups per CU),
// right-looking with the same arithmetic as above: the pivot's square root,
// the column times its reciprocal, the rank-1 update of the trailing lower
// triangle; two workgroup barriers per column.  The first pivot that is not positive and finite ends the loop
// in every thread at once (all read the same LDS word) and sets info.
constexpr int kMidN = 128;

__global__ __launch_bounds__(256) void chol_mid_kernel(const float* __restrict__ A, float* __restrict__ L,
                                                       uint32_t* __restrict__ info, uint32_t n, int upper) {
    __shared__ float a[kMidN * (kMidN + 1)];
    __shared__ int fail_sh;
    const int t = threadIdx.x;
    const int nn = (int)n, ld = nn + 1;
    const size_t mat = blockIdx.x;
    const float* src = A + mat * (size_t)n * n;
    for (int i = t; i < nn * nn; i += 256) {
        const int r = i / nn, c = i - r * nn;
        if (r >= c) a[r * ld + c] = upper ? src[(size_t)c * n + r] : src[(size_t)r * n + c];
    }
    if (t == 0) fail_sh = 0;
    __syncthreads();
    for (int k = 0; k < nn; ++k) {
        const float d = a[k * ld + k];
        if (!(d > 0.0f && d <= FLT_MAX)) {
            if (t == 0) fail_sh = k + 1;
            break;
        }
        const float lkk = sqrtf(d);
        const float inv = 1.0f / lkk;
        // the diagonal entry is written in the update phase, which reads no
        // diagonal entry, so no thread can see it change before reading d
        for (int r = k + 1 + t; r < nn; r += 256) a[r * ld + k] *= inv;
        __syncthreads();
        if (t == 0) a[k * ld + k] = lkk;
        // rows to the four waves in turn, columns to the lanes
        for (int r = k + 1 + (t >> 6); r < nn; r += 4) {
            const float lr = a[r * ld + k];
            for (int c = k + 1 + (t & 63); c <= r; c += 64) a[r * ld + c] = fmaf(-lr, a[c * ld + k], a[r * ld + c]);
        }
        __syncthreads();
    }
    __syncthreads();
    const int fail = fail_sh;
    if (t == 0 && info) info[mat] = (uint32_t)fail;
    float* dst = L + mat * (size_t)n * n;
    for (int i = t; i < nn * nn; i += 256) {
        const int r = i / nn, c = i - r * nn;
        const float v = fail ? qnan() : (r >= c ? a[r * ld + c] : 0.0f);
        if (upper) dst[(size_t)c * n + r] = v;   // U = L^T
        else dst[(size_t)r * n + c] = v;
    }
}

template <int N>
void launch(const float* a, float* l, uint32_t* info, uint32_t batch, uint32_t n, bool upper, hipStream_t s) {
    constexpr int MPW = 64 / N;
    KernelTimer t("chol_small", s);
    hipLaunchKernelGGL((chol_small_kernel<N>), dim3((uint32_t)cdiv(batch, MPW)), dim3(64), 0, s, a, l, info, batch, n,
                       upper ? 1 : 0);
    t.stop();
}

}  // namespace

bool chol_small_fits(uint32_t n) { return n >= 1 && n <= (uint32_t)kMidN; }

void chol_small(const float* a, float* l, uint32_t* info, uint32_t batch, uint32_t n, bool upper, hipStream_t s) {
    if (!chol_small_fits(n)) invalid("[cholesky] chol_small takes n <= 128");
    if (batch == 0) return;
    if (n <= 4) launch<4>(a, l, info, batch, n, upper, s);
    else if (n <= 8) launch<8>(a, l, info, batch, n, upper, s);
    else if (n <= 16) launch<16>(a, l, info, batch, n, upper, s);
    else if (n <= 32) launch<32>(a, l, info, batch, n, upper, s);
    else if (n <= 64) launch<64>(a, l, info, batch, n, upper, s);
    else {
        KernelTimer t("chol_small", s);
        hipLaunchKernelGGL(chol_mid_kernel, dim3(batch), dim3(256), 0, s, a, l, info, n, upper ? 1 : 0);
        t.stop();
    }
    MLA_HIP(hipGetLastError());
}

}  // namespace mla
