// Device ceilings measured on the GPU the mixers run on: streaming-read and
// copy bandwidth of HBM, and the fp32 MFMA issue rate.  bench.py reports them
// beside the datasheet peaks (8.0 TB/s, 157.3 TFLOP/s) that the rooflines use.
// Not part of the mixer ABI: a separate library, libq35probe.so.
#include <hip/hip_runtime.h>

#include <cstddef>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Grid-stride float4 read; one partial sum per thread keeps the loads alive.
typedef float v4 __attribute__((ext_vector_type(4)));

// NT: non-temporal loads (and stores), as the decode kernels stream state.
template <bool NT>
__global__ __launch_bounds__(256) void read_kernel(const v4* __restrict__ p, size_t n4,
                                                   float* __restrict__ out) {
    float acc = 0.0f;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const v4 v = NT ? __builtin_nontemporal_load(p + i) : p[i];
        acc += v.x + v.y + v.z + v.w;
    }
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

template <bool NT>
__global__ __launch_bounds__(256) void copy_kernel(const v4* __restrict__ p, v4* __restrict__ q, size_t n4) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        if (NT)
            __builtin_nontemporal_store(__builtin_nontemporal_load(p + i), q + i);
        else
            q[i] = p[i];
    }
}

// 8 independent v_mfma_f32_16x16x4f32 chains per wave, `iters` rounds.
__global__ __launch_bounds__(256) void mfma_kernel(int iters, float seed, float* __restrict__ out) {
    f32x4 acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float a = seed + threadIdx.x * 1e-7f, b = seed - threadIdx.x * 1e-7f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[k], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

int fail(hipError_t e) { return e == hipSuccess ? 0 : -5; }

// Times `reps` launches of f after one warm-up launch; returns milliseconds.
template <typename F>
hipError_t time_ms(F f, int reps, float* ms) {
    hipEvent_t a, b;
    hipError_t e = hipEventCreate(&a);
    if (e != hipSuccess) return e;
    if ((e = hipEventCreate(&b)) != hipSuccess) return e;
    f();
    if ((e = hipEventRecord(a, nullptr)) != hipSuccess) return e;
    for (int r = 0; r < reps; ++r) f();
    if ((e = hipEventRecord(b, nullptr)) != hipSuccess) return e;
    if ((e = hipEventSynchronize(b)) != hipSuccess) return e;
    e = hipEventElapsedTime(ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return e;
}

}  // namespace

extern "C" {

// Streaming read of `bytes` (multiple of 16), `reps` times: GB/s (1e9 B/s);
// nt != 0: non-temporal loads.
int q35p_hbm_read_gbs(size_t bytes, int reps, int nt, double* gbs) {
    if (!gbs || bytes < 16 || reps < 1) return -1;
    const size_t n4 = bytes / 16;
    const int grid = 2048;
    v4* p = nullptr;
    float* out = nullptr;
    hipError_t e = hipMalloc(&p, n4 * 16);
    if (e == hipSuccess) e = hipMalloc(&out, (size_t)grid * 256 * sizeof(float));
    if (e == hipSuccess) e = hipMemset(p, 0, n4 * 16);
    float ms = 0.0f;
    if (e == hipSuccess)
        e = time_ms([&] {
                if (nt) hipLaunchKernelGGL(read_kernel<true>, dim3(grid), dim3(256), 0, nullptr, p, n4, out);
                else hipLaunchKernelGGL(read_kernel<false>, dim3(grid), dim3(256), 0, nullptr, p, n4, out);
            }, reps, &ms);
    if (e == hipSuccess) *gbs = (double)n4 * 16 * reps / (ms * 1e-3) / 1e9;
    if (p) (void)hipFree(p);
    if (out) (void)hipFree(out);
    return fail(e);
}

// Copy of `bytes` into a second buffer, `reps` times: GB/s counting the bytes
// read plus the bytes written; nt != 0: non-temporal loads and stores.
int q35p_hbm_copy_gbs(size_t bytes, int reps, int nt, double* gbs) {
    if (!gbs || bytes < 16 || reps < 1) return -1;
    const size_t n4 = bytes / 16;
    const int grid = 2048;
    v4 *p = nullptr, *q = nullptr;
    hipError_t e = hipMalloc(&p, n4 * 16);
    if (e == hipSuccess) e = hipMalloc(&q, n4 * 16);
    if (e == hipSuccess) e = hipMemset(p, 0, n4 * 16);
    float ms = 0.0f;
    if (e == hipSuccess)
        e = time_ms([&] {
                if (nt) hipLaunchKernelGGL(copy_kernel<true>, dim3(grid), dim3(256), 0, nullptr, p, q, n4);
                else hipLaunchKernelGGL(copy_kernel<false>, dim3(grid), dim3(256), 0, nullptr, p, q, n4);
            }, reps, &ms);
    if (e == hipSuccess) *gbs = 2.0 * n4 * 16 * reps / (ms * 1e-3) / 1e9;
    if (p) (void)hipFree(p);
    if (q) (void)hipFree(q);
    return fail(e);
}

// fp32 MFMA rate: 2 workgroups of 4 waves per CU, each wave `iters` x 8
// v_mfma_f32_16x16x4f32 (2048 FLOP each): TFLOP/s.
int q35p_mfma_f32_tflops(int iters, double* tflops) {
    if (!tflops || iters < 1) return -1;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int grid = 2 * cus;
    float* out = nullptr;
    if (e == hipSuccess) e = hipMalloc(&out, (size_t)grid * 256 * sizeof(float));
    float ms = 0.0f;
    if (e == hipSuccess)
        e = time_ms([&] { hipLaunchKernelGGL(mfma_kernel, dim3(grid), dim3(256), 0, nullptr, iters, 1.0f, out); },
                    5, &ms);
    if (e == hipSuccess) *tflops = (double)grid * 4 * iters * 8 * 2048.0 * 5 / (ms * 1e-3) / 1e12;
    if (out) (void)hipFree(out);
    return fail(e);
}

}  // extern "C"
