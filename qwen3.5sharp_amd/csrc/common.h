// Device helpers shared by the mixer kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

namespace q35 {

constexpr int kWave = 64;

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Qwen35Ops.SoftplusScalar / Log1pSafe (src/Qwen35Sharp.Model/Qwen35Ops.cs:
// 121-142): identity above 20, exp below -10, otherwise log(1 + e^x) with a
// 4-term Taylor series whenever e^x < 0.5.  The series is part of the
// reference's semantics (up to 1 % off the true softplus near x = -0.7).
__device__ __forceinline__ float softplus_ref(float x) {
    if (x > 20.0f) return x;
    if (x < -10.0f) return expf(x);
    float ex = expf(x);
    if (ex > -0.5f && ex < 0.5f) {
        float x2 = ex * ex;
        return ex - x2 / 2.0f + x2 * ex / 3.0f - x2 * x2 / 4.0f;
    }
    return logf(1.0f + ex);
}

// Butterfly sum over all 64 lanes of a wave.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Sum over lane groups of `width` consecutive lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Device-scope coherent load of a value another workgroup of the same
// launch published before a release fence (bypasses the non-coherent L1).
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup index remapped so that consecutive logical indices share an XCD:
// the hardware deals workgroups round-robin over the 8 XCDs (block b runs on
// XCD b % 8), each with its own L2.  Requires total % 8 == 0; otherwise the
// identity mapping is used.
__device__ __forceinline__ int xcd_remap(int b, int total) {
    if ((total & 7) != 0) return b;
    return (b & 7) * (total >> 3) + (b >> 3);
}

}  // namespace q35
