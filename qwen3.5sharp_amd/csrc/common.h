// Device helpers shared by the mixer kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

namespace q35 {

constexpr int kWave = 64;

// x * sigmoid(x) with the hardware reciprocal (1 ulp) in place of an IEEE
// division; e^-x -> inf gives x * 0 = -0 as the division would.
__device__ __forceinline__ float silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

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

// Workgroup barrier for LDS exchange only: waits for this wave's LDS traffic
// (lgkmcnt) and synchronises, but leaves global loads in flight, unlike
// __syncthreads(), whose fence also drains vmcnt.  Prefetched operands of the
// next step therefore keep streaming across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The values of lanes l and l ^ 16 (rows of 16 lanes swapped in pairs), or
// l and l ^ 32 (the two halves), as (lower lane's, upper lane's) in both
// lanes: one v_permlane16_swap / v_permlane32_swap, a register exchange that
// does not go through the LDS crossbar (a ds_bpermute there queues behind
// other waves' LDS traffic).
__device__ __forceinline__ float2 lanes_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 lanes_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum / max of the pair, the same in both lanes and equal to v + shfl_xor(v, o)
// (fp addition is commutative).
__device__ __forceinline__ float xor16_sum(float v) { const float2 p = lanes_xor16(v); return p.x + p.y; }
__device__ __forceinline__ float xor32_sum(float v) { const float2 p = lanes_xor32(v); return p.x + p.y; }
__device__ __forceinline__ float xor16_max(float v) { const float2 p = lanes_xor16(v); return fmaxf(p.x, p.y); }
__device__ __forceinline__ float xor32_max(float v) { const float2 p = lanes_xor32(v); return fmaxf(p.x, p.y); }

// Butterfly sum over all 64 lanes of a wave (the 32- and 16-lane steps by
// lane swaps, the rest by shuffles within rows).
__device__ __forceinline__ float wave_sum(float v) {
    v = xor32_sum(v);
    v = xor16_sum(v);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = xor32_max(v);
    v = xor16_max(v);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Sum over lane groups of `width` consecutive lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (width >= 64) v = xor32_sum(v);
    if constexpr (width >= 32) v = xor16_sum(v);
#pragma unroll
    for (int o = (width < 16 ? width : 16) / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Non-temporal 16-byte load and store (global_load / global_store_dwordx4 with
// the nt bit): for data streamed through once per call, such as decode states
// and KV rows, so that it does not evict from L2 and MALL what the following
// kernels read.
// Buffer loads straight into LDS (no registers): lane l's 4 or 16 bytes at
// voff + soff of the descriptor's range go to lds + size * l; offsets past
// the range read as zero.  Completion is waited for with vmcnt.
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma_b32(__amdgpu_buffer_rsrc_t rs, void* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 4, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma_b128(__amdgpu_buffer_rsrc_t rs, void* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 16, voff, soff, 0, 0);
}

typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float* p) {
    const nt_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(float* p, float4 v) {
    __builtin_nontemporal_store(nt_f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_f32x4*>(p));
}

// Workgroup index remapped so that consecutive logical indices share an XCD:
// the hardware deals workgroups round-robin over the 8 XCDs (block b runs on
// XCD b % 8), each with its own L2.  Requires total % 8 == 0; otherwise the
// identity mapping is used.
__device__ __forceinline__ int xcd_remap(int b, int total) {
    if ((total & 7) != 0) return b;
    return (b & 7) * (total >> 3) + (b >> 3);
}

// NeoX RoPE over pairs (d, d+32), d < 32 (Ops.RopeRange, Ops.cs:97-133) then
// the zero-centred (1+w) RMSNorm (Qwen35Ops.RmsNormZeroCentered,
// Qwen35Ops.cs:22-66) of one 256-wide head row held as one float4 per lane of
// a wave (lane l: dims 4l..4l+3); the result is also multiplied by post_scale.
// The operands come in registers: c, s = the RoPE table entries 4(l%8)..+3 of
// the token's position (used by lanes 0-15), ww = w[4l..4l+3].  No memory
// access, so callers issue these loads together with others.
__device__ __forceinline__ float4 rope_norm_regs(float4 x, float4 c, float4 s, float4 ww, int lane,
                                                 float eps, float post_scale) {
    float4 p;
    p.x = __shfl_xor(x.x, 8, kWave);
    p.y = __shfl_xor(x.y, 8, kWave);
    p.z = __shfl_xor(x.z, 8, kWave);
    p.w = __shfl_xor(x.w, 8, kWave);
    float4 lo, hi;      // x0' = x0 c - x1 s (lanes 0-7), x1' = x0 s + x1 c (lanes 8-15)
    lo.x = x.x * c.x - p.x * s.x;
    lo.y = x.y * c.y - p.y * s.y;
    lo.z = x.z * c.z - p.z * s.z;
    lo.w = x.w * c.w - p.w * s.w;
    hi.x = p.x * s.x + x.x * c.x;
    hi.y = p.y * s.y + x.y * c.y;
    hi.z = p.z * s.z + x.z * c.z;
    hi.w = p.w * s.w + x.w * c.w;
    if (lane < 8) x = lo;
    else if (lane < 16) x = hi;
    const float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
    const float scale = 1.0f / sqrtf(ss / 256.0f + eps);
    x.x = x.x * scale * (1.0f + ww.x) * post_scale;
    x.y = x.y * scale * (1.0f + ww.y) * post_scale;
    x.z = x.z * scale * (1.0f + ww.z) * post_scale;
    x.w = x.w * scale * (1.0f + ww.w) * post_scale;
    return x;
}

// rope_norm_row with its operands loaded here, all at once (cs/sn: the RoPE
// table row of the token's position).
__device__ __forceinline__ float4 rope_norm_row(float4 x, int lane, const float* __restrict__ cs,
                                                const float* __restrict__ sn,
                                                const float* __restrict__ w, float eps,
                                                float post_scale) {
    const int i0 = 4 * (lane & 7);
    const float4 c = *reinterpret_cast<const float4*>(cs + i0);
    const float4 s = *reinterpret_cast<const float4*>(sn + i0);
    const float4 ww = *reinterpret_cast<const float4*>(w + 4 * lane);
    return rope_norm_regs(x, c, s, ww, lane, eps, post_scale);
}

}  // namespace q35
