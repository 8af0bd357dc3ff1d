// Quantized projections on the device: y[t] = W x[t] for a weight W stored
// as GGUF Q4_K or Q6_K rows, the activation quantized to Q8_K per token,
// as the reference's decode GEMV does.
//
// Reference: Qwen35Model.DecodeLinear (src/Qwen35Sharp.Model/
// Qwen35Model.Decode.cs:56-88) -> MulMatQ4K.Gemv (src/Qwen35Sharp.Kernels/
// MulMatQ4K.cs:12-43) over VecDotQ4K.DotAvx2 (VecDotQ4K.cs:67-126), and
// Q6K.Gemv / Q6K.Gemm (Q6K.cs:301-413) over Q6K.DotAvx2 (Q6K.cs:87-165);
// both quantize the activation with Q8K.QuantizeRow (Q8K.cs:12-146).
//
// Block formats (BlockLayout.cs:32-78), packed:
//   Q4_K (144 B): f16 d, f16 dmin, u8 scales[12], u8 qs[128]
//   Q6_K (210 B): u8 ql[128], u8 qh[64], i8 scales[16], f16 d
//   Q8_K (292 B): f32 d, i8 qs[256], i16 bsums[16]
//
// Results are bit-identical to the reference's AVX2 path: every integer sum
// is exact in any order, and the fp32 part is the reference's own sequence --
// per 256-value block the 8 integer lanes of its _mm256_madd_epi16 sums
// (lane k = bytes 4k..4k+3 of each 32-byte group, here one v_dot4_i32_i8
// per lane and group), converted and accumulated with one FMA per lane and
// block in block order, then its horizontal-sum order.
//
// Work split: the projection is HBM-bound on the weights (4.5 / 6.56 bits a
// weight).  A workgroup takes whole rows (up to 256 blocks), stages their
// contiguous bytes in LDS with 16-byte coalesced loads, and one thread per
// block forms the block's integer lanes; one thread per row then runs the
// fp32 accumulation over the row's blocks in order.  Extra tokens reuse the
// staged weights.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144, Q6K_BYTES = 210, Q8K_BYTES = 292;
constexpr int Q8K_WORDS = Q8K_BYTES / 4;
constexpr int LQ_THREADS = 256;
constexpr int LQ_MAX_NB = 64;      // n_in up to 16384

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// Q8K.QuantizeRow / ScaleBlock (Q8K.cs:12-146): one wave per (256-value
// block, token).  amax = max |x|; the scale's sign is that of the first
// element of magnitude amax; iscale = -127 / max (IEEE division), delta =
// 1 / iscale; q = clamp(round-half-even(x * iscale), -127, 127); bsums =
// sums of 16.
__global__ __launch_bounds__(kWave) void q8k_quantize(const float* __restrict__ x,
                                                      unsigned char* __restrict__ out,
                                                      int n_in) {
    const int b = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int nb = n_in / QK;
    const float4 v = reinterpret_cast<const float4*>(x + (size_t)t * n_in + (size_t)b * QK)[lane];
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, kWave));
    const int e = fabsf(v.x) == amax ? 0 : fabsf(v.y) == amax ? 1 : fabsf(v.z) == amax ? 2
                : fabsf(v.w) == amax ? 3 : 4;
    int first = e < 4 ? 4 * lane + e : 4 * kWave;
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) first = min(first, __shfl_xor(first, m, kWave));
    const int fe = first & 3;
    const float mine = fe == 0 ? v.x : fe == 1 ? v.y : fe == 2 ? v.z : v.w;
    const float mx = __shfl(mine, min(first >> 2, kWave - 1), kWave);

    unsigned char* blk = out + ((size_t)t * nb + b) * Q8K_BYTES;
    int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    float delta = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.0f / mx;
        delta = 1.0f / iscale;
        q0 = min(max((int)rintf(v.x * iscale), -127), 127);
        q1 = min(max((int)rintf(v.y * iscale), -127), 127);
        q2 = min(max((int)rintf(v.z * iscale), -127), 127);
        q3 = min(max((int)rintf(v.w * iscale), -127), 127);
    }
    reinterpret_cast<uint32_t*>(blk + 4)[lane] =
        (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
        ((uint32_t)(q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1, kWave);
    s += __shfl_xor(s, 2, kWave);
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(blk + 260)[lane >> 2] = (int16_t)s;
    if (lane == 0) *reinterpret_cast<float*>(blk) = delta;
}

// Stages `nwords` dwords of token t's Q8_K row into LDS.
__device__ __forceinline__ void stage_q8(uint32_t* __restrict__ q8s, const unsigned char* __restrict__ q8,
                                         int t, int nb, int tid) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(q8 + (size_t)t * nb * Q8K_BYTES);
    for (int i = tid; i < nb * Q8K_WORDS; i += LQ_THREADS) q8s[i] = src[i];
}

// VecDotQ4K.HorizontalSum (VecDotQ4K.cs:145-151).
__device__ __forceinline__ float hsum8(const float (&a)[8]) {
#pragma clang fp contract(off)
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    const float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

// ---------------------------------------------------------------- Q4_K

// The integer lanes of one Q4_K x Q8_K block (VecDotQ4K.cs:74-117): sumi[k]
// (scaled q4.q8 over bytes 4k..4k+3 of each 32-byte group) and prod[k]
// (mins . pairwise bsums, _mm_madd_epi16 order).
__device__ __forceinline__ void q4k_block_lanes(const uint32_t* __restrict__ wb,
                                                const uint32_t* __restrict__ q8b, int (&sumi)[8],
                                                int (&prod)[4]) {
    // Q4K.UnpackScales (Q4K.cs:20-33): bytes 0..7 scales, 8..15 mins.
    const uint32_t s0 = wb[1], s1 = wb[2], s2 = wb[3];
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    const uint32_t u3 = ((s2 >> 4) & kmask2) | (((s1 >> 6) & kmask3) << 4);
    const uint32_t u2 = s1 & kmask1;
    const uint32_t u1 = (s2 & kmask2) | (((s0 >> 6) & kmask3) << 4);
    const uint32_t u0 = s0 & kmask1;
    const uint32_t su[2] = {u0, u1}, mu[2] = {u2, u3};
    // bsums as 8 dwords of two int16 each (Q8_K byte 260 = dword 65)
    const uint32_t* bs = q8b + 65;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t p0 = bs[2 * k], p1 = bs[2 * k + 1];
        const int a0 = (int16_t)(p0 & 0xffff) + (int16_t)(p0 >> 16);
        const int a1 = (int16_t)(p1 & 0xffff) + (int16_t)(p1 >> 16);
        const int m0 = (mu[k >> 1] >> (16 * (k & 1))) & 0xff;
        const int m1 = (mu[k >> 1] >> (16 * (k & 1) + 8)) & 0xff;
        prod[k] = m0 * (int16_t)a0 + m1 * (int16_t)a1;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) sumi[k] = 0;
    const uint32_t* qs = wb + 4;         // 32 dwords
    const uint32_t* q8 = q8b + 1;        // 64 dwords
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int sl = (su[j >> 1] >> (16 * (j & 1))) & 0xff;
        const int sh = (su[j >> 1] >> (16 * (j & 1) + 8)) & 0xff;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t w = qs[8 * j + k];
            const int pl = __builtin_amdgcn_sdot4((int)(w & 0x0f0f0f0fu), (int)q8[16 * j + k], 0, false);
            const int ph = __builtin_amdgcn_sdot4((int)((w >> 4) & 0x0f0f0f0fu), (int)q8[16 * j + 8 + k], 0, false);
            sumi[k] += pl * sl + ph * sh;
        }
    }
}

__global__ __launch_bounds__(LQ_THREADS) void q4k_linear(const unsigned char* __restrict__ w,
                                                         const unsigned char* __restrict__ q8,
                                                         float* __restrict__ y, int n_in, int n_out,
                                                         int tokens, int rows_per_wg) {
#pragma clang fp contract(off)
    const int nb = n_in / QK;
    const int row0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, n_out - row0);
    const int nblk = nrows * nb;
    const int tid = threadIdx.x;

    __shared__ uint4 wsh[LQ_THREADS * (Q4K_BYTES / 16)];   // 36 KiB
    __shared__ uint32_t q8s[LQ_MAX_NB * Q8K_WORDS];        // 18.3 KiB
    __shared__ int lanes[LQ_THREADS][13];

    const uint4* src = reinterpret_cast<const uint4*>(w + (size_t)row0 * nb * Q4K_BYTES);
    for (int i = tid; i < nblk * (Q4K_BYTES / 16); i += LQ_THREADS) wsh[i] = src[i];

    for (int t = 0; t < tokens; ++t) {
        stage_q8(q8s, q8, t, nb, tid);
        __syncthreads();
        if (tid < nblk) {
            int sumi[8], prod[4];
            q4k_block_lanes(reinterpret_cast<const uint32_t*>(wsh + tid * (Q4K_BYTES / 16)),
                            q8s + (tid % nb) * Q8K_WORDS, sumi, prod);
#pragma unroll
            for (int k = 0; k < 8; ++k) lanes[tid][k] = sumi[k];
#pragma unroll
            for (int k = 0; k < 4; ++k) lanes[tid][8 + k] = prod[k];
        }
        __syncthreads();
        if (tid < nrows) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            float accm[4] = {0.f, 0.f, 0.f, 0.f};
            for (int b = 0; b < nb; ++b) {
                const int blk = tid * nb + b;
                const uint32_t hdr = reinterpret_cast<const uint32_t*>(wsh + blk * (Q4K_BYTES / 16))[0];
                const float yd = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]);
                const float d = yd * half_bits_to_float(hdr & 0xffff);
                const float dmin = -yd * half_bits_to_float(hdr >> 16);
#pragma unroll
                for (int k = 0; k < 4; ++k) accm[k] = accm[k] + dmin * (float)lanes[blk][8 + k];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = fmaf((float)lanes[blk][k], d, acc[k]);
            }
            const float m = (accm[0] + accm[2]) + (accm[1] + accm[3]);
            y[(size_t)t * n_out + row0 + tid] = hsum8(acc) + m;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- Q6_K

// Dword of LDS at an arbitrary even byte offset.
__device__ __forceinline__ uint32_t lds_word(const uint32_t* __restrict__ base, int byteoff) {
    const uint32_t lo = base[byteoff >> 2], hi = base[(byteoff >> 2) + 1];
    return __builtin_amdgcn_alignbyte(hi, lo, byteoff & 3);
}

// The integer lanes of one Q6_K x Q8_K block (Q6K.cs:94-156): 6-bit values
// times the scale of their 16-value sub-block, minus 32 (bsums . scales).
__device__ __forceinline__ void q6k_block_lanes(const uint32_t* __restrict__ base, int o,
                                                const uint32_t* __restrict__ q8b, int (&sumi)[8]) {
    int sc[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s = lds_word(base, o + 192 + 4 * i);
        sc[4 * i] = (int8_t)(s & 0xff);
        sc[4 * i + 1] = (int8_t)((s >> 8) & 0xff);
        sc[4 * i + 2] = (int8_t)((s >> 16) & 0xff);
        sc[4 * i + 3] = (int8_t)(s >> 24);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) sumi[k] = 0;
    const uint32_t* q8 = q8b + 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t a = lds_word(base, o + 64 * j + 4 * k);
            const uint32_t c = lds_word(base, o + 64 * j + 32 + 4 * k);
            const uint32_t h = lds_word(base, o + 128 + 32 * j + 4 * k);
            const uint32_t v0 = (a & 0x0f0f0f0fu) | ((h & 0x03030303u) << 4);
            const uint32_t v1 = (c & 0x0f0f0f0fu) | ((h & 0x0c0c0c0cu) << 2);
            const uint32_t v2 = ((a >> 4) & 0x0f0f0f0fu) | (h & 0x30303030u);
            const uint32_t v3 = ((c >> 4) & 0x0f0f0f0fu) | ((h & 0xc0c0c0c0u) >> 2);
            const int hf = k >> 2;
            sumi[k] += sc[8 * j + hf] * __builtin_amdgcn_sdot4((int)v0, (int)q8[32 * j + k], 0, false);
            sumi[k] += sc[8 * j + 2 + hf] * __builtin_amdgcn_sdot4((int)v1, (int)q8[32 * j + 8 + k], 0, false);
            sumi[k] += sc[8 * j + 4 + hf] * __builtin_amdgcn_sdot4((int)v2, (int)q8[32 * j + 16 + k], 0, false);
            sumi[k] += sc[8 * j + 6 + hf] * __builtin_amdgcn_sdot4((int)v3, (int)q8[32 * j + 24 + k], 0, false);
        }
    }
    const uint32_t* bs = q8b + 65;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t p = bs[k];
        sumi[k] -= ((int16_t)(p & 0xffff) * sc[2 * k] + (int16_t)(p >> 16) * sc[2 * k + 1]) * 32;
    }
}

__global__ __launch_bounds__(LQ_THREADS) void q6k_linear(const unsigned char* __restrict__ w,
                                                         const unsigned char* __restrict__ q8,
                                                         float* __restrict__ y, int n_in, int n_out,
                                                         int tokens, int rows_per_wg) {
#pragma clang fp contract(off)
    const int nb = n_in / QK;
    const int row0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, n_out - row0);
    const int nblk = nrows * nb;
    const int tid = threadIdx.x;

    // The workgroup's blocks start at an even byte; they are staged from the
    // 16-byte boundary below, with one 16-byte chunk of slack at each end.
    __shared__ uint4 wsh[(LQ_THREADS * Q6K_BYTES) / 16 + 2];  // 52.5 KiB
    __shared__ uint32_t q8s[LQ_MAX_NB * Q8K_WORDS];
    __shared__ int lanes[LQ_THREADS][9];

    const size_t total = (size_t)n_out * nb * Q6K_BYTES;
    const size_t start = (size_t)row0 * nb * Q6K_BYTES;
    const size_t end = start + (size_t)nblk * Q6K_BYTES;
    const size_t s16 = start & ~(size_t)15;
    const int shift = (int)(start - s16);
    const int nchunks = (int)((end - s16 + 15) >> 4);
    for (int i = tid; i < nchunks; i += LQ_THREADS) {
        const size_t off = s16 + 16 * (size_t)i;
        if (off + 16 <= total) {
            wsh[i] = *reinterpret_cast<const uint4*>(w + off);
        } else {
            // The weight buffer's last chunk: 2-byte loads up to its end.
            uint32_t wd[4] = {0u, 0u, 0u, 0u};
            for (int hb = 0; hb < 8 && off + 2 * hb < total; ++hb)
                wd[hb >> 1] |= (uint32_t)(*reinterpret_cast<const uint16_t*>(w + off + 2 * hb)) << (16 * (hb & 1));
            wsh[i] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        }
    }
    const uint32_t* wbase = reinterpret_cast<const uint32_t*>(wsh);

    for (int t = 0; t < tokens; ++t) {
        stage_q8(q8s, q8, t, nb, tid);
        __syncthreads();
        if (tid < nblk) {
            int sumi[8];
            q6k_block_lanes(wbase, shift + tid * Q6K_BYTES, q8s + (tid % nb) * Q8K_WORDS, sumi);
#pragma unroll
            for (int k = 0; k < 8; ++k) lanes[tid][k] = sumi[k];
        }
        __syncthreads();
        if (tid < nrows) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int b = 0; b < nb; ++b) {
                const int blk = tid * nb + b;
                const int o = shift + blk * Q6K_BYTES + 208;
                const uint32_t dh = lds_word(wbase, o) & 0xffff;
                const float d = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]) * half_bits_to_float(dh);
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = fmaf(d, (float)lanes[blk][k], acc[k]);
            }
            y[(size_t)t * n_out + row0 + tid] = hsum8(acc);
        }
        __syncthreads();
    }
}

}  // namespace

size_t linear_q_work_bytes(int n_in, int tokens) {
    return (size_t)tokens * (n_in / QK) * Q8K_BYTES;
}

hipError_t launch_linear_q(q35m_ctx* c, int qtype, const void* w, const float* x, float* y,
                           int n_in, int n_out, int tokens) {
    const int nb = n_in / QK;
    unsigned char* q8 = reinterpret_cast<unsigned char*>(c->work);
    {
        ProfScope ps_(c, K_Q8K_QUANTIZE);
        hipExtLaunchKernelGGL(q8k_quantize, dim3(nb, tokens), dim3(kWave), 0, c->stream, ps_.a, ps_.b, 0, x,
                              q8, n_in);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int rows_per_wg = LQ_THREADS / nb;
    const int grid = (n_out + rows_per_wg - 1) / rows_per_wg;
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(w);
    if (qtype == 4) {
        ProfScope ps_(c, K_Q4K_LINEAR);
        hipExtLaunchKernelGGL(q4k_linear, dim3(grid), dim3(LQ_THREADS), 0, c->stream, ps_.a, ps_.b, 0, wb, q8,
                              y, n_in, n_out, tokens, rows_per_wg);
    } else {
        ProfScope ps_(c, K_Q6K_LINEAR);
        hipExtLaunchKernelGGL(q6k_linear, dim3(grid), dim3(LQ_THREADS), 0, c->stream, ps_.a, ps_.b, 0, wb, q8,
                              y, n_in, n_out, tokens, rows_per_wg);
    }
    return hipGetLastError();
}

}  // namespace q35
