// Quantized projections on the device: y[t] = W x[t] for a weight W stored
// as GGUF Q4_K, Q5_K, Q6_K, IQ4_XS, Q2_0C or STQ1_0 rows, the activation
// quantized to Q8_K per token, as the reference's decode GEMV does (and F32
// weights, unquantized, at the end of the file).  The Q4_K / Q6_K notes
// below are the model for the other formats, whose sections say where they
// differ.
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
// weight).  q8k_quantize turns each token row into Q8_K blocks (one wave a
// block) in the workspace.  linear_q then runs one 64-thread workgroup per
// group of up to 8 whole rows (at most 64 blocks): it stages the rows'
// contiguous bytes in LDS with 16-byte loads and the token's Q8_K row from
// L2, forms one block's integer lanes per thread, and runs each row's fp32
// accumulation on 8 threads, one per reference lane, in block order.  Extra
// tokens reuse the staged weights.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144, Q6K_BYTES = 210;
// Workspace form of a Q8_K block, 304 bytes (19 x 16): dword 0 d, dwords 4..67
// qs (16-byte aligned), dwords 68..75 bsums; dwords 1..3 unused.
constexpr int Q8K_WORDS = 76;
constexpr int Q8K_QS = 4, Q8K_BS = 68;
constexpr int LQ_THREADS = 64;
constexpr int LQ_MAX_ROWS = 8;     // rows per workgroup (8 threads a row in the fp32 pass)
constexpr int LANES_LD = 13;       // padded stride of the per-block integer lanes in LDS

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// The Q8_K block of 256 values held 16 a lane by a 16-lane group (lane li of
// the group: values 16 li .. 16 li + 15, one bsums group); every lane of the
// wave takes part in the shuffles.  blk null: nothing is written.
__device__ __forceinline__ void q8k_from16(const float (&v)[16], int lane, uint32_t* blk) {
    const int li = lane & 15;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, kWave));
    int e = 16;
#pragma unroll
    for (int i = 15; i >= 0; --i) e = fabsf(v[i]) == amax ? i : e;
    int first = e < 16 ? 16 * li + e : QK;
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) first = min(first, __shfl_xor(first, m, kWave));
    float mine = v[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mine = (first & 15) == i ? v[i] : mine;
    const float mx = __shfl(mine, (lane & ~15) + min(first >> 4, 15), kWave);
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
    int bsum = 0;
    float delta = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.0f / mx;
        delta = 1.0f / iscale;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int q = min(max((int)rintf(v[i] * iscale), -127), 127);
            bsum += q;
            pk[i >> 2] |= (uint32_t)(q & 0xff) << (8 * (i & 3));
        }
    }
    if (blk) {
        *reinterpret_cast<uint4*>(blk + Q8K_QS + 4 * li) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        reinterpret_cast<int16_t*>(blk + Q8K_BS)[li] = (int16_t)bsum;
        if (li == 0) blk[0] = __builtin_bit_cast(uint32_t, delta);
    }
}

// Q8K.QuantizeRow / ScaleBlock (Q8K.cs:12-146), four 256-value blocks of one
// token per wave: a 16-lane group per block, 16 consecutive values a lane (so
// a lane's values are exactly one bsums group).  amax = max |x|; the scale's
// sign is that of the first element of magnitude amax; iscale = -127 / max
// (IEEE division), delta = 1 / iscale; q = clamp(round-half-even(x * iscale),
// -127, 127).  Output: Q8_K blocks [tokens][nb] in the workspace form above.
__global__ __launch_bounds__(kWave) void q8k_quantize(const float* __restrict__ x,
                                                      uint32_t* __restrict__ q8, int nb) {
    const int lane = threadIdx.x, grp = lane >> 4, li = lane & 15;
    const int t = blockIdx.y, b = 4 * blockIdx.x + grp, bb = min(b, nb - 1);
    const float4* src = reinterpret_cast<const float4*>(x + ((size_t)t * nb + bb) * QK + 16 * li);
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 f = src[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
    q8k_from16(v, lane, b < nb ? q8 + ((size_t)t * nb + b) * Q8K_WORDS : nullptr);
}

// VecDotQ4K.HorizontalSum (VecDotQ4K.cs:145-151).
__device__ __forceinline__ float hsum8(const float (&a)[8]) {
#pragma clang fp contract(off)
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    const float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

// ---------------------------------------------------------------- Q4_K

// Every product below has operands well inside 24 bits (6- or 8-bit scales
// times sums of at most 4 x 63 x 127), so it uses the full-rate 24-bit
// multiply.
//
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
    // The block's qs (16 x 16 B) and bsums (8 dwords of two int16), all
    // loads issued before the first product.
    uint4 qv[16], bv[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_QS)[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) bv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_BS)[i];
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(bv);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t p0 = bs[2 * k], p1 = bs[2 * k + 1];
        const int a0 = (int16_t)(p0 & 0xffff) + (int16_t)(p0 >> 16);
        const int a1 = (int16_t)(p1 & 0xffff) + (int16_t)(p1 >> 16);
        const int m0 = (mu[k >> 1] >> (16 * (k & 1))) & 0xff;
        const int m1 = (mu[k >> 1] >> (16 * (k & 1) + 8)) & 0xff;
        prod[k] = __mul24(m0, (int16_t)a0) + __mul24(m1, (int16_t)a1);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) sumi[k] = 0;
    const uint32_t* qs = wb + 4;                                  // 32 dwords
    const uint32_t* q8 = reinterpret_cast<const uint32_t*>(qv);   // 64 dwords
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int sl = (su[j >> 1] >> (16 * (j & 1))) & 0xff;
        const int sh = (su[j >> 1] >> (16 * (j & 1) + 8)) & 0xff;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t w = qs[8 * j + k];
            const int pl = __builtin_amdgcn_sdot4((int)(w & 0x0f0f0f0fu), (int)q8[16 * j + k], 0, false);
            const int ph = __builtin_amdgcn_sdot4((int)((w >> 4) & 0x0f0f0f0fu), (int)q8[16 * j + 8 + k], 0, false);
            sumi[k] += __mul24(pl, sl) + __mul24(ph, sh);
        }
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
    uint4 qv[16], bv[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_QS)[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) bv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_BS)[i];
    const uint32_t* q8 = reinterpret_cast<const uint32_t*>(qv);
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
            sumi[k] += __mul24(sc[8 * j + hf], __builtin_amdgcn_sdot4((int)v0, (int)q8[32 * j + k], 0, false));
            sumi[k] += __mul24(sc[8 * j + 2 + hf], __builtin_amdgcn_sdot4((int)v1, (int)q8[32 * j + 8 + k], 0, false));
            sumi[k] += __mul24(sc[8 * j + 4 + hf], __builtin_amdgcn_sdot4((int)v2, (int)q8[32 * j + 16 + k], 0, false));
            sumi[k] += __mul24(sc[8 * j + 6 + hf], __builtin_amdgcn_sdot4((int)v3, (int)q8[32 * j + 24 + k], 0, false));
        }
    }
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(bv);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t p = bs[k];
        sumi[k] -= (__mul24((int16_t)(p & 0xffff), sc[2 * k]) + __mul24((int16_t)(p >> 16), sc[2 * k + 1])) * 32;
    }
}

// LDS bytes of one workgroup: staged weights (16-byte chunks, one of slack at
// each end; Q6_K only), the token's Q8_K row, the integer lanes and the fp32
// partials.
__host__ __device__ constexpr int lq_wchunks(int qtype, int rows, int nb, int bytes) {
    return qtype == 4 ? 0 : (rows * nb * bytes + 31) / 16 + 1;
}

// NB > 0 fixes the blocks per row at compile time (n_in = 256 NB), so the
// fp32 pass unrolls and issues its LDS reads together; NB = 0 is generic.
template <int QT, int NB>
__global__ __launch_bounds__(LQ_THREADS) void linear_q(const unsigned char* __restrict__ w,
                                                       const uint32_t* __restrict__ q8,
                                                       float* __restrict__ y, int n_in, int n_out,
                                                       int tokens, int rows_per_wg, int row_base) {
#pragma clang fp contract(off)
    constexpr int BB = QT == 4 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int NL = QT == 4 ? 12 : 8;          // integer lanes per block
    extern __shared__ uint4 smem[];
    const int nb = NB > 0 ? NB : n_in / QK, lane = threadIdx.x;
    const int row0 = row_base + blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, n_out - row0);
    const int nblk = nrows * nb;
    uint4* wsh = smem;
    uint32_t* q8s = reinterpret_cast<uint32_t*>(smem + lq_wchunks(QT, rows_per_wg, nb, BB));
    int* lanes = reinterpret_cast<int*>(q8s + nb * Q8K_WORDS);
    float* accs = reinterpret_cast<float*>(lanes + LQ_THREADS * LANES_LD);

    // Q4_K: each thread loads its block (16-byte aligned, 144 B) straight
    // into registers.  Q6_K blocks are 2-byte aligned: the workgroup's rows,
    // contiguous bytes from an even offset, are staged in LDS from the
    // 16-byte boundary below; only the weight buffer's last chunk can be
    // partial, and it is read with 2-byte loads.
    uint4 wreg[QT == 4 ? Q4K_BYTES / 16 : 1];
    const uint32_t* wbase = reinterpret_cast<const uint32_t*>(wsh);
    int shift = 0;
    if constexpr (QT == 4) {
        const uint4* src = reinterpret_cast<const uint4*>(w + ((size_t)row0 * nb + min(lane, nblk - 1)) * BB);
#pragma unroll
        for (int c = 0; c < Q4K_BYTES / 16; ++c) wreg[c] = src[c];
    } else {
        const size_t total = (size_t)n_out * nb * BB;
        const size_t start = (size_t)row0 * nb * BB;
        const size_t s16 = start & ~(size_t)15;
        shift = (int)(start - s16);
        const int nchunks = (int)((start + (size_t)nblk * BB - s16 + 15) >> 4);
        // All of a lane's weight loads are issued before the first LDS store.
        constexpr int MAXC = (LQ_THREADS * BB + 31 + LQ_THREADS * 16 - 1) / (LQ_THREADS * 16) + 1;
        uint4 wv[MAXC];
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const int i = lane + LQ_THREADS * c;
            const size_t off = s16 + 16 * (size_t)i;
            wv[c] = make_uint4(0u, 0u, 0u, 0u);
            if (i < nchunks && off + 16 <= total) wv[c] = *reinterpret_cast<const uint4*>(w + off);
        }
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const int i = lane + LQ_THREADS * c;
            const size_t off = s16 + 16 * (size_t)i;
            if (i < nchunks) {
                if (off + 16 <= total) {
                    wsh[i] = wv[c];
                } else {
                    uint32_t wd[4] = {0u, 0u, 0u, 0u};
                    for (int hb = 0; hb < 8 && off + 2 * hb < total; ++hb)
                        wd[hb >> 1] |= (uint32_t)(*reinterpret_cast<const uint16_t*>(w + off + 2 * hb)) << (16 * (hb & 1));
                    wsh[i] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
                }
            }
        }
    }

    for (int t = 0; t < tokens; ++t) {
        {
            // The token's Q8_K row, nb x 19 16-byte chunks, 8 loads a lane in flight.
            const uint4* src = reinterpret_cast<const uint4*>(q8 + (size_t)t * nb * Q8K_WORDS);
            uint4* dst = reinterpret_cast<uint4*>(q8s);
            const int n4 = nb * (Q8K_WORDS / 4);
            for (int i0 = 0; i0 < n4; i0 += 8 * LQ_THREADS) {
                uint4 qv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    qv[c] = make_uint4(0u, 0u, 0u, 0u);
                    if (i0 + lane + LQ_THREADS * c < n4) qv[c] = src[i0 + lane + LQ_THREADS * c];
                }
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (i0 + lane + LQ_THREADS * c < n4) dst[i0 + lane + LQ_THREADS * c] = qv[c];
            }
        }
        __syncthreads();
        if (lane < nblk) {
            const uint32_t* q8b = q8s + (lane % nb) * Q8K_WORDS;
            int* out = lanes + lane * LANES_LD;
            if constexpr (QT == 4) {
                int sumi[8], prod[4];
                const uint32_t* wb = reinterpret_cast<const uint32_t*>(wreg);
                q4k_block_lanes(wb, q8b, sumi, prod);
#pragma unroll
                for (int k = 0; k < 8; ++k) out[k] = sumi[k];
#pragma unroll
                for (int k = 0; k < 4; ++k) out[8 + k] = prod[k];
                out[12] = (int)wb[0];             // d, dmin of the block
            } else {
                int sumi[8];
                q6k_block_lanes(wbase, shift + lane * BB, q8b, sumi);
#pragma unroll
                for (int k = 0; k < 8; ++k) out[k] = sumi[k];
                out[8] = (int)(lds_word(wbase, shift + lane * BB + 208) & 0xffff);   // d of the block
            }
        }
        __syncthreads();
        // Row r's lane k: one FMA per block in block order (and, for Q4_K,
        // lanes 0..3 also run the min term's multiply-add).
        const int r = lane >> 3, k = lane & 7;
        if (r < nrows) {
            float acc = 0.0f, accm = 0.0f;
#pragma unroll
            for (int b = 0; b < (NB > 0 ? NB : nb); ++b) {
                const int blk = r * nb + b;
                const float yd = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]);
                const int* L = lanes + blk * LANES_LD;
                if constexpr (QT == 4) {
                    const uint32_t hdr = (uint32_t)L[12];
                    const float d = yd * half_bits_to_float(hdr & 0xffff);
                    const float dmin = -yd * half_bits_to_float(hdr >> 16);
                    if (k < 4) accm = accm + dmin * (float)L[8 + k];
                    acc = fmaf((float)L[k], d, acc);
                } else {
                    const float d = yd * half_bits_to_float((uint32_t)L[8]);
                    acc = fmaf(d, (float)L[k], acc);
                }
            }
            accs[r * NL + k] = acc;
            if (QT == 4 && k < 4) accs[r * NL + 8 + k] = accm;
        }
        __syncthreads();
        if (lane < nrows) {
            const float* a = accs + lane * NL;
            const float h[8] = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]};
            float o = hsum8(h);
            if constexpr (QT == 4) o = o + ((a[8] + a[10]) + (a[9] + a[11]));
            y[(size_t)t * n_out + row0 + lane] = o;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- Q5_K, IQ4_XS

// Formats whose reference dot product is scalar (Q5K.Dot, src/Qwen35Sharp.
// Kernels/Q5K.cs:45-95; IQ4XS.Dot, IQ4XS.cs:49-73): exact integer sums per
// block (Q5_K) or per 32-value sub-block (IQ4_XS), then one fp32 chain per
// output in block order with no fused multiply-add.  Their Gemm runs the GEMV
// per token (Q5K.cs:112-117, IQ4XS.cs:99-104), so every token is a GEMV here
// too.  Block formats (BlockLayout.cs:49-66):
//   Q5_K (176 B): f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
//   IQ4_XS (136 B): f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]
constexpr int Q5K_BYTES = 176, IQ4XS_BYTES = 136;
constexpr int QS_TLD = 9;            // LDS stride of a block's chain terms

// Q5_K x Q8_K block: acc = sum_j scale_j (q8 . a over sub-block j) with the
// 5-bit values a = nibble + 16 * (qh bit), sumi = sum_j bsums[j] min[j / 2].
// Group j (64 values) takes the low nibbles of qs[32 j ..] with qh bit 2j
// (q8 bytes 64 j ..) and the high nibbles with qh bit 2j + 1 (q8 bytes
// 64 j + 32 ..).  wb: the block's 44 dwords.
__device__ __forceinline__ void q5k_block_terms(const uint32_t* __restrict__ wb,
                                                const uint32_t* __restrict__ q8b, int& acc, int& sumi) {
    const uint32_t s0 = wb[1], s1 = wb[2], s2 = wb[3];
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    // Q4K.UnpackScales (Q4K.cs:20-33): bytes 0..7 scales, 8..15 mins.
    const uint32_t su[2] = {s0 & kmask1, (s2 & kmask2) | (((s0 >> 6) & kmask3) << 4)};
    const uint32_t mu[2] = {s1 & kmask1, ((s2 >> 4) & kmask2) | (((s1 >> 6) & kmask3) << 4)};
    uint4 qv[16], bv[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_QS)[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) bv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_BS)[i];
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(bv);
    sumi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int m = (mu[j >> 2] >> (8 * (j & 3))) & 0xff;
        sumi += __mul24((int)(int16_t)(bs[j] & 0xffff), m) + __mul24((int)(int16_t)(bs[j] >> 16), m);
    }
    const uint32_t* qh = wb + 4;                                  // 8 dwords
    const uint32_t* qs = wb + 12;                                 // 32 dwords
    const uint32_t* q8 = reinterpret_cast<const uint32_t*>(qv);   // 64 dwords
    acc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int dl = 0, dh = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t wv = qs[8 * j + k], hv = qh[k];
            const uint32_t lo = (wv & 0x0f0f0f0fu) | (((hv >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t hi = ((wv >> 4) & 0x0f0f0f0fu) | (((hv >> (2 * j + 1)) & 0x01010101u) << 4);
            dl = __builtin_amdgcn_sdot4((int)lo, (int)q8[16 * j + k], dl, false);
            dh = __builtin_amdgcn_sdot4((int)hi, (int)q8[16 * j + 8 + k], dh, false);
        }
        const int sl = (su[j >> 1] >> (16 * (j & 1))) & 0xff;
        const int sh = (su[j >> 1] >> (16 * (j & 1) + 8)) & 0xff;
        acc += __mul24(dl, sl) + __mul24(dh, sh);
    }
}

// IQ4_XS x Q8_K block: acc[ib] = q8 . grid[idx] over sub-block ib (16 bytes:
// low nibbles pair with q8 bytes 32 ib .. + 15, high nibbles with 32 ib +
// 16 ..).  The grid (IQ4XS.cs:15-18) is looked up 4 bytes at a time with two
// byte permutes (entries 0-7 and 8-7) and a select on the index's bit 3.
// wb: the block's 34 dwords.
__device__ __forceinline__ void iq4xs_block_terms(const uint32_t* __restrict__ wb,
                                                  const uint32_t* __restrict__ q8b, int (&acc)[8]) {
    // grid bytes: -127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113
    const uint32_t g0 = 0xBFAD9881u, g1 = 0xF6EADDCFu, g2 = 0x26190D01u, g3 = 0x71594535u;
    uint4 qv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = reinterpret_cast<const uint4*>(q8b + Q8K_QS)[i];
    const uint32_t* q8 = reinterpret_cast<const uint32_t*>(qv);
    auto lookup = [&](uint32_t idx) {      // idx: four 4-bit indices, one a byte
        const uint32_t sel = idx & 0x07070707u;
        const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xffu;
        const uint32_t lo = __builtin_amdgcn_perm(g1, g0, sel), hi = __builtin_amdgcn_perm(g3, g2, sel);
        return (lo & ~m) | (hi & m);
    };
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        int a = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t wv = wb[2 + 4 * ib + k];
            a = __builtin_amdgcn_sdot4((int)lookup(wv & 0x0f0f0f0fu), (int)q8[8 * ib + k], a, false);
            a = __builtin_amdgcn_sdot4((int)lookup((wv >> 4) & 0x0f0f0f0fu), (int)q8[8 * ib + 4 + k], a, false);
        }
        acc[ib] = a;
    }
}

// One 64-thread workgroup per group of up to 8 whole rows (at most 64
// blocks, a block a thread, held in registers) and `tok_per_wg` tokens.  Per
// token: the token's Q8_K row is staged in LDS, every thread forms its
// block's integer terms, and one thread per row runs the reference's fp32
// chain over the row's blocks in order.
template <int QT>
__global__ __launch_bounds__(LQ_THREADS) void linear_qs(const unsigned char* __restrict__ w,
                                                        const uint32_t* __restrict__ q8,
                                                        float* __restrict__ y, int n_in, int n_out,
                                                        int tokens, int rows_per_wg, int tok_per_wg) {
#pragma clang fp contract(off)
    constexpr int BB = QT == 5 ? Q5K_BYTES : IQ4XS_BYTES;
    extern __shared__ uint4 smem[];
    const int nb = n_in / QK, lane = threadIdx.x;
    const int row0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, n_out - row0);
    const int nblk = nrows * nb;
    const int t_begin = blockIdx.y * tok_per_wg, t_end = min(tokens, t_begin + tok_per_wg);
    uint32_t* q8s = reinterpret_cast<uint32_t*>(smem);
    float* terms = reinterpret_cast<float*>(q8s + nb * Q8K_WORDS);

    // The thread's block straight into registers (Q5_K blocks are 16-byte
    // multiples, IQ4_XS blocks 8-byte multiples from a 16-byte aligned base).
    uint32_t wb[BB / 4];
    {
        const unsigned char* src = w + ((size_t)row0 * nb + min(lane, nblk - 1)) * BB;
        if constexpr (QT == 5) {
#pragma unroll
            for (int c = 0; c < BB / 16; ++c) reinterpret_cast<uint4*>(wb)[c] = reinterpret_cast<const uint4*>(src)[c];
        } else {
#pragma unroll
            for (int c = 0; c < BB / 8; ++c) reinterpret_cast<uint2*>(wb)[c] = reinterpret_cast<const uint2*>(src)[c];
        }
    }
    for (int t = t_begin; t < t_end; ++t) {
        {
            const uint4* src = reinterpret_cast<const uint4*>(q8 + (size_t)t * nb * Q8K_WORDS);
            uint4* dst = reinterpret_cast<uint4*>(q8s);
            const int n4 = nb * (Q8K_WORDS / 4);
            for (int i0 = 0; i0 < n4; i0 += 8 * LQ_THREADS) {
                uint4 qv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    qv[c] = make_uint4(0u, 0u, 0u, 0u);
                    if (i0 + lane + LQ_THREADS * c < n4) qv[c] = src[i0 + lane + LQ_THREADS * c];
                }
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (i0 + lane + LQ_THREADS * c < n4) dst[i0 + lane + LQ_THREADS * c] = qv[c];
            }
        }
        __syncthreads();
        // Each thread forms its block's terms of the reference's chain (they do
        // not depend on the running sum); one thread per row then adds them in
        // order.
        if (lane < nblk) {
            const uint32_t* q8b = q8s + (lane % nb) * Q8K_WORDS;
            const float yd = __builtin_bit_cast(float, q8b[0]);
            float* out = terms + lane * QS_TLD;
            if constexpr (QT == 5) {
                int acc, sumi;
                q5k_block_terms(wb, q8b, acc, sumi);
                const float d = half_bits_to_float(wb[0] & 0xffff) * yd;
                const float dmin = half_bits_to_float(wb[0] >> 16) * yd;
                out[0] = d * (float)acc - dmin * (float)sumi;
            } else {
                int acc[8];
                iq4xs_block_terms(wb, q8b, acc);
                const uint32_t hdr = wb[0], sl = wb[1];
                const float d = half_bits_to_float(hdr & 0xffff);
#pragma unroll
                for (int ib = 0; ib < 8; ++ib) {
                    const int ls = (int)(((sl >> (8 * (ib >> 1) + 4 * (ib & 1))) & 0xf) |
                                         (((hdr >> (16 + 2 * ib)) & 3) << 4));
                    const float dl = d * (float)(ls - 32);
                    out[ib] = dl * (float)acc[ib] * yd;
                }
            }
        }
        __syncthreads();
        if (lane < nrows) {
            constexpr int NTERM = QT == 5 ? 1 : 8;
            float sumf = 0.0f;
            const float* T = terms + lane * nb * QS_TLD;
            for (int b = 0; b < nb; ++b)
#pragma unroll
                for (int k = 0; k < NTERM; ++k) sumf += T[b * QS_TLD + k];
            y[(size_t)t * n_out + row0 + lane] = sumf;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- Q2_0C, STQ1_0

// Ternary-style formats whose weights sit at 2-byte aligned offsets
// (BlockLayout.cs:77-96):
//   Q2_0C (130 B, 512 values): f16 d, u8 qs[128], value 2 code - 3, codes
//     0..3 four a byte (Q2_0C.cs:12-13)
//   STQ1_0 (42 B, 256 values): u8 qs[32] (4-bit slots), u8 sign[8], f16 d;
//     group g = 16 chunk + gloc holds the values at chunk * 64 + gloc + 16
//     lane through a 32-entry four-lane codebook (STQ1_0.cs:50-75)
// One integer per 256-value Q8_K block (a "unit"): T = the exact signed dot
// of the unit's values with the block's int8 activations, formed as the
// reference does (codes 0..3 or 0..2 times q8, minus 3 or 1 times the bsums
// total).  The fp32 chain per output then follows the reference's order for
// that row: the eight-row panels (Q2Panel.cs:12-46, STQPanel.cs:13-48), one
// FMA per unit, acc = fma((float)T, dw * dx, acc); or the raw-row dot of the
// other rows, Q2_0C.DotAvx2 (Q2_0C.cs:67-79): acc += dw * ((float)T0 * dx0
// + (float)T1 * dx1) per 512 values, and STQ1_0.DotAvx2 (STQ1_0.cs:120-138):
// acc += (dw * dx) * (float)T.  Rows below panel_rows take the panel order.
constexpr int Q2_BYTES = 130, STQ_BYTES = 42;

// Bytes k of the four dwords q[0..3] gathered into dword k (a 4 x 4 byte
// transpose): Q2_0C's byte c of a qs dword holds values 4c .. 4c + 3, so its
// bit pair k of every byte meets the activations 16 i + 4c + k.
__device__ __forceinline__ uint4 byte_transpose(uint4 q) {
    const uint32_t a = __builtin_amdgcn_perm(q.y, q.x, 0x05010400u), b = __builtin_amdgcn_perm(q.y, q.x, 0x07030602u);
    const uint32_t c = __builtin_amdgcn_perm(q.w, q.z, 0x05010400u), d = __builtin_amdgcn_perm(q.w, q.z, 0x07030602u);
    return make_uint4(__builtin_amdgcn_perm(c, a, 0x05040100u), __builtin_amdgcn_perm(c, a, 0x07060302u),
                      __builtin_amdgcn_perm(d, b, 0x05040100u), __builtin_amdgcn_perm(d, b, 0x07060302u));
}

// Sum of a Q8_K block's 16 bsums (the workspace form).
__device__ __forceinline__ int q8k_bsum_total(const uint32_t* __restrict__ q8b) {
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t p = q8b[Q8K_BS + k];
        s += (int16_t)(p & 0xffff) + (int16_t)(p >> 16);
    }
    return s;
}

// Q2_0C half block (64 qs bytes at byte offset o of the staged weights) times
// a Q8_K block whose qs are staged byte-transposed per 16 bytes: 2 I - 3 S.
__device__ __forceinline__ int q2_unit_dot(const uint32_t* __restrict__ base, int o,
                                           const uint32_t* __restrict__ q8b) {
    int dot = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t wv = lds_word(base, o + 4 * i);
        const uint4 r = reinterpret_cast<const uint4*>(q8b + Q8K_QS)[i];
        dot = __builtin_amdgcn_sdot4((int)(wv & 0x03030303u), (int)r.x, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((wv >> 2) & 0x03030303u), (int)r.y, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((wv >> 4) & 0x03030303u), (int)r.z, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((wv >> 6) & 0x03030303u), (int)r.w, dot, false);
    }
    return 2 * dot - 3 * q8k_bsum_total(q8b);
}

// STQ1_0 block at byte offset o times a Q8_K block: encoded - S.  Four groups
// at a time: their slots (nibbles of one 16-bit half of qs) spread to bytes,
// looked up in the two 16-byte codebook halves with byte permutes, the half
// chosen per byte by the group's sign bit; lane L of the four patterns then
// meets activations chunk * 64 + 16 L + 4 i .. + 3.
__device__ __forceinline__ int stq_unit_dot(const uint32_t* __restrict__ base, int o,
                                            const uint32_t* __restrict__ q8b) {
    // STQ1_0.Codebook, entries 0-15 (sign 0) and 16-31 (sign 1), 4 a dword
    constexpr uint32_t L0 = 0x092989A9u, L1 = 0x062686A6u, L2 = 0x121A929Au, L3 = 0x424A626Au;
    constexpr uint32_t H0 = 0xA1812101u, H1 = 0xA4842404u, H2 = 0x98901810u, H3 = 0x68604840u;
    uint32_t qs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) qs[j] = lds_word(base, o + 4 * j);
    const uint32_t sg[2] = {lds_word(base, o + 32), lds_word(base, o + 36)};
    const uint32_t* q8 = q8b + Q8K_QS;
    int enc = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t s16 = (sg[c >> 1] >> (16 * (c & 1))) & 0xffffu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t h = (qs[2 * c + (i >> 1)] >> (16 * (i & 1))) & 0xffffu;
            const uint32_t idx = (h & 0xfu) | ((h & 0xf0u) << 4) | ((h & 0xf00u) << 8) | ((h & 0xf000u) << 12);
            const uint32_t sel = idx & 0x07070707u;
            const uint32_t hib = ((idx >> 3) & 0x01010101u) * 0xffu;
            const uint32_t lo = (__builtin_amdgcn_perm(L1, L0, sel) & ~hib) | (__builtin_amdgcn_perm(L3, L2, sel) & hib);
            const uint32_t hi = (__builtin_amdgcn_perm(H1, H0, sel) & ~hib) | (__builtin_amdgcn_perm(H3, H2, sel) & hib);
            const uint32_t neg = ((((s16 >> (4 * i)) & 0xfu) * 0x00204081u) & 0x01010101u) * 0xffu;
            const uint32_t p = (lo & ~neg) | (hi & neg);
#pragma unroll
            for (int L = 0; L < 4; ++L)
                enc = __builtin_amdgcn_sdot4((int)((p >> (2 * L)) & 0x03030303u), (int)q8[16 * c + 4 * L + i], enc,
                                             false);
        }
    }
    return enc - q8k_bsum_total(q8b);
}

// One 64-thread workgroup per group of up to 8 whole rows (at most 64 units,
// one a thread) and tok_per_wg tokens: the rows' contiguous weight bytes are
// staged in LDS once (as for Q6_K), then per token the Q8_K row is staged,
// every thread forms its unit's T, and one thread per row runs the chain.
template <int QT>
__global__ __launch_bounds__(LQ_THREADS) void linear_qt(const unsigned char* __restrict__ w,
                                                        const uint32_t* __restrict__ q8,
                                                        float* __restrict__ y, int n_in, int n_out,
                                                        int tokens, int rows_per_wg, int tok_per_wg,
                                                        int panel_rows) {
#pragma clang fp contract(off)
    constexpr int UB = QT == 2 ? Q2_BYTES / 2 : STQ_BYTES;   // weight bytes per unit
    extern __shared__ uint4 smem[];
    const int nb = n_in / QK, lane = threadIdx.x;
    const int row0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, n_out - row0);
    const int nunit = nrows * nb;
    const int t_begin = blockIdx.y * tok_per_wg, t_end = min(tokens, t_begin + tok_per_wg);
    const size_t row_bytes = (size_t)nb * UB;
    const int nchunk_max = (rows_per_wg * nb * UB + 31) / 16 + 1;
    uint4* wsh = smem;
    uint32_t* q8s = reinterpret_cast<uint32_t*>(smem + nchunk_max);
    int* tv = reinterpret_cast<int*>(q8s + nb * Q8K_WORDS);
    const uint32_t* wbase = reinterpret_cast<const uint32_t*>(wsh);

    // The rows' bytes from the 16-byte boundary below their even start; only
    // the buffer's last chunk can be partial, read with 2-byte loads.
    const size_t total = (size_t)n_out * row_bytes;
    const size_t start = (size_t)row0 * row_bytes;
    const size_t s16 = start & ~(size_t)15;
    const int shift = (int)(start - s16);
    const int nchunks = (int)((start + (size_t)nrows * row_bytes - s16 + 15) >> 4);
    constexpr int MAXC = (LQ_THREADS * UB + 31 + LQ_THREADS * 16 - 1) / (LQ_THREADS * 16) + 1;
    {
        uint4 wv[MAXC];
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const int i = lane + LQ_THREADS * c;
            const size_t off = s16 + 16 * (size_t)i;
            wv[c] = make_uint4(0u, 0u, 0u, 0u);
            if (i < nchunks && off + 16 <= total) wv[c] = *reinterpret_cast<const uint4*>(w + off);
        }
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const int i = lane + LQ_THREADS * c;
            const size_t off = s16 + 16 * (size_t)i;
            if (i < nchunks) {
                if (off + 16 <= total) {
                    wsh[i] = wv[c];
                } else {
                    uint32_t wd[4] = {0u, 0u, 0u, 0u};
                    for (int hb = 0; hb < 8 && off + 2 * hb < total; ++hb)
                        wd[hb >> 1] |= (uint32_t)(*reinterpret_cast<const uint16_t*>(w + off + 2 * hb)) << (16 * (hb & 1));
                    wsh[i] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
                }
            }
        }
    }

    for (int t = t_begin; t < t_end; ++t) {
        {
            const uint4* src = reinterpret_cast<const uint4*>(q8 + (size_t)t * nb * Q8K_WORDS);
            uint4* dst = reinterpret_cast<uint4*>(q8s);
            const int n4 = nb * (Q8K_WORDS / 4);
            for (int i0 = 0; i0 < n4; i0 += 8 * LQ_THREADS) {
                uint4 qv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    qv[c] = make_uint4(0u, 0u, 0u, 0u);
                    if (i0 + lane + LQ_THREADS * c < n4) qv[c] = src[i0 + lane + LQ_THREADS * c];
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int i = i0 + lane + LQ_THREADS * c;
                    if (i < n4) {
                        const int part = i % (Q8K_WORDS / 4);     // 1..16: qs, 0 and 17..18: d, bsums
                        dst[i] = (QT == 2 && part >= 1 && part <= 16) ? byte_transpose(qv[c]) : qv[c];
                    }
                }
            }
        }
        __syncthreads();
        if (lane < nunit) {
            const int r = lane / nb, b = lane % nb;
            const uint32_t* q8b = q8s + b * Q8K_WORDS;
            if constexpr (QT == 2)
                tv[lane] = q2_unit_dot(wbase, shift + (int)(r * row_bytes) + (b >> 1) * Q2_BYTES + 2 + 64 * (b & 1), q8b);
            else
                tv[lane] = stq_unit_dot(wbase, shift + (int)(r * row_bytes) + b * STQ_BYTES, q8b);
        }
        __syncthreads();
        if (lane < nrows) {
            const int row = row0 + lane;
            const int* T = tv + lane * nb;
            const int o = shift + (int)(lane * row_bytes);
            float acc = 0.0f;
            if (row < panel_rows) {
                for (int b = 0; b < nb; ++b) {
                    const int dof = QT == 2 ? o + (b >> 1) * Q2_BYTES : o + b * STQ_BYTES + 40;
                    const float dw = half_bits_to_float(lds_word(wbase, dof) & 0xffff);
                    const float dx = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]);
                    acc = fmaf((float)T[b], dw * dx, acc);
                }
            } else if constexpr (QT == 2) {
                for (int b = 0; b < nb; b += 2) {
                    const float dw = half_bits_to_float(lds_word(wbase, o + (b >> 1) * Q2_BYTES) & 0xffff);
                    const float dx0 = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]);
                    const float dx1 = __builtin_bit_cast(float, q8s[(b + 1) * Q8K_WORDS]);
                    acc = acc + dw * ((float)T[b] * dx0 + (float)T[b + 1] * dx1);
                }
            } else {
                for (int b = 0; b < nb; ++b) {
                    const float dw = half_bits_to_float(lds_word(wbase, o + b * STQ_BYTES + 40) & 0xffff);
                    const float dx = __builtin_bit_cast(float, q8s[b * Q8K_WORDS]);
                    acc = acc + (dw * dx) * (float)T[b];
                }
            }
            y[(size_t)t * n_out + row] = acc;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- F32

// Qwen35Model.F32Gemm (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:129-140):
// y[t][o] = Ops.DotF32(x[t], W[o]) (Ops.cs:418-449) in its order: 16 FMA
// lanes over 16-float strides (lane j takes elements 16 k + j), one 8-float
// stride into lanes 0-7, then HorizontalSum(acc0 + acc1) and a scalar tail.
// Four threads per output row, thread q holding reference lanes 4q .. 4q+3
// (a float4 of each stride when rows are 16-byte aligned); 64 rows a
// 256-thread workgroup, one token per grid row.
template <bool VEC>
__global__ __launch_bounds__(256) void linear_f32(const float* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ y, int n_in, int n_out) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, q = tid & 3;
    const int row = blockIdx.x * 64 + (tid >> 2), t = blockIdx.y;
    const int rr = min(row, n_out - 1);            // rows past n_out compute row n_out - 1, not stored
    const float* a = x + (size_t)t * n_in;
    const float* b = w + (size_t)rr * n_in;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int i = 0;
    for (; i + 16 <= n_in; i += 16) {
        float av[4], bv[4];
        if constexpr (VEC) {
            const float4 a4 = *reinterpret_cast<const float4*>(a + i + 4 * q);
            const float4 b4 = *reinterpret_cast<const float4*>(b + i + 4 * q);
            av[0] = a4.x; av[1] = a4.y; av[2] = a4.z; av[3] = a4.w;
            bv[0] = b4.x; bv[1] = b4.y; bv[2] = b4.z; bv[3] = b4.w;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) { av[k] = a[i + 4 * q + k]; bv[k] = b[i + 4 * q + k]; }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = fmaf(av[k], bv[k], acc[k]);
    }
    if (i + 8 <= n_in) {
        if (q < 2)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = fmaf(a[i + 4 * q + k], b[i + 4 * q + k], acc[k]);
        i += 8;
    }
    // s_j = acc0_j + acc1_j: threads 0, 1 hold acc0 lanes 0-7, threads 2, 3 acc1.
    float s[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) s[k] = acc[k] + __shfl_xor(acc[k], 2, kWave);
    // HorizontalSum: (s_k + s_{k+4}) pairs, then (0 + 2) + (1 + 3).
    float u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) u[k] = s[k] + __shfl_xor(s[k], 1, kWave);
    if (q == 0 && row < n_out) {
        const float t0 = u[0] + u[2], t1 = u[1] + u[3];
        float sum = t0 + t1;
        for (; i < n_in; ++i) sum += a[i] * b[i];
        y[(size_t)t * n_out + row] = sum;
    }
}

// ---------------------------------------------------------------- Q4_K, several tokens

// The reference's Q4_K path for several tokens (MulMatQ4K.Gemm,
// MulMatQ4K.cs:45-127 -> GemmQ4K.GemmAvx2Tile, GemmQ4K.Avx2.cs:39-207) for
// the first n_out & ~7 outputs: per (token, output row), over blocks b and
// 32-value sub-blocks s in order, acc = fma((float)(sc_s * dot_s), dw * dx,
// acc), with dot_s the exact integer q4 . q8 of the sub-block; per block, mn =
// fma((float)(sum_j min_j (bsums[2j] + bsums[2j+1])), dminw * dx, mn); out =
// acc - mn.  A workgroup of 8 waves takes 64 tokens x 128 rows (wave = 64
// tokens x 16 rows: 4 tiles of 16 x 16).  dot_s of a tile is one
// v_mfma_i32_16x16x32_i8 whose accumulator starts at the bits of 1.5 * 2^23,
// so the result read as fp32 is exactly 1.5 * 2^23 + dot_s (|dot_s| <= 60960
// < 2^22) and (float)(sc * dot_s) = fma(that, sc, -1.5 * 2^23 * sc) exactly
// (the exact value is an integer below 2^24): two VALU operations an output
// per sub-block, the floor the reference's order sets.  The min term's
// integer (at most 8 x 63 x 4064, exact in fp32) is two
// v_mfma_f32_16x16x4f32 on small integers.  Blocks are double-buffered in
// LDS, the next one loaded by buffer loads straight into LDS (16-byte chunks,
// 64 a wave-wide load) while the current one is processed.  The rows and
// tokens of one launch stay below 2 GiB of weights and of activations (the
// host splits larger calls).
constexpr int GT = 64, GR = 128;
constexpr int GW_CHUNKS = GR * Q4K_BYTES / 16;          // 1152
constexpr int GX_CHUNKS = GT * Q8K_WORDS / 4;           // 1216
constexpr int GTHREADS = 512, GRT = GR / 16 / (GTHREADS / 64);   // row tiles a wave: 1
constexpr int GWAVES = GTHREADS / 64;
constexpr int GRUNS = (GX_CHUNKS + 64 * GWAVES - 1) / (64 * GWAVES);   // wave-wide loads a wave: 3
constexpr int kMagic = 0x4B400000;                      // bits of 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(GTHREADS) __attribute__((amdgpu_waves_per_eu(2)))
void q4k_gemm(const unsigned char* __restrict__ w, const uint32_t* __restrict__ q8,
              float* __restrict__ y, int n_in, int n_rows, int n_out, int tokens) {
#pragma clang fp contract(off)
    const int nb = n_in / QK;
    const int row0 = blockIdx.x * GR, tok0 = blockIdx.y * GT;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;

    __shared__ uint4 wsh[2][GW_CHUNKS];
    __shared__ uint4 xsh[2][GX_CHUNKS];

    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(w), 0, (int)((uint32_t)n_rows * nb * Q4K_BYTES), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(q8), 0, (int)((uint32_t)tokens * nb * Q8K_WORDS * 4), 0x00020000);
    // Wave-wide load q covers chunks 64 q .. 64 q + 63; wave w issues q = w,
    // w + 8, w + 16.  Per-lane offsets of block 0 (rows and tokens clamped);
    // block b adds b times the block size as the scalar offset.
    uint32_t wvo[GRUNS], xvo[GRUNS];
#pragma unroll
    for (int m = 0; m < GRUNS; ++m) {
        const int i = 64 * (wave + GWAVES * m) + lane;
        wvo[m] = (uint32_t)min(row0 + i / 9, n_rows - 1) * nb * Q4K_BYTES + 16 * (i % 9);
        xvo[m] = (uint32_t)min(tok0 + i / 19, tokens - 1) * nb * Q8K_WORDS * 4 + 16 * (i % 19);
    }
    auto stage = [&](int b, int buf) {
#pragma unroll
        for (int m = 0; m < GRUNS; ++m) {
            const int q = wave + GWAVES * m;
            if (64 * q < GW_CHUNKS) dma_b128(wrs, &wsh[buf][64 * q], wvo[m], (uint32_t)b * Q4K_BYTES);
            if (64 * q < GX_CHUNKS) dma_b128(xrs, &xsh[buf][64 * q], xvo[m], (uint32_t)b * Q8K_WORDS * 4);
        }
    };

    float acc[4][GRT][4], mn[4][GRT][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < GRT; ++rt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tt][rt][r] = mn[tt][rt][r] = 0.0f;
    const i32x4 magic = {kMagic, kMagic, kMagic, kMagic};

    stage(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const int buf = b & 1;
        if (b + 1 < nb) stage(b + 1, buf ^ 1);
        const uint32_t* W = reinterpret_cast<const uint32_t*>(wsh[buf]);
        const uint32_t* X = reinterpret_cast<const uint32_t*>(xsh[buf]);
        // D rows of tile tt: tokens 16 tt + 4 lg + r; A rows: token 16 tt + l16.
        float dx[4][4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                dx[tt][r] = __builtin_bit_cast(float, X[(16 * tt + 4 * lg + r) * Q8K_WORDS]);
        const uint32_t* wr[GRT];
        float dw[GRT], dmw[GRT];
        uint32_t sl[GRT], sh[GRT], s1[GRT], s2[GRT];
#pragma unroll
        for (int rt = 0; rt < GRT; ++rt) {
            wr[rt] = W + (16 * GRT * wave + 16 * rt + l16) * (Q4K_BYTES / 4);
            const uint32_t hdr = wr[rt][0], S0 = wr[rt][1];
            s1[rt] = wr[rt][2];
            s2[rt] = wr[rt][3];
            dw[rt] = half_bits_to_float(hdr & 0xffff);
            dmw[rt] = half_bits_to_float(hdr >> 16);
            sl[rt] = S0 & 0x3f3f3f3fu;                                   // scales 0-3
            sh[rt] = (s2[rt] & 0x0f0f0f0fu) | ((S0 >> 2) & 0x30303030u);  // scales 4-7
        }
        float cs[4][GRT][4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int rt = 0; rt < GRT; ++rt)
#pragma unroll
                for (int r = 0; r < 4; ++r) cs[tt][rt][r] = dw[rt] * dx[tt][r];
        uint32_t wq[GRT][2] = {};
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) {
            const int g = sb >> 1, hi = sb & 1;
            if (!hi) {
#pragma unroll
                for (int rt = 0; rt < GRT; ++rt) {
                    wq[rt][0] = wr[rt][4 + 8 * g + 2 * lg];
                    wq[rt][1] = wr[rt][4 + 8 * g + 2 * lg + 1];
                }
            }
            long bv[GRT];
            float scf[GRT], negc[GRT];
#pragma unroll
            for (int rt = 0; rt < GRT; ++rt) {
                const uint32_t b0 = hi ? (wq[rt][0] >> 4) & 0x0f0f0f0fu : wq[rt][0] & 0x0f0f0f0fu;
                const uint32_t b1 = hi ? (wq[rt][1] >> 4) & 0x0f0f0f0fu : wq[rt][1] & 0x0f0f0f0fu;
                bv[rt] = (long)(((unsigned long)b1 << 32) | b0);
                scf[rt] = (float)(((sb < 4 ? sl[rt] : sh[rt]) >> (8 * (sb & 3))) & 0xffu);
                negc[rt] = scf[rt] * -kMagicF;
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const uint2 a = *reinterpret_cast<const uint2*>(X + (16 * tt + l16) * Q8K_WORDS + Q8K_QS + 8 * sb + 2 * lg);
                const long av = (long)(((unsigned long)a.y << 32) | a.x);
#pragma unroll
                for (int rt = 0; rt < GRT; ++rt) {
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv[rt], magic, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        // __int_as_float of the element's value: __builtin_bit_cast on a
                        // vector element reads the vector's first word.
                        const float t = fmaf(__int_as_float(d[r]), scf[rt], negc[rt]);
                        acc[tt][rt][r] = fmaf(t, cs[tt][rt][r], acc[tt][rt][r]);
                    }
                    // The sub-block's sums are folded here, not all after the
                    // last sub-block (which would hold 8 tiles of results live).
                    asm volatile("" : "+v"(acc[tt][rt][0]), "+v"(acc[tt][rt][1]), "+v"(acc[tt][rt][2]),
                                 "+v"(acc[tt][rt][3]));
                }
            }
            // keep each sub-block's MFMA results to its own four quads
            __builtin_amdgcn_sched_barrier(0);
        }
        // Min term: j = lg and lg + 4 of this lane's row (B) and token (A).
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const uint32_t* xa = X + (16 * tt + l16) * Q8K_WORDS + Q8K_BS;
            float pa[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t p = xa[lg + 4 * h];
                pa[h] = (float)((int)(int16_t)(p & 0xffff) + (int)(int16_t)(p >> 16));
            }
#pragma unroll
            for (int rt = 0; rt < GRT; ++rt) {
                const float m0 = (float)((s1[rt] >> (8 * lg)) & 63);
                const float m1 = (float)(((s2[rt] >> (8 * lg + 4)) & 15) | (((s1[rt] >> (8 * lg + 6)) & 3) << 4));
                f32x4 md = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[0], m0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                md = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[1], m1, md, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // dx again from LDS rather than live across the sub-blocks
                    const float dxr = __builtin_bit_cast(float, X[(16 * tt + 4 * lg + r) * Q8K_WORDS]);
                    mn[tt][rt][r] = fmaf(md[r], dmw[rt] * dxr, mn[tt][rt][r]);
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < GRT; ++rt) {
            const int row = row0 + 16 * GRT * wave + 16 * rt + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = tok0 + 16 * tt + 4 * lg + r;
                if (row < n_rows && t < tokens) y[(size_t)t * n_out + row] = acc[tt][rt][r] - mn[tt][rt][r];
            }
        }
}


// ---------------------------------------------------------------- Q6_K, several tokens

// The reference's Q6_K path for several tokens keeps the GEMV's arithmetic
// per (token, output row) (Q6K.Gemm, Q6K.cs:301-413, over Q6K.DotAvx2,
// Q6K.cs:87-165): per block, 8 integer lanes sumi[k] = sum over j < 2, m < 4,
// i < 4 of scales[8j + 2m + k/4] * v * q8 (v the unsigned 6-bit value of byte
// b = 4k + i of part j, m), minus 32 (bsums[2k] scales[2k] + bsums[2k+1]
// scales[2k+1]); acc[k] = fma(dx * dw, (float)sumi[k], acc[k]); out =
// hsum8(acc).  Each sumi[k] is exact in int32, so it is formed on
// v_mfma_i32_16x16x64_i8: for lane k, lane group g of the MFMA (j = g / 2,
// m0 = 2 (g % 2)) brings the 8 values of parts (j, m0) and (j, m0 + 1) at
// bytes 4k .. 4k + 3 and, as the other half of K, q8 bytes 32k + 8g .. + 7
// (sub-block 2k + j) against -32 scales[2k + j]: the bsums term without the
// bsums.  The weights scales * v (|.| <= 8064) and -32 scales are split into
// two int8 planes, 128 hi + lo, one MFMA each: sumi = (D_hi << 7) + D_lo.
//
// A workgroup takes 64 tokens x 32 rows; wave w takes rows 16 (w % 2) ..
// + 15 of all 64 tokens for lanes k in {0, 1, 4, 5} (w < 2) or {2, 3, 6, 7},
// so each value split serves four token tiles; at the end the upper waves
// pass a_2 + a_6 and a_3 + a_7 to the lower ones, which finish hsum8 in its
// order.  Blocks go to LDS by buffer loads straight into LDS (no registers,
// double-buffered, one block ahead): per token its 64 qs dwords (dwords
// 16-31 and 48-63 swapped in pairs so the value reads of lane groups 2g and
// 2g + 1 fall on opposite bank parities; with a 66-dword token stride every
// read is conflict-free) and its scale; per row the 53 dwords from the
// 4-byte boundary below its 2-byte-aligned block, realigned on read.  Needs
// n_out * n_in / 256 even (the last row block then ends on a 4-byte
// boundary; otherwise the per-token GEMV runs).  The rows and tokens of one
// launch stay below 2 GiB of weights and of activations (the host splits
// larger calls at even rows).
constexpr int SGT = 64, SGR = 32;
constexpr int SX_STRIDE = 66;      // LDS dwords a token: 64 qs dwords, 2 of padding
constexpr int SW_STRIDE = 53;      // LDS dwords a row: the raw dwords covering its block

struct Q6Stage {
    uint32_t x[SGT * SX_STRIDE];
    float dx[SGT];
    uint32_t w[SGR * SW_STRIDE];
};

typedef const volatile __attribute__((address_space(3))) uint32_t lds_cvu32;

typedef short s16x2 __attribute__((ext_vector_type(2)));

// Four unsigned 6-bit values given doubled (bytes of v2 = 2 v) times sc, as
// the low (& 127) and high (>> 7, two's complement) int8 planes of the
// products sc v.  The doubled 16-bit products 2 sc v are formed in pairs:
// the high plane is their high bytes, the low plane bits 1-7 of their low
// bytes.
__device__ __forceinline__ void q6k_split(uint32_t v2, int sc, uint32_t& lo, uint32_t& hi) {
    const s16x2 s2 = {(short)sc, (short)sc};
    const uint32_t a = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v2, 0x0c010c00u)) * s2);
    const uint32_t b = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v2, 0x0c030c02u)) * s2);
    lo = (__builtin_amdgcn_perm(b, a, 0x06040200u) >> 1) & 0x7f7f7f7fu;
    hi = __builtin_amdgcn_perm(b, a, 0x07050301u);
}

// A operand of lane k = 2 KH + (kk & 1) + 4 (kk >> 1) for token tile tt:
// qs dwords 32j + 8 m0 + k and + 8 (the values' q8), then 8k + 4j + (g & 1)
// and + 2 (sub-block 2k + j: lane groups 2j and 2j + 1 read opposite bank
// parities).  LDS slot s holds qs dword s ^ ((s >> 4) & 1).  Volatile LDS
// reads keep each operand's four dwords in their own registers (merged reads
// would mix operands of different lanes in one register quad).
template <int KH>
__device__ __forceinline__ i32x4 q6k_load_a(lds_cvu32* xv, int kk, int tt, int j, int odd) {
    const int k = 2 * KH + (kk & 1) + 4 * (kk >> 1);
    const int qa_s = 32 * j + 16 * odd + (k ^ odd);
    const int qe_s = (8 * k + 4 * j + odd) ^ ((k >> 1) & 1);
    lds_cvu32* xt = xv + SX_STRIDE * 16 * tt;
    return i32x4{(int)xt[qa_s], (int)xt[qa_s + 8], (int)xt[qe_s], (int)xt[qe_s + 2]};
}

// One staged block: lanes k of half KH for the wave's 16 rows x 64 tokens.
template <int KH>
__device__ __forceinline__ void q6k_gemm_block(const Q6Stage& s, int shift, int rl, int l16, int lg,
                                               float (&acc)[4][4][4]) {
#pragma clang fp contract(off)
    const int j = lg >> 1, odd = lg & 1;
    const i32x4 zero = {0, 0, 0, 0};
    const uint32_t* wr = s.w + SW_STRIDE * rl;
    // dword f of the row's block
    auto wd = [&](int f) { return __builtin_amdgcn_alignbyte(wr[f + 1], wr[f], shift); };
    const float dw = half_bits_to_float(reinterpret_cast<const uint16_t*>(wr)[(shift + 208) >> 1]);
    const uint32_t scw = wd(48 + lg);                        // scales 4 lg .. 4 lg + 3
    float d[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const float4 x4 = *reinterpret_cast<const float4*>(&s.dx[16 * tt + 4 * lg]);
        d[tt][0] = x4.x * dw; d[tt][1] = x4.y * dw; d[tt][2] = x4.z * dw; d[tt][3] = x4.w * dw;
    }
    // right rotations: low (g even) or high nibbles to bits 1-4; qh bits
    // 0-1 / 4-5 (v0) and 2-3 / 6-7 (v1) to bits 5-6
    const uint32_t rq = odd ? 3 : 31, rh0 = odd ? 31 : 27, rh1 = odd ? 1 : 29;
    lds_cvu32* xv = (lds_cvu32*)(s.x + SX_STRIDE * l16);
    // B operands (both planes) of lane k for this lane's row
    auto planes = [&](int kk, i32x4& bh, i32x4& bl) {
        const int k = 2 * KH + (kk & 1) + 4 * (kk >> 1), half = kk >> 1;
        // Doubled 6-bit values of parts (j, m0) and (j, m0 + 1): nibble bits
        // to 1-4 and qh bits to 5-6 of each byte, by rotations.
        const uint32_t qa = wd(16 * j + k), qb = wd(16 * j + 8 + k), qh = wd(32 + 8 * j + k);
        const uint32_t v0 = (__builtin_amdgcn_alignbit(qa, qa, rq) & 0x1e1e1e1eu) |
                            (__builtin_amdgcn_alignbit(qh, qh, rh0) & 0x60606060u);
        const uint32_t v1 = (__builtin_amdgcn_alignbit(qb, qb, rq) & 0x1e1e1e1eu) |
                            (__builtin_amdgcn_alignbit(qh, qh, rh1) & 0x60606060u);
        const int sc0 = (int)(int8_t)(scw >> (8 * half)), sc1 = (int)(int8_t)(scw >> (8 * (2 + half)));
        uint32_t l0, h0, l1, h1;
        q6k_split(v0, sc0, l0, h0);
        q6k_split(v1, sc1, l1, h1);
        // -32 scales[2k + j] = 128 ((-s) >> 2) + 32 ((-s) & 3), bytes replicated
        const int neg = -(int)reinterpret_cast<const int8_t*>(wr)[shift + 192 + 2 * k + j];
        const uint32_t elo = __builtin_amdgcn_perm(0u, (uint32_t)((neg & 3) << 5), 0u);
        const uint32_t ehi = __builtin_amdgcn_perm(0u, (uint32_t)(neg >> 2), 0u);
        bh = i32x4{(int)h0, (int)h1, (int)ehi, (int)ehi};
        bl = i32x4{(int)l0, (int)l1, (int)elo, (int)elo};
    };
    // Each operand's reads go out one step (token tile) ahead of its
    // products; the next lane's B planes are formed after the current
    // lane's last step.
    i32x4 a = q6k_load_a<KH>(xv, 0, 0, j, odd);
    i32x4 bh, bl;
    planes(0, bh, bl);
#pragma unroll
    for (int step = 0; step < 16; ++step) {
        const int kk = step >> 2, tt = step & 3;
        i32x4 an = a;
        if (step < 15) an = q6k_load_a<KH>(xv, (step + 1) >> 2, (step + 1) & 3, j, odd);
        const i32x4 dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bh, zero, 0, 0, 0);
        const i32x4 dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bl, zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int sumi = (int)((unsigned)dh[r] << 7) + dl[r];
            acc[tt][kk][r] = fmaf(d[tt][r], (float)sumi, acc[tt][kk][r]);
        }
        if (tt == 3 && kk < 3) planes(kk + 1, bh, bl);
        a = an;
    }
}

template <int KH>
__device__ __forceinline__ void q6k_gemm_run(Q6Stage (&st)[2], const unsigned char* __restrict__ w,
                                             const uint32_t* __restrict__ q8, float* __restrict__ y, int nb,
                                             int n_rows, int n_out, int tokens, int row0, int tok0, int wave,
                                             int lane) {
#pragma clang fp contract(off)
    const int l16 = lane & 15, lg = lane >> 4, rt = wave & 1;
    const int rl = 16 * rt + l16;                            // this lane's row in the tile
    const uint32_t wbytes = (uint32_t)n_rows * nb * Q6K_BYTES;
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(w), 0, (int)wbytes, 0x00020000);
    const uint32_t blk_x = Q8K_WORDS * 4;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(q8), 0, (int)((uint32_t)tokens * nb * blk_x), 0x00020000);
    // Per-lane offsets, the same for every block: the qs dword of LDS slot
    // `lane` (pairs swapped in dwords 16-31 and 48-63), a token's scale.
    const uint32_t vx = 4u * (Q8K_QS + (lane ^ ((lane >> 4) & 1)));
    const uint32_t vdx = (uint32_t)min(tok0 + lane, tokens - 1) * nb * blk_x;

    auto stage = [&](int b, Q6Stage& s) {
#pragma unroll
        for (int i = 0; i < SGT / 4; ++i) {
            const int t = wave + 4 * i;
            dma_b32(xrs, &s.x[SX_STRIDE * t], vx, ((uint32_t)min(tok0 + t, tokens - 1) * nb + b) * blk_x);
        }
#pragma unroll
        for (int i = 0; i < SGR / 4; ++i) {
            const int r = wave + 4 * i;
            const uint32_t so = (((uint32_t)min(row0 + r, n_rows - 1) * nb + b) * Q6K_BYTES) & ~3u;
            if (lane < SW_STRIDE) dma_b32(wrs, &s.w[SW_STRIDE * r], 4u * lane, so);
        }
        if (wave == 0) dma_b32(xrs, s.dx, vdx, b * blk_x);
    };

    // Byte offset of the row's block in its raw dwords, for even and odd b
    // (blocks are 210 bytes: the offset alternates between 0 and 2).
    const int rpar = (min(row0 + rl, n_rows - 1) * nb) & 1;
    const int shift_e = 2 * rpar, shift_o = 2 * (rpar ^ 1);

    float acc[4][4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tt][kk][r] = 0.0f;

    stage(0, st[0]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const int p = b & 1;
        if (b + 1 < nb) stage(b + 1, st[p ^ 1]);
        q6k_gemm_block<KH>(st[p], p ? shift_o : shift_e, rl, l16, lg, acc);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    // hsum8 (s_k = a_k + a_{k+4}; (s0 + s2) + (s1 + s3)) across the two halves.
    float2* ex = reinterpret_cast<float2*>(st[0].x);
    if (KH == 1)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                ex[(rt * 16 + 4 * tt + r) * 64 + lane] =
                    make_float2(acc[tt][0][r] + acc[tt][2][r], acc[tt][1][r] + acc[tt][3][r]);
    __syncthreads();
    if (KH == 0) {
        const int row = row0 + rl;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float2 o = ex[(rt * 16 + 4 * tt + r) * 64 + lane];
                const float s0 = acc[tt][0][r] + acc[tt][2][r], s1 = acc[tt][1][r] + acc[tt][3][r];
                const float t0 = s0 + o.x, t1 = s1 + o.y;
                const int t = tok0 + 16 * tt + 4 * lg + r;
                if (row < n_rows && t < tokens) y[(size_t)t * n_out + row] = t0 + t1;
            }
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void q6k_gemm(const unsigned char* __restrict__ w, const uint32_t* __restrict__ q8, float* __restrict__ y,
              int n_in, int n_rows, int n_out, int tokens) {
    __shared__ Q6Stage st[2];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nb = n_in / QK, row0 = blockIdx.x * SGR, tok0 = blockIdx.y * SGT;
    if (wave >> 1)
        q6k_gemm_run<1>(st, w, q8, y, nb, n_rows, n_out, tokens, row0, tok0, wave, lane);
    else
        q6k_gemm_run<0>(st, w, q8, y, nb, n_rows, n_out, tokens, row0, tok0, wave, lane);
}


// ---------------------------------------------------------------- block order, several tokens

// Opt-in order for Q6_K with several tokens (q35m_set_projection_order,
// block order): per (token, row) and 256-value block, the whole integer sum
//   isum = sum over the block of scale(sub-block) * (v - 32) * q8
// is formed exactly in int32 (|isum| < 2^31), and the fp32 scales apply once
// per block: acc = fma((float)isum, dw * dx, acc).  The integer part is the
// reference's, exactly; only the fp32 accumulation order differs from its 8
// per-lane chains and their horizontal sum, within fp32 rounding of the
// exact value.  The sub-block scales fold into the weights as two int8
// planes, scale * (v - 32) = 128 hi + lo, so one v_mfma_i32_16x16x64_i8 per
// plane covers 64 values of every sub-block it meets and the 4 K-steps of a
// block accumulate in the MFMA's own int32 registers: no VALU work per
// sub-block or lane, only per block (half the MFMAs of the reference-order
// kernel, which needs one product set per lane).  Operand layout of a
// 64-value K-step ks: lane (n = l16, lane group lg) holds values 64 ks +
// 16 lg .. + 15 of its token (A: 16 consecutive Q8_K bytes) and of its row
// (B: the same values of the row's block, scale-folded), which lie in one
// sub-block, so a lane needs one scale per K-step.  A workgroup of 8 waves
// takes 192 tokens x 128 rows, a wave 192 tokens x 16 rows (12 token tiles,
// so each row's planes serve 12 MFMAs); blocks are double-buffered in LDS
// (155 KiB), the next one loaded by buffer loads straight into LDS.  192
// tokens make 2048 tokens x 2560 rows one round of 220 workgroups, one per
// CU (128 tokens took 320 workgroups, 1.25 rounds: 130 us).
//
// The same scheme for Q4_K (sc * q4 <= 945 as two planes) gives no gain: its
// reference kernel already needs one 16x16x32 product per sub-block, and on
// gfx950 a 16x16x64 product takes the cycles of a 16x16x32 one, so the planes
// double the MFMA work that the saved VALU pays for (190-200 vs 188-205 us
// at 2048 tokens x 2560 -> 8192; one 16x16x32 product per sub-block with
// the scale applied by an int32 multiply-add measured 207 us).  Q4_K keeps
// the reference's order.
constexpr int BT = 192, BR = 128, BTILES = BT / 16;
constexpr int BTHREADS = 512, BWAVES = BTHREADS / 64;
// Only d and qs of a Q8_K block are staged (17 of its 19 16-byte chunks;
// the block sums are not used), 68 words a token.
constexpr int BX_TOK_CHUNKS = Q8K_BS / 4, BX_TOK_WORDS = 4 * BX_TOK_CHUNKS;
constexpr int BX_CHUNKS = BT * BX_TOK_CHUNKS;                               // 3264
constexpr int BX_RUNS = (BX_CHUNKS + 64 * BWAVES - 1) / (64 * BWAVES);      // 7

// Per-lane offsets of block 0 for the activation staging of a workgroup
// (wave-wide load m covers chunks 64 (wave + BWAVES m) ..).
__device__ __forceinline__ void blk_x_offsets(uint32_t (&xvo)[BX_RUNS], int tok0, int tokens, int nb, int wave,
                                              int lane) {
#pragma unroll
    for (int m = 0; m < BX_RUNS; ++m) {
        const int i = 64 * (wave + BWAVES * m) + lane;
        xvo[m] = (uint32_t)min(tok0 + i / BX_TOK_CHUNKS, tokens - 1) * nb * Q8K_WORDS * 4 + 16 * (i % BX_TOK_CHUNKS);
    }
}

// Q6_K in block order.  Weight value w = scale(sub-block of 16) * (v - 32)
// (v the 6-bit value), |w| <= 4096, split as 128 hi + lo (hi in [-32, 32],
// lo in [0, 127]): 2 w = scale * 2v - 64 scale is formed in 16-bit pairs and
// its high byte and bits 1-7 of its low byte are the planes.  The bsums term
// of the reference's lanes is the -32 inside w.  Lane group lg of K-step ks
// takes the 16 values of part (n = ks / 2, j = 2 (ks % 2) + lg / 2) at bytes
// 16 (lg % 2) .. + 15: low (j < 2) or high nibbles of ql bytes 64 n +
// 32 (j % 2) + 16 (lg % 2) .., with bits 2j, 2j + 1 of qh bytes 32 n +
// 16 (lg % 2) ..; they are values 128 n + 32 j + 16 (lg % 2) .., one
// sub-block, i.e. the Q8_K bytes 64 ks + 16 lg .. (as the A operand reads
// them).  Weights are staged per row as the 53 dwords from the 4-byte
// boundary below the row's 2-byte-aligned block (realigned on read).
constexpr int BW6_STRIDE = 53;

__device__ __forceinline__ void q6_split_signed(uint32_t v2, int sc, uint32_t& lo, uint32_t& hi) {
    const s16x2 s2 = {(short)sc, (short)sc};
    const s16x2 o2 = {(short)(64 * sc), (short)(64 * sc)};
    const uint32_t a = __builtin_bit_cast(
        uint32_t, __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v2, 0x0c010c00u)) * s2 - o2);
    const uint32_t b = __builtin_bit_cast(
        uint32_t, __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v2, 0x0c030c02u)) * s2 - o2);
    lo = (__builtin_amdgcn_perm(b, a, 0x06040200u) >> 1) & 0x7f7f7f7fu;
    hi = __builtin_amdgcn_perm(b, a, 0x07050301u);
}

__global__ __launch_bounds__(BTHREADS) __attribute__((amdgpu_waves_per_eu(2)))
void q6k_gemm_blk(const unsigned char* __restrict__ w, const uint32_t* __restrict__ q8, float* __restrict__ y,
                  int n_in, int n_rows, int n_out, int tokens) {
#pragma clang fp contract(off)
    const int nb = n_in / QK;
    const int row0 = blockIdx.x * BR, tok0 = blockIdx.y * BT;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;

    __shared__ uint32_t wsh[2][BR * BW6_STRIDE];
    __shared__ uint4 xsh[2][BX_CHUNKS];

    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(w), 0, (int)((uint32_t)n_rows * nb * Q6K_BYTES), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(q8), 0, (int)((uint32_t)tokens * nb * Q8K_WORDS * 4), 0x00020000);
    uint32_t xvo[BX_RUNS];
    blk_x_offsets(xvo, tok0, tokens, nb, wave, lane);
    auto stage = [&](int b, int buf) {
        // rows wave, wave + 8, ...: one wave-wide load of 53 dwords each
#pragma unroll
        for (int i = 0; i < BR / BWAVES; ++i) {
            const int r = wave + BWAVES * i;
            const uint32_t so = (((uint32_t)min(row0 + r, n_rows - 1) * nb + b) * Q6K_BYTES) & ~3u;
            if (lane < BW6_STRIDE) dma_b32(wrs, &wsh[buf][BW6_STRIDE * r], 4u * lane, so);
        }
#pragma unroll
        for (int m = 0; m < BX_RUNS; ++m)
            if (64 * (wave + BWAVES * m) < BX_CHUNKS)
                dma_b128(xrs, &xsh[buf][64 * (wave + BWAVES * m)], xvo[m], (uint32_t)b * Q8K_WORDS * 4);
    };
    // Byte offset of the row's block in its staged dwords: 0 or 2, alternating with b.
    const int rpar = (min(row0 + 16 * wave + l16, n_rows - 1) * nb) & 1;

    float acc[BTILES][4];
#pragma unroll
    for (int tt = 0; tt < BTILES; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[tt][r] = 0.0f;

    const int h = lg & 1;
    stage(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const int buf = b & 1;
        if (b + 1 < nb) stage(b + 1, buf ^ 1);
        const uint32_t* wr = &wsh[buf][BW6_STRIDE * (16 * wave + l16)];
        const int shift = 2 * (rpar ^ (b & 1));
        const unsigned char* wb = reinterpret_cast<const unsigned char*>(wr) + shift;
        auto wd = [&](int f) { return __builtin_amdgcn_alignbyte(wr[f + 1], wr[f], shift); };
        const uint32_t* X = reinterpret_cast<const uint32_t*>(xsh[buf]);
        i32x4 dh[BTILES], dl[BTILES];
#pragma unroll
        for (int tt = 0; tt < BTILES; ++tt) dh[tt] = dl[tt] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int n = ks >> 1, j = 2 * (ks & 1) + (lg >> 1);
            const int sc = (int)(int8_t)wb[192 + 8 * n + 2 * j + h];
            // rotations: the nibble to bits 1-4, the qh bit pair to bits 5-6
            const uint32_t rq = (j >> 1) ? 3 : 31, rh = (uint32_t)(27 + 2 * j) & 31;
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ql = wd(16 * n + 8 * (j & 1) + 4 * h + i), qh = wd(32 + 8 * n + 4 * h + i);
                const uint32_t v2 = (__builtin_amdgcn_alignbit(ql, ql, rq) & 0x1e1e1e1eu) |
                                    (__builtin_amdgcn_alignbit(qh, qh, rh) & 0x60606060u);
                q6_split_signed(v2, sc, lo[i], hi[i]);
            }
            const i32x4 bh = {(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            const i32x4 bl = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
#pragma unroll
            for (int tt = 0; tt < BTILES; ++tt) {
                const i32x4 a = *reinterpret_cast<const i32x4*>(X + (16 * tt + l16) * BX_TOK_WORDS + Q8K_QS + 16 * ks + 4 * lg);
                dh[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bh, dh[tt], 0, 0, 0);
                dl[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bl, dl[tt], 0, 0, 0);
            }
        }
        const float dw = half_bits_to_float((uint32_t)wb[208] | ((uint32_t)wb[209] << 8));
#pragma unroll
        for (int tt = 0; tt < BTILES; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dxr = __builtin_bit_cast(float, X[(16 * tt + 4 * lg + r) * BX_TOK_WORDS]);
                const int isum = (int)((uint32_t)dh[tt][r] << 7) + dl[tt][r];
                acc[tt][r] = fmaf((float)isum, dw * dxr, acc[tt][r]);
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    const int row = row0 + 16 * wave + l16;
#pragma unroll
    for (int tt = 0; tt < BTILES; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tok0 + 16 * tt + 4 * lg + r;
            if (row < n_rows && t < tokens) y[(size_t)t * n_out + row] = acc[tt][r];
        }
}


// ---------------------------------------------------------------- layer boundary

// Ops.AddInPlace (Ops.cs:677-710) then Qwen35Ops.RmsNormZeroCentered
// (Qwen35Ops.cs:22-64), as Qwen35Model.DecodeBlock chains them around a mixer
// (Qwen35Model.Decode.cs:226-235); one wave per row of dim.  h = hidden +
// delta (fp32 adds, written back), staged in LDS; lanes 0-7 run the
// reference's 8 FMA lanes over the whole 8-element groups in order, then its
// horizontal sum and the dim % 8 tail one element at a time; scale = 1 /
// sqrt(sum / dim + eps) (IEEE); y = (h * scale) * (1 + w).  Q8: y is also
// written as Q8_K blocks (the Q8K.QuantizeRow of the projection that
// follows), formed from the same values.  y may alias hidden (the reference
// normalizes in place): every row is read into LDS before y is written.
template <bool ADD, bool Q8>
__global__ __launch_bounds__(kWave) void add_rmsnorm(float* hidden, const float* __restrict__ delta,
                                                     const float* __restrict__ w, float* y,
                                                     uint32_t* __restrict__ q8, int dim, float eps) {
#pragma clang fp contract(off)
    extern __shared__ float4 rowv[];
    const float* row = reinterpret_cast<const float*>(rowv);
    const int lane = threadIdx.x, t = blockIdx.x, n4 = dim >> 2;
    float4* h4 = reinterpret_cast<float4*>(hidden + (size_t)t * dim);
    for (int i = lane; i < n4; i += kWave) {
        float4 v = h4[i];
        if constexpr (ADD) {
            const float4 d = reinterpret_cast<const float4*>(delta + (size_t)t * dim)[i];
            v.x = v.x + d.x; v.y = v.y + d.y; v.z = v.z + d.z; v.w = v.w + d.w;
            h4[i] = v;
        }
        rowv[i] = v;
    }
    __syncthreads();
    // Q8: the first pass's weights are loaded before the sum of squares, each
    // later pass's during the one before.
    const int grp = lane >> 4, li = lane & 15, nbq = Q8 ? dim / QK : 0;
    float4 wn[4];
    auto load_w = [&](int p) {
        const int k4 = (min(p + grp, nbq - 1) * QK + 16 * li) >> 2;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            wn[i] = w ? reinterpret_cast<const float4*>(w)[k4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    if constexpr (Q8) load_w(0);
    float acc = 0.0f;
    // unrolled so the LDS reads run ahead of the (strictly ordered) FMA chain
    if (lane < 8)
#pragma unroll 32
        for (int j = 0; j < (dim >> 3); ++j) {
            const float x = row[8 * j + lane];
            acc = fmaf(x, x, acc);
        }
    float a[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) a[l] = __shfl(acc, l, kWave);
    float sum = hsum8(a);
    for (int i = dim & ~7; i < dim; ++i) {
        const float sq = row[i] * row[i];
        sum = sum + sq;
    }
    const float scale = 1.0f / sqrtf(sum / (float)dim + eps);
    if (!Q8 && y) {
        float4* y4 = reinterpret_cast<float4*>(y + (size_t)t * dim);
        for (int i = lane; i < n4; i += kWave) {
            const float4 v = rowv[i];
            const float4 g = w ? reinterpret_cast<const float4*>(w)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            y4[i] = make_float4((v.x * scale) * (1.0f + g.x), (v.y * scale) * (1.0f + g.y),
                                (v.z * scale) * (1.0f + g.z), (v.w * scale) * (1.0f + g.w));
        }
    }
    if constexpr (Q8) {
        const int nb = nbq;
        for (int p = 0; p < nb; p += 4) {
            const int b = p + grp, bb = min(b, nb - 1);
            // this lane's 16 values, as float4s; y written from here too
            const int k4 = (bb * QK + 16 * li) >> 2;
            float4 wc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) wc[i] = wn[i];
            if (p + 4 < nb) load_w(p + 4);
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 r = rowv[k4 + i];
                const float4 g = wc[i];
                v[4 * i] = (r.x * scale) * (1.0f + g.x);
                v[4 * i + 1] = (r.y * scale) * (1.0f + g.y);
                v[4 * i + 2] = (r.z * scale) * (1.0f + g.z);
                v[4 * i + 3] = (r.w * scale) * (1.0f + g.w);
            }
            if (y && b < nb) {
                float4* y4 = reinterpret_cast<float4*>(y + (size_t)t * dim) + k4;
#pragma unroll
                for (int i = 0; i < 4; ++i) y4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
            q8k_from16(v, lane, b < nb ? q8 + ((size_t)t * nb + b) * Q8K_WORDS : nullptr);
        }
    }
}

}  // namespace

hipError_t launch_q8k_quantize(q35m_ctx* c, const float* x, void* q8, int n_in, int tokens) {
    const int nb = n_in / QK;
    ProfScope ps_(c, K_Q8K_QUANTIZE);
    hipExtLaunchKernelGGL(q8k_quantize, dim3((nb + 3) / 4, tokens), dim3(kWave), 0, c->stream, ps_.a, ps_.b, 0,
                          x, reinterpret_cast<uint32_t*>(q8), nb);
    return hipGetLastError();
}

hipError_t launch_linear_q_prequant(q35m_ctx* c, int qtype, const void* w, const void* q8, float* y,
                                    int n_in, int n_out, int tokens) {
    const int nb = n_in / QK;
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(w);
    const uint32_t* qb = reinterpret_cast<const uint32_t*>(q8);
    if (qtype == 1 || qtype == 2) {
        // Which rows take the eight-row panel order (MulMatQ2.cs:25-40,
        // MulMatSTQ.cs:25-64): the first n_out & ~7, except STQ1_0 with
        // several tokens: all rows when tokens % 4 == 0 and n_out % 8 == 0,
        // else none.
        int panel_rows = n_out & ~7;
        if (qtype == 1 && tokens > 1) panel_rows = ((tokens & 3) == 0 && (n_out & 7) == 0) ? n_out : 0;
        const int rows_per_wg = min(LQ_THREADS / nb, LQ_MAX_ROWS);
        const int tok_per_wg = 8;
        const int ub = qtype == 2 ? Q2_BYTES / 2 : STQ_BYTES;
        const int nchunk_max = (rows_per_wg * nb * ub + 31) / 16 + 1;
        const dim3 grid((n_out + rows_per_wg - 1) / rows_per_wg, (tokens + tok_per_wg - 1) / tok_per_wg);
        const size_t lds = 16 * (size_t)nchunk_max + (size_t)nb * Q8K_WORDS * 4 + (size_t)LQ_THREADS * 4;
        ProfScope ps_(c, qtype == 2 ? K_Q2_0C_LINEAR : K_STQ1_0_LINEAR);
        if (qtype == 2)
            hipExtLaunchKernelGGL(linear_qt<2>, grid, dim3(LQ_THREADS), lds, c->stream, ps_.a, ps_.b, 0, wb, qb, y,
                                  n_in, n_out, tokens, rows_per_wg, tok_per_wg, panel_rows);
        else
            hipExtLaunchKernelGGL(linear_qt<1>, grid, dim3(LQ_THREADS), lds, c->stream, ps_.a, ps_.b, 0, wb, qb, y,
                                  n_in, n_out, tokens, rows_per_wg, tok_per_wg, panel_rows);
        return hipGetLastError();
    }
    if (qtype == 5 || qtype == 14) {
        // Per-token GEMV; up to 8 tokens a workgroup (the weights stay in
        // registers across them), more tokens over the grid's second axis.
        const int rows_per_wg = min(LQ_THREADS / nb, LQ_MAX_ROWS);
        const int tok_per_wg = 8;
        const dim3 grid((n_out + rows_per_wg - 1) / rows_per_wg, (tokens + tok_per_wg - 1) / tok_per_wg);
        const size_t lds = (size_t)nb * Q8K_WORDS * 4 + (size_t)LQ_THREADS * QS_TLD * 4;
        ProfScope ps_(c, qtype == 5 ? K_Q5K_LINEAR : K_IQ4XS_LINEAR);
        if (qtype == 5)
            hipExtLaunchKernelGGL(linear_qs<5>, grid, dim3(LQ_THREADS), lds, c->stream, ps_.a, ps_.b, 0, wb, qb, y,
                                  n_in, n_out, tokens, rows_per_wg, tok_per_wg);
        else
            hipExtLaunchKernelGGL(linear_qs<14>, grid, dim3(LQ_THREADS), lds, c->stream, ps_.a, ps_.b, 0, wb, qb, y,
                                  n_in, n_out, tokens, rows_per_wg, tok_per_wg);
        return hipGetLastError();
    }
    // The tiled kernels address their operands through buffer descriptors
    // (32-bit offsets): calls with more than 2 GiB of weight rows or of
    // activations go in pieces of whole row and token tiles (even rows), each
    // piece's per-row, per-token arithmetic unchanged.
    auto tiled = [&](auto kern, int kid, int bb, int gr, int gt, int threads, int n_rows) {
        const size_t lim = c->tile_limit;
        const int rmax = (int)std::min<size_t>(n_rows, (lim - 1) / ((size_t)nb * bb) / gr * gr);
        const int tmax = (int)std::min<size_t>(tokens, (lim - 1) / ((size_t)nb * Q8K_WORDS * 4) / gt * gt);
        if (rmax <= 0 || tmax <= 0) return hipErrorInvalidValue;   // one tile over the limit (n_in > 28M)
        for (int r0 = 0; r0 < n_rows; r0 += rmax)
            for (int t0 = 0; t0 < tokens; t0 += tmax) {
                const int nr = std::min(rmax, n_rows - r0), nt = std::min(tmax, tokens - t0);
                ProfScope ps_(c, kid);
                hipExtLaunchKernelGGL(kern, dim3((nr + gr - 1) / gr, (nt + gt - 1) / gt), dim3(threads), 0, c->stream,
                                      ps_.a, ps_.b, 0, wb + (size_t)r0 * nb * bb,
                                      qb + (size_t)t0 * nb * Q8K_WORDS, y + (size_t)t0 * n_out + r0, n_in, nr,
                                      n_out, nt);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
            }
        return hipSuccess;
    };
    // Q4_K with several tokens: the panel order for the first n_out & ~7 rows
    // (the reference's MulMatQ4K.Gemm), the GEMV for the rest.
    const int row_base = (qtype == 4 && tokens > 1) ? (n_out & ~7) : 0;
    if (row_base > 0) {
        const hipError_t e = tiled(q4k_gemm, K_Q4K_GEMM, Q4K_BYTES, GR, GT, GTHREADS, row_base);
        if (e != hipSuccess || row_base == n_out) return e;
    }
    // Q6_K: the tiled kernel from 16 tokens when n_out * n_in / 256 is even
    // (see q6k_gemm), the per-token GEMV otherwise; both keep the same
    // per-token arithmetic, so the results are identical.
    if (qtype == 6 && tokens >= 16 && (((size_t)n_out * nb) & 1) == 0) {
        if (c->proj_order == Q35M_PROJ_BLOCK)
            return tiled(q6k_gemm_blk, K_Q6K_GEMM_BLK, Q6K_BYTES, BR, BT, BTHREADS, n_out);
        return tiled(q6k_gemm, K_Q6K_GEMM, Q6K_BYTES, SGR, SGT, 256, n_out);
    }
    const int rows_per_wg = min(LQ_THREADS / nb, LQ_MAX_ROWS);
    const int grid = (n_out - row_base + rows_per_wg - 1) / rows_per_wg;
    const int bb = qtype == 4 ? Q4K_BYTES : Q6K_BYTES;
    const size_t lds = 16 * (size_t)lq_wchunks(qtype, rows_per_wg, nb, bb) + (size_t)nb * Q8K_WORDS * 4 +
                       (size_t)LQ_THREADS * LANES_LD * 4 + (size_t)LQ_MAX_ROWS * 12 * 4;
    auto launch = [&](auto kern, int kid) {
        ProfScope ps_(c, kid);
        hipExtLaunchKernelGGL(kern, dim3(grid), dim3(LQ_THREADS), lds, c->stream, ps_.a, ps_.b, 0, wb, qb, y,
                              n_in, n_out, tokens, rows_per_wg, row_base);
    };
    if (qtype == 4)
        launch(nb == 10 ? linear_q<4, 10> : nb == 16 ? linear_q<4, 16> : linear_q<4, 0>, K_Q4K_LINEAR);
    else
        launch(nb == 10 ? linear_q<6, 10> : nb == 16 ? linear_q<6, 16> : linear_q<6, 0>, K_Q6K_LINEAR);
    return hipGetLastError();
}

hipError_t launch_linear_q(q35m_ctx* c, int qtype, const void* w, const float* x, float* y,
                           int n_in, int n_out, int tokens) {
    hipError_t e = launch_q8k_quantize(c, x, c->work, n_in, tokens);
    if (e != hipSuccess) return e;
    return launch_linear_q_prequant(c, qtype, w, c->work, y, n_in, n_out, tokens);
}

hipError_t launch_add_rmsnorm(q35m_ctx* c, float* hidden, const float* delta, const float* w, float* y, void* q8,
                              int dim, int tokens, float eps) {
    ProfScope ps_(c, K_ADD_RMSNORM);
    uint32_t* qb = reinterpret_cast<uint32_t*>(q8);
    const size_t lds = (size_t)dim * sizeof(float);
    auto go = [&](auto kern) {
        hipExtLaunchKernelGGL(kern, dim3(tokens), dim3(kWave), lds, c->stream, ps_.a, ps_.b, 0, hidden, delta, w, y,
                              qb, dim, eps);
    };
    if (delta) q8 ? go(add_rmsnorm<true, true>) : go(add_rmsnorm<true, false>);
    else q8 ? go(add_rmsnorm<false, true>) : go(add_rmsnorm<false, false>);
    return hipGetLastError();
}

hipError_t launch_linear_f32(q35m_ctx* c, const float* w, const float* x, float* y, int n_in, int n_out,
                             int tokens) {
    const bool vec = n_in % 4 == 0 && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15) == 0;
    const dim3 grid((n_out + 63) / 64, tokens);
    ProfScope ps_(c, K_F32_LINEAR);
    if (vec)
        hipExtLaunchKernelGGL(linear_f32<true>, grid, dim3(256), 0, c->stream, ps_.a, ps_.b, 0, w, x, y, n_in, n_out);
    else
        hipExtLaunchKernelGGL(linear_f32<false>, grid, dim3(256), 0, c->stream, ps_.a, ps_.b, 0, w, x, y, n_in, n_out);
    return hipGetLastError();
}

size_t linear_q_work_bytes(int n_in, int tokens) {
    return (size_t)tokens * (n_in / QK) * Q8K_WORDS * 4;
}

}  // namespace q35
