/*
 * q35_oracle_quant.c -- CPU restatement of the reference's quantized
 * projections on the decode path: Q8_K activation quantization and the
 * Q4_K x Q8_K and Q6_K x Q8_K dot products behind Qwen35Model.DecodeLinear
 * (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:56-88).
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle).  The product library never
 * links or calls this file.
 *
 * The reference requires AVX2+FMA and runs its AVX2 paths, so those are the
 * ones restated: the integer sums are exact in any order, and the fp32
 * accumulation keeps the reference's 8 lanes (lane k of a 32-byte group holds
 * bytes 4k..4k+3, as _mm256_madd_epi16 leaves them), its FMA and its
 * horizontal-sum order.  Compiled with -ffp-contract=off; fmaf() only where
 * the C# calls Fma.MultiplyAdd.
 *
 * Q5_K and IQ4_XS have scalar paths only in the reference (Q5K.Dot,
 * IQ4XS.Dot): exact integer sums per block or 32-value sub-block, then one
 * short fp32 chain per block in block order with no fused multiply-add, which
 * is restated as written.
 *
 * Q2_0C and STQ1_0 have two fp32 orders in the reference: the eight-row panel
 * kernels (Q2Panel.cs, STQPanel.cs), one FMA per 256-value Q8_K block of an
 * exact integer dot, and the raw-row dot of the remaining rows (Q2_0C.DotAvx2,
 * STQ1_0.DotAvx2), plain multiplies and adds.  Which rows take which order is
 * MulMatQ2 / MulMatSTQ's dispatch, restated in q35o_linear_q.
 *
 * Block formats (src/Qwen35Sharp.Kernels/BlockLayout.cs:32-78), packed:
 *   Q4_K (144 B): u16 d, u16 dmin (fp16), u8 scales[12], u8 qs[128]
 *   Q5_K (176 B): u16 d, u16 dmin (fp16), u8 scales[12], u8 qh[32], u8 qs[128]
 *   Q6_K (210 B): u8 ql[128], u8 qh[64], i8 scales[16], u16 d (fp16)
 *   IQ4_XS (136 B): u16 d (fp16), u16 scales_h, u8 scales_l[4], u8 qs[128]
 *   Q2_0C (130 B, 512 values): u16 d (fp16), u8 qs[128] (4 codes a byte)
 *   STQ1_0 (42 B): u8 qs[32] (4-bit slots), u8 sign[8], u16 d (fp16)
 *   Q8_K (292 B): f32 d, i8 qs[256], i16 bsums[16]
 */
#include "q35_oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

#define QK 256

typedef struct __attribute__((packed)) {
    uint16_t d, dmin;
    uint8_t scales[12];
    uint8_t qs[QK / 2];
} blk_q4k;

typedef struct __attribute__((packed)) {
    uint8_t ql[QK / 2];
    uint8_t qh[QK / 4];
    int8_t scales[QK / 16];
    uint16_t d;
} blk_q6k;

typedef struct __attribute__((packed)) {
    uint16_t d, dmin;
    uint8_t scales[12];
    uint8_t qh[QK / 8];
    uint8_t qs[QK / 2];
} blk_q5k;

typedef struct __attribute__((packed)) {
    uint16_t d, scales_h;
    uint8_t scales_l[QK / 64];
    uint8_t qs[QK / 2];
} blk_iq4xs;

typedef struct __attribute__((packed)) {
    uint16_t d;
    uint8_t qs[128];
} blk_q2_0c;

typedef struct __attribute__((packed)) {
    uint8_t qs[32];
    uint8_t sign[8];
    uint16_t d;
} blk_stq1_0;

typedef struct __attribute__((packed)) {
    float d;
    int8_t qs[QK];
    int16_t bsums[QK / 16];
} blk_q8k;

_Static_assert(sizeof(blk_q4k) == 144, "Q4_K block");
_Static_assert(sizeof(blk_q6k) == 210, "Q6_K block");
_Static_assert(sizeof(blk_q5k) == 176, "Q5_K block");
_Static_assert(sizeof(blk_iq4xs) == 136, "IQ4_XS block");
_Static_assert(sizeof(blk_q8k) == 292, "Q8_K block");

/* HalfBits.ToSingle (BlockLayout.cs:155): the exact fp16 -> fp32 conversion
 * of .NET's Half, subnormals, infinities and NaNs included. */
float q35o_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t u;
    if (ex == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (ex != 0) {
        u = sign | ((ex + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        u = sign;
    } else {
        /* subnormal half: man * 2^-24, exact in fp32 */
        float f = (float)man * 5.9604644775390625e-8f;
        memcpy(&u, &f, 4);
        u |= sign;
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Q8K.ScaleBlock, src/Qwen35Sharp.Kernels/Q8K.cs:81-146 (AVX path): amax =
 * max |x|; the sign is that of the first element whose magnitude is amax;
 * iscale = -127 / max, delta = 1 / iscale.  Returns iscale (0 for an
 * all-zero block, with delta = 0). */
static float q8k_scale_block(const float* src, float* delta) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) {
        const float a = fabsf(src[j]);
        amax = a > amax ? a : amax;  /* _mm256_max_ps(vacc, |x|) keeps vacc on ties */
    }
    if (amax == 0.0f) {
        *delta = 0.0f;
        return 0.0f;
    }
    float max = amax;
    for (int j = 0; j < QK; j++) {
        if (src[j] == amax) { max = amax; break; }
        if (src[j] == -amax) { max = -amax; break; }
    }
    const float iscale = -127.0f / max;
    *delta = 1.0f / iscale;
    return iscale;
}

/* Q8K.QuantizeRow, src/Qwen35Sharp.Kernels/Q8K.cs:12-78 (AVX path):
 * q = clamp(round_half_even(x * iscale), -127, 127), bsums = sums of 16. */
void q35o_q8k_quantize_row(const float* x, void* out, int k) {
    blk_q8k* y = (blk_q8k*)out;
    const int nb = k / QK;
    for (int i = 0; i < nb; i++) {
        const float* src = x + (size_t)i * QK;
        float delta;
        const float iscale = q8k_scale_block(src, &delta);
        if (iscale == 0.0f) {
            memset(&y[i], 0, sizeof(blk_q8k));
            continue;
        }
        y[i].d = delta;
        for (int j = 0; j < QK; j++) {
            const float r = rintf(src[j] * iscale);  /* default mode: ties to even */
            int v = (int)r;
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            y[i].qs[j] = (int8_t)v;
        }
        for (int j = 0; j < QK / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
    }
}

/* Q4K.UnpackScales, src/Qwen35Sharp.Kernels/Q4K.cs:20-33: 8 six-bit scales
 * (bytes 0..7) and 8 six-bit mins (bytes 8..15). */
static void q4k_unpack_scales(const uint8_t* packed, uint8_t out[16]) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    uint32_t u[4];
    memcpy(&u[0], packed, 4);
    memcpy(&u[1], packed + 4, 4);
    memcpy(&u[2], packed + 8, 4);
    u[3] = ((u[2] >> 4) & kmask2) | (((u[1] >> 6) & kmask3) << 4);
    const uint32_t uaux = u[1] & kmask1;
    u[1] = (u[2] & kmask2) | (((u[0] >> 6) & kmask3) << 4);
    u[2] = uaux;
    u[0] &= kmask1;
    memcpy(out, u, 16);
}

/* VecDotQ4K.HorizontalSum, src/Qwen35Sharp.Kernels/VecDotQ4K.cs:145-151. */
static float hsum8(const float a[8]) {
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    const float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* VecDotQ4K.DotAvx2, src/Qwen35Sharp.Kernels/VecDotQ4K.cs:67-126. */
float q35o_q4k_dot(const void* wx, const void* wy, int n) {
    const blk_q4k* x = (const blk_q4k*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    const int nb = n / QK;
    float acc[8] = {0}, acc_min[4] = {0};
    for (int i = 0; i < nb; i++) {
        const float d = y[i].d * q35o_half_to_float(x[i].d);
        const float dmin = -y[i].d * q35o_half_to_float(x[i].dmin);
        uint8_t sm[16];
        q4k_unpack_scales(x[i].scales, sm);
        /* mins . (pairwise bsums): _mm_madd_epi16(mins, hadd(bsums lo, bsums hi)) */
        int32_t prod[4];
        for (int k = 0; k < 4; k++) {
            const int s0 = (int16_t)(y[i].bsums[4 * k] + y[i].bsums[4 * k + 1]);
            const int s1 = (int16_t)(y[i].bsums[4 * k + 2] + y[i].bsums[4 * k + 3]);
            prod[k] = sm[8 + 2 * k] * s0 + sm[8 + 2 * k + 1] * s1;
        }
        for (int k = 0; k < 4; k++) acc_min[k] = acc_min[k] + dmin * (float)prod[k];
        /* sumi lane k: bytes 4k..4k+3 of every 32-byte group */
        int32_t sumi[8] = {0};
        const uint8_t* q4 = x[i].qs;
        const int8_t* q8 = y[i].qs;
        for (int j = 0; j < QK / 64; j++) {
            const int sl = sm[2 * j], sh = sm[2 * j + 1];
            for (int k = 0; k < 8; k++) {
                int pl = 0, ph = 0;
                for (int b = 4 * k; b < 4 * k + 4; b++) {
                    pl += (q4[b] & 0xf) * q8[b];
                    ph += (q4[b] >> 4) * q8[32 + b];
                }
                sumi[k] += pl * sl + ph * sh;
            }
            q4 += 32;
            q8 += 64;
        }
        for (int k = 0; k < 8; k++) acc[k] = fmaf((float)sumi[k], d, acc[k]);
    }
    /* accMin: + MoveHighToLow, then lane 0 + lane 1 */
    const float m = (acc_min[0] + acc_min[2]) + (acc_min[1] + acc_min[3]);
    return hsum8(acc) + m;
}

/* Q6K.DotAvx2, src/Qwen35Sharp.Kernels/Q6K.cs:87-165. */
float q35o_q6k_dot(const void* wx, const void* wy, int n) {
    const blk_q6k* x = (const blk_q6k*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    const int nb = n / QK;
    float acc[8] = {0};
    for (int i = 0; i < nb; i++) {
        const float d = y[i].d * q35o_half_to_float(x[i].d);
        int32_t sumi[8] = {0};
        const uint8_t* ql = x[i].ql;
        const uint8_t* qh = x[i].qh;
        const int8_t* q8 = y[i].qs;
        for (int j = 0; j < QK / 128; j++) {
            for (int b = 0; b < 32; b++) {
                const int h = qh[b];
                const int v[4] = {(ql[b] & 15) | ((h & 3) << 4), (ql[32 + b] & 15) | ((h & 12) << 2),
                                  (ql[b] >> 4) | (h & 48), (ql[32 + b] >> 4) | ((h & 0xc0) >> 2)};
                const int k = b / 4, half = b / 16;
                for (int m = 0; m < 4; m++)
                    sumi[k] += x[i].scales[8 * j + 2 * m + half] * (v[m] * q8[32 * m + b]);
            }
            ql += 64;
            qh += 32;
            q8 += 128;
        }
        /* minus 32 * (bsums . scales), pairwise per lane */
        for (int k = 0; k < 8; k++)
            sumi[k] -= (y[i].bsums[2 * k] * x[i].scales[2 * k] +
                        y[i].bsums[2 * k + 1] * x[i].scales[2 * k + 1]) * 32;
        for (int k = 0; k < 8; k++) acc[k] = fmaf(d, (float)sumi[k], acc[k]);
    }
    return hsum8(acc);
}

/* Q4K.DequantizeRow, src/Qwen35Sharp.Kernels/Q4K.cs:35-59. */
void q35o_q4k_dequantize_row(const void* wx, float* y, int k) {
    const blk_q4k* x = (const blk_q4k*)wx;
    for (int i = 0; i < k / QK; i++) {
        uint8_t sm[16];
        q4k_unpack_scales(x[i].scales, sm);
        const float d = q35o_half_to_float(x[i].d), mn = q35o_half_to_float(x[i].dmin);
        const uint8_t* q = x[i].qs;
        for (int j = 0; j < QK / 64; j++) {
            const float d1 = d * sm[2 * j], m1 = mn * sm[8 + 2 * j];
            const float d2 = d * sm[2 * j + 1], m2 = mn * sm[8 + 2 * j + 1];
            for (int l = 0; l < 32; l++) *y++ = d1 * (q[l] & 0xf) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
        }
    }
}

/* Q6K.DequantizeRow, src/Qwen35Sharp.Kernels/Q6K.cs:9-39. */
void q35o_q6k_dequantize_row(const void* wx, float* y, int k) {
    const blk_q6k* x = (const blk_q6k*)wx;
    for (int i = 0; i < k / QK; i++) {
        const float d = q35o_half_to_float(x[i].d);
        const uint8_t* ql = x[i].ql;
        const uint8_t* qh = x[i].qh;
        const int8_t* sc = x[i].scales;
        for (int n = 0; n < QK; n += 128) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = (ql[l] & 0xf) | ((qh[l] & 3) << 4);
                const int q2 = (ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4);
                const int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                const int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
                y[l] = d * sc[is] * (q1 - 32);
                y[l + 32] = d * sc[is + 2] * (q2 - 32);
                y[l + 64] = d * sc[is + 4] * (q3 - 32);
                y[l + 96] = d * sc[is + 6] * (q4 - 32);
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* Q5K.Dot, src/Qwen35Sharp.Kernels/Q5K.cs:45-95: per block, the 5-bit values
 * a = (nibble) + 16 * (high bit), acc = sum_j scale_j * (q8 . a over
 * sub-block j), sumi = sum_j bsums[j] * min[j / 2] (exact integers); then
 * sumf += d * acc - dmin * sumi with d = fp16(D) * dy, dmin = fp16(Dmin) * dy
 * (int -> float conversions, no fused multiply-add). */
float q35o_q5k_dot(const void* wx, const void* wy, int n) {
    const blk_q5k* x = (const blk_q5k*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    const int nb = n / QK;
    float sumf = 0.0f;
    for (int i = 0; i < nb; i++) {
        int8_t aux[QK];
        const uint8_t* q4 = x[i].qs;
        const uint8_t* hm = x[i].qh;
        int8_t* a = aux;
        uint8_t m = 1;
        for (int j = 0; j < QK / 64; j++) {
            for (int l = 0; l < 32; l++) a[l] = (int8_t)((q4[l] & 0xF) + ((hm[l] & m) != 0 ? 16 : 0));
            a += 32;
            m <<= 1;
            for (int l = 0; l < 32; l++) a[l] = (int8_t)((q4[l] >> 4) + ((hm[l] & m) != 0 ? 16 : 0));
            a += 32;
            m <<= 1;
            q4 += 32;
        }
        uint8_t sm[16];
        q4k_unpack_scales(x[i].scales, sm);
        int sumi = 0;
        for (int j = 0; j < QK / 16; j++) sumi += y[i].bsums[j] * sm[8 + j / 2];
        int acc = 0;
        for (int j = 0; j < QK / 32; j++) {
            const int scale = sm[j];
            for (int l = 0; l < 32; l++) acc += scale * y[i].qs[32 * j + l] * aux[32 * j + l];
        }
        const float d = q35o_half_to_float(x[i].d) * y[i].d;
        const float dmin = q35o_half_to_float(x[i].dmin) * y[i].d;
        sumf += d * acc - dmin * sumi;
    }
    return sumf;
}

/* Q5K.DequantizeRow, src/Qwen35Sharp.Kernels/Q5K.cs:5-43. */
void q35o_q5k_dequantize_row(const void* wx, float* y, int k) {
    const blk_q5k* x = (const blk_q5k*)wx;
    for (int i = 0; i < k / QK; i++) {
        const uint8_t* ql = x[i].qs;
        const uint8_t* qh = x[i].qh;
        const float d = q35o_half_to_float(x[i].d), mn = q35o_half_to_float(x[i].dmin);
        uint8_t sm[16];
        q4k_unpack_scales(x[i].scales, sm);
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0, is = 0; j < QK; j += 64, is += 2) {
            const float d1 = d * sm[is], m1 = mn * sm[8 + is];
            const float d2 = d * sm[is + 1], m2 = mn * sm[8 + is + 1];
            for (int l = 0; l < 32; l++) *y++ = d1 * ((ql[l] & 0xF) + ((qh[l] & u1) != 0 ? 16 : 0)) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * ((ql[l] >> 4) + ((qh[l] & u2) != 0 ? 16 : 0)) - m2;
            ql += 32;
            u1 <<= 2;
            u2 <<= 2;
        }
    }
}

/* IQ4XS.KValues, src/Qwen35Sharp.Kernels/IQ4XS.cs:15-18: the non-linear grid. */
static const int kvalues_iq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                    1,    13,   25,  38,  53,  69,  89,  113};

/* IQ4XS.SubBlockScale, IQ4XS.cs:20-26: ls from 4 low bits (scales_l) and 2
 * high bits (scales_h); dl = fp16(d) * (ls - 32). */
static float iq4xs_dl(const blk_iq4xs* x, int ib) {
    const int ls = ((x->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((x->scales_h >> (2 * ib)) & 3) << 4);
    return q35o_half_to_float(x->d) * (ls - 32);
}

/* IQ4XS.Dot, src/Qwen35Sharp.Kernels/IQ4XS.cs:49-73: per 32-value sub-block
 * the exact integer q8 . grid[idx] (low nibbles then high nibbles of 16
 * bytes), then sumf += dl * acc * d8 (left to right, no fused multiply-add),
 * sub-blocks in order. */
float q35o_iq4xs_dot(const void* wx, const void* wy, int n) {
    const blk_iq4xs* x = (const blk_iq4xs*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    const int nb = n / QK;
    float sumf = 0.0f;
    for (int i = 0; i < nb; i++) {
        const uint8_t* qs = x[i].qs;
        const float d8 = y[i].d;
        for (int ib = 0; ib < QK / 32; ib++) {
            const float dl = iq4xs_dl(&x[i], ib);
            const int8_t* q8 = y[i].qs + 32 * ib;
            int acc = 0;
            for (int j = 0; j < 16; j++) {
                acc += q8[j] * kvalues_iq4[qs[j] & 0xF];
                acc += q8[j + 16] * kvalues_iq4[qs[j] >> 4];
            }
            sumf += dl * acc * d8;
            qs += 16;
        }
    }
    return sumf;
}

/* IQ4XS.DequantizeRow, src/Qwen35Sharp.Kernels/IQ4XS.cs:28-47. */
void q35o_iq4xs_dequantize_row(const void* wx, float* y, int k) {
    const blk_iq4xs* x = (const blk_iq4xs*)wx;
    for (int i = 0; i < k / QK; i++) {
        const uint8_t* qs = x[i].qs;
        for (int ib = 0; ib < QK / 32; ib++) {
            const float dl = iq4xs_dl(&x[i], ib);
            for (int j = 0; j < 16; j++) {
                y[j] = dl * kvalues_iq4[qs[j] & 0xF];
                y[j + 16] = dl * kvalues_iq4[qs[j] >> 4];
            }
            qs += 16;
            y += 32;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Q2_0C                                                                     */
/* ------------------------------------------------------------------------- */

/* Q2_0C.Value (src/Qwen35Sharp.Kernels/Q2_0C.cs:12-13): value j of a block is
 * 2 * code - 3 with code = (qs[j / 4] >> (2 (j % 4))) & 3. */
static int q2_value(const blk_q2_0c* x, int j) {
    return ((x->qs[j / 4] >> ((j & 3) * 2)) & 3) * 2 - 3;
}

/* Exact integer dot of half h (values 256 h .. 256 h + 255) with a Q8_K block. */
static int q2_half_dot(const blk_q2_0c* x, int h, const blk_q8k* y) {
    int s = 0;
    for (int j = 0; j < QK; j++) s += q2_value(x, QK * h + j) * y->qs[j];
    return s;
}

/* Q2_0C.DotAvx2 (Q2_0C.cs:67-79), the raw-row dot: per 512-value block,
 * sum += d * ((float)s0 * y0.d + (float)s1 * y1.d) with s0, s1 the exact
 * integer dots of the two halves against their Q8_K blocks (Dot256's int16
 * lanes hold at most 8 * 768 and never saturate). */
float q35o_q2_0c_dot(const void* wx, const void* wy, int n) {
    const blk_q2_0c* x = (const blk_q2_0c*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    float sum = 0.0f;
    for (int b = 0; b < n / 512; b++) {
        const int s0 = q2_half_dot(&x[b], 0, &y[2 * b]);
        const int s1 = q2_half_dot(&x[b], 1, &y[2 * b + 1]);
        sum += q35o_half_to_float(x[b].d) * ((float)s0 * y[2 * b].d + (float)s1 * y[2 * b + 1].d);
    }
    return sum;
}

/* Q2Panel.Gemv / Gemm (src/Qwen35Sharp.Kernels/Q2Panel.cs:12-46, 48-176) for
 * one output of an eight-row panel: per 256-value Q8_K block b, acc =
 * fma((float)(2 I - 3 S), dw * y[b].d, acc) with I = sum code * q8 (the
 * codes 0..3, exact in the int16 lanes: at most 64 * 3 * 128 each), S = the
 * block's bsums total and dw the weight block's scale (the panel holds it as
 * float, RepackQ2.cs:15).  2 I - 3 S equals the half's signed dot exactly. */
static float q2_panel_dot(const blk_q2_0c* x, const blk_q8k* y, int n) {
    float acc = 0.0f;
    for (int b = 0; b < n / QK; b++) {
        const blk_q2_0c* xb = &x[b / 2];
        int dot = 0, sum = 0;
        for (int j = 0; j < QK; j++)
            dot += ((xb->qs[(QK * (b & 1) + j) / 4] >> ((j & 3) * 2)) & 3) * y[b].qs[j];
        for (int g = 0; g < QK / 16; g++) sum += y[b].bsums[g];
        acc = fmaf((float)(2 * dot - 3 * sum), q35o_half_to_float(xb->d) * y[b].d, acc);
    }
    return acc;
}

/* Q2_0C.DequantizeRow (Q2_0C.cs:15-23). */
void q35o_q2_0c_dequantize_row(const void* wx, float* y, int k) {
    const blk_q2_0c* x = (const blk_q2_0c*)wx;
    for (int b = 0; b < k / 512; b++) {
        const float d = q35o_half_to_float(x[b].d);
        for (int j = 0; j < 512; j++) y[512 * b + j] = (float)q2_value(&x[b], j) * d;
    }
}

/* ------------------------------------------------------------------------- */
/* STQ1_0                                                                    */
/* ------------------------------------------------------------------------- */

/* STQ1_0.Codebook (src/Qwen35Sharp.Kernels/STQ1_0.cs:50-56): the four-lane
 * ternary pattern of slot s with sign bit g is entry 16 g + s, two bits a lane
 * (0 = -1, 1 = 0, 2 = +1). */
static const uint8_t stq_codebook[32] = {
    0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
    0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68,
};

/* STQ1_0.QPack (STQ1_0.cs:58-63): group g's slot is nibble g % 2 of qs[g / 2],
 * its sign bit g % 8 of sign[g / 8]. */
static uint8_t stq_qpack(const blk_stq1_0* x, int g) {
    const int slot = (x->qs[g >> 1] >> ((g & 1) * 4)) & 0x0F;
    const int sign = (x->sign[g >> 3] >> (g & 7)) & 1;
    return stq_codebook[(sign << 4) | slot];
}

/* Exact encoded dot of one block: sum of the 0/1/2 lane codes times q8, value
 * index chunk * 64 + gloc + 16 * lane for group 16 chunk + gloc
 * (STQ1_0.DotChunk16, STQ1_0.cs:146-188; STQ1_0.Code, :68-75). */
static int stq_encoded_dot(const blk_stq1_0* x, const blk_q8k* y) {
    int e = 0;
    for (int g = 0; g < 64; g++) {
        const uint8_t q = stq_qpack(x, g);
        const int chunk = g >> 4, gloc = g & 15;
        for (int lane = 0; lane < 4; lane++)
            e += ((q >> (2 * lane)) & 3) * y->qs[chunk * 64 + gloc + lane * 16];
    }
    return e;
}

static int q8k_total(const blk_q8k* y) {
    int s = 0;
    for (int g = 0; g < QK / 16; g++) s += y->bsums[g];
    return s;
}

/* STQ1_0.DotAvx2 (STQ1_0.cs:120-138), the raw-row dot: per block, sum +=
 * d * y.d * (encoded - activationSum), evaluated left to right ((d * y.d)
 * times the float of the exact ternary dot).  DotScalar (:98-117) gives the
 * same value. */
float q35o_stq1_0_dot(const void* wx, const void* wy, int n) {
    const blk_stq1_0* x = (const blk_stq1_0*)wx;
    const blk_q8k* y = (const blk_q8k*)wy;
    float sum = 0.0f;
    for (int b = 0; b < n / QK; b++) {
        const int t = stq_encoded_dot(&x[b], &y[b]) - q8k_total(&y[b]);
        sum += q35o_half_to_float(x[b].d) * y[b].d * (float)t;
    }
    return sum;
}

/* STQPanel.Gemv / Gemm (src/Qwen35Sharp.Kernels/STQPanel.cs:13-48, 50-191) for
 * one output of an eight-row panel: per block, acc = fma((float)(encoded -
 * S), dw * y.d, acc). */
static float stq_panel_dot(const blk_stq1_0* x, const blk_q8k* y, int n) {
    float acc = 0.0f;
    for (int b = 0; b < n / QK; b++) {
        const int t = stq_encoded_dot(&x[b], &y[b]) - q8k_total(&y[b]);
        acc = fmaf((float)t, q35o_half_to_float(x[b].d) * y[b].d, acc);
    }
    return acc;
}

/* STQ1_0.DequantizeRow (STQ1_0.cs:77-94). */
void q35o_stq1_0_dequantize_row(const void* wx, float* y, int k) {
    const blk_stq1_0* x = (const blk_stq1_0*)wx;
    for (int b = 0; b < k / QK; b++) {
        const float d = q35o_half_to_float(x[b].d);
        for (int g = 0; g < 64; g++) {
            const uint8_t q = stq_qpack(&x[b], g);
            for (int lane = 0; lane < 4; lane++)
                y[QK * b + (g >> 4) * 64 + (g & 15) + lane * 16] = (float)(((q >> (2 * lane)) & 3) - 1) * d;
        }
    }
}

/* GemmQ4K.GemmAvx2Tile (src/Qwen35Sharp.Kernels/GemmQ4K.Avx2.cs:39-207), the
 * reference's Q4_K path for more than one token (MulMatQ4K.Gemm,
 * MulMatQ4K.cs:45-127, over the x8 panels and the BlockQ4Kx8Meta sidecar of
 * RepackQ4K.BuildMeta, RepackQ4K.cs:90-129), for one (token, output) pair:
 * per block b and 32-value sub-block s in order, acc = fma((float)(sc * dot),
 * dw * dx, acc) with dot the exact integer q4 . q8 of the sub-block (its
 * int16 partials never overflow: at most 8 * 15 * 127 each); per block,
 * mn = fma((float)(sum_j min_j * (bsums[2j] + bsums[2j+1])), dminw * dx, mn);
 * the result is acc - mn.  Quantize4x8 gives the same int8 values and scales
 * as Q8K.QuantizeRow (same ScaleBlock and rounding), so q8 is the row's Q8_K
 * blocks. */
static float q4k_panel_dot(const blk_q4k* x, const blk_q8k* y, int n) {
    const int nb = n / QK;
    float acc = 0.0f, mn = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float cs = q35o_half_to_float(x[i].d) * y[i].d;
        const float cm = q35o_half_to_float(x[i].dmin) * y[i].d;
        uint8_t sm[16];
        q4k_unpack_scales(x[i].scales, sm);
        for (int s = 0; s < 8; s++) {
            const int g = s / 2, hi = s % 2;
            int dot = 0;
            for (int l = 0; l < 32; l++) {
                const int q = hi ? (x[i].qs[32 * g + l] >> 4) : (x[i].qs[32 * g + l] & 0xf);
                dot += q * y[i].qs[64 * g + 32 * hi + l];
            }
            acc = fmaf((float)(sm[s] * dot), cs, acc);
        }
        int m = 0;
        for (int j = 0; j < 8; j++) m += sm[8 + j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        mn = fmaf((float)m, cm, mn);
    }
    return acc - mn;
}

/* Qwen35Model.Linear for quantized weights (Qwen35Model.Decode.cs:22-51):
 * MulMatQ4K.Gemv / Gemm (src/Qwen35Sharp.Kernels/MulMatQ4K.cs:12-127),
 * Q6K.Gemv / Gemm (src/Qwen35Sharp.Kernels/Q6K.cs:301-413), Q5K.Gemv / Gemm
 * (Q5K.cs:97-117), IQ4XS.Gemv / Gemm (IQ4XS.cs:75-104), MulMatQ2.Gemv / Gemm
 * (MulMatQ2.cs:19-99) and MulMatSTQ.Gemv / Gemm (MulMatSTQ.cs:19-150): each
 * token row is quantized to Q8_K, then every output is one dot product in the
 * order of the path that computes it (panel orders above for the rows listed
 * below; Q5_K and IQ4_XS run their GEMV per token).  (Q6K.Gemm's four-token
 * DotAvx2x4 gives the same value per token as DotAvx2: the same integer lanes
 * and the same fma per block; Quantize4x8 gives the same values as
 * Q8K.QuantizeRow.)  type 1 = STQ1_0, 2 = Q2_0C (n_in a multiple of 512),
 * 4 = Q4_K, 5 = Q5_K, 6 = Q6_K, 14 = IQ4_XS. */
void q35o_linear_q(int type, const void* w, const float* x, float* y, int n_in, int n_out,
                   int tokens) {
    const int nb = n_in / QK;
    const size_t bsz = type == 4 ? sizeof(blk_q4k) : type == 5 ? sizeof(blk_q5k)
                     : type == 6 ? sizeof(blk_q6k) : type == 14 ? sizeof(blk_iq4xs)
                     : type == 1 ? sizeof(blk_stq1_0) : sizeof(blk_q2_0c);
    const size_t wrow = type == 2 ? (size_t)(n_in / 512) * bsz : (size_t)nb * bsz;
    /* Rows in a panel order:
     * - Q4_K with more than one token: the panel GEMM for the first n_out & ~7
     *   outputs (MulMatQ4K.cs:104-123 sends the rest through VecDotQ4K.Dot);
     * - Q2_0C: the panels (built for the first n_out & ~7 rows when
     *   n_out >= 8, Qwen35Model.cs:531-539) for any token count, the raw dot
     *   for the rest (MulMatQ2.cs:25-40, 89-98; padding to four tokens does
     *   not change a token's values);
     * - STQ1_0: one token as Q2_0C (MulMatSTQ.cs:25-45); several tokens all
     *   rows by panel when tokens % 4 == 0 and n_out % 8 == 0, else all rows
     *   by the raw dot (MulMatSTQ.cs:47-64, 104-150). */
    int panel_rows = 0;
    if (type == 4 && tokens > 1) panel_rows = n_out & ~7;
    if (type == 2) panel_rows = n_out & ~7;
    if (type == 1)
        panel_rows = tokens == 1 ? (n_out & ~7) : ((tokens & 3) == 0 && (n_out & 7) == 0) ? n_out : 0;
    blk_q8k q8[64];
    if (nb > 64) return;
    for (int t = 0; t < tokens; t++) {
        q35o_q8k_quantize_row(x + (size_t)t * n_in, q8, n_in);
        for (int r = 0; r < n_out; r++) {
            const void* wr = (const uint8_t*)w + (size_t)r * wrow;
            float v;
            if (type == 2)
                v = r < panel_rows ? q2_panel_dot((const blk_q2_0c*)wr, q8, n_in) : q35o_q2_0c_dot(wr, q8, n_in);
            else if (type == 1)
                v = r < panel_rows ? stq_panel_dot((const blk_stq1_0*)wr, q8, n_in) : q35o_stq1_0_dot(wr, q8, n_in);
            else if (r < panel_rows)
                v = q4k_panel_dot((const blk_q4k*)wr, q8, n_in);
            else if (type == 4)
                v = q35o_q4k_dot(wr, q8, n_in);
            else if (type == 5)
                v = q35o_q5k_dot(wr, q8, n_in);
            else if (type == 6)
                v = q35o_q6k_dot(wr, q8, n_in);
            else
                v = q35o_iq4xs_dot(wr, q8, n_in);
            y[(size_t)t * n_out + r] = v;
        }
    }
}
