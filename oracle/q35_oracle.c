/*
 * q35_oracle.c -- CPU restatement of the Qwen35Sharp token-mixer ops.
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle and the CPU baseline).  The
 * product library never links or calls this file.
 *
 * Rules followed throughout:
 *  - fp32 arithmetic in the reference's loop order, compiled with
 *    -ffp-contract=off so that a*b+c is never fused behind our back (RyuJIT
 *    does not contract scalar code either).  fmaf() appears exactly where the
 *    C# calls Fma.MultiplyAdd / Fma.MultiplyAddNegated.
 *  - The AVX paths of the reference are the ones restated (the reference
 *    requires AVX2+FMA: tests/Qwen35Sharp.Tests/FastExpTests.cs:13).  An AVX
 *    8-lane accumulator is restated as an array of 8 floats reduced in the
 *    HorizontalSum order of src/Qwen35Sharp.Kernels/VecDotQ4K.cs:145-151.
 *  - MathF.Exp/Sqrt/Pow/Cos/Sin are taken to be glibc expf/sqrtf/powf/cosf/
 *    sinf (CoreCLR on Linux calls the platform libm).
 *
 * Paths cited below are relative to the reference repository root.
 */
#include "q35_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* lane helpers                                                              */
/* ------------------------------------------------------------------------- */

/* VecDotQ4K.HorizontalSum, src/Qwen35Sharp.Kernels/VecDotQ4K.cs:145-151:
 * lower+upper halves, then MoveHighToLow add, then lane0+lane1. */
static float hsum8(const float a[8]) {
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* Ops.HorizontalSum4, src/Qwen35Sharp.Model/Ops.cs:490-497: two hadd stages
 * then lower+upper, i.e. ((x0+x1)+(x2+x3)) + ((x4+x5)+(x6+x7)). */
static float hsum8_hadd(const float a[8]) {
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

/* Ops.HorizontalMax, src/Qwen35Sharp.Model/Ops.cs:268-275 (order-free). */
static float hmax8(const float a[8]) {
    float m = a[0];
    for (int l = 1; l < 8; l++) m = a[l] > m ? a[l] : m;
    return m;
}

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------------- */
/* scalar helpers                                                            */
/* ------------------------------------------------------------------------- */

/* GatedDeltaNetOps.Silu, src/Qwen35Sharp.Model/GatedDeltaNetOps.cs:18 */
float q35o_silu(float x) { return x / (1.0f + expf(-x)); }

/* Qwen35Ops.Log1pSafe, src/Qwen35Sharp.Model/Qwen35Ops.cs:133-142:
 * 4-term Taylor series on (-0.5, 0.5), log(1+x) elsewhere. */
float q35o_log1p_safe(float x) {
    if (x > -0.5f && x < 0.5f) {
        float x2 = x * x;
        return x - x2 / 2.0f + x2 * x / 3.0f - x2 * x2 / 4.0f;
    }
    return logf(1.0f + x);
}

/* Qwen35Ops.SoftplusScalar, src/Qwen35Sharp.Model/Qwen35Ops.cs:121-130 */
float q35o_softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -10.0f) return expf(x);
    float ex = expf(x);
    return q35o_log1p_safe(ex);
}

/* Qwen35Ops.Sigmoid, src/Qwen35Sharp.Model/Qwen35Ops.cs:114-118 */
void q35o_sigmoid(const float* x, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* FastExp.ExpAvx2, src/Qwen35Sharp.Kernels/FastExp.cs:14-45, one lane.
 * Range reduction x = n*ln2 + b with a two-constant ln2 split, a degree-5
 * polynomial for e^b - 1, and scaling by 2^n through the exponent field;
 * the |n| > 126 branch splits the scale factor to reach the subnormal and
 * overflow range. */
float q35o_fast_exp(float x) {
    const float r = 12582912.0f; /* 1.5 * 2^23: rounds to integer in the mantissa */
    float z = fmaf(x, 1.4426950216293335f, r);
    float n = z - r;
    float b = fmaf(-n, 1.4286067655086517e-6f, fmaf(-n, 0.693145751953125f, x));
    uint32_t e = float_to_bits(z) << 23;
    float k = bits_to_float(e + float_to_bits(1.0f));
    float n_abs = fabsf(n);
    int overflow = n_abs > 126.0f;
    float u = b * b;
    float j = fmaf(fmaf(fmaf(0.008301135152578354f, b, 0.04190601035952568f), u,
                        fmaf(0.166665181517601f, b, 0.4999998211860657f)),
                   u, 0.9999998211860657f * b);
    if (!overflow) return fmaf(j, k, k);
    uint32_t g = (n <= 0.0f) ? 0x82000000u : 0u;
    float s1 = bits_to_float(g + 0x7F000000u);
    float s2 = bits_to_float(e - g);
    int huge = n_abs > 192.0f;
    if (huge) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

void q35o_fast_exp_n(const float* x, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = q35o_fast_exp(x[i]);
}

/* ------------------------------------------------------------------------- */
/* Gated-DeltaNet ops                                                        */
/* ------------------------------------------------------------------------- */

/* GatedDeltaNetOps.CausalConv1d, src/Qwen35Sharp.Model/GatedDeltaNetOps.cs:27-53.
 * input/out [channels][seq]; kernel [kernel_size][channels]; tap j multiplies
 * x[t-j] (tap 0 = current token); zero left padding. */
void q35o_causal_conv1d(const float* input, const float* kernel, int kernel_size,
                        int channels, int seq, float* out) {
    for (int c = 0; c < channels; c++) {
        const float* in_ch = input + (long)c * seq;
        float* out_ch = out + (long)c * seq;
        const float* k_ch = kernel + c;
        for (int t = 0; t < seq; t++) {
            float acc = 0.0f;
            for (int j = 0; j < kernel_size; j++) {
                int prev = t - j;
                if (prev < 0) continue;
                acc += k_ch[(long)j * channels] * in_ch[prev];
            }
            out_ch[t] = q35o_silu(acc);
        }
    }
}

/* GatedDeltaNetOps.CausalConv1dUpdate, src/Qwen35Sharp.Model/GatedDeltaNetOps.cs:64-91.
 * conv_state [channels][kernel_size-1], index 0 = oldest; tap j < K-1
 * multiplies state[j], tap K-1 multiplies the new input. */
void q35o_causal_conv1d_update(const float* input, const float* kernel, int kernel_size,
                               int channels, float* conv_state, float* out) {
    int state_len = kernel_size - 1;
    for (int c = 0; c < channels; c++) {
        const float* k_ch = kernel + c;
        float* cs = conv_state + (long)c * state_len;
        int j = 0;
        float acc = 0.0f;
        for (; j < state_len; j++) acc += k_ch[(long)j * channels] * cs[j];
        acc += k_ch[(long)state_len * channels] * input[c];
        out[c] = q35o_silu(acc);
        for (j = 0; j < state_len - 1; j++) cs[j] = cs[j + 1];
        cs[state_len - 1] = input[c];
    }
}

/* GatedDeltaNetOps.DeltaStep, src/Qwen35Sharp.Model/GatedDeltaNetOps.cs:179-229:
 * decay, read kv = S^T k, rank-1 write S += k (beta (v - kv))^T, read S^T q
 * from the updated state. */
static void delta_step(float* S, const float* q_in, const float* k_in, const float* v_in,
                       float decay, float beta, int head_dim, int v_head_dim, float* out,
                       float* kv_mem) {
    for (int a = 0; a < head_dim; a++) {
        float* row = S + (long)a * v_head_dim;
        for (int b = 0; b < v_head_dim; b++) row[b] *= decay;
    }
    for (int b = 0; b < v_head_dim; b++) {
        float acc = 0.0f;
        for (int a = 0; a < head_dim; a++) acc += S[(long)a * v_head_dim + b] * k_in[a];
        kv_mem[b] = acc;
    }
    for (int a = 0; a < head_dim; a++) {
        float k_a = k_in[a];
        float* row = S + (long)a * v_head_dim;
        for (int b = 0; b < v_head_dim; b++) {
            float delta = (v_in[b] - kv_mem[b]) * beta;
            row[b] += k_a * delta;
        }
    }
    for (int b = 0; b < v_head_dim; b++) {
        float acc = 0.0f;
        for (int a = 0; a < head_dim; a++) acc += S[(long)a * v_head_dim + b] * q_in[a];
        out[b] = acc;
    }
}

/* GatedDeltaNetOps.RecurrentGatedDeltaRule,
 * src/Qwen35Sharp.Model/GatedDeltaNetOps.cs:107-171.  Heads outer, tokens
 * inner.  q is scaled by 1/sqrt(head_dim); with l2norm_qk, q and k are
 * divided by sqrt(sum(x^2) + eps) first. */
void q35o_recurrent_gated_delta_rule(const float* q, const float* k, const float* v,
                                     const float* g, const float* beta, float* state,
                                     int tokens, int n_heads, int head_dim, int v_head_dim,
                                     float eps, float* out, int l2norm_qk) {
    float scale_q = 1.0f / sqrtf((float)head_dim);
    float* qn_buf = (float*)malloc(sizeof(float) * (size_t)head_dim);
    float* kn_buf = (float*)malloc(sizeof(float) * (size_t)head_dim);
    float* kv_mem = (float*)malloc(sizeof(float) * (size_t)v_head_dim);
    for (int h = 0; h < n_heads; h++) {
        float* S = state + (long)h * head_dim * v_head_dim;
        for (int i = 0; i < tokens; i++) {
            float g_ih = g[(long)i * n_heads + h];
            float beta_ih = beta[(long)i * n_heads + h];
            float decay = expf(g_ih);
            const float* qh = q + (long)i * n_heads * head_dim + (long)h * head_dim;
            const float* kh = k + (long)i * n_heads * head_dim + (long)h * head_dim;
            const float* vh = v + (long)i * n_heads * v_head_dim + (long)h * v_head_dim;
            float* oh = out + (long)i * n_heads * v_head_dim + (long)h * v_head_dim;
            if (l2norm_qk) {
                float qn = 0.0f, kn = 0.0f;
                for (int a = 0; a < head_dim; a++) {
                    qn += qh[a] * qh[a];
                    kn += kh[a] * kh[a];
                }
                float q_scale = scale_q / sqrtf(qn + eps);
                float k_scale = 1.0f / sqrtf(kn + eps);
                for (int a = 0; a < head_dim; a++) {
                    qn_buf[a] = qh[a] * q_scale;
                    kn_buf[a] = kh[a] * k_scale;
                }
                delta_step(S, qn_buf, kn_buf, vh, decay, beta_ih, head_dim, v_head_dim, oh, kv_mem);
            } else {
                for (int a = 0; a < head_dim; a++) qn_buf[a] = qh[a] * scale_q;
                delta_step(S, qn_buf, kh, vh, decay, beta_ih, head_dim, v_head_dim, oh, kv_mem);
            }
        }
    }
    free(qn_buf);
    free(kn_buf);
    free(kv_mem);
}

/* ------------------------------------------------------------------------- */
/* norms                                                                     */
/* ------------------------------------------------------------------------- */

/* Sum of squares with the AVX 8-lane FMA accumulator and HorizontalSum,
 * then a scalar tail: Qwen35Ops.cs:45-58 (RmsNormZeroCentered) and :88-101
 * (gated RmsNorm). */
static float sumsq_avx(const float* x, int dim) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i <= dim - 8; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    float sum = hsum8(acc);
    for (; i < dim; i++) sum += x[i] * x[i];
    return sum;
}

/* Qwen35Ops.RmsNormZeroCentered(Range), src/Qwen35Sharp.Model/Qwen35Ops.cs:22-66:
 * y = x * (1/sqrt(mean(x^2)+eps)) * (1 + w).  In place (x == y) is allowed. */
void q35o_rms_norm_zero_centered(const float* x, const float* weight, float* y,
                                 int rows, int dim, float eps) {
    for (int r = 0; r < rows; r++) {
        const float* src = x + (long)r * dim;
        float* dst = y + (long)r * dim;
        float sum = sumsq_avx(src, dim);
        float scale = 1.0f / sqrtf(sum / (float)dim + eps);
        for (int i = 0; i < dim; i++) {
            float w = weight ? weight[i] : 0.0f;
            dst[i] = src[i] * scale * (1.0f + w);
        }
    }
}

/* Qwen35Ops.GatedRmsNorm, src/Qwen35Sharp.Model/Qwen35Ops.cs:74-111:
 * y = (x * rsqrt(mean(x^2)+eps) * w) * silu(gate), plain w. */
void q35o_gated_rms_norm(const float* x, const float* weight, const float* gate, float* y,
                         int rows, int dim, float eps) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (long)r * dim;
        const float* gr = gate + (long)r * dim;
        float* yr = y + (long)r * dim;
        float sum = sumsq_avx(xr, dim);
        float scale = 1.0f / sqrtf(sum / (float)dim + eps);
        for (int i = 0; i < dim; i++) {
            float w = weight ? weight[i] : 1.0f;
            float n = xr[i] * scale * w;
            float gg = gr[i];
            yr[i] = n * (gg / (1.0f + expf(-gg)));
        }
    }
}

/* ------------------------------------------------------------------------- */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------- */

/* Ops.EnsureRopeTable, src/Qwen35Sharp.Model/Ops.cs:135-160: fp32 frequency
 * 1/base^(i/half), fp32 angle pos*freq, libm cosf/sinf of that angle. */
void q35o_rope_table(int cap, int half, float base_freq, float* cos_out, float* sin_out) {
    float* freqs = (float*)malloc(sizeof(float) * (size_t)half);
    for (int i = 0; i < half; i++) freqs[i] = 1.0f / powf(base_freq, (float)i / (float)half);
    for (int pos = 0; pos < cap; pos++)
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freqs[i];
            cos_out[(long)pos * half + i] = cosf(angle);
            sin_out[(long)pos * half + i] = sinf(angle);
        }
    free(freqs);
}

/* Ops.NeoXRoPE / RopeRange, src/Qwen35Sharp.Model/Ops.cs:75-133: rotate the
 * pairs (i, i+half), i < half, of each head row at position start_pos + t. */
void q35o_neox_rope(float* x, int tokens, int heads, int head_dim, int rope_dim,
                    int start_pos, float base_freq) {
    int half = rope_dim / 2;
    int needed = start_pos + tokens;
    int cap = needed > 4096 ? needed : 4096;
    float* cs = (float*)malloc(sizeof(float) * (size_t)cap * half);
    float* sn = (float*)malloc(sizeof(float) * (size_t)cap * half);
    q35o_rope_table(cap, half, base_freq, cs, sn);
    int rows = tokens * heads;
    for (int r = 0; r < rows; r++) {
        int t = r / heads;
        int h = r - t * heads;
        const float* c_row = cs + (long)(start_pos + t) * half;
        const float* s_row = sn + (long)(start_pos + t) * half;
        float* row = x + ((long)t * heads + h) * head_dim;
        for (int i = 0; i < half; i++) {
            float c = c_row[i], s = s_row[i];
            float x0 = row[i], x1 = row[i + half];
            row[i] = x0 * c - x1 * s;
            row[i + half] = x0 * s + x1 * c;
        }
    }
    free(cs);
    free(sn);
}

/* ------------------------------------------------------------------------- */
/* attention                                                                 */
/* ------------------------------------------------------------------------- */

/* Ops.DotF32, src/Qwen35Sharp.Model/Ops.cs:418-449: two 8-lane FMA
 * accumulators over 16-float strides, one over a trailing 8, HorizontalSum of
 * their sum, scalar tail. */
static float dot_f32(const float* a, const float* b, int n) {
    float acc0[8] = {0}, acc1[8] = {0};
    int i = 0;
    for (; i <= n - 16; i += 16)
        for (int l = 0; l < 8; l++) {
            acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
            acc1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], acc1[l]);
        }
    for (; i <= n - 8; i += 8)
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = acc0[l] + acc1[l];
    float sum = hsum8(s);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* Qwen35Model.F32Gemm, src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:129-140:
 * y[t][o] = DotF32(x[t], W[o]) for W [n_out][n_in] row-major (the reference's
 * Linear / DecodeLinear for F32 weights, Decode.cs:43-45, 77-79). */
void q35o_linear_f32(const float* w, const float* x, float* y, int n_in, int n_out, int tokens) {
    for (int t = 0; t < tokens; t++)
        for (int o = 0; o < n_out; o++)
            y[(size_t)t * n_out + o] = dot_f32(x + (size_t)t * n_in, w + (size_t)o * n_in, n_in);
}

/* Ops.DotF32x4, src/Qwen35Sharp.Model/Ops.cs:535-588 */
static void dot_f32x4(const float* q, const float* k0, const float* k1, const float* k2,
                      const float* k3, int n, float* dst, float scale) {
    float a0[8] = {0}, a1[8] = {0}, a2[8] = {0}, a3[8] = {0};
    int i = 0;
    for (; i <= n - 8; i += 8)
        for (int l = 0; l < 8; l++) {
            float qv = q[i + l];
            a0[l] = fmaf(qv, k0[i + l], a0[l]);
            a1[l] = fmaf(qv, k1[i + l], a1[l]);
            a2[l] = fmaf(qv, k2[i + l], a2[l]);
            a3[l] = fmaf(qv, k3[i + l], a3[l]);
        }
    float s0 = hsum8(a0), s1 = hsum8(a1), s2 = hsum8(a2), s3 = hsum8(a3);
    for (; i < n; i++) {
        float qv = q[i];
        s0 += qv * k0[i];
        s1 += qv * k1[i];
        s2 += qv * k2[i];
        s3 += qv * k3[i];
    }
    dst[0] = s0 * scale;
    dst[1] = s1 * scale;
    dst[2] = s2 * scale;
    dst[3] = s3 * scale;
}

/* Ops.Dot2x4, src/Qwen35Sharp.Model/Ops.cs:452-487 (n a multiple of 8). */
static void dot_2x4(const float* q0, const float* q1, const float* k, int kv_stride, int n,
                    float* dst0, float* dst1, float scale) {
    const float* kk[4] = {k, k + kv_stride, k + 2L * kv_stride, k + 3L * kv_stride};
    float acc[2][4][8];
    memset(acc, 0, sizeof(acc));
    for (int i = 0; i < n; i += 8)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 8; l++) {
                acc[0][r][l] = fmaf(q0[i + l], kk[r][i + l], acc[0][r][l]);
                acc[1][r][l] = fmaf(q1[i + l], kk[r][i + l], acc[1][r][l]);
            }
    for (int r = 0; r < 4; r++) {
        dst0[r] = hsum8_hadd(acc[0][r]) * scale;
        dst1[r] = hsum8_hadd(acc[1][r]) * scale;
    }
}

static int workers_for(int n_threads, int count) {
    if (n_threads < 1) n_threads = 1;
    return n_threads < count ? n_threads : count;
}

/* Ops.AttentionScores, src/Qwen35Sharp.Model/Ops.cs:281-357.  Heads are split
 * over workers as [heads*w/W, heads*(w+1)/W) (CpuThreadPool.For). */
static void scores_heads(const float* q, const float* cache_k, float* scores, int h_begin,
                         int h_end, int group, int head_dim, int q_len, int kv_len, int q_dim,
                         int kv_stride, float scale, int start_pos) {
    for (int h = h_begin; h < h_end; h++) {
        int kvh = h / group;
        const float* k_base = cache_k + (long)kvh * head_dim;
        int qt = 0;
        if ((head_dim & 7) == 0) {
            for (; qt + 1 < q_len; qt += 2) {
                const float* q0 = q + (long)qt * q_dim + (long)h * head_dim;
                const float* q1 = q0 + q_dim;
                float* row0 = scores + ((long)h * q_len + qt) * kv_len;
                float* row1 = row0 + kv_len;
                int allowed = kv_len < start_pos + qt + 2 ? kv_len : start_pos + qt + 2;
                int kt = 0;
                for (; kt + 3 < allowed; kt += 4)
                    dot_2x4(q0, q1, k_base + (long)kt * kv_stride, kv_stride, head_dim,
                            row0 + kt, row1 + kt, scale);
                for (; kt < allowed; kt++) {
                    const float* kh = k_base + (long)kt * kv_stride;
                    row0[kt] = dot_f32(q0, kh, head_dim) * scale;
                    row1[kt] = dot_f32(q1, kh, head_dim) * scale;
                }
            }
        }
        for (; qt < q_len; qt++) {
            const float* qh = q + (long)qt * q_dim + (long)h * head_dim;
            float* row = scores + ((long)h * q_len + qt) * kv_len;
            int allowed = kv_len < start_pos + qt + 1 ? kv_len : start_pos + qt + 1;
            int kt = 0;
            for (; kt + 3 < allowed; kt += 4) {
                const float* k0 = k_base + (long)(kt + 0) * kv_stride;
                dot_f32x4(qh, k0, k0 + kv_stride, k0 + 2L * kv_stride, k0 + 3L * kv_stride,
                          head_dim, row + kt, scale);
            }
            for (; kt < allowed; kt++) {
                const float* kh = k_base + (long)kt * kv_stride;
                row[kt] = dot_f32(qh, kh, head_dim) * scale;
            }
        }
    }
}

void q35o_attention_scores(const float* q, const float* cache_k, float* scores, int heads,
                           int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                           int kv_stride, float scale, int start_pos, int n_threads) {
    int group = heads / kv_heads;
    int W = workers_for(n_threads, heads);
#pragma omp parallel num_threads(W)
    {
        int w = 0, nw = 1;
#ifdef _OPENMP
        w = omp_get_thread_num();
        nw = omp_get_num_threads();
#endif
        scores_heads(q, cache_k, scores, heads * w / nw, heads * (w + 1) / nw, group, head_dim,
                     q_len, kv_len, q_dim, kv_stride, scale, start_pos);
    }
}

/* Ops.SoftmaxRow, src/Qwen35Sharp.Model/Ops.cs:188-252: max seeded at -80,
 * shifted logits floored at -80, FastExp on 8-lane blocks and libm expf on
 * the tail (or everywhere when n < 8), normalise by 1/sum. */
static void softmax_row(float* row, int n) {
    int i = 0;
    float mx, sum;
    if (n >= 8) {
        float vmax[8];
        for (int l = 0; l < 8; l++) vmax[l] = -80.0f;
        for (; i <= n - 8; i += 8)
            for (int l = 0; l < 8; l++) vmax[l] = row[i + l] > vmax[l] ? row[i + l] : vmax[l];
        mx = hmax8(vmax);
        for (; i < n; i++)
            if (row[i] > mx) mx = row[i];
        float vsum[8] = {0};
        i = 0;
        for (; i <= n - 8; i += 8)
            for (int l = 0; l < 8; l++) {
                float sh = row[i + l] - mx;
                sh = sh > -80.0f ? sh : -80.0f;
                float e = q35o_fast_exp(sh);
                row[i + l] = e;
                vsum[l] = vsum[l] + e;
            }
        sum = hsum8(vsum);
        for (; i < n; i++) {
            float e = expf(fmaxf(row[i] - mx, -80.0f));
            row[i] = e;
            sum += e;
        }
    } else {
        mx = -80.0f;
        for (i = 0; i < n; i++)
            if (row[i] > mx) mx = row[i];
        sum = 0.0f;
        for (i = 0; i < n; i++) {
            float e = expf(fmaxf(row[i] - mx, -80.0f));
            row[i] = e;
            sum += e;
        }
    }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (i = 0; i < n; i++) row[i] *= inv;
}

/* Ops.SoftmaxCausal, src/Qwen35Sharp.Model/Ops.cs:162-186: only the visible
 * prefix min(kv_len, start+q+1) is normalised; the masked tail is zeroed. */
void q35o_softmax_causal(float* scores, int heads, int q_len, int kv_len, int start_pos,
                         int n_threads) {
    int W = workers_for(n_threads, heads);
#pragma omp parallel num_threads(W)
    {
        int w = 0, nw = 1;
#ifdef _OPENMP
        w = omp_get_thread_num();
        nw = omp_get_num_threads();
#endif
        for (int h = heads * w / nw; h < heads * (w + 1) / nw; h++)
            for (int qi = 0; qi < q_len; qi++) {
                float* row = scores + ((long)h * q_len + qi) * kv_len;
                int allowed = kv_len < start_pos + qi + 1 ? kv_len : start_pos + qi + 1;
                softmax_row(row, allowed);
                for (int j = allowed; j < kv_len; j++) row[j] = 0.0f;
            }
    }
}

/* Ops.Axpy64, src/Qwen35Sharp.Model/Ops.cs:500-533: 64 outputs held in
 * registers, kt ascending, FMA. */
static void axpy64(const float* w, const float* v, int kv_stride, int count, float* dst) {
    float acc[64];
    for (int j = 0; j < 64; j++) acc[j] = 0.0f;
    for (int kt = 0; kt < count; kt++) {
        float wv = w[kt];
        const float* row = v + (long)kt * kv_stride;
        for (int j = 0; j < 64; j++) acc[j] = fmaf(wv, row[j], acc[j]);
    }
    for (int j = 0; j < 64; j++) dst[j] = acc[j];
}

/* Ops.AxpyF32, src/Qwen35Sharp.Model/Ops.cs:590-622 */
static void axpy_f32(float* y, const float* x, float a, int n) {
    int i = 0;
    for (; i <= n - 8; i += 8)
        for (int l = 0; l < 8; l++) y[i + l] = fmaf(a, x[i + l], y[i + l]);
    for (; i < n; i++) y[i] += a * x[i];
}

/* Ops.AttentionCombine, src/Qwen35Sharp.Model/Ops.cs:359-415 */
void q35o_attention_combine(const float* cache_v, const float* scores, float* output,
                            int heads, int kv_heads, int head_dim, int q_len, int kv_len,
                            int q_dim, int kv_stride, int start_pos, int n_threads) {
    int group = heads / kv_heads;
    int W = workers_for(n_threads, heads);
#pragma omp parallel num_threads(W)
    {
        int w = 0, nw = 1;
#ifdef _OPENMP
        w = omp_get_thread_num();
        nw = omp_get_num_threads();
#endif
        for (int h = heads * w / nw; h < heads * (w + 1) / nw; h++) {
            int kvh = h / group;
            const float* v_base = cache_v + (long)kvh * head_dim;
            for (int qt = 0; qt < q_len; qt++) {
                const float* row = scores + ((long)h * q_len + qt) * kv_len;
                float* out_h = output + (long)qt * q_dim + (long)h * head_dim;
                int allowed = kv_len < start_pos + qt + 1 ? kv_len : start_pos + qt + 1;
                int d = 0;
                for (; d + 63 < head_dim; d += 64)
                    axpy64(row, v_base + d, kv_stride, allowed, out_h + d);
                if (d < head_dim) {
                    for (int i = d; i < head_dim; i++) out_h[i] = 0.0f;
                    for (int kt = 0; kt < allowed; kt++)
                        axpy_f32(out_h + d, v_base + (long)kt * kv_stride + d, row[kt],
                                 head_dim - d);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* mixer glue                                                                */
/* ------------------------------------------------------------------------- */

/* Qwen35Model.DecodeLinearAttn steps 2-6,
 * src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:348-397.  core_out (may be
 * NULL) receives the pre-norm recurrence output. */
void q35o_deltanet_decode(const q35o_dims* d, const float* qkv, const float* z,
                          const float* b, const float* a, const float* conv_w,
                          const float* ssm_a, const float* dt_bias, const float* ssm_norm,
                          float* conv_state, float* state, float* out, float* core_out) {
    int nk = d->n_k_heads, nv = d->n_v_heads, hd = d->head_k_dim;
    int key_dim = nk * hd, value_dim = nv * hd;
    int conv_dim = 2 * key_dim + value_dim;
    int repeat = nv / nk;
    float* conv_out = (float*)malloc(sizeof(float) * (size_t)conv_dim);
    float* q = (float*)malloc(sizeof(float) * (size_t)nv * hd);
    float* k = (float*)malloc(sizeof(float) * (size_t)nv * hd);
    float* v = (float*)malloc(sizeof(float) * (size_t)value_dim);
    float* beta = (float*)malloc(sizeof(float) * (size_t)nv);
    float* g = (float*)malloc(sizeof(float) * (size_t)nv);
    float* o = (float*)malloc(sizeof(float) * (size_t)nv * hd);

    q35o_causal_conv1d_update(qkv, conv_w, d->conv_kernel, conv_dim, conv_state, conv_out);
    const float* raw_q = conv_out;
    const float* raw_k = conv_out + key_dim;
    const float* raw_v = conv_out + 2 * key_dim;
    for (int kh = 0; kh < nk; kh++)
        for (int rep = 0; rep < repeat; rep++) {
            int vh = kh * repeat + rep;
            for (int j = 0; j < hd; j++) {
                q[vh * hd + j] = raw_q[kh * hd + j];
                k[vh * hd + j] = raw_k[kh * hd + j];
            }
        }
    for (int j = 0; j < value_dim; j++) v[j] = raw_v[j];
    q35o_sigmoid(b, beta, nv);
    for (int i = 0; i < nv; i++) g[i] = ssm_a[i] * q35o_softplus(a[i] + dt_bias[i]);
    q35o_recurrent_gated_delta_rule(q, k, v, g, beta, state, 1, nv, hd, hd, d->eps, o, 1);
    if (core_out) memcpy(core_out, o, sizeof(float) * (size_t)nv * hd);
    q35o_gated_rms_norm(o, ssm_norm, z, out, nv, hd, d->eps);

    free(conv_out); free(q); free(k); free(v); free(beta); free(g); free(o);
}

/* Qwen35Model.PrefillLinearAttn steps 2-6,
 * src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:181-260.
 *
 * The channel-major copy of qkv and the conv output are laid out back to
 * back, 64-byte aligned, as the reference's scratch arena lays them out
 * (Qwen35Model.cs:411-426), so the conv-state write-back for T < 3 reads past
 * the channel row into the same neighbouring data as the reference
 * (Qwen35Model.Prefill.cs:195-204).  conv_state is written, never read
 * (the prefill conv zero-pads and ignores it: GatedDeltaNetOps.cs:45-47). */
void q35o_deltanet_prefill(const q35o_dims* d, int T, const float* qkv, const float* z,
                           const float* b, const float* a, const float* conv_w,
                           const float* ssm_a, const float* dt_bias, const float* ssm_norm,
                           float* conv_state, float* state, float* out, float* core_out) {
    int nk = d->n_k_heads, nv = d->n_v_heads, hd = d->head_k_dim;
    int key_dim = nk * hd, value_dim = nv * hd;
    int conv_dim = 2 * key_dim + value_dim;
    int repeat = nv / nk;
    long ct = (long)conv_dim * T;
    long ch_floats = ((ct * 4 + 63) & ~63L) / 4;
    float* arena = (float*)calloc((size_t)(ch_floats + ct), sizeof(float));
    float* qkv_ch = arena;
    float* conv_out_ch = arena + ch_floats;
    for (int c = 0; c < conv_dim; c++)
        for (int t = 0; t < T; t++) qkv_ch[(long)c * T + t] = qkv[(long)t * conv_dim + c];
    q35o_causal_conv1d(qkv_ch, conv_w, d->conv_kernel, conv_dim, T, conv_out_ch);

    int state_len = d->conv_kernel - 1 > 1 ? d->conv_kernel - 1 : 1;
    for (int c = 0; c < conv_dim; c++) {
        float* cs = conv_state + (long)c * state_len;
        int tail_start = T - state_len;
        if (tail_start < 0) tail_start = 0;
        for (int j = 0; j < state_len; j++) cs[j] = qkv_ch[(long)c * T + tail_start + j];
    }

    float* qs = (float*)malloc(sizeof(float) * (size_t)T * nv * hd);
    float* ks = (float*)malloc(sizeof(float) * (size_t)T * nv * hd);
    float* vs = (float*)malloc(sizeof(float) * (size_t)T * value_dim);
    for (int t = 0; t < T; t++) {
        for (int kh = 0; kh < nk; kh++)
            for (int rep = 0; rep < repeat; rep++) {
                int vh = kh * repeat + rep;
                for (int j = 0; j < hd; j++) {
                    qs[(long)t * nv * hd + vh * hd + j] = conv_out_ch[(long)(kh * hd + j) * T + t];
                    ks[(long)t * nv * hd + vh * hd + j] =
                        conv_out_ch[(long)(key_dim + kh * hd + j) * T + t];
                }
            }
        for (int j = 0; j < value_dim; j++)
            vs[(long)t * value_dim + j] = conv_out_ch[(long)(2 * key_dim + j) * T + t];
    }
    float* beta = (float*)malloc(sizeof(float) * (size_t)T * nv);
    float* g = (float*)malloc(sizeof(float) * (size_t)T * nv);
    q35o_sigmoid(b, beta, T * nv);
    for (int i = 0; i < T * nv; i++) {
        int head = i % nv;
        g[i] = ssm_a[head] * q35o_softplus(a[i] + dt_bias[head]);
    }
    float* o = (float*)malloc(sizeof(float) * (size_t)T * nv * hd);
    q35o_recurrent_gated_delta_rule(qs, ks, vs, g, beta, state, T, nv, hd, hd, d->eps, o, 1);
    if (core_out) memcpy(core_out, o, sizeof(float) * (size_t)T * nv * hd);
    q35o_gated_rms_norm(o, ssm_norm, z, out, T * nv, hd, d->eps);

    free(arena); free(qs); free(ks); free(vs); free(beta); free(g); free(o);
}

/* Shared body of DecodeAttention / PrefillAttention after the projections:
 * src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:294-323 (seq = 1) and
 * src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:113-149 (seq = T).
 * k and v ([T][kv_dim]) are the projection outputs; the reference writes them
 * straight into cache rows start..start+T-1 and RoPEs / norms K there. */
static void attn_mixer(const q35o_dims* d, int start, int T, const float* q_gate,
                       const float* k, const float* v, const float* q_norm,
                       const float* k_norm, float* cache_k, float* cache_v, float* out,
                       int n_threads) {
    int heads = d->n_heads, kv_heads = d->n_kv_heads, dim = d->head_dim;
    int q_dim = heads * dim, k_dim = kv_heads * dim;
    float* q = (float*)malloc(sizeof(float) * (size_t)T * q_dim);
    float* gate = (float*)malloc(sizeof(float) * (size_t)T * q_dim);
    float* kc = cache_k + (long)start * k_dim;
    float* vc = cache_v + (long)start * k_dim;
    memcpy(kc, k, sizeof(float) * (size_t)T * k_dim);
    memcpy(vc, v, sizeof(float) * (size_t)T * k_dim);
    for (int t = 0; t < T; t++) {
        const float* row = q_gate + (long)t * 2 * q_dim;
        for (int h = 0; h < heads; h++) {
            int base = h * 2 * dim;
            for (int j = 0; j < dim; j++) {
                q[(long)t * q_dim + h * dim + j] = row[base + j];
                gate[(long)t * q_dim + h * dim + j] = row[base + dim + j];
            }
        }
    }
    q35o_neox_rope(q, T, heads, dim, d->rope_dim, start, d->rope_base);
    q35o_neox_rope(kc, T, kv_heads, dim, d->rope_dim, start, d->rope_base);
    q35o_rms_norm_zero_centered(q, q_norm, q, T * heads, dim, d->eps);
    q35o_rms_norm_zero_centered(kc, k_norm, kc, T * kv_heads, dim, d->eps);

    int kv_len = start + T;
    float scale = 1.0f / sqrtf((float)dim);
    float* sc = (float*)malloc(sizeof(float) * (size_t)heads * T * kv_len);
    q35o_attention_scores(q, cache_k, sc, heads, kv_heads, dim, T, kv_len, q_dim, k_dim, scale,
                          start, n_threads);
    q35o_softmax_causal(sc, heads, T, kv_len, start, n_threads);
    q35o_attention_combine(cache_v, sc, out, heads, kv_heads, dim, T, kv_len, q_dim, k_dim,
                           start, n_threads);
    long total = (long)T * q_dim;
    for (long i = 0; i < total; i++) out[i] *= 1.0f / (1.0f + expf(-gate[i]));
    free(q); free(gate); free(sc);
}

void q35o_attn_decode(const q35o_dims* d, int start, const float* q_gate, const float* k,
                      const float* v, const float* q_norm, const float* k_norm,
                      float* cache_k, float* cache_v, float* out, int n_threads) {
    attn_mixer(d, start, 1, q_gate, k, v, q_norm, k_norm, cache_k, cache_v, out, n_threads);
}

void q35o_attn_prefill(const q35o_dims* d, int start, int T, const float* q_gate,
                       const float* k, const float* v, const float* q_norm,
                       const float* k_norm, float* cache_k, float* cache_v, float* out,
                       int n_threads) {
    attn_mixer(d, start, T, q_gate, k, v, q_norm, k_norm, cache_k, cache_v, out, n_threads);
}
