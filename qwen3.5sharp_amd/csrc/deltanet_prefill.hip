// Gated-DeltaNet prefill mixer for T tokens of one sequence: chunked WY form
// (chunk C = 64) on fp32 MFMA.
//
// Reference: Qwen35Model.PrefillLinearAttn steps 2-6
// (src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:181-260), whose recurrence is
// the sequential GatedDeltaNetOps.RecurrentGatedDeltaRule
// (GatedDeltaNetOps.cs:107-229).  Per head and token, with decay a_t = e^{g_t}:
//   S_t = a_t S_{t-1} + k_t d_t^T,  d_t = beta_t (v_t - a_t S_{t-1}^T k_t),
//   o_t = S_t^T q_t.
// Within a chunk whose state on entry is S0, with G_i = g_0 + ... + g_i and
// gamma_i = e^{G_i}, unrolling the recurrence gives (Yang et al., "Gated Delta
// Networks", arXiv:2412.06464; "Parallelizing Linear Transformers with the
// Delta Rule over Sequence Length", arXiv:2406.06484):
//   (I + A) D = diag(beta) (V - diag(gamma) K S0),
//       A_ij = beta_i e^{G_i - G_j} (k_i . k_j) for j < i (strictly lower)
//   D = U - W S0,  U = T diag(beta) V,  W = T diag(beta gamma) K,  T = (I+A)^-1
//   O = diag(gamma) Q S0 + (M o Q K^T) D,  M_ij = e^{G_i - G_j} for j <= i
//   S_C = gamma_last S0 + K^T diag(e^{G_last - G}) D
// Only e^{G_i - G_j} with j <= i (never e^{G_i} e^{-G_j}) is formed, with G
// accumulated in fp64, so nothing overflows and the decays of long chunks
// (G reaches ~ -2000) keep full fp32 accuracy.
//
// Kernels:
//  1. deltanet_prefill_prep: zero-padded causal conv with the prefill tap
//     order (tap j multiplies x[t-j], GatedDeltaNetOps.cs:27-53) + SiLU, read
//     straight from the token-major qkv (no transpose); q/k L2 norm (q also
//     scaled by 1/sqrt(dk)); beta = sigmoid(b), g = ssm_a * softplus(a +
//     dt_bias) (Prefill.cs:239-248).
//  2. deltanet_conv_writeback: conv window <- last K-1 raw inputs
//     (Prefill.cs:192-204), reproducing the reference's read past the channel
//     row when T < K-1.
//  3. dn_chunk_prep (one workgroup per k-head and chunk; the R v-heads of the
//     k-head share K K^T and Q K^T): K K^T and Q K^T on MFMA, the decay masks,
//     T = (I+A)^-1 by blocked forward substitution (16x16 diagonal blocks
//     inverted in registers, off-diagonal blocks applied on MFMA), then
//     W and U on MFMA.  Emits W, U, M o QK^T, gamma, e^{G_last - G}.
//  4. dn_chunk_scan (one workgroup per v-head and 16-column tile of the
//     state): walks the chunks in order with the state tile in MFMA
//     accumulators: D = U - W S, O = gamma Q S + (M o QK^T) D,
//     S = gamma_last S + K^T (e^{G_last-G} D).  Column tiles are independent
//     (the rule is separable over dv), so 8 workgroups per head run in
//     parallel; the 8 tiles of a head share an XCD so W, Q, K stay in its L2.
//  5. deltanet_gated_norm: gated RMSNorm per (token, v-head) row.
//
// MFMA: v_mfma_f32_16x16x4f32.  Lane l = 16g + c holds A[c][g] and B[g][c];
// D register r holds D[4g + r][c].  A 16-deep product is 4 instructions; in
// instruction s lane group g supplies reduction index 4g + s, so a D tile can
// be fed back as the B operand register by register.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc += A(16x16 block, float4 per lane = reduction 4g..4g+3) * B(D-layout tile)
__device__ __forceinline__ f32x4 mfma16x4(float4 a, f32x4 b, f32x4 acc) {
    acc = mfma16(a.x, b[0], acc);
    acc = mfma16(a.y, b[1], acc);
    acc = mfma16(a.z, b[2], acc);
    acc = mfma16(a.w, b[3], acc);
    return acc;
}

constexpr int CH = 64;        // chunk length
constexpr int LDK = 132;      // padded LDS row stride of [64][128] tiles
constexpr int LDA = 68;       // padded LDS row stride of [64][64] tiles

struct PrefillWork {
    float* qhat;   // [T][nk][dk]  L2-normed, scaled by 1/sqrt(dk)
    float* khat;   // [T][nk][dk]
    float* vv;     // [T][nv][dv]
    float* beta;   // [T][nv]
    float* gl;     // [T][nv]   g (log decay)
    float* core;   // [T][nv][dv] pre-norm recurrence output
    float* W;      // [nv][nch][64][128]
    float* U;      // [nv][nch][64][128]
    float* Aqk;    // [nv][nch][64][64]
    float* gam;    // [nv][nch][64]   e^{G_i}
    float* gdec;   // [nv][nch][64]   e^{G_last - G_i}
};

size_t work_floats(const Dims& d, int T, int nch) {
    return (size_t)T * (2 * d.key_dim + 2 * d.value_dim + 2 * d.nv) +
           (size_t)d.nv * nch * (2 * CH * kDk + CH * CH + 2 * CH);
}

PrefillWork carve(float* w, const Dims& d, int T, int nch) {
    PrefillWork p;
    p.qhat = w;
    p.khat = p.qhat + (size_t)T * d.key_dim;
    p.vv = p.khat + (size_t)T * d.key_dim;
    p.beta = p.vv + (size_t)T * d.value_dim;
    p.gl = p.beta + (size_t)T * d.nv;
    p.core = p.gl + (size_t)T * d.nv;
    p.W = p.core + (size_t)T * d.value_dim;
    p.U = p.W + (size_t)d.nv * nch * CH * kDk;
    p.Aqk = p.U + (size_t)d.nv * nch * CH * kDk;
    p.gam = p.Aqk + (size_t)d.nv * nch * CH * CH;
    p.gdec = p.gam + (size_t)d.nv * nch * CH;
    return p;
}

__global__ __launch_bounds__(kDk) void deltanet_prefill_prep(
    const float* __restrict__ qkv, const float* __restrict__ bin, const float* __restrict__ ain,
    const float* __restrict__ conv_w, const float* __restrict__ ssm_a,
    const float* __restrict__ dt_bias, PrefillWork w, int T, int nk, int nv, float eps) {
    const int t = blockIdx.x, hb = blockIdx.y, tid = threadIdx.x;
    const int key_dim = nk * kDk, conv_dim = 2 * key_dim + nv * kDk;
    int c;
    if (hb < nk) c = hb * kDk + tid;
    else if (hb < 2 * nk) c = key_dim + (hb - nk) * kDk + tid;
    else c = 2 * key_dim + (hb - 2 * nk) * kDk + tid;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kConvK; ++j)
        if (t - j >= 0) acc += conv_w[(size_t)j * conv_dim + c] * qkv[(size_t)(t - j) * conv_dim + c];
    const float y = silu(acc);
    if (hb < 2 * nk) {
        __shared__ float red[2];
        const float ss = wave_sum(y * y);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        const float n2 = red[0] + red[1];
        const int kh = hb < nk ? hb : hb - nk;
        const size_t off = ((size_t)t * nk + kh) * kDk + tid;
        if (hb < nk) w.qhat[off] = y * ((1.0f / sqrtf((float)kDk)) / sqrtf(n2 + eps));
        else w.khat[off] = y * (1.0f / sqrtf(n2 + eps));
    } else {
        const int vh = hb - 2 * nk;
        w.vv[((size_t)t * nv + vh) * kDk + tid] = y;
        if (tid == 0) {
            const size_t gi = (size_t)t * nv + vh;
            w.beta[gi] = 1.0f / (1.0f + expf(-bin[gi]));
            w.gl[gi] = ssm_a[vh] * softplus_ref(ain[gi] + dt_bias[vh]);
        }
    }
}

// cs[c][j] = qkvCh[c*T + tail + j] over the channel-major copy qkvCh [C][T]
// followed (64-byte aligned, as the reference's arena) by the conv output
// [C][T]; for T >= 3 this is x[T-3+j][c].
__global__ void deltanet_conv_writeback(const float* __restrict__ qkv,
                                        const float* __restrict__ conv_w, float* __restrict__ cs,
                                        int T, int conv_dim) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= conv_dim) return;
    const long ct = (long)conv_dim * T;
    const long ch_floats = ((ct * 4 + 63) & ~63L) / 4;
    const int tail = T - kConvState > 0 ? T - kConvState : 0;
    for (int j = 0; j < kConvState; ++j) {
        const long idx = (long)c * T + tail + j;
        float val;
        if (idx < ct) {
            val = qkv[(idx % T) * conv_dim + idx / T];
        } else if (idx < ch_floats) {
            val = 0.0f;  // arena padding (never reached when conv_dim*T is a multiple of 16)
        } else {
            const long o = idx - ch_floats;
            const int cc = (int)(o / T), tt = (int)(o % T);
            float acc = 0.0f;
            for (int k = 0; k < kConvK; ++k)
                if (tt - k >= 0) acc += conv_w[(size_t)k * conv_dim + cc] * qkv[(size_t)(tt - k) * conv_dim + cc];
            val = acc / (1.0f + expf(-acc));
        }
        cs[(size_t)c * kConvState + j] = val;
    }
}

// Lower-triangular 16x16 blocks (rb >= cb) of a 64x64 matrix, in work order.
__constant__ int kTriRb[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
__constant__ int kTriCb[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};

__global__ __launch_bounds__(256) void dn_chunk_prep(PrefillWork w, int T, int nk, int nv,
                                                     int nch) {
    const int kh = blockIdx.x / nch, n = blockIdx.x % nch;
    const int R = nv / nk;
    const int t0 = n * CH;
    const int tn = min(CH, T - t0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;

    __shared__ float Ks[CH][LDK];
    __shared__ float QV[CH][LDK];    // Q^ of the chunk, then V of each v-head
    __shared__ float KK[CH][LDA];
    __shared__ float QK[CH][LDA];
    __shared__ float Am[CH][LDA];    // -A (strictly lower)
    __shared__ float Td[4][16][17];  // inverses of the 16x16 diagonal blocks of I + A
    __shared__ double Gd[CH];
    __shared__ float bet[CH], gam[CH];

    for (int idx = tid; idx < CH * (kDk / 4); idx += 256) {
        const int r = idx / (kDk / 4), c4 = idx % (kDk / 4);
        float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), qx = kx;
        if (r < tn) {
            const size_t off = ((size_t)(t0 + r) * nk + kh) * kDk + 4 * c4;
            kx = *reinterpret_cast<const float4*>(w.khat + off);
            qx = *reinterpret_cast<const float4*>(w.qhat + off);
        }
        *reinterpret_cast<float4*>(&Ks[r][4 * c4]) = kx;
        *reinterpret_cast<float4*>(&QV[r][4 * c4]) = qx;
    }
    __syncthreads();

    // K K^T and Q K^T, lower 16x16 blocks only: 20 blocks, 5 per wave.
    for (int bi = wave; bi < 20; bi += 4) {
        const int mat = bi / 10, rb = kTriRb[bi % 10], cb = kTriCb[bi % 10];
        const float(*src)[LDK] = mat ? QV : Ks;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < kDk / 16; ++q) {
            const float4 a = *reinterpret_cast<const float4*>(&src[16 * rb + c16][16 * q + 4 * g]);
            const float4 b = *reinterpret_cast<const float4*>(&Ks[16 * cb + c16][16 * q + 4 * g]);
            acc = mfma16(a.x, b.x, acc);
            acc = mfma16(a.y, b.y, acc);
            acc = mfma16(a.z, b.z, acc);
            acc = mfma16(a.w, b.w, acc);
        }
        float(*dst)[LDA] = mat ? QK : KK;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[16 * rb + 4 * g + r][16 * cb + c16] = acc[r];
    }
    __syncthreads();

    for (int rr = 0; rr < R; ++rr) {
        const int vh = kh * R + rr;
        const size_t cidx = (size_t)vh * nch + n;
        // Gates and the fp64 running sum of g; padded tokens get beta = g = 0.
        if (wave == 0) {
            const int t = min(t0 + lane, T - 1);
            const bool valid = lane < tn;
            const float bv = w.beta[(size_t)t * nv + vh], gv = w.gl[(size_t)t * nv + vh];
            const float b = valid ? bv : 0.0f;
            double G = valid ? (double)gv : 0.0;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const double up = __shfl_up(G, o, kWave);
                if (lane >= o) G += up;
            }
            Gd[lane] = G;
            bet[lane] = b;
            gam[lane] = expf((float)G);
            w.gam[cidx * CH + lane] = expf((float)G);
        }
        // V of this v-head (Q^ is no longer needed).
        for (int idx = tid; idx < CH * (kDk / 4); idx += 256) {
            const int r = idx / (kDk / 4), c4 = idx % (kDk / 4);
            float4 vx = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < tn) vx = *reinterpret_cast<const float4*>(w.vv + ((size_t)(t0 + r) * nv + vh) * kDk + 4 * c4);
            *reinterpret_cast<float4*>(&QV[r][4 * c4]) = vx;
        }
        __syncthreads();
        if (wave == 1) w.gdec[cidx * CH + lane] = expf((float)(Gd[CH - 1] - Gd[lane]));
        // Decay masks: -A (strictly lower) into LDS, M o QK^T to the workspace.
        float* aqk = w.Aqk + cidx * CH * CH;
        for (int idx = tid; idx < CH * CH; idx += 256) {
            const int i = idx / CH, j = idx % CH;
            const float dcy = j <= i ? expf((float)(Gd[i] - Gd[j])) : 0.0f;
            Am[i][j] = j < i ? -bet[i] * dcy * KK[i][j] : 0.0f;
            aqk[idx] = j <= i ? dcy * QK[i][j] : 0.0f;
        }
        __syncthreads();
        // Inverse of each unit-lower 16x16 diagonal block of I + A by forward
        // substitution: column j of the inverse, x_i = sum_{m<i} (-A)_im x_m.
        if (lane < 16) {
            const int j = lane, b0 = 16 * wave;
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float s = i == j ? 1.0f : 0.0f;
#pragma unroll
                for (int m = 0; m < i; ++m) s += Am[b0 + i][b0 + m] * x[m];
                x[i] = i < j ? 0.0f : s;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) Td[wave][i][j] = x[i];
        }
        __syncthreads();
        // Y = (I + A)^-1 X for X = diag(beta gamma) K^ (-> W) and diag(beta) V (-> U),
        // block row by block row; wave takes column blocks wave + 4k of the 16.
        for (int k4 = 0; k4 < 4; ++k4) {
            const int cbk = wave + 4 * k4;
            const bool isV = cbk >= 8;
            const int cc = (cbk & 7) * 16;
            const float(*src)[LDK] = isV ? QV : Ks;
            float* dst = (isV ? w.U : w.W) + cidx * CH * kDk;
            f32x4 Y[4];
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) {
                f32x4 acc;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * ib + 4 * g + r;
                    const float sc = isV ? bet[row] : bet[row] * gam[row];
                    acc[r] = src[row][cc + c16] * sc;
                }
#pragma unroll
                for (int jb = 0; jb < ib; ++jb) {
                    const float4 a = *reinterpret_cast<const float4*>(&Am[16 * ib + c16][16 * jb + 4 * g]);
                    acc = mfma16x4(a, Y[jb], acc);
                }
                const float4 tdv = make_float4(Td[ib][c16][4 * g], Td[ib][c16][4 * g + 1],
                                               Td[ib][c16][4 * g + 2], Td[ib][c16][4 * g + 3]);
                f32x4 y = {0.f, 0.f, 0.f, 0.f};
                Y[ib] = mfma16x4(tdv, acc, y);
#pragma unroll
                for (int r = 0; r < 4; ++r) dst[(16 * ib + 4 * g + r) * kDk + cc + c16] = Y[ib][r];
            }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void dn_chunk_scan(PrefillWork w, float* __restrict__ state,
                                                     int T, int nk, int nv, int nch) {
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int vh = L / 8, tl = L % 8;
    const int kh = vh / (nv / nk);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int col = 16 * tl + c16;
    float* S = state + (size_t)vh * kDk * kDk;

    // State rows 32*wave + 16b + 4g + r, column col, as two D-layout tiles.
    f32x4 Sb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) Sb[b][r] = S[(size_t)(32 * wave + 16 * b + 4 * g + r) * kDk + col];

    __shared__ f32x4 red[4][2][4][64];
    __shared__ f32x4 dl[4][64];

    for (int n = 0; n < nch; ++n) {
        const int t0 = n * CH;
        const size_t cidx = (size_t)vh * nch + n;
        const float* Wc = w.W + cidx * CH * kDk;
        const float* Uc = w.U + cidx * CH * kDk;
        const float* Ac = w.Aqk + cidx * CH * CH;
        const float* gm = w.gam + cidx * CH;
        const float* gd = w.gdec + cidx * CH;

        // Loads that do not depend on the state go out first.
        float kT[4][2][4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int t = min(t0 + 16 * tb + 4 * g + s, T - 1);
                const float* kr = w.khat + ((size_t)t * nk + kh) * kDk + 32 * wave + c16;
                kT[tb][0][s] = kr[0];
                kT[tb][1][s] = kr[16];
            }
        f32x4 uu, gmo, gdv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uu[r] = Uc[(size_t)(16 * wave + 4 * g + r) * kDk + col];
            gmo[r] = gm[16 * wave + 4 * g + r];
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) gdv[tb][r] = gd[16 * tb + 4 * g + r];
        const float glast = gm[CH - 1];

        // Partial W S and Q S over this wave's 32 state rows, all 4 token blocks.
        f32x4 pws[4], pqs[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            pws[tb] = {0.f, 0.f, 0.f, 0.f};
            pqs[tb] = {0.f, 0.f, 0.f, 0.f};
            const int tq = min(t0 + 16 * tb + c16, T - 1);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int k0 = 32 * wave + 16 * b + 4 * g;
                const float4 wa = *reinterpret_cast<const float4*>(Wc + (size_t)(16 * tb + c16) * kDk + k0);
                const float4 qa = *reinterpret_cast<const float4*>(w.qhat + ((size_t)tq * nk + kh) * kDk + k0);
                pws[tb] = mfma16x4(wa, Sb[b], pws[tb]);
                pqs[tb] = mfma16x4(qa, Sb[b], pqs[tb]);
            }
            red[wave][0][tb][lane] = pws[tb];
            red[wave][1][tb][lane] = pqs[tb];
        }
        __syncthreads();
        // Token block `wave`: D = U - W S, and the Q S rows of the output.
        f32x4 ws = red[0][0][wave][lane], qs = red[0][1][wave][lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) {
            ws += red[v][0][wave][lane];
            qs += red[v][1][wave][lane];
        }
        dl[wave][lane] = uu - ws;
        __syncthreads();
        f32x4 D[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) D[tb] = dl[tb][lane];

        // O rows of token block `wave` = gamma Q S + (M o QK^T) D (causal: blocks <= wave).
        f32x4 o = gmo * qs;
        for (int tb = 0; tb <= wave; ++tb) {
            const float4 aa = *reinterpret_cast<const float4*>(Ac + (size_t)(16 * wave + c16) * CH + 16 * tb + 4 * g);
            o = mfma16x4(aa, D[tb], o);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 16 * wave + 4 * g + r;
            if (t < T) w.core[((size_t)t * nv + vh) * kDk + col] = o[r];
        }
        // S = gamma_last S + K^T (e^{G_last - G} D).
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            f32x4 acc = Sb[b] * glast;
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                const f32x4 dd = D[tb] * gdv[tb];
                acc = mfma16(kT[tb][b][0], dd[0], acc);
                acc = mfma16(kT[tb][b][1], dd[1], acc);
                acc = mfma16(kT[tb][b][2], dd[2], acc);
                acc = mfma16(kT[tb][b][3], dd[3], acc);
            }
            Sb[b] = acc;
        }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[(size_t)(32 * wave + 16 * b + 4 * g + r) * kDk + col] = Sb[b][r];
}

// Qwen35Ops.GatedRmsNorm (Qwen35Ops.cs:74-111) over rows of dv = 128.
__global__ __launch_bounds__(kDk) void deltanet_gated_norm(const float* __restrict__ core,
                                                           const float* __restrict__ z,
                                                           const float* __restrict__ wnorm,
                                                           float* __restrict__ out, float eps) {
    const size_t row = blockIdx.x;
    const int e = threadIdx.x;
    const float x = core[row * kDk + e];
    __shared__ float red[2];
    const float ss = wave_sum(x * x);
    if ((e & 63) == 0) red[e >> 6] = ss;
    __syncthreads();
    const float rs = 1.0f / sqrtf((red[0] + red[1]) / (float)kDk + eps);
    out[row * kDk + e] = x * rs * wnorm[e] * silu(z[row * kDk + e]);
}

}  // namespace

size_t deltanet_prefill_work_bytes(const Dims& d, int T) {
    return work_floats(d, T, (T + CH - 1) / CH) * sizeof(float);
}

hipError_t launch_deltanet_prefill(q35m_ctx* c, int layer, int seq, int T, const float* qkv,
                                   const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    const int nch = (T + CH - 1) / CH;
    PrefillWork w = carve(c->work, d, T, nch);
    float* state = L.state + (size_t)seq * d.nv * kDk * kDk;
    float* cs = L.conv + (size_t)seq * d.conv_dim * kConvState;
    hipError_t e;
    {
        ProfScope ps_(c, K_DN_PREFILL_PREP);
        hipLaunchKernelGGL(deltanet_prefill_prep, dim3(T, 2 * d.nk + d.nv), dim3(kDk), 0,
                           c->stream, qkv, b, a, L.conv_w, L.ssm_a, L.dt_bias, w, T, d.nk, d.nv,
                           d.eps);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CONV_WRITEBACK);
        hipLaunchKernelGGL(deltanet_conv_writeback, dim3((d.conv_dim + 255) / 256), dim3(256), 0,
                           c->stream, qkv, L.conv_w, cs, T, d.conv_dim);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CHUNK_PREP);
        hipLaunchKernelGGL(dn_chunk_prep, dim3(d.nk * nch), dim3(256), 0, c->stream, w, T, d.nk,
                           d.nv, nch);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CHUNK_SCAN);
        hipLaunchKernelGGL(dn_chunk_scan, dim3(d.nv * 8), dim3(256), 0, c->stream, w, state, T,
                           d.nk, d.nv, nch);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_GATED_NORM);
        hipLaunchKernelGGL(deltanet_gated_norm, dim3((unsigned)T * d.nv), dim3(kDk), 0, c->stream,
                           w.core, z, L.ssm_norm, out, d.eps);
    }
    return hipGetLastError();
}

}  // namespace q35
