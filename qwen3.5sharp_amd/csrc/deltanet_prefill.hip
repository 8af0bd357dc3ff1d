// Gated-DeltaNet prefill mixer for T tokens of one sequence.
//
// Reference: Qwen35Model.PrefillLinearAttn steps 2-6
// (src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:181-260).
//
//  1. deltanet_prefill_prep: zero-padded causal conv with the prefill tap
//     order (tap j multiplies x[t-j], GatedDeltaNetOps.cs:27-53) + SiLU,
//     read straight from the token-major qkv (no transpose), q/k L2 norm
//     (q also scaled by 1/sqrt(dk)), beta = sigmoid(b), g = ssm_a *
//     softplus(a + dt_bias) (Prefill.cs:239-248).
//  2. deltanet_conv_writeback: conv window <- last K-1 raw inputs
//     (Prefill.cs:192-204), reproducing the reference's read past the
//     channel row when T < K-1.
//  3. deltanet_prefill_scan: the delta rule over the T tokens from the
//     sequence's current state, one workgroup per (v-head, 32-column tile)
//     with the state tile held in registers for the whole sequence.
//  4. deltanet_gated_norm: gated RMSNorm per (token, v-head) row.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int TB = 32;
constexpr int NSPLIT = kDk / TB;
constexpr int NT = 256;

struct PrefillWork {
    float* qhat;   // [T][nk][dk]  L2-normed, scaled by 1/sqrt(dk)
    float* khat;   // [T][nk][dk]
    float* vv;     // [T][nv][dv]
    float* beta;   // [T][nv]
    float* decay;  // [T][nv]   exp(g)
    float* gl;     // [T][nv]   g (log decay)
    float* core;   // [T][nv][dv] pre-norm recurrence output
};

PrefillWork carve(float* w, const Dims& d, int T) {
    PrefillWork p;
    p.qhat = w;
    p.khat = p.qhat + (size_t)T * d.key_dim;
    p.vv = p.khat + (size_t)T * d.key_dim;
    p.beta = p.vv + (size_t)T * d.value_dim;
    p.decay = p.beta + (size_t)T * d.nv;
    p.gl = p.decay + (size_t)T * d.nv;
    p.core = p.gl + (size_t)T * d.nv;
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
            const float g = ssm_a[vh] * softplus_ref(ain[gi] + dt_bias[vh]);
            w.gl[gi] = g;
            w.decay[gi] = expf(g);
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

__global__ __launch_bounds__(NT) void deltanet_prefill_scan(PrefillWork w,
                                                            float* __restrict__ state, int T,
                                                            int nk, int nv) {
    const int vh = blockIdx.x / NSPLIT, b0 = (blockIdx.x % NSPLIT) * TB;
    const int kh = vh / (nv / nk);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c4 = tid & 7, rg = tid >> 3;
    float* S = state + (size_t)vh * kDk * kDk;
    float4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        s[j] = *reinterpret_cast<const float4*>(S + (size_t)(rg + 32 * j) * kDk + b0 + 4 * c4);

    __shared__ float colred[2][4][TB][2];
    __shared__ float qkred[2][4];

    auto load_tok = [&](int t, float* qa, float* ka, float4& v4, float& beta, float& decay) {
        const float* qh = w.qhat + ((size_t)t * nk + kh) * kDk;
        const float* kk = w.khat + ((size_t)t * nk + kh) * kDk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qa[j] = qh[rg + 32 * j];
            ka[j] = kk[rg + 32 * j];
        }
        v4 = *reinterpret_cast<const float4*>(w.vv + ((size_t)t * nv + vh) * kDk + b0 + 4 * c4);
        beta = w.beta[(size_t)t * nv + vh];
        decay = w.decay[(size_t)t * nv + vh];
    };

    float qa[4], ka[4], beta, decay;
    float4 v4;
    load_tok(0, qa, ka, v4, beta, decay);
    for (int t = 0; t < T; ++t) {
        float nqa[4], nka[4], nbeta = 0.f, ndecay = 0.f;
        float4 nv4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t + 1 < T) load_tok(t + 1, nqa, nka, nv4, nbeta, ndecay);
        const int buf = t & 1;
        float kvp[4] = {0.f, 0.f, 0.f, 0.f}, sqp[4] = {0.f, 0.f, 0.f, 0.f}, qkp = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kvp[0] += s[j].x * ka[j]; kvp[1] += s[j].y * ka[j]; kvp[2] += s[j].z * ka[j]; kvp[3] += s[j].w * ka[j];
            sqp[0] += s[j].x * qa[j]; sqp[1] += s[j].y * qa[j]; sqp[2] += s[j].z * qa[j]; sqp[3] += s[j].w * qa[j];
            qkp += qa[j] * ka[j];
        }
#pragma unroll
        for (int o = 8; o < 64; o <<= 1) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                kvp[c] += __shfl_xor(kvp[c], o, kWave);
                sqp[c] += __shfl_xor(sqp[c], o, kWave);
            }
            qkp += __shfl_xor(qkp, o, kWave);
        }
        if (lane < 8)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                colred[buf][wave][4 * lane + c][0] = kvp[c];
                colred[buf][wave][4 * lane + c][1] = sqp[c];
            }
        if (lane == 0) qkred[buf][wave] = qkp;
        __syncthreads();
        const float qk = qkred[buf][0] + qkred[buf][1] + qkred[buf][2] + qkred[buf][3];
        const float vvals[4] = {v4.x, v4.y, v4.z, v4.w};
        float delta[4], o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = 4 * c4 + c;
            const float kv = colred[buf][0][col][0] + colred[buf][1][col][0] + colred[buf][2][col][0] + colred[buf][3][col][0];
            const float sq = colred[buf][0][col][1] + colred[buf][1][col][1] + colred[buf][2][col][1] + colred[buf][3][col][1];
            delta[c] = beta * (vvals[c] - decay * kv);
            o[c] = decay * sq + qk * delta[c];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j].x = decay * s[j].x + ka[j] * delta[0];
            s[j].y = decay * s[j].y + ka[j] * delta[1];
            s[j].z = decay * s[j].z + ka[j] * delta[2];
            s[j].w = decay * s[j].w + ka[j] * delta[3];
        }
        if (rg == 0)
            *reinterpret_cast<float4*>(w.core + ((size_t)t * nv + vh) * kDk + b0 + 4 * c4) =
                make_float4(o[0], o[1], o[2], o[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qa[j] = nqa[j];
            ka[j] = nka[j];
        }
        v4 = nv4;
        beta = nbeta;
        decay = ndecay;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(S + (size_t)(rg + 32 * j) * kDk + b0 + 4 * c4) = s[j];
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
    return (size_t)T * (2 * d.key_dim + 2 * d.value_dim + 3 * d.nv) * sizeof(float);
}

hipError_t launch_deltanet_prefill(q35m_ctx* c, int layer, int seq, int T, const float* qkv,
                                   const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    PrefillWork w = carve(c->work, d, T);
    float* state = L.state + (size_t)seq * d.nv * kDk * kDk;
    float* cs = L.conv + (size_t)seq * d.conv_dim * kConvState;
    {
        ProfScope ps_(c, K_DN_PREFILL_PREP);
        hipLaunchKernelGGL(deltanet_prefill_prep, dim3(T, 2 * d.nk + d.nv), dim3(kDk), 0, c->stream, qkv,
                           b, a, L.conv_w, L.ssm_a, L.dt_bias, w, T, d.nk, d.nv, d.eps);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CONV_WRITEBACK);
        hipLaunchKernelGGL(deltanet_conv_writeback, dim3((d.conv_dim + 255) / 256), dim3(256), 0,
                           c->stream, qkv, L.conv_w, cs, T, d.conv_dim);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_PREFILL_SCAN);
        hipLaunchKernelGGL(deltanet_prefill_scan, dim3(d.nv * NSPLIT), dim3(NT), 0, c->stream, w, state,
                           T, d.nk, d.nv);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_GATED_NORM);
        hipLaunchKernelGGL(deltanet_gated_norm, dim3((unsigned)T * d.nv), dim3(kDk), 0, c->stream,
                           w.core, z, L.ssm_norm, out, d.eps);
    }
    return hipGetLastError();
}

}  // namespace q35
