// Gated-DeltaNet decode mixer, one token per sequence, fused into one launch:
// conv-window update + SiLU, q/k L2 norm, beta/decay gates, one delta-rule
// step of the fp32 state, gated RMSNorm.
//
// Reference: Qwen35Model.DecodeLinearAttn steps 2-6
// (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:348-397) over
// GatedDeltaNetOps.CausalConv1dUpdate (GatedDeltaNetOps.cs:64-91),
// RecurrentGatedDeltaRule/DeltaStep (GatedDeltaNetOps.cs:107-229) and
// Qwen35Ops.GatedRmsNorm (Qwen35Ops.cs:74-111).
//
// Work split.  One workgroup per (sequence, k-head) owns everything that k-head
// touches: the q/k conv channels of the k-head, and the R = H_v/H_k v-heads that
// read them (their value channels and their [128][128] states, R * 64 KiB).
// Every conv window therefore has exactly one reader and one writer, the gated
// norm sees a whole head, and no two workgroups exchange data.  Each v-head
// gets 256 threads; a thread holds 4 columns x 16 rows of its head's state in
// registers, so the state streams through HBM exactly once (read, then write).
//
// One step of the delta rule, with decay a = exp(g):
//   S' = a S + k delta^T,  delta = beta (v - a S^T k),  o = S'^T q
//      = a S^T q + (q.k) delta
// so one pass over S yields both dot products and the update.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int TPH = 256;      // threads per v-head

__device__ __forceinline__ float conv_update_tap(const float* __restrict__ conv_w,
                                                 const float* __restrict__ cs,
                                                 const float* __restrict__ x, int c,
                                                 int conv_dim) {
    // CausalConv1dUpdate: taps 0..2 multiply the window (oldest first), tap 3
    // the new input (GatedDeltaNetOps.cs:79-84).
    const float* cc = cs + (size_t)c * kConvState;
    float acc = conv_w[c] * cc[0];
    acc += conv_w[conv_dim + c] * cc[1];
    acc += conv_w[2 * conv_dim + c] * cc[2];
    acc += conv_w[3 * conv_dim + c] * x[c];
    return silu(acc);
}

__device__ __forceinline__ void conv_shift(float* __restrict__ cs, const float* __restrict__ x,
                                           int c) {
    float* cc = cs + (size_t)c * kConvState;
    const float c1 = cc[1], c2 = cc[2];
    cc[0] = c1;
    cc[1] = c2;
    cc[2] = x[c];
}

// kMaxR bounds R = H_v/H_k (2: 512 threads, no register pressure; 4: 1024).
template <int kMaxR>
__global__ __launch_bounds__(TPH * kMaxR) void deltanet_decode_kernel(
    const float* __restrict__ qkv, const float* __restrict__ zin, const float* __restrict__ bin,
    const float* __restrict__ ain, float* __restrict__ out, const float* __restrict__ conv_w,
    const float* __restrict__ ssm_a, const float* __restrict__ dt_bias,
    const float* __restrict__ ssm_norm, float* __restrict__ state, float* __restrict__ conv,
    int nk, int nv, float eps, SeqBatch sb) {
    const int R = nv / nk;
    const int i = blockIdx.x / nk, kh = blockIdx.x % nk;
    const int key_dim = nk * kDk, value_dim = nv * kDk, conv_dim = 2 * key_dim + value_dim;
    const int seq = sb.seq[i];
    const int t = threadIdx.x;
    const int rr = t / TPH, tid = t % TPH;          // v-head within the group, thread in head
    const int lane = t & 63, wave = tid >> 6;       // wave within the head (0..3)
    const int vh = kh * R + rr;

    float* S = state + ((size_t)seq * nv + vh) * kDk * kDk;
    float* cs = conv + (size_t)seq * conv_dim * kConvState;
    const float* x = qkv + (size_t)i * conv_dim;

    // Thread owns columns 4*c4..4*c4+3 of rows rg + 8j, j = 0..15; a wave's
    // load covers two full 512-byte rows.  Issued first to overlap the conv.
    const int c4 = tid & 31, rg = tid >> 5;
    float4 s[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        s[j] = *reinterpret_cast<const float4*>(S + (size_t)(rg + 8 * j) * kDk + 4 * c4);

    __shared__ float qk_s[2 * kDk];            // SiLU(conv) of q (0..127) and k (128..255)
    __shared__ float v_s[kMaxR][kDk];
    __shared__ float gates[kMaxR][2];
    __shared__ float red[4][2];
    __shared__ float colred[kMaxR][4][kDk][2];
    __shared__ float o_s[kMaxR][kDk];
    __shared__ float nred[kMaxR][2];

    const int qk_c = t < kDk ? kh * kDk + t : key_dim + kh * kDk + (t - kDk);
    const int v_c = 2 * key_dim + vh * kDk + tid;
    if (t < 2 * kDk) qk_s[t] = conv_update_tap(conv_w, cs, x, qk_c, conv_dim);
    if (tid < kDk) v_s[rr][tid] = conv_update_tap(conv_w, cs, x, v_c, conv_dim);
    if (tid == 0) {
        // beta = sigmoid(b), g = ssm_a * softplus(a + dt_bias) (Decode.cs:378-386)
        gates[rr][0] = 1.0f / (1.0f + expf(-bin[(size_t)i * nv + vh]));
        const float g = ssm_a[vh] * softplus_ref(ain[(size_t)i * nv + vh] + dt_bias[vh]);
        gates[rr][1] = expf(g);
    }
    __syncthreads();

    // L2 norms of q and k, and q.k (GatedDeltaNetOps.cs:144-151), by the
    // first four waves of the workgroup.
    if (t < 2 * kDk) {
        float a0, a1 = 0.0f;
        if (t < kDk) {
            const float qv = qk_s[t];
            a0 = qv * qv;
            a1 = qv * qk_s[kDk + t];
        } else {
            const float kv = qk_s[t];
            a0 = kv * kv;
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if (lane == 0) {
            red[t >> 6][0] = a0;
            red[t >> 6][1] = a1;
        }
    }
    __syncthreads();
    const float q_scale = (1.0f / sqrtf((float)kDk)) / sqrtf(red[0][0] + red[1][0] + eps);
    const float k_scale = 1.0f / sqrtf(red[2][0] + red[3][0] + eps);
    const float qk = (red[0][1] + red[1][1]) * q_scale * k_scale;
    const float beta = gates[rr][0], decay = gates[rr][1];

    // Partial S^T k and S^T q over this thread's 16 rows.
    float kvp[4] = {0.f, 0.f, 0.f, 0.f}, sqp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int a = rg + 8 * j;
        const float qa = qk_s[a] * q_scale, ka = qk_s[kDk + a] * k_scale;
        kvp[0] += s[j].x * ka; kvp[1] += s[j].y * ka; kvp[2] += s[j].z * ka; kvp[3] += s[j].w * ka;
        sqp[0] += s[j].x * qa; sqp[1] += s[j].y * qa; sqp[2] += s[j].z * qa; sqp[3] += s[j].w * qa;
    }
    // rg = 2*wave + (lane >> 5): fold the two row groups of a wave, then the waves.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        kvp[c] += __shfl_xor(kvp[c], 32, kWave);
        sqp[c] += __shfl_xor(sqp[c], 32, kWave);
    }
    if (lane < 32)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            colred[rr][wave][4 * c4 + c][0] = kvp[c];
            colred[rr][wave][4 * c4 + c][1] = sqp[c];
        }
    __syncthreads();

    float delta[4], o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = 4 * c4 + c;
        const float kv = colred[rr][0][col][0] + colred[rr][1][col][0] + colred[rr][2][col][0] +
                         colred[rr][3][col][0];
        const float sq = colred[rr][0][col][1] + colred[rr][1][col][1] + colred[rr][2][col][1] +
                         colred[rr][3][col][1];
        delta[c] = beta * (v_s[rr][col] - decay * kv);
        o[c] = decay * sq + qk * delta[c];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float ka = qk_s[kDk + rg + 8 * j] * k_scale;
        float4 n;
        n.x = decay * s[j].x + ka * delta[0];
        n.y = decay * s[j].y + ka * delta[1];
        n.z = decay * s[j].z + ka * delta[2];
        n.w = decay * s[j].w + ka * delta[3];
        *reinterpret_cast<float4*>(S + (size_t)(rg + 8 * j) * kDk + 4 * c4) = n;
    }
    if (rg == 0)
#pragma unroll
        for (int c = 0; c < 4; ++c) o_s[rr][4 * c4 + c] = o[c];
    __syncthreads();

    // Gated RMSNorm of each head (plain weight, Qwen35Ops.cs:98-110).
    const float ov = tid < kDk ? o_s[rr][tid] : 0.0f;
    const float ss = wave_sum(ov * ov);
    if (lane == 0 && wave < 2) nred[rr][wave] = ss;
    // Advance the conv windows (GatedDeltaNetOps.cs:86-89): every read of them
    // happened before the first barrier.
    if (t < 2 * kDk) conv_shift(cs, x, qk_c);
    if (tid < kDk) conv_shift(cs, x, v_c);
    __syncthreads();
    if (tid < kDk) {
        const float rs = 1.0f / sqrtf((nred[rr][0] + nred[rr][1]) / (float)kDk + eps);
        const size_t off = (size_t)i * value_dim + (size_t)vh * kDk + tid;
        out[off] = ov * rs * ssm_norm[tid] * silu(zin[off]);
    }
}

}  // namespace

hipError_t launch_deltanet_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* qkv,
                                  const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    const int R = d.nv / d.nk;
    {
        ProfScope ps_(c, K_DN_DECODE);
        if (R <= 2)
            hipLaunchKernelGGL(deltanet_decode_kernel<2>, dim3(sb.n * d.nk), dim3(TPH * R), 0,
                               c->stream, qkv, z, b, a, out, L.conv_w, L.ssm_a, L.dt_bias,
                               L.ssm_norm, L.state, L.conv, d.nk, d.nv, d.eps, sb);
        else
            hipLaunchKernelGGL(deltanet_decode_kernel<4>, dim3(sb.n * d.nk), dim3(TPH * R), 0,
                               c->stream, qkv, z, b, a, out, L.conv_w, L.ssm_a, L.dt_bias,
                               L.ssm_norm, L.state, L.conv, d.nk, d.nv, d.eps, sb);
    }
    return hipGetLastError();
}

}  // namespace q35
