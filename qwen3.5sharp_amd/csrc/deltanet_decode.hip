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
// Work split.  The delta rule is separable over dv columns: kv[b], delta[b]
// and S[:, b] depend on column b only.  A workgroup owns one 32-column tile
// of one v-head's state (128 rows x 32 cols = 16 KiB), read once into
// registers and written once, so the state streams through HBM exactly once.
// The R = H_v/H_k v-heads that share a k-head and their 4 column tiles form a
// group of 8 workgroups; they all need the k-head's q/k conv outputs, which
// each recomputes (256 channels, L2-resident).  The group is placed on one XCD.
//
// Cross-workgroup steps (the gated norm needs all 128 outputs of a head; the
// shared q/k conv window needs exactly one writer, after every reader) are
// done by the last workgroup of the group to arrive at a completion counter.
// Each member publishes its outputs, fences, then increments; the member that
// sees count == 8-1 resets the counter, normalises the group's outputs and
// shifts the group's conv windows.  Every member has read its conv inputs
// before it increments, so the shift cannot race a reader.
//
// One step of the delta rule, with decay a = exp(g):
//   S' = a S + k delta^T,  delta = beta (v - a S^T k),  o = S'^T q
//      = a S^T q + (q.k) delta
// so one pass over S yields both dot products and the update.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int TB = 32;             // dv columns per workgroup
constexpr int NSPLIT = kDk / TB;   // column tiles per head
constexpr int NT = 256;            // threads per workgroup

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
    float c1 = cc[1], c2 = cc[2];
    cc[0] = c1;
    cc[1] = c2;
    cc[2] = x[c];
}

__global__ __launch_bounds__(NT) void deltanet_decode_kernel(
    const float* __restrict__ qkv, const float* __restrict__ zin, const float* __restrict__ bin,
    const float* __restrict__ ain, float* __restrict__ out, const float* __restrict__ conv_w,
    const float* __restrict__ ssm_a, const float* __restrict__ dt_bias,
    const float* __restrict__ ssm_norm, float* __restrict__ state, float* __restrict__ conv,
    unsigned* __restrict__ counters, int nk, int nv, float eps, SeqBatch sb) {
    const int R = nv / nk;
    const int M = R * NSPLIT;
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int group = L / M, member = L % M;
    const int i = group / nk, kh = group % nk;
    const int vh = kh * R + member / NSPLIT;
    const int b0 = (member % NSPLIT) * TB;
    const int key_dim = nk * kDk, value_dim = nv * kDk, conv_dim = 2 * key_dim + value_dim;
    const int seq = sb.seq[i];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    float* S = state + ((size_t)seq * nv + vh) * kDk * kDk;
    float* cs = conv + (size_t)seq * conv_dim * kConvState;
    const float* x = qkv + (size_t)i * conv_dim;

    // Thread owns columns b0 + 4*c4 .. +3 of rows rg, rg+32, rg+64, rg+96.
    // The state loads go out first so their latency overlaps the conv work.
    const int c4 = tid & 7, rg = tid >> 3;
    float4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        s[j] = *reinterpret_cast<const float4*>(S + (size_t)(rg + 32 * j) * kDk + b0 + 4 * c4);

    __shared__ float qk_s[2 * kDk];     // SiLU(conv) of q (0..127) and k (128..255)
    __shared__ float v_s[TB];
    __shared__ float red[4][2];
    __shared__ float colred[4][TB][2];
    __shared__ float gates[2];
    __shared__ unsigned last_flag;

    {
        const int c = tid < kDk ? kh * kDk + tid : key_dim + kh * kDk + (tid - kDk);
        qk_s[tid] = conv_update_tap(conv_w, cs, x, c, conv_dim);
    }
    if (tid < TB) v_s[tid] = conv_update_tap(conv_w, cs, x, 2 * key_dim + vh * kDk + b0 + tid,
                                            conv_dim);
    if (tid == 0) {
        // beta = sigmoid(b), g = ssm_a * softplus(a + dt_bias) (Decode.cs:378-386)
        gates[0] = 1.0f / (1.0f + expf(-bin[(size_t)i * nv + vh]));
        float g = ssm_a[vh] * softplus_ref(ain[(size_t)i * nv + vh] + dt_bias[vh]);
        gates[1] = expf(g);
    }
    __syncthreads();

    // L2 norms of q and k, and q.k (GatedDeltaNetOps.cs:144-151).
    {
        float a0, a1 = 0.0f;
        if (tid < kDk) {
            float qv = qk_s[tid];
            a0 = qv * qv;
            a1 = qv * qk_s[kDk + tid];
        } else {
            float kv = qk_s[tid];
            a0 = kv * kv;
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if (lane == 0) {
            red[wave][0] = a0;
            red[wave][1] = a1;
        }
    }
    __syncthreads();
    const float qn = red[0][0] + red[1][0];
    const float qk_raw = red[0][1] + red[1][1];
    const float kn = red[2][0] + red[3][0];
    const float q_scale = (1.0f / sqrtf((float)kDk)) / sqrtf(qn + eps);
    const float k_scale = 1.0f / sqrtf(kn + eps);
    const float qk = qk_raw * q_scale * k_scale;
    const float beta = gates[0], decay = gates[1];

    // Partial S^T k and S^T q over this thread's 4 rows.
    float kvp[4] = {0.f, 0.f, 0.f, 0.f}, sqp[4] = {0.f, 0.f, 0.f, 0.f}, kr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int a = rg + 32 * j;
        const float qa = qk_s[a] * q_scale, ka = qk_s[kDk + a] * k_scale;
        kr[j] = ka;
        kvp[0] += s[j].x * ka; kvp[1] += s[j].y * ka; kvp[2] += s[j].z * ka; kvp[3] += s[j].w * ka;
        sqp[0] += s[j].x * qa; sqp[1] += s[j].y * qa; sqp[2] += s[j].z * qa; sqp[3] += s[j].w * qa;
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            kvp[c] += __shfl_xor(kvp[c], o, kWave);
            sqp[c] += __shfl_xor(sqp[c], o, kWave);
        }
    if (lane < 8)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            colred[wave][4 * lane + c][0] = kvp[c];
            colred[wave][4 * lane + c][1] = sqp[c];
        }
    __syncthreads();

    float delta[4], o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = 4 * c4 + c;
        const float kv = colred[0][col][0] + colred[1][col][0] + colred[2][col][0] + colred[3][col][0];
        const float sq = colred[0][col][1] + colred[1][col][1] + colred[2][col][1] + colred[3][col][1];
        delta[c] = beta * (v_s[col] - decay * kv);
        o[c] = decay * sq + qk * delta[c];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float4 n;
        n.x = decay * s[j].x + kr[j] * delta[0];
        n.y = decay * s[j].y + kr[j] * delta[1];
        n.z = decay * s[j].z + kr[j] * delta[2];
        n.w = decay * s[j].w + kr[j] * delta[3];
        *reinterpret_cast<float4*>(S + (size_t)(rg + 32 * j) * kDk + b0 + 4 * c4) = n;
    }
    float* orow = out + (size_t)i * value_dim + (size_t)vh * kDk + b0;
    if (rg == 0) *reinterpret_cast<float4*>(orow + 4 * c4) = make_float4(o[0], o[1], o[2], o[3]);

    // Publish, then count arrivals; the last member finishes the group.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(&counters[i * nk + kh], 1u);
        last_flag = (prev == (unsigned)(M - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    if (tid == 0) atomicExch(&counters[i * nk + kh], 0u);

    // Gated RMSNorm over each of the R heads (plain weight, Qwen35Ops.cs:98-110).
    __shared__ float nred[4];
    for (int hb = 0; hb < R; hb += 2) {
        const int hr = hb + (tid >> 7);
        const bool valid = hr < R;
        const int e = tid & 127;
        const size_t off = (size_t)i * value_dim + (size_t)(kh * R + hr) * kDk + e;
        const float ov = valid ? load_coherent(out + off) : 0.0f;
        const float ss = wave_sum(ov * ov);
        if (lane == 0) nred[wave] = ss;
        __syncthreads();
        const float tot = nred[wave & ~1] + nred[wave | 1];
        const float rs = 1.0f / sqrtf(tot / (float)kDk + eps);
        if (valid) out[off] = ov * rs * ssm_norm[e] * silu(zin[off]);
        __syncthreads();
    }

    // Advance the conv windows of the group's channels (GatedDeltaNetOps.cs:86-89).
    conv_shift(cs, x, tid < kDk ? kh * kDk + tid : key_dim + kh * kDk + (tid - kDk));
    for (int idx = tid; idx < R * kDk; idx += NT) conv_shift(cs, x, 2 * key_dim + kh * R * kDk + idx);
}

}  // namespace

hipError_t launch_deltanet_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* qkv,
                                  const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    const int R = d.nv / d.nk;
    const int blocks = sb.n * d.nk * R * NSPLIT;
    {
        ProfScope ps_(c, K_DN_DECODE);
        hipLaunchKernelGGL(deltanet_decode_kernel, dim3(blocks), dim3(NT), 0, c->stream, qkv, z, b, a,
                           out, L.conv_w, L.ssm_a, L.dt_bias, L.ssm_norm, L.state, L.conv, c->counters,
                           d.nk, d.nv, d.eps, sb);
    }
    return hipGetLastError();
}

}  // namespace q35
