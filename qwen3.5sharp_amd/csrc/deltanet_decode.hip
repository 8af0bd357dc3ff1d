// Gated-DeltaNet decode mixer, one token per sequence: conv-window update +
// SiLU, q/k L2 norm, beta/decay gates, one delta-rule step of the fp32 state,
// gated RMSNorm.
//
// Reference: Qwen35Model.DecodeLinearAttn steps 2-6
// (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:348-397) over
// GatedDeltaNetOps.CausalConv1dUpdate (GatedDeltaNetOps.cs:64-91),
// RecurrentGatedDeltaRule/DeltaStep (GatedDeltaNetOps.cs:107-229) and
// Qwen35Ops.GatedRmsNorm (Qwen35Ops.cs:74-111).
//
// Work split.  One workgroup of 256 threads per (sequence, v-head) streams the
// head's [128][128] fp32 state through HBM exactly once (read, then write,
// both non-temporal: the states of a stack of layers and sequences do not fit
// the MALL, and kept out of it they leave it to the KV rows of the attention
// layers) from registers: a thread holds 4 columns x 16 rows.  Each workgroup
// recomputes the conv + L2 norms of the 256 q/k channels of its k-head (a few
// KiB, cache resident, shared by the H_v/H_k v-heads of the k-head) and owns
// the 128 value channels of its head; the gated norm needs only the head.
// The conv operands are loaded before the state so that the conv, the norms
// and the gates run while the state is in flight.
//
// Conv windows: the q/k windows of a k-head are held once per v-head that
// shares it (copy vh % R; copy 0 is the reference layout's), so each
// workgroup reads and rewrites only windows that no other workgroup touches,
// in place.  Inside the workgroup, the shifted windows are stored after the
// first barrier, by which point every thread has consumed its window loads
// (threads 128-255 also read value channel 127, whose window thread 127
// rewrites).  Nothing about the windows depends on the host or on a step
// count, so a captured step replays correctly any number of times.
//
// Column slices of a head (more, smaller workgroups) were measured slower at
// batch 1 and 8: the gated norm then needs a second launch.
//
// One step of the delta rule, with decay a = exp(g):
//   S' = a S + k delta^T,  delta = beta (v - a S^T k),  o = S'^T q
//      = a S^T q + (q.k) delta
// so one pass over S yields both dot products and the update.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int NT = 256;

// Operands of one channel's CausalConv1dUpdate (GatedDeltaNetOps.cs:64-91):
// the 3-sample window (oldest first), the 4 taps and the new input.
struct ConvOperands {
    float w0, w1, w2, w3, c0, c1, c2, x;
};

__device__ __forceinline__ ConvOperands conv_load(const float* __restrict__ conv_w,
                                                  const float* __restrict__ win,
                                                  const float* __restrict__ x, int c,
                                                  int conv_dim) {
    const float* cc = win + (size_t)c * kConvState;
    return {conv_w[c], conv_w[conv_dim + c], conv_w[2 * conv_dim + c], conv_w[3 * conv_dim + c],
            cc[0],     cc[1],                cc[2],                    x[c]};
}

// Taps 0..2 multiply the window, tap 3 the new input (GatedDeltaNetOps.cs:79-84).
__device__ __forceinline__ float conv_out(const ConvOperands& o) {
    float acc = o.w0 * o.c0;
    acc += o.w1 * o.c1;
    acc += o.w2 * o.c2;
    acc += o.w3 * o.x;
    return silu(acc);
}

// Window shift (GatedDeltaNetOps.cs:86-89), in place.
__device__ __forceinline__ void conv_shift(const ConvOperands& o, float* __restrict__ win, int c) {
    float* dd = win + (size_t)c * kConvState;
    dd[0] = o.c1;
    dd[1] = o.c2;
    dd[2] = o.x;
}

__global__ __launch_bounds__(NT) void deltanet_decode_kernel(
    const float* __restrict__ qkv, const float* __restrict__ zin, const float* __restrict__ bin,
    const float* __restrict__ ain, float* __restrict__ out, const float* __restrict__ conv_w,
    const float* __restrict__ ssm_a, const float* __restrict__ dt_bias,
    const float* __restrict__ ssm_norm, float* __restrict__ state, float* __restrict__ conv,
    int nk, int nv, float eps, SeqBatch sb) {
    constexpr int C4N = kDk / 4;      // float4 columns
    constexpr int RG = NT / C4N;      // row groups
    constexpr int RPT = kDk / RG;     // rows per thread
    const int vh = blockIdx.x % nv;
    const int i = blockIdx.x / nv;
    const int R = nv / nk, kh = vh / R, rep = vh % R;
    const int key_dim = nk * kDk, value_dim = nv * kDk, conv_dim = 2 * key_dim + value_dim;
    const int seq = sb.seq[i];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c4 = t % C4N, rg = t / C4N;

    float* S = state + ((size_t)seq * nv + vh) * kDk * kDk;
    // This sequence's window block; the q/k windows of copy `rep`.
    float* win = conv + (size_t)seq * ((size_t)conv_dim + (size_t)(R - 1) * 2 * key_dim) * kConvState;
    float* win_qk = rep == 0 ? win : win + ((size_t)conv_dim + (size_t)(rep - 1) * 2 * key_dim) * kConvState;
    const float* x = qkv + (size_t)i * conv_dim;

    __shared__ float qk_s[2 * kDk];            // SiLU(conv) of q (0..127) and k (128..255)
    __shared__ float v_s[kDk];
    __shared__ float red[4][2];
    __shared__ float colred[4][kDk][2];

    // Load order: the small conv and gate operands first, then the state
    // of the head, so the conv, norms and gates are computed while it is
    // still in flight (the barriers before its first use wait on LDS only).
    const int qk_c = t < kDk ? kh * kDk + t : key_dim + kh * kDk + (t - kDk);
    const int v_c = 2 * key_dim + vh * kDk + min(t, kDk - 1);
    const ConvOperands oq = conv_load(conv_w, win_qk, x, qk_c, conv_dim);
    const ConvOperands ov = conv_load(conv_w, win, x, v_c, conv_dim);
    const float b_in = bin[(size_t)i * nv + vh], a_in = ain[(size_t)i * nv + vh];
    const float sa = ssm_a[vh], dtb = dt_bias[vh];
    // Operands of the gated norm at the end: channels 4 c4 .. 4 c4 + 3 (used
    // by the first row group, loaded by every thread).
    const size_t o_off = (size_t)i * value_dim + (size_t)vh * kDk + 4 * c4;
    const float4 z4 = *reinterpret_cast<const float4*>(zin + o_off);
    const float4 nw4 = *reinterpret_cast<const float4*>(ssm_norm + 4 * c4);

    // Thread owns columns 4*c4 .. +3 of rows rg + RG*j.  The loads stay in
    // row order (the scheduler may not reorder them across the barriers), so
    // the products below can start on the first rows while later ones are
    // still arriving.
    float4 s[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        s[j] = load_nt(S + (size_t)(rg + RG * j) * kDk + 4 * c4);
        __builtin_amdgcn_sched_barrier(0);
    }

    qk_s[t] = conv_out(oq);
    // Threads t >= 128 recompute the head's last value channel and store the
    // same value: an unconditional store keeps its loads ahead of the state's.
    v_s[min(t, kDk - 1)] = conv_out(ov);
    // beta = sigmoid(b), decay = exp(ssm_a * softplus(a + dt_bias))
    // (Decode.cs:378-386); uniform, computed by every thread.
    const float beta = 1.0f / (1.0f + expf(-b_in));
    const float decay = expf(sa * softplus_ref(a_in + dtb));
    lds_barrier();
    // Every thread's window loads are consumed (their conv outputs are in
    // LDS), so the windows are rewritten in place: this workgroup's q/k copy
    // and its head's value windows, one thread per channel.
    conv_shift(oq, win_qk, qk_c);
    if (t < kDk) conv_shift(ov, win, v_c);

    // L2 norms of q and k, and q.k (GatedDeltaNetOps.cs:144-151): waves 0-1
    // hold q, waves 2-3 hold k.  Their sums go to LDS beside the column sums
    // below, behind the same barrier.
    {
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
            red[wave][0] = a0;
            red[wave][1] = a1;
        }
    }

    // Partial S^T k and S^T q over this thread's rows, on the conv outputs
    // before the norms (so they do not wait for the norms' reduction): the
    // scales apply to the column sums, S^T (s k) = s (S^T k).
    float kvp[4] = {0.f, 0.f, 0.f, 0.f}, sqp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int a = rg + RG * j;
        const float qa = qk_s[a], ka = qk_s[kDk + a];
        kvp[0] += s[j].x * ka; kvp[1] += s[j].y * ka; kvp[2] += s[j].z * ka; kvp[3] += s[j].w * ka;
        sqp[0] += s[j].x * qa; sqp[1] += s[j].y * qa; sqp[2] += s[j].z * qa; sqp[3] += s[j].w * qa;
    }
    // Lanes c4 + C4N*r of a wave share columns: fold them, then the waves.
#pragma unroll
    for (int m = C4N; m < kWave; m <<= 1)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            kvp[c] += __shfl_xor(kvp[c], m, kWave);
            sqp[c] += __shfl_xor(sqp[c], m, kWave);
        }
    if (lane < C4N)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            colred[wave][4 * c4 + c][0] = kvp[c];
            colred[wave][4 * c4 + c][1] = sqp[c];
        }
    lds_barrier();
    const float q_scale = (1.0f / sqrtf((float)kDk)) / sqrtf(red[0][0] + red[1][0] + eps);
    const float k_scale = 1.0f / sqrtf(red[2][0] + red[3][0] + eps);
    const float qk = (red[0][1] + red[1][1]) * q_scale * k_scale;

    float delta[4], o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = 4 * c4 + c;
        const float kv = (colred[0][col][0] + colred[1][col][0] + colred[2][col][0] + colred[3][col][0]) * k_scale;
        const float sq = (colred[0][col][1] + colred[1][col][1] + colred[2][col][1] + colred[3][col][1]) * q_scale;
        delta[c] = beta * (v_s[col] - decay * kv);
        o[c] = decay * sq + qk * delta[c];
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const float ka = qk_s[kDk + rg + RG * j] * k_scale;
        float4 n;
        n.x = decay * s[j].x + ka * delta[0];
        n.y = decay * s[j].y + ka * delta[1];
        n.z = decay * s[j].z + ka * delta[2];
        n.w = decay * s[j].w + ka * delta[3];
        store_nt(S + (size_t)(rg + RG * j) * kDk + 4 * c4, n);
    }

    // Gated RMSNorm of the head (plain weight, Qwen35Ops.cs:98-110).  Each
    // half wave (one row group, all 32 column groups) holds the whole head's
    // o, so the sum of squares is a 32-lane reduction, no exchange; the first
    // row group writes the output.
    const float ss = group_sum<32>(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
    if (rg == 0) {
        const float rs = 1.0f / sqrtf(ss / (float)kDk + eps);
        float4 r;
        r.x = o[0] * rs * nw4.x * silu(z4.x);
        r.y = o[1] * rs * nw4.y * silu(z4.y);
        r.z = o[2] * rs * nw4.z * silu(z4.z);
        r.w = o[3] * rs * nw4.w * silu(z4.w);
        *reinterpret_cast<float4*>(out + o_off) = r;
    }
}

}  // namespace

hipError_t launch_deltanet_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* qkv,
                                  const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    ProfScope ps_(c, K_DN_DECODE);
    hipExtLaunchKernelGGL(deltanet_decode_kernel, dim3(sb.n * d.nv), dim3(NT), 0, c->stream, ps_.a, ps_.b, 0, qkv, z,
                       b, a, out, L.conv_w, L.ssm_a, L.dt_bias, L.ssm_norm, L.state, L.conv, d.nk,
                       d.nv, d.eps, sb);
    return hipGetLastError();
}

}  // namespace q35
