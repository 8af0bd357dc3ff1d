// Gated GQA attention prefill for T tokens of one sequence starting at row
// `start` of its KV cache.
//
// Reference: Qwen35Model.PrefillAttention after the projections
// (src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:113-149): q|gate
// de-interleave, K/V written into cache rows start.., NeoX RoPE then (1+w)
// RMSNorm on q and on the cached K rows, causal softmax attention over
// start+T rows with scale 1/sqrt(head_dim), times sigmoid(gate).
//
//  1. attn_prefill_prep: rotate/norm q (scale folded in) into the workspace,
//     rotate/norm K into the cache, copy V into the cache.
//  2. attn_prefill_flash: causal flash attention, one workgroup per (q head,
//     32-row query block), K/V streamed through LDS in 32-row tiles, online
//     softmax; the [T][kvLen] score matrix is never materialised.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

__global__ __launch_bounds__(kWave) void attn_prefill_prep(
    const float* __restrict__ q_gate, const float* __restrict__ knew,
    const float* __restrict__ vnew, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float* __restrict__ K, float* __restrict__ V,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    float* __restrict__ qbuf, int start, int nh, int nkv, float eps) {
    const int t = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const int pos = start + t;
    const int kv_dim = nkv * kHd;
    const float* cs = rope_cos + (size_t)pos * kRopeHalf;
    const float* sn = rope_sin + (size_t)pos * kRopeHalf;
    if (r < nh) {
        const float* qrow = q_gate + (size_t)t * 2 * nh * kHd + (size_t)r * 2 * kHd;
        float4 x = *reinterpret_cast<const float4*>(qrow + 4 * lane);
        x = rope_norm_row(x, lane, cs, sn, q_norm, eps, 1.0f / sqrtf((float)kHd));
        *reinterpret_cast<float4*>(qbuf + ((size_t)t * nh + r) * kHd + 4 * lane) = x;
    } else {
        const int kvh = r - nh;
        float4 x = *reinterpret_cast<const float4*>(knew + (size_t)t * kv_dim + kvh * kHd + 4 * lane);
        x = rope_norm_row(x, lane, cs, sn, k_norm, eps, 1.0f);
        *reinterpret_cast<float4*>(K + (size_t)pos * kv_dim + kvh * kHd + 4 * lane) = x;
        const float4 v = *reinterpret_cast<const float4*>(vnew + (size_t)t * kv_dim + kvh * kHd + 4 * lane);
        *reinterpret_cast<float4*>(V + (size_t)pos * kv_dim + kvh * kHd + 4 * lane) = v;
    }
}

constexpr int QB = 32;   // query rows per workgroup
constexpr int KT = 32;   // key rows per tile
constexpr int KPAD = kHd + 4;

// Thread layout: row r = tid / 8 of the query block; sub = tid % 8 owns 32
// interleaved dims.  Scores are reduced over the 8 lanes of a row.
__global__ __launch_bounds__(256) void attn_prefill_flash(
    const float* __restrict__ qbuf, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ q_gate, float* __restrict__ out, int start, int T, int nh,
    int nkv) {
    const int qb = blockIdx.x, h = blockIdx.y;
    const int kvh = h / kGqaGroup;
    const int kv_dim = nkv * kHd;
    const int tid = threadIdx.x, r = tid >> 3, sub = tid & 7;
    const int t = qb * QB + r;
    const bool valid = t < T;
    const int my_len = start + (valid ? t : (T - 1)) + 1;   // visible rows of this query
    const int blk_last = min(T - 1, qb * QB + QB - 1);
    const int blk_len = start + blk_last + 1;                // rows the block must visit

    __shared__ float Ks[KT][KPAD];
    __shared__ float Vs[KT][KPAD];

    // Lane `sub` of a row owns dims sub, sub+8, ..., sub+248 (conflict-free LDS reads).
    float q[32];
    {
        const float* qrow = qbuf + ((size_t)(valid ? t : T - 1) * nh + h) * kHd + sub;
#pragma unroll
        for (int d = 0; d < 32; ++d) q[d] = qrow[8 * d];
    }
    float o[32];
#pragma unroll
    for (int d = 0; d < 32; ++d) o[d] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    for (int p0 = 0; p0 < blk_len; p0 += KT) {
        __syncthreads();
        // Stage K and V rows p0..p0+KT-1 (rows past blk_len are never used).
        for (int idx = tid; idx < KT * (kHd / 4); idx += 256) {
            const int pr = idx / (kHd / 4), c4 = idx % (kHd / 4);
            const int p = p0 + pr;
            float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
            if (p < blk_len) {
                kx = *reinterpret_cast<const float4*>(K + (size_t)p * kv_dim + kvh * kHd + 4 * c4);
                vx = *reinterpret_cast<const float4*>(V + (size_t)p * kv_dim + kvh * kHd + 4 * c4);
            }
            *reinterpret_cast<float4*>(&Ks[pr][4 * c4]) = kx;
            *reinterpret_cast<float4*>(&Vs[pr][4 * c4]) = vx;
        }
        __syncthreads();
        float s[KT];
#pragma unroll
        for (int pr = 0; pr < KT; ++pr) {
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < 32; ++d) a += q[d] * Ks[pr][sub + 8 * d];
            s[pr] = group_sum<8>(a);
        }
        float mt = m;
#pragma unroll
        for (int pr = 0; pr < KT; ++pr) {
            if (p0 + pr >= my_len) s[pr] = -INFINITY;
            mt = fmaxf(mt, s[pr]);
        }
        const float alpha = m == -INFINITY ? 0.0f : __expf(m - mt);
        l *= alpha;
#pragma unroll
        for (int d = 0; d < 32; ++d) o[d] *= alpha;
#pragma unroll
        for (int pr = 0; pr < KT; ++pr) {
            const float e = s[pr] == -INFINITY ? 0.0f : __expf(s[pr] - mt);
            l += e;
#pragma unroll
            for (int d = 0; d < 32; ++d) o[d] += e * Vs[pr][sub + 8 * d];
        }
        m = mt;
    }
    if (!valid) return;
    const float* grow = q_gate + (size_t)t * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd + sub;
    float* orow = out + ((size_t)t * nh + h) * kHd + sub;
    const float inv = 1.0f / l;
#pragma unroll
    for (int d = 0; d < 32; ++d) orow[8 * d] = o[d] * inv * (1.0f / (1.0f + expf(-grow[8 * d])));
}

}  // namespace

size_t attn_prefill_work_bytes(const Dims& d, int T) {
    return (size_t)T * d.q_dim * sizeof(float);
}

hipError_t launch_attn_prefill(q35m_ctx* c, int layer, int seq, int start, int T,
                               const float* q_gate, const float* k, const float* v, float* out) {
    const Dims& d = c->d;
    const AttnLayer& L = c->full[layer];
    float* K = L.k_cache + (size_t)seq * c->cap * d.kv_dim;
    float* V = L.v_cache + (size_t)seq * c->cap * d.kv_dim;
    float* qbuf = c->work;
    {
        ProfScope ps_(c, K_ATTN_PREFILL_PREP);
        hipLaunchKernelGGL(attn_prefill_prep, dim3(T, d.nh + d.nkv), dim3(kWave), 0, c->stream, q_gate,
                           k, v, L.q_norm, L.k_norm, K, V, c->rope_cos, c->rope_sin, qbuf, start, d.nh,
                           d.nkv, d.eps);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_ATTN_PREFILL_FLASH);
        hipLaunchKernelGGL(attn_prefill_flash, dim3((T + QB - 1) / QB, d.nh), dim3(256), 0, c->stream,
                           qbuf, K, V, q_gate, out, start, T, d.nh, d.nkv);
    }
    return hipGetLastError();
}

}  // namespace q35
