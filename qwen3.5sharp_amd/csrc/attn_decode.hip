// Gated GQA attention decode (one new token per sequence): split-K flash
// decode over the KV cache.
//
// Reference: Qwen35Model.DecodeAttention after the projections
// (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:294-323): q|gate
// de-interleave, NeoX partial RoPE (Ops.cs:75-133) then the zero-centred
// (1+w) RMSNorm (Qwen35Ops.cs:22-66) on q and on the new K row written into
// the cache, scores scaled by 1/sqrt(head_dim) (Ops.AttentionScores,
// Ops.cs:281-357), causal softmax (Ops.SoftmaxCausal, Ops.cs:163-252),
// P.V (Ops.AttentionCombine, Ops.cs:360-415), times sigmoid(gate).
//
// Pass 1 (attn_decode_partial): one workgroup per (sequence, kv head, chunk of
// P positions).  The 4 q heads of the kv head share every K/V row it reads,
// so each cache byte is read once per token.  Each workgroup recomputes the
// 4 rotated, normed q rows (4 KiB of input); the workgroup whose chunk holds
// the new position also rotates/norms the new K row and writes K and V into
// the cache (single writer) and uses them from LDS.  It emits, per q head, the
// chunk's max score m, sum of exp l, and unnormalised o = sum exp(s-m) v.
// Pass 2 (attn_decode_merge): per (sequence, q head) the chunks are merged
// with the usual log-sum-exp rescaling and the sigmoid gate is applied.
//
// Online softmax is the two-pass softmax regrouped; it omits the reference's
// -80 floor on shifted logits, which only touches weights below e^-80
// relative to the row maximum (invisible in fp32 next to the maximum's 1).
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int NT = 256;

// RoPE (pairs (d, d+32), d < 32) and the (1+w) RMSNorm of one 256-wide head
// row held as one float4 per lane of a wave (lane l: dims 4l..4l+3).
__device__ __forceinline__ float4 rope_norm_row(float4 x, int lane, const float* __restrict__ cs,
                                                const float* __restrict__ sn,
                                                const float* __restrict__ w, float eps,
                                                float post_scale) {
    float4 p;
    p.x = __shfl_xor(x.x, 8, kWave);
    p.y = __shfl_xor(x.y, 8, kWave);
    p.z = __shfl_xor(x.z, 8, kWave);
    p.w = __shfl_xor(x.w, 8, kWave);
    if (lane < 16) {
        const int i0 = 4 * (lane & 7);
        const float4 c = *reinterpret_cast<const float4*>(cs + i0);
        const float4 s = *reinterpret_cast<const float4*>(sn + i0);
        if (lane < 8) {   // x0' = x0 c - x1 s
            x.x = x.x * c.x - p.x * s.x;
            x.y = x.y * c.y - p.y * s.y;
            x.z = x.z * c.z - p.z * s.z;
            x.w = x.w * c.w - p.w * s.w;
        } else {          // x1' = x0 s + x1 c
            x.x = p.x * s.x + x.x * c.x;
            x.y = p.y * s.y + x.y * c.y;
            x.z = p.z * s.z + x.z * c.z;
            x.w = p.w * s.w + x.w * c.w;
        }
    }
    const float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
    const float scale = 1.0f / sqrtf(ss / (float)kHd + eps);
    const float4 ww = *reinterpret_cast<const float4*>(w + 4 * lane);
    x.x = x.x * scale * (1.0f + ww.x) * post_scale;
    x.y = x.y * scale * (1.0f + ww.y) * post_scale;
    x.z = x.z * scale * (1.0f + ww.z) * post_scale;
    x.w = x.w * scale * (1.0f + ww.w) * post_scale;
    return x;
}

template <int P>
__global__ __launch_bounds__(NT) void attn_decode_partial(
    const float* __restrict__ q_gate, const float* __restrict__ knew,
    const float* __restrict__ vnew, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    float* __restrict__ part_o, float* __restrict__ part_ml, int nkv, int cap, int nchunks,
    float eps, SeqBatch sb) {
    const int c = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
    const int pos = sb.pos[i];
    const int p0 = c * P;
    if (p0 > pos) return;
    const int np = min(P, pos + 1 - p0);
    const int nh = nkv * kGqaGroup;
    const int kv_dim = nkv * kHd;
    const size_t seq_off = (size_t)sb.seq[i] * cap * kv_dim + (size_t)kvh * kHd;
    float* K = k_cache + seq_off;
    float* V = v_cache + seq_off;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    __shared__ float4 q_s[kGqaGroup][kHd / 4];
    __shared__ float4 knew_s[kHd / 4];
    __shared__ float4 vnew_s[kHd / 4];
    __shared__ float sc[kGqaGroup][P];
    __shared__ float ml[kGqaGroup][2];
    __shared__ float4 obuf[4][kGqaGroup][kHd / 4];

    const float* cs = rope_cos + (size_t)pos * kRopeHalf;
    const float* sn = rope_sin + (size_t)pos * kRopeHalf;
    const bool has_new = pos < p0 + P;
    {
        // q of head kvh*4 + wave; the attention scale 1/16 is folded in.
        const int h = kvh * kGqaGroup + wave;
        const float* qrow = q_gate + (size_t)i * 2 * nh * kHd + (size_t)h * 2 * kHd;
        float4 x = *reinterpret_cast<const float4*>(qrow + 4 * lane);
        q_s[wave][lane] = rope_norm_row(x, lane, cs, sn, q_norm, eps, 1.0f / sqrtf((float)kHd));
    }
    if (has_new) {
        if (wave == 0) {
            float4 x = *reinterpret_cast<const float4*>(knew + (size_t)i * kv_dim + kvh * kHd + 4 * lane);
            x = rope_norm_row(x, lane, cs, sn, k_norm, eps, 1.0f);
            knew_s[lane] = x;
            *reinterpret_cast<float4*>(K + (size_t)pos * kv_dim + 4 * lane) = x;
        } else if (wave == 1) {
            float4 x = *reinterpret_cast<const float4*>(vnew + (size_t)i * kv_dim + kvh * kHd + 4 * lane);
            vnew_s[lane] = x;
            *reinterpret_cast<float4*>(V + (size_t)pos * kv_dim + 4 * lane) = x;
        }
    }
    __syncthreads();

    // Scores: 16 teams of 16 lanes; a lane holds dims {4*l16 + 64*m .. +3}.
    {
        const int team = tid >> 4, l16 = tid & 15;
        float4 qr[kGqaGroup][4];
#pragma unroll
        for (int h = 0; h < kGqaGroup; ++h)
#pragma unroll
            for (int m = 0; m < 4; ++m) qr[h][m] = q_s[h][l16 + 16 * m];
        for (int pp = team; pp < np; pp += 16) {
            const int pabs = p0 + pp;
            float4 kk[4];
            if (pabs == pos) {
#pragma unroll
                for (int m = 0; m < 4; ++m) kk[m] = knew_s[l16 + 16 * m];
            } else {
                const float4* krow = reinterpret_cast<const float4*>(K + (size_t)pabs * kv_dim);
#pragma unroll
                for (int m = 0; m < 4; ++m) kk[m] = krow[l16 + 16 * m];
            }
            float acc[kGqaGroup];
#pragma unroll
            for (int h = 0; h < kGqaGroup; ++h) {
                float a = 0.0f;
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    a += qr[h][m].x * kk[m].x + qr[h][m].y * kk[m].y + qr[h][m].z * kk[m].z +
                         qr[h][m].w * kk[m].w;
                acc[h] = group_sum<16>(a);
            }
            if (l16 == 0)
#pragma unroll
                for (int h = 0; h < kGqaGroup; ++h) sc[h][pp] = acc[h];
        }
    }
    __syncthreads();

    // Chunk softmax, one wave per q head.
    {
        float m = -INFINITY;
        for (int pp = lane; pp < np; pp += 64) m = fmaxf(m, sc[wave][pp]);
        m = wave_max(m);
        float l = 0.0f;
        for (int pp = lane; pp < np; pp += 64) {
            const float e = __expf(sc[wave][pp] - m);
            sc[wave][pp] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            ml[wave][0] = m;
            ml[wave][1] = l;
        }
    }
    __syncthreads();

    // P.V: thread owns dims 4*d4..+3 of all 4 heads over positions pp = ps mod 4.
    {
        const int d4 = tid & 63, ps = tid >> 6;
        float4 acc[kGqaGroup];
#pragma unroll
        for (int h = 0; h < kGqaGroup; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int pp = ps; pp < np; pp += 4) {
            const int pabs = p0 + pp;
            const float4 vv = pabs == pos
                                  ? vnew_s[d4]
                                  : reinterpret_cast<const float4*>(V + (size_t)pabs * kv_dim)[d4];
#pragma unroll
            for (int h = 0; h < kGqaGroup; ++h) {
                const float e = sc[h][pp];
                acc[h].x += e * vv.x;
                acc[h].y += e * vv.y;
                acc[h].z += e * vv.z;
                acc[h].w += e * vv.w;
            }
        }
#pragma unroll
        for (int h = 0; h < kGqaGroup; ++h) obuf[ps][h][d4] = acc[h];
    }
    __syncthreads();
    {
        const int h = tid >> 6, d4 = tid & 63;
        float4 o = obuf[0][h][d4];
#pragma unroll
        for (int ps = 1; ps < 4; ++ps) {
            const float4 t = obuf[ps][h][d4];
            o.x += t.x; o.y += t.y; o.z += t.z; o.w += t.w;
        }
        const size_t pidx = (((size_t)i * nkv + kvh) * nchunks + c) * kGqaGroup + h;
        reinterpret_cast<float4*>(part_o + pidx * kHd)[d4] = o;
        if (d4 == 0) {
            part_ml[2 * pidx] = ml[h][0];
            part_ml[2 * pidx + 1] = ml[h][1];
        }
    }
}

__global__ __launch_bounds__(kHd) void attn_decode_merge(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const float* __restrict__ q_gate, float* __restrict__ out, int nkv, int nchunks, int P,
    SeqBatch sb) {
    const int h = blockIdx.x, i = blockIdx.y, d = threadIdx.x;
    const int nh = nkv * kGqaGroup;
    const int kvh = h / kGqaGroup, hl = h % kGqaGroup;
    const int nc = (sb.pos[i] + 1 + P - 1) / P;
    float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
    const size_t base = ((size_t)i * nkv + kvh) * nchunks;
    for (int c = 0; c < nc; ++c) {
        const size_t pidx = (base + c) * kGqaGroup + hl;
        const float m = part_ml[2 * pidx], l = part_ml[2 * pidx + 1];
        const float o = part_o[pidx * kHd + d];
        const float mn = fmaxf(M, m);
        const float a = __expf(M - mn), b = __expf(m - mn);
        Lsum = Lsum * a + l * b;
        O = O * a + o * b;
        M = mn;
    }
    const float gate = q_gate[(size_t)i * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd + d];
    out[(size_t)i * nh * kHd + (size_t)h * kHd + d] = (O / Lsum) * (1.0f / (1.0f + expf(-gate)));
}

int pick_chunk(int n, int nkv, int max_len) {
    // Smallest chunk that still gives >= 4 workgroups per CU (256 CUs); at least 64.
    static const int sizes[3] = {256, 128, 64};
    for (int s : sizes)
        if ((long)n * nkv * ((max_len + s - 1) / s) >= 1024) return s;
    return 64;
}

}  // namespace

size_t attn_decode_work_bytes(const Dims& d, int n, int max_kv_len) {
    const int P = pick_chunk(n, d.nkv, max_kv_len);
    const size_t nchunks = (max_kv_len + P - 1) / P;
    return (size_t)n * d.nkv * nchunks * kGqaGroup * (kHd + 2) * sizeof(float);
}

hipError_t launch_attn_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* q_gate,
                              const float* k, const float* v, float* out) {
    const Dims& d = c->d;
    const AttnLayer& L = c->full[layer];
    int max_len = 0;
    for (int i = 0; i < sb.n; ++i) max_len = max(max_len, sb.pos[i] + 1);
    const int P = pick_chunk(sb.n, d.nkv, max_len);
    const int nchunks = (max_len + P - 1) / P;
    float* part_o = c->work;
    float* part_ml = part_o + (size_t)sb.n * d.nkv * nchunks * kGqaGroup * kHd;
    dim3 grid(nchunks, d.nkv, sb.n);
    {
    ProfScope ps_(c, K_ATTN_DECODE_PARTIAL);
    switch (P) {
        case 256:
            hipLaunchKernelGGL(attn_decode_partial<256>, grid, dim3(NT), 0, c->stream, q_gate, k, v,
                               L.q_norm, L.k_norm, L.k_cache, L.v_cache, c->rope_cos, c->rope_sin,
                               part_o, part_ml, d.nkv, c->cap, nchunks, d.eps, sb);
            break;
        case 128:
            hipLaunchKernelGGL(attn_decode_partial<128>, grid, dim3(NT), 0, c->stream, q_gate, k, v,
                               L.q_norm, L.k_norm, L.k_cache, L.v_cache, c->rope_cos, c->rope_sin,
                               part_o, part_ml, d.nkv, c->cap, nchunks, d.eps, sb);
            break;
        default:
            hipLaunchKernelGGL(attn_decode_partial<64>, grid, dim3(NT), 0, c->stream, q_gate, k, v,
                               L.q_norm, L.k_norm, L.k_cache, L.v_cache, c->rope_cos, c->rope_sin,
                               part_o, part_ml, d.nkv, c->cap, nchunks, d.eps, sb);
            break;
    }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_ATTN_DECODE_MERGE);
        hipLaunchKernelGGL(attn_decode_merge, dim3(d.nh, sb.n), dim3(kHd), 0, c->stream, part_o, part_ml,
                           q_gate, out, d.nkv, nchunks, P, sb);
    }
    return hipGetLastError();
}

}  // namespace q35
