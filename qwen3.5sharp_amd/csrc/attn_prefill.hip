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
//  2. attn_prefill_flash: causal flash attention on fp32 MFMA, one workgroup
//     per (group of up to 4 q heads sharing a kv head, 16-row query block),
//     K/V streamed through LDS in 32-row tiles, online softmax; the
//     [T][kvLen] score matrix is never materialised.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

__global__ __launch_bounds__(kWave) void attn_prefill_prep(
    const float* __restrict__ q_gate, const float* __restrict__ knew,
    const float* __restrict__ vnew, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float* __restrict__ K, float* __restrict__ V,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    float* __restrict__ qbuf, int start, int nh, int nkv, int cap, float eps) {
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
        // Head-major cache: row pos of kv head kvh at (kvh * cap + pos) * 256.
        const size_t row = ((size_t)kvh * cap + pos) * kHd;
        *reinterpret_cast<float4*>(K + row + 4 * lane) = x;
        const float4 v = *reinterpret_cast<const float4*>(vnew + (size_t)t * kv_dim + kvh * kHd + 4 * lane);
        *reinterpret_cast<float4*>(V + row + 4 * lane) = v;
    }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int QR = 16;          // query rows per workgroup (per head)
constexpr int KT = 32;          // key rows per tile
constexpr int LDKV = kHd + 4;   // padded LDS row stride of the K/V tiles

// Causal flash attention on fp32 MFMA (v_mfma_f32_16x16x4f32).  Workgroup =
// (head group y, 16 query rows): the group is hg = min(4, q heads per kv
// head) q heads hg y .. hg y + hg - 1 of one kv head, and wave w is q head
// hg y + w, so the group's q heads share every K/V tile staged in LDS (with
// fewer than 4 heads the spare waves repeat the last head and store nothing).  Per 32-row key tile a wave
// computes S^T = K Q^T (positions x queries), so each lane's D column is one
// query: the online-softmax max/sum and the rescale of O^T = V^T P^T are
// per lane, and S^T's D tile feeds P^T = B operand register by register.
// Lane l = 16g + c: Q operand holds Q[row c][64g + s], s < 64 (reduction index
// of instruction s for lane group g), O^T register r of block db holds
// O[row c][16 db + 4g + r].  The next K/V tile is loaded into registers while
// the current one computes.  Heavy and light query blocks are paired per CU.
__global__ __launch_bounds__(256, 2) void attn_prefill_flash(
    const float* __restrict__ qbuf, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ q_gate, float* __restrict__ out, int start, int T, int nh,
    int nkv, int hg, int cap) {
    // Work items ranked by cost (query block, heaviest first; head groups
    // innermost).  Workgroup L < half takes rank L and workgroup half + m
    // takes rank total-1-m, so the two workgroups the dispatcher places on one
    // CU when the whole grid is resident (L and L + half) carry a heavy and a
    // light query block: causal work is balanced per CU, not per workgroup.
    const int groups = nh / hg;
    const int nqb = (T + QR - 1) / QR;
    const int total = nqb * groups, half = (total + 1) / 2, L = blockIdx.x;
    const int rank = L < half ? L : total - 1 - (L - half);
    const int qb = nqb - 1 - rank / groups, y = rank % groups;
    const int kvh = y * hg / (nh / nkv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const bool stores = wave < hg;           // uniform per wave
    const int h = hg * y + min(wave, hg - 1);
    const int r0 = qb * QR;
    const int blk_len = start + min(T - 1, r0 + QR - 1) + 1;
    const int my_t = min(r0 + c16, T - 1);
    const int my_len = start + my_t + 1;
    // Head-major cache: kv head kvh's rows are [cap][256] from kvh * cap * 256.
    const float* Kh = K + (size_t)kvh * cap * kHd;
    const float* Vh = V + (size_t)kvh * cap * kHd;

    __shared__ float Ks[KT][LDKV];
    __shared__ float Vs[KT][LDKV];

    float qreg[64];
    {
        const float* qrow = qbuf + ((size_t)my_t * nh + h) * kHd + 64 * g;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float4 x = *reinterpret_cast<const float4*>(qrow + 4 * u);
            qreg[4 * u] = x.x; qreg[4 * u + 1] = x.y; qreg[4 * u + 2] = x.z; qreg[4 * u + 3] = x.w;
        }
    }
    f32x4 O[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) O[db] = {0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    // Staging: thread loads float4 idx = tid + 256 i (i < 8) of the 32 x 64
    // float4 tile, i.e. row 4 i + tid / 64, float4 column tid % 64.  Rows past
    // blk_len read row 0 instead (finite data; their scores are masked), so
    // no select waits on the loads, and the refill is unconditional.
    const int srow = tid >> 6, sc4 = tid & 63;
    float4 sk0, sk1, sk2, sk3, sk4, sk5, sk6, sk7;
    float4 sv0, sv1, sv2, sv3, sv4, sv5, sv6, sv7;
#define Q35_LOAD_ROW(i, p0)                                                                  \
    {                                                                                      \
        const int p = (p0) + 4 * (i) + srow;                                               \
        const size_t off = (size_t)(p < blk_len ? p : 0) * kHd + 4 * sc4;                  \
        sk##i = *reinterpret_cast<const float4*>(Kh + off);                                \
        sv##i = *reinterpret_cast<const float4*>(Vh + off);                                \
    }
#define Q35_LOAD_TILE(p0)                                                                    \
    Q35_LOAD_ROW(0, p0) Q35_LOAD_ROW(1, p0) Q35_LOAD_ROW(2, p0) Q35_LOAD_ROW(3, p0)            \
    Q35_LOAD_ROW(4, p0) Q35_LOAD_ROW(5, p0) Q35_LOAD_ROW(6, p0) Q35_LOAD_ROW(7, p0)
#define Q35_STORE_ROW(i)                                                                     \
    *reinterpret_cast<float4*>(&Ks[4 * (i) + srow][4 * sc4]) = sk##i;                       \
    *reinterpret_cast<float4*>(&Vs[4 * (i) + srow][4 * sc4]) = sv##i;
    Q35_LOAD_TILE(0)
    for (int p0 = 0; p0 < blk_len; p0 += KT) {
        lds_barrier();
        Q35_STORE_ROW(0) Q35_STORE_ROW(1) Q35_STORE_ROW(2) Q35_STORE_ROW(3)
        Q35_STORE_ROW(4) Q35_STORE_ROW(5) Q35_STORE_ROW(6) Q35_STORE_ROW(7)
        lds_barrier();
        Q35_LOAD_TILE(p0 + KT)
#undef Q35_LOAD_ROW
#undef Q35_LOAD_TILE
#undef Q35_STORE_ROW

        // S^T for positions p0 + 16 pb + (4g + r), queries c16.
        f32x4 st[2];
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float4 a = *reinterpret_cast<const float4*>(&Ks[16 * pb + c16][64 * g + 4 * u]);
                acc = mfma16(a.x, qreg[4 * u], acc);
                acc = mfma16(a.y, qreg[4 * u + 1], acc);
                acc = mfma16(a.z, qreg[4 * u + 2], acc);
                acc = mfma16(a.w, qreg[4 * u + 3], acc);
            }
            st[pb] = acc;
        }
        // Online softmax down this lane's query column.
        float mt = m_run;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int p = p0 + 16 * pb + 4 * g + r;
                if (p >= my_len) st[pb][r] = -INFINITY;
                mt = fmaxf(mt, st[pb][r]);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
        const float alpha = __expf(m_run - mt);
        float ls = 0.0f;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __expf(st[pb][r] - mt);
                st[pb][r] = e;
                ls += e;
            }
        ls += __shfl_xor(ls, 16, kWave);
        ls += __shfl_xor(ls, 32, kWave);
        l_run = l_run * alpha + ls;
        m_run = mt;
        // O^T = alpha O^T + V^T P^T.
#pragma unroll
        for (int db = 0; db < 16; ++db) {
            f32x4 acc = O[db] * alpha;
#pragma unroll
            for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2)
                    acc = mfma16(Vs[16 * pb + 4 * g + s2][16 * db + c16], st[pb][s2], acc);
            O[db] = acc;
        }
    }
    const int t = r0 + c16;
    if (t >= T || !stores) return;
    const float inv = 1.0f / l_run;
    const float* grow = q_gate + (size_t)t * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd;
    float* orow = out + ((size_t)t * nh + h) * kHd;
#pragma unroll
    for (int db = 0; db < 16; ++db) {
        const int d0 = 16 * db + 4 * g;
        const float4 gt = *reinterpret_cast<const float4*>(grow + d0);
        float4 r;
        r.x = O[db][0] * inv * (1.0f / (1.0f + expf(-gt.x)));
        r.y = O[db][1] * inv * (1.0f / (1.0f + expf(-gt.y)));
        r.z = O[db][2] * inv * (1.0f / (1.0f + expf(-gt.z)));
        r.w = O[db][3] * inv * (1.0f / (1.0f + expf(-gt.w)));
        *reinterpret_cast<float4*>(orow + d0) = r;
    }
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
        hipExtLaunchKernelGGL(attn_prefill_prep, dim3(T, d.nh + d.nkv), dim3(kWave), 0, c->stream, ps_.a, ps_.b, 0, q_gate,
                           k, v, L.q_norm, L.k_norm, K, V, c->rope_cos, c->rope_sin, qbuf, start, d.nh,
                           d.nkv, c->cap, d.eps);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        // Head groups of up to 4 q heads of one kv head.
        const int g = d.nh / d.nkv, hg = g < 4 ? g : 4;
        ProfScope ps_(c, K_ATTN_PREFILL_FLASH);
        hipExtLaunchKernelGGL(attn_prefill_flash, dim3((T + QR - 1) / QR * (d.nh / hg)), dim3(256), 0,
                           c->stream, ps_.a, ps_.b, 0, qbuf, K, V, q_gate, out, start, T, d.nh, d.nkv, hg,
                           c->cap);
    }
    return hipGetLastError();
}

}  // namespace q35
