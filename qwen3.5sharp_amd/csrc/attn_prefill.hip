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
//     its key range split between two halves of the workgroup, K/V streamed
//     through LDS in 32-row tiles, online softmax; the [T][kvLen] score
//     matrix is never materialised.
#include <algorithm>


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
constexpr int LDKV = kHd + 4;   // padded LDS row stride of the K tiles
constexpr int LDVT = KT + 4;    // padded LDS row stride of the transposed V tiles

// Causal flash attention on fp32 MFMA (v_mfma_f32_16x16x4f32).  Workgroup =
// (head group y, 16 query rows) in two halves of 4 waves: half 0 takes the
// first ceil(n/2) of the block's n key tiles, half 1 the rest, each with its
// own K/V tiles in LDS, and half 0 merges the two online-softmax states at
// the end (max, sum and the unnormalised output rescaled to the common max).
// So every workgroup keeps 8 waves busy on half of its block's key range, and
// one workgroup a CU, dispatched heaviest first, balances the causal work
// over the CUs.  Within a half the group is hg = min(4, q heads per kv head)
// q heads hg y .. hg y + hg - 1 of one kv head, and wave w of the half is q
// head hg y + w, so the group's q heads share every K/V tile (with fewer than
// 4 heads the spare waves repeat the last head and store nothing).  Per
// 32-row key tile a wave computes S^T = K Q^T (positions x queries), so each
// lane's D column is one query: the online-softmax max/sum and the rescale of
// O^T = V^T P^T are per lane, and S^T's D tile feeds P^T = B operand register
// by register.  Lane l = 16g + c: Q operand holds Q[row c][64g + s], s < 64
// (reduction index of instruction s for lane group g), O^T register r of
// block db holds O[row c][16 db + 4g + r].  V tiles are stored transposed
// (dims x positions), so a lane's four P.V operands of a 16-position block are
// one 16-byte read; P.V runs four output blocks at a time (four independent
// accumulation chains, each in the order pb, s2), S one key-row block ahead
// in its operand reads.  The next K tile goes to LDS by buffer loads straight
// into LDS once every wave is past S, the next V tile into registers.
__global__ __launch_bounds__(512, 1) void attn_prefill_flash(
    const float* __restrict__ qbuf, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ q_gate, float* __restrict__ out, int start, int T, int nh,
    int nkv, int hg, int cap) {
    const int groups = nh / hg;
    const int nqb = (T + QR - 1) / QR;
    const int rank = blockIdx.x;                 // heaviest query blocks first
    const int qb = nqb - 1 - rank / groups, y = rank % groups;
    const int kvh = y * hg / (nh / nkv);
    const int tid = threadIdx.x, lane = tid & 63;
    // Wave-uniform (readfirstlane): the K tile loads take them as scalar
    // offsets and LDS bases.
    const int half = __builtin_amdgcn_readfirstlane(tid >> 8);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6) & 3, htid = tid & 255;
    const int g = lane >> 4, c16 = lane & 15;
    const bool stores = wave < hg;           // uniform per wave
    const int h = hg * y + min(wave, hg - 1);
    const int r0 = qb * QR;
    const int blk_len = start + min(T - 1, r0 + QR - 1) + 1;
    const int my_t = min(r0 + c16, T - 1);
    const int my_len = start + my_t + 1;
    // Key tiles of this half: [t_begin, t_begin + n_iter), the last one past
    // blk_len (fully masked) when half 1 has one tile fewer.
    const int n_tiles = (blk_len + KT - 1) / KT, n_iter = (n_tiles + 1) / 2;
    const int p_begin = half * n_iter * KT;
    // Head-major cache: kv head kvh's rows are [cap][256] from kvh * cap * 256.
    const float* Kh = K + (size_t)kvh * cap * kHd;
    const float* Vh = V + (size_t)kvh * cap * kHd;

    // K tiles (row-major) and V tiles (transposed: dims x positions, so a
    // lane's P.V operands for 4 positions are one 16-byte read) of each half;
    // at the end, the merge's exchange area.
    struct Tiles {
        float k[KT][LDKV];
        float vt[kHd][LDVT];
    };
    __shared__ Tiles smem[2];
    float (*Ks)[LDKV] = smem[half].k;
    float (*Vt)[LDVT] = smem[half].vt;

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

    // Staging.  K: wave w of the half loads rows w, w + 4, ... of the tile
    // by buffer loads straight into LDS (one 1 KiB row a load).  V (stored
    // transposed): thread row htid % 32, float4 columns htid / 32 + 8 i, so
    // that the transposed stores of 32 lanes land on 32 consecutive words.
    // Rows past blk_len read row 0 instead (finite data; their scores are
    // masked), so no select waits on the loads, and the refill is
    // unconditional.
    // The host keeps start + T <= kPrefillMaxRows = 2^21 rows, so a row's
    // offset fits 31 bits and its last 16-byte load ends at most at byte 2^31:
    // the range is whole rows, up to exactly 2^31 bytes (the 32-bit
    // num_records field is unsigned; 0x80000000 as its bit pattern).
    const uint32_t krange = (uint32_t)(std::min<size_t>((size_t)cap, (size_t)kPrefillMaxRows) * kHd * sizeof(float));
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Kh), 0, (int)krange, 0x00020000);
    auto load_k = [&](int p0) {
#pragma unroll
        for (int i = 0; i < KT / 4; ++i) {
            const int r = wave + 4 * i, p = p0 + r;
            dma_b128(krs, &Ks[r][0], 16u * lane, (uint32_t)(p < blk_len ? p : 0) * kHd * sizeof(float));
        }
    };
    const int vrow = htid & 31, vc4 = htid >> 5;
    float4 sv0, sv1, sv2, sv3, sv4, sv5, sv6, sv7;
#define Q35_LOAD_ROW(i, p0)                                                                  \
    {                                                                                      \
        const int pv = (p0) + vrow;                                                        \
        sv##i = *reinterpret_cast<const float4*>(Vh + (size_t)(pv < blk_len ? pv : 0) * kHd +  \
                                                 4 * (vc4 + 8 * (i)));                      \
    }
#define Q35_LOAD_TILE(p0)                                                                    \
    Q35_LOAD_ROW(0, p0) Q35_LOAD_ROW(1, p0) Q35_LOAD_ROW(2, p0) Q35_LOAD_ROW(3, p0)            \
    Q35_LOAD_ROW(4, p0) Q35_LOAD_ROW(5, p0) Q35_LOAD_ROW(6, p0) Q35_LOAD_ROW(7, p0)
#define Q35_STORE_ROW(i)                                                                     \
    Vt[4 * (vc4 + 8 * (i)) + 0][vrow] = sv##i.x;                                            \
    Vt[4 * (vc4 + 8 * (i)) + 1][vrow] = sv##i.y;                                            \
    Vt[4 * (vc4 + 8 * (i)) + 2][vrow] = sv##i.z;                                            \
    Vt[4 * (vc4 + 8 * (i)) + 3][vrow] = sv##i.w;
    load_k(p_begin);
    Q35_LOAD_TILE(p_begin)
    for (int it = 0; it < n_iter; ++it) {
        const int p0 = p_begin + it * KT;
        // The K tile has landed and every wave is past the previous P.V.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        Q35_STORE_ROW(0) Q35_STORE_ROW(1) Q35_STORE_ROW(2) Q35_STORE_ROW(3)
        Q35_STORE_ROW(4) Q35_STORE_ROW(5) Q35_STORE_ROW(6) Q35_STORE_ROW(7)

        // S^T for positions p0 + 16 pb + (4g + r), queries c16.
        f32x4 st[2];
        {
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            float4 a0 = *reinterpret_cast<const float4*>(&Ks[c16][64 * g]);
            float4 a1 = *reinterpret_cast<const float4*>(&Ks[16 + c16][64 * g]);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                float4 n0 = a0, n1 = a1;
                if (u < 15) {
                    n0 = *reinterpret_cast<const float4*>(&Ks[c16][64 * g + 4 * (u + 1)]);
                    n1 = *reinterpret_cast<const float4*>(&Ks[16 + c16][64 * g + 4 * (u + 1)]);
                }
                acc0 = mfma16(a0.x, qreg[4 * u], acc0);
                acc1 = mfma16(a1.x, qreg[4 * u], acc1);
                acc0 = mfma16(a0.y, qreg[4 * u + 1], acc0);
                acc1 = mfma16(a1.y, qreg[4 * u + 1], acc1);
                acc0 = mfma16(a0.z, qreg[4 * u + 2], acc0);
                acc1 = mfma16(a1.z, qreg[4 * u + 2], acc1);
                acc0 = mfma16(a0.w, qreg[4 * u + 3], acc0);
                acc1 = mfma16(a1.w, qreg[4 * u + 3], acc1);
                a0 = n0; a1 = n1;
            }
            st[0] = acc0; st[1] = acc1;
        }
        // Every wave is past S (the K tile is free) and the V tile is
        // stored: refill K, load the next V into registers.
        lds_barrier();
        if (it + 1 < n_iter) {
            load_k(p0 + KT);
            Q35_LOAD_TILE(p0 + KT)
        }
#undef Q35_LOAD_ROW
#undef Q35_LOAD_TILE
#undef Q35_STORE_ROW
        // Online softmax down this lane's query column.  A column with no
        // unmasked position yet (half 1 only) keeps m = -inf, l = 0, O = 0.
        float mt = m_run;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int p = p0 + 16 * pb + 4 * g + r;
                if (p >= my_len) st[pb][r] = -INFINITY;
                mt = fmaxf(mt, st[pb][r]);
            }
        mt = xor16_max(mt);
        mt = xor32_max(mt);
        const bool live = mt != -INFINITY;
        const float alpha = live ? __expf(m_run - mt) : 1.0f;
        float ls = 0.0f;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = live ? __expf(st[pb][r] - mt) : 0.0f;
                st[pb][r] = e;
                ls += e;
            }
        ls = xor16_sum(ls);
        ls = xor32_sum(ls);
        l_run = l_run * alpha + ls;
        m_run = mt;
        // O^T = alpha O^T + V^T P^T.
#pragma unroll
        for (int db = 0; db < 16; ++db) O[db] = O[db] * alpha;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int dq = 0; dq < 4; ++dq) {
                float4 v[4];
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    v[d] = *reinterpret_cast<const float4*>(&Vt[16 * (4 * dq + d) + c16][16 * pb + 4 * g]);
#pragma unroll
                for (int d = 0; d < 4; ++d) O[4 * dq + d] = mfma16(v[d].x, st[pb][0], O[4 * dq + d]);
#pragma unroll
                for (int d = 0; d < 4; ++d) O[4 * dq + d] = mfma16(v[d].y, st[pb][1], O[4 * dq + d]);
#pragma unroll
                for (int d = 0; d < 4; ++d) O[4 * dq + d] = mfma16(v[d].z, st[pb][2], O[4 * dq + d]);
#pragma unroll
                for (int d = 0; d < 4; ++d) O[4 * dq + d] = mfma16(v[d].w, st[pb][3], O[4 * dq + d]);
            }
    }
    // Merge: half 1 hands (m, l, O) to half 0 through LDS (the tile buffers,
    // free after the last barrier of the loop).
    static_assert(4 * 64 * 66 * sizeof(float) <= sizeof(Tiles), "merge exchange fits one half's tiles");
    float* xch = &smem[0].k[0][0];
    float* xo = xch + (size_t)(wave * 64 + lane) * 64;
    float* xml = xch + (size_t)4 * 64 * 64 + (size_t)(wave * 64 + lane) * 2;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (half == 1) {
#pragma unroll
        for (int db = 0; db < 16; ++db)
            *reinterpret_cast<float4*>(xo + 4 * db) = make_float4(O[db][0], O[db][1], O[db][2], O[db][3]);
        xml[0] = m_run;
        xml[1] = l_run;
    }
    __syncthreads();
    if (half == 1) return;
    const float m1 = xml[0], l1 = xml[1];
    const float m = fmaxf(m_run, m1);
    const float a0 = __expf(m_run - m), a1 = m1 == -INFINITY ? 0.0f : __expf(m1 - m);
    const float l = l_run * a0 + l1 * a1;
    const int t = r0 + c16;
    if (t >= T || !stores) return;
    const float inv = 1.0f / l;
    const float* grow = q_gate + (size_t)t * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd;
    float* orow = out + ((size_t)t * nh + h) * kHd;
#pragma unroll
    for (int db = 0; db < 16; ++db) {
        const int d0 = 16 * db + 4 * g;
        const float4 o1 = *reinterpret_cast<const float4*>(xo + 4 * db);
        const float4 gt = *reinterpret_cast<const float4*>(grow + d0);
        float4 r;
        r.x = (O[db][0] * a0 + o1.x * a1) * inv * (1.0f / (1.0f + expf(-gt.x)));
        r.y = (O[db][1] * a0 + o1.y * a1) * inv * (1.0f / (1.0f + expf(-gt.y)));
        r.z = (O[db][2] * a0 + o1.z * a1) * inv * (1.0f / (1.0f + expf(-gt.z)));
        r.w = (O[db][3] * a0 + o1.w * a1) * inv * (1.0f / (1.0f + expf(-gt.w)));
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
        hipExtLaunchKernelGGL(attn_prefill_flash, dim3((T + QR - 1) / QR * (d.nh / hg)), dim3(512), 0,
                           c->stream, ps_.a, ps_.b, 0, qbuf, K, V, q_gate, out, start, T, d.nh, d.nkv, hg,
                           c->cap);
    }
    return hipGetLastError();
}

}  // namespace q35
