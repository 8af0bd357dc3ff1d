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
// Pass 1 (attn_decode_partial): one workgroup per (sequence, kv head, chunk c
// of NSUB 64-row sub-chunks).  Chunk c holds the sub-chunks c, c + nchunks,
// c + 2 nchunks, ... so the workgroups of one cache that run together stream
// adjacent rows.  The 4 q heads of the kv head share every K/V row it reads,
// so each cache byte is read once per token.  A sub-chunk is processed with
// every K and V load issued before any arithmetic (64 KiB of K and 64 KiB of
// V in flight per workgroup), which is what keeps HBM busy; the first
// sub-chunk's loads go out before the q preparation, so that preparation
// (each workgroup rotates and norms the 4 q rows, 4 KiB of input) costs no
// memory round trip of its own.  The workgroup that holds the new position
// also rotates/norms the new K row, writes K and V into the cache (single
// writer) and takes them from LDS.  It emits, per q head, the chunk's max
// score m, sum of exp l and unnormalised o = sum exp(s - m) v.
// Pass 2 (attn_decode_merge): per (sequence, q head) the chunks are merged by
// log-sum-exp rescaling and the sigmoid gate is applied.
//
// Online softmax is the two-pass softmax regrouped; it omits the reference's
// -80 floor on shifted logits, which only touches weights below e^-80
// relative to the row maximum (invisible in fp32 next to the maximum's 1).
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int NT = 256;
constexpr int SUB = 64;   // positions per sub-chunk

__device__ __forceinline__ float4 sel4(bool c, float4 a, float4 b) {
    return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

template <int NSUB>
__global__ __launch_bounds__(NT, 2) void attn_decode_partial(
    const float* __restrict__ q_gate, const float* __restrict__ knew,
    const float* __restrict__ vnew, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    float* __restrict__ part_o, float* __restrict__ part_ml, int nkv, int cap, int nchunks,
    float eps, SeqBatch sb) {
    const int c = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
    const int pos = sb.pos[i];
    // Workgroup c takes the sub-chunks c, c + nchunks, c + 2 nchunks, ...: the
    // workgroups of one cache that run together read adjacent rows.
    if (c * SUB > pos) return;
    const int nh = nkv * kGqaGroup;
    const int kv_dim = nkv * kHd;
    // Cache of one (sequence, kv head): [cap][256], head-major.
    const size_t seq_off = ((size_t)sb.seq[i] * nkv + kvh) * cap * kHd;
    float* K = k_cache + seq_off;
    float* V = v_cache + seq_off;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    __shared__ float4 q_s[kGqaGroup][kHd / 4];
    __shared__ float4 knew_s[kHd / 4];
    __shared__ float4 vnew_s[kHd / 4];
    // Scores / weights and the rescale factors, double-buffered by sub-chunk
    // parity so two barriers per sub-chunk suffice.
    __shared__ float sc[2][kGqaGroup][SUB];
    __shared__ float al_s[2][kGqaGroup];
    __shared__ float ml_s[kGqaGroup][2];
    __shared__ float4 obuf[4][kGqaGroup][kHd / 4];

    // Score layout: 16 teams of 16 lanes, team t scores positions t + 16m
    // (m < 4); lane l16 holds dims {4*l16 + 64*j .. +3}, j < 4.
    // P.V layout: thread holds dims 4*d4..+3 of all 4 heads, positions ps + 4m.
    const int team = tid >> 4, l16 = tid & 15;
    const int d4 = tid & 63, ps = tid >> 6;
    const bool owner = (pos / SUB) % nchunks == c;   // holds the new position

    // Operands of the q / new-row preparation, loaded before the first
    // sub-chunk's K/V so that their latency hides behind it: wave w prepares
    // q of head 4 kvh + w; waves 0 and 1 also take the new K and V rows.
    const int hq = kvh * kGqaGroup + wave;
    const float4 xq = *reinterpret_cast<const float4*>(
        q_gate + (size_t)i * 2 * nh * kHd + (size_t)hq * 2 * kHd + 4 * lane);
    const float4 xn = *reinterpret_cast<const float4*>(
        (wave == 1 ? vnew : knew) + (size_t)i * kv_dim + kvh * kHd + 4 * lane);
    const float4 rc = *reinterpret_cast<const float4*>(rope_cos + (size_t)pos * kRopeHalf + 4 * (lane & 7));
    const float4 rs = *reinterpret_cast<const float4*>(rope_sin + (size_t)pos * kRopeHalf + 4 * (lane & 7));
    const float4 wq = *reinterpret_cast<const float4*>(q_norm + 4 * lane);
    const float4 wk = *reinterpret_cast<const float4*>(k_norm + 4 * lane);

    // K/V rows of sub-chunk `S0` into kk / vv, all loads unconditional: rows
    // past pos read row pos instead (its scores are masked, its V rows are
    // zeroed before P.V), and row pos itself, which this launch writes, is
    // replaced by the new row from LDS.
#define Q35_LOAD_K(S0)                                                                           \
    _Pragma("unroll") for (int m = 0; m < 4; ++m) {                                              \
        const float4* krow = reinterpret_cast<const float4*>(                                    \
            K + (size_t)min((S0) + team + 16 * m, pos) * kHd);                                   \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) kk[m][j] = krow[l16 + 16 * j];             \
    }
#define Q35_LOAD_V(S0)                                                                           \
    _Pragma("unroll") for (int m = 0; m < 16; ++m) {                                             \
        const float4* vrow = reinterpret_cast<const float4*>(                                    \
            V + (size_t)min((S0) + ps + 4 * m, pos) * kHd);                                      \
        vv[m] = vrow[d4];                                                                        \
    }

    // One sub-chunk at s0 from kk / vv: scores (q re-read from LDS per head,
    // so its 64 registers per thread are not held across the K/V loads), the
    // online softmax (wave h owns head h, lane = position) and P.V.  Score and
    // weight buffers alternate by sub-chunk parity PAR.
#define Q35_SCORES(PAR)                                                                          \
    {                                                                                            \
        if (owner) {                           /* uniform: the new K row from LDS */             \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                      \
                const float4 kn = knew_s[l16 + 16 * j];                                          \
                _Pragma("unroll") for (int m = 0; m < 4; ++m)                                    \
                    kk[m][j] = sel4(s0 + team + 16 * m == pos, kn, kk[m][j]);                    \
            }                                                                                    \
        }                                                                                        \
        float a[4][kGqaGroup];                                                                   \
        _Pragma("unroll") for (int h = 0; h < kGqaGroup; ++h) {                                  \
            float4 qh[4];                                                                        \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) qh[j] = q_s[h][l16 + 16 * j];          \
            _Pragma("unroll") for (int m = 0; m < 4; ++m) {                                      \
                float t = 0.0f;                                                                  \
                _Pragma("unroll") for (int j = 0; j < 4; ++j)                                    \
                    t += qh[j].x * kk[m][j].x + qh[j].y * kk[m][j].y + qh[j].z * kk[m][j].z +    \
                         qh[j].w * kk[m][j].w;                                                   \
                a[m][h] = group_sum<16>(t);                                                      \
            }                                                                                    \
        }                                                                                        \
        if (l16 == 0)                                                                            \
            _Pragma("unroll") for (int m = 0; m < 4; ++m)                                        \
                _Pragma("unroll") for (int h = 0; h < kGqaGroup; ++h)                            \
                    sc[PAR][h][team + 16 * m] = a[m][h];                                         \
    }
#define Q35_SOFTMAX_PV(PAR)                                                                      \
    {                                                                                            \
        const int np = min(SUB, pos + 1 - s0);                                                   \
        lds_barrier();                                                                           \
        {                                                                                        \
            const float s = lane < np ? sc[PAR][wave][lane] : -INFINITY;                         \
            const float mx = fmaxf(m_run, wave_max(s));                                          \
            const float e = lane < np ? __expf(s - mx) : 0.0f;                                   \
            const float alpha = __expf(m_run - mx);     /* 0 on the first sub-chunk */           \
            l_run = l_run * alpha + wave_sum(e);                                                 \
            m_run = mx;                                                                          \
            sc[PAR][wave][lane] = e;                                                             \
            if (lane == 0) al_s[PAR][wave] = alpha;                                              \
        }                                                                                        \
        lds_barrier();                                                                           \
        _Pragma("unroll") for (int h = 0; h < kGqaGroup; ++h) {                                  \
            const float alpha = al_s[PAR][h];                                                    \
            acc[h].x *= alpha; acc[h].y *= alpha; acc[h].z *= alpha; acc[h].w *= alpha;          \
        }                                                                                        \
        if (owner || np < SUB) {               /* uniform: rows past pos, the new V row */        \
            const float4 vn = vnew_s[d4];                                                        \
            _Pragma("unroll") for (int m = 0; m < 16; ++m) {                                     \
                const int pp = ps + 4 * m;                                                       \
                vv[m] = sel4(pp >= np, make_float4(0.f, 0.f, 0.f, 0.f),                          \
                             sel4(s0 + pp == pos, vn, vv[m]));                                   \
            }                                                                                    \
        }                                                                                        \
        _Pragma("unroll") for (int m = 0; m < 16; ++m) {                                         \
            const int pp = ps + 4 * m;                                                           \
            _Pragma("unroll") for (int h = 0; h < kGqaGroup; ++h) {                              \
                const float e = sc[PAR][h][pp];                                                  \
                acc[h].x += e * vv[m].x;                                                         \
                acc[h].y += e * vv[m].y;                                                         \
                acc[h].z += e * vv[m].z;                                                         \
                acc[h].w += e * vv[m].w;                                                         \
            }                                                                                    \
        }                                                                                        \
    }

    float m_run = -INFINITY, l_run = 0.0f;     // per head (wave = head in the softmax step)
    float4 acc[kGqaGroup];
#pragma unroll
    for (int h = 0; h < kGqaGroup; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);

    // The first sub-chunk's loads go out before the q preparation.
    int s0 = c * SUB;
    float4 kk[4][4];
    float4 vv[16];
    Q35_LOAD_K(s0)
    Q35_LOAD_V(s0)
    // q rows (the attention scale 1/sqrt(256) folded in); the owner also
    // rotates/norms the new K row and writes K and V into the cache.
    q_s[wave][lane] = rope_norm_regs(xq, rc, rs, wq, lane, eps, 1.0f / sqrtf((float)kHd));
    if (owner && wave < 2) {
        float4* dst = reinterpret_cast<float4*>((wave == 0 ? K : V) + (size_t)pos * kHd) + lane;
        if (wave == 0) {
            const float4 x = rope_norm_regs(xn, rc, rs, wk, lane, eps, 1.0f);
            knew_s[lane] = x;
            *dst = x;
        } else {
            vnew_s[lane] = xn;
            *dst = xn;
        }
    }
    lds_barrier();
    // Software pipeline: the next sub-chunk's K loads go out once the scores
    // have consumed kk, its V loads once P.V has consumed vv.
    // The last sub-chunk runs after the loop, without loads for a next one.
    int sub = 0;
    for (;;) {
        const int s1 = s0 + nchunks * SUB;
        if (sub + 1 == NSUB || s1 > pos) break;     // uniform across the workgroup
        const int par = sub & 1;
        Q35_SCORES(par)
        Q35_LOAD_K(s1)
        Q35_SOFTMAX_PV(par)
        Q35_LOAD_V(s1)
        ++sub;
        s0 = s1;
    }
    {
        const int par = sub & 1;
        Q35_SCORES(par)
        Q35_SOFTMAX_PV(par)
    }
#undef Q35_LOAD_K
#undef Q35_LOAD_V
#undef Q35_SCORES
#undef Q35_SOFTMAX_PV

#pragma unroll
    for (int h = 0; h < kGqaGroup; ++h) obuf[ps][h][d4] = acc[h];
    if (lane == 0) {
        ml_s[wave][0] = m_run;
        ml_s[wave][1] = l_run;
    }
    __syncthreads();
    {
        const int h = tid >> 6;
        float4 o = obuf[0][h][d4];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            const float4 t = obuf[q][h][d4];
            o.x += t.x; o.y += t.y; o.z += t.z; o.w += t.w;
        }
        const size_t pidx = (((size_t)i * nkv + kvh) * nchunks + c) * kGqaGroup + h;
        reinterpret_cast<float4*>(part_o + pidx * kHd)[d4] = o;
        if (d4 == 0) {
            part_ml[2 * pidx] = ml_s[h][0];
            part_ml[2 * pidx + 1] = ml_s[h][1];
        }
    }
}

// Merge of the chunk partials of one (sequence, q head, 64-dim slice): 256
// threads; thread holds 4 dims (d4 = t % 16) of the slice and folds the
// chunks c = t / 16 (mod 16) into a running (m, l, o) by log-sum-exp
// rescaling, MU chunks per round with all their loads issued together; the 16
// running triples of a column are then folded the same way through LDS.  One
// memory round trip per MU chunks (the gate is loaded up front).
constexpr int MT = 256;
constexpr int MSLICE = 64;                 // dims per merge workgroup
constexpr int MD4 = MSLICE / 4;            // float4 columns per slice
constexpr int MG = MT / MD4;               // chunk groups
constexpr int MU = 4;                      // chunks per thread per round

__global__ __launch_bounds__(MT) void attn_decode_merge(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const float* __restrict__ q_gate, float* __restrict__ out, int nkv, int nchunks, SeqBatch sb) {
    const int h = blockIdx.x / (kHd / MSLICE), slice = blockIdx.x % (kHd / MSLICE);
    const int i = blockIdx.y, t = threadIdx.x;
    const int nh = nkv * kGqaGroup;
    const int kvh = h / kGqaGroup, hl = h % kGqaGroup;
    const int nc = min(nchunks, sb.pos[i] / SUB + 1);
    const size_t base = ((size_t)i * nkv + kvh) * nchunks;
    __shared__ float4 obuf[MG][MD4];
    __shared__ float mbuf[MG], lbuf[MG];

    const int d4 = t % MD4, g = t / MD4;
    const int col = slice * MD4 + d4;
    // Gate of this thread's 4 output dims (used by threads t < MD4).
    const int dim = slice * MSLICE + 4 * d4;
    const float4 gt = *reinterpret_cast<const float4*>(
        q_gate + (size_t)i * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd + dim);

    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = g; c0 < nc; c0 += MG * MU) {
        float mc[MU], lc[MU];
        float4 oc[MU];
#pragma unroll
        for (int u = 0; u < MU; ++u) {
            const size_t pidx = (base + min(c0 + u * MG, nc - 1)) * kGqaGroup + hl;
            mc[u] = part_ml[2 * pidx];
            lc[u] = part_ml[2 * pidx + 1];
            oc[u] = reinterpret_cast<const float4*>(part_o + pidx * kHd)[col];
        }
#pragma unroll
        for (int u = 0; u < MU; ++u) {
            const bool valid = c0 + u * MG < nc;
            const float mn = valid ? fmaxf(m, mc[u]) : m;
            const float a = __expf(m - mn);             // 0 while m is -inf
            const float b = valid ? __expf(mc[u] - mn) : 0.0f;
            l = l * a + lc[u] * b;
            o.x = o.x * a + oc[u].x * b;
            o.y = o.y * a + oc[u].y * b;
            o.z = o.z * a + oc[u].z * b;
            o.w = o.w * a + oc[u].w * b;
            m = mn;
        }
    }
    obuf[g][d4] = o;
    if (d4 == 0) {
        mbuf[g] = m;
        lbuf[g] = l;
    }
    __syncthreads();
    if (t < MD4) {
        float M = mbuf[0];
#pragma unroll
        for (int w = 1; w < MG; ++w) M = fmaxf(M, mbuf[w]);
        float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < MG; ++w) {
            const float f = __expf(mbuf[w] - M);        // 0 for groups without chunks
            const float4 ow = obuf[w][t];
            s.x += ow.x * f; s.y += ow.y * f; s.z += ow.z * f; s.w += ow.w * f;
            L += lbuf[w] * f;
        }
        const float inv = 1.0f / L;
        float4 r;
        r.x = s.x * inv * (1.0f / (1.0f + expf(-gt.x)));
        r.y = s.y * inv * (1.0f / (1.0f + expf(-gt.y)));
        r.z = s.z * inv * (1.0f / (1.0f + expf(-gt.z)));
        r.w = s.w * inv * (1.0f / (1.0f + expf(-gt.w)));
        *reinterpret_cast<float4*>(out + (size_t)i * nh * kHd + (size_t)h * kHd + dim) = r;
    }
}

// Sub-chunks per workgroup: as many as keep >= 1024 workgroups (4 per CU),
// at most 8, so partials stay small next to the cache they summarise.
int pick_nsub(int n, int nkv, int max_len) {
    for (int ns = 8; ns > 1; ns >>= 1)
        if ((long)n * nkv * ((max_len + SUB * ns - 1) / (SUB * ns)) >= 1024) return ns;
    return 1;
}

}  // namespace

size_t attn_decode_work_bytes(const Dims& d, int n, int max_kv_len) {
    const int chunk = SUB * pick_nsub(n, d.nkv, max_kv_len);
    const size_t nchunks = (max_kv_len + chunk - 1) / chunk;
    return (size_t)n * d.nkv * nchunks * kGqaGroup * (kHd + 2) * sizeof(float);
}

hipError_t launch_attn_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* q_gate,
                              const float* k, const float* v, float* out) {
    const Dims& d = c->d;
    const AttnLayer& L = c->full[layer];
    int max_len = 0;
    for (int i = 0; i < sb.n; ++i) max_len = max(max_len, sb.pos[i] + 1);
    const int nsub = pick_nsub(sb.n, d.nkv, max_len);
    const int chunk = SUB * nsub;
    const int nchunks = (max_len + chunk - 1) / chunk;
    float* part_o = c->work;
    float* part_ml = part_o + (size_t)sb.n * d.nkv * nchunks * kGqaGroup * kHd;
    const dim3 grid(nchunks, d.nkv, sb.n);
    {
        ProfScope ps_(c, K_ATTN_DECODE_PARTIAL);
#define Q35_PARTIAL(NS)                                                                          \
    hipExtLaunchKernelGGL(attn_decode_partial<NS>, grid, dim3(NT), 0, c->stream, ps_.a, ps_.b, 0, q_gate, k, v,      \
                       L.q_norm, L.k_norm, L.k_cache, L.v_cache, c->rope_cos, c->rope_sin,       \
                       part_o, part_ml, d.nkv, c->cap, nchunks, d.eps, sb)
        if (nsub == 8) Q35_PARTIAL(8);
        else if (nsub == 4) Q35_PARTIAL(4);
        else if (nsub == 2) Q35_PARTIAL(2);
        else Q35_PARTIAL(1);
#undef Q35_PARTIAL
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_ATTN_DECODE_MERGE);
        hipExtLaunchKernelGGL(attn_decode_merge, dim3(d.nh * (kHd / MSLICE), sb.n), dim3(MT), 0, c->stream, ps_.a, ps_.b, 0, part_o,
                           part_ml, q_gate, out, d.nkv, nchunks, sb);
    }
    return hipGetLastError();
}

}  // namespace q35
