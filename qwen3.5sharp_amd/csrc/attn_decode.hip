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
// A sequence at length pos attends over pos + 1 rows: the pos cached rows
// [0, pos) and the new row, which comes from the inputs.
//
// Pass 1 (attn_decode_partial): one workgroup per (sequence, kv head, chunk c
// of NSUB sub-chunks of R cached rows; R = 64, or 16 for batch-1 shapes).
// Chunk c holds the sub-chunks c, c + nchunks, c + 2 nchunks, ... so the
// workgroups of one cache that run together stream adjacent rows; the cached
// rows are split exactly, so the grid has no second round of workgroups that
// each hold a single row.  The 4 q heads of the kv head share every K/V row it
// reads, so each cache byte is read once per token.  A sub-chunk is processed
// with every K and V load issued before any arithmetic (R KiB of K and of V in
// flight per workgroup), which is what keeps HBM busy; the cache rows are
// loaded non-temporally (each is read once per token, and the caches of a
// long context do not fit the 256 MB MALL); the first
// sub-chunk's loads go out before the q preparation, so that preparation
// (each workgroup rotates and norms the 4 q rows, 4 KiB of input) costs no
// memory round trip of its own.  Chunk 0 also rotates/norms the new K row,
// writes K and V into the cache row pos (single writer; no workgroup reads
// that row from memory) and folds the new row into its softmax from LDS
// after its cached rows.  Every chunk emits, per q head, its max score m,
// sum of exp l and unnormalised o = sum exp(s - m) v.
// Pass 2 (attn_decode_merge): per (sequence, q head, 32-dim slice) the chunk
// partials are rescaled to the maximum of their maxima and summed, in one
// round of loads, and the sigmoid gate is applied.
//
// Online softmax is the two-pass softmax regrouped; it omits the reference's
// -80 floor on shifted logits, which only touches weights below e^-80
// relative to the row maximum (invisible in fp32 next to the maximum's 1).
#include <type_traits>

#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

constexpr int NT = 256;
constexpr int SUB = 64;   // positions per sub-chunk

template <int NSUB, int HPW, int R>
__global__ __launch_bounds__(NT, 2) void attn_decode_partial(
    const float* __restrict__ q_gate, const float* __restrict__ knew,
    const float* __restrict__ vnew, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    float* __restrict__ part_o, float* __restrict__ part_ml, const int* __restrict__ lens, int nkv, int ng,
    int cap, int nchunks, float eps, SeqBatch sb) {
    constexpr int QPW = (HPW + 3) / 4;       // q heads of the group per wave in per-head phases
    const int c = blockIdx.x, y = blockIdx.y, i = blockIdx.z;
    const int kvh = y / ng;                  // head group y: q heads HPW y .. HPW y + HPW - 1
    // Cached rows [0, pos); the new row is pos.  The host keeps every length
    // below the capacity; the clamp only keeps the row addresses in the cache.
    const int pos = min(lens[sb.seq[i]], cap - 1);
    const bool has_rows = c * R < pos;       // uniform
    const bool owner = c == 0;               // holds the new row
    const bool writer = owner && y % ng == 0;   // one group per kv head writes it to the cache
    if (!has_rows && !owner) return;
    const int last = max(pos - 1, 0);        // last cached row (row 0 when there is none)
    const int nh = nkv * ng * HPW;
    const int kv_dim = nkv * kHd;
    // Cache of one (sequence, kv head): [cap][256], head-major.
    const size_t seq_off = ((size_t)sb.seq[i] * nkv + kvh) * cap * kHd;
    float* K = k_cache + seq_off;
    float* V = v_cache + seq_off;
    // `wave` provably below 4, so per-head branches that every wave takes
    // (wave + 4 k < HPW for HPW >= 4) fold away.
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & (NT / kWave - 1);

    __shared__ float4 q_s[HPW][kHd / 4];
    __shared__ float4 knew_s[kHd / 4];
    __shared__ float4 vnew_s[kHd / 4];
    // Scores / weights and the rescale factors, double-buffered by sub-chunk
    // parity so two barriers per sub-chunk suffice.
    __shared__ float sc[2][HPW][SUB];
    __shared__ float al_s[2][HPW];
    __shared__ float nr_s[HPW][2];           // new row: rescale factor, weight
    __shared__ float ml_s[HPW][2];
    __shared__ float4 obuf[4][HPW][kHd / 4];

    // Score layout: 16 teams of 16 lanes, team t scores positions t + 16m
    // (m < 4); lane l16 holds dims {4*l16 + 64*j .. +3}, j < 4.
    // P.V layout: thread holds dims 4*d4..+3 of all HPW heads, positions ps + 4m.
    // Per-head phases (q preparation, softmax): wave w takes the group's heads
    // w, w + 4, ... (none when w >= HPW).
    const int team = tid >> 4, l16 = tid & 15;
    const int d4 = tid & 63, ps = tid >> 6;

    // Operands of the q / new-row preparation, loaded before the first
    // sub-chunk's K/V so that their latency hides behind it; waves 0 and 1 of
    // the owner also take the new K and V rows.
    float4 xq[QPW];
#pragma unroll
    for (int k = 0; k < QPW; ++k) {
        const int hh = min(wave + 4 * k, HPW - 1);
        xq[k] = *reinterpret_cast<const float4*>(
            q_gate + (size_t)i * 2 * nh * kHd + (size_t)(HPW * y + hh) * 2 * kHd + 4 * lane);
    }
    const float4 xn = *reinterpret_cast<const float4*>(
        (wave == 1 ? vnew : knew) + (size_t)i * kv_dim + kvh * kHd + 4 * lane);
    const float4 rc = *reinterpret_cast<const float4*>(rope_cos + (size_t)pos * kRopeHalf + 4 * (lane & 7));
    const float4 rs = *reinterpret_cast<const float4*>(rope_sin + (size_t)pos * kRopeHalf + 4 * (lane & 7));
    const float4 wq = *reinterpret_cast<const float4*>(q_norm + 4 * lane);
    const float4 wk = *reinterpret_cast<const float4*>(k_norm + 4 * lane);
    // Keeps these loads ahead of the K/V loads below (the compiler would
    // otherwise sink them to their uses, behind the cache rows, and the q
    // preparation would then wait for every row).
    asm volatile("" ::: "memory");

    // K/V rows of sub-chunk `S0` into kk / vv, all loads unconditional: rows
    // past the last cached row read that row instead (their scores are masked
    // to weight 0).
#define Q35_LOAD_K(S0)                                                                           \
    _Pragma("unroll") for (int m = 0; m < R / 16; ++m) {                                         \
        const float4* krow = reinterpret_cast<const float4*>(                                    \
            K + (size_t)min((S0) + team + 16 * m, last) * kHd);                                  \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) kk[m][j] = load_nt(&krow[l16 + 16 * j].x); \
    }
#define Q35_LOAD_V(S0)                                                                           \
    _Pragma("unroll") for (int m = 0; m < R / 4; ++m) {                                          \
        const float4* vrow = reinterpret_cast<const float4*>(                                    \
            V + (size_t)min((S0) + ps + 4 * m, last) * kHd);                                     \
        vv[m] = load_nt(&vrow[d4].x);                                                            \
    }

    // One sub-chunk at s0 from kk / vv: scores (q re-read from LDS per head,
    // so its registers are not held across the K/V loads), the online
    // softmax (lane = position) and P.V.  Score and weight buffers alternate
    // by sub-chunk parity PAR.
#define Q35_SCORE_ONE(m, h)                                                                      \
    {                                                                                            \
        float t = 0.0f;                                                                          \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                          \
            const float4 qj = q_s[h][l16 + 16 * j];                                              \
            t += qj.x * kk[m][j].x + qj.y * kk[m][j].y + qj.z * kk[m][j].z + qj.w * kk[m][j].w;  \
        }                                                                                        \
        a[m][h] = group_sum<16>(t);                                                              \
    }
    // With one sub-chunk a workgroup, its rows are scored in load order (row
    // block m outer), so the first blocks are scored while later K rows are
    // still arriving; pipelined sub-chunks keep each head's q in registers
    // across the four blocks instead.
#define Q35_SCORES(PAR)                                                                          \
    {                                                                                            \
        float a[R / 16][HPW];                                                                    \
        if constexpr (NSUB == 1) {                                                               \
            _Pragma("unroll") for (int m = 0; m < R / 16; ++m)                                   \
                _Pragma("unroll") for (int h = 0; h < HPW; ++h) Q35_SCORE_ONE(m, h)              \
        } else {                                                                                 \
            _Pragma("unroll") for (int h = 0; h < HPW; ++h) {                                    \
                float4 qh[4];                                                                    \
                _Pragma("unroll") for (int j = 0; j < 4; ++j) qh[j] = q_s[h][l16 + 16 * j];      \
                _Pragma("unroll") for (int m = 0; m < R / 16; ++m) {                             \
                    float t = 0.0f;                                                              \
                    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                \
                        t += qh[j].x * kk[m][j].x + qh[j].y * kk[m][j].y + qh[j].z * kk[m][j].z +\
                             qh[j].w * kk[m][j].w;                                               \
                    a[m][h] = group_sum<16>(t);                                                  \
                }                                                                                \
            }                                                                                    \
        }                                                                                        \
        if (l16 == 0)                                                                            \
            _Pragma("unroll") for (int m = 0; m < R / 16; ++m)                                   \
                _Pragma("unroll") for (int h = 0; h < HPW; ++h)                                  \
                    sc[PAR][h][team + 16 * m] = a[m][h];                                         \
    }
#define Q35_SOFTMAX_PV(PAR)                                                                      \
    {                                                                                            \
        const int np = min(R, pos - s0);                                                         \
        lds_barrier();                                                                           \
        _Pragma("unroll") for (int k = 0; k < QPW; ++k) {                                        \
            const int hh = wave + 4 * k;                                                         \
            if (hh < HPW) {                                                                      \
                const float s = lane < np ? sc[PAR][hh][lane] : -INFINITY;                       \
                const float mx = fmaxf(m_run[k], wave_max(s));                                   \
                const float e = lane < np ? __expf(s - mx) : 0.0f;                               \
                const float alpha = __expf(m_run[k] - mx);     /* 0 on the first sub-chunk */    \
                l_run[k] = l_run[k] * alpha + wave_sum(e);                                       \
                m_run[k] = mx;                                                                   \
                sc[PAR][hh][lane] = e;                                                           \
                if (lane == 0) al_s[PAR][hh] = alpha;                                            \
            }                                                                                    \
        }                                                                                        \
        lds_barrier();                                                                           \
        _Pragma("unroll") for (int h = 0; h < HPW; ++h) {                                        \
            const float alpha = al_s[PAR][h];                                                    \
            acc[h].x *= alpha; acc[h].y *= alpha; acc[h].z *= alpha; acc[h].w *= alpha;          \
        }                                                                                        \
        /* masked positions carry weight exactly 0 (their V rows are row last) */               \
        _Pragma("unroll") for (int m = 0; m < R / 4; ++m) {                                      \
            const int pp = ps + 4 * m;                                                           \
            _Pragma("unroll") for (int h = 0; h < HPW; ++h) {                                    \
                const float e = sc[PAR][h][pp];                                                  \
                acc[h].x += e * vv[m].x;                                                         \
                acc[h].y += e * vv[m].y;                                                         \
                acc[h].z += e * vv[m].z;                                                         \
                acc[h].w += e * vv[m].w;                                                         \
            }                                                                                    \
        }                                                                                        \
    }

    float m_run[QPW], l_run[QPW];            // the wave's heads
#pragma unroll
    for (int k = 0; k < QPW; ++k) {
        m_run[k] = -INFINITY;
        l_run[k] = 0.0f;
    }
    float4 acc[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);

    // The first sub-chunk's loads go out before the q preparation.
    int s0 = c * R;
    float4 kk[R / 16][4];
    float4 vv[R / 4];
    // Issued unconditionally (the owner of a sequence with no cached rows
    // reads row 0 and never uses it): behind a branch, the waits of the q
    // preparation below would also cover these loads.  K rows go out in
    // row-block order, then V, and stay in that order, so the scores of a
    // block wait on its K rows alone.
    Q35_LOAD_K(s0)
    __builtin_amdgcn_sched_barrier(0);
    Q35_LOAD_V(s0)
    __builtin_amdgcn_sched_barrier(0);
    // q rows (the attention scale 1/sqrt(256) folded in); the owner also
    // rotates/norms the new K row, and the writer writes K and V into the cache.
#pragma unroll
    for (int k = 0; k < QPW; ++k)
        if (wave + 4 * k < HPW)
            q_s[wave + 4 * k][lane] = rope_norm_regs(xq[k], rc, rs, wq, lane, eps, 1.0f / sqrtf((float)kHd));
    if (owner && wave < 2) {
        float4* dst = reinterpret_cast<float4*>((wave == 0 ? K : V) + (size_t)pos * kHd) + lane;
        if (wave == 0) {
            const float4 x = rope_norm_regs(xn, rc, rs, wk, lane, eps, 1.0f);
            knew_s[lane] = x;
            if (writer) *dst = x;
        } else {
            vnew_s[lane] = xn;
            if (writer) *dst = xn;
        }
    }
    lds_barrier();
    if (has_rows) {
        // Software pipeline: the next sub-chunk's K loads go out once the
        // scores have consumed kk, its V loads once P.V has consumed vv.  The
        // last sub-chunk runs after the loop, without loads for a next one.
        int sub = 0;
        for (;;) {
            const int s1 = s0 + nchunks * R;
            if (sub + 1 == NSUB || s1 >= pos) break;     // uniform across the workgroup
            const int par = sub & 1;
            Q35_SCORES(par)
            Q35_LOAD_K(s1)
            Q35_SOFTMAX_PV(par)
            Q35_LOAD_V(s1)
            ++sub;
            s0 = s1;
        }
        const int par = sub & 1;
        Q35_SCORES(par)
        Q35_SOFTMAX_PV(par)
    }
#undef Q35_LOAD_K
#undef Q35_LOAD_V
#undef Q35_SCORES
#undef Q35_SCORE_ONE
#undef Q35_SOFTMAX_PV

    if (owner) {
        // The new row, from LDS: each head's wave scores it against q and
        // folds it into the head's running softmax (m_run = -inf when the
        // sequence has no cached rows: alpha = 0).
#pragma unroll
        for (int k = 0; k < QPW; ++k) {
            const int hh = wave + 4 * k;
            if (hh < HPW) {
                const float4 qh = q_s[hh][lane], kn = knew_s[lane];
                const float s = wave_sum(qh.x * kn.x + qh.y * kn.y + qh.z * kn.z + qh.w * kn.w);
                const float mx = fmaxf(m_run[k], s);
                const float alpha = __expf(m_run[k] - mx);
                const float e = __expf(s - mx);
                l_run[k] = l_run[k] * alpha + e;
                m_run[k] = mx;
                if (lane == 0) {
                    nr_s[hh][0] = alpha;
                    nr_s[hh][1] = e;
                }
            }
        }
        lds_barrier();
        const float4 vn = vnew_s[d4];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            const float al = nr_s[h][0];
            const float en = ps == 0 ? nr_s[h][1] : 0.0f;    // added once per dim
            acc[h].x = acc[h].x * al + en * vn.x;
            acc[h].y = acc[h].y * al + en * vn.y;
            acc[h].z = acc[h].z * al + en * vn.z;
            acc[h].w = acc[h].w * al + en * vn.w;
        }
    }

#pragma unroll
    for (int h = 0; h < HPW; ++h) obuf[ps][h][d4] = acc[h];
#pragma unroll
    for (int k = 0; k < QPW; ++k)
        if (lane == 0 && wave + 4 * k < HPW) {
            ml_s[wave + 4 * k][0] = m_run[k];
            ml_s[wave + 4 * k][1] = l_run[k];
        }
    __syncthreads();
    for (int h = tid >> 6; h < HPW; h += 4) {
        float4 o = obuf[0][h][d4];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            const float4 t = obuf[q][h][d4];
            o.x += t.x; o.y += t.y; o.z += t.z; o.w += t.w;
        }
        const size_t pidx = (((size_t)i * nkv * ng + y) * nchunks + c) * HPW + h;
        reinterpret_cast<float4*>(part_o + pidx * kHd)[d4] = o;
        if (d4 == 0) {
            part_ml[2 * pidx] = ml_s[h][0];
            part_ml[2 * pidx + 1] = ml_s[h][1];
        }
    }
}

// Merge of the chunk partials of one (sequence, q head, 32-dim slice): 256
// threads.  Every wave forms the maximum M of the chunk maxima itself (its
// lanes stride the chunks; nothing is exchanged between waves).  Thread t
// holds 4 dims (d4 = t % 8) of the slice and sums the chunks t / 8, t / 8 +
// 32, ... weighted by w_c = e^{m_c - M}: l = sum w_c l_c, o = sum w_c o_c,
// up to MU chunks per thread with all their loads issued together with those
// of the maxima, so up to 128 chunks take one memory round trip and no
// exponential waits on another (a running log-sum-exp fold chains two per
// step).  The 32 partial sums of a column are added by butterfly within each
// wave (8 per wave) and then across the 4 waves in LDS.  Every chunk that ran
// holds at least one row (chunk 0 the new one), so M is finite.  The loads
// address all nchunks partials, not only the nc that ran, so they do not wait
// for the sequence length; partials past nc (not written by this call) are
// loaded and masked out by selects.
constexpr int MT = 256;
constexpr int MSLICE = 32;                 // dims per merge workgroup
constexpr int MD4 = MSLICE / 4;            // float4 columns per slice
constexpr int MG = MT / MD4;               // chunk groups
constexpr int MU = 4;                      // chunks per thread per round

__global__ __launch_bounds__(MT) void attn_decode_merge(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const float* __restrict__ q_gate, float* __restrict__ out, const int* __restrict__ lens, int nh, int hpw,
    int nchunks, int rows, int cap, SeqBatch sb) {
    const int h = blockIdx.x / (kHd / MSLICE), slice = blockIdx.x % (kHd / MSLICE);
    const int i = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int y = h / hpw, hl = h % hpw;     // head group of the partials
    const size_t base = ((size_t)i * (nh / hpw) + y) * nchunks;
    __shared__ float4 obuf[4][MD4];
    __shared__ float lbuf[4];

    const int d4 = t % MD4, g = t / MD4;
    const int col = slice * MD4 + d4;
    // Gate of this thread's 4 output dims (used by wave 0's first MD4 lanes).
    const int dim = slice * MSLICE + 4 * d4;
    const float4 gt = *reinterpret_cast<const float4*>(
        q_gate + (size_t)i * 2 * nh * kHd + (size_t)h * 2 * kHd + kHd + dim);

    float mc[MU], lc[MU];
    float4 oc[MU];
    auto load_round = [&](int c0) {
#pragma unroll
        for (int u = 0; u < MU; ++u) {
            const size_t pidx = (base + min(c0 + u * MG, nchunks - 1)) * hpw + hl;
            mc[u] = part_ml[2 * pidx];
            lc[u] = part_ml[2 * pidx + 1];
            oc[u] = reinterpret_cast<const float4*>(part_o + pidx * kHd)[col];
        }
    };
    load_round(g);
    float mw[2];                             // the maxima of chunks lane, lane + 64
#pragma unroll
    for (int k = 0; k < 2; ++k) mw[k] = part_ml[2 * ((base + min(lane + kWave * k, nchunks - 1)) * hpw + hl)];
    const int pos = min(lens[sb.seq[i]], cap - 1);
    const int nc = max(1, min(nchunks, (pos + rows - 1) / rows));   // chunks that ran
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < 2; ++k) M = fmaxf(M, lane + kWave * k < nc ? mw[k] : -INFINITY);
    for (int c = lane + 2 * kWave; c < nc; c += kWave) M = fmaxf(M, part_ml[2 * ((base + c) * hpw + hl)]);
    M = wave_max(M);

    float l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = g; c0 < nc; c0 += MG * MU) {
        if (c0 != g) load_round(c0);
#pragma unroll
        for (int u = 0; u < MU; ++u)
            if (c0 + u * MG < nc) {
                const float wc = __expf(mc[u] - M);
                l = fmaf(wc, lc[u], l);
                o.x = fmaf(wc, oc[u].x, o.x);
                o.y = fmaf(wc, oc[u].y, o.y);
                o.z = fmaf(wc, oc[u].z, o.z);
                o.w = fmaf(wc, oc[u].w, o.w);
            }
    }
    // Butterfly over the 8 groups of each wave (lanes d4 + 8 k share a column).
#pragma unroll
    for (int k = MD4; k < kWave; k <<= 1) {
        l += __shfl_xor(l, k, kWave);
        o.x += __shfl_xor(o.x, k, kWave);
        o.y += __shfl_xor(o.y, k, kWave);
        o.z += __shfl_xor(o.z, k, kWave);
        o.w += __shfl_xor(o.w, k, kWave);
    }
    if (lane < MD4) {
        obuf[wave][lane] = o;
        if (lane == 0) lbuf[wave] = l;
    }
    __syncthreads();
    if (t < MD4) {
        const float4 o1 = obuf[1][t], o2 = obuf[2][t], o3 = obuf[3][t];
        o.x = (o.x + o1.x) + (o2.x + o3.x);
        o.y = (o.y + o1.y) + (o2.y + o3.y);
        o.z = (o.z + o1.z) + (o2.z + o3.z);
        o.w = (o.w + o1.w) + (o2.w + o3.w);
        const float inv = 1.0f / ((l + lbuf[1]) + (lbuf[2] + lbuf[3]));
        float4 r;
        r.x = o.x * inv * (1.0f / (1.0f + expf(-gt.x)));
        r.y = o.y * inv * (1.0f / (1.0f + expf(-gt.y)));
        r.z = o.z * inv * (1.0f / (1.0f + expf(-gt.z)));
        r.w = o.w * inv * (1.0f / (1.0f + expf(-gt.w)));
        *reinterpret_cast<float4*>(out + (size_t)i * nh * kHd + (size_t)h * kHd + dim) = r;
    }
}

// Sub-chunks of `rows` rows in a cached range of max_cached rows.
int max_subchunks(int max_cached, int rows) { return (max_cached + rows - 1) / rows; }

// q heads per workgroup: the whole group of a kv head up to 8 (1, 2, 4 or 8),
// groups of 8 beyond (each re-reads the kv head's cache).
int heads_per_wg(const Dims& d) {
    const int g = d.nh / d.nkv;
    return g <= 8 ? g : 8;
}

// Split of one call: rows per sub-chunk, sub-chunks per workgroup (NSUB),
// workgroups per head group (chunks), for ng = sequences x head groups and
// the longest cached range.  Two workgroups fit a CU (slots = 2 x CUs):
//  - fewer 64-row sub-chunks than CUs in all: one sub-chunk a workgroup;
//  - else 16-row sub-chunks spread over one round of workgroups (slots / ng
//    per head group), when at most 8 per workgroup cover the rows: each
//    workgroup holds one 16-row sub-chunk's loads in flight at a time,
//    refilled by the software pipeline, instead of 64 rows at once.  Up to 4
//    a workgroup, the rows go as 4 per workgroup (fewer, longer workgroups);
//  - else 64-row sub-chunks, 4 a workgroup if that keeps one round, else 8.
// Measured per call, partial + merge, batch 1 unless stated: 8193 rows 17.9 us
// as 4 x 16 rows (15.6 us partial as 1 x 64 before: 19.5 us); 8320 rows 19.5
// us as 8 x 16 (2 x 64 rows: 24.5, 1 x 64: 21.7); 12288 rows 22.9 (2 x 64:
// 26.3); 16384 rows 28.0 (4 x 64: 28.2, 2 x 64: 28.9); two sequences at 8192
// rows 28.0 (2 x 64: 28.7); four at 4096 rows 28.3 (4 x 64: 28.3, 2 x 64:
// 29.0); 32767 rows 47.8 as 4 x 64 (8 x 64: 46.7, 8 x 16: 49.4).  For the
// 8-sequence 32K stack, 16 sub-chunks of 32 rows or 32 of 16 measured
// 332-334 against 327 us as 8 x 64.
DecodePlan plan_decode(const Dims& d, int n, int max_cached, int n_cu) {
    const long ng = (long)n * (d.nh / heads_per_wg(d));
    const long slots = 2L * n_cu;
    const int max64 = max_subchunks(max_cached, SUB);
    const int max16 = max_subchunks(max_cached, SUB / 4);
    // (With 8 q heads a workgroup the one-sub-chunk kernel needs more than
    // 256 VGPRs; the same 64 rows a workgroup go as 4 x 16 rows instead.)
    if (ng * max64 < n_cu)
        return heads_per_wg(d) >= 8 ? DecodePlan{SUB / 4, 4, max(1, (max16 + 3) / 4)} : DecodePlan{SUB, 1, max(1, max64)};
    const int nch = (int)max(1L, slots / ng);
    const int need = (max16 + nch - 1) / nch;
    if (need <= 4) return {SUB / 4, 4, max(1, (max16 + 3) / 4)};
    if (need <= 8) return {SUB / 4, 8, nch};
    if (ng * ((max64 + 3) / 4) <= slots) return {SUB, 4, (max64 + 3) / 4};
    return {SUB, 8, (max64 + 7) / 8};
}

}  // namespace

DecodePlan plan_attn_decode(const q35m_ctx* c, int n, int max_cached) {
    return plan_decode(c->d, n, max_cached, c->n_cu);
}

// Fixed device scratch of q35m_attn_decode_noalloc: the split-K partials of
// one call (kNoAllocScratchBytes).  Every GPU the library runs on holds its
// own copy until the process ends.  Host code never passes this name to a
// kernel (on the host it is only a stand-in for the symbol): it uses the
// device address that attn_decode_scratch_address returns.
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

hipError_t attn_decode_scratch_address(float** ptr) {
    return hipGetSymbolAddress(reinterpret_cast<void**>(ptr), HIP_SYMBOL(scratch));
}

size_t attn_decode_work_bytes(const q35m_ctx* c, int n, const DecodePlan& p) {
    return (size_t)n * c->d.nh * p.nchunks * (kHd + 2) * sizeof(float);
}

hipError_t launch_attn_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const DecodePlan& p,
                              const float* q_gate, const float* k, const float* v, float* out, float* work) {
    const Dims& d = c->d;
    const AttnLayer& L = c->full[layer];
    const int hpw = heads_per_wg(d);
    const int groups = d.nh / hpw, ng = groups / d.nkv;
    const int nsub = p.nsub, nchunks = p.nchunks;
    float* part_o = work;
    float* part_ml = part_o + (size_t)sb.n * d.nh * nchunks * kHd;
    const dim3 grid(nchunks, groups, sb.n);
    {
        const int kid = p.rows != SUB ? (nsub == 8 ? K_ATTN_DECODE_PARTIAL8R16 : K_ATTN_DECODE_PARTIAL4R16)
                      : nsub == 8 ? K_ATTN_DECODE_PARTIAL8
                      : nsub == 4 ? K_ATTN_DECODE_PARTIAL4 : K_ATTN_DECODE_PARTIAL1;
        ProfScope ps_(c, kid);
        auto go = [&](auto kern) {
            hipExtLaunchKernelGGL(kern, grid, dim3(NT), 0, c->stream, ps_.a, ps_.b, 0, q_gate, k, v, L.q_norm,
                                  L.k_norm, L.k_cache, L.v_cache, c->rope_cos, c->rope_sin, part_o, part_ml,
                                  c->dev_len, d.nkv, ng, c->cap, nchunks, d.eps, sb);
        };
        auto by_nsub = [&](auto h) {
            constexpr int H = decltype(h)::value;
            if (p.rows != SUB) {
                if (nsub == 8) go(attn_decode_partial<8, H, SUB / 4>);
                else go(attn_decode_partial<4, H, SUB / 4>);
            }
            else if (nsub == 8) go(attn_decode_partial<8, H, SUB>);
            else if (nsub == 4) go(attn_decode_partial<4, H, SUB>);
            else if constexpr (H < 8) go(attn_decode_partial<1, H, SUB>);
        };
        if (hpw == 8) by_nsub(std::integral_constant<int, 8>());
        else if (hpw == 4) by_nsub(std::integral_constant<int, 4>());
        else if (hpw == 2) by_nsub(std::integral_constant<int, 2>());
        else by_nsub(std::integral_constant<int, 1>());
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    {
        ProfScope ps_(c, K_ATTN_DECODE_MERGE);
        hipExtLaunchKernelGGL(attn_decode_merge, dim3(d.nh * (kHd / MSLICE), sb.n), dim3(MT), 0, c->stream,
                              ps_.a, ps_.b, 0, part_o, part_ml, q_gate, out, c->dev_len, d.nh, hpw, nchunks,
                              p.rows, c->cap, sb);
    }
    return hipGetLastError();
}

}  // namespace q35
