// Gated-DeltaNet prefill mixer for T tokens of one sequence: chunked WY form
// (chunk C = 64) on fp32 MFMA.
//
// Reference: Qwen35Model.PrefillLinearAttn steps 2-6
// (src/Qwen35Sharp.Model/Qwen35Model.Prefill.cs:181-260), whose recurrence is
// the sequential GatedDeltaNetOps.RecurrentGatedDeltaRule
// (GatedDeltaNetOps.cs:107-229).  Per head and token, with decay a_t = e^{g_t}:
//   S_t = a_t S_{t-1} + k_t d_t^T,  d_t = beta_t (v_t - a_t S_{t-1}^T k_t),
//   o_t = S_t^T q_t.
// Within a chunk whose state on entry is S0, with G_i = g_0 + ... + g_i and
// gamma_i = e^{G_i}, unrolling the recurrence gives (Yang et al., "Gated Delta
// Networks", arXiv:2412.06464; "Parallelizing Linear Transformers with the
// Delta Rule over Sequence Length", arXiv:2406.06484):
//   (I + A) D = diag(beta) (V - diag(gamma) K S0),
//       A_ij = beta_i e^{G_i - G_j} (k_i . k_j) for j < i (strictly lower)
//   D = U - W S0,  U = T diag(beta) V,  W = T diag(beta gamma) K,  T = (I+A)^-1
//   O = diag(gamma) Q S0 + (M o Q K^T) D,  M_ij = e^{G_i - G_j} for j <= i
//   S_C = gamma_last S0 + K^T diag(e^{G_last - G}) D
// Only e^{G_i - G_j} with j <= i (never e^{G_i} e^{-G_j}) is formed, with G
// accumulated in fp64, so nothing overflows and the decays of long chunks
// (G reaches ~ -2000) keep full fp32 accuracy.
//
// Kernels:
//  1. deltanet_conv_writeback (T < K-1 only): the conv window write-back
//     reproducing the reference's read past the channel row.
//  2. dn_chunk_prep (one workgroup per k-head and chunk; the R v-heads of the
//     k-head share K K^T and Q K^T): the zero-padded causal conv with the
//     prefill tap order (tap j multiplies x[t-j], GatedDeltaNetOps.cs:27-53)
//     + SiLU of the chunk's q, k and v channels, read straight from the
//     token-major qkv; q/k L2 norm (q also scaled by 1/sqrt(dk)); beta =
//     sigmoid(b), g = ssm_a * softplus(a + dt_bias) (Prefill.cs:239-248); for
//     T >= K-1 the conv window <- last K-1 raw inputs (Prefill.cs:192-204).
//     Then K K^T and Q K^T on MFMA, the decay masks, T = (I+A)^-1 by blocked
//     forward substitution (16x16 diagonal blocks inverted in registers,
//     off-diagonal blocks applied on MFMA), and W and U on MFMA.  Emits q^,
//     k^, W, U, M o QK^T, gamma, e^{G_last - G}.
//  3. dn_chunk_scan (one workgroup per v-head and 16-column tile of the
//     state): the only sequential part.  Four waves walk the chunks in order
//     with the state tile in MFMA accumulators, record D = U - W S of every
//     chunk, and apply S = gamma_last S + K^T (e^{G_last-G} D); four more
//     waves form the inter-chunk output diag(gamma) Q S of every chunk from
//     the entry state the first four leave in LDS, so the states themselves
//     never go to memory.  Column tiles are independent (the rule is
//     separable over dv), so 8 workgroups per head run in parallel; the 8
//     tiles of a head share an XCD so W, Q and K stay in its L2.
//  4. dn_chunk_out (one workgroup per v-head and chunk, all in parallel):
//     O = diag(gamma) Q S + (M o QK^T) D from the recorded inter-chunk output
//     and D, with the gated RMSNorm fused into the epilogue.
//
// MFMA: v_mfma_f32_16x16x4f32.  Lane l = 16g + c holds A[c][g] and B[g][c];
// D register r holds D[4g + r][c].  A 16-deep product is 4 instructions; in
// instruction s lane group g supplies reduction index 4g + s, so a D tile can
// be fed back as the B operand register by register.
#include "common.h"
#include "q35mix_internal.h"

namespace q35 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc += A(16x16 block, float4 per lane = reduction 4g..4g+3) * B(D-layout tile)
__device__ __forceinline__ f32x4 mfma16x4(float4 a, f32x4 b, f32x4 acc) {
    acc = mfma16(a.x, b[0], acc);
    acc = mfma16(a.y, b[1], acc);
    acc = mfma16(a.z, b[2], acc);
    acc = mfma16(a.w, b[3], acc);
    return acc;
}

constexpr int CH = 64;        // chunk length
constexpr int CB = CH * kDk;  // floats in one [64 tokens][128] chunk block
constexpr int LDA = 68;       // padded LDS row stride of [64][64] tiles

// Operand layouts of one chunk block [64 tokens][128 dims], chosen so that
// every MFMA operand is one coalesced float4 per lane (1 KiB per wave):
//  A layout: lane (g, c) holds X[16 tb + c][16 kb + 4g + s], s = 0..3
//            (the A operand of an MFMA whose reduction index is the dim).
//  D layout: lane (g, c) holds X[16 tb + 4g + s][16 kb + c]
//            (an MFMA D tile; also the A operand of a product reducing over
//             tokens, e.g. K^T D).
// Both are [4 tb][8 kb][64 lanes][4] inside the block.
__device__ __forceinline__ const float4* blk4(const float* base, int tb, int kb, int lane) {
    return reinterpret_cast<const float4*>(base + (size_t)((tb * 8 + kb) * 64 + lane) * 4);
}

struct PrefillWork {
    float* qa;     // [nk][nch] chunk blocks, A layout: q^ (L2-normed, / sqrt(dk))
    float* kt;     // [nk][nch] D layout: k^
    float* wa;     // [nv][nch] A layout: W
    float* ud;     // [nv][nch] D layout: U
    float* aqk;    // [nv][nch][4 rb][4 cb][64][4]: lane (g,c) holds (M o QK^T)[16rb+c][16cb+4g+s]
    float* gam;    // [nv][nch][64]   e^{G_i}
    float* gdec;   // [nv][nch][64]   e^{G_last - G_i}
    float* oi;     // [nv][nch] chunk blocks, D layout: diag(gamma) Q S of each chunk
    float* dh;     // [nv][nch] chunk blocks, D layout: D = U - W S of each chunk
};

size_t work_floats(const Dims& d, int nch) {
    return (size_t)nch * CB * (2 * d.nk + 4 * d.nv) + (size_t)d.nv * nch * (CH * CH + 2 * CH);
}

PrefillWork carve(float* w, const Dims& d, int nch) {
    PrefillWork p;
    const size_t kblk = (size_t)d.nk * nch * CB, vblk = (size_t)d.nv * nch * CB;
    p.qa = w;
    p.kt = p.qa + kblk;
    p.wa = p.kt + kblk;
    p.ud = p.wa + vblk;
    p.aqk = p.ud + vblk;
    p.gam = p.aqk + (size_t)d.nv * nch * CH * CH;
    p.gdec = p.gam + (size_t)d.nv * nch * CH;
    p.oi = p.gdec + (size_t)d.nv * nch * CH;
    p.dh = p.oi + vblk;
    return p;
}

// SiLU of the zero-padded causal conv of channel c (prefill tap order: tap j
// multiplies x[t - j], GatedDeltaNetOps.cs:27-53) over the N tokens from
// `ts`; tokens at or past T give 0.  conv_load issues the N + 3 raw-input
// loads and the 4 tap weights so callers can put them in flight early;
// conv_finish applies the taps.  Each qkv element is read once per range.  For T >= 3 the range that
// holds token T - 1 also writes the conv window <- the last K - 1 raw inputs
// (Prefill.cs:192-204).
//
// The raw inputs come through a buffer descriptor based at row r0 of qkv and
// ending at row T: rows before 0 (negative offsets wrap past the end) and
// rows from T on fall outside it and load as 0, which is the conv's zero
// padding, so the loads need no clamps or masks.  Offsets stay below 2^31 for
// any T (a chunk spans 67 rows of the descriptor).
struct QkvRows {
    __amdgpu_buffer_rsrc_t rsrc;
    int r0;
};

__device__ __forceinline__ QkvRows qkv_rows(const float* qkv, int conv_dim, int T, int r0) {
    const long long bytes = (long long)(T - r0) * conv_dim * sizeof(float);
    return {__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(qkv + (size_t)r0 * conv_dim), 0,
                                              (int)min(bytes, 0x7fffffffLL), 0x00020000),
            r0};
}

// `ts` is wave-uniform, so the row offsets are scalar work.
template <int N>
__device__ __forceinline__ void conv_load(const QkvRows& q, const float* __restrict__ conv_w, int c,
                                          int conv_dim, int ts, float (&x)[N + 3], float4& wt) {
    wt = make_float4(conv_w[c], conv_w[conv_dim + c], conv_w[2 * conv_dim + c], conv_w[3 * conv_dim + c]);
#pragma unroll
    for (int j = 0; j < N + 3; ++j) {
        const int row = ts - 3 + j - q.r0;
        x[j] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(q.rsrc, (row * conv_dim + c) * 4, 0, 0));
    }
}

// The window write-back reloads the three raw inputs rather than selecting
// them from x: a select by the uniform T - ts becomes one scalar mask per
// element, which the compiler keeps live across the caller's loops.  A q/k
// channel's window is also written to the `nextra` further copies that the
// decode of the k-head's other v-heads reads (after the [conv_dim][3]
// block, qk_dim channels each); value channels pass nextra = 0.
template <int N>
__device__ __forceinline__ void conv_finish(const QkvRows& q, float4 wt, float* __restrict__ cs, int c,
                                            int conv_dim, int T, int ts, float (&x)[N + 3], float (&y)[N],
                                            int nextra, int qk_dim) {
    if (T >= kConvState && ts <= T - 1 && T - 1 < ts + N) {
        float wv[kConvState];
#pragma unroll
        for (int j = 0; j < kConvState; ++j) {
            const int row = T - kConvState + j - q.r0;
            wv[j] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(q.rsrc, (row * conv_dim + c) * 4, 0, 0));
            cs[(size_t)c * kConvState + j] = wv[j];
        }
        for (int r = 0; r < nextra; ++r)
#pragma unroll
            for (int j = 0; j < kConvState; ++j)
                cs[((size_t)conv_dim + (size_t)r * qk_dim + c) * kConvState + j] = wv[j];
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
        // Taps in the reference's order: j = 0 (current) .. 3 (x[t-3]), zero pad.
        float acc = wt.x * x[j + 3];
        acc += wt.y * x[j + 2];
        acc += wt.z * x[j + 1];
        acc += wt.w * x[j];
        y[j] = ts + j < T ? silu(acc) : 0.0f;
    }
}

// cs[c][j] = qkvCh[c*T + tail + j] over the channel-major copy qkvCh [C][T]
// followed (64-byte aligned, as the reference's arena) by the conv output
// [C][T]; for T >= 3 this is x[T-3+j][c].  The windows of the qk_dim q/k
// channels also go to the nextra copies after the [conv_dim][3] block.
__global__ void deltanet_conv_writeback(const float* __restrict__ qkv,
                                        const float* __restrict__ conv_w, float* __restrict__ cs,
                                        int T, int conv_dim, int nextra, int qk_dim) {
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
        if (c < qk_dim)
            for (int r = 0; r < nextra; ++r) cs[((size_t)conv_dim + (size_t)r * qk_dim + c) * kConvState + j] = val;
    }
}

// Lower-triangular 16x16 blocks (rb >= cb) of a 64x64 matrix, in work order.
// Block i = 0..9 is (rb, cb) = (0,0), (1,0), (1,1), (2,0), ..., (3,3); i is
// wave-uniform, so this is scalar arithmetic.
__device__ __forceinline__ int tri_rb(int i) { return (i >= 1) + (i >= 3) + (i >= 6); }
__device__ __forceinline__ int tri_cb(int i) { return i - tri_rb(i) * (tri_rb(i) + 1) / 2; }

// One workgroup per (k-head, chunk): the conv, gates and L2 norms of the
// chunk's inputs (Prefill.cs:181-248), then the chunked WY preparation.
//  - q and k of the k-head: conv + SiLU (thread = channel, 32 tokens) into a
//    row-major LDS tile, L2 norm per token (q also / sqrt(dk)); q goes to the
//    workspace in the A layout (the scan's Q S) and stays in LDS for Q K^T
//    (in the space the per-head tiles take later), k goes out in the D
//    layout (the scan's K^T D) and stays in LDS for the rest.
//  - beta = sigmoid(b), g = ssm_a * softplus(a + dt_bias) of the R v-heads.
//  - K K^T and (Q K^T)^T once for the R v-heads (their 20 lower 16x16 blocks,
//    5 per wave, kept in registers); (Q K^T)^T = K Q^T comes out of the MFMA
//    already in the A layout of M o QK^T that dn_chunk_out reads.
//  - Per v-head: the decay masks, the 16x16 diagonal-block inverses of I + A,
//    and the blocked forward substitution for W (right-hand sides from the k
//    tile; written in the A layout through an LDS transpose) and U (v conv'd
//    into LDS 64 channels at a time; written in the D layout straight from
//    the MFMA tile).
// The normalised q, k, v thus never make a round trip through HBM except
// the q and k blocks the scan needs.
__global__ __launch_bounds__(256, 2) void dn_chunk_prep(
    const float* __restrict__ qkv, const float* __restrict__ bin, const float* __restrict__ ain,
    const float* __restrict__ conv_w, const float* __restrict__ ssm_a,
    const float* __restrict__ dt_bias, PrefillWork w, float* __restrict__ cs, int T, int nk,
    int nv, int nch, float eps) {
    const int kh = blockIdx.x / nch, n = blockIdx.x % nch;
    const int R = nv / nk;
    const int t0 = n * CH;
    const int tn = min(CH, T - t0);
    const int key_dim = nk * kDk, conv_dim = 2 * key_dim + nv * kDk;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;

    __shared__ float Ks[CH][kDk + 4];  // k^ of the chunk, row-major
    // Vs (64 channels of v, row-major) and Am (-A, the strictly lower part of
    // the lower blocks) of the per-head phase share their space with Qs, the
    // chunk's q^ (row-major), which is needed only until Q K^T is formed.
    static_assert(CH * (kDk + 4) <= 2 * CH * LDA, "q^ tile must fit in the v and A tiles");
    __shared__ float4 vaq[2 * CH * LDA / 4];
    float (*Vs)[LDA] = reinterpret_cast<float (*)[LDA]>(vaq);
    float (*Am)[LDA] = reinterpret_cast<float (*)[LDA]>(reinterpret_cast<float*>(vaq) + CH * LDA);
    float (*Qs)[kDk + 4] = reinterpret_cast<float (*)[kDk + 4]>(vaq);
    __shared__ float Td[4][16][17];    // inverses of the 16x16 diagonal blocks of I + A
    __shared__ double Gd[kMaxVPerK][CH];
    __shared__ float bet[kMaxVPerK][CH], gam[kMaxVPerK][CH];
    __shared__ float nrm[CH];

    // Inputs of beta and g of the R v-heads (wave = v-head, lane = token;
    // padded tokens read the last row and are masked below; waves past R
    // repeat the last v-head and store nothing).  They are formed after the
    // conv loads below are out, so those loads do not wait on these.
    const int grr = min(wave, R - 1), gj = lane, gvh = kh * R + grr;
    const size_t gi = (size_t)min(t0 + gj, T - 1) * nv + gvh;
    const float gb_in = bin[gi], ga_in = ain[gi], g_sa = ssm_a[gvh], g_dt = dt_bias[gvh];

    // q, then k: conv'd into Qs, Ks (thread = channel tid % 128, tokens 32
    // (tid / 128) ..), then the per-token sum of squares (thread = (token,
    // quarter)).
    // The raw inputs of both are loaded up front.
    const int cq = tid & (kDk - 1), hq = __builtin_amdgcn_readfirstlane(tid >> 7);
    const int cq_q = kh * kDk + cq, cq_k = key_dim + kh * kDk + cq;
    const QkvRows rows = qkv_rows(qkv, conv_dim, T, max(t0 - 3, 0));
    float xq[35], xk[35];
    float4 wq, wk;
    conv_load<32>(rows, conv_w, cq_q, conv_dim, t0 + 32 * hq, xq, wq);
    conv_load<32>(rows, conv_w, cq_k, conv_dim, t0 + 32 * hq, xk, wk);
    __builtin_amdgcn_sched_barrier(0);
    {
        // Gates of every v-head at once, one wave each, formed by every
        // thread (so the loads above stay where they are) and stored by the
        // waves below R: beta, g, the fp64 running sum G of g (padded tokens
        // get beta = g = 0), gamma = e^G and e^{G_last - G}.
        const bool valid = gj < tn;
        const float bv = 1.0f / (1.0f + expf(-gb_in));
        const float gv = g_sa * softplus_ref(ga_in + g_dt);
        double G = valid ? (double)gv : 0.0;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double up = __shfl_up(G, o, kWave);
            if (lane >= o) G += up;
        }
        const double Glast = __shfl(G, CH - 1, kWave);
        if (wave < R) {
            const size_t cidx = (size_t)gvh * nch + n;
            Gd[wave][lane] = G;
            bet[wave][lane] = valid ? bv : 0.0f;
            const float gm = __expf((float)G);
            gam[wave][lane] = gm;
            w.gam[cidx * CH + lane] = gm;
            w.gdec[cidx * CH + lane] = __expf((float)(Glast - G));
        }
    }
    auto conv_qk = [&](float (*X)[kDk + 4], int ch, float4 wt, float (&x)[35], float (&y)[32]) {
        conv_finish<32>(rows, wt, cs, ch, conv_dim, T, t0 + 32 * hq, x, y, R - 1, 2 * key_dim);
#pragma unroll
        for (int j = 0; j < 32; ++j) X[32 * hq + j][cq] = y[j];
        lds_barrier();
        {
            // Lanes l, l + 16, l + 32, l + 48 of a wave take the four quarters
            // of one row (16 rows a wave), so the 16 lanes of each LDS read
            // pass touch 16 rows at one column offset: no bank conflicts.
            // The quarter sums combine as (p0 + p1) + (p2 + p3).
            const int row = (tid & 15) + 16 * wave, part = lane >> 4;
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float4 v = *reinterpret_cast<const float4*>(&X[row][32 * part + 4 * e]);
                acc += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
            acc = xor16_sum(acc);
            acc = xor32_sum(acc);
            if (part == 0) nrm[row] = __builtin_amdgcn_rsqf(acc + eps);   // 1 / |x|
        }
        lds_barrier();
    };
    const size_t kidx = (size_t)kh * nch + n;
    {
        float y[32];
        conv_qk(Qs, cq_q, wq, xq, y);
        // q^ = q / |q| / sqrt(dk) in place and to the workspace, A layout:
        // float4 o4 = (tb * 8 + kb) * 64 + lane holds row 16 tb + c, columns
        // 16 kb + 4 g ..  (The k conv's first barrier orders these reads of
        // nrm before its norms overwrite it.)
        float4* qA = reinterpret_cast<float4*>(w.qa + kidx * CB);
        const float pre = 1.0f / sqrtf((float)kDk);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int o4 = tid + 256 * i, bk = o4 >> 6, ln = o4 & 63;
            const int row = 16 * (bk >> 3) + (ln & 15), col = 16 * (bk & 7) + 4 * (ln >> 4);
            const float sc = pre * nrm[row];
            const float4 v = *reinterpret_cast<const float4*>(&Qs[row][col]);
            const float4 qv = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
            qA[o4] = qv;
            *reinterpret_cast<float4*>(&Qs[row][col]) = qv;
        }
        conv_qk(Ks, cq_k, wk, xk, y);
        // k^ = k / |k| in place (thread owns its channel's 32 rows).
#pragma unroll
        for (int j = 0; j < 32; ++j) Ks[32 * hq + j][cq] = y[j] * nrm[32 * hq + j];
    }
    lds_barrier();

    // Block bi: bi < 10 -> K K^T block (rb, cb), rows 16rb + 4g + r, cols 16cb + c;
    //           bi >= 10 -> (Q K^T)^T block: D rows = keys 16cb + 4g + r, cols = queries 16rb + c.
    // The operands (from LDS; Q^ rows read as the A layout) of block m + 1
    // are in flight while block m's 32 MFMAs run.
    f32x4 blk[5];
    float4 oa[2][8], ob[2][8];
    auto load_blk = [&](int m, float4 (&a)[8], float4 (&b)[8]) {
        const int bi = wave + 4 * m;
        const int mat = bi / 10, rb = tri_rb(bi % 10), cb = tri_cb(bi % 10);
        const int ra = mat ? cb : rb;
#pragma unroll
        for (int q = 0; q < kDk / 16; ++q)
            a[q] = *reinterpret_cast<const float4*>(&Ks[16 * ra + c16][16 * q + 4 * g]);
        if (mat) {
#pragma unroll
            for (int q = 0; q < kDk / 16; ++q)
                b[q] = *reinterpret_cast<const float4*>(&Qs[16 * rb + c16][16 * q + 4 * g]);
        } else {
#pragma unroll
            for (int q = 0; q < kDk / 16; ++q)
                b[q] = *reinterpret_cast<const float4*>(&Ks[16 * cb + c16][16 * q + 4 * g]);
        }
    };
    load_blk(0, oa[0], ob[0]);
#pragma unroll
    for (int m = 0; m < 5; ++m) {
        if (m + 1 < 5) load_blk(m + 1, oa[(m + 1) & 1], ob[(m + 1) & 1]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < kDk / 16; ++q) {
            const float4 a = oa[m & 1][q], b = ob[m & 1][q];
            acc = mfma16(a.x, b.x, acc);
            acc = mfma16(a.y, b.y, acc);
            acc = mfma16(a.z, b.z, acc);
            acc = mfma16(a.w, b.w, acc);
        }
        blk[m] = acc;
    }
    // k^ to the workspace, D layout: float4 o4 holds rows 16 tb + 4 g + s,
    // column 16 kb + c.
    {
        float4* kD = reinterpret_cast<float4*>(w.kt + kidx * CB);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int o4 = tid + 256 * i, bk = o4 >> 6, ln = o4 & 63;
            const int r0 = 16 * (bk >> 3) + 4 * (ln >> 4), c0 = 16 * (bk & 7) + (ln & 15);
            kD[o4] = make_float4(Ks[r0][c0], Ks[r0 + 1][c0], Ks[r0 + 2][c0], Ks[r0 + 3][c0]);
        }
    }
    lds_barrier();   // Qs is read for the last time above; Am and Vs reuse it

#pragma unroll 1
    for (int rr = 0; rr < R; ++rr) {
        const int vh = kh * R + rr;
        const size_t cidx = (size_t)vh * nch + n;
        // v of this head, conv'd 64 channels at a time into Vs (thread =
        // channel tid % 64, tokens 16 (tid / 64) ..); the raw inputs of both
        // halves go out now, behind the gates, masks and diagonal inverses.
        const int cl = tid & 63, qt = wave;
        float xv[2][19];
        float4 wv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
            conv_load<16>(rows, conv_w, 2 * key_dim + vh * kDk + 64 * h + cl, conv_dim, t0 + 16 * qt,
                          xv[h], wv[h]);
        const double* Gh = Gd[rr];
        const float* bh = bet[rr];
        const float* gh = gam[rr];
        // Decay masks on the register blocks: -A into LDS, M o QK^T to the workspace.
        float* aqk = w.aqk + cidx * CH * CH;
#pragma unroll
        for (int m = 0; m < 5; ++m) {
            const int bi = wave + 4 * m;
            const int mat = bi / 10, rb = tri_rb(bi % 10), cb = tri_cb(bi % 10);
            if (mat == 0) {
                const int j = 16 * cb + c16;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = 16 * rb + 4 * g + r;
                    Am[i][j] = j < i ? -bh[i] * __expf((float)(Gh[i] - Gh[j])) * blk[m][r] : 0.0f;
                }
            } else {
                const int iq = 16 * rb + c16;   // query token
                float4 v;
                float* vp = reinterpret_cast<float*>(&v);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int jk = 16 * cb + 4 * g + r;   // key token
                    vp[r] = jk <= iq ? __expf((float)(Gh[iq] - Gh[jk])) * blk[m][r] : 0.0f;
                }
                reinterpret_cast<float4*>(aqk)[(rb * 4 + cb) * 64 + lane] = v;
            }
        }
        lds_barrier();
        // Inverse of the unit-lower 16x16 diagonal block `wave` of I + A on
        // MFMA: with L its strictly lower part (L^16 = 0),
        //   (I + L)^-1 = sum_{k<16} (-L)^k = (I + L^8)(I + L^4)(I + L^2)(I - L)
        // exactly; the factors commute.  A product X Y takes X in the A
        // layout, which is the D layout of X^T, so the powers of L^T are
        // formed beside those of L (L^8 is needed transposed only).
        {
            const int b0 = 16 * wave;
            f32x4 dl, dt, id;                // D layouts of L, L^T and I
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dl[r] = -Am[b0 + 4 * g + r][b0 + c16];
                dt[r] = -Am[b0 + c16][b0 + 4 * g + r];
                id[r] = 4 * g + r == c16 ? 1.0f : 0.0f;
            }
            auto mm = [](f32x4 xt, f32x4 y) {    // X Y from D(X^T) and D(Y)
                return mfma16x4(make_float4(xt[0], xt[1], xt[2], xt[3]), y, f32x4{0.f, 0.f, 0.f, 0.f});
            };
            const f32x4 l2 = mm(dt, dl), l2t = mm(dl, dt);
            const f32x4 l4 = mm(l2t, l2), l4t = mm(l2, l2t);
            const f32x4 l8t = mm(l4, l4t);
            f32x4 x = id - dl;                   // I - L
            x = mm(id + l2t, x);
            x = mm(id + l4t, x);
            x = mm(id + l8t, x);
#pragma unroll
            for (int r = 0; r < 4; ++r) Td[wave][4 * g + r][c16] = x[r];
        }
        lds_barrier();
        // Y = (I + A)^-1 X for X = diag(beta gamma) K^ (-> W) and diag(beta) V (-> U),
        // block row by block row.  Pass h: the wave solves K block wave + 4h and
        // v block wave + 4h together (two independent MFMA chains sharing the
        // A and T operands; Vs holds v channels 64 h .. + 63).  W goes out in
        // the A layout as Y^T = X^T T^T, one more MFMA per block on the same
        // operands (the D tile of Y^T is Y in the A layout).
        float* wA = w.wa + cidx * CB;
        float* uD = w.ud + cidx * CB;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kb = wave + 4 * h;
            {
                float y[16];
                const int ch = 2 * key_dim + vh * kDk + 64 * h + cl;
                conv_finish<16>(rows, wv[h], cs, ch, conv_dim, T, t0 + 16 * qt, xv[h], y, 0, 0);
                if (h == 1) lds_barrier();   // every wave is past the first half
#pragma unroll
                for (int j = 0; j < 16; ++j) Vs[16 * qt + j][cl] = y[j];
                lds_barrier();
            }
            f32x4 YK[4], YV[4];
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) {
                f32x4 accK, accV;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * ib + 4 * g + r;
                    const float bt = bh[row];
                    accK[r] = Ks[row][16 * kb + c16] * bt * gh[row];
                    accV[r] = Vs[row][16 * wave + c16] * bt;
                }
#pragma unroll
                for (int jb = 0; jb < ib; ++jb) {
                    const float4 a = *reinterpret_cast<const float4*>(&Am[16 * ib + c16][16 * jb + 4 * g]);
                    accK = mfma16x4(a, YK[jb], accK);
                    accV = mfma16x4(a, YV[jb], accV);
                }
                const float4 tdv = make_float4(Td[ib][c16][4 * g], Td[ib][c16][4 * g + 1],
                                               Td[ib][c16][4 * g + 2], Td[ib][c16][4 * g + 3]);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                YK[ib] = mfma16x4(tdv, accK, zero);
                YV[ib] = mfma16x4(tdv, accV, zero);
                const f32x4 wt = mfma16x4(make_float4(accK[0], accK[1], accK[2], accK[3]),
                                          f32x4{tdv.x, tdv.y, tdv.z, tdv.w}, zero);
                reinterpret_cast<float4*>(uD)[(ib * 8 + kb) * 64 + lane] =
                    make_float4(YV[ib][0], YV[ib][1], YV[ib][2], YV[ib][3]);
                reinterpret_cast<float4*>(wA)[(ib * 8 + kb) * 64 + lane] =
                    make_float4(wt[0], wt[1], wt[2], wt[3]);
            }
        }
        lds_barrier();
    }
}

// Operands of one chunk for one wave of dn_chunk_scan, each a coalesced float4
// per lane; none depends on the state, so the next chunk's set is loaded while
// the current one computes.
struct ScanOps {
    float4 wa[4][2];             // W (A operand of W S), this wave's 32 state rows
    float4 kt[4][2];             // K^ (A operand of K^T D), same rows
    float4 ut;                   // U, token block `wave`, this column tile
    float4 gdv;                  // e^{G_last - G}, token block `wave`
    float glast;                 // gamma_last
};

// Operands of diag(gamma) Q S for one token block of one chunk.
struct QsOps {
    float4 qa[8];                // Q^ blocks (tb, kb = 0..7), A layout
    float4 gm;                   // gamma of the block's rows 4g .. 4g+3
};

// The operands used first in a chunk (W, U, the decays) and K^, loaded in
// different phases of the previous chunk so that the L2 reads spread over it.
__device__ __forceinline__ void load_scan_w(const PrefillWork& w, ScanOps& o, int n, int vh,
                                            int tl, int nch, int wave, int g, int lane) {
    const size_t cidx = (size_t)vh * nch + n;
    const float* wA = w.wa + cidx * CB;
    const float* uD = w.ud + cidx * CB;
    const float* gd = w.gdec + cidx * CH;
    o.glast = w.gam[cidx * CH + CH - 1];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int b = 0; b < 2; ++b) o.wa[tb][b] = *blk4(wA, tb, 2 * wave + b, lane);
    o.ut = *blk4(uD, wave, tl, lane);
    o.gdv = *reinterpret_cast<const float4*>(gd + 16 * wave + 4 * g);
}

__device__ __forceinline__ void load_scan_k(const PrefillWork& w, ScanOps& o, int n, int kh,
                                            int nch, int wave, int lane) {
    const float* kD = w.kt + ((size_t)kh * nch + n) * CB;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int b = 0; b < 2; ++b) o.kt[tb][b] = *blk4(kD, tb, 2 * wave + b, lane);
}

__device__ __forceinline__ void load_qs_ops(const PrefillWork& w, QsOps& o, int n, int vh, int kh,
                                            int nch, int tb, int g, int lane) {
    const size_t cidx = (size_t)vh * nch + n, kidx = (size_t)kh * nch + n;
    const float* qA = w.qa + kidx * CB;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) o.qa[kb] = *blk4(qA, tb, kb, lane);
    o.gm = *reinterpret_cast<const float4*>(w.gam + cidx * CH + 16 * tb + 4 * g);
}

__device__ __forceinline__ f32x4 v4(float4 a) { return f32x4{a.x, a.y, a.z, a.w}; }

// The sequential part: one workgroup per (v-head, 16-column tile).  Waves 0-3
// run the chain: wave w owns state rows 32w..32w+31 of the tile (two D-layout
// 16x16 tiles, kept in MFMA accumulators across chunks); per chunk they write
// D = U - W S for dn_chunk_out and apply S = gamma_last S + K^T (e^{G_last-G}
// D).  Waves 4-7 (one per token block, lower issue priority) form the
// inter-chunk output diag(gamma) Q S of each chunk from the entry state the
// chain waves leave in LDS; their products fill the matrix pipe while the
// chain waits on LDS and barriers.  Both kinds of wave pass the same two
// barriers per chunk.  Column tiles are independent (the rule is separable
// over dv), so 8 workgroups per head run in parallel, on one XCD so W, Q and
// K stay in its L2.
__global__ __launch_bounds__(512) void dn_chunk_scan(PrefillWork w, float* __restrict__ state,
                                                     int nk, int nv, int nch) {
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int vh = L / 8, tl = L % 8;
    const int kh = vh / (nv / nk);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;

    // Per-wave partials of W S and the decayed D blocks, and the entry state
    // of the chunk ([kb][lane], D layout), double-buffered by chunk parity.
    __shared__ f32x4 red[2][4][4][64];
    __shared__ f32x4 dg[2][4][64];
    __shared__ f32x4 sbuf[2][8][64];

    if (wave >= 4) {
        // Inter-chunk output of token block q.  The entry state of chunk n is
        // read between the chunk's two barriers (the chain rewrites that
        // buffer only after the next chunk's second barrier); half of the
        // products run before the second barrier, half after it, behind the
        // loads of the next chunk's Q^ (issued while the chain runs K^T D).
        __builtin_amdgcn_s_setprio(0);
        const int q = wave - 4;
        QsOps a0, a1;
        load_qs_ops(w, a0, 0, vh, kh, nch, q, g, lane);
        auto qs_chunk = [&](const QsOps& cur, QsOps& nxt, int n) {
            const int par = n & 1;
            lds_barrier();
            f32x4 Sk[8];
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) Sk[kb] = sbuf[par][kb][lane];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) acc = mfma16x4(cur.qa[kb], Sk[kb], acc);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            __builtin_amdgcn_sched_barrier(0);
            load_qs_ops(w, nxt, min(n + 1, nch - 1), vh, kh, nch, q, g, lane);
#pragma unroll
            for (int kb = 4; kb < 8; ++kb) acc = mfma16x4(cur.qa[kb], Sk[kb], acc);
            *reinterpret_cast<f32x4*>(w.oi + ((size_t)vh * nch + n) * CB +
                                      (size_t)((q * 8 + tl) * 64 + lane) * 4) = acc * v4(cur.gm);
        };
        const int npair = nch / 2;
        for (int it = 0; it < npair; ++it) {
            qs_chunk(a0, a1, 2 * it);
            qs_chunk(a1, a0, 2 * it + 1);
        }
        if (2 * npair < nch) qs_chunk(a0, a1, nch - 1);
        return;
    }

    __builtin_amdgcn_s_setprio(2);
    const int col = 16 * tl + c16;
    float* S = state + (size_t)vh * kDk * kDk;
    f32x4 Sb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) Sb[b][r] = S[(size_t)(32 * wave + 16 * b + 4 * g + r) * kDk + col];

    // One chunk: the entry state to LDS, D, then the state update.  The
    // operands of chunk `pf` (the next; clamped, so the last chunk reloads
    // itself) are loaded into `nxt`: W, U and the decays interleaved 1:1
    // with the MFMAs of W S, K^ with those of K^T D, so the operand reads
    // (L2 hits, shared by the 8 column tiles of a head) spread over the chunk
    // and every operand has a whole chunk to arrive.
    auto chunk = [&](const ScanOps& cur, ScanOps& nxt, int n, int pf) {
        const int par = n & 1;
        const size_t cidx = (size_t)vh * nch + n;
#pragma unroll
        for (int b = 0; b < 2; ++b) sbuf[par][2 * wave + b][lane] = Sb[b];
        load_scan_w(w, nxt, min(pf, nch - 1), vh, tl, nch, wave, g, lane);
        // Partial W S over this wave's 32 state rows, all 4 token blocks.
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            f32x4 pws = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int b = 0; b < 2; ++b) pws = mfma16x4(cur.wa[tb][b], Sb[b], pws);
            red[par][wave][tb][lane] = pws;
        }
#pragma unroll
        for (int i = 0; i < 11; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // one VMEM read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 21, 0);
        lds_barrier();
        // Wave w forms D = U - W S of token block w, records it, and shares
        // e^{G_last - G} D with the other waves (each needs all 4 blocks for
        // its rows of the update).
        {
            f32x4 ws = red[par][0][wave][lane];
#pragma unroll
            for (int v = 1; v < 4; ++v) ws += red[par][v][wave][lane];
            const f32x4 dw = v4(cur.ut) - ws;
            *reinterpret_cast<f32x4*>(w.dh + cidx * CB + (size_t)((wave * 8 + tl) * 64 + lane) * 4) = dw;
            dg[par][wave][lane] = dw * v4(cur.gdv);
        }
        lds_barrier();
        f32x4 D[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) D[tb] = dg[par][tb][lane];
        load_scan_k(w, nxt, min(pf, nch - 1), kh, nch, wave, lane);
        // S = gamma_last S + K^T (e^{G_last - G} D).
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            f32x4 acc = Sb[b] * cur.glast;
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) acc = mfma16x4(cur.kt[tb][b], D[tb], acc);
            Sb[b] = acc;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
    };
    // Operands run one chunk ahead: two register sets in rotation, no copies.
    ScanOps o0, o1;
    load_scan_w(w, o0, 0, vh, tl, nch, wave, g, lane);
    load_scan_k(w, o0, 0, kh, nch, wave, lane);
    const int npair = nch / 2;
    for (int it = 0; it < npair; ++it) {
        chunk(o0, o1, 2 * it, 2 * it + 1);
        chunk(o1, o0, 2 * it + 1, 2 * it + 2);
    }
    if (2 * npair < nch) chunk(o0, o1, nch - 1, nch);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[(size_t)(32 * wave + 16 * b + 4 * g + r) * kDk + col] = Sb[b][r];
}

// Chunk outputs, in parallel over (v-head, chunk), with the gated RMSNorm
// (Qwen35Ops.GatedRmsNorm, Qwen35Ops.cs:74-111) fused:
//   O = diag(gamma) Q S + (M o Q K^T) D,  out = O * rms(O)^-1 * w * SiLU(z),
// where diag(gamma) Q S comes from dn_chunk_scan.  Wave w computes column
// tiles 2w, 2w+1 of all 4 token blocks: the inter-chunk output and D columns
// stay in registers; the 10 causal blocks of M o QK^T (shared by the 4 waves)
// are staged in LDS.  O goes row-major through LDS, so the RMS of a row is a
// 32-lane reduction and z and out move as coalesced float4 rows.
__global__ __launch_bounds__(256, 3) void dn_chunk_out(PrefillWork w, const float* __restrict__ z,
                                                    const float* __restrict__ wnorm,
                                                    float* __restrict__ out, int T, int nv,
                                                    int nch, float eps) {
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    // v-heads vary fastest, so the z rows and output rows in flight are whole
    // token rows (16 KiB) rather than one 512-byte column of many rows.
    const int vh = L % nv, n = L / nv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const size_t cidx = (size_t)vh * nch + n;
    const float* oD = w.oi + cidx * CB;
    const float* dD = w.dh + cidx * CB;
    const float4* aq = reinterpret_cast<const float4*>(w.aqk + cidx * CH * CH);

    __shared__ float o_s[CH][kDk + 4];    // row-major output tile
    __shared__ float4 a_s[10][64];        // causal blocks (tb, j <= tb) of M o QK^T

    // Load order: M o QK^T first (staged into LDS), then the inter-chunk
    // output and D, then z for the epilogue.
    const int t0 = n * CH;
    // A thread's columns are the same in every row it handles (4 (tid % 32)).
    const float4 wn = reinterpret_cast<const float4*>(wnorm)[tid & 31];
    float4 zr[8];
    f32x4 O[4][2];
    {
        // M o QK^T: the 640 float4 of the causal blocks, up to 3 per thread.
        auto aload = [&](int i) {
            const int o4 = min(tid + 256 * i, 10 * 64 - 1);
            const int blk = o4 >> 6, tb = blk < 1 ? 0 : blk < 3 ? 1 : blk < 6 ? 2 : 3;
            const int j = blk - tb * (tb + 1) / 2;
            return aq[(tb * 4 + j) * 64 + (o4 & 63)];
        };
        const float4 av0 = aload(0), av1 = aload(1), av2 = aload(2);
        __builtin_amdgcn_sched_barrier(0);     // keep the loads above ahead of the rest
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) O[tb][cc] = v4(*blk4(oD, tb, 2 * wave + cc, lane));
        f32x4 Dc[4][2];           // D[16 tb .. +15][16 (2w + cc) .. +15], D layout
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) Dc[tb][cc] = v4(*blk4(dD, tb, 2 * wave + cc, lane));
        // z rows of this (chunk, v-head): float4 o4 = tid + 256 i is row
        // o4 / 32, columns 4 (o4 % 32) ..; rows past T read row T - 1 and are
        // not stored.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int o4 = tid + 256 * i, t = min(t0 + (o4 >> 5), T - 1);
            zr[i] = reinterpret_cast<const float4*>(z + ((size_t)t * nv + vh) * kDk)[o4 & 31];
        }
        // Threads past the 640 float4 rewrite the last one with the same value
        // (an unconditional store keeps these loads ahead of the others).
        a_s[tid >> 6][tid & 63] = av0;
        a_s[(tid + 256) >> 6][tid & 63] = av1;
        {
            const int o4 = min(tid + 512, 10 * 64 - 1);
            a_s[o4 >> 6][o4 & 63] = av2;
        }
        lds_barrier();
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int tb = j; tb < 4; ++tb) {
                const float4 a = a_s[tb * (tb + 1) / 2 + j][lane];
                O[tb][0] = mfma16x4(a, Dc[j][0], O[tb][0]);
                O[tb][1] = mfma16x4(a, Dc[j][1], O[tb][1]);
            }
    }
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o_s[16 * tb + 4 * g + r][32 * wave + c16] = O[tb][0][r];
            o_s[16 * tb + 4 * g + r][32 * wave + 16 + c16] = O[tb][1][r];
        }
    lds_barrier();
    // Row-major epilogue: lanes 0-31 of a wave hold one row, 32-63 the next.
    // The output is not read again by this path, so it is streamed out with
    // non-temporal stores (it does not sit dirty in L2 at the kernel's end).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int o4 = tid + 256 * i, row = o4 >> 5, c4 = o4 & 31, t = t0 + row;
        const float4 o = *reinterpret_cast<const float4*>(&o_s[row][4 * c4]);
        float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
#pragma unroll
        for (int m = 1; m < 32; m <<= 1) ss += __shfl_xor(ss, m, kWave);
        if (t >= T) continue;
        const float rs = 1.0f / sqrtf(ss / (float)kDk + eps);
        float4 r;
        r.x = o.x * rs * wn.x * silu(zr[i].x);
        r.y = o.y * rs * wn.y * silu(zr[i].y);
        r.z = o.z * rs * wn.z * silu(zr[i].z);
        r.w = o.w * rs * wn.w * silu(zr[i].w);
        __builtin_nontemporal_store(v4(r), reinterpret_cast<f32x4*>(out + ((size_t)t * nv + vh) * kDk) + c4);
    }
}

}  // namespace

size_t deltanet_prefill_work_bytes(const Dims& d, int T) {
    return work_floats(d, (T + CH - 1) / CH) * sizeof(float);
}

hipError_t launch_deltanet_prefill(q35m_ctx* c, int layer, int seq, int T, const float* qkv,
                                   const float* z, const float* b, const float* a, float* out) {
    const Dims& d = c->d;
    const DeltaNetLayer& L = c->lin[layer];
    const int nch = (T + CH - 1) / CH;
    PrefillWork w = carve(c->work, d, nch);
    float* state = L.state + (size_t)seq * d.nv * kDk * kDk;
    float* cs = L.conv_window(seq, d.win_floats());
    hipError_t e;
    if (T < kConvState) {
        ProfScope ps_(c, K_DN_CONV_WRITEBACK);
        hipExtLaunchKernelGGL(deltanet_conv_writeback, dim3((d.conv_dim + 255) / 256), dim3(256), 0,
                           c->stream, ps_.a, ps_.b, 0, qkv, L.conv_w, cs, T, d.conv_dim, d.nv / d.nk - 1,
                           2 * d.key_dim);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    {
        ProfScope ps_(c, K_DN_CHUNK_PREP);
        hipExtLaunchKernelGGL(dn_chunk_prep, dim3(d.nk * nch), dim3(256), 0, c->stream, ps_.a, ps_.b, 0, qkv,
                           b, a, L.conv_w, L.ssm_a, L.dt_bias, w, cs, T, d.nk, d.nv, nch, d.eps);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CHUNK_SCAN);
        hipExtLaunchKernelGGL(dn_chunk_scan, dim3(d.nv * 8), dim3(512), 0, c->stream, ps_.a, ps_.b, 0, w, state, d.nk,
                           d.nv, nch);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    {
        ProfScope ps_(c, K_DN_CHUNK_OUT);
        hipExtLaunchKernelGGL(dn_chunk_out, dim3(d.nv * nch), dim3(256), 0, c->stream, ps_.a, ps_.b, 0, w, z,
                           L.ssm_norm, out, T, d.nv, nch, d.eps);
    }
    return hipGetLastError();
}

}  // namespace q35
