// Host side of libq35mix.so: context lifecycle, state ownership, weights,
// argument checking and the C ABI entry points of include/q35mix.h.
//
// The context replaces the mixer-state fields of Qwen35Model
// (src/Qwen35Sharp.Model/Qwen35Model.cs:23-36, allocation :100-136) with
// hipMalloc'd HBM buffers carrying an extra sequence dimension.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>

#include "q35mix_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory) return fail(Q35M_ERR_OOM, "%s: %s", what, hipGetErrorString(e));
    return fail(Q35M_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                        \
    do {                                           \
        hipError_t e_ = (expr);                    \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

int alloc_zero(q35m_ctx* c, void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) return Q35M_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    c->allocations.push_back(*p);
    e = hipMemsetAsync(*p, 0, bytes, c->stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemsetAsync");
    return Q35M_OK;
}

void release(q35m_ctx* c) {
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto& p : c->pending) {
        c->event_pool.push_back(p.a);
        c->event_pool.push_back(p.b);
    }
    c->pending.clear();
    for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
    c->event_pool.clear();
    for (void* p : c->allocations) (void)hipFree(p);
    c->allocations.clear();
    if (c->work) (void)hipFree(c->work);
    c->work = nullptr;
    if (c->stream) (void)hipStreamDestroy(c->stream);
    c->stream = nullptr;
}

int check_ctx(const q35m_ctx* c) {
    if (!c) return fail(Q35M_ERR_INVALID, "null context");
    return Q35M_OK;
}

int check_seq(const q35m_ctx* c, int seq) {
    if (seq < 0 || seq >= c->n_seqs)
        return fail(Q35M_ERR_INVALID, "sequence %d out of range [0, %d)", seq, c->n_seqs);
    return Q35M_OK;
}

int check_layer(const q35m_ctx* c, int layer, bool recurrent) {
    if (layer < 0 || layer >= c->cfg.num_layers)
        return fail(Q35M_ERR_INVALID, "layer %d out of range [0, %d)", layer, c->cfg.num_layers);
    if ((c->is_recurrent[layer] != 0) != recurrent)
        return fail(Q35M_ERR_INVALID, "layer %d is a %s layer", layer,
                    c->is_recurrent[layer] ? "Gated-DeltaNet" : "full-attention");
    return Q35M_OK;
}

// Ops.EnsureRopeTable (src/Qwen35Sharp.Model/Ops.cs:135-160), built on the
// host with the same fp32 operations (powf, fp32 angle, cosf/sinf) so the
// device table equals the reference's bit for bit.
void build_rope_table(int cap, int half, float base, std::vector<float>& cs,
                      std::vector<float>& sn) {
    std::vector<float> freqs(half);
    for (int i = 0; i < half; i++) freqs[i] = 1.0f / powf(base, (float)i / (float)half);
    cs.resize((size_t)cap * half);
    sn.resize((size_t)cap * half);
    for (int pos = 0; pos < cap; pos++)
        for (int i = 0; i < half; i++) {
            volatile float angle = (float)pos * freqs[i];
            cs[(size_t)pos * half + i] = cosf(angle);
            sn[(size_t)pos * half + i] = sinf(angle);
        }
}

// The batch of sequence ids of a decode call (distinct, in range).  With
// max_cached non-null, every sequence must have room for the new row, and
// *max_cached receives the longest cached length in the batch.
int build_seq_batch(const q35m_ctx* c, int n, const int* seqs, q35::SeqBatch* sb, int* max_cached) {
    if (n < 1 || n > q35::kMaxBatch)
        return fail(Q35M_ERR_CAPACITY, "batch of %d sequences (1..%d per call)", n, q35::kMaxBatch);
    if (!seqs) return fail(Q35M_ERR_INVALID, "null seqs");
    sb->n = n;
    int mx = 0;
    for (int i = 0; i < n; i++) {
        int r = check_seq(c, seqs[i]);
        if (r) return r;
        for (int j = 0; j < i; j++)
            if (seqs[j] == seqs[i]) return fail(Q35M_ERR_INVALID, "sequence %d repeated", seqs[i]);
        sb->seq[i] = seqs[i];
        if (max_cached) {
            const int p = c->kv_len[seqs[i]];
            if (p >= c->cap)
                return fail(Q35M_ERR_CAPACITY, "sequence %d: KV cache full (%d rows)", seqs[i], c->cap);
            mx = p > mx ? p : mx;
        }
    }
    if (max_cached) *max_cached = mx;
    return Q35M_OK;
}

// Mixer activations are read and written as 16-byte vectors.
int check_activations(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs) {
        if (!p) return fail(Q35M_ERR_INVALID, "null activation pointer");
        if ((uintptr_t)p & 15) return fail(Q35M_ERR_INVALID, "activation pointers must be 16-byte aligned");
    }
    return Q35M_OK;
}

// A sequence's length changed on the host: its device copy is rewritten
// before the next launch that reads it.
void set_len(q35m_ctx* c, int seq, int len) {
    c->kv_len[seq] = len;
    c->len_dirty[seq] = 1;
}

// Device address of the decode attention's fixed scratch, looked up once per
// device (with that device current) and kept for the process.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

int scratch_for_device(int device, float** out) {
    if (device < 0 || device >= kMaxDevices) return fail(Q35M_ERR_NO_DEVICE, "device %d out of range", device);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[device]) {
        float* p = nullptr;
        hipError_t e = q35::attn_decode_scratch_address(&p);
        if (e != hipSuccess || !p) return hip_fail(e == hipSuccess ? hipErrorInvalidSymbol : e, "hipGetSymbolAddress(scratch)");
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return Q35M_OK;
}

}  // namespace

// Sets the thread's last error from another translation unit.
int q35_set_error(int code, const char* msg) { return fail(code, "%s", msg); }

// The mixer dims a weight loader was given must be the context's: the
// weight setters copy context-sized byte counts.
int q35_check_mixer_dims(const q35m_ctx* c, int num_layers, const unsigned char* is_recurrent, int conv_dim,
                         int n_v_heads, int v_head_dim, int head_dim) {
    if (num_layers != c->cfg.num_layers)
        return fail(Q35M_ERR_INVALID, "num_layers %d, the context has %d", num_layers, c->cfg.num_layers);
    for (int l = 0; l < num_layers; l++)
        if ((is_recurrent[l] != 0) != (c->is_recurrent[l] != 0))
            return fail(Q35M_ERR_INVALID, "layer %d: is_recurrent %d, the context's layer is %s", l,
                        is_recurrent[l] != 0, c->is_recurrent[l] ? "Gated-DeltaNet" : "full-attention");
    if (conv_dim != c->d.conv_dim || n_v_heads != c->d.nv || v_head_dim != q35::kDk || head_dim != q35::kHd)
        return fail(Q35M_ERR_INVALID,
                    "dims conv %d, v heads %d, v head dim %d, head dim %d; the context has %d, %d, %d, %d",
                    conv_dim, n_v_heads, v_head_dim, head_dim, c->d.conv_dim, c->d.nv, q35::kDk, q35::kHd);
    return Q35M_OK;
}


namespace q35 {

const char* kernel_name(int id) {
    static const char* names[K_COUNT] = {
        "deltanet_decode_kernel", "deltanet_conv_writeback", "dn_chunk_prep",
        "dn_chunk_scan",          "dn_chunk_out",            "attn_decode_partial<1>",
        "attn_decode_partial<4>",  "attn_decode_partial<8>",
        "attn_decode_merge",      "attn_prefill_prep",       "attn_prefill_flash",
        "q8k_quantize",           "linear_q<4>",             "linear_q<6>",
        "q4k_gemm", "q6k_gemm", "add_rmsnorm", "linear_qs<5>", "linear_qs<14>", "linear_f32", "linear_qt<2>",
        "linear_qt<1>", "attn_decode_partial<4,16>", "attn_decode_partial<8,16>", "q6k_gemm_blk"};
    return (id >= 0 && id < K_COUNT) ? names[id] : nullptr;
}

static hipEvent_t take_event(q35m_ctx* c) {
    if (!c->event_pool.empty()) {
        hipEvent_t e = c->event_pool.back();
        c->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

ProfScope::ProfScope(q35m_ctx* ctx, int id) : c(ctx), kid(id) {
    if (!c->profile) return;
    a = take_event(c);
    b = a ? take_event(c) : nullptr;
    if (!b && a) {
        c->event_pool.push_back(a);
        a = nullptr;
    }
}

ProfScope::~ProfScope() {
    if (a && b) c->pending.push_back({a, b, kid});
}

// Folds finished event pairs into the per-kernel totals.
static hipError_t collect_profile(q35m_ctx* c) {
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return e;
    for (auto& p : c->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            c->prof_ms[p.kid] += ms;
            c->prof_n[p.kid] += 1;
        }
        c->event_pool.push_back(p.a);
        c->event_pool.push_back(p.b);
    }
    c->pending.clear();
    return hipSuccess;
}

hipError_t ensure_work(q35m_ctx* c, size_t bytes) {
    if (bytes <= c->work_bytes) return hipSuccess;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return e;
    if (c->work) (void)hipFree(c->work);
    c->work = nullptr;
    c->work_bytes = 0;
    size_t want = bytes + (bytes >> 3);
    e = hipMalloc((void**)&c->work, want);
    if (e != hipSuccess) return e;
    c->work_bytes = want;
    return hipSuccess;
}

}  // namespace q35

extern "C" {

const char* q35m_last_error(void) { return g_last_error.c_str(); }

int q35m_device_count(int* count) {
    if (!count) return fail(Q35M_ERR_INVALID, "null count");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) {
        *count = 0;
        return fail(Q35M_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    }
    return Q35M_OK;
}

int q35m_create(const q35m_config* cfg, int n_seqs, int kv_capacity, q35m_ctx** out) {
    if (!out) return fail(Q35M_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (!cfg) return fail(Q35M_ERR_INVALID, "null config");
    if (cfg->num_layers <= 0) return fail(Q35M_ERR_INVALID, "num_layers must be positive");
    if (n_seqs <= 0) return fail(Q35M_ERR_INVALID, "n_seqs must be positive");
    if (kv_capacity <= 0) return fail(Q35M_ERR_INVALID, "kv_capacity must be positive");
    if (cfg->ssm_state_size != q35::kDk || cfg->ssm_conv_kernel != q35::kConvK)
        return fail(Q35M_ERR_UNSUPPORTED, "DeltaNet kernels are built for dk = dv = %d, %d taps",
                    q35::kDk, q35::kConvK);
    if (cfg->ssm_group_count <= 0 || cfg->ssm_time_step_rank <= 0 ||
        cfg->ssm_time_step_rank % cfg->ssm_group_count != 0)
        return fail(Q35M_ERR_INVALID, "ssm_time_step_rank must be a positive multiple of "
                                      "ssm_group_count");
    if (cfg->ssm_time_step_rank / cfg->ssm_group_count > q35::kMaxVPerK)
        return fail(Q35M_ERR_UNSUPPORTED, "at most %d v-heads per k-head", q35::kMaxVPerK);
    if (cfg->ssm_inner_size != cfg->ssm_time_step_rank * cfg->ssm_state_size)
        return fail(Q35M_ERR_INVALID, "ssm_inner_size must equal ssm_time_step_rank * "
                                      "ssm_state_size");
    if (cfg->head_dim != q35::kHd || cfg->rope_dim != q35::kRopeDim)
        return fail(Q35M_ERR_UNSUPPORTED, "attention kernels are built for head_dim %d, rope_dim %d",
                    q35::kHd, q35::kRopeDim);
    if (cfg->num_kv_heads <= 0 || cfg->num_heads <= 0 || cfg->num_heads % cfg->num_kv_heads != 0)
        return fail(Q35M_ERR_INVALID, "num_heads must be a positive multiple of num_kv_heads");
    {
        const int g = cfg->num_heads / cfg->num_kv_heads;
        if (!(g == 1 || g == 2 || g == 4 || g % 8 == 0))
            return fail(Q35M_ERR_UNSUPPORTED,
                        "attention kernels take 1, 2, 4 or a multiple of 8 q heads per kv head (got %d)", g);
    }
    if (!(cfg->eps > 0.0f) || !(cfg->rope_base > 0.0f))
        return fail(Q35M_ERR_INVALID, "eps and rope_base must be positive");
    if (!cfg->is_recurrent && cfg->full_attention_interval <= 0)
        return fail(Q35M_ERR_INVALID, "full_attention_interval must be positive");

    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return fail(Q35M_ERR_NO_DEVICE, "no HIP device available");

    q35m_ctx* c = new q35m_ctx();
    c->cfg = *cfg;
    c->cfg.is_recurrent = nullptr;
    c->n_seqs = n_seqs;
    if (const char* e = std::getenv("Q35M_TILE_LIMIT_BYTES")) {
        const unsigned long long v = std::strtoull(e, nullptr, 10);
        if (v > 0 && v < c->tile_limit) c->tile_limit = (size_t)v;
    }
    c->cap = kv_capacity;
    (void)hipGetDevice(&c->device);
    {
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, c->device) == hipSuccess &&
            ncu > 0)
            c->n_cu = ncu;
    }
    q35::Dims& d = c->d;
    d.nk = cfg->ssm_group_count;
    d.nv = cfg->ssm_time_step_rank;
    d.key_dim = d.nk * q35::kDk;
    d.value_dim = d.nv * q35::kDk;
    d.conv_dim = 2 * d.key_dim + d.value_dim;
    d.nh = cfg->num_heads;
    d.nkv = cfg->num_kv_heads;
    d.q_dim = d.nh * q35::kHd;
    d.kv_dim = d.nkv * q35::kHd;
    d.eps = cfg->eps;
    d.rope_base = cfg->rope_base;
    c->is_recurrent.resize(cfg->num_layers);
    for (int l = 0; l < cfg->num_layers; l++)
        c->is_recurrent[l] = cfg->is_recurrent ? (cfg->is_recurrent[l] != 0)
                                               : ((l + 1) % cfg->full_attention_interval != 0);
    c->kv_len.assign(n_seqs, 0);
    c->len_dirty.assign(n_seqs, 0);
    c->marks.assign(n_seqs, q35::DropMarks());

    int r = Q35M_OK;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        r = hip_fail(e, "hipStreamCreate");
        delete c;
        return r;
    }
    // The device is current here: its fixed decode-attention scratch.
    if ((r = scratch_for_device(c->device, &c->noalloc_scratch))) {
        std::string msg = g_last_error;
        release(c);
        delete c;
        g_last_error = msg;
        return r;
    }
    c->lin.resize(cfg->num_layers);
    c->full.resize(cfg->num_layers);
    size_t state_bytes = (size_t)n_seqs * d.nv * q35::kDk * q35::kDk * sizeof(float);
    size_t conv_bytes = (size_t)n_seqs * d.win_floats() * sizeof(float);
    size_t kv_bytes = (size_t)n_seqs * kv_capacity * d.kv_dim * sizeof(float);
    r = alloc_zero(c, (void**)&c->dev_len, (size_t)n_seqs * sizeof(int));
    for (int l = 0; l < cfg->num_layers && r == Q35M_OK; l++) {
        if (c->is_recurrent[l]) {
            q35::DeltaNetLayer& L = c->lin[l];
            r = alloc_zero(c, (void**)&L.state, state_bytes);
            if (!r) r = alloc_zero(c, (void**)&L.conv, conv_bytes);
            if (!r) r = alloc_zero(c, (void**)&L.conv_w, (size_t)q35::kConvK * d.conv_dim * 4);
            if (!r) r = alloc_zero(c, (void**)&L.ssm_a, (size_t)d.nv * 4);
            if (!r) r = alloc_zero(c, (void**)&L.dt_bias, (size_t)d.nv * 4);
            if (!r) r = alloc_zero(c, (void**)&L.ssm_norm, (size_t)q35::kDk * 4);
        } else {
            q35::AttnLayer& L = c->full[l];
            r = alloc_zero(c, (void**)&L.k_cache, kv_bytes);
            if (!r) r = alloc_zero(c, (void**)&L.v_cache, kv_bytes);
            if (!r) r = alloc_zero(c, (void**)&L.q_norm, (size_t)q35::kHd * 4);
            if (!r) r = alloc_zero(c, (void**)&L.k_norm, (size_t)q35::kHd * 4);
        }
    }
    if (!r) {
        c->rope_cap = kv_capacity > 4096 ? kv_capacity : 4096;
        std::vector<float> cs, sn;
        build_rope_table(c->rope_cap, q35::kRopeHalf, cfg->rope_base, cs, sn);
        size_t tb = cs.size() * sizeof(float);
        r = alloc_zero(c, (void**)&c->rope_cos, tb);
        if (!r) r = alloc_zero(c, (void**)&c->rope_sin, tb);
        if (!r) {
            e = hipMemcpyAsync(c->rope_cos, cs.data(), tb, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess)
                e = hipMemcpyAsync(c->rope_sin, sn.data(), tb, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
            if (e != hipSuccess) r = hip_fail(e, "RoPE table upload");
        }
    }
    if (r) {
        std::string msg = g_last_error;
        release(c);
        delete c;
        g_last_error = msg;
        return r;
    }
    *out = c;
    return Q35M_OK;
}

int q35m_destroy(q35m_ctx* ctx) {
    int r = check_ctx(ctx);
    if (r) return r;
    release(ctx);
    delete ctx;
    return Q35M_OK;
}

int q35m_reset(q35m_ctx* ctx, int seq) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    const q35::Dims& d = ctx->d;
    size_t sb = (size_t)d.nv * q35::kDk * q35::kDk * sizeof(float);
    size_t cb = d.win_floats() * sizeof(float);
    for (int l = 0; l < ctx->cfg.num_layers; l++) {
        if (!ctx->is_recurrent[l]) continue;
        HIP_TRY(hipMemsetAsync((char*)ctx->lin[l].state + sb * seq, 0, sb, ctx->stream), "reset");
        HIP_TRY(hipMemsetAsync(ctx->lin[l].conv_window(seq, d.win_floats()), 0, cb, ctx->stream), "reset");
    }
    set_len(ctx, seq, 0);
    ctx->marks[seq].drop(0);
    return Q35M_OK;
}

int q35m_truncate(q35m_ctx* ctx, int seq, int length) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (length < 0) return fail(Q35M_ERR_INVALID, "negative length %d", length);
    if (length > ctx->kv_len[seq])
        return fail(Q35M_ERR_RANGE, "cannot extend cache from %d to %d", ctx->kv_len[seq], length);
    if (length < ctx->kv_len[seq]) ctx->marks[seq].drop(length);
    set_len(ctx, seq, length);
    return Q35M_OK;
}

int q35m_advance(q35m_ctx* ctx, int seq, int n) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (n < 0) return fail(Q35M_ERR_INVALID, "negative advance %d", n);
    if ((long)ctx->kv_len[seq] + n > ctx->cap)
        return fail(Q35M_ERR_CAPACITY, "sequence %d: length %d + %d exceeds capacity %d", seq,
                    ctx->kv_len[seq], n, ctx->cap);
    set_len(ctx, seq, ctx->kv_len[seq] + n);
    return Q35M_OK;
}

int q35m_kv_len(const q35m_ctx* ctx, int seq, int* length) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (!length) return fail(Q35M_ERR_INVALID, "null length");
    *length = ctx->kv_len[seq];
    return Q35M_OK;
}

int q35m_set_deltanet_weights(q35m_ctx* ctx, int layer, const float* conv_w, const float* ssm_a,
                              const float* dt_bias, const float* ssm_norm) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, true);
    if (r) return r;
    if (!conv_w || !ssm_a || !dt_bias || !ssm_norm) return fail(Q35M_ERR_INVALID, "null weight");
    q35::DeltaNetLayer& L = ctx->lin[layer];
    const q35::Dims& d = ctx->d;
    HIP_TRY(hipMemcpyAsync(L.conv_w, conv_w, (size_t)q35::kConvK * d.conv_dim * 4,
                           hipMemcpyHostToDevice, ctx->stream), "upload conv_w");
    HIP_TRY(hipMemcpyAsync(L.ssm_a, ssm_a, (size_t)d.nv * 4, hipMemcpyHostToDevice, ctx->stream),
            "upload ssm_a");
    HIP_TRY(hipMemcpyAsync(L.dt_bias, dt_bias, (size_t)d.nv * 4, hipMemcpyHostToDevice,
                           ctx->stream), "upload dt_bias");
    HIP_TRY(hipMemcpyAsync(L.ssm_norm, ssm_norm, (size_t)q35::kDk * 4, hipMemcpyHostToDevice,
                           ctx->stream), "upload ssm_norm");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload weights");
    L.has_weights = true;
    return Q35M_OK;
}

int q35m_set_attn_weights(q35m_ctx* ctx, int layer, const float* q_norm, const float* k_norm) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, false);
    if (r) return r;
    if (!q_norm || !k_norm) return fail(Q35M_ERR_INVALID, "null weight");
    q35::AttnLayer& L = ctx->full[layer];
    HIP_TRY(hipMemcpyAsync(L.q_norm, q_norm, q35::kHd * 4, hipMemcpyHostToDevice, ctx->stream),
            "upload q_norm");
    HIP_TRY(hipMemcpyAsync(L.k_norm, k_norm, q35::kHd * 4, hipMemcpyHostToDevice, ctx->stream),
            "upload k_norm");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload weights");
    L.has_weights = true;
    return Q35M_OK;
}

int q35m_deltanet_decode(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* qkv,
                         const float* z, const float* b, const float* a, float* out) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, true);
    if (r) return r;
    if (!ctx->lin[layer].has_weights) return fail(Q35M_ERR_INVALID, "layer %d has no weights", layer);
    if ((r = check_activations({qkv, z, b, a, out}))) return r;
    q35::SeqBatch sb;
    r = build_seq_batch(ctx, n, seqs, &sb, nullptr);
    if (r) return r;
    HIP_TRY(q35::launch_deltanet_decode(ctx, layer, sb, qkv, z, b, a, out), "deltanet_decode");
    return Q35M_OK;
}

int q35m_deltanet_prefill(q35m_ctx* ctx, int layer, int seq, int T, const float* qkv,
                          const float* z, const float* b, const float* a, float* out) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, true);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (!ctx->lin[layer].has_weights) return fail(Q35M_ERR_INVALID, "layer %d has no weights", layer);
    if (T < 1) return fail(Q35M_ERR_INVALID, "T must be >= 1 (got %d)", T);
    if ((r = check_activations({qkv, z, b, a, out}))) return r;
    HIP_TRY(q35::ensure_work(ctx, q35::deltanet_prefill_work_bytes(ctx->d, T)), "workspace");
    HIP_TRY(q35::launch_deltanet_prefill(ctx, layer, seq, T, qkv, z, b, a, out), "deltanet_prefill");
    return Q35M_OK;
}

int q35m_attn_decode(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* q_gate,
                     const float* k, const float* v, float* out) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, false);
    if (r) return r;
    if (!ctx->full[layer].has_weights) return fail(Q35M_ERR_INVALID, "layer %d has no weights", layer);
    if ((r = check_activations({q_gate, k, v, out}))) return r;
    q35::SeqBatch sb;
    int max_cached = 0;
    r = build_seq_batch(ctx, n, seqs, &sb, &max_cached);
    if (r) return r;
    const q35::DecodePlan p = q35::plan_attn_decode(ctx, n, max_cached);
    HIP_TRY(q35::ensure_work(ctx, q35::attn_decode_work_bytes(ctx, n, p)), "workspace");
    HIP_TRY(q35::flush_lengths(ctx), "attn_decode lengths");
    HIP_TRY(q35::launch_attn_decode(ctx, layer, sb, p, q_gate, k, v, out, ctx->work), "attn_decode");
    return Q35M_OK;
}

int q35m_attn_decode_noalloc(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* q_gate,
                             const float* k, const float* v, float* out) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, false);
    if (r) return r;
    if (!ctx->full[layer].has_weights) return fail(Q35M_ERR_INVALID, "layer %d has no weights", layer);
    if ((r = check_activations({q_gate, k, v, out}))) return r;
    if (!ctx->noalloc_scratch) return fail(Q35M_ERR_NO_DEVICE, "no device scratch");
    q35::SeqBatch sb;
    int max_cached = 0;
    r = build_seq_batch(ctx, n, seqs, &sb, &max_cached);
    if (r) return r;
    const q35::DecodePlan p = q35::plan_attn_decode(ctx, n, max_cached);
    const size_t need = q35::attn_decode_work_bytes(ctx, n, p);
    if (need > q35::kNoAllocScratchBytes)
        return fail(Q35M_ERR_CAPACITY,
                    "attn_decode_noalloc: this batch needs %zu bytes of split-K partials, the fixed scratch "
                    "holds %zu (use q35m_attn_decode, or fewer sequences per call)",
                    need, q35::kNoAllocScratchBytes);
    // No per-kernel timers here: they may create events.
    const bool prof = ctx->profile;
    ctx->profile = false;
    hipError_t e = q35::flush_lengths(ctx);
    if (e == hipSuccess) e = q35::launch_attn_decode(ctx, layer, sb, p, q_gate, k, v, out, ctx->noalloc_scratch);
    ctx->profile = prof;
    HIP_TRY(e, "attn_decode_noalloc");
    return Q35M_OK;
}

int q35m_attn_prefill(q35m_ctx* ctx, int layer, int seq, int T, const float* q_gate,
                      const float* k, const float* v, float* out) {
    int r = check_ctx(ctx);
    if (!r) r = check_layer(ctx, layer, false);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (!ctx->full[layer].has_weights) return fail(Q35M_ERR_INVALID, "layer %d has no weights", layer);
    if (T < 1) return fail(Q35M_ERR_INVALID, "T must be >= 1 (got %d)", T);
    if ((r = check_activations({q_gate, k, v, out}))) return r;
    int start = ctx->kv_len[seq];
    if ((long)start + T > ctx->cap)
        return fail(Q35M_ERR_CAPACITY, "sequence %d: %d + %d rows exceed KV capacity %d", seq, start,
                    T, ctx->cap);
    if ((long)start + T > q35::kPrefillMaxRows)
        return fail(Q35M_ERR_UNSUPPORTED, "attention prefill reads at most %d cached rows (sequence %d "
                    "would reach %d)", q35::kPrefillMaxRows, seq, start + T);
    HIP_TRY(q35::ensure_work(ctx, q35::attn_prefill_work_bytes(ctx->d, T)), "workspace");
    HIP_TRY(q35::launch_attn_prefill(ctx, layer, seq, start, T, q_gate, k, v, out), "attn_prefill");
    return Q35M_OK;
}

static int check_linear_dims(int n_in, int n_out, int tokens) {
    if (n_in < 256 || n_in > 16384 || n_in % 256)
        return fail(Q35M_ERR_UNSUPPORTED, "n_in must be a multiple of 256 in [256, 16384] (got %d)", n_in);
    if (n_out < 1) return fail(Q35M_ERR_INVALID, "n_out must be >= 1 (got %d)", n_out);
    if (tokens < 1 || tokens > 65535)
        return fail(Q35M_ERR_INVALID, "tokens must be in [1, 65535] (got %d)", tokens);
    return Q35M_OK;
}

static int check_linear_type(int qtype, int n_in) {
    if (qtype == 2 && n_in % 512)
        return fail(Q35M_ERR_UNSUPPORTED, "Q2_0C rows need a multiple of 512 inputs (got %d)", n_in);
    return Q35M_OK;
}

static int linear_q(q35m_ctx* ctx, int qtype, const void* w, const float* x, float* y, int n_in,
                    int n_out, int tokens) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!w || !x || !y) return fail(Q35M_ERR_INVALID, "null pointer");
    if (((uintptr_t)w & 15) || ((uintptr_t)x & 15))
        return fail(Q35M_ERR_INVALID, "weights and input must be 16-byte aligned");
    if ((r = check_linear_dims(n_in, n_out, tokens))) return r;
    if ((r = check_linear_type(qtype, n_in))) return r;
    HIP_TRY(q35::ensure_work(ctx, q35::linear_q_work_bytes(n_in, tokens)), "workspace");
    HIP_TRY(q35::launch_linear_q(ctx, qtype, w, x, y, n_in, n_out, tokens), "linear_q");
    return Q35M_OK;
}

int q35m_set_projection_order(q35m_ctx* ctx, int order) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (order != Q35M_PROJ_REFERENCE && order != Q35M_PROJ_BLOCK)
        return fail(Q35M_ERR_INVALID, "unknown projection order %d", order);
    ctx->proj_order = order;
    return Q35M_OK;
}

size_t q35m_q8k_bytes(int n_in, int tokens) {
    return (n_in > 0 && tokens > 0) ? q35::linear_q_work_bytes(n_in, tokens) : 0;
}

int q35m_quantize_q8k(q35m_ctx* ctx, const float* x, void* q8, int n_in, int tokens) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!x || !q8) return fail(Q35M_ERR_INVALID, "null pointer");
    if (((uintptr_t)x & 15) || ((uintptr_t)q8 & 15))
        return fail(Q35M_ERR_INVALID, "input and Q8_K buffer must be 16-byte aligned");
    if ((r = check_linear_dims(n_in, 1, tokens))) return r;
    HIP_TRY(q35::launch_q8k_quantize(ctx, x, q8, n_in, tokens), "quantize_q8k");
    return Q35M_OK;
}

static void free_alloc(q35m_ctx* c, void* p) {
    for (size_t i = 0; i < c->allocations.size(); i++)
        if (c->allocations[i] == p) {
            c->allocations.erase(c->allocations.begin() + (long)i);
            break;
        }
    (void)hipFree(p);
}

int q35m_grow(q35m_ctx* ctx, int kv_capacity) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (kv_capacity < ctx->cap)
        return fail(Q35M_ERR_RANGE, "cannot shrink the KV capacity from %d to %d", ctx->cap, kv_capacity);
    if (kv_capacity == ctx->cap) return Q35M_OK;
    const q35::Dims& d = ctx->d;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "grow");
    // New caches first; the context keeps the old ones until every copy is done.
    std::vector<float*> fresh;
    const size_t row = (size_t)q35::kHd * sizeof(float);
    const size_t kv_bytes = (size_t)ctx->n_seqs * kv_capacity * d.kv_dim * sizeof(float);
    hipError_t e = hipSuccess;
    for (int l = 0; l < ctx->cfg.num_layers && !r && e == hipSuccess; l++) {
        if (ctx->is_recurrent[l]) continue;
        for (float* old : {ctx->full[l].k_cache, ctx->full[l].v_cache}) {
            float* p = nullptr;
            if ((r = alloc_zero(ctx, (void**)&p, kv_bytes))) break;
            fresh.push_back(p);
            // [seq][kv_head] blocks of [capacity][head_dim]: one strided copy
            e = hipMemcpy2DAsync(p, row * kv_capacity, old, row * ctx->cap, row * ctx->cap,
                                 (size_t)ctx->n_seqs * d.nkv, hipMemcpyDeviceToDevice, ctx->stream);
            if (e != hipSuccess) break;
        }
    }
    float *rc = nullptr, *rs = nullptr;
    if (!r && e == hipSuccess && kv_capacity > ctx->rope_cap) {
        std::vector<float> cs, sn;
        build_rope_table(kv_capacity, q35::kRopeHalf, ctx->cfg.rope_base, cs, sn);
        const size_t tb = cs.size() * sizeof(float);
        r = alloc_zero(ctx, (void**)&rc, tb);
        if (!r) r = alloc_zero(ctx, (void**)&rs, tb);
        if (!r) e = hipMemcpyAsync(rc, cs.data(), tb, hipMemcpyHostToDevice, ctx->stream);
        if (!r && e == hipSuccess) e = hipMemcpyAsync(rs, sn.data(), tb, hipMemcpyHostToDevice, ctx->stream);
    }
    hipError_t es = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = es;
    if (r || e != hipSuccess) {
        for (float* p : fresh) free_alloc(ctx, p);
        if (rc) free_alloc(ctx, rc);
        if (rs) free_alloc(ctx, rs);
        return r ? r : hip_fail(e, "grow");
    }
    size_t k = 0;
    for (int l = 0; l < ctx->cfg.num_layers; l++) {
        if (ctx->is_recurrent[l]) continue;
        free_alloc(ctx, ctx->full[l].k_cache);
        free_alloc(ctx, ctx->full[l].v_cache);
        ctx->full[l].k_cache = fresh[k++];
        ctx->full[l].v_cache = fresh[k++];
    }
    if (rc) {
        free_alloc(ctx, ctx->rope_cos);
        free_alloc(ctx, ctx->rope_sin);
        ctx->rope_cos = rc;
        ctx->rope_sin = rs;
        ctx->rope_cap = kv_capacity;
    }
    ctx->cap = kv_capacity;
    ctx->generation++;
    return Q35M_OK;
}

size_t q35m_snapshot_bytes(const q35m_ctx* ctx) {
    if (!ctx) return 0;
    const q35::Dims& d = ctx->d;
    const size_t per = ((size_t)d.nv * q35::kDk * q35::kDk + d.win_floats()) * sizeof(float);
    size_t n = 0;
    for (int l = 0; l < ctx->cfg.num_layers; l++) n += ctx->is_recurrent[l] ? 1 : 0;
    return n * per;
}

// One sequence's recurrent state and current conv window of every DeltaNet
// layer, in layer order, to or from a device buffer (asynchronous copies on
// the context stream).
static int snapshot_copy(q35m_ctx* ctx, int seq, char* dev, bool save) {
    const q35::Dims& d = ctx->d;
    const size_t sb = (size_t)d.nv * q35::kDk * q35::kDk * sizeof(float);
    const size_t cb = d.win_floats() * sizeof(float);
    for (int l = 0; l < ctx->cfg.num_layers; l++) {
        if (!ctx->is_recurrent[l]) continue;
        char* st = (char*)ctx->lin[l].state + sb * seq;
        char* cw = (char*)ctx->lin[l].conv_window(seq, d.win_floats());
        HIP_TRY(hipMemcpyAsync(save ? dev : st, save ? st : dev, sb, hipMemcpyDeviceToDevice, ctx->stream),
                "snapshot");
        dev += sb;
        HIP_TRY(hipMemcpyAsync(save ? dev : cw, save ? cw : dev, cb, hipMemcpyDeviceToDevice, ctx->stream),
                "snapshot");
        dev += cb;
    }
    return Q35M_OK;
}

static int snapshot_check(q35m_ctx* ctx, int seq, const void* dev, size_t bytes, const void* info) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    const size_t need = q35m_snapshot_bytes(ctx);
    if (!info || (!dev && need)) return fail(Q35M_ERR_INVALID, "null pointer");
    if (bytes < need) return fail(Q35M_ERR_INVALID, "snapshot buffer of %zu bytes, %zu needed", bytes, need);
    return Q35M_OK;
}

int q35m_snapshot_save(q35m_ctx* ctx, int seq, void* dev, size_t bytes, q35m_snapshot_info* info) {
    int r = snapshot_check(ctx, seq, dev, bytes, info);
    if (r) return r;
    if ((r = snapshot_copy(ctx, seq, (char*)dev, true))) return r;
    info->kv_len = ctx->kv_len[seq];
    info->epoch = ctx->marks[seq].save();
    return Q35M_OK;
}

static int snapshot_refused(const q35m_ctx* ctx, int seq, const q35m_snapshot_info* info) {
    return fail(Q35M_ERR_RANGE,
                "snapshot at length %d no longer matches sequence %d at length %d (the sequence was shorter "
                "than that since the save: reset, truncate, restore to a shorter length, or K/V rows written)",
                info->kv_len, seq, ctx->kv_len[seq]);
}

int q35m_snapshot_valid(const q35m_ctx* ctx, int seq, const q35m_snapshot_info* info) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    if (!info) return fail(Q35M_ERR_INVALID, "null snapshot info");
    if (!ctx->marks[seq].restorable(info->epoch, info->kv_len, ctx->kv_len[seq]))
        return snapshot_refused(ctx, seq, info);
    return Q35M_OK;
}

int q35m_snapshot_restore(q35m_ctx* ctx, int seq, const void* dev, size_t bytes,
                          q35m_snapshot_info* info) {
    int r = snapshot_check(ctx, seq, dev, bytes, info);
    if (r) return r;
    if (!ctx->marks[seq].restorable(info->epoch, info->kv_len, ctx->kv_len[seq]))
        return snapshot_refused(ctx, seq, info);
    if ((r = snapshot_copy(ctx, seq, const_cast<char*>((const char*)dev), false))) return r;
    // Rows at and above the restored length will be written again: snapshots
    // longer than it no longer hold (this one and shorter ones still do).
    if (info->kv_len < ctx->kv_len[seq]) ctx->marks[seq].drop(info->kv_len);
    set_len(ctx, seq, info->kv_len);
    return Q35M_OK;
}

int q35m_reuse_plan(const int* cached, int n_cached, const int* prompt, int n_prompt,
                    const int* snap_lens, int n_snaps, int* truncate_to, int* suffix_start, int* snap) {
    if (n_cached < 0 || n_prompt < 0 || n_snaps < 0)
        return fail(Q35M_ERR_INVALID, "negative count (cached %d, prompt %d, snapshots %d)", n_cached, n_prompt,
                    n_snaps);
    if ((n_cached && !cached) || (n_prompt && !prompt) || (n_snaps && !snap_lens) || !truncate_to ||
        !suffix_start || !snap)
        return fail(Q35M_ERR_INVALID, "null pointer");
    // KvCacheAlign.Plan: an empty prompt keeps nothing; a prompt cached whole
    // keeps all but its last token; otherwise the common prefix.
    int keep = 0;
    if (n_prompt > 0) {
        const int n = n_cached < n_prompt ? n_cached : n_prompt;
        int common = 0;
        while (common < n && cached[common] == prompt[common]) ++common;
        keep = common == n_prompt ? n_prompt - 1 : common;
    }
    int best = -1;
    if (n_snaps > 0) {
        for (int i = 0; i < n_snaps; ++i)
            if (snap_lens[i] >= 0 && snap_lens[i] <= keep && (best < 0 || snap_lens[i] > snap_lens[best]))
                best = i;
        keep = best < 0 ? 0 : snap_lens[best];
    }
    *truncate_to = keep;
    *suffix_start = keep;
    *snap = best;
    return Q35M_OK;
}

int q35m_add_rmsnorm(q35m_ctx* ctx, float* hidden, const float* delta, const float* weight, float* y, void* q8,
                     int dim, int tokens, float eps) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!hidden || (!y && !q8)) return fail(Q35M_ERR_INVALID, "null hidden, or neither y nor q8 given");
    if (((uintptr_t)hidden | (uintptr_t)delta | (uintptr_t)weight | (uintptr_t)y | (uintptr_t)q8) & 15)
        return fail(Q35M_ERR_INVALID, "buffers must be 16-byte aligned");
    if (tokens < 1 || dim < 4) return fail(Q35M_ERR_INVALID, "dim %d, tokens %d", dim, tokens);
    if (dim % 4 || dim > 16384) return fail(Q35M_ERR_UNSUPPORTED, "dim %d: a multiple of 4 up to 16384", dim);
    if (q8 && dim % 256) return fail(Q35M_ERR_UNSUPPORTED, "Q8_K output needs dim a multiple of 256 (%d)", dim);
    if (!(eps >= 0.0f)) return fail(Q35M_ERR_INVALID, "eps must be >= 0");
    HIP_TRY(q35::launch_add_rmsnorm(ctx, hidden, delta, weight, y, q8, dim, tokens, eps), "add_rmsnorm");
    return Q35M_OK;
}

static int linear_q_prequant(q35m_ctx* ctx, int qtype, const void* w, const void* q8, float* y,
                             int n_in, int n_out, int tokens) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!w || !q8 || !y) return fail(Q35M_ERR_INVALID, "null pointer");
    if (((uintptr_t)w & 15) || ((uintptr_t)q8 & 15))
        return fail(Q35M_ERR_INVALID, "weights and Q8_K buffer must be 16-byte aligned");
    if ((r = check_linear_dims(n_in, n_out, tokens))) return r;
    if ((r = check_linear_type(qtype, n_in))) return r;
    HIP_TRY(q35::launch_linear_q_prequant(ctx, qtype, w, q8, y, n_in, n_out, tokens), "linear_q");
    return Q35M_OK;
}

int q35m_linear_q4k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens) {
    return linear_q_prequant(ctx, 4, w, q8, y, n_in, n_out, tokens);
}

int q35m_linear_q6k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens) {
    return linear_q_prequant(ctx, 6, w, q8, y, n_in, n_out, tokens);
}

int q35m_linear_q4k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens) {
    return linear_q(ctx, 4, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_f32(q35m_ctx* ctx, const float* w, const float* x, float* y, int n_in, int n_out,
                    int tokens) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!w || !x || !y) return fail(Q35M_ERR_INVALID, "null pointer");
    if (n_in < 1 || n_out < 1) return fail(Q35M_ERR_INVALID, "n_in %d, n_out %d", n_in, n_out);
    if (tokens < 1 || tokens > 65535)
        return fail(Q35M_ERR_INVALID, "tokens must be in [1, 65535] (got %d)", tokens);
    HIP_TRY(q35::launch_linear_f32(ctx, w, x, y, n_in, n_out, tokens), "linear_f32");
    return Q35M_OK;
}

int q35m_linear_q5k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens) {
    return linear_q(ctx, 5, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_iq4xs(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                      int tokens) {
    return linear_q(ctx, 14, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_q5k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens) {
    return linear_q_prequant(ctx, 5, w, q8, y, n_in, n_out, tokens);
}

int q35m_linear_iq4xs_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                               int n_out, int tokens) {
    return linear_q_prequant(ctx, 14, w, q8, y, n_in, n_out, tokens);
}

int q35m_linear_q6k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens) {
    return linear_q(ctx, 6, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_q2_0c(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                      int tokens) {
    return linear_q(ctx, 2, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_stq1_0(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                       int tokens) {
    return linear_q(ctx, 1, w, x, y, n_in, n_out, tokens);
}

int q35m_linear_q2_0c_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                               int n_out, int tokens) {
    return linear_q_prequant(ctx, 2, w, q8, y, n_in, n_out, tokens);
}

int q35m_linear_stq1_0_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                                int n_out, int tokens) {
    return linear_q_prequant(ctx, 1, w, q8, y, n_in, n_out, tokens);
}

static int state_locate(q35m_ctx* ctx, int layer, int seq, int kind, char** base, size_t* bytes) {
    int r = check_ctx(ctx);
    if (!r) r = check_seq(ctx, seq);
    if (r) return r;
    const q35::Dims& d = ctx->d;
    if (kind == Q35M_STATE_RECURRENT || kind == Q35M_STATE_CONV) {
        r = check_layer(ctx, layer, true);
        if (r) return r;
        if (kind == Q35M_STATE_RECURRENT) {
            *bytes = (size_t)d.nv * q35::kDk * q35::kDk * sizeof(float);
            *base = (char*)ctx->lin[layer].state + *bytes * seq;
        } else {
            *bytes = (size_t)d.conv_dim * q35::kConvState * sizeof(float);
            *base = (char*)ctx->lin[layer].conv_window(seq, d.win_floats());
        }
        return Q35M_OK;
    }
    if (kind == Q35M_STATE_KEYS || kind == Q35M_STATE_VALUES) {
        r = check_layer(ctx, layer, false);
        if (r) return r;
        *bytes = (size_t)ctx->cap * d.kv_dim * sizeof(float);
        float* cache = kind == Q35M_STATE_KEYS ? ctx->full[layer].k_cache : ctx->full[layer].v_cache;
        *base = (char*)cache + *bytes * seq;
        return Q35M_OK;
    }
    return fail(Q35M_ERR_INVALID, "unknown state kind %d", kind);
}

// K/V caches are head-major on the device ([kv_heads][cap][head_dim] per
// (layer, seq)); state I/O moves whole rows in the reference layout
// [rows][kv_heads * head_dim], one strided 2-D copy per kv head.
static hipError_t kv_copy(q35m_ctx* ctx, char* dev, void* host, size_t bytes, bool to_host) {
    const q35::Dims& d = ctx->d;
    const size_t row_bytes = (size_t)d.kv_dim * sizeof(float), head_bytes = q35::kHd * sizeof(float);
    const size_t rows = bytes / row_bytes;
    if (rows == 0) return hipSuccess;
    for (int h = 0; h < d.nkv; h++) {
        char* dh = dev + (size_t)h * ctx->cap * head_bytes;
        char* hh = static_cast<char*>(host) + (size_t)h * head_bytes;
        hipError_t e = to_host ? hipMemcpy2DAsync(hh, row_bytes, dh, head_bytes, head_bytes, rows,
                                                  hipMemcpyDeviceToHost, ctx->stream)
                               : hipMemcpy2DAsync(dh, head_bytes, hh, row_bytes, head_bytes, rows,
                                                  hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

static bool is_kv(int kind) { return kind == Q35M_STATE_KEYS || kind == Q35M_STATE_VALUES; }

int q35m_state_read(q35m_ctx* ctx, int layer, int seq, int kind, void* host, size_t bytes) {
    char* base;
    size_t cap_bytes;
    int r = state_locate(ctx, layer, seq, kind, &base, &cap_bytes);
    if (r) return r;
    if (!host) return fail(Q35M_ERR_INVALID, "null host buffer");
    if (bytes > cap_bytes)
        return fail(Q35M_ERR_INVALID, "read of %zu bytes exceeds the %zu-byte state", bytes, cap_bytes);
    if (is_kv(kind)) {
        if (bytes % ((size_t)ctx->d.kv_dim * sizeof(float)))
            return fail(Q35M_ERR_INVALID, "K/V reads move whole rows of %d floats", ctx->d.kv_dim);
        HIP_TRY(kv_copy(ctx, base, host, bytes, true), "state_read");
    } else {
        HIP_TRY(hipMemcpyAsync(host, base, bytes, hipMemcpyDeviceToHost, ctx->stream), "state_read");
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "state_read");
    return Q35M_OK;
}

int q35m_state_write(q35m_ctx* ctx, int layer, int seq, int kind, const void* host,
                     size_t bytes) {
    char* base;
    size_t cap_bytes;
    int r = state_locate(ctx, layer, seq, kind, &base, &cap_bytes);
    if (r) return r;
    if (!host) return fail(Q35M_ERR_INVALID, "null host buffer");
    if (bytes > cap_bytes)
        return fail(Q35M_ERR_INVALID, "write of %zu bytes exceeds the %zu-byte state", bytes,
                    cap_bytes);
    if (is_kv(kind)) {
        if (bytes % ((size_t)ctx->d.kv_dim * sizeof(float)))
            return fail(Q35M_ERR_INVALID, "K/V writes move whole rows of %d floats", ctx->d.kv_dim);
        // Rows from 0 are about to change: as a drop of the length to 0.
        ctx->marks[seq].drop(0);
        HIP_TRY(kv_copy(ctx, base, const_cast<void*>(host), bytes, false), "state_write");
    } else {
        HIP_TRY(hipMemcpyAsync(base, host, bytes, hipMemcpyHostToDevice, ctx->stream), "state_write");
        if (kind == Q35M_STATE_CONV) {
            // The q/k channels' windows (the block's first 2 * key_dim rows)
            // into the decode copies after the [conv_dim][3] block.
            const size_t qk = (size_t)2 * ctx->d.key_dim * q35::kConvState * sizeof(float);
            const size_t nq = bytes < qk ? bytes : qk;
            const size_t blk = (size_t)ctx->d.conv_dim * q35::kConvState * sizeof(float);
            for (int r = 1; r < ctx->d.nv / ctx->d.nk && nq; r++)
                HIP_TRY(hipMemcpyAsync(base + blk + (size_t)(r - 1) * qk, base, nq, hipMemcpyDeviceToDevice,
                                       ctx->stream),
                        "state_write");
        }
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "state_write");
    return Q35M_OK;
}

int q35m_state_device_ptr(q35m_ctx* ctx, int layer, int seq, int kind, void** dptr,
                          size_t* bytes) {
    char* base;
    size_t cap_bytes;
    int r = state_locate(ctx, layer, seq, kind, &base, &cap_bytes);
    if (r) return r;
    if (dptr) *dptr = base;
    if (bytes) *bytes = cap_bytes;
    return Q35M_OK;
}

int q35m_sync(q35m_ctx* ctx) {
    int r = check_ctx(ctx);
    if (r) return r;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "sync");
    return Q35M_OK;
}

void* q35m_stream(q35m_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int q35m_profile(q35m_ctx* ctx, int enable) {
    int r = check_ctx(ctx);
    if (r) return r;
    HIP_TRY(q35::collect_profile(ctx), "profile");
    ctx->profile = enable != 0;
    for (int k = 0; k < q35::K_COUNT; k++) {
        ctx->prof_ms[k] = 0.0;
        ctx->prof_n[k] = 0;
    }
    return Q35M_OK;
}

int q35m_profile_read(q35m_ctx* ctx, int kernel, double* total_ms, long* launches) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (kernel < 0 || kernel >= q35::K_COUNT)
        return fail(Q35M_ERR_INVALID, "kernel id %d out of range [0, %d)", kernel, q35::K_COUNT);
    HIP_TRY(q35::collect_profile(ctx), "profile_read");
    if (total_ms) *total_ms = ctx->prof_ms[kernel];
    if (launches) *launches = ctx->prof_n[kernel];
    return Q35M_OK;
}

const char* q35m_profile_kernel_name(int kernel) { return q35::kernel_name(kernel); }

int q35m_malloc(void** dptr, size_t bytes) {
    if (!dptr) return fail(Q35M_ERR_INVALID, "null pointer");
    *dptr = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return fail(Q35M_ERR_NO_DEVICE, "no HIP device available");
    HIP_TRY(hipMalloc(dptr, bytes), "hipMalloc");
    return Q35M_OK;
}

int q35m_free(void* dptr) {
    if (!dptr) return Q35M_OK;
    HIP_TRY(hipFree(dptr), "hipFree");
    return Q35M_OK;
}

int q35m_copy_h2d(q35m_ctx* ctx, void* dst, const void* src, size_t bytes) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!dst || !src) return fail(Q35M_ERR_INVALID, "null pointer");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "copy_h2d");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "copy_h2d");
    return Q35M_OK;
}

int q35m_copy_d2h(q35m_ctx* ctx, void* dst, const void* src, size_t bytes) {
    int r = check_ctx(ctx);
    if (r) return r;
    if (!dst || !src) return fail(Q35M_ERR_INVALID, "null pointer");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "copy_d2h");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "copy_d2h");
    return Q35M_OK;
}

}  // extern "C"
