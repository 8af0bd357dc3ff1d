// Device-resident sequence lengths and the captured decode step.
//
// The reference's decode forward (Qwen35Model.Forward, src/Qwen35Sharp.Model/
// Qwen35Model.cs:231-291) runs every layer's mixer at the sequence's current
// length and then advances it once (`_cacheLen += seq`, :287).  Here the
// lengths also live in device memory (q35m_ctx::dev_len), the decode
// attention kernels read them there, and a decode graph ends each step with
// a one-thread-per-sequence kernel that advances them.  So the whole step --
// every layer's mixer launches plus the advance -- is captured once into a
// HIP graph and the same graph is replayed for every token: nothing in it is
// tied to the position it was captured at.  (The DeltaNet conv windows need
// no per-step host state either: each decode workgroup rewrites its own copy
// of its windows in place.)
//
// Host changes to a length (reset, truncate, advance, snapshot restore) set
// the host copy and mark the sequence; flush_lengths writes every marked
// length with one small kernel before the next launch that reads them.
#include <cstdarg>
#include <cstdio>
#include <vector>

#include "common.h"
#include "q35mix_internal.h"

int q35_set_error(int code, const char* msg);

namespace q35 {
namespace {

struct LenSet {
    int n;
    int seq[kMaxBatch];
    int len[kMaxBatch];
};

// One thread per entry; the sequences of one launch are distinct.
__global__ __launch_bounds__(64) void lengths_set(int* __restrict__ lens, LenSet s) {
    const int t = threadIdx.x;
    if (t < s.n) lens[s.seq[t]] = s.len[t];
}

__global__ __launch_bounds__(64) void lengths_add(int* __restrict__ lens, SeqBatch sb, int k) {
    const int t = threadIdx.x;
    if (t < sb.n) lens[sb.seq[t]] += k;
}

}  // namespace

hipError_t flush_lengths(q35m_ctx* c) {
    LenSet s;
    s.n = 0;
    for (int q = 0; q < c->n_seqs; ++q) {
        if (!c->len_dirty[q]) continue;
        s.seq[s.n] = q;
        s.len[s.n] = c->kv_len[q];
        if (++s.n == kMaxBatch) {
            hipLaunchKernelGGL(lengths_set, dim3(1), dim3(64), 0, c->stream, c->dev_len, s);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            s.n = 0;
        }
    }
    if (s.n) {
        hipLaunchKernelGGL(lengths_set, dim3(1), dim3(64), 0, c->stream, c->dev_len, s);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    for (int q = 0; q < c->n_seqs; ++q) c->len_dirty[q] = 0;
    return hipSuccess;
}

hipError_t launch_lengths_add(q35m_ctx* c, const SeqBatch& sb, int k) {
    hipLaunchKernelGGL(lengths_add, dim3(1), dim3(64), 0, c->stream, c->dev_len, sb, k);
    return hipGetLastError();
}

}  // namespace q35

struct q35m_decode_graph {
    q35m_ctx* ctx = nullptr;
    q35::SeqBatch sb{};
    std::vector<q35m_decode_io> io;
    int max_len = 0;
    q35::DecodePlan plan{};
    float* partials = nullptr;      // split-K partials of the attention layers (owned)
    unsigned generation = 0;        // of the context at capture
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

int gfail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int gfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return q35_set_error(code, buf);
}

int ghip(hipError_t e, const char* what) {
    return gfail(e == hipErrorOutOfMemory ? Q35M_ERR_OOM : Q35M_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// The launches of one step, in layer order, then the advance.  Used for the
// capture and for the launch-by-launch run alike.
hipError_t enqueue_step(q35m_decode_graph* g) {
    q35m_ctx* c = g->ctx;
    for (int l = 0; l < c->cfg.num_layers; ++l) {
        const q35m_decode_io& x = g->io[l];
        hipError_t e;
        if (c->is_recurrent[l])
            e = q35::launch_deltanet_decode(c, l, g->sb, x.in0, x.in1, x.in2, x.in3, x.out);
        else
            e = q35::launch_attn_decode(c, l, g->sb, g->plan, x.in0, x.in1, x.in2, x.out, g->partials);
        if (e != hipSuccess) return e;
    }
    return q35::launch_lengths_add(c, g->sb, 1);
}

void release_graph(q35m_decode_graph* g) {
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->partials) {
        (void)hipStreamSynchronize(g->ctx->stream);
        (void)hipFree(g->partials);
    }
    g->exec = nullptr;
    g->graph = nullptr;
    g->partials = nullptr;
}

}  // namespace

extern "C" {

int q35m_decode_graph_create(q35m_ctx* ctx, int n, const int* seqs, const q35m_decode_io* io, int max_len,
                             q35m_decode_graph** out) {
    if (!out) return gfail(Q35M_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (!ctx) return gfail(Q35M_ERR_INVALID, "null context");
    if (!io || !seqs) return gfail(Q35M_ERR_INVALID, "null io or seqs");
    if (n < 1 || n > q35::kMaxBatch)
        return gfail(Q35M_ERR_CAPACITY, "batch of %d sequences (1..%d per graph)", n, q35::kMaxBatch);
    if (max_len < 1 || max_len > ctx->cap)
        return gfail(Q35M_ERR_CAPACITY, "max_len %d outside [1, %d] (the KV capacity)", max_len, ctx->cap);
    auto* g = new q35m_decode_graph();
    g->ctx = ctx;
    g->sb.n = n;
    for (int i = 0; i < n; ++i) {
        if (seqs[i] < 0 || seqs[i] >= ctx->n_seqs) {
            delete g;
            return gfail(Q35M_ERR_INVALID, "sequence %d out of range [0, %d)", seqs[i], ctx->n_seqs);
        }
        for (int j = 0; j < i; ++j)
            if (seqs[j] == seqs[i]) {
                delete g;
                return gfail(Q35M_ERR_INVALID, "sequence %d repeated", seqs[i]);
            }
        g->sb.seq[i] = seqs[i];
    }
    const int L = ctx->cfg.num_layers;
    g->io.assign(io, io + L);
    bool any_attn = false;
    for (int l = 0; l < L; ++l) {
        const q35m_decode_io& x = io[l];
        const bool rec = ctx->is_recurrent[l] != 0;
        const bool weights = rec ? ctx->lin[l].has_weights : ctx->full[l].has_weights;
        if (!weights) {
            delete g;
            return gfail(Q35M_ERR_INVALID, "layer %d has no weights", l);
        }
        if (!x.in0 || !x.in1 || !x.in2 || !x.out || (rec && !x.in3)) {
            delete g;
            return gfail(Q35M_ERR_INVALID, "layer %d: null activation pointer", l);
        }
        if (((uintptr_t)x.in0 | (uintptr_t)x.in1 | (uintptr_t)x.in2 | (uintptr_t)x.out |
             (uintptr_t)(rec ? x.in3 : nullptr)) & 15) {
            delete g;
            return gfail(Q35M_ERR_INVALID, "layer %d: activation pointers must be 16-byte aligned", l);
        }
        any_attn |= !rec;
    }
    g->max_len = max_len;
    g->plan = q35::plan_attn_decode(ctx, n, max_len - 1);
    g->generation = ctx->generation;
    if (any_attn) {
        const hipError_t e = hipMalloc((void**)&g->partials, q35::attn_decode_work_bytes(ctx, n, g->plan));
        if (e != hipSuccess) {
            delete g;
            return ghip(e, "decode graph partials");
        }
    }
    // Capture (no per-kernel timers: they would record events into the graph).
    const bool prof = ctx->profile;
    ctx->profile = false;
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        const hipError_t el = enqueue_step(g);
        e = hipStreamEndCapture(ctx->stream, &g->graph);
        if (el != hipSuccess) e = el;
    }
    ctx->profile = prof;
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        const int r = ghip(e, "decode graph capture");
        release_graph(g);
        delete g;
        return r;
    }
    *out = g;
    return Q35M_OK;
}

int q35m_decode_graph_run(q35m_decode_graph* g, int replay) {
    if (!g) return gfail(Q35M_ERR_INVALID, "null decode graph");
    q35m_ctx* c = g->ctx;
    if (c->generation != g->generation)
        return gfail(Q35M_ERR_RANGE, "the KV caches moved (q35m_grow) since the graph was captured; create it again");
    for (int i = 0; i < g->sb.n; ++i) {
        const int s = g->sb.seq[i];
        if (c->kv_len[s] >= g->max_len)
            return gfail(Q35M_ERR_CAPACITY, "sequence %d holds %d rows; the graph was captured for at most %d", s,
                         c->kv_len[s], g->max_len);
    }
    hipError_t e = q35::flush_lengths(c);
    if (e == hipSuccess) e = replay ? hipGraphLaunch(g->exec, c->stream) : enqueue_step(g);
    if (e != hipSuccess) return ghip(e, "decode graph run");
    for (int i = 0; i < g->sb.n; ++i) c->kv_len[g->sb.seq[i]] += 1;   // the step advanced the device copy
    return Q35M_OK;
}

int q35m_decode_graph_destroy(q35m_decode_graph* g) {
    if (!g) return Q35M_OK;
    release_graph(g);
    delete g;
    return Q35M_OK;
}

}  // extern "C"
