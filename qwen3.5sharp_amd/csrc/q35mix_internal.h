// Internal declarations shared by the host ABI (context.cpp) and the kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/q35mix.h"
#include "snapshot_marks.h"

namespace q35 {

// Dims the kernels are compiled for.
constexpr int kDk = 128;        // DeltaNet key/value head dim (ssm_state_size)
constexpr int kConvK = 4;       // conv taps
constexpr int kConvState = 3;   // conv window length (K - 1)
constexpr int kHd = 256;        // full-attention head dim
constexpr int kRopeDim = 64;    // rotated dims
constexpr int kRopeHalf = 32;
constexpr int kMaxBatch = 64;   // sequences per mixer launch
constexpr int kMaxVPerK = 4;    // DeltaNet v-heads per k-head (chunk prep stages their gates)
// Rows of one (sequence, kv head) the prefill flash kernel can address: its
// K tiles come through a buffer descriptor (32-bit byte offsets, 1 KiB a row).
constexpr int kPrefillMaxRows = 1 << 21;

// Per-launch sequence batch (sequence ids only), passed by value in the
// kernel arguments.  Positions are not in it: kernels read each sequence's
// length from the context's device array, so a captured launch stays valid
// as the lengths move.
struct SeqBatch {
    int n;
    int seq[kMaxBatch];
};

// Conv windows of one (layer, sequence): the reference's [conv_dim][3]
// (oldest first), followed by R - 1 more copies of the windows of the
// 2 * key_dim q/k channels ([R - 1][2 * key_dim][3]), R = v-heads per k-head.
// Decode workgroup (sequence, v-head vh) reads and rewrites copy vh % R of its
// k-head's q/k windows (copy 0 is the one inside the reference block) and its
// own head's value windows, each in place and by no other workgroup, so the
// window update needs no double buffer and no host-held parity.  Every copy
// holds the same values; state I/O reads the reference block and writes all.
struct DeltaNetLayer {
    float* conv_w = nullptr;   // [K][conv_dim]
    float* ssm_a = nullptr;    // [H_v]
    float* dt_bias = nullptr;  // [H_v]
    float* ssm_norm = nullptr; // [dv]
    float* state = nullptr;    // [n_seqs][H_v][dk][dv]
    float* conv = nullptr;     // [n_seqs][win_floats], the layout above
    float* conv_window(int seq, size_t win_floats) const { return conv + (size_t)seq * win_floats; }
    bool has_weights = false;
};

struct AttnLayer {
    float* q_norm = nullptr;   // [head_dim]
    float* k_norm = nullptr;   // [head_dim]
    float* k_cache = nullptr;  // [n_seqs][kv_heads][cap][head_dim], head-major
    float* v_cache = nullptr;  // [n_seqs][kv_heads][cap][head_dim]
    bool has_weights = false;
};

// Kernel ids for the optional per-kernel event timers (the device-side
// counterpart of the reference's Qwen35Model.ProfileEnabled/Ticks* counters,
// Qwen35Model.cs:42-72).
enum KernelId {
    K_DN_DECODE = 0,
    K_DN_CONV_WRITEBACK,
    K_DN_CHUNK_PREP,
    K_DN_CHUNK_SCAN,
    K_DN_CHUNK_OUT,
    K_ATTN_DECODE_PARTIAL1,   // attn_decode_partial<NSUB> by sub-chunks (of 64 rows) per workgroup
    K_ATTN_DECODE_PARTIAL4,
    K_ATTN_DECODE_PARTIAL8,
    K_ATTN_DECODE_MERGE,
    K_ATTN_PREFILL_PREP,
    K_ATTN_PREFILL_FLASH,
    K_Q8K_QUANTIZE,
    K_Q4K_LINEAR,
    K_Q6K_LINEAR,
    K_Q4K_GEMM,
    K_Q6K_GEMM,
    K_ADD_RMSNORM,
    K_Q5K_LINEAR,
    K_IQ4XS_LINEAR,
    K_F32_LINEAR,
    K_Q2_0C_LINEAR,
    K_STQ1_0_LINEAR,
    K_ATTN_DECODE_PARTIAL4R16,   // attn_decode_partial, 4 sub-chunks of 16 rows per workgroup
    K_ATTN_DECODE_PARTIAL8R16,   // attn_decode_partial, up to 8 sub-chunks of 16 rows per workgroup
    K_Q6K_GEMM_BLK,              // block-order Q6_K projection (q35m_set_projection_order)
    K_COUNT
};
const char* kernel_name(int id);

struct Dims {
    int nk, nv;          // DeltaNet k / v heads
    int key_dim, value_dim, conv_dim;
    int nh, nkv;         // attention heads
    int q_dim, kv_dim;
    float eps;
    float rope_base;
    // Floats of one (layer, sequence) conv-window block: the reference window
    // plus nv / nk - 1 copies of the q/k channels' windows.
    size_t win_floats() const { return ((size_t)conv_dim + (size_t)(nv / nk - 1) * 2 * key_dim) * kConvState; }
};

}  // namespace q35

struct q35m_ctx {
    int device = 0;
    int n_cu = 256;                    // compute units of the device
    hipStream_t stream = nullptr;
    q35m_config cfg{};
    q35::Dims d{};
    int n_seqs = 0;
    int cap = 0;                       // KV rows per (layer, seq)
    std::vector<unsigned char> is_recurrent;
    std::vector<q35::DeltaNetLayer> lin;   // indexed by layer (empty for GQA layers)
    std::vector<q35::AttnLayer> full;      // indexed by layer (empty for DeltaNet layers)
    std::vector<int> kv_len;           // per seq (host copy; exact, see dev_len)
    // Per seq: the drops of its length (and rewrites of its rows from 0), which
    // decide whether a linear-state snapshot still matches its K/V rows.
    std::vector<q35::DropMarks> marks;
    // Per-sequence lengths on the device, which the decode attention kernels
    // read (so a captured decode step replays at the current position).  The
    // host changes kv_len and marks the sequence in len_dirty; flush_lengths
    // enqueues one small kernel that writes every marked length before the
    // next launch that reads them.  A decode graph's replay advances both.
    int* dev_len = nullptr;
    std::vector<unsigned char> len_dirty;
    // Bumped whenever the K/V caches or the RoPE table move (q35m_grow): a
    // decode graph captured before holds their old addresses and refuses to run.
    unsigned generation = 0;
    float* rope_cos = nullptr;         // [rope_cap][32]
    float* rope_sin = nullptr;
    int rope_cap = 0;
    float* work = nullptr;             // scratch for split-K partials and prefill
    size_t work_bytes = 0;
    float* noalloc_scratch = nullptr;  // the device's fixed scratch (q35m_attn_decode_noalloc)
    // Largest weight or activation piece (bytes) one tiled-projection launch
    // addresses: 2 GiB (32-bit buffer offsets); the environment variable
    // Q35M_TILE_LIMIT_BYTES, read at create, lowers it (tests use it to make
    // ordinary shapes go in pieces).
    size_t tile_limit = (size_t)1 << 31;
    // Accumulation order of the projections for several tokens
    // (q35m_set_projection_order): Q35M_PROJ_REFERENCE or Q35M_PROJ_BLOCK.
    int proj_order = Q35M_PROJ_REFERENCE;
    std::vector<void*> allocations;
    // Per-kernel event timers (off unless q35m_profile enables them).
    bool profile = false;
    struct EventPair { hipEvent_t a, b; int kid; };
    std::vector<EventPair> pending;
    std::vector<hipEvent_t> event_pool;
    double prof_ms[q35::K_COUNT] = {};
    long prof_n[q35::K_COUNT] = {};
};

namespace q35 {

// Kernel launchers (return hipError_t of the launch).
hipError_t launch_deltanet_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const float* qkv,
                                  const float* z, const float* b, const float* a, float* out);
hipError_t launch_deltanet_prefill(q35m_ctx* c, int layer, int seq, int T, const float* qkv,
                                   const float* z, const float* b, const float* a, float* out);
size_t deltanet_prefill_work_bytes(const Dims& d, int T);
// Split of one decode-attention launch: rows per sub-chunk, sub-chunks per
// workgroup, workgroups (chunks) per head group.  It is chosen from the
// batch size and the longest cached length the launch must cover; the
// kernels take each sequence's actual length from the device, so one plan
// serves every length up to that bound (chunks past a sequence's rows exit).
struct DecodePlan {
    int rows, nsub, nchunks;
};
DecodePlan plan_attn_decode(const q35m_ctx* c, int n, int max_cached);
// Bytes of split-K partials a launch of n sequences under plan p writes.
size_t attn_decode_work_bytes(const q35m_ctx* c, int n, const DecodePlan& p);
// Decode attention: the split-K partials live in `work`, of at least
// attn_decode_work_bytes(c, sb.n, p) bytes.
hipError_t launch_attn_decode(q35m_ctx* c, int layer, const SeqBatch& sb, const DecodePlan& p,
                              const float* q_gate, const float* k, const float* v, float* out, float* work);
// Writes the lengths marked in c->len_dirty to c->dev_len (one small kernel
// per 64 sequences; nothing when none is marked).
hipError_t flush_lengths(q35m_ctx* c);
// dev_len[seq] += k for the sequences of sb, on the context stream.
hipError_t launch_lengths_add(q35m_ctx* c, const SeqBatch& sb, int k);
// Size of the fixed device scratch of q35m_attn_decode_noalloc.
constexpr size_t kNoAllocScratchBytes = Q35M_NOALLOC_SCRATCH_BYTES;
// Device address of that scratch on the current device (call with the device
// current; each device has its own copy).
hipError_t attn_decode_scratch_address(float** ptr);
hipError_t launch_attn_prefill(q35m_ctx* c, int layer, int seq, int start, int T,
                               const float* q_gate, const float* k, const float* v, float* out);
size_t attn_prefill_work_bytes(const Dims& d, int T);
hipError_t launch_linear_q(q35m_ctx* c, int qtype, const void* w, const float* x, float* y,
                           int n_in, int n_out, int tokens);
hipError_t launch_add_rmsnorm(q35m_ctx* c, float* hidden, const float* delta, const float* w, float* y, void* q8,
                              int dim, int tokens, float eps);
size_t linear_q_work_bytes(int n_in, int tokens);
hipError_t launch_linear_f32(q35m_ctx* c, const float* w, const float* x, float* y, int n_in, int n_out,
                             int tokens);
hipError_t launch_q8k_quantize(q35m_ctx* c, const float* x, void* q8, int n_in, int tokens);
hipError_t launch_linear_q_prequant(q35m_ctx* c, int qtype, const void* w, const void* q8, float* y,
                                    int n_in, int n_out, int tokens);

// Ensures ctx->work holds at least `bytes` (synchronises before regrowing).
hipError_t ensure_work(q35m_ctx* c, size_t bytes);

// Event timer bracketing one kernel launch when profiling is on.
// Per-kernel timer: when profiling is on, a and b are bound to the dispatch of
// the kernel launched in the scope (hipExtLaunchKernelGGL start/stop events),
// so they time its execution and not the gaps around it; otherwise both are
// null and the launch is a plain one.
struct ProfScope {
    q35m_ctx* c;
    int kid;
    hipEvent_t a = nullptr, b = nullptr;
    ProfScope(q35m_ctx* ctx, int id);
    ~ProfScope();
};

}  // namespace q35
