/*
 * q35mix.h -- C ABI of libq35mix.so, the MI355X (gfx950) token mixers of
 * Qwen3.5-style hybrid models: the Gated-DeltaNet recurrence and the gated
 * GQA full-attention layer, for decode and prefill.
 *
 * The library is a drop-in for the mixer section of the reference's layer
 * (between the projections and the output projection).  It owns, in HBM, the
 * state the reference keeps in Qwen35Model fields: the DeltaNet recurrent
 * state [H_v][dk][dv] and conv state [conv_dim][K-1] of every linear layer,
 * and the K/V cache of every full-attention layer (the reference's
 * [capacity][kv_heads*head_dim] rows, held head-major on the device), per
 * sequence.  Around the mixers it also offers what the reference runs on
 * either side of them: the projections over every weight type its dispatch
 * knows (Q4_K, Q5_K, Q6_K, IQ4_XS, Q2_0C, STQ1_0 with activations quantized
 * to Q8_K, and F32), the layer boundary (residual add + zero-centred
 * RMSNorm, optionally emitting Q8_K), KV growth, a linear-state snapshot and
 * prefix-reuse planning, a GGUF reader that uploads the mixers' F32 weights,
 * and a whole decode step (every layer's mixer and the length advance)
 * captured once into a HIP graph and replayed per token.  Paths in
 * citations are relative to the reference repository root.
 *
 * Conventions
 *  - Every entry point returns an int status: Q35M_OK (0) or a negative
 *    Q35M_ERR_* code; q35m_last_error() returns a thread-local message.
 *  - Activation pointers (qkv, z, b, a, q_gate, k, v, out) are DEVICE
 *    pointers to fp32, row-major, last index fastest, 16-byte aligned (the
 *    kernels move them as 16-byte vectors; q35m_malloc's buffers are).
 *    Weight setters and state read/write take HOST pointers.
 *  - One context = one device and one HIP stream.  Mixer calls enqueue on
 *    that stream and return; q35m_sync() waits.  A context has no internal
 *    locking (the reference model is single-threaded too); separate contexts
 *    may be driven from separate threads.
 *  - Positions follow the reference: every layer of a forward pass writes
 *    K/V at the sequence's current length, and q35m_advance() moves the
 *    length once per pass (Qwen35Model.cs:235, 287).  The decode kernels
 *    read the lengths from device memory, so a captured decode step (see
 *    q35m_decode_graph_create) stays valid as they move.
 */
#ifndef Q35MIX_H
#define Q35MIX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q35M_OK 0
#define Q35M_ERR_INVALID (-1)     /* bad argument (ArgumentException family)         */
#define Q35M_ERR_UNSUPPORTED (-2) /* dims the kernels are not built for              */
#define Q35M_ERR_CAPACITY (-3)    /* KV capacity or batch limit exceeded             */
#define Q35M_ERR_NO_DEVICE (-4)   /* no usable HIP device                            */
#define Q35M_ERR_HIP (-5)         /* HIP runtime error                               */
#define Q35M_ERR_OOM (-6)         /* device allocation failed                        */
#define Q35M_ERR_RANGE (-7)       /* truncate beyond the current length              */

/* Mixer hyper-parameters: the mixer fields of ModelConfig
 * (src/Qwen35Sharp.Model/ModelConfig.cs:19-54).  The kernels are built for
 * ssm_state_size = 128 (dk = dv), head_dim = 256, rope_dim = 64,
 * ssm_conv_kernel = 4; head counts are free within: num_heads = G *
 * num_kv_heads with G = 1, 2, 4 or a multiple of 8, and ssm_time_step_rank =
 * R * ssm_group_count with R = 1 .. 4. */
typedef struct q35m_config {
    int num_layers;
    int num_heads;          /* full-attention q heads            (16)  */
    int num_kv_heads;       /* full-attention kv heads           (4)   */
    int head_dim;           /* full-attention head dim           (256) */
    int rope_dim;           /* rotated dims per head             (64)  */
    float rope_base;        /* NeoX RoPE base                    (1e7) */
    int ssm_conv_kernel;    /* depthwise conv taps               (4)   */
    int ssm_inner_size;     /* value dim = v_heads * dv          (4096)*/
    int ssm_state_size;     /* dk = dv                           (128) */
    int ssm_time_step_rank; /* DeltaNet v heads                  (32)  */
    int ssm_group_count;    /* DeltaNet k heads                  (16)  */
    float eps;              /* RMS / L2 epsilon                  (1e-6)*/
    int full_attention_interval; /* layer i is GQA iff (i+1) % interval == 0 (4);
                                    ignored when is_recurrent != NULL      */
    const unsigned char* is_recurrent; /* [num_layers] or NULL (ModelConfig.cs:75-103) */
} q35m_config;

typedef struct q35m_ctx q35m_ctx;

/* State kinds for q35m_state_read / q35m_state_write / q35m_state_device_ptr. */
#define Q35M_STATE_RECURRENT 0 /* DeltaNet S [H_v][dk][dv], Qwen35Model.cs:31-32          */
#define Q35M_STATE_CONV 1      /* DeltaNet conv window [conv_dim][K-1], oldest first,
                                  GatedDeltaNetOps.cs:76 (code layout)                    */
#define Q35M_STATE_KEYS 2      /* K cache rows [len][kv_heads*head_dim], post-RoPE/norm */
#define Q35M_STATE_VALUES 3    /* V cache rows [len][kv_heads*head_dim]                 */
/* State read/write move the reference layouts above (K/V: whole rows only).
 * On the device the K and V caches are head-major, [kv_heads][capacity]
 * [head_dim] per (layer, seq), which is what q35m_state_device_ptr exposes. */

/* ---- lifecycle -------------------------------------------------------- */

/* Replaces the state allocation of the Qwen35Model constructor
 * (Qwen35Model.cs:100-136): allocates, zero-filled, the per-(layer, seq)
 * recurrent state, conv state and K/V cache of `kv_capacity` rows for
 * `n_seqs` independent sequences, builds the RoPE table, creates the stream. */
int q35m_create(const q35m_config* cfg, int n_seqs, int kv_capacity, q35m_ctx** out);
int q35m_destroy(q35m_ctx* ctx);
/* Qwen35Model.ResetCache (Qwen35Model.cs:200-212): zero the DeltaNet state
 * and conv state of every linear layer for `seq`, and set its length to 0. */
int q35m_reset(q35m_ctx* ctx, int seq);
/* Qwen35Model.TruncateCache (Qwen35Model.cs:214-222): move the KV length only;
 * refuses to extend (Q35M_ERR_RANGE).  The linear state is not rolled back. */
int q35m_truncate(q35m_ctx* ctx, int seq, int length);
/* `_cacheLen += seq` at the end of Qwen35Model.Forward (Qwen35Model.cs:287). */
int q35m_advance(q35m_ctx* ctx, int seq, int n);
/* KV growth: Qwen35Model.EnsureCache (Qwen35Model.cs:293-353) grows the
 * caches by doubling when a forward pass would pass the capacity; here the
 * caller grows the context to kv_capacity rows (every sequence, every GQA
 * layer; the rows held and the lengths are kept, the RoPE table is extended).
 * Synchronises the stream; a smaller capacity is Q35M_ERR_RANGE. */
int q35m_grow(q35m_ctx* ctx, int kv_capacity);
/* Linear-state snapshot, so a truncation can roll the recurrent state back
 * too (the reference cannot: TruncateCache moves the KV length only,
 * Qwen35Model.cs:214-222).  save copies sequence seq's DeltaNet state and
 * conv window of every linear layer into a device buffer of
 * q35m_snapshot_bytes() bytes and fills info (its length and a stamp of the
 * save); restore copies them back into the same sequence and sets the length
 * to info->kv_len.  K/V rows are not copied: restore needs the rows below
 * that length unchanged since the save, i.e. the sequence never shorter than
 * the snapshot since then, and refuses (Q35M_ERR_RANGE) a snapshot saved
 * before a reset, a truncate or restore to a length below its own, or a K/V
 * state write of that sequence, and one longer than the sequence.  Snapshots
 * at or below every length the sequence was cut to stay restorable, the one
 * just restored included, any number of times.  Copies are asynchronous on
 * the context stream. */
typedef struct q35m_snapshot_info {
    int kv_len;
    unsigned int epoch;   /* stamp of the save in the sequence's history */
} q35m_snapshot_info;
size_t q35m_snapshot_bytes(const q35m_ctx* ctx);
int q35m_snapshot_save(q35m_ctx* ctx, int seq, void* dev, size_t bytes, q35m_snapshot_info* info);
int q35m_snapshot_restore(q35m_ctx* ctx, int seq, const void* dev, size_t bytes,
                          q35m_snapshot_info* info);
/* Q35M_OK when q35m_snapshot_restore would accept the snapshot `info` of
 * sequence seq now, Q35M_ERR_RANGE when it would refuse it.  No device work;
 * a host keeping several snapshots passes only the accepted ones' lengths to
 * q35m_reuse_plan. */
int q35m_snapshot_valid(const q35m_ctx* ctx, int seq, const q35m_snapshot_info* info);
int q35m_kv_len(const q35m_ctx* ctx, int seq, int* length);
/* Prefix reuse: KvCacheAlign.Plan (src/Qwen35Sharp.Model/KvCacheAlign.cs:
 * 20-28, called by Qwen35Model.AlignPrompt, Qwen35Model.cs:224-229).  Keeps the
 * longest common prefix of the token ids the sequence holds (cached) and the
 * new prompt; when the prompt is cached whole, all but its last token, which
 * is forwarded again so the caller gets fresh logits.  *truncate_to is the
 * length to cut the sequence to, *suffix_start the first prompt token to
 * forward (the two are equal).  A truncation moves the KV length only, as in
 * the reference, so it leaves the DeltaNet state of the longer sequence: with
 * n_snaps > 0 the plan covers the linear state too.  snap_lens holds the
 * lengths of the caller's snapshots of the sequence (any order); *snap is the
 * index of the longest one not past the kept prefix, or -1 when there is none
 * (then the caller resets the sequence), and *truncate_to / *suffix_start move
 * back to its length (0 with -1), so restoring that snapshot and forwarding
 * prompt[*suffix_start..] continues from a consistent state (pass only
 * snapshots q35m_snapshot_valid accepts).  With n_snaps = 0,
 * *snap is -1 and the plan is the reference's.  No context, no device work;
 * a negative count or a null pointer for a non-empty array is Q35M_ERR_INVALID. */
int q35m_reuse_plan(const int* cached, int n_cached, const int* prompt, int n_prompt,
                    const int* snap_lens, int n_snaps, int* truncate_to, int* suffix_start, int* snap);

/* ---- weights (host -> HBM once; Qwen35Model.LoadWeights F32 tensors,
 *      Qwen35Model.cs:468-474) --------------------------------------------- */

/* conv_w [K][conv_dim] indexed W[j*conv_dim + c] (GatedDeltaNetOps.cs:48, 82);
 * ssm_a [H_v] already -exp(A_log) (Qwen35Model.Decode.cs:379); dt_bias [H_v];
 * ssm_norm [dv]. */
int q35m_set_deltanet_weights(q35m_ctx* ctx, int layer, const float* conv_w, const float* ssm_a,
                              const float* dt_bias, const float* ssm_norm);
/* q_norm, k_norm [head_dim], applied as (1 + w) (Qwen35Ops.cs:59-63). */
int q35m_set_attn_weights(q35m_ctx* ctx, int layer, const float* q_norm, const float* k_norm);

/* ---- mixers (device pointers; enqueue on the context stream) ---------- */

/* DecodeLinearAttn steps 2-6 (Qwen35Model.Decode.cs:348-397) for n
 * sequences at once (seqs: HOST array of n distinct sequence ids):
 * conv update + SiLU, q/k L2 norm, beta = sigmoid(b),
 * g = ssm_a * softplus(a + dt_bias), one delta-rule step of the state,
 * gated RMSNorm.  qkv [n][conv_dim], z [n][H_v*dv], b, a [n][H_v];
 * out [n][H_v*dv]. */
int q35m_deltanet_decode(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* qkv,
                         const float* z, const float* b, const float* a, float* out);

/* PrefillLinearAttn steps 2-6 (Qwen35Model.Prefill.cs:181-260) for T >= 1
 * tokens of one sequence: zero-padded causal conv (the stored conv window is
 * ignored, GatedDeltaNetOps.cs:45-47), conv-window write-back of the last
 * K-1 raw inputs (Qwen35Model.Prefill.cs:192-204, including its read past
 * the channel row when T < K-1), the delta rule from the current state, and
 * the gated RMSNorm.  qkv [T][conv_dim], z [T][H_v*dv], b, a [T][H_v];
 * out [T][H_v*dv]. */
int q35m_deltanet_prefill(q35m_ctx* ctx, int layer, int seq, int T, const float* qkv,
                          const float* z, const float* b, const float* a, float* out);

/* DecodeAttention steps after the projections (Qwen35Model.Decode.cs:294-323)
 * for n sequences: writes K (RoPE'd, (1+w)-normed) and V at row kv_len(seq),
 * RoPEs and norms q, attends causally over kv_len+1 rows with scale
 * 1/sqrt(head_dim), multiplies by sigmoid(gate).  q_gate [n][heads*2*head_dim]
 * interleaved per head [q_h | gate_h]; k, v [n][kv_heads*head_dim];
 * out [n][heads*head_dim].  Does not advance the length. */
int q35m_attn_decode(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* q_gate,
                     const float* k, const float* v, float* out);

/* The same as q35m_attn_decode, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): it calls no hipMalloc, hipFree or other allocating
 * routine.  No counterpart in the reference.  The split-K partials go to a
 * fixed device array of Q35M_NOALLOC_SCRATCH_BYTES that the library holds
 * on every GPU it runs on until the process ends; a call that would need
 * more is refused with Q35M_ERR_CAPACITY.  The partials take
 * n * num_heads * nchunks * 1032 bytes, nchunks = ceil(longest cached length /
 * 512) once the batch is large enough to split each cache into 8-sub-chunk
 * workgroups (8 sequences at 32K rows: 8.5 MB); smaller batches split into
 * fewer, shorter chunks and stay under about 2 MB.  Every call on one GPU shares that
 * array: calls that overlap on one GPU (other contexts or streams) race.
 * The per-kernel timers are not used by this entry point. */
#define Q35M_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int q35m_attn_decode_noalloc(q35m_ctx* ctx, int layer, int n, const int* seqs, const float* q_gate,
                             const float* k, const float* v, float* out);

/* PrefillAttention steps after the projections (Qwen35Model.Prefill.cs:
 * 113-149) for T tokens of one sequence starting at row kv_len(seq).
 * q_gate [T][heads*2*head_dim]; k, v [T][kv_heads*head_dim];
 * out [T][heads*head_dim].  Does not advance the length.  kv_len(seq) + T
 * may reach 2097152 rows at most (Q35M_ERR_UNSUPPORTED beyond). */
int q35m_attn_prefill(q35m_ctx* ctx, int layer, int seq, int T, const float* q_gate,
                      const float* k, const float* v, float* out);

/* ---- one decode step of every layer, captured once, replayed per token ---- */

/* Per-layer activations of a decode step, device pointers fixed for the life
 * of the graph (each run reads the inputs found there and writes the outputs
 * there).  DeltaNet layers take q35m_deltanet_decode's arguments: in0 = qkv
 * [n][conv_dim], in1 = z [n][H_v*dv], in2 = b [n][H_v], in3 = a [n][H_v],
 * out [n][H_v*dv].  Full-attention layers take q35m_attn_decode's: in0 = q_gate
 * [n][heads*2*head_dim], in1 = k, in2 = v [n][kv_heads*head_dim], in3 unused,
 * out [n][heads*head_dim]. */
typedef struct q35m_decode_io {
    const float* in0;
    const float* in1;
    const float* in2;
    const float* in3;
    float* out;
} q35m_decode_io;

typedef struct q35m_decode_graph q35m_decode_graph;

/* The decode forward of one token for each of n sequences, mixers only
 * (Qwen35Model.Forward, Qwen35Model.cs:231-291): every layer's mixer in layer
 * order, as q35m_deltanet_decode / q35m_attn_decode run them, then every
 * sequence's length advanced by one (`_cacheLen += seq`, :287), captured once
 * into a HIP graph on the context stream (io: [num_layers] entries, seqs: HOST
 * array of n distinct ids).  Replays read the lengths from the device, so one
 * graph serves every token.  The attention split is chosen for lengths up to
 * max_len rows (1 <= max_len <= the KV capacity); a run at which a sequence
 * already holds max_len rows is refused (Q35M_ERR_CAPACITY).  The graph owns
 * its split-K partials (allocated here); runs allocate nothing.  No
 * counterpart in the reference, which has no device to capture for. */
int q35m_decode_graph_create(q35m_ctx* ctx, int n, const int* seqs, const q35m_decode_io* io, int max_len,
                             q35m_decode_graph** out);
/* Enqueues one step on the context stream: replay != 0 launches the captured
 * graph; replay == 0 issues the same kernel launches one by one (identical
 * results; the per-kernel timers see them).  Advances the lengths the host
 * reports (q35m_kv_len) as well.  Refused (Q35M_ERR_RANGE) once q35m_grow has
 * moved the caches: create the graph again. */
int q35m_decode_graph_run(q35m_decode_graph* g, int replay);
/* Waits for the context stream, then frees the graph (before q35m_destroy). */
int q35m_decode_graph_destroy(q35m_decode_graph* g);

/* ---- GGUF weights (GgufFile, src/Qwen35Sharp.Gguf/GgufFile.cs:27-170) ---- */

/* Opens (memory-maps, read-only) and parses a GGUF v2/v3 file: metadata,
 * tensor infos, the data section at general.alignment (default 32, a power of
 * two), as GgufFile does.  Bad magic or layout: Q35M_ERR_INVALID; another
 * version: Q35M_ERR_UNSUPPORTED.  Needs no device. */
typedef struct q35m_gguf q35m_gguf;
int q35m_gguf_open(const char* path, q35m_gguf** out);
int q35m_gguf_close(q35m_gguf* g);
/* A tensor's ggml type, dims (GGUF order, innermost first; unused dims 1),
 * host pointer into the mapping and byte size (0 for a type this reader does
 * not size; F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K and IQ4_XS are sized).
 * Unknown name: Q35M_ERR_RANGE.  Any pointer but g and name may be NULL. */
int q35m_gguf_tensor(const q35m_gguf* g, const char* name, int* type, int64_t dims[4], int* n_dims,
                     const void** data, size_t* bytes);
/* Metadata values (GgufFile.GetInt32/GetUint32, GetFloat32, GetString);
 * strings stay valid until q35m_gguf_close.  Missing key: Q35M_ERR_RANGE. */
int q35m_gguf_int(const q35m_gguf* g, const char* key, int64_t* value);
int q35m_gguf_float(const q35m_gguf* g, const char* key, double* value);
int q35m_gguf_string(const q35m_gguf* g, const char* key, const char** value);
/* The F32 branch of Qwen35Model.LoadWeights (Qwen35Model.cs:463-474) for the
 * token mixers: per layer, blk.N.ssm_conv1d.weight [4][conv_dim],
 * blk.N.ssm_a, blk.N.ssm_dt.bias [n_v_heads], blk.N.ssm_norm.weight
 * [v_head_dim] (linear layers) or blk.N.attn_q_norm.weight,
 * blk.N.attn_k_norm.weight [head_dim] (GQA layers), uploaded with
 * q35m_set_deltanet_weights / q35m_set_attn_weights.  A missing tensor is
 * Q35M_ERR_RANGE, a non-F32 one Q35M_ERR_UNSUPPORTED, a wrong size
 * Q35M_ERR_INVALID.  num_layers, is_recurrent and the dims must be the
 * context's (Q35M_ERR_INVALID otherwise). */
int q35m_load_mixer_weights(q35m_ctx* ctx, const q35m_gguf* g, int num_layers, const unsigned char* is_recurrent,
                            int conv_dim, int n_v_heads, int v_head_dim, int head_dim);

/* ---- state I/O in the reference layouts (snapshot / restore / parity) -- */

int q35m_state_read(q35m_ctx* ctx, int layer, int seq, int kind, void* host, size_t bytes);
int q35m_state_write(q35m_ctx* ctx, int layer, int seq, int kind, const void* host,
                     size_t bytes);
/* Device address and size of one state buffer, for zero-copy callers.  For
 * Q35M_STATE_CONV it is the window in the reference layout; the decode also
 * keeps one more copy of the q/k channels' windows per further v-head of a
 * k-head (after that block), so write windows with q35m_state_write, which
 * updates every copy, rather than through this address. */
int q35m_state_device_ptr(q35m_ctx* ctx, int layer, int seq, int kind, void** dptr,
                          size_t* bytes);

/* ---- stream, staging memory, errors ----------------------------------- */

int q35m_sync(q35m_ctx* ctx);
/* The context's hipStream_t, for event timing and ordering by the caller. */
void* q35m_stream(q35m_ctx* ctx);
int q35m_device_count(int* count);

/* Quantized projections: y[t][n_out] = W x[t] for t < tokens, W given as
 * GGUF rows of n_in/256 blocks in device memory, Q4_K (144 B a block) or
 * Q6_K (210 B), x and y fp32 row-major [tokens][n_in] / [tokens][n_out] in
 * device memory.  Each token row is quantized to Q8_K first, as the reference
 * does.  Replaces Qwen35Model.DecodeLinear / Linear
 * (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:22-88) over MulMatQ4K.Gemv
 * (src/Qwen35Sharp.Kernels/MulMatQ4K.cs:12-43) and Q6K.Gemv / Q6K.Gemm
 * (src/Qwen35Sharp.Kernels/Q6K.cs:301-353): results are bit-identical to the
 * reference's AVX2 GEMV, and for Q4_K with tokens > 1 to its packed panel
 * GEMM (MulMatQ4K.Gemm, MulMatQ4K.cs:45-127 -> GemmQ4K.GemmAvx2Tile,
 * GemmQ4K.Avx2.cs:39-207) for the first n_out & ~7 outputs and the GEMV for
 * the rest, as the reference splits them.  w and x must be 16-byte aligned;
 * n_in a multiple of 256 up to 16384. */
int q35m_linear_q4k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens);
int q35m_linear_q6k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens);
/* The same for Q5_K (176 B a block) and IQ4_XS (136 B) weights: Q5K.Gemv /
 * Q5K.Gemm (src/Qwen35Sharp.Kernels/Q5K.cs:97-117) and IQ4XS.Gemv /
 * IQ4XS.Gemm (src/Qwen35Sharp.Kernels/IQ4XS.cs:75-104), whose scalar dot
 * products (Q5K.Dot, Q5K.cs:45-95; IQ4XS.Dot, IQ4XS.cs:49-73) run per token;
 * results are bit-identical to them. */
int q35m_linear_q5k(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                    int tokens);
int q35m_linear_iq4xs(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                      int tokens);
/* The same for Q2_0C (130 B a block of 512 values; n_in a multiple of 512)
 * and STQ1_0 (42 B a block of 256) weights: MulMatQ2.Gemv / Gemm
 * (src/Qwen35Sharp.Kernels/MulMatQ2.cs:19-99) and MulMatSTQ.Gemv / Gemm
 * (src/Qwen35Sharp.Kernels/MulMatSTQ.cs:19-150), as Qwen35Model.Linear /
 * DecodeLinear dispatch them (Qwen35Model.Decode.cs:31-36, 65-70).  Each
 * output is bit-identical to the reference's path for it: the eight-row
 * panel kernels (Q2Panel.cs, STQPanel.cs; the panels exist for the first
 * n_out & ~7 rows) or the raw-row dot (Q2_0C.DotAvx2, STQ1_0.DotAvx2) for
 * the rest; STQ1_0 with tokens > 1 takes the panels for all rows when
 * tokens % 4 == 0 and n_out % 8 == 0 and the raw dot for all rows
 * otherwise, as MulMatSTQ.Gemm does. */
int q35m_linear_q2_0c(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                      int tokens);
int q35m_linear_stq1_0(q35m_ctx* ctx, const void* w, const float* x, float* y, int n_in, int n_out,
                       int tokens);
/* F32 weights W [n_out][n_in] row-major in device memory (Qwen35Model.F32Gemm,
 * src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:129-140, the reference's Linear
 * and DecodeLinear for F32 tensors): y[t][o] = Ops.DotF32(x[t], W[o])
 * (Ops.cs:418-449), bit-identical to it; any n_in >= 1. */
int q35m_linear_f32(q35m_ctx* ctx, const float* w, const float* x, float* y, int n_in, int n_out,
                    int tokens);

/* Accumulation order of the quantized projections for several tokens.
 * Q35M_PROJ_REFERENCE (the default): the reference's fp32 order, bit for bit
 * (see above).  Q35M_PROJ_BLOCK: for Q6_K with tokens >= 16 (and n_out * n_in
 * / 256 even), the exact integer sum of each 256-value block (scale * (v -
 * 32) * q8 over all its sub-blocks, in int32) times its fp32 scales, once per
 * block: the reference's integer part exactly, its 8 per-lane fp32 chains
 * regrouped, so results agree with it within fp32 rounding of the exact value
 * rather than bit for bit (about 2x faster at 2048 tokens).  Other formats,
 * one token and the other Q6_K shapes keep the reference's order.  No
 * counterpart in the reference (it has one order per path). */
#define Q35M_PROJ_REFERENCE 0
#define Q35M_PROJ_BLOCK 1
int q35m_set_projection_order(q35m_ctx* ctx, int order);

/* The layer boundary around a mixer: hidden[t] += delta[t] (fp32 adds,
 * written back; delta NULL: no add), then y[t] = RmsNormZeroCentered(hidden[t],
 * weight) = (h * scale) * (1 + weight) with scale = 1 / sqrt(mean(h^2) + eps),
 * the sum of squares in the reference's order (8 FMA lanes, horizontal sum,
 * dim % 8 tail) (weight NULL: 0).  When q8 is non-NULL y is also written as
 * Q8_K blocks (q35m_q8k_bytes(dim, tokens) bytes, as q35m_quantize_q8k writes
 * them) for the projection that follows; y may then be NULL.  All rows
 * [tokens][dim] fp32 in device memory, buffers 16-byte aligned; dim a multiple
 * of 4 up to 16384 (of 256 with q8).  Replaces Ops.AddInPlace
 * (src/Qwen35Sharp.Model/Ops.cs:677-710) followed by
 * Qwen35Ops.RmsNormZeroCentered (src/Qwen35Sharp.Model/Qwen35Ops.cs:22-64), as
 * Qwen35Model.DecodeBlock uses them (Qwen35Model.Decode.cs:226-235: attn_norm
 * with delta NULL, then the residual add and post_attention_norm); results
 * are bit-identical to the reference's. */
int q35m_add_rmsnorm(q35m_ctx* ctx, float* hidden, const float* delta, const float* weight, float* y, void* q8,
                     int dim, int tokens, float eps);

/* The same in two steps, for several projections of one activation:
 * q35m_quantize_q8k writes the Q8_K blocks of x [tokens][n_in] into a device
 * buffer of q35m_q8k_bytes(n_in, tokens) bytes (a BlockQ8K's fields in
 * 304 bytes: f32 d, 12 unused bytes, i8 qs[256], i16 bsums[16]), and the
 * _prequant entry points read them.  Replaces
 * Q8K.QuantizeRow (src/Qwen35Sharp.Kernels/Q8K.cs:12-78) followed by
 * Qwen35Model.GemvPrequant (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs:
 * 89-112), as the reference's attention decode uses them
 * (Qwen35Model.Decode.cs:286-292).  x, q8 and w must be 16-byte aligned. */
size_t q35m_q8k_bytes(int n_in, int tokens);
int q35m_quantize_q8k(q35m_ctx* ctx, const float* x, void* q8, int n_in, int tokens);
int q35m_linear_q4k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens);
int q35m_linear_q6k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens);
int q35m_linear_q5k_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                             int n_out, int tokens);
int q35m_linear_iq4xs_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                               int n_out, int tokens);
int q35m_linear_q2_0c_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                               int n_out, int tokens);
int q35m_linear_stq1_0_prequant(q35m_ctx* ctx, const void* w, const void* q8, float* y, int n_in,
                                int n_out, int tokens);

/* Per-kernel HIP event timers, the device-side counterpart of the
 * reference's Qwen35Model.ProfileEnabled / Ticks* counters
 * (Qwen35Model.cs:42-72).  q35m_profile(ctx, 1) zeroes the totals and times
 * every following kernel launch on the context stream with events recorded
 * around it; q35m_profile_read synchronises and returns the total
 * milliseconds and launch count of kernel id `kernel`; kernel ids run from 0
 * up to the first id for which q35m_profile_kernel_name returns NULL.
 * Timing adds event records between launches: leave it off when measuring
 * throughput. */
int q35m_profile(q35m_ctx* ctx, int enable);
int q35m_profile_read(q35m_ctx* ctx, int kernel, double* total_ms, long* launches);
const char* q35m_profile_kernel_name(int kernel);
int q35m_malloc(void** dptr, size_t bytes);
int q35m_free(void* dptr);
int q35m_copy_h2d(q35m_ctx* ctx, void* dst, const void* src, size_t bytes);
int q35m_copy_d2h(q35m_ctx* ctx, void* dst, const void* src, size_t bytes);
const char* q35m_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
