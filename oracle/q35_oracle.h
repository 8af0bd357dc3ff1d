/*
 * q35_oracle.h -- CPU restatement of the Qwen35Sharp token-mixer ops.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle: it restates the
 * reference C# algorithms in plain C, in the reference's loop order and fp32
 * arithmetic, so that tests can check the HIP kernels against it and so that
 * bench.py can time it as the CPU baseline.  Nothing in the product library
 * (libq35mix.so) links, loads or calls this code.
 *
 * Every function cites the reference file:line it follows.  Paths are
 * relative to the reference repository root.
 */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers (src/Qwen35Sharp.Model/Qwen35Ops.cs, GatedDeltaNetOps.cs) ---- */
float q35o_silu(float x);
float q35o_softplus(float x);
float q35o_log1p_safe(float x);
float q35o_fast_exp(float x);
void q35o_fast_exp_n(const float* x, float* y, int n);
void q35o_sigmoid(const float* x, float* y, int n);

/* ---- Gated-DeltaNet ops (src/Qwen35Sharp.Model/GatedDeltaNetOps.cs) ---- */
void q35o_causal_conv1d(const float* input, const float* kernel, int kernel_size,
                        int channels, int seq, float* out);
void q35o_causal_conv1d_update(const float* input, const float* kernel, int kernel_size,
                               int channels, float* conv_state, float* out);
void q35o_recurrent_gated_delta_rule(const float* q, const float* k, const float* v,
                                     const float* g, const float* beta, float* state,
                                     int tokens, int n_heads, int head_dim, int v_head_dim,
                                     float eps, float* out, int l2norm_qk);

/* ---- Qwen3.5 norms (src/Qwen35Sharp.Model/Qwen35Ops.cs) ---- */
void q35o_rms_norm_zero_centered(const float* x, const float* weight, float* y,
                                 int rows, int dim, float eps);
void q35o_gated_rms_norm(const float* x, const float* weight, const float* gate, float* y,
                         int rows, int dim, float eps);

/* ---- attention ops (src/Qwen35Sharp.Model/Ops.cs) ---- */
void q35o_rope_table(int cap, int half, float base_freq, float* cos_out, float* sin_out);
void q35o_neox_rope(float* x, int tokens, int heads, int head_dim, int rope_dim,
                    int start_pos, float base_freq);
void q35o_attention_scores(const float* q, const float* cache_k, float* scores, int heads,
                           int kv_heads, int head_dim, int q_len, int kv_len, int q_dim,
                           int kv_stride, float scale, int start_pos, int n_threads);
void q35o_softmax_causal(float* scores, int heads, int q_len, int kv_len, int start_pos,
                         int n_threads);
void q35o_attention_combine(const float* cache_v, const float* scores, float* output,
                            int heads, int kv_heads, int head_dim, int q_len, int kv_len,
                            int q_dim, int kv_stride, int start_pos, int n_threads);

/* ---- mixer glue (src/Qwen35Sharp.Model/Qwen35Model.Decode.cs / .Prefill.cs) ---- */
typedef struct q35o_dims {
    int n_k_heads;   /* SsmGroupCount */
    int n_v_heads;   /* SsmTimeStepRank */
    int head_k_dim;  /* SsmStateSize (used as both dk and dv) */
    int conv_kernel; /* SsmConvKernel */
    int n_heads;     /* NumHeads (full attention) */
    int n_kv_heads;  /* NumKvHeads */
    int head_dim;    /* HeadDim */
    int rope_dim;    /* RopeDim */
    float rope_base; /* RopeBase */
    float eps;       /* Eps */
} q35o_dims;

void q35o_deltanet_decode(const q35o_dims* d, const float* qkv, const float* z,
                          const float* b, const float* a, const float* conv_w,
                          const float* ssm_a, const float* dt_bias, const float* ssm_norm,
                          float* conv_state, float* state, float* out, float* core_out);
void q35o_deltanet_prefill(const q35o_dims* d, int T, const float* qkv, const float* z,
                           const float* b, const float* a, const float* conv_w,
                           const float* ssm_a, const float* dt_bias, const float* ssm_norm,
                           float* conv_state, float* state, float* out, float* core_out);
void q35o_attn_decode(const q35o_dims* d, int start, const float* q_gate, const float* k,
                      const float* v, const float* q_norm, const float* k_norm,
                      float* cache_k, float* cache_v, float* out, int n_threads);
void q35o_attn_prefill(const q35o_dims* d, int start, int T, const float* q_gate,
                       const float* k, const float* v, const float* q_norm,
                       const float* k_norm, float* cache_k, float* cache_v, float* out,
                       int n_threads);

/* Quantized projections (q35_oracle_quant.c). */
float q35o_half_to_float(uint16_t h);
void q35o_q8k_quantize_row(const float* x, void* out, int k);
float q35o_q4k_dot(const void* w, const void* q8, int n);
float q35o_q6k_dot(const void* w, const void* q8, int n);
void q35o_q4k_dequantize_row(const void* w, float* y, int k);
void q35o_q6k_dequantize_row(const void* w, float* y, int k);
void q35o_linear_f32(const float* w, const float* x, float* y, int n_in, int n_out, int tokens);
float q35o_q5k_dot(const void* w, const void* q8, int n);
float q35o_iq4xs_dot(const void* w, const void* q8, int n);
void q35o_q5k_dequantize_row(const void* w, float* y, int k);
void q35o_iq4xs_dequantize_row(const void* w, float* y, int k);
float q35o_q2_0c_dot(const void* w, const void* q8, int n);
float q35o_stq1_0_dot(const void* w, const void* q8, int n);
void q35o_q2_0c_dequantize_row(const void* w, float* y, int k);
void q35o_stq1_0_dequantize_row(const void* w, float* y, int k);
void q35o_linear_q(int type, const void* w, const float* x, float* y, int n_in, int n_out,
                   int tokens);

#ifdef __cplusplus
}
#endif
/* Ops.AddInPlace + Qwen35Ops.RmsNormZeroCentered (q35_oracle_norm.c). */
void q35o_add_rmsnorm(float* hidden, const float* delta, const float* w, float* y, int dim, int rows,
                      float eps);

#endif
