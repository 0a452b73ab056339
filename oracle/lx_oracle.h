/*
 * lx_oracle.h — CPU oracle for the DiT / Qwen2 fused-op path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * algorithms (Larynx src/flow/ and src/llm/ sources, with the PyTorch
 * semantics of tests/flow_reference.py), used as the test oracle for the HIP
 * library and, in bench.py, as the timed CPU baseline.  It is never linked
 * into or called by the product path (larynx_amd/liblxops.so).
 *
 * Numerics: tensors are stored fp32 between ops (as in the reference), every
 * reduction and transcendental is evaluated in fp64.  Two quantities are
 * deliberately rounded to fp32 the way the reference forms them, because
 * their rounding is part of the reference's result at long sequence length:
 *   - rotary angles: fp32(pos) * fp32 inv_freq, rounded to fp32
 *     (flow_reference.py:79, 96; the HF Qwen2 rotary does the same);
 *   - sinusoid angles: (1000 * t) * expf(-j * fp32(ln(1e4)/127)), in fp32
 *     (src/flow/flow_matching.cpp:14-17).
 * All tensors are host pointers, row-major in the PyTorch sense.
 */
#ifndef LX_ORACLE_H
#define LX_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

#include <stdint.h>

void orc_set_threads(int n);
int orc_get_threads(void);

/* Deterministic synthetic data: n values ~ N(0, std^2) for (seed, stream). */
void orc_fill_normal(float* out, long n, uint64_t seed, uint64_t stream, float std);

/* ---- per-op --------------------------------------------------------- */
void orc_adaln(const float* x, const float* shift, const float* scale, long mod_stride, float* y,
               int B, int T, int D, float eps);
void orc_linear(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
                int M, int N, int K);
void orc_silu_vec(const float* x, float* y, long n);
void orc_gelu_tanh(const float* h, float* y, long n);
void orc_gated_residual(float* x, const float* y, const float* gate, long gate_stride, int B,
                        int T, int D);
void orc_rope_inv_freq(float base, int dim, float* out);
void orc_rope_partial(float* q, const int* pos, int B, int T, int ld, int rot_dim, float base);
void orc_timestep_embed(const float* t, int B, int half_dim, float scale, float* out);
void orc_time_mlp(const float* t, int B, const float* w0, const float* b0, const float* w2,
                  const float* b2, int D, float* out);
void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int D, float eps);
void orc_rope_neox(float* qk, const int* pos, int rows, int n_heads, int head_dim, int ld,
                   float theta);
void orc_swiglu(const float* gate, const float* up, float* out, long n);
int orc_embed_gather(const float* table, long n_rows, int D, const int* ids, int n, float* out);
void orc_attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv,
                   float* o, int ldo, int B, int Tq, int Tk, int n_heads, int n_kv_heads,
                   int head_dim, float scale, int causal, int q_offset);
void orc_conv_pos_mish(const float* x, const float* w, const float* bias, const float* resid,
                       float* y, int B, int T, int C, int G, int K);

/* ---- DiT estimator / CFM --------------------------------------------- */
typedef struct orc_dit_block {
  const float *attn_norm_w, *attn_norm_b, *to_q_w, *to_q_b, *to_k_w, *to_k_b, *to_v_w, *to_v_b,
      *to_out_w, *to_out_b, *ff0_w, *ff0_b, *ff2_w, *ff2_b;
} orc_dit_block;

typedef struct orc_dit {
  int dim, depth, heads, head_dim, ff_inner, mel_dim;
  const float *time_mlp_0_w, *time_mlp_0_b, *time_mlp_2_w, *time_mlp_2_b;
  const float *input_proj_w, *input_proj_b;
  const float *conv_pos_1_w, *conv_pos_1_b, *conv_pos_2_w, *conv_pos_2_b;
  const orc_dit_block* blocks;
  const float *norm_out_w, *norm_out_b, *proj_out_w, *proj_out_b;
} orc_dit;

/* Captures (any may be NULL): time_embed (B,D); input_proj, conv_pos,
 * input_embed, norm_out (B,T,D); blocks (depth,B,T,D). */
typedef struct orc_dit_capture {
  float *time_embed, *input_proj, *conv_pos, *input_embed, *blocks, *norm_out;
} orc_dit_capture;

/* DiT.forward: x, mu, cond (B, mel, T); spks (B, mel); t (B); dphi (B, mel, T). */
int orc_dit_forward(const orc_dit* w, int B, int T, const float* x, const float* mu,
                    const float* cond, const float* spks, const float* t, float* dphi,
                    const orc_dit_capture* cap);
/* One CFM Euler step on x (mel, T), CFG pair built inside. */
int orc_cfm_step(const orc_dit* w, int T, float* x, const float* mu, const float* cond,
                 const float* spks, float t, float dt, float cfg_rate);
/* CausalConditionalCFM.solve_euler with the cosine t_span. */
int orc_cfm_solve(const orc_dit* w, int T, float* x, const float* mu, const float* cond,
                  const float* spks, int n_steps, float cfg_rate);

/* ---- Flow frontend (FlowDecoder::infer before the CFM solve) ---------------- */
typedef struct orc_flow_front {
  int vocab, spk_in, mel, channels;
  const float *input_embedding;           /* (vocab, mel)            */
  const float *spk_affine_w, *spk_affine_b; /* (mel, spk_in), (mel)   */
  const float *pre_conv1_w, *pre_conv1_b;   /* (channels, mel, 4)     */
  const float *pre_conv2_w, *pre_conv2_b;   /* (mel, channels, 3)     */
} orc_flow_front;

/* ids: Tseq clamped token ids (prompt then tokens); prompt_feat (mel_len1, mel);
 * spk_embedding (spk_in).  Outputs (any may be NULL except mu/cond/spk):
 * spk (mel), token_embed (Tseq, mel), pre (Tseq, mel), mu (mel, 2 Tseq),
 * cond (mel, 2 Tseq).  Returns 0, or -3 for an id outside the table. */
int orc_flow_frontend(const orc_flow_front* w, const int* ids, int Tseq, const float* prompt_feat,
                      int mel_len1, const float* spk_embedding, float* spk, float* token_embed,
                      float* pre, float* mu, float* cond);

/* ---- Qwen2 -------------------------------------------------------------- */
typedef struct orc_qwen2_layer {
  const float *q_w, *q_b, *k_w, *k_b, *v_w, *v_b, *o_w, *gate_w, *up_w, *down_w, *in_norm,
      *post_norm;
} orc_qwen2_layer;

typedef struct orc_qwen2 {
  int hidden, intermediate, n_heads, n_kv_heads, head_dim, n_layers, text_vocab, speech_vocab;
  float rms_eps, rope_theta;
  const float *embed_tokens, *speech_embedding, *final_norm, *llm_decoder;
  const orc_qwen2_layer* layers;
} orc_qwen2;

/* LLM::build_lm_input; returns L or a negative error (-3 bad id). */
int orc_qwen2_build_lm_input(const orc_qwen2* w, const int* text, int n_text, const int* speech,
                             int n_speech, float* out);
/* Runs L new rows at positions [past, past+L) against a host KV cache of
 * capacity cap rows per layer (k_cache/v_cache: n_layers x cap x KV), appending
 * the new keys/values.  x: (L, H) in, logits (L, speech_vocab) out (may be
 * NULL), hidden (n_layers, L, H) and final_norm (L, H) captures may be NULL. */
int orc_qwen2_forward(const orc_qwen2* w, const float* x_in, int L, int past, float* k_cache,
                      float* v_cache, int cap, float* logits, float* hidden, float* final_norm);

#ifdef __cplusplus
}
#endif

#endif
