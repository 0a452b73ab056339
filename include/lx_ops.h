/*
 * lx_ops.h — C-ABI of the MI355X (gfx950) op library `liblxops.so`.
 *
 * Every entry point replaces one group of ggml graph nodes on the hot path of
 * Larynx's CosyVoice3 Flow DiT estimator and Qwen2 LM. The citation on each
 * declaration names the reference node(s) it stands in for (paths relative to
 * the Larynx source tree).
 *
 * Conventions (shared by every function):
 *   - All tensor pointers are DEVICE pointers (hipMalloc'd or torch CUDA
 *     tensors), fp32, contiguous row-major in the PyTorch sense.  A PyTorch
 *     (B, T, C) tensor is byte-identical to ggml's [C, T, B] ("Space B" of the
 *     reference, docs/FLOW.md §2).  Exceptions are marked HOST.
 *   - Return value: LX_OK (0) on success, a negative LX_ERR_* code otherwise.
 *     Bad arguments are rejected before any work is enqueued.  Errors are never
 *     silently clamped: a bad token id is an error, not a zero row.
 *   - Work is enqueued on `stream` (0 = the default stream); no call
 *     synchronises unless documented.  No per-op call allocates device memory;
 *     the composite objects (lx_dit, lx_qwen2) allocate at create time only.
 *   - Reentrant per stream: calls on different streams touching disjoint
 *     buffers may overlap.
 */
#ifndef LX_OPS_H
#define LX_OPS_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LX_OK = 0,
  LX_ERR_ARG = -1,     /* null pointer, bad shape, unsupported size */
  LX_ERR_LAUNCH = -2,  /* hipLaunch / hipGetLastError failure */
  LX_ERR_RANGE = -3,   /* token id outside its embedding table */
  LX_ERR_ALLOC = -4,   /* device allocation failed (create calls only) */
  LX_ERR_STATE = -5    /* call out of order (e.g. decode before prefill) */
};

/* Library identity: returns a static string naming the build and target. */
const char* lx_version(void);
/* Last error string of the calling thread (static storage, never NULL). */
const char* lx_last_error(void);

/* ------------------------------------------------------------------------ */
/* Flow DiT fused row / pointwise ops                                        */
/* ------------------------------------------------------------------------ */

/* a1/a2 — AdaLayerNorm modulation:
 *   y[b,t,:] = LN_eps(x[b,t,:]) * (1 + scale[b,:]) + shift[b,:]
 * LN: biased variance, no affine.  x, y: (B, T, D).  shift/scale rows are
 * `mod_stride` floats apart, so they may point straight into the chunked AdaLN
 * embedding (B, 6*D) with mod_stride = 6*D (no chunk copies); mod_stride 0
 * gives every batch row the same shift/scale.  y may alias x.
 * Replaces ada_ln (src/flow/ops.cpp:94-104: ggml_norm + add(scale,1) + mul +
 * add) and the view_chunk conts (src/flow/dit.cpp:26-31, 57-62, 134-135).
 * D % 4 == 0, D <= 4096. */
int lx_adaln_modulate_f32(const float* x, const float* shift, const float* scale,
                          long mod_stride, float* y, int B, int T, int D, float eps,
                          hipStream_t stream);

/* The gated residual of a projection computed as `splits` K slices, folded into
 * the next modulated LayerNorm (one pass over the row):
 *   h = h + gate_b * ((partials[0] + ... + partials[splits-1]) + bias)
 *   y = LayerNorm_eps(h) * (1 + scale_b) + shift_b        (when y != NULL)
 * h: (B, T, D) updated in place; partials: `splits` (<= 4) slices of (B*T, D),
 * partial_stride floats apart, summed in slice order (splits 0: h is only
 * normalised); bias (D) or NULL; gate / shift / scale: per-batch rows as in
 * lx_gated_residual_f32 / lx_adaln_modulate_f32.  All pointers 16-byte aligned.
 * Replaces the gated residual x + gate * (to_out / ff output) of
 * src/flow/dit.cpp:71,77 plus the next ada_ln (src/flow/ops.cpp:94-104). */
int lx_adaln_resid_f32(float* h, const float* partials, int splits, long partial_stride,
                       const float* bias, const float* gate, long gate_stride,
                       const float* shift, const float* scale, long mod_stride, float* y,
                       int B, int T, int D, float eps, hipStream_t stream);
/* The same with y written as two-part packed rows (lx_linear_bx's a_packed
 * operand; bit-identical products to the fp32 y it packs): how the estimator
 * feeds its three-product QKV and FF0 projections.  No counterpart in the
 * reference (its activations stay fp32). */
int lx_adaln_resid_packed_f32(float* h, const float* partials, int splits, long partial_stride,
                              const float* bias, const float* gate, long gate_stride,
                              const float* shift, const float* scale, long mod_stride, void* y,
                              int B, int T, int D, float eps, hipStream_t stream);

/* AdaLN modulation embedding (GEMV over the batch rows):
 *   emb[b, :] = W @ silu(c[b, :]) + bias,   W: (n_out, D) row-major.
 * Replaces linear(attn_norm_w, attn_norm_b, ggml_silu(t)) (src/flow/dit.cpp:56)
 * and the norm_out linear (src/flow/dit.cpp:133).  B <= 16, B * D * 4 <= 64 KiB. */
int lx_adaln_emb_f32(const float* c, const float* W, const float* bias, float* emb,
                     int B, int D, int n_out, hipStream_t stream);

/* a3 — partial interleaved (GPT-J) rotary, in place on q and k (k may be NULL):
 * for channels c < rot_dim, pairs (2i, 2i+1) of every row (b, t) rotate by
 * angle = fp32(pos[t]) * inv_freq[i], inv_freq[i] = 1/base^(2i/rot_dim) in fp32.
 * Channels >= rot_dim are untouched.  q, k: (B, T, ld) with the row stride `ld`
 * in floats; pos: device int32[T].
 * Replaces rope_partial (src/flow/ops.cpp:85-92: permute + ggml_rope_ext
 * NORMAL n_dims=64 base 1e4 + permute + cont).  rot_dim even, <= 128. */
int lx_rope_partial_interleaved_f32(float* q, float* k, const int* pos, int B, int T,
                                    int ld, int rot_dim, float base, hipStream_t stream);

/* a4 — tanh-GELU: y = 0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3))).
 * y may alias h.  Replaces gelu_tanh (src/flow/ops.cpp:73-83, 9 ggml nodes). */
int lx_gelu_tanh_f32(const float* h, float* y, long n, hipStream_t stream);

/* a5 — gated residual, in place: x[b,t,:] += gate[b,:] * y[b,t,:].
 * gate rows are `gate_stride` floats apart (may point into the AdaLN emb; 0:
 * one gate row for every batch row).
 * Replaces ggml_add(x, ggml_mul(y, gate)) (src/flow/dit.cpp:71, 77). */
int lx_gated_residual_f32(float* x, const float* y, const float* gate, long gate_stride,
                          int B, int T, int D, hipStream_t stream);

/* a6 — sinusoidal timestep embedding:
 *   out[b, j]          = sin(scale * t[b] * e^(-j ln(1e4)/(half_dim-1)))
 *   out[b, half_dim+j] = cos(...),                 j < half_dim.
 * t: device float[B]; out: (B, 2*half_dim).  Replaces the sinusoid half of
 * time_embed_host (src/flow/flow_matching.cpp:13-20). */
int lx_timestep_embed_f32(const float* t, int B, int half_dim, float scale, float* out,
                          hipStream_t stream);

/* a6 — full TimestepEmbedding: sinusoid(256, scale 1000) -> Linear(256->D) ->
 * SiLU -> Linear(D->D).  w0: (D, 256), w2: (D, D).  work: device scratch of at
 * least B*(256 + D) floats.  B <= 16, B * D * 4 <= 64 KiB.  Replaces
 * time_embed_host (src/flow/flow_matching.cpp:10-42) on the device. */
int lx_time_mlp_f32(const float* t, int B, const float* w0, const float* b0,
                    const float* w2, const float* b2, int D, float* work, float* out,
                    hipStream_t stream);

/* lx_time_mlp_f32 without the workspace argument: the hidden layer lives in a
 * library-owned device array (64 KiB per device, held until the process ends),
 * so the call allocates nothing and needs no caller memory beyond t, the
 * weights and out.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops).
 * B * D <= 16384, else LX_ERR_ARG.  All calls on one device share the array:
 * calls that overlap on one device (e.g. on two streams) race. */
int lx_time_mlp_f32_noalloc(const float* t, int B, const float* w0, const float* b0,
                            const float* w2, const float* b2, int D, float* out,
                            hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Qwen2 fused ops                                                           */
/* ------------------------------------------------------------------------ */

/* a10 — RMSNorm: y = x / sqrt(mean(x^2) + eps) * w.  x, y: (rows, D).
 * Replaces rms_norm (src/llm/ops.cpp:7-11: ggml_rms_norm + mul). */
int lx_rmsnorm_f32(const float* x, const float* w, float* y, int rows, int D, float eps,
                   hipStream_t stream);

/* a11 — NEOX rotary, in place: row r holds n_heads heads of head_dim; within a
 * head pairs (i, i + head_dim/2) rotate by fp32(pos[r]) * theta^(-2i/head_dim).
 * qk: (rows, ld) floats with the heads packed from column 0; pos: device
 * int32[rows].  Replaces rope_full (src/llm/ops.cpp:21-30, GGML_ROPE_TYPE_NEOX). */
int lx_rope_neox_f32(float* qk, const int* pos, int rows, int n_heads, int head_dim,
                     int ld, float theta, hipStream_t stream);

/* a12 — SwiGLU gate: out = silu(gate) * up, elementwise over n.
 * Replaces ggml_mul(ggml_silu(gate), up) (src/llm/llm.cpp:167-169, 285-287). */
int lx_swiglu_f32(const float* gate, const float* up, float* out, long n,
                  hipStream_t stream);

/* a13 — embedding gather: out[i, :] = table[ids[i], :], bit-exact copy.
 * ids is a HOST int32 array (the reference holds token ids on the host); every
 * id is checked against [0, n_rows) before any work is enqueued and a bad id
 * returns LX_ERR_RANGE with nothing written.  table: (n_rows, D); out: (n, D).
 * Replaces the per-row ggml_backend_tensor_get copies of build_lm_input
 * (src/llm/llm.cpp:63-100), decode (src/llm/llm.cpp:226-230) and the flow
 * token ggml_get_rows (src/flow/flow.cpp:150-151). */
int lx_embed_gather_f32(const float* table, long n_rows, int D, const int* ids, int n,
                        float* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Dense parts (MFMA fp32)                                                   */
/* ------------------------------------------------------------------------ */

/* Epilogues fused into the projection GEMM  acc = x @ W^T (+ bias). */
enum {
  LX_EPI_NONE = 0,          /* y = acc + bias                                   */
  LX_EPI_GELU_TANH = 1,     /* y = gelu_tanh(acc + bias)                        */
  LX_EPI_GATED_RESID = 2,   /* y[m,:] += gate[m / rows_per_batch, :] * (acc+bias) */
  LX_EPI_ROPE_PARTIAL = 3,  /* y = acc + bias, then partial interleaved rotary on
                               columns c with (c % rope_section) < rot_dim and
                               c < rope_sections * rope_section; position of row
                               m is pos[m % rows_per_batch]                       */
  LX_EPI_RESID = 4,         /* y[m,:] += acc (+ bias)                           */
  LX_EPI_SWIGLU_PAIRED = 5  /* W rows interleave gate/up: y[m, j] =
                               silu(acc[2j]) * acc[2j+1]; y has N/2 columns      */
};

typedef struct lx_epilogue {
  int kind;                 /* LX_EPI_* */
  int rows_per_batch;       /* T: row m belongs to batch m / T (GATED_RESID, ROPE) */
  const float* gate;        /* GATED_RESID: gate rows, gate_stride floats apart  */
  long gate_stride;
  const int* pos;           /* ROPE_PARTIAL: device int32[rows_per_batch]        */
  int rot_dim;              /* ROPE_PARTIAL: rotated channels per section (even) */
  int rope_section;         /* ROPE_PARTIAL: columns per rotated section         */
  int rope_sections;        /* ROPE_PARTIAL: number of leading sections rotated  */
  float rope_base;          /* ROPE_PARTIAL: frequency base                      */
} lx_epilogue;

/* Linear: y = epi(x @ W^T + bias).  x: (M, K) with row stride ldx; W: (N, K)
 * row-major (torch nn.Linear weight == ggml [K, N]); bias: (N) or NULL;
 * y: (M, N) with row stride ldy (N/2 columns for SWIGLU_PAIRED).  K and ldx
 * multiples of 4, x and W 16-byte aligned; y needs no alignment (aligned
 * outputs take the float4 epilogue).
 * Replaces linear() = ggml_mul_mat + ggml_add (src/flow/ops.cpp:20-26,
 * src/llm/ops.cpp:13-19) plus whatever node the epilogue absorbs.
 * epi may be NULL (== LX_EPI_NONE). */
int lx_linear_f32(const float* x, int ldx, const float* W, const float* bias, float* y,
                  int ldy, int M, int N, int K, const lx_epilogue* epi,
                  hipStream_t stream);

/* Split-operand linear, fp32 arithmetic on the bf16 matrix cores: every
 * operand is split into three bf16 parts (w = w0 + w1 + w2, exact for normal
 * values) and each product is formed from the six parts a_i * w_j with
 * i + j <= 2, accumulated in fp32 (error at the fp32 level, about 1e-6 of the
 * result's magnitude).  lx_split_planes_f32 writes the planes of an (N, K)
 * weight once (3 * N * K bf16: plane p at p * N * K; n = N * K, a multiple of
 * 4); lx_linear_split_f32 then computes y = epi(x @ W^T + bias) from them, as
 * lx_linear_f32 does from W.  tile 0: 128 x 128 output tiles (N a multiple of
 * 128), tile 1: 128 x 64 (N a multiple of 64); K a multiple of 32, ldx of 4;
 * x, planes, y, bias and the gate 16-byte aligned.  Replaces the same
 * linear() = ggml_mul_mat + ggml_add (src/flow/ops.cpp:20-26) as
 * lx_linear_f32; the planes have no counterpart in the reference (its weights
 * stay fp32), they are what the estimator keeps for its projections. */
int lx_split_planes_f32(const float* W, void* planes, long n, hipStream_t stream);
int lx_linear_split_f32(const float* x, int ldx, const void* planes, const float* bias,
                        float* y, int ldy, int M, int N, int K, const lx_epilogue* epi,
                        int tile, hipStream_t stream);

/* Split-operand linear with the weight in MFMA fragment order: the same fp32
 * arithmetic on the bf16 matrix cores as lx_linear_split_f32 (three-part
 * operand splits, six products, fp32 accumulation), in the layout the
 * estimator runs its projections in.  lx_wfrag_pack_f32 writes an (N, K)
 * weight once in fragment order (3 * N * K bf16; N a multiple of 32, K of 16).
 * A is fp32 (M, K) with row stride lda.  Outputs:
 *   LX_BX_OUT_F32      Y = epi(A @ W^T + bias) (row stride ldy), every
 *                      lx_epilogue kind (SWIGLU_PAIRED: N / 2 columns);
 *   LX_BX_OUT_PARTIAL  the raw products of `slices` K slices, slice s into
 *                      Y + s * slice_stride (no bias, no epilogue): the
 *                      consumer sums the slices in slice order.  Each slice
 *                      spans ceil(K / 64 / slices) 64-wide steps, the last
 *                      the remainder, which must not be empty.
 * Tiles of bm (128 or 64) rows x 128 columns: N a multiple of 128, K of 64;
 * A, Wf, Y, bias and the gate 16-byte aligned.
 * Optional stream-K scratch (OUT_F32): with ws (at least 2 * CUs * bm * 128
 * floats, CUs = 256 on MI355X) and counters (one per output tile, zeroed once
 * by the caller and left zeroed by every call), one workgroup per compute unit
 * takes an equal share of the tiles' k range; a tile shared by several
 * workgroups is summed by the last to finish, in k order (deterministic, no
 * waiting).  Calls sharing one ws / counters pair must not overlap.
 * split_tail = 1 with ws and counters (one slice; the fp32 or packed output, any
 * operand form):
 * when the tile count T lies between CUs and 2 * CUs, CUs tiles run whole and
 * each of the other T - CUs runs as S workgroups over consecutive k ranges (S
 * the largest of 2..8 with (T - CUs) * S <= CUs, a multiple of 8, and at most
 * K / 64 ranges), so every CU holds one whole tile and at most one part of a
 * split one (at B*T = 1000 the 384 QKV tiles: 256 whole, 128 split in two).
 * The last part of a split tile to finish sums the parts' products in k order
 * and applies the epilogue (deterministic, no waiting).  ws needs CUs * bm *
 * 128 floats, counters one per tile; other shapes run as without scratch.
 * products: 6 (or 0) forms each element pair as the six products of the
 * three-part splits (fp32-level error, the default); 3 uses two-part splits
 * (x0 + x1, 16 significant bits each) and the three products a0 b0 + a0 b1 +
 * a1 b0: half the matrix-core work and two thirds of the W traffic, each
 * product within about 2^-16 of a * b (the packed weight is the same).
 * Two-part packed rows (three products; the packed output on bm 64; no
 * stream-K): an fp32 row
 * packed as 16 bytes per aligned group of four values x, the four bf16(x) and
 * then the four bf16(x - bf16(x)) -- the same bytes, addresses and row stride
 * as the fp32 row.  a_packed = 1: A holds such rows (the GEMM does not split
 * it again; results are bit-identical to the fp32 A it was packed from).
 * out = LX_BX_OUT_PACKED: Y receives the fp32 epilogue's result (no epilogue,
 * GELU or rotary) as packed rows from column pack_from on (a multiple of 4;
 * the columns before it stay fp32), for the next such GEMM or the
 * three-product attention (K and V).  The estimator passes its activations
 * this way with three products (lx_adaln_resid_packed_f32,
 * lx_attention_np_f32's out_packed and kv_packed).
 * Replaces linear() = ggml_mul_mat + ggml_add (src/flow/ops.cpp:20-26) with the
 * node its epilogue absorbs; the fragment-ordered weight has no counterpart
 * in the reference (its weights stay fp32). */
enum { LX_BX_OUT_F32 = 0, LX_BX_OUT_PARTIAL = 1, LX_BX_OUT_PACKED = 2 };
typedef struct lx_linear_bx {
  const float* A;
  long lda;
  const void* Wf;
  const float* bias;
  const lx_epilogue* epi;
  int out;
  float* Y;
  long ldy, slice_stride;
  int M, N, K;
  int bm;
  int slices;
  float* ws;
  size_t ws_floats;
  unsigned* counters;
  int n_counters;
  int products;
  int a_packed;
  int pack_from;
  int split_tail;
} lx_linear_bx;
int lx_wfrag_pack_f32(const float* W, void* Wf, int N, int K, hipStream_t stream);
int lx_linear_bx_f32(const lx_linear_bx* g, hipStream_t stream);

/* Scaled-dot-product attention (flash-style, scores never stored; fp32
 * arithmetic, on the fp32 matrix cores or, for grids that fill the CUs in whole
 * rounds, on the bf16 ones with every operand split into three bf16 parts and
 * six exact partial products accumulated in fp32):
 *   o[b, t, h*hd:(h+1)*hd] = softmax(scale * q_h k_g^T [+ causal mask]) v_g
 * with g = h / (n_heads / n_kv_heads) (GQA, consecutive like HF repeat_kv).
 * q: (B, Tq, *) row stride ldq, head h at column h*hd; k, v: (B, Tk, *) row
 * strides ldk/ldv, kv head g at column g*hd; o: (B, Tq, *) row stride ldo.
 * causal != 0: query i (absolute position q_offset + i) sees keys <= that
 * position.  head_dim must be 64.
 * Replaces attention() (src/flow/dit.cpp:34-51; src/llm/ops.cpp:49-65) and
 * repeat_kv (src/llm/ops.cpp:32-47). */
int lx_attention_f32(const float* q, int ldq, const float* k, int ldk, const float* v,
                     int ldv, float* o, int ldo, int B, int Tq, int Tk, int n_heads,
                     int n_kv_heads, int head_dim, float scale, int causal, int q_offset,
                     hipStream_t stream);
/* lx_attention_f32 with the split-operand kernel's product count: 6 (as
 * lx_attention_f32) or 3 (two bf16 parts per operand, three products: about
 * half the matrix-core work; the grids that run the fp32 kernel ignore it).
 * out_packed != 0: o receives two-part packed rows (lx_linear_bx's a_packed
 * operand) instead of fp32.  kv_packed != 0: k and v are two-part packed rows
 * (lx_linear_bx's LX_BX_OUT_PACKED), for three products on the layouts of the
 * split kernel (64-query grids of at least 256 workgroups, 128-query grids of
 * whole rounds); other shapes return an error.  The estimator calls it with
 * its lx_dit_set_products setting and, with three products, packed K/V from
 * its QKV projection where they apply and packed output for its out
 * projection. */
int lx_attention_np_f32(const float* q, int ldq, const float* k, int ldk, const float* v,
                        int ldv, float* o, int ldo, int B, int Tq, int Tk, int n_heads,
                        int n_kv_heads, int head_dim, float scale, int causal, int q_offset,
                        int products, int out_packed, int kv_packed,
                        hipStream_t stream);

/* Causal grouped conv1d + Mish (one CausalConvPositionEmbedding half):
 *   y[b,t,oc] = mish(bias[oc] + sum_{k<K, ic<C/G} w[oc, ic, k] *
 *                                 x[b, t-(K-1)+k, g*(C/G)+ic]) (+ resid[b,t,oc])
 * with g = oc / (C/G) and x = 0 for negative time (left pad K-1).  x, y, resid:
 * (B, T, C); resid may be NULL; y must not alias x.  `wp` is the weight in the
 * tap-major layout written by lx_conv_pack_weight_f32.  C/G must be 64,
 * K <= 32.  Replaces ggml_pad_ext + grouped_conv1d + mish (+ add)
 * (src/flow/dit.cpp:113-122; src/flow/ops.cpp:28-71). */
int lx_conv_pos_mish_f32(const float* x, const float* wp, const float* bias,
                         const float* resid, float* y, int B, int T, int C, int G, int K,
                         hipStream_t stream);

/* Packs a torch Conv1d weight w (C, C/G, K) into the tap-major layout
 * wp (G, K, C/G, C/G) used above (same element count; done once at load,
 * like the reference's GGUF conversion). */
int lx_conv_pack_weight_f32(const float* w, float* wp, int C, int G, int K,
                            hipStream_t stream);

/* lx_conv_pos_mish_f32 as fp32 arithmetic on the bf16 matrix cores: the
 * operand splits and product counts of lx_linear_bx (products 3 or 6), the
 * input window split once per workgroup, the weight `wf` in MFMA fragment
 * order written by lx_conv_frag_pack_f32 (3 * C * 64 * K bf16, 16-byte
 * aligned).  Same arguments, shapes and result otherwise (error of the
 * products as lx_linear_bx's).  Replaces the same nodes as
 * lx_conv_pos_mish_f32 (src/flow/dit.cpp:113-122); the estimator runs it with
 * its lx_dit_set_products setting. */
int lx_conv_pos_mish_bx_f32(const float* x, const void* wf, const float* bias,
                            const float* resid, float* y, int B, int T, int C, int G, int K,
                            int products, hipStream_t stream);
/* Packs a torch Conv1d weight w (C, 64, K) (C/G = 64, K <= 32) into the
 * fragment order read above (done once at load). */
int lx_conv_frag_pack_f32(const float* w, void* wf, int C, int G, int K, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* DiT estimator and CFM Euler loop (host C++ over the ops above)            */
/* ------------------------------------------------------------------------ */

/* Per-block weights, torch nn.Linear layout (out, in); device pointers.
 * Mirrors FlowWeights::Block (src/flow/internal.h:72-87). */
typedef struct lx_dit_block_weights {
  const float* attn_norm_w; const float* attn_norm_b;   /* (6D, D), (6D) */
  const float* to_q_w; const float* to_q_b;              /* (D, D), (D)   */
  const float* to_k_w; const float* to_k_b;
  const float* to_v_w; const float* to_v_b;
  const float* to_out_w; const float* to_out_b;          /* (D, D), (D)   */
  const float* ff0_w; const float* ff0_b;                /* (F, D), (F)   */
  const float* ff2_w; const float* ff2_b;                /* (D, F), (D)   */
} lx_dit_block_weights;

/* Whole-estimator weights.  Mirrors FlowWeights (src/flow/internal.h:46-94)
 * minus the frontend tensors. */
typedef struct lx_dit_weights {
  int dim, depth, heads, head_dim, ff_inner, mel_dim;    /* 1024,22,16,64,2048,80 */
  const float* time_mlp_0_w; const float* time_mlp_0_b;  /* (D, 256), (D)        */
  const float* time_mlp_2_w; const float* time_mlp_2_b;  /* (D, D), (D)          */
  const float* input_proj_w; const float* input_proj_b;  /* (D, 4*mel), (D)      */
  const float* conv_pos_1_w; const float* conv_pos_1_b;  /* (D, 64, 31), (D)    */
  const float* conv_pos_2_w; const float* conv_pos_2_b;
  const lx_dit_block_weights* blocks;                    /* HOST array [depth]   */
  const float* norm_out_w; const float* norm_out_b;      /* (2D, D), (2D)        */
  const float* proj_out_w; const float* proj_out_b;      /* (mel, D), (mel)      */
} lx_dit_weights;

typedef struct lx_dit lx_dit;

/* Builds an estimator for batches of B rows and up to max_T frames.  Weights
 * are re-packed into library-owned device memory (QKV fused, conv taps
 * transposed, all AdaLN linears stacked), so the caller's buffers may be freed
 * afterwards.  Replaces build_dit + ggml_backend_alloc_ctx_tensors
 * (src/flow/dit.cpp:83-145; src/flow/flow.cpp:184-200). */
int lx_dit_create(const lx_dit_weights* w, int B, int max_T, lx_dit** out);
void lx_dit_destroy(lx_dit* dit);

/* One estimator forward (DiT.forward):
 *   x, mu, cond: (B, mel, T) ("Space A", torch (B, C, T)); spks: (B, mel);
 *   t: device float[B] timesteps in [0, 1]; dphi out: (B, mel, T).
 * The time embedding is computed on the device from t.
 * Replaces one ggml_backend_graph_compute of the DiT graph
 * (src/flow/flow.cpp:244-254) with its host time_embed_host. */
int lx_dit_forward(lx_dit* dit, const float* x, const float* mu, const float* cond,
                   const float* spks, const float* t, float* dphi, int T,
                   hipStream_t stream);

/* Stage capture for parity tests (FlowDebug, include/larynx/flow/flow.h:15-34).
 * When non-NULL, the next lx_dit_forward calls write: time_embed (B, D),
 * input_proj / conv_pos / input_embed (B, T, D), blocks (depth, B, T, D),
 * norm_out (B, T, D).  Pass NULL pointers to disable each. */
typedef struct lx_dit_capture {
  float* time_embed; float* input_proj; float* conv_pos; float* input_embed;
  float* blocks; float* norm_out;
} lx_dit_capture;
int lx_dit_set_capture(lx_dit* dit, const lx_dit_capture* cap);

/* Arithmetic of the block projections (q|k|v, out, FF0, FF2, on the
 * fragment-order split-operand GEMM lx_linear_bx) and of attention
 * (lx_attention_np_f32): products = 3 (the default: two bf16 parts per
 * operand, a0 b0 + a0 b1 + a1 b0; max relative error about 5e-6 per projection
 * at B = 2, T = 500) or 6 (three parts, i + j <= 2: about 1.3e-6, the level of
 * an fp32 GEMM; projections 1.4-1.55x and attention 1.3-1.65x the time).  After
 * 22 blocks at T = 500 the estimator output is within 1.2e-6 (3) and 4.8e-7 (6)
 * of the oracle.  No counterpart in the reference, whose ggml projections are
 * fp32 SGEMM (src/flow/ops.cpp:20-26). */
int lx_dit_set_products(lx_dit* dit, int products);

/* Full CFM Euler solve with classifier-free guidance, device resident
 * (CausalConditionalCFM.solve_euler; src/flow/flow.cpp:202-274):
 *   t_span = 1 - cos(linspace(0,1,n_steps+1) * pi/2)
 *   per step: dphi = est([x;x], [mu;0], [spks;0], [cond;0], [t;t])
 *             x += dt * ((1+cfg) dphi[0] - cfg dphi[1])
 * x: in/out (mel, T) — the initial noise z on entry, the solution on return;
 * mu, cond: (mel, T); spks: (mel).  The estimator must have B == 2. */
int lx_cfm_solve(lx_dit* dit, float* x, const float* mu, const float* cond,
                 const float* spks, int T, int n_steps, float cfg_rate,
                 hipStream_t stream);

/* One Euler step of the above, for timing and resumable loops:
 * t and dt are host scalars. */
int lx_cfm_step(lx_dit* dit, float* x, const float* mu, const float* cond,
                const float* spks, int T, float t, float dt, float cfg_rate,
                hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Flow decoder: frontend + estimator + CFM (FlowDecoder::infer)             */
/* ------------------------------------------------------------------------ */

/* Frontend weights, torch layouts, device pointers.  Mirrors the frontend
 * tensors of FlowWeights (src/flow/internal.h:49-57; GGUF names
 * input_embedding.weight, spk_embed_affine_layer.*, pre_lookahead_layer.*,
 * src/flow/gguf.cpp:45-53). */
typedef struct lx_flow_frontend_weights {
  int vocab;      /* 6561 speech tokens                        */
  int spk_in;     /* 192: speaker embedding width (<= 1024)    */
  int channels;   /* 1024: PreLookahead conv1 output channels  */
  const float* input_embedding;                          /* (vocab, mel)        */
  const float* spk_affine_w; const float* spk_affine_b;  /* (mel, spk_in), (mel)*/
  const float* pre_conv1_w; const float* pre_conv1_b;    /* (channels, mel, 4)  */
  const float* pre_conv2_w; const float* pre_conv2_b;    /* (mel, channels, 3)  */
} lx_flow_frontend_weights;

typedef struct lx_flow lx_flow;

/* FlowDecoder::load equivalent over already-resident weights: builds the
 * frontend (weights re-packed for the im2col GEMMs) and a B = 2 estimator for
 * up to max_tokens speech tokens (MEL_T = 2 * max_tokens frames).  Replaces
 * FlowDecoder::load (src/flow/flow.cpp:49-61) minus the GGUF file read. */
int lx_flow_create(const lx_dit_weights* dit, const lx_flow_frontend_weights* fw,
                   int max_tokens, lx_flow** out);
void lx_flow_destroy(lx_flow* flow);

/* FlowDebug pre-DiT stages (include/larynx/flow/flow.h:15-22); NULL disables
 * each: spk (mel), token_embed (Tseq, mel), prelookahead (Tseq, mel),
 * mu (mel, MEL_T), cond (mel, MEL_T). */
typedef struct lx_flow_capture {
  float* spk; float* token_embed; float* prelookahead; float* mu; float* cond;
} lx_flow_capture;
int lx_flow_set_capture(lx_flow* flow, const lx_flow_capture* cap);

/* The decoder's B = 2 estimator (owned by the decoder, valid until
 * lx_flow_destroy), for the FlowDebug DiT stages at CFM step 1
 * (include/larynx/flow/flow.h:24-31; captured in src/flow/flow.cpp:261-270):
 * lx_dit_set_capture on it, then one lx_dit_forward over the step-1 inputs
 * ([z; z], [mu; 0], [cond; 0], [spk; 0], t = 0).  NULL for a NULL decoder. */
lx_dit* lx_flow_estimator(lx_flow* flow);

/* FlowDecoder::infer (src/flow/flow.cpp:111-290, finalize = true):
 *   prompt_tokens[n_prompt], tokens[n_tokens]: HOST speech token ids; negative
 *     ids are clamped to 0 as the reference does, ids >= vocab -> LX_ERR_RANGE;
 *   prompt_feat: (mel_len1, mel) prompt mel frames; spk_embedding: (spk_in);
 *   noise_z: (mel, MEL_T) CFM start noise, MEL_T = 2 (n_prompt + n_tokens);
 *   mel: out, (mel, MEL_T - mel_len1).
 * Frontend (spk affine, token gather, PreLookahead, mu/cond) then the 10-step
 * CFG Euler solve.  mel_len1 must be below MEL_T. */
int lx_flow_infer(lx_flow* flow, const int32_t* prompt_tokens, int n_prompt,
                  const int32_t* tokens, int n_tokens, const float* prompt_feat, int mel_len1,
                  const float* spk_embedding, const float* noise_z, float* mel,
                  hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Qwen2 LM (host C++ over the ops above; device-resident KV cache)          */
/* ------------------------------------------------------------------------ */

/* Mirrors LLMWeights::Layer (src/llm/internal.h:48-61), torch layout. */
typedef struct lx_qwen2_layer_weights {
  const float* q_w; const float* q_b;        /* (H, H), (H)          */
  const float* k_w; const float* k_b;        /* (KV, H), (KV)        */
  const float* v_w; const float* v_b;        /* (KV, H), (KV)        */
  const float* o_w;                          /* (H, H)               */
  const float* gate_w; const float* up_w;    /* (I, H)               */
  const float* down_w;                       /* (H, I)               */
  const float* in_norm; const float* post_norm; /* (H)               */
} lx_qwen2_layer_weights;

typedef struct lx_qwen2_weights {
  int hidden, intermediate, n_heads, n_kv_heads, head_dim, n_layers;
  int text_vocab, speech_vocab;
  float rms_eps, rope_theta;
  const float* embed_tokens;                 /* (text_vocab, H)      */
  const float* speech_embedding;             /* (speech_vocab, H)    */
  const float* final_norm;                   /* (H)                  */
  const float* llm_decoder;                  /* (speech_vocab, H)    */
  const lx_qwen2_layer_weights* layers;      /* HOST array [n_layers]*/
} lx_qwen2_weights;

typedef struct lx_qwen2 lx_qwen2;

/* Replaces LLM::load's weight upload (src/llm/llm.cpp:50-61); the tables are
 * referenced, the layer weights re-packed (QKV fused, gate/up interleaved).
 * max_ctx bounds prompt + generated tokens (KV cache capacity), 1..4096.
 * Geometry: head_dim 64, hidden <= 2048, hidden + 2 * 64 * n_kv_heads <= 2048,
 * intermediate <= 6144, at most 8 query heads per kv head (Qwen2-0.5B:
 * 896 / 4864 / 14:2); else LX_ERR_ARG. */
int lx_qwen2_create(const lx_qwen2_weights* w, int max_ctx, lx_qwen2** out);
void lx_qwen2_destroy(lx_qwen2* m);

/* LLM::build_lm_input (src/llm/llm.cpp:63-100): lm_input (L, H) =
 * [speech_emb[6561]; embed_tokens[text...]; speech_emb[6563];
 *  speech_emb[prompt_speech...]].  Ids are HOST arrays, all validated first
 * (LX_ERR_RANGE on any bad id).  L_out receives L.  out: device (L, H). */
int lx_qwen2_build_lm_input(lx_qwen2* m, const int* text_tokens, int n_text,
                            const int* prompt_speech, int n_speech, float* out, int* L_out,
                            hipStream_t stream);

/* LLM::prefill (src/llm/llm.cpp:102-216): causal 24-layer pass over lm_input
 * (L, H) (device), resets and fills the KV cache.  logits (L, speech_vocab)
 * device, may be NULL; hidden (n_layers, L, H) and final_norm (L, H) capture
 * buffers may be NULL. */
int lx_qwen2_prefill(lx_qwen2* m, const float* lm_input, int L, float* logits,
                     float* hidden, float* final_norm, hipStream_t stream);

/* LLM::decode (src/llm/llm.cpp:218-327): one token (HOST id in
 * [0, speech_vocab)) at position cache_len, appends to the device KV cache.
 * logits: device (speech_vocab); final_norm: device (H) or NULL.
 * The position lives in device memory, so the layer stack is captured into a
 * HIP graph on the first decode (on a stream of the object's own) and
 * replayed on `stream` for every later token (see lx_qwen2_set_decode_graph).
 * Calls on one object must not overlap. */
int lx_qwen2_decode(lx_qwen2* m, int token, float* logits, float* final_norm,
                    hipStream_t stream);

/* Decode launch mode: enable != 0 (the default) replays the captured layer
 * stack as a HIP graph; 0 launches the same kernels eagerly on `stream` (for
 * callers that capture decode into graphs of their own, and for checking the
 * two bit for bit).  No counterpart in the reference, which rebuilds its ggml
 * graph every step (src/llm/llm.cpp:232-275). */
int lx_qwen2_set_decode_graph(lx_qwen2* m, int enable);

/* Prefill projections' split-operand products, 3 (the default) or 6, as
 * lx_dit_set_products (decode's GEMVs are fp32 either way).  No counterpart
 * in the reference (src/llm/llm.cpp:141-173 runs fp32 ggml_mul_mat). */
int lx_qwen2_set_products(lx_qwen2* m, int products);

/* LLM::cache_len / cache_key / cache_value (include/larynx/llm/llm.h:77-84).
 * The cache of layer l is (cache_len, n_kv_heads * head_dim) roped keys /
 * raw values on the device; pointers stay valid until destroy. */
int lx_qwen2_cache_len(const lx_qwen2* m);
const float* lx_qwen2_cache_key(const lx_qwen2* m, int layer);
const float* lx_qwen2_cache_value(const lx_qwen2* m, int layer);
/* Sets cache_len (<= max_ctx) without touching the contents, so a caller can
 * load a synthetic cache through the pointers above (benchmarks, tests). */
int lx_qwen2_set_cache_len(lx_qwen2* m, int len);

/* ------------------------------------------------------------------------ */
/* GGUF v3 weight files and the model loaders over them                      */
/* ------------------------------------------------------------------------ */

/* A parsed GGUF v3 file (docs/WEIGHT_FORMAT.md §1-3 of the reference; read there
 * by ggml's gguf_init_from_file + upload_gguf_weights,
 * include/larynx/backend.h:48-87).  lx_gguf_open validates the header, the
 * metadata and every tensor's extent against the file size, then (unless
 * LX_GGUF_HOST_ONLY) streams the data section into one device allocation
 * owned by the object.  Only unquantised tensor types are accepted (F32, F16,
 * BF16, F64, I8..I64); the CosyVoice3 checkpoints are all F32.  Bad files are
 * LX_ERR_ARG with a message naming the problem. */
typedef struct lx_gguf lx_gguf;
enum { LX_GGUF_HOST_ONLY = 1 };
int lx_gguf_open(const char* path, int flags, lx_gguf** out);
void lx_gguf_close(lx_gguf* gguf);
int lx_gguf_n_tensors(const lx_gguf* gguf);
/* Index of a tensor by name (the PyTorch state_dict key), or -1. */
int lx_gguf_find(const lx_gguf* gguf, const char* name);
/* name (owned by the object), ggml type, n_dims and ne[4] (fastest first,
 * i.e. the torch shape reversed; unused dims 1), byte size.  Any out pointer
 * may be NULL. */
int lx_gguf_tensor_info(const lx_gguf* gguf, int index, const char** name, int* type,
                        int* n_dims, int64_t* ne, uint64_t* nbytes);
/* Device pointer of a tensor's data (NULL in host-only mode). */
const void* lx_gguf_tensor_data(const lx_gguf* gguf, int index);
/* String-valued metadata (general.architecture, general.name), or NULL. */
const char* lx_gguf_get_string(const lx_gguf* gguf, const char* key);

/* FlowDecoder::load (src/flow/flow.cpp:49-61, src/flow/gguf.cpp:24-135): the
 * flow checkpoint's tensors (frontend names at the top level, the estimator
 * under decoder.estimator.), geometry read from their shapes; the file's
 * device copy is released once the decoder has packed its own. */
int lx_flow_load(const char* path, int max_tokens, lx_flow** out);
/* LLM::load (src/llm/llm.cpp:50-61, src/llm/gguf.cpp:30-100): names under
 * llm.model.model. plus speech_embedding / llm_decoder; the model copies every
 * tensor into its own memory and releases the file's device copy. */
int lx_qwen2_load(const char* path, int max_ctx, lx_qwen2** out);

#ifdef __cplusplus
}
#endif

#endif /* LX_OPS_H */
