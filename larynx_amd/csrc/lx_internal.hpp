// Internal (non-ABI) entry points shared between the kernel files and the
// host-side estimator / Qwen2 code.
#pragma once

#include <vector>

#include "lx_common.hpp"

namespace lx {

// Device allocations of a composite object (lx_dit, lx_qwen2, lx_flow), made
// at create time and released together when the object is destroyed.
struct Arena {
  std::vector<void*> ptrs;
  ~Arena() {
    for (void* p : ptrs) (void)hipFree(p);
  }
  template <typename T>
  T* alloc(size_t n) {
    void* p = nullptr;
    if (n == 0) n = 1;
    if (hipMalloc(&p, n * sizeof(T)) != hipSuccess) return nullptr;
    ptrs.push_back(p);
    return static_cast<T*>(p);
  }
};

#define LX_TRY(expr)              \
  do {                            \
    int _rc = (expr);             \
    if (_rc != LX_OK) return _rc; \
  } while (0)

// y[b, n] = act_out(sum_k W[n, k] * act_in(x[b, k]) + bias[n]); act: 0 none, 1 silu.
int gemv(const float* x, int B, int K, const float* W, const float* bias, float* y, long N,
         long ldy, int act_in, int act_out, hipStream_t stream);

// Sinusoid coefficients c_j = exp(-j ln(1e4) / (half - 1)), j < half (host).
void timestep_coeff(int half, float* c);

// TimestepEmbedding on the device: sinusoid(256, scale 1000) of t -> Linear ->
// SiLU -> Linear, the sinusoid formed inside the first layer's kernel.  t is
// read from device memory (tdev) or, when tdev is null, taken from the host
// array thost (B values).  hid: B * D floats of scratch.
int time_mlp(const float* tdev, const float* thost, int B, const float* w0, const float* b0,
             const float* w2, const float* b2, int D, float* hid, float* out, hipStream_t stream);

// Skinny-M path of lx_linear_f32 (M <= 8) with the same epilogue contract.
int gemv_epi(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
             int M, int N, int K, const lx_epilogue* epi, hipStream_t stream);

// DiT input packing: A[b*T + t, :] = [x[b,:,t], cond[b,:,t], mu[b,:,t], spks[b,:]]
// (the concat order of src/flow/dit.cpp:109), A row stride 4*mel.  x of batch b
// starts at x + b * x_bstride (mel*T for a (B, mel, T) tensor; 0 feeds the same
// x to every batch row, as the CFG pair does).  cfg != 0: cond, mu, spks are
// the conditional row's tensors and the other rows get zeros
// (src/flow/flow.cpp:215-224).
int dit_pack_input(const float* x, long x_bstride, const float* cond, const float* mu,
                   const float* spks, int cfg, float* A, int B, int T, int mel,
                   hipStream_t stream);

// (B*T, mel) row-major -> (B, mel, T): the proj_out permute + cont of
// src/flow/dit.cpp:139-140.
int dit_unpack_output(const float* P, float* dphi, int B, int T, int mel, hipStream_t stream);

// CFG combine + Euler update straight from the proj_out rows:
// x[c, t] += dt * (a * P[t, c] - b * P[T + t, c]), where P is the sum of
// `splits` K slices `slice` floats apart (slice order) plus bias (may be null).
int cfm_euler_update(float* x, const float* P, int splits, long slice, const float* bias, int T,
                     int mel, float dt, float a, float b, hipStream_t stream);

// P (rows, mel) = sum of the split-K slices of ws (slice order) + bias.
int proj_reduce(const float* ws, int splits, long slice, const float* bias, float* P, int rows,
                int mel, hipStream_t stream);

// Duplicate a (rows, n) block into (copies * rows, n) (CFG batch [v; v] / [v; 0]).
int fill_batch(float* dst, const float* src, long n, int copies, int zero_tail,
               hipStream_t stream);

// Transpose the grouped-conv weight (C, C/G, K) into tap-major (G, K, C/G oc, C/G ic).
int conv_weight_pack(const float* w, float* wp, int C, int G, int K, hipStream_t stream);

// Iota: p[i] = i for i < n.
int iota_i32(int* p, int n, hipStream_t stream);
// Fill n floats with value.
int fill_f32(float* p, long n, float value, hipStream_t stream);

// Interleave two (rows, K) matrices row by row: out[2r] = a[r], out[2r+1] = b[r].
int interleave_rows(const float* a, const float* b, float* out, int rows, int K,
                    hipStream_t stream);

// ---- split-K GEMM (lx_gemm.hip) and its reduce / epilogue kernels (lx_splitk.hip) ----
// ws[s] (M, N) = x[:, s*ksplit : (s+1)*ksplit] @ W[:, same]^T, s < splits (no bias).
int gemm_splitk_partials(const float* x, int ldx, const float* W, int ldw, float* ws, int M,
                         int N, int K, int splits, int ksplit, hipStream_t stream);
// Number of K slices (and slice width, a multiple of 64) that gives the
// (M, N) tile grid about two workgroups per CU.
int gemm_splitk_plan(int M, int N, int K, int* ksplit);
// lx_linear_f32 whose tile launch, when its tiles leave a partial last round
// over the CUs, runs the tail tiles as K slices that the last-arriving slice
// of each tile sums in slice order (deterministic, no waiting): ws holds up to
// ws_floats of partial tiles, arrivals one counter per tail tile (n_arrivals of
// them), zeroed once by the caller and left zeroed by every launch.  Falls back
// to the plain launch when no split applies or the scratch is too small.
int linear_split_tail(const float* x, int ldx, const float* W, const float* bias, float* y,
                      int ldy, int M, int N, int K, const lx_epilogue* epi, float* ws,
                      size_t ws_floats, unsigned* arrivals, int n_arrivals, hipStream_t stream);
// Three bf16 planes of n fp32 values (n % 4 == 0): x = x0 + x1 + x2 with x0 =
// bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1); plane p at planes + p * n.
int split_planes(const float* w, void* planes, long n, hipStream_t stream);
// lx_linear_f32 on the bf16 matrix cores with split operands: W given as the
// three planes of split_planes over its (N, K) values, x split in the kernel,
// six products per element pair, fp32 accumulation.  Tiles of 128 x 128
// (narrow: 128 x 64, for N that leaves the wide tiles a partial round);
// N % 128 (narrow: 64) == 0, K % 32 == 0; every epilogue but SWIGLU_PAIRED;
// y, bias and gate 16-byte aligned.
int linear_split(const float* x, int ldx, const void* Wp, const float* bias, float* y, int ldy,
                 int M, int N, int K, const lx_epilogue* epi, int narrow, hipStream_t stream);
// Scratch floats a split tail of this shape uses (0: none) and its tail tiles.
size_t split_tail_ws_floats(int M, int N, int K, int* tail_tiles);
// x[m, :] += sum_s ws[s][m, :] (+ bias); then, if norm_w, hn[m, :] =
// RMSNorm(x[m, :]) * norm_w (the next sub-layer's input norm).  Rows of N floats.
int splitk_resid_rmsnorm(const float* ws, int splits, int M, int N, const float* bias, float* x,
                         const float* norm_w, float eps, float* hn, hipStream_t stream,
                         int out_packed = 0);
// v = sum_s ws[s][m, :] + bias over the fused q|k|v row (n_heads + 2 n_kv_heads
// heads of 64); NEOX rotary at position pos[m] on the q and k heads; q ->
// q_out[m, 0:n_heads*64] (row stride ldq), k / v -> k_cache / v_cache row
// row0 + m (row stride n_kv_heads*64).
int splitk_qkv_rope_cache(const float* ws, int splits, int M, const float* bias, int n_heads,
                          int n_kv_heads, const int* pos, const float* inv_freq, float* q_out,
                          int ldq, float* k_cache, float* v_cache, int row0, hipStream_t stream);

// lx_adaln_resid_f32, with y as two-part packed rows when out_packed
// (lx_adaln_resid_packed_f32).
int adaln_resid(float* h, const float* partials, int splits, long partial_stride,
                const float* bias, const float* gate, long gate_stride, const float* shift,
                const float* scale, long mod_stride, float* y, int B, int T, int D, float eps,
                int out_packed, hipStream_t stream);

// ---- split-operand GEMM with W in fragment order (lx_gemm_bx.hip) ----
// lx_linear_bx_f32 (arguments and outputs as declared in lx_ops.h).
int linear_bx(const lx_linear_bx& g, hipStream_t stream);
// Parts per split tile of lx_linear_bx's split tail for an (M, N, K) launch on
// bm-row tiles (0: the split tail does not apply), and the ws it needs.
int bx_split_parts(int M, int N, int K, int bm);
size_t bx_split_ws_floats(int bm);
// lx_attention_f32 with the split-operand kernel's product count (3 or 6; the
// fp32 kernel, which small grids run, ignores it).
int attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv, float* o,
              int ldo, int B, int Tq, int Tk, int n_heads, int n_kv_heads, int head_dim,
              float scale, int causal, int q_offset, int products, int out_packed,
              hipStream_t stream, int kv_packed = 0);
// Whether attention() runs this shape on the three-product split kernel, the
// one that reads K and V as two-part packed rows (kv_packed).
bool attention_takes_packed_kv(int B, int Tq, int n_heads, int products);
// W (N, K) -> fragment order (3 * N * K bf16); N % 32 == 0, K % 16 == 0.
int wfrag_pack(const float* W, void* Wf, int N, int K, hipStream_t stream);

// ---- single-token decode (lx_decode.hip) ----
enum { DEC_QKV_ROPE = 0, DEC_SWIGLU = 1, DEC_RESID = 2, DEC_HEAD = 3 };

// y = epi(W @ norm(x) + bias) for one activation row x (K), W (N, K).
//   DEC_QKV_ROPE: x RMSNorm'ed with norm_w; columns [0, q_cols) -> y (q),
//     [q_cols, q_cols + kv_cols) -> k_cache[pos], the rest -> v_cache[pos];
//     NEOX rotary (head_dim 64, device table inv_freq) on the first rope_heads heads.
//   DEC_SWIGLU: x RMSNorm'ed; W rows interleaved (gate_i, up_i);
//     y[i] = silu(gate_i) * up_i.
//   DEC_RESID: y[n] += (W x)[n] (no norm).
//   DEC_HEAD: x RMSNorm'ed; y[n] = (W x)[n]; y2 (K), if set, receives norm(x).
struct DecGemvArgs {
  const float* x = nullptr;
  const float* norm_w = nullptr;
  float eps = 0.0f;
  const float* W = nullptr;
  const float* bias = nullptr;
  float* y = nullptr;
  float* y2 = nullptr;
  long N = 0;
  int K = 0;
  const int* pos = nullptr;  // device: position of the token
  int q_cols = 0, kv_cols = 0, rope_heads = 0;
  float* k_cache = nullptr;
  float* v_cache = nullptr;
  const float* inv_freq = nullptr;  // device: 32 rotary inverse frequencies
};
int dec_gemv(int epi, const DecGemvArgs& a, hipStream_t stream);
// True when the decode kernels cover this geometry (K = hidden <= 2048,
// K = intermediate <= 6144).
bool dec_supported(int hidden, int intermediate);

// Split-key GQA attention of one query row over keys [0, *pos] of the cache.
struct DecAttnArgs {
  const float* q = nullptr;  // (n_heads * 64), roped
  const float* k_cache = nullptr;
  const float* v_cache = nullptr;
  int ld = 0;                // cache row stride (n_kv_heads * 64)
  const int* pos = nullptr;  // device
  float scale = 0.0f;
  int rep = 0;               // n_heads / n_kv_heads
  int n_heads = 0;
  int max_rows = 0;          // cache capacity (rows)
  float* part = nullptr;     // n_kv_heads * part_group_stride floats
  long part_group_stride = 0;
  float* out = nullptr;      // (n_heads * 64)
};
// Position + 1 <= dec_attention_split_keys(): one launch over the single
// split, writing the normalised output.
int dec_attention(const DecAttnArgs& a, int n_kv_heads, hipStream_t stream);
// Longer caches: the split partial pass, then the merge fused into o_proj +
// residual (o: DEC_RESID arguments, x unused).  Split class `cls` covers up to
// the cls-th split count; dec_attention_class(n_split) picks it (-1: past
// dec_attention_max_ctx()).
int dec_attention_o(const DecAttnArgs& a, int n_kv_heads, int cls, const DecGemvArgs& o,
                    hipStream_t stream);
int dec_attention_class(int n_split);
constexpr int kDecAttnClasses = 16;  // split classes of dec_attention_o
int dec_attention_split_keys();
int dec_attention_splits(int max_ctx);
int dec_attention_max_ctx();  // largest cache the merge covers
// floats per kv head of the partial-state buffer
long dec_attention_part_floats(int max_ctx, int rep);
// x = table[row]; *d_pos = pos.
int dec_begin(const float* table, long row, int D, float* x, int* d_pos, int pos,
              hipStream_t stream);

// ---- flow frontend (lx_frontend.hip) ----
// y[o] = W[o, :] . (x / sqrt(max(|x|^2, 1e-12))) + b[o]; x (K <= 1024), W (N, K).
int flow_spk_affine(const float* x, int K, const float* W, const float* b, float* y, int N,
                    hipStream_t s);
// A[t, k*C + c] = f(x[t + k - pad_left, c]) (0 outside [0, T)); f = leaky_relu(0.01) if leaky.
int flow_im2col(const float* x, int T, int C, int Kw, int pad_left, int leaky, float* A,
                hipStream_t s);
// mu[c, t'] = pre[t' / ratio, c]; cond[c, t'] = prompt_feat[t', c] (t' < mel_len1) else 0.
int flow_pack_mu_cond(const float* pre, int Tseq, int ratio, const float* prompt_feat,
                      int mel_len1, int mel, float* mu, float* cond, hipStream_t s);
// Conv1d weight (OC, IC, K) -> (OC, K * IC) with column k * IC + ic.
int conv_kmajor_pack(const float* w, int OC, int IC, int K, float* wp, hipStream_t s);

// ---- weight files (lx_gguf.cpp / lx_qwen2.cpp) ----
// Copies the embedding tables the model references into its own device memory
// (synchronous), so the weight file's device copy can be released.
int qwen2_own_tables(lx_qwen2* m);

// Conv weight (C, 64, K) -> MFMA fragment order (lx_conv_frag_pack_f32), and the
// split-operand grouped conv + Mish on it (lx_conv_pos_mish_bx_f32).
int conv_frag_pack(const float* w, void* wf, int C, int G, int K, hipStream_t stream);
int conv_pos_mish_bx(const float* x, const void* wf, const float* bias, const float* resid,
                     float* y, int B, int T, int C, int G, int K, int products,
                     hipStream_t stream);
// Grouped conv + Mish with tap-major packed weights (lx_conv_pos_mish_f32).
int conv_pos_mish_packed(const float* x, const float* wp, const float* bias, const float* resid,
                         float* y, int B, int T, int C, int G, int K, hipStream_t stream);

}  // namespace lx
