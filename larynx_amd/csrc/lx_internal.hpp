// Internal (non-ABI) entry points shared between the kernel files and the
// host-side estimator / Qwen2 code.
#pragma once

#include "lx_common.hpp"

namespace lx {

// y[b, n] = act_out(sum_k W[n, k] * act_in(x[b, k]) + bias[n]); act: 0 none, 1 silu.
int gemv(const float* x, int B, int K, const float* W, const float* bias, float* y, long N,
         long ldy, int act_in, int act_out, hipStream_t stream);

// Skinny-M path of lx_linear_f32 (M <= 8) with the same epilogue contract.
int gemv_epi(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
             int M, int N, int K, const lx_epilogue* epi, hipStream_t stream);

// DiT input packing: A[b*T + t, :] = [x[b,:,t], cond[b,:,t], mu[b,:,t], spks[b,:]]
// (the concat order of src/flow/dit.cpp:109), A row stride 4*mel.
int dit_pack_input(const float* x, const float* cond, const float* mu, const float* spks,
                   float* A, int B, int T, int mel, hipStream_t stream);

// (B*T, mel) row-major -> (B, mel, T): the proj_out permute + cont of
// src/flow/dit.cpp:139-140.
int dit_unpack_output(const float* P, float* dphi, int B, int T, int mel, hipStream_t stream);

// CFG combine + Euler update straight from the proj_out rows:
// x[c, t] += dt * (a * P[t, c] - b * P[T + t, c]).
int cfm_euler_update(float* x, const float* P, int T, int mel, float dt, float a, float b,
                     hipStream_t stream);

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

// Strided 2-D copy: dst[r, c] = src[r, c] for r < rows, c < cols.
int copy_rows(const float* src, int lds, float* dst, int ldd, int rows, int cols,
              hipStream_t stream);

// Flash-decoding for one query row per batch (Tq == 1); `part` holds
// attention_decode_part_floats(B, Tk, n_heads) floats.
int attention_decode_split(const float* q, int ldq, const float* k, int ldk, const float* v,
                           int ldv, float* o, int ldo, int B, int Tk, int n_heads,
                           int n_kv_heads, float scale, float* part, hipStream_t stream);
size_t attention_decode_part_floats(int B, int Tk, int n_heads);

// Grouped conv + Mish with tap-major packed weights (lx_conv_pos_mish_f32).
int conv_pos_mish_packed(const float* x, const float* wp, const float* bias, const float* resid,
                         float* y, int B, int T, int C, int G, int K, hipStream_t stream);

}  // namespace lx
