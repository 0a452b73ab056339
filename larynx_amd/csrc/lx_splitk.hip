// Reduce passes of the split-K projections, each fused with what follows the
// projection in a Qwen2 prefill layer (src/llm/llm.cpp:141-173):
//   - splitk_resid_rmsnorm: residual add of o_proj / down_proj
//     (llm.cpp:160, 171) and the RMSNorm that opens the next sub-layer
//     (post_attention_layernorm, the next layer's input_layernorm, or the final
//     norm; src/llm/ops.cpp:7-11);
//   - splitk_qkv_rope_cache: q/k/v bias, NEOX rotary on q and k
//     (src/llm/ops.cpp:21-30) and the KV cache append (llm.cpp:200-204).
// The K slices are summed in a fixed order, so results are reproducible.
#include "lx_common.hpp"
#include "lx_gemm_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int kHD = 64;

constexpr int kMaxSplits = 9;  // K slices a reduce pass sums (all loads in flight)

// Sum of the K slices of float4 slot i (< N4) of a row: every slice's load is
// issued before the first add (slices past `splits` re-read slice 0 and are
// dropped), then the adds run in slice order.
__device__ __forceinline__ float4 sum_slices(const float* __restrict__ ws, int splits, long slice,
                                             long row_off, int i) {
  float4 p[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s)
    p[s] = reinterpret_cast<const float4*>(ws + (s < splits ? s : 0) * slice + row_off)[i];
  float4 sum = p[0];
#pragma unroll
  for (int s = 1; s < kMaxSplits; ++s)
    if (s < splits) {
      sum.x += p[s].x;
      sum.y += p[s].y;
      sum.z += p[s].z;
      sum.w += p[s].w;
    }
  return sum;
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup (256 threads) per row; thread t owns float4 slots t + 256 j.
template <int NV>
__global__ __launch_bounds__(256) void resid_rmsnorm_kernel(const float* __restrict__ ws,
                                                            int splits, int M, int N,
                                                            const float* __restrict__ bias,
                                                            float* x, const float* __restrict__ w,
                                                            float eps, float* hn, int pk) {
  __shared__ float red[4];
  const int row = blockIdx.x, t = threadIdx.x;
  const int N4 = N >> 2;
  float4* xr = reinterpret_cast<float4*>(x + (long)row * N);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = min(t + 256 * j, N4 - 1);
    float4 a = xr[i];
    float4 sum = sum_slices(ws, splits, (long)M * N, (long)row * N, i);
    if (bias) {
      const float4 b = reinterpret_cast<const float4*>(bias)[i];
      sum.x += b.x;
      sum.y += b.y;
      sum.z += b.z;
      sum.w += b.w;
    }
    a.x = a.x + sum.x;
    a.y = a.y + sum.y;
    a.z = a.z + sum.z;
    a.w = a.w + sum.w;
    v[j] = t + 256 * j < N4 ? a : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (t + 256 * j < N4) xr[t + 256 * j] = v[j];
  if (!w) return;
  // RMSNorm of the updated row
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  const float r = 1.0f / sqrtf(block_sum256(ss, red) / (float)N + eps);
  float4* hr = reinterpret_cast<float4*>(hn + (long)row * N);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = t + 256 * j;
    if (i < N4) {
      const float4 g = reinterpret_cast<const float4*>(w)[i];
      float4 o;
      o.x = (v[j].x * r) * g.x;
      o.y = (v[j].y * r) * g.y;
      o.z = (v[j].z * r) * g.z;
      o.w = (v[j].w * r) * g.w;
      if (pk)  // two-part packed row for the three-product GEMM
        reinterpret_cast<uintx4_t*>(hr)[i] = pack2_bf16(floatx4{o.x, o.y, o.z, o.w});
      else
        hr[i] = o;
    }
  }
}

// One workgroup per row of the fused q|k|v projection (NQKV <= 1024 * NV
// floats), staged in LDS so the NEOX pairs (c, c + 32) of every head are at
// hand.
template <int NV>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const float* __restrict__ ws, int splits, int M, int NQKV, const float* __restrict__ bias,
    int n_heads, int n_kv_heads, const int* __restrict__ pos, const float* __restrict__ inv_freq,
    float* q_out, int ldq, float* k_cache, float* v_cache, int row0) {
  extern __shared__ float rl[];  // one row of NQKV
  const int row = blockIdx.x, t = threadIdx.x;
  const int N4 = NQKV >> 2;
  const float ang = (float)pos[row] * inv_freq[t & 31];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = min(t + 256 * j, N4 - 1);
    float4 v = sum_slices(ws, splits, (long)M * NQKV, (long)row * NQKV, i);
    const float4 b = reinterpret_cast<const float4*>(bias)[i];
    v.x += b.x;
    v.y += b.y;
    v.z += b.z;
    v.w += b.w;
    if (t + 256 * j < N4) *reinterpret_cast<float4*>(rl + 4 * i) = v;
  }
  // rotary: thread = (head slot, pair index p = t % 32); angle = fp32(pos) * inv_freq[p]
  float sn, cs;
  sincosf(ang, &sn, &cs);
  __syncthreads();
  const int p = t & 31;
  for (int h = t >> 5; h < n_heads + n_kv_heads; h += 8) {
    float* ptr = rl + h * kHD + p;
    const float x0 = ptr[0], x1 = ptr[kHD / 2];
    ptr[0] = x0 * cs - x1 * sn;
    ptr[kHD / 2] = x1 * cs + x0 * sn;
  }
  __syncthreads();
  const int Q = n_heads * kHD, KV = n_kv_heads * kHD;
  float* qr = q_out + (long)row * ldq;
  float* kr = k_cache + (long)(row0 + row) * KV;
  float* vr = v_cache + (long)(row0 + row) * KV;
  for (int i = t; i < N4; i += 256) {
    const int c = 4 * i;
    const float4 val = *reinterpret_cast<const float4*>(rl + c);
    if (c < Q)
      *reinterpret_cast<float4*>(qr + c) = val;
    else if (c < Q + KV)
      *reinterpret_cast<float4*>(kr + (c - Q)) = val;
    else
      *reinterpret_cast<float4*>(vr + (c - Q - KV)) = val;
  }
}

}  // namespace

int splitk_resid_rmsnorm(const float* ws, int splits, int M, int N, const float* bias, float* x,
                         const float* norm_w, float eps, float* hn, hipStream_t stream,
                         int out_packed) {
  LX_REQUIRE(ws && x && M > 0 && N > 0 && N % 4 == 0 && splits >= 1 && splits <= kMaxSplits &&
                 (!norm_w || hn),
             "splitk_resid_rmsnorm: bad args");
  const int nv = (N / 4 + 255) / 256;
  if (nv <= 1)
    hipLaunchKernelGGL(resid_rmsnorm_kernel<1>, dim3(M), dim3(256), 0, stream, ws, splits, M, N,
                       bias, x, norm_w, eps, hn, out_packed ? 1 : 0);
  else if (nv <= 2)
    hipLaunchKernelGGL(resid_rmsnorm_kernel<2>, dim3(M), dim3(256), 0, stream, ws, splits, M, N,
                       bias, x, norm_w, eps, hn, out_packed ? 1 : 0);
  else if (nv <= 4)
    hipLaunchKernelGGL(resid_rmsnorm_kernel<4>, dim3(M), dim3(256), 0, stream, ws, splits, M, N,
                       bias, x, norm_w, eps, hn, out_packed ? 1 : 0);
  else {
    set_error("splitk_resid_rmsnorm: N=%d too wide", N);
    return LX_ERR_ARG;
  }
  return check_launch("resid_rmsnorm_kernel");
}

int splitk_qkv_rope_cache(const float* ws, int splits, int M, const float* bias, int n_heads,
                          int n_kv_heads, const int* pos, const float* inv_freq, float* q_out,
                          int ldq, float* k_cache, float* v_cache, int row0, hipStream_t stream) {
  const int NQKV = (n_heads + 2 * n_kv_heads) * kHD;
  LX_REQUIRE(ws && bias && pos && inv_freq && q_out && k_cache && v_cache && M > 0 && splits >= 1 &&
                 ldq % 4 == 0 && ldq >= n_heads * kHD && row0 >= 0,
             "splitk_qkv_rope_cache: bad args");
  LX_REQUIRE(splits <= kMaxSplits, "splitk_qkv_rope_cache: %d slices > %d", splits, kMaxSplits);
  LX_REQUIRE(NQKV <= 2048, "splitk_qkv_rope_cache: row of %d too wide", NQKV);
  const size_t lds = (size_t)NQKV * sizeof(float);
  if (NQKV <= 1024)
    hipLaunchKernelGGL(qkv_rope_cache_kernel<1>, dim3(M), dim3(256), lds, stream, ws, splits, M,
                       NQKV, bias, n_heads, n_kv_heads, pos, inv_freq, q_out, ldq, k_cache,
                       v_cache, row0);
  else
    hipLaunchKernelGGL(qkv_rope_cache_kernel<2>, dim3(M), dim3(256), lds, stream, ws, splits, M,
                       NQKV, bias, n_heads, n_kv_heads, pos, inv_freq, q_out, ldq, k_cache,
                       v_cache, row0);
  return check_launch("qkv_rope_cache_kernel");
}

}  // namespace lx
