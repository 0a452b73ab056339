// Skinny products y = act_out(W @ act_in(x) + bias) for a handful of rows
// (B <= 8): the AdaLN modulation linears and the time-embedding MLP.  These
// are weight-streaming (HBM-bound on W), so each wave owns R output rows at a
// time, keeps R float4 weight loads in flight per lane, and reduces with
// wave64 shuffles.  The activations are staged in LDS with act_in applied.
#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kGemvRows = 4;
constexpr int kGemvBMax = 8;

template <int ACT_IN, int ACT_OUT>
__global__ __launch_bounds__(kGemvWaves * kWave) void gemv_kernel(
    const float* __restrict__ x, int B, int K, const float* __restrict__ W,
    const float* __restrict__ bias, float* __restrict__ y, long N, long ldy) {
  extern __shared__ float xs[];  // B * K
  for (int i = threadIdx.x; i < B * K; i += blockDim.x) {
    float v = x[i];
    if (ACT_IN == 1) v = v / (1.0f + expf(-v));
    xs[i] = v;
  }
  __syncthreads();
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int K4 = K >> 2;
  const float4* xs4 = reinterpret_cast<const float4*>(xs);
  const long step = (long)gridDim.x * kGemvWaves * kGemvRows;
  for (long n0 = ((long)blockIdx.x * kGemvWaves + wave) * kGemvRows; n0 < N; n0 += step) {
    float acc[kGemvRows][kGemvBMax];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
      for (int b = 0; b < kGemvBMax; ++b) acc[r][b] = 0.0f;
#pragma unroll 4
    for (int k4 = lane; k4 < K4; k4 += kWave) {
      float4 w[kGemvRows];
      // weights are read exactly once per call: streaming cache policy
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r)
        w[r] = (n0 + r < N) ? ld_nt(reinterpret_cast<const float4*>(W + (n0 + r) * K) + k4)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int b = 0; b < kGemvBMax; ++b) {
        if (b < B) {
          float4 xv = xs4[b * K4 + k4];
#pragma unroll
          for (int r = 0; r < kGemvRows; ++r)
            acc[r][b] += (w[r].x * xv.x + w[r].y * xv.y) + (w[r].z * xv.z + w[r].w * xv.w);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
#pragma unroll
      for (int b = 0; b < kGemvBMax; ++b) {
        if (b < B) {
          float s = wave_sum(acc[r][b]);
          if (lane == 0 && n0 + r < N) {
            float v = s + (bias ? bias[n0 + r] : 0.0f);
            if (ACT_OUT == 1) v = v / (1.0f + expf(-v));
            y[b * ldy + n0 + r] = v;
          }
        }
      }
    }
  }
}

}  // namespace

int gemv(const float* x, int B, int K, const float* W, const float* bias, float* y, long N,
         long ldy, int act_in, int act_out, hipStream_t stream) {
  LX_REQUIRE(x && W && y, "gemv: null pointer");
  LX_REQUIRE(B > 0 && B <= kGemvBMax && K > 0 && K % 4 == 0 && N > 0,
             "gemv: bad shape B=%d K=%d N=%ld", B, K, N);
  LX_REQUIRE((size_t)B * K * sizeof(float) <= 64 * 1024, "gemv: B*K too large for LDS");
  LX_REQUIRE(((uintptr_t)W) % 16 == 0, "gemv: W must be 16-byte aligned");
  long rows_per_block = (long)kGemvWaves * kGemvRows;
  long g = (N + rows_per_block - 1) / rows_per_block;
  if (g > 4096) g = 4096;
  dim3 grid((unsigned)g), block(kGemvWaves * kWave);
  size_t lds = (size_t)B * K * sizeof(float);
  if (act_in == 0 && act_out == 0)
    hipLaunchKernelGGL((gemv_kernel<0, 0>), grid, block, lds, stream, x, B, K, W, bias, y, N, ldy);
  else if (act_in == 1 && act_out == 0)
    hipLaunchKernelGGL((gemv_kernel<1, 0>), grid, block, lds, stream, x, B, K, W, bias, y, N, ldy);
  else if (act_in == 0 && act_out == 1)
    hipLaunchKernelGGL((gemv_kernel<0, 1>), grid, block, lds, stream, x, B, K, W, bias, y, N, ldy);
  else
    hipLaunchKernelGGL((gemv_kernel<1, 1>), grid, block, lds, stream, x, B, K, W, bias, y, N, ldy);
  return check_launch("gemv_kernel");
}

}  // namespace lx

using namespace lx;

extern "C" int lx_adaln_emb_f32(const float* c, const float* W, const float* bias,
                                float* emb, int B, int D, int n_out, hipStream_t stream) {
  return gemv(c, B, D, W, bias, emb, n_out, n_out, /*act_in=*/1, /*act_out=*/0, stream);
}

extern "C" int lx_time_mlp_f32(const float* t, int B, const float* w0, const float* b0,
                               const float* w2, const float* b2, int D, float* work,
                               float* out, hipStream_t stream) {
  LX_REQUIRE(t && w0 && b0 && w2 && b2 && work && out, "time_mlp: null pointer");
  LX_REQUIRE(B > 0 && B <= kGemvBMax && D > 0 && D % 4 == 0, "time_mlp: bad shape");
  const int F = 256;  // SinusPositionEmbedding(256)
  float* sinus = work;
  float* hid = work + (long)B * F;
  int rc = lx_timestep_embed_f32(t, B, F / 2, 1000.0f, sinus, stream);
  if (rc) return rc;
  rc = gemv(sinus, B, F, w0, b0, hid, D, D, 0, /*act_out=silu*/ 1, stream);
  if (rc) return rc;
  return gemv(hid, B, D, w2, b2, out, D, D, 0, 0, stream);
}
