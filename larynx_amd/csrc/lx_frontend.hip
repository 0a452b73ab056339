// Flow frontend kernels: the "run once per utterance" graph of
// FlowDecoder::infer (src/flow/flow.cpp:139-156) that turns speech tokens,
// the prompt mel and the speaker embedding into the CFM inputs mu, cond, spks.
//
//   spk   = spk_affine(l2_normalize(spk_embedding))          (ops.cpp:106-112)
//   embed = input_embedding[clamp(tokens, 0)]                 (flow.cpp:128-130, 150-151)
//   pre   = PreLookaheadLayer(embed)                          (prelookahead.cpp:8-20)
//           conv1 (k = 4, right pad 3) -> leaky_relu(0.01) -> conv2 (k = 3, left pad 2)
//           -> + embed
//   mu    = repeat_interleave(pre, 2) over time, as (mel, 2 Tseq)   (ops.cpp:114-122)
//   cond  = [prompt_feat^T | 0]  as (mel, MEL_T)              (flow.cpp:155-156)
//
// The two convolutions run as GEMMs on the matrix cores over im2col rows built
// here (k-major: row t holds x[t + k - pad_left][c] at column k * C + c), with
// the conv weights re-packed once to the same (OC, K * IC) order.
#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

// spk[o] = sum_k W[o, k] * x[k] / sqrt(max(sum_k x[k]^2, 1e-12)) + b[o].
// One workgroup: the norm is a block reduction, then one wave per output row.
__global__ __launch_bounds__(256) void spk_affine_kernel(const float* __restrict__ x, int K,
                                                         const float* __restrict__ W,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ y, int N) {
  __shared__ float part[4];
  __shared__ float xs[1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float s = 0.0f;
  for (int k = threadIdx.x; k < K; k += 256) {
    const float v = x[k];
    xs[k] = v;
    s += v * v;
  }
  s = wave_sum(s);
  if (lane == 0) part[wave] = s;
  __syncthreads();
  const float ss = (part[0] + part[1]) + (part[2] + part[3]);
  // ggml_clamp(sum_rows(sqr(x)), 1e-12, inf) then sqrt, then x / denom
  const float denom = sqrtf(fmaxf(ss, 1e-12f));
  for (int o = wave; o < N; o += 4) {
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc += W[(long)o * K + k] * (xs[k] / denom);
    acc = wave_sum(acc);
    if (lane == 0) y[o] = acc + b[o];
  }
}

// A[t, k*C + c] = x[t + k - pad_left, c] (zero outside [0, T)), optionally
// through leaky_relu(0.01).  One thread per float4 of A.
template <bool LEAKY>
__global__ __launch_bounds__(256) void im2col_kmajor_kernel(const float* __restrict__ x, int T,
                                                            int C, int Kw, int pad_left,
                                                            float* __restrict__ A) {
  const int C4 = C >> 2;
  const long n = (long)T * Kw * C4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    const int t = (int)(i / ((long)Kw * C4));
    const int rem = (int)(i - (long)t * Kw * C4);
    const int k = rem / C4, c4 = rem - k * C4;
    const int src = t + k - pad_left;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (src >= 0 && src < T) {
      v = reinterpret_cast<const float4*>(x + (long)src * C)[c4];
      if (LEAKY) {
        v.x = v.x > 0.0f ? v.x : 0.01f * v.x;
        v.y = v.y > 0.0f ? v.y : 0.01f * v.y;
        v.z = v.z > 0.0f ? v.z : 0.01f * v.z;
        v.w = v.w > 0.0f ? v.w : 0.01f * v.w;
      }
    }
    reinterpret_cast<float4*>(A + (long)t * Kw * C)[rem] = v;
  }
}

// mu[c, t'] = pre[t' / ratio, c] (t' < ratio * Tseq); cond[c, t'] =
// prompt_feat[t', c] for t' < mel_len1, else 0.  Both (mel, MEL_T).
__global__ __launch_bounds__(256) void pack_mu_cond_kernel(const float* __restrict__ pre,
                                                           int Tseq, int ratio,
                                                           const float* __restrict__ prompt_feat,
                                                           int mel_len1, int mel,
                                                           float* __restrict__ mu,
                                                           float* __restrict__ cond) {
  const int MT = Tseq * ratio;
  const long n = (long)mel * MT;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    const int c = (int)(i / MT), t = (int)(i - (long)c * MT);
    mu[i] = pre[(long)(t / ratio) * mel + c];
    cond[i] = t < mel_len1 ? prompt_feat[(long)t * mel + c] : 0.0f;
  }
}

// Conv1d weight (OC, IC, K) -> (OC, K * IC), column k * IC + ic.
__global__ __launch_bounds__(256) void conv_kmajor_pack_kernel(const float* __restrict__ w,
                                                               int OC, int IC, int K,
                                                               float* __restrict__ wp) {
  const long n = (long)OC * IC * K;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    const long oc = i / ((long)IC * K);
    const int rem = (int)(i - oc * IC * K);
    const int ic = rem / K, k = rem - ic * K;
    wp[oc * (long)K * IC + (long)k * IC + ic] = w[i];
  }
}

inline unsigned grid1d(long n) {
  long g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  if (g < 1) g = 1;
  return (unsigned)g;
}

}  // namespace

int flow_spk_affine(const float* x, int K, const float* W, const float* b, float* y, int N,
                    hipStream_t s) {
  LX_REQUIRE(x && W && b && y && K > 0 && K <= 1024 && N > 0, "spk_affine: bad args");
  hipLaunchKernelGGL(spk_affine_kernel, dim3(1), dim3(256), 0, s, x, K, W, b, y, N);
  return check_launch("spk_affine_kernel");
}

int flow_im2col(const float* x, int T, int C, int Kw, int pad_left, int leaky, float* A,
                hipStream_t s) {
  LX_REQUIRE(x && A && T > 0 && C > 0 && C % 4 == 0 && Kw > 0 && pad_left >= 0 &&
                 pad_left < Kw,
             "im2col: bad args");
  const long n = (long)T * Kw * (C / 4);
  if (leaky)
    hipLaunchKernelGGL(im2col_kmajor_kernel<true>, dim3(grid1d(n)), dim3(256), 0, s, x, T, C, Kw,
                       pad_left, A);
  else
    hipLaunchKernelGGL(im2col_kmajor_kernel<false>, dim3(grid1d(n)), dim3(256), 0, s, x, T, C, Kw,
                       pad_left, A);
  return check_launch("im2col_kmajor_kernel");
}

int flow_pack_mu_cond(const float* pre, int Tseq, int ratio, const float* prompt_feat,
                      int mel_len1, int mel, float* mu, float* cond, hipStream_t s) {
  LX_REQUIRE(pre && mu && cond && (prompt_feat || mel_len1 == 0) && Tseq > 0 && ratio > 0 &&
                 mel > 0 && mel_len1 >= 0 && mel_len1 <= Tseq * ratio,
             "pack_mu_cond: bad args");
  const long n = (long)mel * Tseq * ratio;
  hipLaunchKernelGGL(pack_mu_cond_kernel, dim3(grid1d(n)), dim3(256), 0, s, pre, Tseq, ratio,
                     prompt_feat, mel_len1, mel, mu, cond);
  return check_launch("pack_mu_cond_kernel");
}

int conv_kmajor_pack(const float* w, int OC, int IC, int K, float* wp, hipStream_t s) {
  LX_REQUIRE(w && wp && OC > 0 && IC > 0 && K > 0, "conv_kmajor_pack: bad args");
  hipLaunchKernelGGL(conv_kmajor_pack_kernel, dim3(grid1d((long)OC * IC * K)), dim3(256), 0, s, w,
                     OC, IC, K, wp);
  return check_launch("conv_kmajor_pack_kernel");
}

}  // namespace lx
