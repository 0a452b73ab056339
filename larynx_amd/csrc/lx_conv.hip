// CausalConvPositionEmbedding half: left-padded grouped conv1d (groups of 64
// channels, kernel K) + bias + Mish (+ residual), as an implicit GEMM on the
// matrix cores.  Per (batch, group, 64-frame tile) the input window
// [64 + K - 1 frames x 64 channels] sits in LDS for the whole kernel and the
// 64x64 weight slab of each tap streams through a double-buffered LDS slot:
//   out[t, oc] = sum_k sum_ic window[t + k, ic] * w_k[oc, ic].
// Weights are pre-packed tap-major, wp[g][k][oc][ic], so each tap slab is a
// contiguous 16 KB read.
#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int CG = 64;        // channels per group
constexpr int TT = 64;        // frames per tile
constexpr int LDW = CG + 4;   // LDS row stride

template <int KMAX>
__global__ __launch_bounds__(256) void conv_mish_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ wp,
                                                        const float* __restrict__ bias,
                                                        const float* resid, float* y, int T,
                                                        int C, int K) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xw = smem;                           // [TT + KMAX - 1][LDW]
  float* wk = smem + (TT + KMAX - 1) * LDW;   // [2][CG][LDW]
  const int t0 = blockIdx.x * TT;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;

  // Input window: frames t0-(K-1) .. t0+TT-1, zero outside [0, T).
  const int nrow = TT + K - 1;
  for (int i = tid; i < nrow * (CG / 4); i += 256) {
    const int row = i / (CG / 4), c4 = (i % (CG / 4)) * 4;
    const int tg = t0 - (K - 1) + row;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tg >= 0 && tg < T)
      v = *reinterpret_cast<const float4*>(x + ((long)b * T + tg) * C + g * CG + c4);
    *reinterpret_cast<float4*>(xw + row * LDW + c4) = v;
  }
  const float* wg = wp + (long)g * K * CG * CG;
  // Tap slabs: 64 oc x 64 ic = 1024 float4, four per thread, register staged
  // (native vectors, no lambdas: keeps the staging in VGPRs).
  floatx4 wr0, wr1, wr2, wr3;
#define LX_WLOAD(k)                                                              \
  do {                                                                           \
    const floatx4* src = reinterpret_cast<const floatx4*>(wg + (long)(k) * CG * CG); \
    wr0 = src[tid];                                                              \
    wr1 = src[tid + 256];                                                        \
    wr2 = src[tid + 512];                                                        \
    wr3 = src[tid + 768];                                                        \
  } while (0)
#define LX_WSTORE(buf)                                                           \
  do {                                                                           \
    float* dst = wk + (buf) * CG * LDW;                                          \
    *reinterpret_cast<floatx4*>(dst + ((tid) >> 4) * LDW + ((tid) & 15) * 4) = wr0; \
    *reinterpret_cast<floatx4*>(dst + ((tid + 256) >> 4) * LDW + ((tid) & 15) * 4) = wr1; \
    *reinterpret_cast<floatx4*>(dst + ((tid + 512) >> 4) * LDW + ((tid) & 15) * 4) = wr2; \
    *reinterpret_cast<floatx4*>(dst + ((tid + 768) >> 4) * LDW + ((tid) & 15) * 4) = wr3; \
  } while (0)
  LX_WLOAD(0);
  LX_WSTORE(0);
  __syncthreads();

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int buf = k & 1;
    if (k + 1 < K) LX_WLOAD(k + 1);
    const float* a = xw + (wm * 32 + r + k) * LDW + h * 32;
    const float* w = wk + buf * CG * LDW + (wn * 32 + r) * LDW + h * 32;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const floatx4 av = *reinterpret_cast<const floatx4*>(a + 4 * j);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(w + 4 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], bv[e], acc, 0, 0, 0);
    }
    if (k + 1 < K) LX_WSTORE(buf ^ 1);
    __syncthreads();
  }
#undef LX_WLOAD
#undef LX_WSTORE
  // Epilogue through LDS (reuse the window region: TT x LDW floats).
  float* cs = smem;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = wm * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
    cs[row * LDW + wn * 32 + r] = acc[i];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = tid + 256 * j;
    const int row = idx >> 4, c4 = (idx & 15) * 4;
    const int t = t0 + row;
    if (t >= T) continue;
    float4 v = *reinterpret_cast<const float4*>(cs + row * LDW + c4);
    const int oc = g * CG + c4;
    const long off = ((long)b * T + t) * C + oc;
    v.x = mish(v.x + bias[oc + 0]);
    v.y = mish(v.y + bias[oc + 1]);
    v.z = mish(v.z + bias[oc + 2]);
    v.w = mish(v.w + bias[oc + 3]);
    if (resid) {
      float4 rr = *reinterpret_cast<const float4*>(resid + off);
      v.x = rr.x + v.x;
      v.y = rr.y + v.y;
      v.z = rr.z + v.z;
      v.w = rr.w + v.w;
    }
    *reinterpret_cast<float4*>(y + off) = v;
  }
}

// torch Conv1d weight (C, C/G, K) -> tap-major (G, K, C/G oc, C/G ic).
__global__ void conv_pack_kernel(const float* __restrict__ w, float* __restrict__ wp, int C,
                                 int G, int K) {
  const int cg = C / G;
  const long n = (long)C * cg * K;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    // destination index -> (g, k, oc_l, ic)
    long rem = i;
    const int ic = (int)(rem % cg);
    rem /= cg;
    const int ocl = (int)(rem % cg);
    rem /= cg;
    const int k = (int)(rem % K);
    const int g = (int)(rem / K);
    const int oc = g * cg + ocl;
    wp[i] = w[((long)oc * cg + ic) * K + k];
  }
}

}  // namespace

int conv_weight_pack(const float* w, float* wp, int C, int G, int K, hipStream_t stream) {
  LX_REQUIRE(w && wp && C > 0 && G > 0 && C % G == 0 && K > 0, "conv_weight_pack: bad args");
  long n = (long)C * (C / G) * K;
  long grid = (n + 255) / 256;
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(conv_pack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, wp, C, G, K);
  return check_launch("conv_pack_kernel");
}

int conv_pos_mish_packed(const float* x, const float* wp, const float* bias, const float* resid,
                         float* y, int B, int T, int C, int G, int K, hipStream_t stream) {
  LX_REQUIRE(x && wp && bias && y, "conv_pos_mish: null pointer");
  LX_REQUIRE(B > 0 && T > 0 && C > 0 && G > 0 && C % G == 0, "conv_pos_mish: bad shape");
  LX_REQUIRE(C / G == CG, "conv_pos_mish: channels per group must be 64 (got %d)", C / G);
  LX_REQUIRE(K >= 1 && K <= 32, "conv_pos_mish: kernel size %d not in [1, 32]", K);
  LX_REQUIRE(x != y, "conv_pos_mish: y must not alias x");
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)wp | (uintptr_t)(resid ? resid : x)) % 16 == 0,
             "conv_pos_mish: pointers must be 16-byte aligned");
  const size_t lds = ((size_t)(TT + 32 - 1) * LDW + 2 * CG * LDW) * sizeof(float);
  dim3 grid((T + TT - 1) / TT, G, B);
  hipLaunchKernelGGL(conv_mish_kernel<32>, grid, dim3(256), lds, stream, x, wp, bias, resid, y, T,
                     C, K);
  return check_launch("conv_mish_kernel");
}

}  // namespace lx

using namespace lx;

extern "C" int lx_conv_pack_weight_f32(const float* w, float* wp, int C, int G, int K,
                                       hipStream_t stream) {
  return conv_weight_pack(w, wp, C, G, K, stream);
}

extern "C" int lx_conv_pos_mish_f32(const float* x, const float* wp, const float* bias,
                                    const float* resid, float* y, int B, int T, int C, int G,
                                    int K, hipStream_t stream) {
  return conv_pos_mish_packed(x, wp, bias, resid, y, B, T, C, G, K, stream);
}
