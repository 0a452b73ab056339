// CausalConvPositionEmbedding half: left-padded grouped conv1d (groups of 64
// channels, kernel K) + bias + Mish (+ residual), as an implicit GEMM on the
// matrix cores.  Per (batch, group, 64-frame tile) the input window
// [64 + K - 1 frames x 64 channels] sits in LDS for the whole kernel and the
// 64x64 weight slab of each tap streams through a double-buffered LDS slot
// (one per tap group, see conv_mish_kernel):
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

// NG groups of 4 waves (2 x 2 waves of 32 x 32 outputs each).  With NG = 2 the
// groups split the taps, group 0 taps [0, K0), group 1 taps [K0, K) with
// K0 = ceil(K / 2), each with its own double-buffered tap slab, the input
// window shared: a grid of one workgroup per CU then has two waves per SIMD
// to hide the per-tap slab wait and barrier, and the two partial tiles are
// summed through LDS in a fixed order (group 1 then group 0).  Large grids
// (several workgroups per CU) take NG = 1, whose 43 KB of LDS fits three.
template <int KMAX, int NG>
__global__ __launch_bounds__(256 * NG) void conv_mish_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ wp,
                                                             const float* __restrict__ bias,
                                                             const float* resid, float* y, int T,
                                                             int C, int K) {
  constexpr int kConvGroups = NG;
  constexpr int kConvThreads = 256 * NG;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xw = smem;                           // [TT + KMAX - 1][LDW]
  const int t0 = blockIdx.x * TT;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = wave >> 2;                   // tap group
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;
  const int gtid = tid & 255;
  float* wk = smem + (TT + KMAX - 1) * LDW + kg * 2 * CG * LDW;  // this group's [2][CG][LDW]

  // Input window: frames t0-(K-1) .. t0+TT-1, zero outside [0, T); every
  // thread's loads are issued before its LDS stores.
  constexpr int kWin = (TT + KMAX - 1) * (CG / 4);                 // float4 slots (max)
  constexpr int kWinPer = (kWin + kConvThreads - 1) / kConvThreads;
  const int nwin = (TT + K - 1) * (CG / 4);
  {
    float4 v[kWinPer];
#pragma unroll
    for (int u = 0; u < kWinPer; ++u) {
      const int i = tid + u * kConvThreads;
      const int row = i / (CG / 4), c4 = (i % (CG / 4)) * 4;
      const int tg = t0 - (K - 1) + row;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < nwin && tg >= 0 && tg < T)
        v[u] = *reinterpret_cast<const float4*>(x + ((long)b * T + tg) * C + g * CG + c4);
    }
#pragma unroll
    for (int u = 0; u < kWinPer; ++u) {
      const int i = tid + u * kConvThreads;
      if (i < nwin) *reinterpret_cast<float4*>(xw + (i / (CG / 4)) * LDW + (i % (CG / 4)) * 4) = v[u];
    }
  }
  const int K0 = (K + NG - 1) / NG;
  const int kbeg = kg == 0 ? 0 : K0;
  const int kcnt = kg == 0 ? K0 : K - K0;     // this group's taps (K0 or K0 - 1)
  const float* wg = wp + (long)g * K * CG * CG;
  // Tap slabs: 64 oc x 64 ic = 1024 float4, four per thread of the group,
  // register staged (native vectors, no lambdas: keeps the staging in VGPRs).
  floatx4 wr0, wr1, wr2, wr3;
#define LX_WLOAD(k)                                                              \
  do {                                                                           \
    const floatx4* src = reinterpret_cast<const floatx4*>(wg + (long)(k) * CG * CG); \
    wr0 = src[gtid];                                                             \
    wr1 = src[gtid + 256];                                                       \
    wr2 = src[gtid + 512];                                                       \
    wr3 = src[gtid + 768];                                                       \
  } while (0)
#define LX_WSTORE(buf)                                                           \
  do {                                                                           \
    float* dst = wk + (buf) * CG * LDW;                                          \
    *reinterpret_cast<floatx4*>(dst + ((gtid) >> 4) * LDW + ((gtid) & 15) * 4) = wr0; \
    *reinterpret_cast<floatx4*>(dst + ((gtid + 256) >> 4) * LDW + ((gtid) & 15) * 4) = wr1; \
    *reinterpret_cast<floatx4*>(dst + ((gtid + 512) >> 4) * LDW + ((gtid) & 15) * 4) = wr2; \
    *reinterpret_cast<floatx4*>(dst + ((gtid + 768) >> 4) * LDW + ((gtid) & 15) * 4) = wr3; \
  } while (0)
  if (kcnt > 0) {
    LX_WLOAD(kbeg);
    LX_WSTORE(0);
  }
  __syncthreads();

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  // Both groups run K0 iterations (uniform barriers); a group with fewer taps
  // idles through its last one.
  for (int kk = 0; kk < K0; ++kk) {
    const int buf = kk & 1;
    const bool live = kk < kcnt;
    if (kk + 1 < kcnt) LX_WLOAD(kbeg + kk + 1);
    if (live) {
      const float* a = xw + (wm * 32 + r + kbeg + kk) * LDW + h * 32;
      const float* w = wk + buf * CG * LDW + (wn * 32 + r) * LDW + h * 32;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const floatx4 av = *reinterpret_cast<const floatx4*>(a + 4 * j);
        const floatx4 bv = *reinterpret_cast<const floatx4*>(w + 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], bv[e], acc, 0, 0, 0);
      }
    }
    if (kk + 1 < kcnt) LX_WSTORE(buf ^ 1);
    __syncthreads();
  }
#undef LX_WLOAD
#undef LX_WSTORE
  // Reduce the two tap groups through LDS (reuse the window region: TT x LDW
  // floats), group 1 first, then the epilogue over 64 x 64 outputs.
  float* cs = smem;
#pragma unroll
  for (int grp = kConvGroups - 1; grp >= 0; --grp) {
    if (kg == grp) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = wm * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        float v = acc[i];
        if (grp < kConvGroups - 1) v += cs[row * LDW + wn * 32 + r];
        cs[row * LDW + wn * 32 + r] = v;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < TT * CG / 4 / kConvThreads; ++j) {
    const int idx = tid + kConvThreads * j;
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
  dim3 grid((T + TT - 1) / TT, G, B);
  // Two tap groups when the grid gives each CU at most two workgroups
  // (T = 500: 256 workgroups, 48.5 -> 43.4 us); one otherwise (T = 3000: 1504
  // workgroups, three resident per CU: 230 us, against 242 with two groups).
  const bool two = (long)grid.x * grid.y * grid.z <= 2 * 256;
  const int ng = two ? 2 : 1;
  const size_t lds = ((size_t)(TT + 32 - 1) * LDW + (size_t)ng * 2 * CG * LDW) * sizeof(float);
  auto kern = two ? conv_mish_kernel<32, 2> : conv_mish_kernel<32, 1>;
  static LdsLimit once[2];  // [two]
  if (lds > 64 * 1024) {
    const int rc = raise_lds_limit((const void*)kern, lds, once[two], "conv_pos_mish");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(kern, grid, dim3(256 * ng), lds, stream, x, wp, bias, resid, y, T, C, K);
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
