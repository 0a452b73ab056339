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
#include "lx_gemm_common.hpp"
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

// Split-operand form of the same implicit GEMM on the bf16 matrix cores
// (v_mfma_f32_32x32x16_bf16), the operand splits of gemm_bx_kernel: NP = 6
// (three bf16 parts per operand, the six products a_i w_j with i + j <= 2) or
// NP = 3 (two parts, a0 w0 + a0 w1 + a1 w0).
//   - The input window [TT + K - 1 frames x 64 channels] is split once into
//     NPL bf16 planes in LDS, rows padded to 144 bytes: any 16 consecutive
//     rows at one 16-byte chunk (the A-fragment reads of 16 lanes) start on
//     16 distinct 4-bank groups, and a fragment's address is the lane's base
//     plus a constant per (tap, row block, k step, part) — no swizzle
//     arithmetic in the tap loop.
//   - The weight is packed once in MFMA fragment order (conv_frag_pack_kernel):
//     per (group, tap, 32-channel output block, 16-channel k step) three 1 KB
//     parts of the 64 lanes' 16-byte B fragments; each wave streams its
//     block's fragments two taps ahead into registers (buffer loads, the
//     wave-uniform offset in a scalar register).  No LDS for the weight, no
//     barrier in the tap loop.
//   - 8 waves: wave w owns output channels 32 (w % 2) .. + 31 of all 64 frames
//     (two 32 x 32 accumulators) for the taps of group w / 2 (ceil(K / 4)
//     taps each); the four groups' partial tiles go to LDS together and the
//     epilogue sums them in a fixed order (group 3 first), then bias + Mish
//     (+ residual).
constexpr int kCbWaves = 8;
constexpr int kCbThreads = 64 * kCbWaves;
constexpr int kCbTapGroups = kCbWaves / 2;
constexpr int kCbWinRows = TT + 31;  // K <= 32
constexpr int kCbRS = CG + 8;        // bf16 per window row (144 bytes)

template <int NP>
constexpr size_t conv_bx_lds() {
  constexpr size_t win = (size_t)(NP == 6 ? 3 : 2) * kCbWinRows * kCbRS * 2;
  constexpr size_t red = (size_t)kCbTapGroups * TT * LDW * 4;  // the groups' partial tiles
  return win > red ? win : red;
}

typedef unsigned cb_uintx4 __attribute__((ext_vector_type(4)));

template <int NP>
__global__ __launch_bounds__(kCbThreads) void conv_bx_kernel(const float* __restrict__ x,
                                                             const __bf16* __restrict__ wf,
                                                             const float* __restrict__ bias,
                                                             const float* resid, float* y, int T,
                                                             int C, int K) {
  constexpr int NPL = NP == 6 ? 3 : 2;
  constexpr int PLANE = kCbWinRows * kCbRS;  // bf16 per plane
  extern __shared__ __attribute__((aligned(16))) __bf16 sw[];
  const int t0 = blockIdx.x * TT;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ob = wave & 1, tgrp = wave >> 1;
  const int r = lane & 31, h = lane >> 5;

  const int K0 = (K + kCbTapGroups - 1) / kCbTapGroups;
  const int kb = min(K, tgrp * K0), ke = min(K, kb + K0);
  // fragment (tap k, k step ks, part p) of this wave's output block at byte
  // ((g K + k) 24 + ob 12 + ks 3 + p) 1024 + 16 lane of wf (two blocks x 4
  // steps x 3 parts per tap); the host keeps wf below 2^31 bytes
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(wf), (short)0, (int)((long)gridDim.y * K * 24 * 1024), 0x00020000);
  const int wbase = (g * K * 24 + ob * 12) * 1024;
  const int wl = lane * 16;
  constexpr int kPa6[6] = {2, 1, 0, 1, 0, 0}, kPw6[6] = {0, 1, 2, 0, 1, 0};
  constexpr int kPa3[3] = {1, 0, 0}, kPw3[3] = {0, 1, 0};
  auto load_w = [&](cb_uintx4 (*wv)[3], int k) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int p = 0; p < NPL; ++p)
        wv[ks][p] = __builtin_bit_cast(
            cb_uintx4, __builtin_amdgcn_raw_buffer_load_b128(
                           wrs, wl, wbase + (k * 24 + ks * 3 + p) * 1024, 0));
  };
  // the first two taps' fragments are in flight while the window is staged
  cb_uintx4 w0[4][3], w1[4][3], w2[4][3];
  if (kb < ke) load_w(w0, kb);
  if (kb + 1 < ke) load_w(w1, kb + 1);

  // Window rows 0 .. TT + K - 2 hold frames t0 - (K - 1) + row (zero outside
  // [0, T)); every thread's loads are issued before its splits and stores.
  constexpr int kPer = (kCbWinRows * (CG / 4) + kCbThreads - 1) / kCbThreads;
  const int nwin = (TT + K - 1) * (CG / 4);
  {
    floatx4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = tid + u * kCbThreads;
      const int row = i >> 4, c4 = (i & 15) * 4;
      const int tf = t0 - (K - 1) + row;
      v[u] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (i < nwin && tf >= 0 && tf < T)
        v[u] = *reinterpret_cast<const floatx4*>(x + ((long)b * T + tf) * C + g * CG + c4);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = tid + u * kCbThreads;
      if (i >= nwin) continue;
      const int row = i >> 4, c4 = (i & 15) * 4;
      __bf16* dst = sw + row * kCbRS + c4;
      const bf16x4_t x0 = __builtin_convertvector(v[u], bf16x4_t);
      const floatx4 r1 = v[u] - bf16x4_back(x0);
      const bf16x4_t x1 = __builtin_convertvector(r1, bf16x4_t);
      *reinterpret_cast<bf16x4_t*>(dst) = x0;
      *reinterpret_cast<bf16x4_t*>(dst + PLANE) = x1;
      if (NPL == 3)
        *reinterpret_cast<bf16x4_t*>(dst + 2 * PLANE) =
            __builtin_convertvector(r1 - bf16x4_back(x1), bf16x4_t);
    }
  }
  __syncthreads();

  floatx16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
  // lane's A-fragment base: window row r, channels 8 h .. 8 h + 7
  const __bf16* abase = sw + r * kCbRS + h * 8;
  // tap k with its fragments in wc; the loads of tap k + 2 go into wn (the
  // set tap k - 1 has finished with): two taps of latency cover
  auto tap = [&](int k, cb_uintx4 (*wc)[3], cb_uintx4 (*wn)[3]) {
    if (k + 2 < ke) load_w(wn, k + 2);
    const __bf16* ak = abase + k * kCbRS;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      cb_uintx4 fa[2][3];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int p = 0; p < NPL; ++p)
          fa[rb][p] = *reinterpret_cast<const cb_uintx4*>(ak + rb * 32 * kCbRS + ks * 16 +
                                                          p * PLANE);
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(sbf16x8, fa[rb][NP == 6 ? kPa6[q] : kPa3[q]]),
              __builtin_bit_cast(sbf16x8, wc[ks][NP == 6 ? kPw6[q] : kPw3[q]]), acc[rb], 0, 0, 0);
    }
  };
  int k = kb;
  for (; k + 2 < ke; k += 3) {
    tap(k, w0, w2);
    tap(k + 1, w1, w0);
    tap(k + 2, w2, w1);
  }
  if (k < ke) tap(k, w0, w2);
  if (k + 1 < ke) tap(k + 1, w1, w0);
  __syncthreads();  // every wave is done with the window

  // Each tap group's partial tile into its own LDS region (over the window),
  // one barrier, then the epilogue sums them in a fixed order (group 3 first)
  // and adds bias + Mish (+ residual) over the 64 x 64 outputs.
  float* cs = reinterpret_cast<float*>(sw);
  {
    float* mine = cs + tgrp * TT * LDW;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = rb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        mine[row * LDW + ob * 32 + r] = acc[rb][i];
      }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TT * CG / 4 / kCbThreads; ++j) {
    const int idx = tid + kCbThreads * j;
    const int row = idx >> 4, c4 = (idx & 15) * 4;
    const int t = t0 + row;
    if (t >= T) continue;
    float4 v = *reinterpret_cast<const float4*>(cs + (kCbTapGroups - 1) * TT * LDW + row * LDW + c4);
#pragma unroll
    for (int grp = kCbTapGroups - 2; grp >= 0; --grp) {
      const float4 u = *reinterpret_cast<const float4*>(cs + grp * TT * LDW + row * LDW + c4);
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
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

// torch Conv1d weight (C, 64, K) -> MFMA fragment order for conv_bx_kernel:
// wf[((((g * K + k) * 2 + ob) * 4 + ks) * 3 + p) * 512 + l * 8 + j] = part p of
// w[oc = 64 g + 32 ob + l % 32][ic = 16 ks + (l / 32) * 8 + j][k] (the B
// operand of v_mfma_f32_32x32x16_bf16 for lane l; parts as gemm_bx's split).
__global__ void conv_frag_pack_kernel(const float* __restrict__ w, __bf16* __restrict__ wf, int G,
                                      int K) {
  const long total = (long)G * K * 2 * 4 * 64;
  const long t = blockIdx.x * 256L + threadIdx.x;
  if (t >= total) return;
  const int l = (int)(t % 64);
  long rest = t / 64;
  const int ks = (int)(rest % 4);
  rest /= 4;
  const int ob = (int)(rest % 2);
  rest /= 2;
  const int k = (int)(rest % K);
  const int g = (int)(rest / K);
  const int oc = g * CG + ob * 32 + l % 32;
  const int ic0 = ks * 16 + (l / 32) * 8;
  __bf16* dst = wf + ((((long)g * K + k) * 2 + ob) * 4 + ks) * 3 * 512 + l * 8;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    floatx4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = w[((long)oc * CG + ic0 + 4 * hh + e) * K + k];
    const bf16x4_t x0 = __builtin_convertvector(v, bf16x4_t);
    const floatx4 r1 = v - bf16x4_back(x0);
    const bf16x4_t x1 = __builtin_convertvector(r1, bf16x4_t);
    const bf16x4_t x2 = __builtin_convertvector(r1 - bf16x4_back(x1), bf16x4_t);
    *reinterpret_cast<bf16x4_t*>(dst + 4 * hh) = x0;
    *reinterpret_cast<bf16x4_t*>(dst + 512 + 4 * hh) = x1;
    *reinterpret_cast<bf16x4_t*>(dst + 1024 + 4 * hh) = x2;
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

int conv_frag_pack(const float* w, void* wf, int C, int G, int K, hipStream_t stream) {
  LX_REQUIRE(w && wf && C > 0 && G > 0 && C % G == 0 && C / G == CG && K >= 1 && K <= 32,
             "conv_frag_pack: bad args (C=%d G=%d K=%d; 64 channels per group, K <= 32)", C, G, K);
  LX_REQUIRE((uintptr_t)wf % 16 == 0, "conv_frag_pack: wf must be 16-byte aligned");
  const long total = (long)G * K * 2 * 4 * 64;
  hipLaunchKernelGGL(conv_frag_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     stream, w, static_cast<__bf16*>(wf), G, K);
  return check_launch("conv_frag_pack_kernel");
}

int conv_pos_mish_bx(const float* x, const void* wf, const float* bias, const float* resid,
                     float* y, int B, int T, int C, int G, int K, int products,
                     hipStream_t stream) {
  LX_REQUIRE(x && wf && bias && y, "conv_pos_mish_bx: null pointer");
  LX_REQUIRE(B > 0 && T > 0 && C > 0 && G > 0 && C % G == 0, "conv_pos_mish_bx: bad shape");
  LX_REQUIRE(C / G == CG, "conv_pos_mish_bx: channels per group must be 64 (got %d)", C / G);
  LX_REQUIRE(K >= 1 && K <= 32, "conv_pos_mish_bx: kernel size %d not in [1, 32]", K);
  LX_REQUIRE(products == 3 || products == 6, "conv_pos_mish_bx: products=%d must be 3 or 6",
             products);
  LX_REQUIRE(x != y, "conv_pos_mish_bx: y must not alias x");
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)wf | (uintptr_t)(resid ? resid : x)) % 16 ==
                 0,
             "conv_pos_mish_bx: pointers must be 16-byte aligned");
  LX_REQUIRE(G <= 65535 && B <= 65535 && (long)G * K * 24 * 1024 < (1L << 31),
             "conv_pos_mish_bx: grid or weight too large");
  const dim3 grid((T + TT - 1) / TT, G, B);
  static LdsLimit once[2];  // [six products]
  if (products == 3) {
    const int rc = raise_lds_limit((const void*)conv_bx_kernel<3>, conv_bx_lds<3>(), once[0],
                                   "conv_pos_mish_bx");
    if (rc) return rc;
    hipLaunchKernelGGL(conv_bx_kernel<3>, grid, dim3(kCbThreads), conv_bx_lds<3>(), stream, x,
                       static_cast<const __bf16*>(wf), bias, resid, y, T, C, K);
  } else {
    const int rc = raise_lds_limit((const void*)conv_bx_kernel<6>, conv_bx_lds<6>(), once[1],
                                   "conv_pos_mish_bx");
    if (rc) return rc;
    hipLaunchKernelGGL(conv_bx_kernel<6>, grid, dim3(kCbThreads), conv_bx_lds<6>(), stream, x,
                       static_cast<const __bf16*>(wf), bias, resid, y, T, C, K);
  }
  return check_launch("conv_bx_kernel");
}

}  // namespace lx

using namespace lx;

extern "C" int lx_conv_frag_pack_f32(const float* w, void* wf, int C, int G, int K,
                                     hipStream_t stream) {
  return conv_frag_pack(w, wf, C, G, K, stream);
}

extern "C" int lx_conv_pos_mish_bx_f32(const float* x, const void* wf, const float* bias,
                                       const float* resid, float* y, int B, int T, int C, int G,
                                       int K, int products, hipStream_t stream) {
  return conv_pos_mish_bx(x, wf, bias, resid, y, B, T, C, G, K, products, stream);
}

extern "C" int lx_conv_pack_weight_f32(const float* w, float* wp, int C, int G, int K,
                                       hipStream_t stream) {
  return conv_weight_pack(w, wp, C, G, K, stream);
}

extern "C" int lx_conv_pos_mish_f32(const float* x, const float* wp, const float* bias,
                                    const float* resid, float* y, int B, int T, int C, int G,
                                    int K, hipStream_t stream) {
  return conv_pos_mish_packed(x, wp, bias, resid, y, B, T, C, G, K, stream);
}
