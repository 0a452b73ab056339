// Skinny products y = act_out(W @ act_in(x) + bias) for a handful of rows
// (B <= 16): the AdaLN modulation linears and the time-embedding MLP.  These
// are weight-streaming (HBM-bound on W), so each wave owns R output rows at a
// time, keeps R float4 weight loads in flight per lane, and reduces with
// wave64 shuffles.  The activations are staged in LDS with act_in applied.
#include <atomic>
#include <cstring>
#include <mutex>

#include "lx_common.hpp"
#include "lx_internal.hpp"

// Hidden layer of lx_time_mlp_f32_noalloc (B * D floats): a device array in
// place of the caller's workspace, for callers that cannot allocate.  Each
// device holds its own copy until the process ends; every call on a device
// shares it, so calls that overlap on one device race.  64 KiB covers every
// shape the second layer's GEMV accepts (B * D * 4 bytes of LDS <= 64 KiB).
constexpr long kTimeMlpScratchFloats = 16384;
static __device__ __align__(256) float scratch[kTimeMlpScratchFloats];

namespace lx {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kGemvRows = 4;
constexpr int kGemvBMax = 16;   // input rows of one launch
constexpr int kGemvBSmall = 8;  // below it the lighter instantiation (fewer accumulators)

// Dot products of the staged activations xs (B x K, LDS) with rows of W: each
// wave owns R output rows at a time (R = 4 streams large W with 4 rows of
// loads in flight per lane; R = 1 spreads a small W over more workgroups).
template <int R, int ACT_OUT, int BM>
__device__ __forceinline__ void gemv_rows(const float* xs, int B, int K,
                                          const float* __restrict__ W,
                                          const float* __restrict__ bias, float* __restrict__ y,
                                          long N, long ldy) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int K4 = K >> 2;
  const float4* xs4 = reinterpret_cast<const float4*>(xs);
  const long step = (long)gridDim.x * kGemvWaves * R;
  for (long n0 = ((long)blockIdx.x * kGemvWaves + wave) * R; n0 < N; n0 += step) {
    // bias first: its latency overlaps the weight stream
    float bv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) bv[r] = (bias && n0 + r < N) ? bias[n0 + r] : 0.0f;
    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < BM; ++b) acc[r][b] = 0.0f;
#pragma unroll 4
    for (int k4 = lane; k4 < K4; k4 += kWave) {
      float4 w[R];
      // weights are read exactly once per call: streaming cache policy
#pragma unroll
      for (int r = 0; r < R; ++r)
        w[r] = (n0 + r < N) ? ld_nt(reinterpret_cast<const float4*>(W + (n0 + r) * K) + k4)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        if (b < B) {
          float4 xv = xs4[b * K4 + k4];
#pragma unroll
          for (int r = 0; r < R; ++r)
            acc[r][b] += (w[r].x * xv.x + w[r].y * xv.y) + (w[r].z * xv.z + w[r].w * xv.w);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        if (b < B) {
          float s = wave_sum(acc[r][b]);
          if (lane == 0 && n0 + r < N) {
            float v = s + bv[r];
            if (ACT_OUT == 1) v = v / (1.0f + expf(-v));
            y[b * ldy + n0 + r] = v;
          }
        }
      }
    }
  }
}

template <int ACT_IN, int ACT_OUT, int R, int BM>
__global__ __launch_bounds__(kGemvWaves * kWave) void gemv_kernel(
    const float* __restrict__ x, int B, int K, const float* __restrict__ W,
    const float* __restrict__ bias, float* __restrict__ y, long N, long ldy) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // B * K
  // Stage act_in(x): float4 loads, all of a thread's loads issued before the
  // first LDS store (B * K is at most 16K floats: 16 float4 per thread).
  const int n4 = (B * K) >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  for (int i0 = threadIdx.x; i0 < n4; i0 += 4 * (int)blockDim.x) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * (int)blockDim.x;
      v[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * (int)blockDim.x;
      if (i < n4) {
        if (ACT_IN == 1) {
          v[u].x = v[u].x / (1.0f + expf(-v[u].x));
          v[u].y = v[u].y / (1.0f + expf(-v[u].y));
          v[u].z = v[u].z / (1.0f + expf(-v[u].z));
          v[u].w = v[u].w / (1.0f + expf(-v[u].w));
        }
        xs4[i] = v[u];
      }
    }
  }
  __syncthreads();
  gemv_rows<R, ACT_OUT, BM>(xs, B, K, W, bias, y, N, ldy);
}

// First layer of the time MLP with the sinusoidal embedding of t (a6) formed
// in LDS: xs[b, j] = sin(scale t_b c_j), xs[b, half + j] = cos(scale t_b c_j),
// the same expression as the standalone timestep kernel.  t comes from device
// memory (tdev) or, when tdev is null, from the kernel arguments.
struct TimeArgs {
  float c[128];  // c_j = exp(-j ln(1e4) / (half - 1))
  float t[kGemvBMax];
};

template <int BM>
__global__ __launch_bounds__(kGemvWaves * kWave) void time_mlp0_kernel(
    const float* __restrict__ tdev, TimeArgs ta, int B, int half, float scale,
    const float* __restrict__ W, const float* __restrict__ bias, float* __restrict__ y, long N) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // B * 2 half
  for (int i = threadIdx.x; i < B * half; i += blockDim.x) {
    const int b = i / half, j = i - b * half;
    const float ts = scale * (tdev ? tdev[b] : ta.t[b]);
    const float ang = ts * ta.c[j];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    xs[b * 2 * half + j] = sn;
    xs[b * 2 * half + half + j] = cs;
  }
  __syncthreads();
  gemv_rows<1, 1, BM>(xs, B, 2 * half, W, bias, y, N, N);
}

}  // namespace

int gemv(const float* x, int B, int K, const float* W, const float* bias, float* y, long N,
         long ldy, int act_in, int act_out, hipStream_t stream) {
  LX_REQUIRE(x && W && y, "gemv: null pointer");
  LX_REQUIRE(B > 0 && B <= kGemvBMax && K > 0 && K % 4 == 0 && N > 0,
             "gemv: bad shape B=%d K=%d N=%ld", B, K, N);
  LX_REQUIRE((size_t)B * K * sizeof(float) <= 64 * 1024, "gemv: B*K too large for LDS");
  LX_REQUIRE(((uintptr_t)W | (uintptr_t)x) % 16 == 0, "gemv: x and W must be 16-byte aligned");
  // Four rows per wave once there are enough rows to fill the device with
  // them (the stacked AdaLN projection), one row per wave below that (the
  // time MLP: 1024 rows -> 256 workgroups).
  const bool wide = N >= 4L * kGemvWaves * 256 * kGemvRows;
  long rows_per_block = (long)kGemvWaves * (wide ? kGemvRows : 1);
  long g = (N + rows_per_block - 1) / rows_per_block;
  if (g > 4096) g = 4096;
  dim3 grid((unsigned)g), block(kGemvWaves * kWave);
  size_t lds = (size_t)B * K * sizeof(float);
#define LX_GEMV_LAUNCH_BM(AI, AO, BM)                                                              \
  if (wide)                                                                                        \
    hipLaunchKernelGGL((gemv_kernel<AI, AO, kGemvRows, BM>), grid, block, lds, stream, x, B, K, W, \
                       bias, y, N, ldy);                                                           \
  else                                                                                             \
    hipLaunchKernelGGL((gemv_kernel<AI, AO, 1, BM>), grid, block, lds, stream, x, B, K, W, bias,   \
                       y, N, ldy);
#define LX_GEMV_LAUNCH(AI, AO)                    \
  if (B <= kGemvBSmall) {                         \
    LX_GEMV_LAUNCH_BM(AI, AO, kGemvBSmall)        \
  } else {                                        \
    LX_GEMV_LAUNCH_BM(AI, AO, kGemvBMax)          \
  }
  if (act_in == 0 && act_out == 0) {
    LX_GEMV_LAUNCH(0, 0)
  } else if (act_in == 1 && act_out == 0) {
    LX_GEMV_LAUNCH(1, 0)
  } else if (act_in == 0 && act_out == 1) {
    LX_GEMV_LAUNCH(0, 1)
  } else {
    LX_GEMV_LAUNCH(1, 1)
  }
#undef LX_GEMV_LAUNCH
#undef LX_GEMV_LAUNCH_BM
  return check_launch("gemv_kernel");
}

int time_mlp(const float* tdev, const float* thost, int B, const float* w0, const float* b0,
             const float* w2, const float* b2, int D, float* hid, float* out, hipStream_t stream) {
  LX_REQUIRE((tdev || thost) && w0 && b0 && w2 && b2 && hid && out, "time_mlp: null pointer");
  LX_REQUIRE(B > 0 && B <= kGemvBMax && D > 0 && D % 4 == 0, "time_mlp: bad shape");
  LX_REQUIRE(((uintptr_t)w0 | (uintptr_t)hid) % 16 == 0, "time_mlp: w0 and work must be 16-byte aligned");
  const int half = 128;  // SinusPositionEmbedding(256)
  TimeArgs ta;
  std::memset(&ta, 0, sizeof(ta));
  timestep_coeff(half, ta.c);
  if (!tdev)
    for (int b = 0; b < B; ++b) ta.t[b] = thost[b];
  const long rows_per_block = kGemvWaves;  // one row per wave
  const long g = (D + rows_per_block - 1) / rows_per_block;
  if (B <= kGemvBSmall)
    hipLaunchKernelGGL(time_mlp0_kernel<kGemvBSmall>, dim3((unsigned)g), dim3(kGemvWaves * kWave),
                       (size_t)B * 2 * half * sizeof(float), stream, tdev, ta, B, half, 1000.0f,
                       w0, b0, hid, (long)D);
  else
    hipLaunchKernelGGL(time_mlp0_kernel<kGemvBMax>, dim3((unsigned)g), dim3(kGemvWaves * kWave),
                       (size_t)B * 2 * half * sizeof(float), stream, tdev, ta, B, half, 1000.0f,
                       w0, b0, hid, (long)D);
  LX_TRY(check_launch("time_mlp0_kernel"));
  return gemv(hid, B, D, w2, b2, out, D, D, 0, 0, stream);
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
  LX_REQUIRE(t && work, "time_mlp: null pointer");
  // work: B * (256 + D) floats; the hidden layer uses the last B * D of them.
  return time_mlp(t, nullptr, B, w0, b0, w2, b2, D, work + (long)B * 256, out, stream);
}

namespace {

constexpr int kScratchDevices = 64;
std::atomic<float*> g_scratch_addr[kScratchDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up once per device
// with that device current (each device's copy lives at its own address; the
// array's name in host code is only a handle for the lookup).
int scratch_address(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("time_mlp_noalloc: hipGetDevice failed");
    return LX_ERR_LAUNCH;
  }
  LX_REQUIRE(dev >= 0 && dev < kScratchDevices, "time_mlp_noalloc: device %d out of range", dev);
  float* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !addr) {
        set_error("time_mlp_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
        return LX_ERR_LAUNCH;
      }
      p = static_cast<float*>(addr);
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return LX_OK;
}

}  // namespace

extern "C" int lx_time_mlp_f32_noalloc(const float* t, int B, const float* w0, const float* b0,
                                       const float* w2, const float* b2, int D, float* out,
                                       hipStream_t stream) {
  LX_REQUIRE(t, "time_mlp_noalloc: null pointer");
  LX_REQUIRE(B > 0 && D > 0 && (long)B * D <= kTimeMlpScratchFloats,
             "time_mlp_noalloc: B*D = %ld exceeds the %ld-float device scratch", (long)B * D,
             kTimeMlpScratchFloats);
  float* hid = nullptr;
  LX_TRY(scratch_address(&hid));
  // Every element of the hidden layer is written by the first layer's kernel
  // before the second reads it: nothing has to start at zero.
  return time_mlp(t, nullptr, B, w0, b0, w2, b2, D, hid, out, stream);
}
