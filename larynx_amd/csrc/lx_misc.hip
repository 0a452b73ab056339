// Layout kernels around the estimator: the Space A <-> Space B transposes of
// the DiT input/output (src/flow/dit.cpp:99-109, 139-140), the fused CFG +
// Euler update of the CFM loop (src/flow/flow.cpp:256-259), and small fills.
#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

// A[b*T + t, j]: j in [0,mel) x, [mel,2mel) cond, [2mel,3mel) mu, [3mel,4mel) spks.
// 32x32 tiles through LDS so both the (C, T) reads and the (T, 4C) writes
// are coalesced.  x rows of batch b start at b * xbs (0: one x for every row).
// With cfg set, cond / mu / spks are single (unbatched) tensors for batch 0 and
// zero for the other rows (the unconditional half of the CFG pair).
__global__ __launch_bounds__(256) void pack_input_kernel(const float* __restrict__ x, long xbs,
                                                         const float* __restrict__ cond,
                                                         const float* __restrict__ mu,
                                                         const float* __restrict__ spks, int cfg,
                                                         float* __restrict__ A, int T, int mel) {
  __shared__ float tile[32][33];
  const int b = blockIdx.z;
  const int src = blockIdx.y;  // 0 x, 1 cond, 2 mu, 3 spks
  const int ctiles = (mel + 31) / 32;
  const int ct = blockIdx.x % ctiles, tt = blockIdx.x / ctiles;
  const int c0 = ct * 32, t0 = tt * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const float* s = src == 0 ? x : src == 1 ? cond : mu;
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, t = t0 + tx;
    float v = 0.0f;
    if (c < mel && t < T && (src == 0 || !cfg || b == 0))
      v = src == 3   ? spks[(long)b * mel + c]
          : src == 0 ? s[(long)b * xbs + (long)c * T + t]
                     : s[((long)b * mel + c) * T + t];
    tile[i][tx] = v;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int t = t0 + i, c = c0 + tx;
    if (c < mel && t < T) A[((long)b * T + t) * (4 * mel) + src * mel + c] = tile[tx][i];
  }
}

// P (B*T, mel) -> dphi (B, mel, T)
__global__ __launch_bounds__(256) void unpack_output_kernel(const float* __restrict__ P,
                                                            float* __restrict__ out, int T,
                                                            int mel) {
  __shared__ float tile[32][33];
  const int b = blockIdx.z;
  const int ctiles = (mel + 31) / 32;
  const int ct = blockIdx.x % ctiles, tt = blockIdx.x / ctiles;
  const int c0 = ct * 32, t0 = tt * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int t = t0 + i, c = c0 + tx;
    tile[i][tx] = (c < mel && t < T) ? P[((long)b * T + t) * mel + c] : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, t = t0 + tx;
    if (c < mel && t < T) out[((long)b * mel + c) * T + t] = tile[tx][i];
  }
}

constexpr int kProjSlicesMax = 8;  // K slices the proj_out consumers sum

// Row t, column c of the proj_out rows: the K slices of a split-K product
// summed in slice order, then the bias (P itself when splits = 1, no bias).
// Every slice's load is issued before the first add (slices past `splits`
// re-read slice 0 and are dropped).
__device__ __forceinline__ float proj_row_val(const float* __restrict__ P, int splits, long slice,
                                              const float* __restrict__ bias, long idx, int c) {
  float p[kProjSlicesMax];
#pragma unroll
  for (int s = 0; s < kProjSlicesMax; ++s) p[s] = P[(s < splits ? s : 0) * slice + idx];
  float v = p[0];
#pragma unroll
  for (int s = 1; s < kProjSlicesMax; ++s)
    if (s < splits) v += p[s];
  return bias ? v + bias[c] : v;
}

// x[c, t] += dt * (a * P[t, c] - bb * P[T + t, c])
__global__ __launch_bounds__(256) void euler_kernel(float* __restrict__ x,
                                                    const float* __restrict__ P, int splits,
                                                    long slice, const float* __restrict__ bias,
                                                    int T, int mel, float dt, float a, float bb) {
  __shared__ float t0s[32][33], t1s[32][33];
  const int ctiles = (mel + 31) / 32;
  const int ct = blockIdx.x % ctiles, tt = blockIdx.x / ctiles;
  const int c0 = ct * 32, t0 = tt * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int t = t0 + i, c = c0 + tx;
    const bool ok = c < mel && t < T;
    t0s[i][tx] = ok ? proj_row_val(P, splits, slice, bias, (long)t * mel + c, c) : 0.0f;
    t1s[i][tx] = ok ? proj_row_val(P, splits, slice, bias, ((long)T + t) * mel + c, c) : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, t = t0 + tx;
    if (c < mel && t < T) {
      const float comb = a * t0s[tx][i] - bb * t1s[tx][i];
      float* xp = x + (long)c * T + t;
      *xp = *xp + dt * comb;
    }
  }
}

// P[r, c] = sum of the K slices (slice order) + bias[c]
__global__ void proj_reduce_kernel(const float* __restrict__ ws, int splits, long slice,
                                   const float* __restrict__ bias, float* __restrict__ P, int mel,
                                   long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    P[i] = proj_row_val(ws, splits, slice, bias, i, (int)(i % mel));
}

__global__ void fill_batch_kernel(float* dst, const float* __restrict__ src, long n, int copies,
                                  int zero_tail) {
  const long total = n * copies;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    const long j = i % n;
    dst[i] = (zero_tail && i >= n) ? 0.0f : src[j];
  }
}

__global__ void iota_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = i;
}

__global__ void fill_kernel(float* p, long n, float v) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void interleave_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                  float* __restrict__ out, int rows, int K) {
  const long n = (long)2 * rows * K;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    const long row = i / K;
    const int k = (int)(i - row * K);
    const long src = row >> 1;
    out[i] = (row & 1) ? b[src * K + k] : a[src * K + k];
  }
}


inline unsigned grid1d(long n) {
  long g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  if (g < 1) g = 1;
  return (unsigned)g;
}

}  // namespace

int dit_pack_input(const float* x, long x_bstride, const float* cond, const float* mu,
                   const float* spks, int cfg, float* A, int B, int T, int mel,
                   hipStream_t stream) {
  const int ctiles = (mel + 31) / 32, ttiles = (T + 31) / 32;
  hipLaunchKernelGGL(pack_input_kernel, dim3(ctiles * ttiles, 4, B), dim3(256), 0, stream, x,
                     x_bstride, cond, mu, spks, cfg, A, T, mel);
  return check_launch("pack_input_kernel");
}

int dit_unpack_output(const float* P, float* dphi, int B, int T, int mel, hipStream_t stream) {
  const int ctiles = (mel + 31) / 32, ttiles = (T + 31) / 32;
  hipLaunchKernelGGL(unpack_output_kernel, dim3(ctiles * ttiles, 1, B), dim3(256), 0, stream, P,
                     dphi, T, mel);
  return check_launch("unpack_output_kernel");
}

int cfm_euler_update(float* x, const float* P, int splits, long slice, const float* bias, int T,
                     int mel, float dt, float a, float b, hipStream_t stream) {
  LX_REQUIRE(splits >= 1 && splits <= kProjSlicesMax, "euler: %d K slices", splits);
  const int ctiles = (mel + 31) / 32, ttiles = (T + 31) / 32;
  hipLaunchKernelGGL(euler_kernel, dim3(ctiles * ttiles), dim3(256), 0, stream, x, P, splits,
                     slice, bias, T, mel, dt, a, b);
  return check_launch("euler_kernel");
}

int proj_reduce(const float* ws, int splits, long slice, const float* bias, float* P, int rows,
                int mel, hipStream_t stream) {
  LX_REQUIRE(splits >= 1 && splits <= kProjSlicesMax, "proj_reduce: %d K slices", splits);
  const long n = (long)rows * mel;
  hipLaunchKernelGGL(proj_reduce_kernel, dim3(grid1d(n)), dim3(256), 0, stream, ws, splits, slice,
                     bias, P, mel, n);
  return check_launch("proj_reduce_kernel");
}

int fill_batch(float* dst, const float* src, long n, int copies, int zero_tail,
               hipStream_t stream) {
  hipLaunchKernelGGL(fill_batch_kernel, dim3(grid1d(n * copies)), dim3(256), 0, stream, dst, src,
                     n, copies, zero_tail);
  return check_launch("fill_batch_kernel");
}

int iota_i32(int* p, int n, hipStream_t stream) {
  hipLaunchKernelGGL(iota_kernel, dim3(grid1d(n)), dim3(256), 0, stream, p, n);
  return check_launch("iota_kernel");
}

int fill_f32(float* p, long n, float value, hipStream_t stream) {
  hipLaunchKernelGGL(fill_kernel, dim3(grid1d(n)), dim3(256), 0, stream, p, n, value);
  return check_launch("fill_kernel");
}

int interleave_rows(const float* a, const float* b, float* out, int rows, int K,
                    hipStream_t stream) {
  hipLaunchKernelGGL(interleave_kernel, dim3(grid1d((long)2 * rows * K)), dim3(256), 0, stream, a,
                     b, out, rows, K);
  return check_launch("interleave_kernel");
}


}  // namespace lx
