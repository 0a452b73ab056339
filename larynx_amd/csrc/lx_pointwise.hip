// Pointwise / gather ops of the DiT block and the Qwen2 layer.  Each kernel
// is a single HBM pass: float4 loads and stores, grid-stride loops sized to
// keep every CU busy, tables (rotary inverse frequencies, sinusoid
// coefficients, token ids) passed by value in the kernel arguments.
#include <cmath>
#include <cstring>

#include "lx_common.hpp"

namespace lx {

void rope_inv_freq(float base, int dim, float* out) {
  for (int i = 0; i < dim / 2; ++i) {
    float e = (float)(2 * i) / (float)dim;
    float p = (float)std::pow((double)base, (double)e);
    out[i] = 1.0f / p;
  }
}

namespace {

template <int N>
struct Table {
  float v[N];
};

constexpr int kGatherChunk = 960;  // ids per launch: 3840 of the 4096 bytes of kernel arguments
struct IdChunk {
  int id[kGatherChunk];
};

inline int grid_for(long work, int block) {
  long g = (work + block - 1) / block;
  // 256 CUs x 8 resident blocks is plenty to saturate HBM; beyond that the
  // grid-stride loop takes over.
  if (g > 2048) g = 2048;
  if (g < 1) g = 1;
  return (int)g;
}

// Elementwise kernels process kUnroll float4 per thread per pass, with all
// loads issued before any arithmetic (memory-level parallelism on HBM).
constexpr int kUnroll = 4;
constexpr int kEwBlock = 256;

inline unsigned ew_grid(long n4) {
  long g = (n4 + (long)kEwBlock * kUnroll - 1) / ((long)kEwBlock * kUnroll);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return (unsigned)g;
}

__global__ __launch_bounds__(kEwBlock) void gelu_kernel(const float* h, float* y, long n4, long n) {
  const long stride = (long)gridDim.x * kEwBlock * kUnroll;
  for (long i0 = (long)blockIdx.x * kEwBlock * kUnroll + threadIdx.x; i0 < n4; i0 += stride) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long i = min(i0 + (long)u * kEwBlock, n4 - 1);
      v[u] = ld_nt(reinterpret_cast<const float4*>(h) + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long i = i0 + (long)u * kEwBlock;
      if (i < n4) {
        float4 o;
        o.x = gelu_tanh(v[u].x);
        o.y = gelu_tanh(v[u].y);
        o.z = gelu_tanh(v[u].z);
        o.w = gelu_tanh(v[u].w);
        st_nt(reinterpret_cast<float4*>(y) + i, o);
      }
    }
  }
  // scalar tail (n not a multiple of 4)
  long t = n4 * 4 + (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) y[t] = gelu_tanh(h[t]);
}

// x[row, :] += gate[row / T, :] * y[row, :].  Threads own float4 columns and
// walk rows (kUnroll rows in flight per thread), so the gate float4 and the
// batch index come from 32-bit row arithmetic, not a division per element.
__global__ __launch_bounds__(kEwBlock) void gated_residual_kernel(
    float* x, const float* __restrict__ y, const float* __restrict__ gate, long gate_stride,
    int rows, int T, int D4) {
  for (int c4 = threadIdx.x; c4 < D4; c4 += kEwBlock) {
    for (int r0 = blockIdx.x * kUnroll; r0 < rows; r0 += gridDim.x * kUnroll) {
      float4 a[kUnroll], v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const long i = (long)min(r0 + u, rows - 1) * D4 + c4;
        a[u] = ld_nt(reinterpret_cast<const float4*>(x) + i);
        v[u] = ld_nt(reinterpret_cast<const float4*>(y) + i);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int row = r0 + u;
        if (row < rows) {
          const float4 g = reinterpret_cast<const float4*>(gate + (long)(row / T) * gate_stride)[c4];
          a[u].x += v[u].x * g.x;
          a[u].y += v[u].y * g.y;
          a[u].z += v[u].z * g.z;
          a[u].w += v[u].w * g.w;
          st_nt(reinterpret_cast<float4*>(x) + (long)row * D4 + c4, a[u]);
        }
      }
    }
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

__global__ __launch_bounds__(kEwBlock) void swiglu_kernel(const float* __restrict__ gate,
                                                          const float* __restrict__ up,
                                                          float* out, long n4, long n) {
  const long stride = (long)gridDim.x * kEwBlock * kUnroll;
  for (long i0 = (long)blockIdx.x * kEwBlock * kUnroll + threadIdx.x; i0 < n4; i0 += stride) {
    float4 g[kUnroll], u4[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long i = min(i0 + (long)u * kEwBlock, n4 - 1);
      g[u] = ld_nt(reinterpret_cast<const float4*>(gate) + i);
      u4[u] = ld_nt(reinterpret_cast<const float4*>(up) + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long i = i0 + (long)u * kEwBlock;
      if (i < n4) {
        float4 o;
        o.x = silu_mul(g[u].x, u4[u].x);
        o.y = silu_mul(g[u].y, u4[u].y);
        o.z = silu_mul(g[u].z, u4[u].z);
        o.w = silu_mul(g[u].w, u4[u].w);
        st_nt(reinterpret_cast<float4*>(out) + i, o);
      }
    }
  }
  long t = n4 * 4 + (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) out[t] = silu_mul(gate[t], up[t]);
}

// Partial interleaved rotary over a 2-D grid: blockIdx.y = batch, blockIdx.x =
// a run of RB frames, thread = (frame in the run, pair).  No 64-bit index
// arithmetic; the q / k pair loads are issued before the position is read and
// the angle formed, and one sincos per pair serves both q and k (same
// position).  P = pairs per row rounded up to a power of two (<= 64).
template <int P>
__global__ __launch_bounds__(256) void rope_partial_kernel(float* q, float* k,
                                                           const int* __restrict__ pos, int T,
                                                           int ld, int half, Table<64> inv) {
  constexpr int RB = 256 / P;
  const int p = threadIdx.x % P;
  const int t = blockIdx.x * RB + threadIdx.x / P;
  if (t >= T || p >= half) return;
  const long row = (long)blockIdx.y * T + t;
  float2* pq = reinterpret_cast<float2*>(q + row * ld) + p;
  const float2 xq = ld_nt(pq);
  float2 xk = make_float2(0.f, 0.f);
  float2* pk = nullptr;
  if (k) {
    pk = reinterpret_cast<float2*>(k + row * ld) + p;
    xk = ld_nt(pk);
  }
  const float ang = (float)pos[t] * inv.v[p];
  float sn, cs;
  rope_sincos(ang, &sn, &cs);
  st_nt(pq, make_float2(xq.x * cs - xq.y * sn, xq.y * cs + xq.x * sn));
  if (k) st_nt(pk, make_float2(xk.x * cs - xk.y * sn, xk.y * cs + xk.x * sn));
}

// NEOX rotary: thread = (row, head, pair); pair (i, i + hd/2).
__global__ void rope_neox_kernel(float* qk, const int* __restrict__ pos, long rows,
                                 int n_heads, int hd, int ld, Table<64> inv) {
  const int half = hd / 2;
  const long n = rows * n_heads * half;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    long row = i / (n_heads * half);
    int rem = (int)(i - row * (n_heads * half));
    int h = rem / half;
    int p = rem - h * half;
    float ang = (float)pos[row] * inv.v[p];
    float s, c;
    rope_sincos(ang, &s, &c);
    float* ptr = qk + row * ld + h * hd + p;
    float x0 = __builtin_nontemporal_load(ptr), x1 = __builtin_nontemporal_load(ptr + half);
    __builtin_nontemporal_store(x0 * c - x1 * s, ptr);
    __builtin_nontemporal_store(x1 * c + x0 * s, ptr + half);
  }
}

__global__ void timestep_kernel(const float* __restrict__ t, int B, int half, float scale,
                                float* out, Table<256> coeff) {
  int b = blockIdx.x;
  float ts = scale * t[b];
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    float ang = ts * coeff.v[j];
    float s, c;
    sincosf(ang, &s, &c);
    out[(long)b * 2 * half + j] = s;
    out[(long)b * 2 * half + half + j] = c;
  }
}

// Gather: block per output row; bit-exact float copies.
__global__ void gather_kernel4(const float4* __restrict__ table, int D4, IdChunk ids,
                               float4* out) {
  const float4* src = table + (long)ids.id[blockIdx.x] * D4;
  float4* dst = out + (long)blockIdx.x * D4;
  for (int i = threadIdx.x; i < D4; i += blockDim.x) st_nt(dst + i, ld_nt(src + i));
}

__global__ void gather_kernel1(const float* __restrict__ table, int D, IdChunk ids,
                               float* out) {
  const float* src = table + (long)ids.id[blockIdx.x] * D;
  float* dst = out + (long)blockIdx.x * D;
  for (int i = threadIdx.x; i < D; i += blockDim.x) dst[i] = src[i];
}

}  // namespace

// Coefficients exactly as the reference host loop forms them
// (src/flow/flow_matching.cpp:14-17): fp32 product then expf.
void timestep_coeff(int half, float* c) {
  const float step = (float)(std::log(10000.0) / (double)(half - 1));
  for (int j = 0; j < half; ++j) c[j] = expf(-(float)j * step);
}

}  // namespace lx

using namespace lx;

extern "C" int lx_gelu_tanh_f32(const float* h, float* y, long n, hipStream_t stream) {
  LX_REQUIRE(h && y && n >= 0, "gelu: bad args");
  LX_REQUIRE(((uintptr_t)h | (uintptr_t)y) % 16 == 0, "gelu: pointers must be 16-byte aligned");
  if (n == 0) return LX_OK;
  long n4 = n / 4;
  hipLaunchKernelGGL(gelu_kernel, dim3(ew_grid(n4)), dim3(kEwBlock), 0, stream, h, y, n4, n);
  return check_launch("gelu_kernel");
}

extern "C" int lx_gated_residual_f32(float* x, const float* y, const float* gate,
                                     long gate_stride, int B, int T, int D,
                                     hipStream_t stream) {
  LX_REQUIRE(x && y && gate, "gated_residual: null pointer");
  LX_REQUIRE(B > 0 && T > 0 && D > 0 && D % 4 == 0, "gated_residual: bad shape");
  LX_REQUIRE((gate_stride == 0 || gate_stride >= D) && gate_stride % 4 == 0,
             "gated_residual: bad gate_stride");
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)gate) % 16 == 0,
             "gated_residual: pointers must be 16-byte aligned");
  LX_REQUIRE((long)B * T * (D / 4) < (1L << 31), "gated_residual: too many elements");
  const int rows = B * T;
  // kUnroll rows per block pass; D/4 columns over the block's threads
  long g = (rows + kUnroll - 1) / kUnroll;
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(gated_residual_kernel, dim3((unsigned)g), dim3(kEwBlock), 0, stream, x, y,
                     gate, gate_stride, rows, T, D / 4);
  return check_launch("gated_residual_kernel");
}

extern "C" int lx_swiglu_f32(const float* gate, const float* up, float* out, long n,
                             hipStream_t stream) {
  LX_REQUIRE(gate && up && out && n >= 0, "swiglu: bad args");
  LX_REQUIRE(((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) % 16 == 0,
             "swiglu: pointers must be 16-byte aligned");
  if (n == 0) return LX_OK;
  long n4 = n / 4;
  hipLaunchKernelGGL(swiglu_kernel, dim3(ew_grid(n4)), dim3(kEwBlock), 0, stream, gate, up, out,
                     n4, n);
  return check_launch("swiglu_kernel");
}

extern "C" int lx_rope_partial_interleaved_f32(float* q, float* k, const int* pos, int B,
                                               int T, int ld, int rot_dim, float base,
                                               hipStream_t stream) {
  LX_REQUIRE(q && pos, "rope_partial: null pointer");
  LX_REQUIRE(B > 0 && T > 0, "rope_partial: bad shape");
  LX_REQUIRE(rot_dim > 0 && rot_dim % 2 == 0 && rot_dim <= 128 && rot_dim <= ld,
             "rope_partial: rot_dim=%d must be even, <= 128 and <= ld=%d", rot_dim, ld);
  LX_REQUIRE(((uintptr_t)q % 8 == 0) && (k == nullptr || (uintptr_t)k % 8 == 0) && ld % 2 == 0,
             "rope_partial: pairs must be 8-byte aligned");
  Table<64> inv;
  std::memset(&inv, 0, sizeof(inv));
  rope_inv_freq(base, rot_dim, inv.v);
  LX_REQUIRE((long)B * T * ld < (1L << 40) && B <= 65535, "rope_partial: tensor too large");
  const int half = rot_dim / 2;
  const int P = half <= 8 ? 8 : half <= 16 ? 16 : half <= 32 ? 32 : 64;
  const int rb = 256 / P;
  dim3 grid((T + rb - 1) / rb, B);
#define LX_ROPE_CASE(PP)                                                                       \
  case PP:                                                                                     \
    hipLaunchKernelGGL(rope_partial_kernel<PP>, grid, dim3(256), 0, stream, q, k, pos, T, ld, \
                       half, inv);                                                             \
    break;
  switch (P) {
    LX_ROPE_CASE(8)
    LX_ROPE_CASE(16)
    LX_ROPE_CASE(32)
    LX_ROPE_CASE(64)
  }
#undef LX_ROPE_CASE
  return check_launch("rope_partial_kernel");
}

extern "C" int lx_rope_neox_f32(float* qk, const int* pos, int rows, int n_heads,
                                int head_dim, int ld, float theta, hipStream_t stream) {
  LX_REQUIRE(qk && pos, "rope_neox: null pointer");
  LX_REQUIRE(rows > 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 128,
             "rope_neox: bad shape");
  LX_REQUIRE(ld >= n_heads * head_dim, "rope_neox: ld=%d < n_heads*head_dim", ld);
  Table<64> inv;
  std::memset(&inv, 0, sizeof(inv));
  rope_inv_freq(theta, head_dim, inv.v);
  long n = (long)rows * n_heads * (head_dim / 2);
  hipLaunchKernelGGL(rope_neox_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, qk, pos,
                     (long)rows, n_heads, head_dim, ld, inv);
  return check_launch("rope_neox_kernel");
}

extern "C" int lx_timestep_embed_f32(const float* t, int B, int half_dim, float scale,
                                     float* out, hipStream_t stream) {
  LX_REQUIRE(t && out, "timestep_embed: null pointer");
  LX_REQUIRE(B > 0 && half_dim > 1 && half_dim <= 256, "timestep_embed: bad shape");
  Table<256> coeff;
  std::memset(&coeff, 0, sizeof(coeff));
  timestep_coeff(half_dim, coeff.v);
  hipLaunchKernelGGL(timestep_kernel, dim3(B), dim3(128), 0, stream, t, B, half_dim, scale, out,
                     coeff);
  return check_launch("timestep_kernel");
}

extern "C" int lx_embed_gather_f32(const float* table, long n_rows, int D, const int* ids,
                                   int n, float* out, hipStream_t stream) {
  LX_REQUIRE(table && out && (ids || n == 0), "embed_gather: null pointer");
  LX_REQUIRE(n_rows > 0 && D > 0 && n >= 0, "embed_gather: bad shape");
  for (int i = 0; i < n; ++i) {
    if (ids[i] < 0 || (long)ids[i] >= n_rows) {
      set_error("embed_gather: id %d at position %d outside [0, %ld)", ids[i], i, n_rows);
      return LX_ERR_RANGE;
    }
  }
  const bool vec = D % 4 == 0 && ((uintptr_t)table | (uintptr_t)out) % 16 == 0;
  for (int base = 0; base < n; base += kGatherChunk) {
    int cnt = n - base < kGatherChunk ? n - base : kGatherChunk;
    IdChunk chunk;
    std::memset(&chunk, 0, sizeof(chunk));
    std::memcpy(chunk.id, ids + base, sizeof(int) * cnt);
    if (vec)
      hipLaunchKernelGGL(gather_kernel4, dim3(cnt), dim3(256), 0, stream,
                         reinterpret_cast<const float4*>(table), D / 4, chunk,
                         reinterpret_cast<float4*>(out + (long)base * D));
    else
      hipLaunchKernelGGL(gather_kernel1, dim3(cnt), dim3(256), 0, stream, table, D, chunk,
                         out + (long)base * D);
    int rc = check_launch("gather_kernel");
    if (rc != LX_OK) return rc;
  }
  return LX_OK;
}
