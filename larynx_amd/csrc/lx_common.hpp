// Shared helpers for the gfx950 kernels of liblxops: error plumbing, wave64
// reductions and the MFMA vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "lx_ops.h"

namespace lx {

constexpr int kWave = 64;  // CDNA wavefront width

// Thread-local last-error message backing lx_last_error().
void set_error(const char* fmt, ...);

// Checks hipGetLastError after a launch; records and returns LX_ERR_LAUNCH.
int check_launch(const char* what);

#define LX_REQUIRE(cond, ...)        \
  do {                               \
    if (!(cond)) {                   \
      ::lx::set_error(__VA_ARGS__);  \
      return LX_ERR_ARG;             \
    }                                \
  } while (0)

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// tanh-approximated GELU with the literal constants of the reference
// (src/flow/ops.cpp:75-82), evaluated in the same operation order.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c0 = 0.044715f;
  const float c1 = 0.7978845608028654f;
  float x3 = (x * x) * x;
  float inner = (x + x3 * c0) * c1;
  return (0.5f * x) * (tanhf(inner) + 1.0f);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Mish: x * tanh(softplus(x)), softplus = log1p(exp(x)), linear above 20
// (torch.nn.functional.softplus threshold).
__device__ __forceinline__ float mish(float x) {
  float sp = x > 20.0f ? x : log1pf(expf(x));
  return x * tanhf(sp);
}

// Host-side tables shared by the rotary paths: inv_freq[i] = 1 / base^(2i/dim)
// as fp32(pow) followed by an fp32 reciprocal, which reproduces torch's
// `1.0 / (base ** (arange(0, dim, 2).float() / dim))` bit for bit.
void rope_inv_freq(float base, int dim, float* out);

// Kernel-argument carrier for small per-launch tables (<= 64 entries).
struct FreqTable {
  float v[64];
};

}  // namespace lx
