// Shared helpers for the gfx950 kernels of liblxops: error plumbing, wave64
// reductions and the MFMA vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
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

// Devices (ids 0-63) on which one kernel's dynamic-LDS limit has been raised.
struct LdsLimit {
  std::atomic<unsigned long long> devices{0};
};

// Raises `kern`'s dynamic LDS limit to `bytes` on the current device, once per
// device (the attribute belongs to each device's copy of the code object).
// Concurrent first calls may both set it, which is harmless.
inline int raise_lds_limit(const void* kern, size_t bytes, LdsLimit& once, const char* what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("%s: hipGetDevice failed", what);
    return LX_ERR_LAUNCH;
  }
  const unsigned long long bit = dev >= 0 && dev < 64 ? 1ull << dev : 0ull;
  if (bit && (once.devices.load(std::memory_order_acquire) & bit)) return LX_OK;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) !=
      hipSuccess) {
    set_error("%s: cannot raise the LDS limit to %zu bytes", what, bytes);
    return LX_ERR_LAUNCH;
  }
  once.devices.fetch_or(bit, std::memory_order_release);
  return LX_OK;
}

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Streaming float4 access with the non-temporal cache policy
// (global_load/store_dwordx4 ... nt) for data a kernel touches exactly once:
// on MI355X, read+write streams of 16-98 MB run 13-33% faster with it than
// with the default policy (the lines do not displace reused data in L2/MALL).
__device__ __forceinline__ float4 ld_nt(const float4* p) {
  float4 v;
  v.x = __builtin_nontemporal_load(&p->x);
  v.y = __builtin_nontemporal_load(&p->y);
  v.z = __builtin_nontemporal_load(&p->z);
  v.w = __builtin_nontemporal_load(&p->w);
  return v;
}
__device__ __forceinline__ void st_nt(float4* p, float4 v) {
  __builtin_nontemporal_store(v.x, &p->x);
  __builtin_nontemporal_store(v.y, &p->y);
  __builtin_nontemporal_store(v.z, &p->z);
  __builtin_nontemporal_store(v.w, &p->w);
}
__device__ __forceinline__ float2 ld_nt(const float2* p) {
  float2 v;
  v.x = __builtin_nontemporal_load(&p->x);
  v.y = __builtin_nontemporal_load(&p->y);
  return v;
}
__device__ __forceinline__ void st_nt(float2* p, float2 v) {
  __builtin_nontemporal_store(v.x, &p->x);
  __builtin_nontemporal_store(v.y, &p->y);
}

// Wave64 reductions without the LDS crossbar: DPP moves within each 16-lane
// row, then the gfx950 half-row / half-wave swaps.  Each step combines two
// groups that already hold uniform partial results (lane ^ 1, lane ^ 2, the
// other quad of each 8-lane half row, the other half of each row, lane ^ 16,
// lane ^ 32), and a + b == b + a, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each 16 lanes

// sin and cos of a rotary angle: Cody and Waite's additive argument reduction
// by 2*pi in two parts (the high part 6.28125 has 8 significant bits, so
// k * 6.28125 and the first subtraction are exact for |k| < 2^16; the low part
// carries the rest of 2*pi to fp32), then the hardware sine and cosine
// (v_sin_f32 / v_cos_f32, argument in revolutions) of the reduced angle in
// [-pi, pi].  Angles past 2^17 rad take the library sincosf.
__device__ __forceinline__ void rope_sincos(float a, float* s, float* c) {
  if (fabsf(a) < 131072.0f) {
    const float k = rintf(a * 0.159154937f);
    float r = fmaf(-k, 6.28125f, a);
    r = fmaf(-k, 1.93530717e-3f, r);
    const float rev = r * 0.159154937f;
    *s = __builtin_amdgcn_sinf(rev);
    *c = __builtin_amdgcn_cosf(rev);
  } else {
    sincosf(a, s, c);
  }
}

// Value held by lane ^ 16 / lane ^ 32.
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<kDppXor1>(v);
  v += dpp_mov<kDppXor2>(v);
  v += dpp_mov<kDppHalfMirror>(v);
  v += dpp_mov<kDppMirror>(v);
  v += lane_xor16(v);
  v += lane_xor32(v);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<kDppXor1>(v));
  v = fmaxf(v, dpp_mov<kDppXor2>(v));
  v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_mov<kDppMirror>(v));
  v = fmaxf(v, lane_xor16(v));
  v = fmaxf(v, lane_xor32(v));
  return v;
}

// tanh-approximated GELU, 0.5 x (1 + tanh(u)) with u = 0.7978845608028654 (x +
// 0.044715 x^3), the literal constants of the reference (src/flow/ops.cpp:75-82).
// It is evaluated through the identity 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)) with
// the hardware exp2 and reciprocal (each within about 1 ulp): a handful of VALU
// instructions instead of a full-range tanhf, so a standalone GELU pass stays
// memory bound.  Saturates cleanly: e^(-2u) -> inf gives -0, -> 0 gives x.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c0 = 0.044715f;
  const float c1 = 0.7978845608028654f;
  const float m2log2e = -2.8853900817779268f;  // -2 log2(e)
  float x3 = (x * x) * x;
  float u = (x + x3 * c0) * c1;
  float e = __builtin_amdgcn_exp2f(u * m2log2e);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Mish: x * tanh(softplus(x)), softplus = log1p(e^x).  With e^s = 1 + e^x,
// tanh(s) = (e^2s - 1) / (e^2s + 1) = n / (n + 2), n = e^x (e^x + 2): one
// hardware exp2 and one reciprocal (each within about 1 ulp) instead of
// log1pf, expf and tanhf, which made the conv epilogue a third of its launch.
// Above 20 (torch.nn.functional.softplus's threshold) the factor is 1.0f; far
// below zero e^x -> 0 gives x * 0.
__device__ __forceinline__ float mish(float x) {
  if (x > 20.0f) return x;
  const float e = __builtin_amdgcn_exp2f(x * 1.4426950408889634f);  // log2(e)
  const float n = e * (e + 2.0f);
  return x * (n * __builtin_amdgcn_rcpf(n + 2.0f));
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
