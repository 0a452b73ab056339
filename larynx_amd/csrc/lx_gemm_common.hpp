// Shared pieces of the GEMM kernels (lx_gemm.hip, lx_gemm_bx.hip): the
// epilogue arguments and float4 epilogue, the bf16 operand-split helpers and
// the LDS chunk swizzle of the split-operand tiles.
#pragma once

#include "lx_common.hpp"

namespace lx {

struct EpiArgs {
  int kind;
  int vec;        // y, bias, gate rows 16-byte aligned: float4 epilogue path
  int pack_from;  // packed output: columns below it stay fp32
  int rows_per_batch;
  const float* gate;
  long gate_stride;
  const int* pos;
  int rot_dim, section, sections;
  float inv_freq[64];
};

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned uintx2_t __attribute__((ext_vector_type(2)));
typedef unsigned uintx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 bf16x4_back(bf16x4_t h);

// Two-part packed rows (the A operand of the three-product split-operand GEMM,
// written once by its producer): each aligned group of four fp32 values x as
// 16 bytes, the four leading parts bf16(x), then the four remainders
// bf16(x - bf16(x)) -- the same roundings as the GEMM's own split, in the
// bytes the fp32 group would occupy.  Contraction is off here: fused with the
// producer's last multiply (GELU's x * r, attention's sum * 1/l) the remainder
// would be taken from the unrounded product, not from the fp32 value.
__device__ __forceinline__ uintx4_t pack2_bf16(floatx4 v) {
#pragma clang fp contract(off)
  const bf16x4_t x0 = __builtin_convertvector(v, bf16x4_t);
  const bf16x4_t x1 = __builtin_convertvector(v - bf16x4_back(x0), bf16x4_t);
  const uintx2_t u0 = __builtin_bit_cast(uintx2_t, x0), u1 = __builtin_bit_cast(uintx2_t, x1);
  return uintx4_t{u0[0], u0[1], u1[0], u1[1]};
}

__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float ang) {
  float s, c;
  rope_sincos(ang, &s, &c);
  float a = x0 * c - x1 * s;
  float b = x1 * c + x0 * s;
  x0 = a;
  x1 = b;
}

// float4 epilogue of 4 columns n..n+3 (all < N) of row m with its operands
// already loaded: b = bias[n..n+3], g = gate row segment, yo = the residual.
// Same per-component operations as epilogue4.  PK: the result is stored as a
// two-part packed group (pack2_bf16) instead of four floats from column
// ep.pack_from on.
template <int EPI, bool PK = false>
__device__ __forceinline__ void epilogue4v(float* Y, int ldy, int m, int n, float4 v, float4 b,
                                           float4 g, float4 yo, int posm, const EpiArgs& ep) {
  float vv[4] = {v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w};
  if (EPI == LX_EPI_SWIGLU_PAIRED) {
    float2 o;
    o.x = (vv[0] / (1.0f + expf(-vv[0]))) * vv[1];
    o.y = (vv[2] / (1.0f + expf(-vv[2]))) * vv[3];
    *reinterpret_cast<float2*>(Y + (long)m * ldy + (n >> 1)) = o;
    return;
  }
  if (EPI == LX_EPI_GELU_TANH) {
#pragma unroll
    for (int e = 0; e < 4; ++e) vv[e] = gelu_tanh(vv[e]);
  }
  if (EPI == LX_EPI_ROPE_PARTIAL) {
    const int cs = n % ep.section;
    if (n < ep.sections * ep.section && cs < ep.rot_dim) {
      const float p = (float)posm;
      const int i0 = cs >> 1;
      rotate_pair(vv[0], vv[1], p * ep.inv_freq[i0]);
      rotate_pair(vv[2], vv[3], p * ep.inv_freq[i0 + 1]);
    }
  }
  float4 o = make_float4(vv[0], vv[1], vv[2], vv[3]);
  if (EPI == LX_EPI_GATED_RESID)
    o = make_float4(yo.x + vv[0] * g.x, yo.y + vv[1] * g.y, yo.z + vv[2] * g.z, yo.w + vv[3] * g.w);
  else if (EPI == LX_EPI_RESID)
    o = make_float4(yo.x + vv[0], yo.y + vv[1], yo.z + vv[2], yo.w + vv[3]);
  if (PK && n >= ep.pack_from)
    *reinterpret_cast<uintx4_t*>(Y + (long)m * ldy + n) = pack2_bf16(floatx4{o.x, o.y, o.z, o.w});
  else
    *reinterpret_cast<float4*>(Y + (long)m * ldy + n) = o;
}

typedef __bf16 sbf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ floatx16 mfma_split6x(const sbf16x8* a, const sbf16x8* b, floatx16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
}

__device__ __forceinline__ floatx4 bf16x4_back(bf16x4_t h) {
  const uintx2_t u = __builtin_bit_cast(uintx2_t, h);
  floatx4 f;
  f[0] = __uint_as_float(u[0] << 16);
  f[1] = __uint_as_float(u[0] & 0xffff0000u);
  f[2] = __uint_as_float(u[1] << 16);
  f[3] = __uint_as_float(u[1] & 0xffff0000u);
  return f;
}

constexpr int kSplitBK = 32;
// LDS rows of 32 bf16 (64 bytes, unpadded) whose four 16-byte chunks are
// XOR-swizzled by (row / 8) % 4: the staging stores (four rows per 256-byte
// pass) and the fragment reads (32 rows, one chunk each) both hit distinct
// banks.
constexpr int kSplitRS = kSplitBK;  // bf16 per LDS row
__device__ __forceinline__ int split_col(int row, int c) {
  return ((((c >> 3) ^ (row >> 3)) & 3) << 3) | (c & 7);
}

// Epilogue arguments of an lx_epilogue over N output columns.
int make_epi(const lx_epilogue* e, int N, EpiArgs* out);
// float4 epilogue: output rows, bias and gate rows 16-byte aligned.
bool epi_vec_ok(const EpiArgs& ep, const float* y, int ldy, const float* bias);

}  // namespace lx
