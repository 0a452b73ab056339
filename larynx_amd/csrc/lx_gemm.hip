// fp32 projection GEMM on the CDNA4 matrix cores: y = epi(x @ W^T + bias).
//
//   - v_mfma_f32_32x32x2f32, fp32 in / fp32 accumulate (no reduced-precision
//     shortcut: the reference pins fp32 GEMMs, cf. its TF32 ADR).
//   - 64x64 output tile per 256-thread workgroup, one 32x32 accumulator per
//     wave64; K staged through LDS in 32-wide slabs, double buffered, with the
//     next slab's global loads in flight during the current slab's MFMAs.
//   - Within a slab, lane half h consumes k = h*16 + s at MFMA step s, so each
//     lane's operands are 16 contiguous floats (four ds_read_b128).
//   - Workgroup ids are remapped so the tiles resident on one XCD are a
//     contiguous run down M for a few N columns: each XCD streams its own W
//     slabs through its own L2.
//   - The epilogue stages the accumulator tile in LDS, then every thread
//     processes row-contiguous float4s, which gives coalesced global traffic
//     and lets pairwise epilogues (rotary pairs, gate/up pairs) see both halves.
#include <cstring>

#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, PAD = 4;
constexpr int LDA = BK + PAD;  // LDS row stride (floats) of the A / W slabs
constexpr int LDC = BN + 4;    // LDS row stride of the epilogue tile

struct EpiArgs {
  int kind;
  int rows_per_batch;
  const float* gate;
  long gate_stride;
  const int* pos;
  int rot_dim, section, sections;
  float inv_freq[64];
};

__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float ang) {
  float s, c;
  sincosf(ang, &s, &c);
  float a = x0 * c - x1 * s;
  float b = x1 * c + x0 * s;
  x0 = a;
  x1 = b;
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_nt_kernel(const float* __restrict__ X, int ldx,
                                                      const float* __restrict__ W,
                                                      const float* __restrict__ bias, float* Y,
                                                      int ldy, int M, int N, int K,
                                                      EpiArgs ep) {
  __shared__ __attribute__((aligned(16))) float smem[2 * (BM + BN) * LDA];
  float* As = smem;                    // [2][BM][LDA]
  float* Ws = smem + 2 * BM * LDA;     // [2][BN][LDA]

  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int nwg = tiles_m * tiles_n;
  int id = blockIdx.x;
  const int full = (nwg / 8) * 8;
  if (id < full) id = (id % 8) * (full / 8) + id / 8;  // XCD-contiguous runs
  const int tm = id % tiles_m;
  const int tn = id / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;

  // Global -> LDS mapping: 2 float4 per thread per operand per slab.
  const int lrow = tid >> 3;       // 0..31 (+32 for the second float4)
  const int lc4 = (tid & 7) * 4;   // k offset within the slab
  const float* xa0 = X + (long)min(m0 + lrow, M - 1) * ldx;
  const float* xa1 = X + (long)min(m0 + lrow + 32, M - 1) * ldx;
  const float* wb0 = W + (long)min(n0 + lrow, N - 1) * K;
  const float* wb1 = W + (long)min(n0 + lrow + 32, N - 1) * K;
  const bool va0 = m0 + lrow < M, va1 = m0 + lrow + 32 < M;
  const bool vb0 = n0 + lrow < N, vb1 = n0 + lrow + 32 < N;

  float4 ra0, ra1, rb0, rb1;
  auto gload = [&](int k0) {
    const int k = k0 + lc4;
    const bool kin = k < K;  // K % 4 == 0, so a float4 is all-in or all-out
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    ra0 = (va0 && kin) ? *reinterpret_cast<const float4*>(xa0 + k) : z;
    ra1 = (va1 && kin) ? *reinterpret_cast<const float4*>(xa1 + k) : z;
    rb0 = (vb0 && kin) ? *reinterpret_cast<const float4*>(wb0 + k) : z;
    rb1 = (vb1 && kin) ? *reinterpret_cast<const float4*>(wb1 + k) : z;
  };
  auto sstore = [&](int buf) {
    float* a = As + buf * BM * LDA;
    float* w = Ws + buf * BN * LDA;
    *reinterpret_cast<float4*>(a + lrow * LDA + lc4) = ra0;
    *reinterpret_cast<float4*>(a + (lrow + 32) * LDA + lc4) = ra1;
    *reinterpret_cast<float4*>(w + lrow * LDA + lc4) = rb0;
    *reinterpret_cast<float4*>(w + (lrow + 32) * LDA + lc4) = rb1;
  };

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    const float* a = As + buf * BM * LDA + (wm * 32 + r) * LDA + h * 16;
    const float* w = Ws + buf * BN * LDA + (wn * 32 + r) * LDA + h * 16;
    float4 af[4], bf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      af[j] = *reinterpret_cast<const float4*>(a + 4 * j);
      bf[j] = *reinterpret_cast<const float4*>(w + 4 * j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[j].x, bf[j].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[j].y, bf[j].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[j].z, bf[j].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[j].w, bf[j].w, acc, 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: accumulator tile -> LDS (reusing the slab buffers).
  float* Cs = smem;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = wm * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
    Cs[row * LDC + wn * 32 + r] = acc[i];
  }
  __syncthreads();

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = tid + j * 256;
    const int row = idx >> 4;
    const int c = (idx & 15) * 4;
    const int m = m0 + row, n = n0 + c;
    if (m >= M || n >= N) continue;
    float4 v = *reinterpret_cast<const float4*>(Cs + row * LDC + c);
    float vv[4] = {v.x, v.y, v.z, v.w};
    const int nv = min(4, N - n);
    if (bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nv) vv[e] += bias[n + e];
    }
    if (EPI == LX_EPI_SWIGLU_PAIRED) {
      // columns (n, n+1) and (n+2, n+3) are (gate, up) pairs of outputs n/2, n/2+1
      float* yr = Y + (long)m * ldy + (n >> 1);
      if (nv >= 2) yr[0] = (vv[0] / (1.0f + expf(-vv[0]))) * vv[1];
      if (nv >= 4) yr[1] = (vv[2] / (1.0f + expf(-vv[2]))) * vv[3];
      continue;
    }
    if (EPI == LX_EPI_GELU_TANH) {
#pragma unroll
      for (int e = 0; e < 4; ++e) vv[e] = gelu_tanh(vv[e]);
    }
    if (EPI == LX_EPI_ROPE_PARTIAL) {
      const int cs = n % ep.section;
      if (n < ep.sections * ep.section && cs < ep.rot_dim) {
        const int t = m % ep.rows_per_batch;
        const float p = (float)ep.pos[t];
        const int i0 = cs >> 1;
        rotate_pair(vv[0], vv[1], p * ep.inv_freq[i0]);
        if (cs + 2 < ep.rot_dim) rotate_pair(vv[2], vv[3], p * ep.inv_freq[i0 + 1]);
      }
    }
    float* yp = Y + (long)m * ldy + n;
    if (EPI == LX_EPI_GATED_RESID) {
      const float* g = ep.gate + (long)(m / ep.rows_per_batch) * ep.gate_stride + n;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nv) yp[e] = yp[e] + vv[e] * g[e];
    } else if (EPI == LX_EPI_RESID) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nv) yp[e] = yp[e] + vv[e];
    } else if (nv == 4 && ((ldy & 3) == 0)) {
      *reinterpret_cast<float4*>(yp) = make_float4(vv[0], vv[1], vv[2], vv[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nv) yp[e] = vv[e];
    }
  }
}

// Skinny-M variant: one wave per output column pair, the M (<= 8) rows of x
// staged in LDS; weight-streaming like gemv.
constexpr int kSkinnyMax = 8;

template <int EPI>
__global__ __launch_bounds__(256) void gemv_epi_kernel(const float* __restrict__ X, int ldx,
                                                       const float* __restrict__ W,
                                                       const float* __restrict__ bias, float* Y,
                                                       int ldy, int M, int N, int K,
                                                       EpiArgs ep) {
  extern __shared__ float xs[];  // M * K
  for (int i = threadIdx.x; i < M * K; i += blockDim.x) {
    int m = i / K, k = i - m * K;
    xs[i] = X[(long)m * ldx + k];
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int K4 = K >> 2;
  const float4* xs4 = reinterpret_cast<const float4*>(xs);
  // each wave handles 2 adjacent columns (a rotary / gate-up pair) per step
  for (long n0 = ((long)blockIdx.x * 4 + wave) * 2; n0 < N; n0 += (long)gridDim.x * 8) {
    float acc[2][kSkinnyMax];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int m = 0; m < kSkinnyMax; ++m) acc[c][m] = 0.0f;
    for (int k4 = lane; k4 < K4; k4 += kWave) {
      float4 w0 = reinterpret_cast<const float4*>(W + n0 * K)[k4];
      float4 w1 = (n0 + 1 < N) ? reinterpret_cast<const float4*>(W + (n0 + 1) * K)[k4]
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int m = 0; m < kSkinnyMax; ++m) {
        if (m < M) {
          float4 xv = xs4[m * K4 + k4];
          acc[0][m] += (w0.x * xv.x + w0.y * xv.y) + (w0.z * xv.z + w0.w * xv.w);
          acc[1][m] += (w1.x * xv.x + w1.y * xv.y) + (w1.z * xv.z + w1.w * xv.w);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kSkinnyMax; ++m) {
      if (m >= M) break;
      float v0 = wave_sum(acc[0][m]);
      float v1 = wave_sum(acc[1][m]);
      if (lane != 0) continue;
      const bool has1 = n0 + 1 < N;
      if (bias) {
        v0 += bias[n0];
        if (has1) v1 += bias[n0 + 1];
      }
      if (EPI == LX_EPI_SWIGLU_PAIRED) {
        Y[(long)m * ldy + (n0 >> 1)] = (v0 / (1.0f + expf(-v0))) * v1;
        continue;
      }
      if (EPI == LX_EPI_GELU_TANH) {
        v0 = gelu_tanh(v0);
        v1 = gelu_tanh(v1);
      }
      if (EPI == LX_EPI_ROPE_PARTIAL) {
        const int cs = (int)(n0 % ep.section);
        if (n0 < (long)ep.sections * ep.section && cs < ep.rot_dim) {
          const float p = (float)ep.pos[m % ep.rows_per_batch];
          rotate_pair(v0, v1, p * ep.inv_freq[cs >> 1]);
        }
      }
      float* yp = Y + (long)m * ldy + n0;
      if (EPI == LX_EPI_GATED_RESID) {
        const float* g = ep.gate + (long)(m / ep.rows_per_batch) * ep.gate_stride + n0;
        yp[0] = yp[0] + v0 * g[0];
        if (has1) yp[1] = yp[1] + v1 * g[1];
      } else if (EPI == LX_EPI_RESID) {
        yp[0] = yp[0] + v0;
        if (has1) yp[1] = yp[1] + v1;
      } else {
        yp[0] = v0;
        if (has1) yp[1] = v1;
      }
    }
  }
}

int make_epi(const lx_epilogue* e, int N, EpiArgs* out) {
  std::memset(out, 0, sizeof(*out));
  out->kind = e ? e->kind : LX_EPI_NONE;
  out->rows_per_batch = 1;
  if (!e) return LX_OK;
  switch (e->kind) {
    case LX_EPI_NONE:
    case LX_EPI_GELU_TANH:
    case LX_EPI_RESID:
      break;
    case LX_EPI_GATED_RESID:
      LX_REQUIRE(e->gate && e->rows_per_batch > 0 && e->gate_stride >= 0,
                 "linear: GATED_RESID needs gate and rows_per_batch");
      out->rows_per_batch = e->rows_per_batch;
      out->gate = e->gate;
      out->gate_stride = e->gate_stride;
      break;
    case LX_EPI_ROPE_PARTIAL:
      LX_REQUIRE(e->pos && e->rows_per_batch > 0, "linear: ROPE needs pos and rows_per_batch");
      LX_REQUIRE(e->rot_dim > 0 && e->rot_dim % 4 == 0 && e->rot_dim <= 128,
                 "linear: ROPE rot_dim=%d must be a multiple of 4, <= 128", e->rot_dim);
      LX_REQUIRE(e->rope_section >= e->rot_dim && e->rope_section % 4 == 0 &&
                     e->rope_sections >= 1 && (long)e->rope_section * e->rope_sections <= N,
                 "linear: bad ROPE sections");
      out->rows_per_batch = e->rows_per_batch;
      out->pos = e->pos;
      out->rot_dim = e->rot_dim;
      out->section = e->rope_section;
      out->sections = e->rope_sections;
      rope_inv_freq(e->rope_base, e->rot_dim, out->inv_freq);
      break;
    case LX_EPI_SWIGLU_PAIRED:
      LX_REQUIRE(N % 2 == 0, "linear: SWIGLU_PAIRED needs even N");
      break;
    default:
      set_error("linear: unknown epilogue kind %d", e->kind);
      return LX_ERR_ARG;
  }
  return LX_OK;
}

}  // namespace

int gemv_epi(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
             int M, int N, int K, const lx_epilogue* epi, hipStream_t stream) {
  EpiArgs ep;
  int rc = make_epi(epi, N, &ep);
  if (rc) return rc;
  LX_REQUIRE(M >= 1 && M <= kSkinnyMax, "gemv_epi: M=%d", M);
  LX_REQUIRE((size_t)M * K * sizeof(float) <= 64 * 1024, "gemv_epi: M*K too large");
  long g = (N + 7) / 8;
  if (g > 4096) g = 4096;
  size_t lds = (size_t)M * K * sizeof(float);
#define LX_GEMV_CASE(E)                                                                      \
  case E:                                                                                    \
    hipLaunchKernelGGL(gemv_epi_kernel<E>, dim3((unsigned)g), dim3(256), lds, stream, x, ldx, \
                       W, bias, y, ldy, M, N, K, ep);                                         \
    break;
  switch (ep.kind) {
    LX_GEMV_CASE(LX_EPI_NONE)
    LX_GEMV_CASE(LX_EPI_GELU_TANH)
    LX_GEMV_CASE(LX_EPI_GATED_RESID)
    LX_GEMV_CASE(LX_EPI_ROPE_PARTIAL)
    LX_GEMV_CASE(LX_EPI_RESID)
    LX_GEMV_CASE(LX_EPI_SWIGLU_PAIRED)
  }
#undef LX_GEMV_CASE
  return check_launch("gemv_epi_kernel");
}

}  // namespace lx

using namespace lx;

extern "C" int lx_linear_f32(const float* x, int ldx, const float* W, const float* bias,
                             float* y, int ldy, int M, int N, int K, const lx_epilogue* epi,
                             hipStream_t stream) {
  LX_REQUIRE(x && W && y, "linear: null pointer");
  LX_REQUIRE(M > 0 && N > 0 && K > 0, "linear: bad shape M=%d N=%d K=%d", M, N, K);
  LX_REQUIRE(K % 4 == 0 && ldx % 4 == 0 && ldx >= K, "linear: K=%d and ldx=%d must be multiples of 4",
             K, ldx);
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)W) % 16 == 0, "linear: x and W must be 16-byte aligned");
  const int kind = epi ? epi->kind : LX_EPI_NONE;
  LX_REQUIRE(ldy >= (kind == LX_EPI_SWIGLU_PAIRED ? N / 2 : N), "linear: ldy=%d too small", ldy);
  if (M <= kSkinnyMax && (size_t)M * K * sizeof(float) <= 64 * 1024)
    return gemv_epi(x, ldx, W, bias, y, ldy, M, N, K, epi, stream);
  EpiArgs ep;
  int rc = make_epi(epi, N, &ep);
  if (rc) return rc;
  if (kind == LX_EPI_SWIGLU_PAIRED)
    LX_REQUIRE(ldy % 2 == 0, "linear: SWIGLU_PAIRED needs even ldy");
  const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  LX_REQUIRE(tiles < (1L << 31), "linear: too many tiles");
  dim3 grid((unsigned)tiles), block(256);
#define LX_GEMM_CASE(E)                                                                       \
  case E:                                                                                     \
    hipLaunchKernelGGL(gemm_nt_kernel<E>, grid, block, 0, stream, x, ldx, W, bias, y, ldy, M, \
                       N, K, ep);                                                             \
    break;
  switch (kind) {
    LX_GEMM_CASE(LX_EPI_NONE)
    LX_GEMM_CASE(LX_EPI_GELU_TANH)
    LX_GEMM_CASE(LX_EPI_GATED_RESID)
    LX_GEMM_CASE(LX_EPI_ROPE_PARTIAL)
    LX_GEMM_CASE(LX_EPI_RESID)
    LX_GEMM_CASE(LX_EPI_SWIGLU_PAIRED)
  }
#undef LX_GEMM_CASE
  return check_launch("gemm_nt_kernel");
}
