// Row-reduction ops: AdaLN-modulated LayerNorm (DiT) and RMSNorm (Qwen2).
//
// One wave64 owns one row at a time.  The row is read once into registers
// (float4 per lane per 256 channels), mean and centred variance are two
// shuffle reductions over those registers, and the output is written once:
// one HBM read + one HBM write per element, both with the streaming cache
// policy.  The (1 + scale) / shift vectors of the block's batches are staged in
// LDS once per workgroup.
//
// The modulated LayerNorms take a block of four waves over `gpb` consecutive
// groups of four rows (wave w: row w of each group): each wave requests its
// next row before it reduces and writes the current one, so that at large
// row counts the reads of one row overlap the writes of the previous one
// instead of every wave reading, then every wave writing.
#include "lx_common.hpp"
#include "lx_gemm_common.hpp"

namespace lx {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, 256 threads: 250 blocks at 1000 rows
// Row groups per block of the modulated LayerNorms: about three blocks per CU
// (768), at most kMaxGroups groups each.  B=2, T=3000 (1500 groups): 2 groups
// per block, AdaLN 9.8 -> 9.4 us and with the folded K slices 24.4 -> 22.4 us;
// 3 or 4 groups per block (500 / 375 blocks) 10.9-12.0 and 26.9 us.
constexpr int kRowBlocks = 768;
constexpr int kMaxGroups = 8;
inline int row_gpb(int rows) {
  const int groups = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int g = (groups + kRowBlocks / 2) / kRowBlocks;
  return g < 1 ? 1 : (g > kMaxGroups ? kMaxGroups : g);
}

template <int NV>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void adaln_kernel(
    const float* x, const float* __restrict__ shift,
    const float* __restrict__ scale, long mod_stride, float* y, int rows,
    int T, int D, float eps, int gpb) {
  // LDS: (1 + scale) and shift for the batches this block touches.
  extern __shared__ float smem[];
  const int D4 = D >> 2;
  const int row0 = blockIdx.x * gpb * kRowsPerBlock;
  const int rend = min(row0 + gpb * kRowsPerBlock, rows);
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  auto load_row = [&](float4* v, int row) {
    const float4* xr = reinterpret_cast<const float4*>(x + (long)min(row, rows - 1) * D);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + j * kWave;
      v[j] = i < D4 ? ld_nt(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  // Issue this wave's first row loads first so their latency overlaps the
  // modulation staging below.
  float4 v[NV], nv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) nv[j] = make_float4(0.f, 0.f, 0.f, 0.f);  // read by the last copy
  load_row(v, row0 + wave);
  const int b_first = row0 / T;
  const int nb = (rend - 1) / T - b_first + 1;
  for (int bi = 0; bi < nb; ++bi) {
    const float4* sc = reinterpret_cast<const float4*>(scale + (long)(b_first + bi) * mod_stride);
    const float4* sh = reinterpret_cast<const float4*>(shift + (long)(b_first + bi) * mod_stride);
    float4* s1 = reinterpret_cast<float4*>(smem + (2 * bi) * D);
    float4* s2 = reinterpret_cast<float4*>(smem + (2 * bi + 1) * D);
    for (int i = threadIdx.x; i < D4; i += blockDim.x) {
      float4 a = sc[i];
      s1[i] = make_float4(1.0f + a.x, 1.0f + a.y, 1.0f + a.z, 1.0f + a.w);
      s2[i] = sh[i];
    }
  }
  __syncthreads();
  for (int r = row0 + wave; r < rend; r += kRowsPerBlock) {
    // the next row's loads go out before this row is reduced and written
    if (r + kRowsPerBlock < rend) load_row(nv, r + kRowsPerBlock);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = wave_sum(s) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      int i = lane + j * kWave;
      if (i < D4) {
        float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
        q += (a * a + b * b) + (c * c + d * d);
      }
    }
    const float var = wave_sum(q) / (float)D;  // biased, as ggml_norm / nn.LayerNorm
    const float rstd = 1.0f / sqrtf(var + eps);
    const int bi = r / T - b_first;
    const float4* s1 = reinterpret_cast<const float4*>(smem + (2 * bi) * D);
    const float4* s2 = reinterpret_cast<const float4*>(smem + (2 * bi + 1) * D);
    float4* yr = reinterpret_cast<float4*>(y + (long)r * D);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      int i = lane + j * kWave;
      if (i < D4) {
        float4 m = s1[i], h = s2[i], o;
        o.x = ((v[j].x - mean) * rstd) * m.x + h.x;
        o.y = ((v[j].y - mean) * rstd) * m.y + h.y;
        o.z = ((v[j].z - mean) * rstd) * m.z + h.z;
        o.w = ((v[j].w - mean) * rstd) * m.w + h.w;
        st_nt(yr + i, o);
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = nv[j];
  }
}

// The gated residual of a K-split projection folded into the next modulated
// LayerNorm, one wave per row:
//   h[r] = h[r] + gate_b * ((P_0[r] + ... + P_{S-1}[r]) + bias)   (S >= 1)
//   y[r] = LN(h[r]) * (1 + scale_b) + shift_b                     (y != null)
// The partial products are summed in slice order; the residual update is the
// projection epilogue's own expression (h + (acc + bias) * gate).  The
// (1 + scale), shift and gate rows of the batches a block touches and the bias
// are staged in LDS.
template <int NV, int SMAX>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void adaln_resid_kernel(
    float* h, const float* P, int S, long pstride, const float* __restrict__ bias,
    const float* __restrict__ gate, long gate_stride, const float* __restrict__ shift,
    const float* __restrict__ scale, long mod_stride, float* y, int rows, int T, int D,
    float eps, int pk, int gpb) {
  extern __shared__ float smem[];
  const int D4 = D >> 2;
  const int row0 = blockIdx.x * gpb * kRowsPerBlock;
  const int rend = min(row0 + gpb * kRowsPerBlock, rows);
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  // a row and its partial rows, every load in flight before any is used
  auto load_row = [&](float4* v, float4 (*pv)[NV], int row) {
    const float4* hr = reinterpret_cast<const float4*>(h + (long)row * D);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + j * kWave;
      v[j] = i < D4 ? hr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int sl = 0; sl < SMAX; ++sl)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = lane + j * kWave;
        pv[sl][j] = sl < S && i < D4
                        ? ld_nt(reinterpret_cast<const float4*>(P + sl * pstride + (long)row * D) + i)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  };
  // The next row is prefetched while a row's operands take at most 16 float4
  // per lane (two such sets stay within 128 VGPRs); wider rows or more slices
  // load each row when its turn comes.
  constexpr bool PF = NV * (1 + SMAX) <= 16;
  constexpr int PS = SMAX > 0 ? SMAX : 1;
  float4 v[NV], pv[PS][NV];
  float4 nv[PF ? NV : 1], npv[PF ? PS : 1][PF ? NV : 1];
  if constexpr (PF) {  // read by the copy after a wave's last row
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      nv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int sl = 0; sl < PS; ++sl) npv[sl][j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  load_row(v, pv, min(row0 + wave, rows - 1));
  const int b_first = row0 / T;
  const int nb = (rend - 1) / T - b_first + 1;
  // LDS: per batch (1 + scale), shift, gate; then the bias
  float* sb = smem + 3 * nb * D;
  for (int bi = 0; bi < nb; ++bi) {
    const float4* sc = reinterpret_cast<const float4*>(scale + (long)(b_first + bi) * mod_stride);
    const float4* sh = reinterpret_cast<const float4*>(shift + (long)(b_first + bi) * mod_stride);
    const float4* ga = reinterpret_cast<const float4*>(gate + (long)(b_first + bi) * gate_stride);
    float4* s1 = reinterpret_cast<float4*>(smem + (3 * bi) * D);
    float4* s2 = reinterpret_cast<float4*>(smem + (3 * bi + 1) * D);
    float4* s3 = reinterpret_cast<float4*>(smem + (3 * bi + 2) * D);
    for (int i = threadIdx.x; i < D4; i += blockDim.x) {
      if (y) {
        const float4 a = sc[i];
        s1[i] = make_float4(1.0f + a.x, 1.0f + a.y, 1.0f + a.z, 1.0f + a.w);
        s2[i] = sh[i];
      }
      if (S > 0) s3[i] = ga[i];
    }
  }
  if (S > 0)
    for (int i = threadIdx.x; i < D4; i += blockDim.x)
      reinterpret_cast<float4*>(sb)[i] =
          bias ? reinterpret_cast<const float4*>(bias)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  for (int row = row0 + wave; row < rend; row += kRowsPerBlock) {
    // the next row's loads go out before this row is reduced and written
    if constexpr (PF) {
      if (row + kRowsPerBlock < rend) load_row(nv, npv, row + kRowsPerBlock);
    } else if (row != row0 + wave) {
      load_row(v, pv, row);
    }
    const int bi = row / T - b_first;
    float4* hr = reinterpret_cast<float4*>(h + (long)row * D);
    if (SMAX > 0 && S > 0) {
      const float4* g4 = reinterpret_cast<const float4*>(smem + (3 * bi + 2) * D);
      const float4* b4 = reinterpret_cast<const float4*>(sb);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = lane + j * kWave;
        if (i >= D4) continue;
        float4 a = pv[0][j];
#pragma unroll
        for (int sl = 1; sl < SMAX; ++sl)
          if (sl < S) a = make_float4(a.x + pv[sl][j].x, a.y + pv[sl][j].y, a.z + pv[sl][j].z,
                                      a.w + pv[sl][j].w);
        const float4 b = b4[i], g = g4[i];
        v[j] = make_float4(v[j].x + (a.x + b.x) * g.x, v[j].y + (a.y + b.y) * g.y,
                           v[j].z + (a.z + b.z) * g.z, v[j].w + (a.w + b.w) * g.w);
        hr[i] = v[j];
      }
    }
    if (y) {
      float sm = 0.0f;
#pragma unroll
      for (int j = 0; j < NV; ++j) sm += (v[j].x + v[j].y) + (v[j].z + v[j].w);
      const float mean = wave_sum(sm) / (float)D;
      float q = 0.0f;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = lane + j * kWave;
        if (i < D4) {
          const float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
          q += (a * a + b * b) + (c * c + d * d);
        }
      }
      const float var = wave_sum(q) / (float)D;  // biased, as ggml_norm / nn.LayerNorm
      const float rstd = 1.0f / sqrtf(var + eps);
      const float4* s1 = reinterpret_cast<const float4*>(smem + (3 * bi) * D);
      const float4* s2 = reinterpret_cast<const float4*>(smem + (3 * bi + 1) * D);
      float4* yr = reinterpret_cast<float4*>(y + (long)row * D);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = lane + j * kWave;
        if (i < D4) {
          const float4 m = s1[i], sh = s2[i];
          float4 o;
          o.x = ((v[j].x - mean) * rstd) * m.x + sh.x;
          o.y = ((v[j].y - mean) * rstd) * m.y + sh.y;
          o.z = ((v[j].z - mean) * rstd) * m.z + sh.z;
          o.w = ((v[j].w - mean) * rstd) * m.w + sh.w;
          if (pk)  // two-part packed row for the three-product GEMM
            reinterpret_cast<uintx4_t*>(yr)[i] = pack2_bf16(floatx4{o.x, o.y, o.z, o.w});
          else
            yr[i] = o;
        }
      }
    }
    if constexpr (PF) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        v[j] = nv[j];
#pragma unroll
        for (int sl = 0; sl < PS; ++sl) pv[sl][j] = npv[sl][j];
      }
    }
  }
}

template <int NV>
__global__ __launch_bounds__(kRowsPerBlock * kWave) void rmsnorm_kernel(
    const float* x, const float* __restrict__ w, float* y, int rows, int D, float eps) {
  extern __shared__ float smem[];
  const int D4 = D >> 2;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kRowsPerBlock + wave;
  const bool live = row < rows;
  const float4* xr = reinterpret_cast<const float4*>(x + (long)min(row, rows - 1) * D);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    int i = lane + j * kWave;
    v[j] = i < D4 ? ld_nt(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int i = threadIdx.x; i < D4; i += blockDim.x)
    reinterpret_cast<float4*>(smem)[i] = reinterpret_cast<const float4*>(w)[i];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    s += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  const float ms = wave_sum(s) / (float)D;
  const float r = 1.0f / sqrtf(ms + eps);
  __syncthreads();
  if (!live) return;
  float4* yr = reinterpret_cast<float4*>(y + (long)row * D);
  const float4* ws = reinterpret_cast<const float4*>(smem);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    int i = lane + j * kWave;
    if (i < D4) {
      float4 g = ws[i], o;
      o.x = (v[j].x * r) * g.x;
      o.y = (v[j].y * r) * g.y;
      o.z = (v[j].z * r) * g.z;
      o.w = (v[j].w * r) * g.w;
      st_nt(yr + i, o);
    }
  }
}

}  // namespace
}  // namespace lx

using namespace lx;

extern "C" int lx_adaln_modulate_f32(const float* x, const float* shift, const float* scale,
                                     long mod_stride, float* y, int B, int T, int D,
                                     float eps, hipStream_t stream) {
  LX_REQUIRE(x && shift && scale && y, "adaln: null pointer");
  LX_REQUIRE(B > 0 && T > 0 && D > 0, "adaln: bad shape B=%d T=%d D=%d", B, T, D);
  LX_REQUIRE(D % 4 == 0 && D <= 16 * 256, "adaln: D=%d must be a multiple of 4 and <= 4096", D);
  LX_REQUIRE((mod_stride == 0 || mod_stride >= D) && mod_stride % 4 == 0,
             "adaln: bad mod_stride %ld", mod_stride);
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)shift | (uintptr_t)scale) % 16 == 0,
             "adaln: pointers must be 16-byte aligned");
  const int rows = B * T;
  int gpb = row_gpb(rows);
  // A block's R = gpb * kRowsPerBlock rows touch at most ceil(R / T) + 1
  // batches; fewer groups per block where those batches' vectors would not fit.
  auto batches = [&](int g) {
    const int R = g * kRowsPerBlock;
    const int span = (T >= R) ? 2 : (R / T + 2);
    return span < B ? span : B;
  };
  while (gpb > 1 && (size_t)2 * batches(gpb) * D * sizeof(float) > 64 * 1024) --gpb;
  const size_t lds = (size_t)2 * batches(gpb) * D * sizeof(float);
  LX_REQUIRE(lds <= 64 * 1024, "adaln: T=%d too small for D=%d", T, D);
  const int rpb = gpb * kRowsPerBlock;
  const int nblk = (rows + rpb - 1) / rpb;
  const int nv = (D / 4 + kWave - 1) / kWave;
  if (nv <= 4)
    hipLaunchKernelGGL(adaln_kernel<4>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, shift, scale, mod_stride, y, rows, T, D, eps, gpb);
  else if (nv <= 8)
    hipLaunchKernelGGL(adaln_kernel<8>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, shift, scale, mod_stride, y, rows, T, D, eps, gpb);
  else
    hipLaunchKernelGGL(adaln_kernel<16>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, shift, scale, mod_stride, y, rows, T, D, eps, gpb);
  return check_launch("adaln_kernel");
}

namespace lx {
int adaln_resid(float* h, const float* partials, int splits, long partial_stride,
                const float* bias, const float* gate, long gate_stride, const float* shift,
                const float* scale, long mod_stride, float* y, int B, int T, int D, float eps,
                int out_packed, hipStream_t stream) {
  LX_REQUIRE(h && shift && scale, "adaln_resid: null pointer");
  LX_REQUIRE(B > 0 && T > 0 && D > 0, "adaln_resid: bad shape B=%d T=%d D=%d", B, T, D);
  LX_REQUIRE(D % 4 == 0 && D <= 16 * 256, "adaln_resid: D=%d must be a multiple of 4, <= 4096",
             D);
  LX_REQUIRE(splits >= 0 && splits <= 4, "adaln_resid: %d partial slices (at most 4)", splits);
  LX_REQUIRE(splits == 0 || (partials && gate && partial_stride >= (long)B * T * D &&
                             partial_stride % 4 == 0 && (gate_stride == 0 || gate_stride >= D) &&
                             gate_stride % 4 == 0),
             "adaln_resid: bad partials / gate");
  LX_REQUIRE(splits > 0 || y, "adaln_resid: nothing to do");
  LX_REQUIRE((mod_stride == 0 || mod_stride >= D) && mod_stride % 4 == 0,
             "adaln_resid: bad mod_stride %ld", mod_stride);
  LX_REQUIRE(((uintptr_t)h | (uintptr_t)y | (uintptr_t)shift | (uintptr_t)scale |
              (uintptr_t)partials | (uintptr_t)gate | (uintptr_t)bias) % 16 == 0,
             "adaln_resid: pointers must be 16-byte aligned");
  const int rows = B * T;
  int gpb = row_gpb(rows);
  auto batches = [&](int g) {
    const int R = g * kRowsPerBlock;
    const int span = (T >= R) ? 2 : (R / T + 2);
    return span < B ? span : B;
  };
  while (gpb > 1 && ((size_t)3 * batches(gpb) + 1) * D * sizeof(float) > 64 * 1024) --gpb;
  const size_t lds = ((size_t)3 * batches(gpb) + 1) * D * sizeof(float);
  LX_REQUIRE(lds <= 64 * 1024, "adaln_resid: T=%d too small for D=%d", T, D);
  const int rpb = gpb * kRowsPerBlock;
  const int nblk = (rows + rpb - 1) / rpb;
  LX_REQUIRE(splits == 0 || D <= 8 * 256, "adaln_resid: D=%d above 2048 with partials", D);
  const int nv = (D / 4 + kWave - 1) / kWave;
#define LX_AR(NVV, SM)                                                                          \
  hipLaunchKernelGGL((adaln_resid_kernel<NVV, SM>), dim3(nblk), dim3(kRowsPerBlock * kWave), lds,     \
                     stream, h, partials, splits, partial_stride, bias, gate, gate_stride, shift, \
                     scale, mod_stride, y, rows, T, D, eps, out_packed ? 1 : 0, gpb)
  if (nv <= 4 && splits <= 2)
    LX_AR(4, 2);
  else if (nv <= 4)
    LX_AR(4, 4);
  else if (nv <= 8 && splits <= 2)
    LX_AR(8, 2);
  else if (nv <= 8)
    LX_AR(8, 4);
  else
    LX_AR(16, 0);  // splits == 0 here
#undef LX_AR
  return check_launch("adaln_resid_kernel");
}
}  // namespace lx

extern "C" int lx_adaln_resid_f32(float* h, const float* partials, int splits,
                                  long partial_stride, const float* bias, const float* gate,
                                  long gate_stride, const float* shift, const float* scale,
                                  long mod_stride, float* y, int B, int T, int D, float eps,
                                  hipStream_t stream) {
  return adaln_resid(h, partials, splits, partial_stride, bias, gate, gate_stride, shift, scale,
                     mod_stride, y, B, T, D, eps, 0, stream);
}

extern "C" int lx_adaln_resid_packed_f32(float* h, const float* partials, int splits,
                                         long partial_stride, const float* bias,
                                         const float* gate, long gate_stride,
                                         const float* shift, const float* scale,
                                         long mod_stride, void* y, int B, int T, int D, float eps,
                                         hipStream_t stream) {
  LX_REQUIRE(y, "adaln_resid_packed: null output");
  return adaln_resid(h, partials, splits, partial_stride, bias, gate, gate_stride, shift, scale,
                     mod_stride, static_cast<float*>(y), B, T, D, eps, 1, stream);
}

extern "C" int lx_rmsnorm_f32(const float* x, const float* w, float* y, int rows, int D,
                              float eps, hipStream_t stream) {
  LX_REQUIRE(x && w && y, "rmsnorm: null pointer");
  LX_REQUIRE(rows > 0 && D > 0 && D % 4 == 0 && D <= 16 * 256, "rmsnorm: bad shape rows=%d D=%d",
             rows, D);
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)w) % 16 == 0,
             "rmsnorm: pointers must be 16-byte aligned");
  const int nblk = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const size_t lds = (size_t)D * sizeof(float);
  const int nv = (D / 4 + kWave - 1) / kWave;
  if (nv <= 4)
    hipLaunchKernelGGL(rmsnorm_kernel<4>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, w, y, rows, D, eps);
  else if (nv <= 8)
    hipLaunchKernelGGL(rmsnorm_kernel<8>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, w, y, rows, D, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<16>, dim3(nblk), dim3(kRowsPerBlock * kWave), lds, stream,
                       x, w, y, rows, D, eps);
  return check_launch("rmsnorm_kernel");
}
