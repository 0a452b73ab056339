// Scaled-dot-product attention, fp32 on the CDNA4 matrix cores.
//
// Prefill / DiT path (Tq > 1): one wave64 per (batch, head, 32-query tile).
// Scores are formed transposed, S^T = K Q^T, with v_mfma_f32_32x32x2f32 so
// that in the accumulator layout every lane owns ONE query column (lane & 31)
// and 16 keys of the 32-key block.  Row statistics of the online softmax are
// therefore per-lane scalars (plus one cross-half exchange), and the
// probabilities P^T already sit in the B-operand layout of the second MFMA,
// O^T += V^T P^T, with no transpose: accumulator register i of lane half h is
// key (i/4)*8 + h*4 + i%4, which is exactly the k index that lane half h
// contributes at MFMA step i.  Scores are never written to memory (the
// reference materialises KQ [T, T, heads, B]).
//
// Decode path (Tq == 1): flash-decoding.  Keys are split across workgroups
// (256 keys each, one thread per key for the scores, one lane per channel for
// P V), then a second kernel merges the per-split (max, sum, o) triples.
#include <cmath>

#include "lx_common.hpp"

namespace lx {
namespace {

constexpr int kHD = 64;  // head dim handled by these kernels

__global__ __launch_bounds__(64) void attn_mfma_kernel(
    const float* __restrict__ q, int ldq, const float* __restrict__ k, int ldk,
    const float* __restrict__ v, int ldv, float* __restrict__ o, int ldo, int Tq, int Tk,
    int H, int rep, float scale, int causal, int q_offset) {
  __shared__ __attribute__((aligned(16))) float Os[32 * (kHD + 4)];
  const int lane = threadIdx.x;
  const int r = lane & 31, h = lane >> 5;
  const int q0 = blockIdx.x * 32;
  const int head = blockIdx.y;
  const int b = blockIdx.z;
  const int g = head / rep;

  // Q^T operand: lane holds Q[q0 + r][h*32 + s] * scale, s = 0..31.
  float qf[32];
  {
    const float* qrow = q + ((long)b * Tq + min(q0 + r, Tq - 1)) * ldq + head * kHD + h * 32;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float4 t = reinterpret_cast<const float4*>(qrow)[j];
      qf[4 * j + 0] = t.x * scale;
      qf[4 * j + 1] = t.y * scale;
      qf[4 * j + 2] = t.z * scale;
      qf[4 * j + 3] = t.w * scale;
    }
  }
  const int my_q = q_offset + q0 + r;  // absolute position of this lane's query
  int kend = Tk;
  if (causal) kend = min(Tk, q_offset + min(q0 + 31, Tq - 1) + 1);

  floatx16 o0, o1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o0[i] = 0.0f;
    o1[i] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;

  const float* kbase = k + (long)b * Tk * ldk + g * kHD;
  const float* vbase = v + (long)b * Tk * ldv + g * kHD;
  for (int kb = 0; kb < kend; kb += 32) {
    float kf[32];
    const float* krow = kbase + (long)min(kb + r, Tk - 1) * ldk + h * 32;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float4 t = reinterpret_cast<const float4*>(krow)[j];
      kf[4 * j + 0] = t.x;
      kf[4 * j + 1] = t.y;
      kf[4 * j + 2] = t.z;
      kf[4 * j + 3] = t.w;
    }
    floatx16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j], qf[j], s, 0, 0, 0);

    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb + (i >> 2) * 8 + h * 4 + (i & 3);
      const bool ok = key < Tk && (!causal || key <= my_q);
      s[i] = ok ? s[i] : -INFINITY;
      mloc = fmaxf(mloc, s[i]);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = expf(m_run - m_new);  // 0 on the first block
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = expf(s[i] - m_new);
      psum += s[i];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] *= alpha;
      o1[i] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = min(kb + (i >> 2) * 8 + h * 4 + (i & 3), Tk - 1);
      const float* vrow = vbase + (long)key * ldv;
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[r], s[i], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 + r], s[i], o1, 0, 0, 0);
    }
  }
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l_tot;
  // O^T accumulator: register i of tile t is channel t*32 + (i/4)*8 + h*4 + i%4.
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int d = (i >> 2) * 8 + h * 4 + (i & 3);
    Os[r * (kHD + 4) + d] = o0[i] * inv;
    Os[r * (kHD + 4) + 32 + d] = o1[i] * inv;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int idx = lane + j * 64;  // 512 float4 = 32 rows x 16
    const int row = idx >> 4, c = (idx & 15) * 4;
    if (q0 + row < Tq) {
      float4 t = *reinterpret_cast<const float4*>(Os + row * (kHD + 4) + c);
      *reinterpret_cast<float4*>(o + ((long)b * Tq + q0 + row) * ldo + head * kHD + c) = t;
    }
  }
}

constexpr int kSplit = 256;  // keys per decode workgroup

// Partial pass: grid (H, n_split, B); 256 threads; thread = key for scores.
__global__ __launch_bounds__(256) void attn_decode_partial(
    const float* __restrict__ q, const float* __restrict__ k, int ldk,
    const float* __restrict__ v, int ldv, int Tk, int rep, float scale,
    float* __restrict__ part, int n_split, int ldq, int H) {
  __shared__ float qs[kHD];
  __shared__ float ps[kSplit];
  __shared__ float red[8];
  __shared__ float osum[4][kHD];
  const int head = blockIdx.x, sp = blockIdx.y, b = blockIdx.z;
  const int g = head / rep;
  const int tid = threadIdx.x;
  if (tid < kHD) qs[tid] = q[(long)b * ldq + head * kHD + tid] * scale;
  __syncthreads();
  const int key = sp * kSplit + tid;
  float sc = -INFINITY;
  if (key < Tk) {
    const float4* kr = reinterpret_cast<const float4*>(k + ((long)b * Tk + key) * ldk + g * kHD);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kHD / 4; ++j) {
      float4 t = kr[j];
      acc += (t.x * qs[4 * j] + t.y * qs[4 * j + 1]) + (t.z * qs[4 * j + 2] + t.w * qs[4 * j + 3]);
    }
    sc = acc;
  }
  // block max
  float m = wave_max(sc);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float p = key < Tk ? expf(sc - m) : 0.0f;
  ps[tid] = p;
  float l = wave_sum(p);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
  // P V: wave w sums keys w, w+4, ...; lane = channel.
  const int wave = tid >> 6, lane = tid & 63;
  float acc = 0.0f;
  const int nk = min(kSplit, Tk - sp * kSplit);
  for (int j = wave; j < nk; j += 4)
    acc += ps[j] * v[((long)b * Tk + sp * kSplit + j) * ldv + g * kHD + lane];
  osum[wave][lane] = acc;
  __syncthreads();
  float* out = part + (((long)b * H + head) * n_split + sp) * (kHD + 2);
  if (tid < kHD) out[tid] = (osum[0][tid] + osum[1][tid]) + (osum[2][tid] + osum[3][tid]);
  if (tid == 0) {
    out[kHD] = m;
    out[kHD + 1] = (red[4] + red[5]) + (red[6] + red[7]);
  }
}

__global__ __launch_bounds__(64) void attn_decode_merge(const float* __restrict__ part,
                                                        int n_split, float* __restrict__ o,
                                                        int ldo, int H) {
  const int head = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const float* p = part + ((long)b * H + head) * n_split * (kHD + 2);
  float m = -INFINITY;
  for (int s = 0; s < n_split; ++s) m = fmaxf(m, p[s * (kHD + 2) + kHD]);
  float l = 0.0f, acc = 0.0f;
  for (int s = 0; s < n_split; ++s) {
    const float w = expf(p[s * (kHD + 2) + kHD] - m);
    l += w * p[s * (kHD + 2) + kHD + 1];
    acc += w * p[s * (kHD + 2) + lane];
  }
  o[(long)b * ldo + head * kHD + lane] = acc / l;
}

}  // namespace

int attention_decode_split(const float* q, int ldq, const float* k, int ldk, const float* v,
                           int ldv, float* o, int ldo, int B, int Tk, int n_heads,
                           int n_kv_heads, float scale, float* part, hipStream_t stream) {
  const int rep = n_heads / n_kv_heads;
  const int n_split = (Tk + kSplit - 1) / kSplit;
  hipLaunchKernelGGL(attn_decode_partial, dim3(n_heads, n_split, B), dim3(256), 0, stream, q, k,
                     ldk, v, ldv, Tk, rep, scale, part, n_split, ldq, n_heads);
  int rc = check_launch("attn_decode_partial");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_decode_merge, dim3(n_heads, B), dim3(64), 0, stream, part, n_split, o,
                     ldo, n_heads);
  return check_launch("attn_decode_merge");
}

size_t attention_decode_part_floats(int B, int Tk, int n_heads) {
  return (size_t)B * n_heads * ((Tk + kSplit - 1) / kSplit) * (kHD + 2);
}

}  // namespace lx

using namespace lx;

extern "C" int lx_attention_f32(const float* q, int ldq, const float* k, int ldk,
                                const float* v, int ldv, float* o, int ldo, int B, int Tq,
                                int Tk, int n_heads, int n_kv_heads, int head_dim, float scale,
                                int causal, int q_offset, hipStream_t stream) {
  LX_REQUIRE(q && k && v && o, "attention: null pointer");
  LX_REQUIRE(B > 0 && Tq > 0 && Tk > 0 && n_heads > 0 && n_kv_heads > 0,
             "attention: bad shape");
  LX_REQUIRE(head_dim == kHD, "attention: head_dim=%d (only 64 is supported)", head_dim);
  LX_REQUIRE(n_heads % n_kv_heads == 0, "attention: n_heads %% n_kv_heads != 0");
  LX_REQUIRE(ldq >= n_heads * kHD && ldo >= n_heads * kHD && ldk >= n_kv_heads * kHD &&
                 ldv >= n_kv_heads * kHD,
             "attention: row strides too small");
  LX_REQUIRE(ldq % 4 == 0 && ldk % 4 == 0 && ldo % 4 == 0 &&
                 ((uintptr_t)q | (uintptr_t)k | (uintptr_t)o) % 16 == 0,
             "attention: q/k/o rows must be 16-byte aligned");
  LX_REQUIRE(q_offset >= 0, "attention: q_offset < 0");
  if (causal) LX_REQUIRE(q_offset + Tq <= Tk, "attention: causal needs q_offset + Tq <= Tk");
  const int rep = n_heads / n_kv_heads;
  dim3 grid((Tq + 31) / 32, n_heads, B);
  hipLaunchKernelGGL(attn_mfma_kernel, grid, dim3(64), 0, stream, q, ldq, k, ldk, v, ldv, o, ldo,
                     Tq, Tk, n_heads, rep, scale, causal, q_offset);
  return check_launch("attn_mfma_kernel");
}
