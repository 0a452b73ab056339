// Qwen2 single-token decode kernels (one row of activations, batch 1).
//
// The decode step is a weight stream: 59.6 MB of fp32 weights per layer and a
// few KB of activations.  Each projection is one launch in which every wave
// owns R output rows, issues all R x NL float4 weight loads of its rows at once
// (the K dimension is split over the 64 lanes, NL float4 per lane), and
// reduces with wave64 shuffles.  What the reference runs as separate ggml nodes
// around each projection is folded into the projection's launch:
//   - RMSNorm of the input row (src/llm/ops.cpp:7-11) is recomputed by every
//     wave from its own slice of x (no normalised copy is written);
//   - q/k/v bias, NEOX rotary on q and k (src/llm/ops.cpp:21-30) and the KV
//     cache append (src/llm/llm.cpp:200-204) happen in the QKV epilogue;
//   - silu(gate) * up (src/llm/llm.cpp:284-288) in the gate/up epilogue;
//   - the residual adds (src/llm/llm.cpp:281, 289) in the o / down epilogues.
// Attention over the cache is split-key GQA: one workgroup per (64-key split,
// kv head) scores all query heads of its group, then one workgroup per query
// head merges the partial softmax states; while the whole cache fits one split
// the first pass writes the output and the merge pass is left out.
//
// The position (= cache length before the token) is read from device memory,
// so one capture of a layer stack into a HIP graph serves every position.
#include <cmath>

#include "lx_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int kHD = 64;      // head_dim
constexpr int kKeys = 64;    // keys per attention split
constexpr int kMaxRep = 8;   // query heads per kv head
constexpr int kMergePerWave = 16;  // splits per merge wave: <= 64 splits, 4096 keys

__device__ __forceinline__ float dot4(float4 a, float4 b) {
  return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
}

// Row mapping of wave `gw`, slot r (0 <= r < R).
template <int EPI, int R>
__device__ __forceinline__ long dec_row(long gw, int r) {
  if (EPI == DEC_QKV_ROPE) {
    // columns (c, c+1, c+32, c+33) of one 64-wide head: the two NEOX pairs
    // (c, c+32) and (c+1, c+33) land in the same wave
    const long head = gw >> 4;
    const int c = (int)(gw & 15) * 2;
    return head * kHD + c + (r & 1) + (r >> 1) * (kHD / 2);
  }
  return gw * R + r;
}

template <int EPI, int R, int NL, bool NORM>
__global__ __launch_bounds__(256) void dec_gemv_kernel(DecGemvArgs a) {
  static_assert(R == 1 || R == 2 || R == 4, "R must be a power of two <= 4");
  const int lane = threadIdx.x & 63;
  const long gw = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int K4 = a.K >> 2;
  long rows[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rows[r] = dec_row<EPI, R>(gw, r);
    live[r] = rows[r] < a.N;
  }
  if (!live[0]) return;
  // the rotary table (one entry per lane) is requested first, so waiting for
  // it does not wait for the weight stream (loads retire in order)
  float inv_lane = 0.0f;
  if (EPI == DEC_QKV_ROPE) inv_lane = a.inv_freq[lane & 31];
  // weight stream first: every load of the wave's rows in flight together,
  // with the streaming cache policy (1.46 GB of weights per token cannot stay
  // cached).
  // Loads are unconditional (row and k clamped into the matrix) so none of
  // them waits behind a branch; lanes past K see x = 0, rows past N are
  // discarded.
  float4 w[R][NL];
  const float4* W4 = reinterpret_cast<const float4*>(a.W);
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NL; ++j)
      w[r][j] = ld_nt(W4 + min(rows[r], a.N - 1) * K4 + min(lane + j * 64, K4 - 1));
  // everything the epilogue reads is requested before the first wait
  int pos = 0;
  if (EPI == DEC_QKV_ROPE) pos = *a.pos;
  float bv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) bv[r] = a.bias ? a.bias[min(rows[r], a.N - 1)] : 0.0f;
  float res = 0.0f;
  if (EPI == DEC_RESID) res = a.y[min(dec_row<EPI, R>(gw, lane & (R - 1)), a.N - 1)];
  float4 xv[NL];
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
#pragma unroll
  for (int j = 0; j < NL; ++j) xv[j] = x4[min(lane + j * 64, K4 - 1)];
  float4 g[NL];
  if (NORM) {
    const float4* g4 = reinterpret_cast<const float4*>(a.norm_w);
#pragma unroll
    for (int j = 0; j < NL; ++j) g[j] = g4[min(lane + j * 64, K4 - 1)];
  }
  float rs_sin[2] = {0.0f, 0.0f}, rs_cos[2] = {1.0f, 1.0f};
  if (EPI == DEC_QKV_ROPE) {
    // rotation of the wave's two NEOX pairs, computed under the weight stream
    const int c = (int)(gw & 15) * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      sincosf((float)pos * __shfl(inv_lane, c + i, 64), &rs_sin[i], &rs_cos[i]);
  }
#pragma unroll
  for (int j = 0; j < NL; ++j)
    if (lane + j * 64 >= K4) xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (NORM) {
    // y = (x * rsqrt(mean(x^2) + eps)) * w, as the standalone RMSNorm kernel
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NL; ++j) s += dot4(xv[j], xv[j]);
    const float ms = wave_sum(s) / (float)a.K;
    const float rs = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      xv[j].x = (xv[j].x * rs) * g[j].x;
      xv[j].y = (xv[j].y * rs) * g[j].y;
      xv[j].z = (xv[j].z * rs) * g[j].z;
      xv[j].w = (xv[j].w * rs) * g[j].w;
    }
    if (EPI == DEC_HEAD && a.y2 && gw == 0) {
      float4* o4 = reinterpret_cast<float4*>(a.y2);
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const int k4 = lane + j * 64;
        if (k4 < K4) o4[k4] = xv[j];
      }
    }
  }
  float v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NL; ++j) acc += dot4(w[r][j], xv[j]);
    v[r] = wave_sum(acc) + bv[r];
  }
  if (EPI == DEC_QKV_ROPE) {
    // rows r0 = c, r1 = c+1, r2 = c+32, r3 = c+33 of head `head`
    if ((gw >> 4) < a.rope_heads) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float x0 = v[i], x1 = v[2 + i];
        v[i] = x0 * rs_cos[i] - x1 * rs_sin[i];
        v[2 + i] = x1 * rs_cos[i] + x0 * rs_sin[i];
      }
    }
    if (lane < R) {
      const long col = dec_row<EPI, R>(gw, lane);
      float val = v[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) val = v[r];
      if (col < a.q_cols) {
        a.y[col] = val;
      } else if (col < a.q_cols + a.kv_cols) {
        a.k_cache[(long)pos * a.kv_cols + (col - a.q_cols)] = val;
      } else {
        a.v_cache[(long)pos * a.kv_cols + (col - a.q_cols - a.kv_cols)] = val;
      }
    }
    return;
  }
  if (EPI == DEC_SWIGLU) {
    // interleaved rows (2i, 2i+1) = (gate_i, up_i)
    if (lane < R / 2) {
      float g = v[0], u = v[1];
#pragma unroll
      for (int r = 1; r < R / 2; ++r)
        if (lane == r) {
          g = v[2 * r];
          u = v[2 * r + 1];
        }
      const long row = gw * R + 2 * lane;
      if (row < a.N) a.y[row >> 1] = (g / (1.0f + expf(-g))) * u;
    }
    return;
  }
  if (lane < R) {
    float val = v[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) val = v[r];
    const long n = dec_row<EPI, R>(gw, lane);
    if (n < a.N) {
      if (EPI == DEC_RESID)
        a.y[n] = res + val;
      else
        a.y[n] = val;
    }
  }
}

// Split-key GQA decode attention, partial pass.  grid (max_splits,
// n_kv_heads), 256 threads.  The workgroup of split `sp` takes keys
// [64 sp, 64 sp + 64) of its kv head and scores them against the kv head's
// `rep` query heads (wave w: heads w and w + 4).  With a single split it
// writes the normalised output; otherwise (max, sum, unnormalised o) per head
// for dec_attn_merge_kernel.  The K/V tile loads do not wait for the
// position: rows are clamped into the cache and masked afterwards.
__global__ __launch_bounds__(256) void dec_attn_partial_kernel(DecAttnArgs a) {
  __shared__ float ks[kKeys][kHD + 4];
  __shared__ float vs[kKeys][kHD];
  __shared__ float qs[2 * kMaxRep][kHD];  // rows >= rep are clamped copies, never read
  __shared__ float ps[kMaxRep][kKeys];
  const int sp = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int k0 = sp * kKeys;
  float4 kt[4], vt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
    const long off = (long)min(k0 + row, a.max_rows - 1) * a.ld + g * kHD + c4 * 4;
    kt[i] = *reinterpret_cast<const float4*>(a.k_cache + off);
    vt[i] = *reinterpret_cast<const float4*>(a.v_cache + off);
  }
  float4 q = *reinterpret_cast<const float4*>(a.q + (long)(g * a.rep + min(tid >> 4, a.rep - 1)) *
                                                       kHD + (tid & 15) * 4);
  // the tiles go to LDS before the position is consulted, so the loads above
  // stay ahead of the (scalar) position load instead of waiting for it
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
    *reinterpret_cast<float4*>(&ks[row][c4 * 4]) = kt[i];
    *reinterpret_cast<float4*>(&vs[row][c4 * 4]) = vt[i];
  }
  q.x *= a.scale;
  q.y *= a.scale;
  q.z *= a.scale;
  q.w *= a.scale;
  *reinterpret_cast<float4*>(&qs[tid >> 4][(tid & 15) * 4]) = q;
  const int Tk = *a.pos + 1;
  const int n_split = (Tk + kKeys - 1) / kKeys;
  if (sp >= n_split) return;
  const int nk = min(kKeys, Tk - k0);
  __syncthreads();
  // scores: lane = key
  float m[2], l[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int h = wave + 4 * hh;
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
    if (h >= a.rep) continue;
    float sc = -INFINITY;
    if (lane < nk) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < kHD / 4; ++j)
        acc += dot4(*reinterpret_cast<const float4*>(&ks[lane][4 * j]),
                    *reinterpret_cast<const float4*>(&qs[h][4 * j]));
      sc = acc;
    }
    const float mx = wave_max(sc);
    const float p = lane < nk ? expf(sc - mx) : 0.0f;
    ps[h][lane] = p;
    m[hh] = mx;
    l[hh] = wave_sum(p);
  }
  __syncthreads();
  // P V: lane = channel (rows past nk carry p = 0 and are never read)
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int h = wave + 4 * hh;
    if (h >= a.rep) continue;
    float acc = 0.0f;
    for (int j = 0; j < nk; ++j) acc += ps[h][j] * vs[j][lane];
    if (n_split == 1) {
      a.out[(long)(g * a.rep + h) * kHD + lane] = acc / l[hh];
    } else {
      float* dst = a.part + (long)g * a.part_group_stride + ((long)sp * a.rep + h) * (kHD + 2);
      dst[lane] = acc;
      if (lane == 0) {
        dst[kHD] = m[hh];
        dst[kHD + 1] = l[hh];
      }
    }
  }
}

// Merge pass: grid (n_heads), 256 threads.  Wave w reads splits w, w + 4, ...
// (all loads of a thread issued together), lane = channel; the rescaled sums
// are combined across the four waves in LDS.  Nothing to do for one split.
__global__ __launch_bounds__(256) void dec_attn_merge_kernel(DecAttnArgs a) {
  __shared__ float red_m[4], red_l[4];
  __shared__ float red_o[4][kHD];
  const int h = blockIdx.x, g = h / a.rep, hr = h - g * a.rep;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int Tk = *a.pos + 1;
  const int n_split = (Tk + kKeys - 1) / kKeys;
  if (n_split == 1) return;
  const float* base = a.part + (long)g * a.part_group_stride + (long)hr * (kHD + 2);
  const long sstride = (long)a.rep * (kHD + 2);
  // unconditional loads from clamped (written) splits, masked afterwards
  float mo[kMergePerWave], mm[kMergePerWave], ml[kMergePerWave];
#pragma unroll
  for (int i = 0; i < kMergePerWave; ++i) {
    const float* src = base + min(wave + 4 * i, n_split - 1) * sstride;
    mo[i] = src[lane];
    mm[i] = src[kHD];
    ml[i] = src[kHD + 1];
  }
#pragma unroll
  for (int i = 0; i < kMergePerWave; ++i)
    if (wave + 4 * i >= n_split) {
      mo[i] = 0.0f;
      mm[i] = -INFINITY;
      ml[i] = 0.0f;
    }
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergePerWave; ++i) M = fmaxf(M, mm[i]);
  if (lane == 0) red_m[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  float L = 0.0f, O = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergePerWave; ++i) {
    const float wgt = mm[i] == -INFINITY ? 0.0f : expf(mm[i] - M);
    L += wgt * ml[i];
    O += wgt * mo[i];
  }
  red_o[wave][lane] = O;
  if (lane == 0) red_l[wave] = L;
  __syncthreads();
  if (wave == 0) {
    const float Ls = (red_l[0] + red_l[1]) + (red_l[2] + red_l[3]);
    const float Os = (red_o[0][lane] + red_o[1][lane]) + (red_o[2][lane] + red_o[3][lane]);
    a.out[(long)h * kHD + lane] = Os / Ls;
  }
}

// Writes the position and the token's embedding row (bit-exact copy).
__global__ __launch_bounds__(256) void dec_begin_kernel(const float* __restrict__ table, long row,
                                                        int D4, float* __restrict__ x, int* d_pos,
                                                        int pos) {
  const float4* src = reinterpret_cast<const float4*>(table) + row * D4;
  float4* dst = reinterpret_cast<float4*>(x);
  for (int i = threadIdx.x; i < D4; i += blockDim.x) dst[i] = src[i];
  if (threadIdx.x == 0) *d_pos = pos;
}

template <int EPI, int R, int NL, bool NORM>
int launch_gemv(const DecGemvArgs& a, long waves, hipStream_t s) {
  // one wave per workgroup until the grid covers the CUs four times over
  int wpb = 1;
  while (wpb < 4 && waves / (wpb * 2) >= 1024) wpb *= 2;
  const long blocks = (waves + wpb - 1) / wpb;
  hipLaunchKernelGGL((dec_gemv_kernel<EPI, R, NL, NORM>), dim3((unsigned)blocks), dim3(64 * wpb),
                     0, s, a);
  return check_launch("dec_gemv_kernel");
}

}  // namespace

int dec_nl(int K) { return (K / 4 + 63) / 64; }

bool dec_supported(int hidden, int intermediate) {
  return dec_nl(hidden) <= 8 && dec_nl(intermediate) <= 24 && hidden % 4 == 0 &&
         intermediate % 4 == 0;
}

int dec_gemv(int epi, const DecGemvArgs& a, hipStream_t s) {
  LX_REQUIRE(a.W && a.x && a.y && a.N > 0 && a.K > 0 && a.K % 4 == 0, "dec_gemv: bad args");
  const int nl = dec_nl(a.K);
  switch (epi) {
    case DEC_QKV_ROPE: {
      LX_REQUIRE(a.N % kHD == 0 && a.pos && a.k_cache && a.v_cache, "dec_gemv: qkv args");
      const long waves = a.N / 4;
      if (nl <= 4) return launch_gemv<DEC_QKV_ROPE, 4, 4, true>(a, waves, s);
      if (nl <= 8) return launch_gemv<DEC_QKV_ROPE, 4, 8, true>(a, waves, s);
      break;
    }
    case DEC_SWIGLU: {
      LX_REQUIRE(a.N % 4 == 0, "dec_gemv: swiglu needs N % 4 == 0");
      const long waves = a.N / 4;
      if (nl <= 4) return launch_gemv<DEC_SWIGLU, 4, 4, true>(a, waves, s);
      if (nl <= 8) return launch_gemv<DEC_SWIGLU, 4, 8, true>(a, waves, s);
      break;
    }
    case DEC_RESID: {
      if (nl <= 4) return launch_gemv<DEC_RESID, 2, 4, false>(a, (a.N + 1) / 2, s);
      if (nl <= 8) return launch_gemv<DEC_RESID, 2, 8, false>(a, (a.N + 1) / 2, s);
      if (nl <= 19) return launch_gemv<DEC_RESID, 1, 19, false>(a, a.N, s);
      if (nl <= 24) return launch_gemv<DEC_RESID, 1, 24, false>(a, a.N, s);
      break;
    }
    case DEC_HEAD: {
      if (nl <= 4) return launch_gemv<DEC_HEAD, 2, 4, true>(a, (a.N + 1) / 2, s);
      if (nl <= 8) return launch_gemv<DEC_HEAD, 2, 8, true>(a, (a.N + 1) / 2, s);
      break;
    }
  }
  set_error("dec_gemv: unsupported epilogue %d or K=%d", epi, a.K);
  return LX_ERR_ARG;
}

int dec_attention(const DecAttnArgs& a, int n_kv_heads, bool one_split, hipStream_t s) {
  const int max_splits = dec_attention_splits(a.max_rows);
  LX_REQUIRE(a.rep >= 1 && a.rep <= kMaxRep && a.ld % 4 == 0 && a.max_rows >= 1 &&
                 max_splits <= 4 * kMergePerWave,
             "dec_attention: bad args");
  // one_split: the caller guarantees position + 1 <= kKeys, so the single
  // split's workgroups write the normalised output and no merge is launched
  hipLaunchKernelGGL(dec_attn_partial_kernel, dim3(one_split ? 1 : max_splits, n_kv_heads),
                     dim3(256), 0, s, a);
  int rc = check_launch("dec_attn_partial_kernel");
  if (rc || one_split) return rc;
  hipLaunchKernelGGL(dec_attn_merge_kernel, dim3(n_kv_heads * a.rep), dim3(256), 0, s, a);
  return check_launch("dec_attn_merge_kernel");
}

int dec_attention_split_keys() { return kKeys; }

int dec_attention_splits(int max_ctx) { return (max_ctx + kKeys - 1) / kKeys; }
int dec_attention_max_ctx() { return 4 * kMergePerWave * kKeys; }

int dec_begin(const float* table, long row, int D, float* x, int* d_pos, int pos,
              hipStream_t s) {
  LX_REQUIRE(D % 4 == 0, "dec_begin: D %% 4 != 0");
  hipLaunchKernelGGL(dec_begin_kernel, dim3(1), dim3(256), 0, s, table, row, D / 4, x, d_pos,
                     pos);
  return check_launch("dec_begin_kernel");
}

}  // namespace lx
