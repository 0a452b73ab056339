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
// kv head) scores all query heads of its group; while the whole cache fits one
// split that pass writes the output, past it every workgroup of the o_proj
// launch merges the partial softmax states itself before its rows (five
// launches per layer at every cache length).
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
constexpr int kMaxHeads = 32;  // query heads of the fused merge + o_proj (hidden <= 2048)
constexpr int kMaxSplits = 64;     // 64-key splits the merge covers: 4096 keys
// One partial softmax state per (split, query head): 64 unnormalised output
// channels, the running maximum at [64] and the sum at [65], padded to 68
// floats so every record starts 16-byte aligned (float4 reads of the channels).
constexpr int kPart = 68;

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

// Split-key GQA decode attention, partial pass.  grid (splits, n_kv_heads),
// 256 threads.  The workgroup of split `sp` takes keys
// [64 sp, 64 sp + 64) of its kv head and scores them against the kv head's
// `rep` query heads (wave w: heads w and w + 4).  With a single split it
// writes the normalised output; otherwise (max, sum, unnormalised o) per head
// for the merge in dec_merge_o_kernel.  The K/V tile loads do not wait for the
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
  if (sp >= n_split) {
    // a split past the keys (launches of more than one split only): its state
    // is the empty one, so the merge adds exact zeros and needs no position
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int h = wave + 4 * hh;
      if (h >= a.rep) continue;
      float* dst = a.part + (long)g * a.part_group_stride + ((long)sp * a.rep + h) * kPart;
      dst[lane] = 0.0f;
      if (lane == 0) {
        dst[kHD] = -INFINITY;
        dst[kHD + 1] = 0.0f;
      }
    }
    return;
  }
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
      float* dst = a.part + (long)g * a.part_group_stride + ((long)sp * a.rep + h) * kPart;
      dst[lane] = acc;
      if (lane == 0) {
        dst[kHD] = m[hh];
        dst[kHD + 1] = l[hh];
      }
    }
  }
}

// Attention merge fused into o_proj + residual, for caches longer than one
// 64-key split (src/llm/llm.cpp:254-281).  grid (ceil(hidden / 8)), 512
// threads; wave w owns o_proj row 8 * blockIdx.x + w.  Every workgroup first
// merges the partial softmax states of all query heads itself, so no
// workgroup waits for another and nothing is published: wave w merges heads
// w, w + 8, ...; lane (split group sg = lane / 16, channel quad c4 = lane % 16)
// sums splits sg, sg + 4, ... of its head in split order, the (max, sum) of
// split sg + 4 c4 is read by lane (sg, c4) and reaches the other lanes through a
// lane shuffle, and the four split groups are added with the two half-wave
// swaps.  The merged row (n_heads * 64 floats) goes to LDS for the projection.
// The launch reads the states of splits [0, nrec), nrec = min(4 * SPL,
// allocated splits); the partial pass wrote every one of them in the same
// launch order (splits past the keys as empty states), so the merge does not
// read the position.  The states of the wave's first two heads are requested
// before the o_proj weights (the first head's only, past 4 splits per group or
// 16 heads), so waiting for them does not wait for the weight stream (loads
// retire in order), which stays in flight through the merge.
// SPL = splits per split group.
template <int SPL>
__device__ __forceinline__ void merge_load(const DecAttnArgs& a, int h, int sg, int c4, int smax,
                                           float4 (&ov)[SPL], float& mv, float& lv) {
  const int g = h / a.rep, hr = h - g * a.rep;
  const float* base = a.part + (long)g * a.part_group_stride + (long)hr * kPart;
  const long ss = (long)a.rep * kPart;
#pragma unroll
  for (int i = 0; i < SPL; ++i)
    ov[i] = *reinterpret_cast<const float4*>(base + min(sg + 4 * i, smax) * ss + 4 * c4);
  const float* st = base + min(sg + 4 * c4, smax) * ss + kHD;
  mv = st[0];
  lv = st[1];
}

template <int SPL>
__device__ __forceinline__ float4 merge_head(const float4 (&ov)[SPL], float mv, float lv, int sg,
                                             int c4, int nrec) {
  const bool own_live = sg + 4 * c4 < nrec;
  const float M = wave_max(own_live ? mv : -INFINITY);
  const float w_own = own_live ? expf(mv - M) : 0.0f;
  const float L = wave_sum(own_live ? w_own * lv : 0.0f);
  float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const float wi = __shfl(w_own, sg * 16 + i, 64);
    if (sg + 4 * i < nrec) {
      O.x += wi * ov[i].x;
      O.y += wi * ov[i].y;
      O.z += wi * ov[i].z;
      O.w += wi * ov[i].w;
    }
  }
  O.x += lane_xor16(O.x);
  O.y += lane_xor16(O.y);
  O.z += lane_xor16(O.z);
  O.w += lane_xor16(O.w);
  O.x += lane_xor32(O.x);
  O.y += lane_xor32(O.y);
  O.z += lane_xor32(O.z);
  O.w += lane_xor32(O.w);
  return make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
}

constexpr int kMergeWaves = 8;  // waves (= o_proj rows) per workgroup

template <int SPL, int NL>
__global__ __launch_bounds__(64 * kMergeWaves) void dec_merge_o_kernel(DecAttnArgs at,
                                                                       DecGemvArgs o) {
  constexpr int HPW = NL / 2;  // heads per wave: 16 heads (hidden <= 1024) or 32
  // heads whose states are requested ahead of the weights: two while there are
  // at most 4 splits per group (measured faster), one for more splits or 32
  // heads (the second head's states then queue behind the weight stream)
  constexpr int HE = (NL <= 4 && SPL <= 4) ? 2 : 1;
  __shared__ float4 xs[kMaxHeads * kHD / 4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sg = lane >> 4, c4 = lane & 15;
  const int NH = at.n_heads;
  const int nrec = min((at.max_rows + kKeys - 1) / kKeys, 4 * SPL);
  float4 ov[HE][SPL];
  float mv[HE], lv[HE];
#pragma unroll
  for (int e = 0; e < HE; ++e)
    merge_load<SPL>(at, min(wave + kMergeWaves * e, NH - 1), sg, c4, nrec - 1, ov[e], mv[e],
                    lv[e]);
  const long row = (long)blockIdx.x * kMergeWaves + wave;
  const long rc = min(row, o.N - 1);
  const int K4 = o.K >> 2;
  const float4* W4 = reinterpret_cast<const float4*>(o.W) + rc * K4;
  float4 w[NL];
#pragma unroll
  for (int j = 0; j < NL; ++j) w[j] = ld_nt(W4 + min(lane + j * 64, K4 - 1));
  const float res = o.y[rc];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    const int h = wave + kMergeWaves * hh;
    if (hh >= HE && h < NH)
      merge_load<SPL>(at, h, sg, c4, nrec - 1, ov[hh % HE], mv[hh % HE], lv[hh % HE]);
    if (h < NH) {
      const float4 r = merge_head<SPL>(ov[hh % HE], mv[hh % HE], lv[hh % HE], sg, c4, nrec);
      if (sg == 0) xs[h * (kHD / 4) + c4] = r;
    }
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int k4 = lane + j * 64;
    if (k4 < K4) acc += dot4(w[j], xs[k4]);
  }
  const float v = wave_sum(acc);
  if (row < o.N && lane == 0) o.y[row] = res + v;
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

// Split counts the fused merge + o_proj launches cover (4 * SPL, SPL = 1..16),
// ascending: each launch reads the partial states of at most 3 splits past
// the ones in use.
constexpr int kNumSplitClasses = kMaxSplits / 4;
constexpr int split_class_cap(int c) { return 4 * (c + 1); }
static_assert(kNumSplitClasses == kDecAttnClasses, "split classes");

int dec_attention(const DecAttnArgs& a, int n_kv_heads, hipStream_t s) {
  LX_REQUIRE(a.rep >= 1 && a.rep <= kMaxRep && a.ld % 4 == 0 && a.max_rows >= 1,
             "dec_attention: bad args");
  // the caller guarantees position + 1 <= kKeys: the single split's
  // workgroups write the normalised output
  hipLaunchKernelGGL(dec_attn_partial_kernel, dim3(1, n_kv_heads), dim3(256), 0, s, a);
  return check_launch("dec_attn_partial_kernel");
}

template <int SPL, int NL>
int launch_merge_o(const DecAttnArgs& a, const DecGemvArgs& o, hipStream_t s) {
  hipLaunchKernelGGL((dec_merge_o_kernel<SPL, NL>),
                     dim3((unsigned)((o.N + kMergeWaves - 1) / kMergeWaves)),
                     dim3(64 * kMergeWaves), 0, s, a, o);
  return check_launch("dec_merge_o_kernel");
}

int dec_attention_o(const DecAttnArgs& a, int n_kv_heads, int cls, const DecGemvArgs& o,
                    hipStream_t s) {
  const int max_splits = dec_attention_splits(a.max_rows);
  LX_REQUIRE(a.rep >= 1 && a.rep <= kMaxRep && a.ld % 4 == 0 && a.max_rows >= 1 &&
                 max_splits <= kMaxSplits && cls >= 0 && cls < kNumSplitClasses &&
                 a.n_heads == n_kv_heads * a.rep && a.n_heads <= kMaxHeads,
             "dec_attention_o: bad args");
  LX_REQUIRE(o.W && o.y && o.N > 0 && o.K == a.n_heads * kHD, "dec_attention_o: bad o_proj args");
  const int cap = split_class_cap(cls);
  hipLaunchKernelGGL(dec_attn_partial_kernel, dim3(min(max_splits, cap), n_kv_heads), dim3(256),
                     0, s, a);
  LX_TRY(check_launch("dec_attn_partial_kernel"));
  const int nl = dec_nl(o.K);
  LX_REQUIRE(nl <= 8, "dec_attention_o: hidden %d past 2048", o.K);
#define LX_MERGE_O(SPL)                                               \
  case SPL:                                                           \
    if (nl <= 4) return launch_merge_o<SPL, 4>(a, o, s);              \
    return launch_merge_o<SPL, 8>(a, o, s);
  switch (cap / 4) {
    LX_MERGE_O(1)
    LX_MERGE_O(2)
    LX_MERGE_O(3)
    LX_MERGE_O(4)
    LX_MERGE_O(5)
    LX_MERGE_O(6)
    LX_MERGE_O(7)
    LX_MERGE_O(8)
    LX_MERGE_O(9)
    LX_MERGE_O(10)
    LX_MERGE_O(11)
    LX_MERGE_O(12)
    LX_MERGE_O(13)
    LX_MERGE_O(14)
    LX_MERGE_O(15)
    LX_MERGE_O(16)
  }
#undef LX_MERGE_O
  set_error("dec_attention_o: no launch for %d splits", cap);
  return LX_ERR_ARG;
}

int dec_attention_class(int n_split) {
  for (int c = 0; c < kNumSplitClasses; ++c)
    if (n_split <= split_class_cap(c)) return c;
  return -1;
}

int dec_attention_split_keys() { return kKeys; }

int dec_attention_splits(int max_ctx) { return (max_ctx + kKeys - 1) / kKeys; }
int dec_attention_max_ctx() { return kMaxSplits * kKeys; }

long dec_attention_part_floats(int max_ctx, int rep) {
  return ((long)dec_attention_splits(max_ctx) * rep * kPart + 31) / 32 * 32;
}

int dec_begin(const float* table, long row, int D, float* x, int* d_pos, int pos,
              hipStream_t s) {
  LX_REQUIRE(D % 4 == 0, "dec_begin: D %% 4 != 0");
  hipLaunchKernelGGL(dec_begin_kernel, dim3(1), dim3(256), 0, s, table, row, D / 4, x, d_pos,
                     pos);
  return check_launch("dec_begin_kernel");
}

}  // namespace lx
