// Scaled-dot-product attention, fp32 on the CDNA4 matrix cores.
//
// Prefill / DiT path: per (batch, head, query tile), see attn_flash_kernel.
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
// The single-token Qwen2 decode attention lives with the other decode
// kernels (lx_decode.hip).
#include <cmath>
#include <type_traits>

#include "lx_common.hpp"
#include "lx_gemm_common.hpp"

namespace lx {
namespace {

constexpr int kHD = 64;  // head dim handled by these kernels

// Flash attention, QS x KS waves per workgroup: a (32 QS)-query tile of one
// (batch, head) split as QS query sub-tiles (32 queries each) x KS key parts.
// Every (32 KS)-key tile of K and V is loaded once into LDS (coalesced) and
// read by all waves; wave (qs, ks) scores its 32 queries against keys
// [ks*32, ks*32 + 32) of each tile.  The KS key parts of a query sub-tile are
// merged through LDS at the end in a fixed order (deterministic).
// DB: K/V double buffered in LDS (one barrier per tile); otherwise one LDS
// buffer (two barriers per tile), the next tile waiting in registers, which
// halves the LDS of a workgroup so that two fit on a CU.
// Softmax runs in base 2: q is pre-scaled by scale * log2(e), so p = exp2(s - m).
constexpr int kLD = kHD + 4;     // LDS row stride (floats)
constexpr float kLazy = 8.0f;    // reference-max slack of the online softmax (log2 units)

template <int QS, int KS, bool DB>
constexpr size_t flash_lds() {
  // K, V x (1 or 2) buffers of 32 KS rows; reused after the loop for the merge
  // ((KS - 1) partial states of 64 lanes x 34 floats per query sub-tile) and
  // the transposed output tile (QS x 32 rows of kLD).
  return (size_t)2 * (DB ? 2 : 1) * 32 * KS * kLD * sizeof(float);
}

// Four output channels: fp32, or (opk) a two-part packed group for the
// three-product GEMM that consumes the attention output.
__device__ __forceinline__ void store_o4(float* p, floatx4 w, int opk) {
  if (opk)
    *reinterpret_cast<uintx4_t*>(p) = pack2_bf16(w);
  else
    *reinterpret_cast<floatx4*>(p) = w;
}

template <int QS, int KS, bool DB, bool BUF>
__global__ __launch_bounds__(64 * QS * KS) void attn_flash_kernel(
    const float* __restrict__ q, int ldq, const float* __restrict__ k, int ldk,
    const float* __restrict__ v, int ldv, float* __restrict__ o, int ldo, int Tq, int Tk,
    int n_heads, int rep, float qscale, int causal, int q_offset, int opk) {
  constexpr int kQT = 32 * QS;   // queries per workgroup
  constexpr int KT = 32 * KS;    // keys per LDS tile
  constexpr int NT = 64 * QS * KS;   // threads
  constexpr int LPT = KT * 16 / NT;  // float4 per thread per operand tile
  static_assert(LPT * NT == KT * 16, "operand tile must split evenly over the threads");
  static_assert(QS * (KS - 1) * 64 * 34 + QS * 32 * kLD <= 2 * (DB ? 2 : 1) * KT * kLD,
                "merge space");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* Ks = lds;                                  // [DB ? 2 : 1][KT][kLD]
  float* Vs = lds + (DB ? 2 : 1) * KT * kLD;        // [DB ? 2 : 1][KT][kLD]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qs = wave % QS, ks = wave / QS;
  const int lane = tid & 63, r = lane & 31, h = lane >> 5;
  // XCD-aware work order.  The dispatcher deals workgroups round-robin over
  // the eight XCDs (linear id mod 8), each with its own L2; renumber them so
  // that consecutive work items, the query tiles of one (batch, head) that
  // read the same K and V tiles, run on one XCD and share its L2 copy instead
  // of each XCD fetching every head's K and V.
  const int nq = (Tq + kQT - 1) / kQT;
  int work;
  {
    const int n = gridDim.x, x = blockIdx.x & 7, per = n >> 3, rem = n & 7;
    work = x * per + min(x, rem) + (blockIdx.x >> 3);
  }
  const int qtile = work % nq, bh = work / nq;
  const int head = bh % n_heads, b = bh / n_heads, g = head / rep;
  const int qt0 = qtile * kQT;
  const int q0 = qt0 + qs * 32;

  // Q^T operand: lane holds Q[q0 + r][h*32 + s] * scale * log2(e), s = 0..31.
  floatx4 qf[8];
  {
    const float* qrow = q + ((long)b * Tq + min(q0 + r, Tq - 1)) * ldq + head * kHD + h * 32;
#pragma unroll
    for (int j = 0; j < 8; ++j) qf[j] = *reinterpret_cast<const floatx4*>(qrow + 4 * j) * qscale;
  }
  const int my_q = q_offset + q0 + r;
  const int kend = causal ? min(Tk, q_offset + min(qt0 + kQT - 1, Tq - 1) + 1) : Tk;
  const int ntiles = (kend + KT - 1) / KT;

  // K/V tile loader: 2 x 16 KT float4 per tile, LPT + LPT per thread.  BUF:
  // buffer descriptors over this (batch, kv head)'s rows, per-lane byte
  // offsets fixed and the tile advancing through the scalar offset; keys past
  // Tk read as zeros (they are masked).  Otherwise 64-bit addresses with keys
  // clamped.
  const float* kbase = k + (long)b * Tk * ldk + g * kHD;
  const float* vbase = v + (long)b * Tk * ldv + g * kHD;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)kbase, (short)0, BUF ? (int)(((long)(Tk - 1) * ldk + kHD) * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)vbase, (short)0, BUF ? (int)(((long)(Tk - 1) * ldv + kHD) * 4) : 0, 0x00020000);
  floatx4 rk[LPT], rv[LPT];
  auto gload = [&](int t) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int idx = tid + NT * j;
      const int row = idx >> 4, c = (idx & 15) * 4;
      if (BUF) {
        rk[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, (row * ldk + c) * 4, t * KT * ldk * 4, 0);
        rv[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (row * ldv + c) * 4, t * KT * ldv * 4, 0);
      } else {
        const int key = min(t * KT + row, Tk - 1);
        rk[j] = *reinterpret_cast<const floatx4*>(kbase + (long)key * ldk + c);
        rv[j] = *reinterpret_cast<const floatx4*>(vbase + (long)key * ldv + c);
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int idx = tid + NT * j;
      const int row = idx >> 4, c = (idx & 15) * 4;
      *reinterpret_cast<floatx4*>(Ks + (buf * KT + row) * kLD + c) = rk[j];
      *reinterpret_cast<floatx4*>(Vs + (buf * KT + row) * kLD + c) = rv[j];
    }
  };

  floatx16 o0, o1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o0[i] = 0.0f;
    o1[i] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;
  float m_use = 0.0f;        // m_run, or 0 while the query has seen no unmasked key
  float m_thr = -INFINITY;   // m_run + kLazy

  // Per-lane LDS bases; buffer, block and register offsets below are
  // compile-time immediates of the LDS instructions.
  const float* kfrag = Ks + (ks * 32 + r) * kLD + h * 32;
  const float* vcol = Vs + (ks * 32 + h * 4) * kLD + r;
  // Scores, softmax and P V of this wave's 32 keys (first key kb) of the tile
  // in LDS buffer buf; MASK applies the key bounds (Tk, causal).
  auto block = [&](auto mask_c, int buf, int kb) {
    constexpr bool MASK = decltype(mask_c)::value;
    const float* krow = kfrag + buf * KT * kLD;
    floatx16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const floatx4 kv = *reinterpret_cast<const floatx4*>(krow + 4 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[e], qf[j][e], s, 0, 0, 0);
    }
    // S^T register i of lane half h is key kb + (i/4)*8 + h*4 + i%4 for query r.
    if (MASK) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + (i >> 2) * 8 + h * 4 + (i & 3);
        const bool ok = key < Tk && (!causal || key <= my_q);
        s[i] = ok ? s[i] : -INFINITY;
      }
    }
    // Lazy rescaling: m_run is the softmax reference, not necessarily the
    // running maximum.  It moves (and O, l are rescaled) only when a query's
    // maximum exceeds it by more than kLazy (log2 units), so p <= 2^kLazy and
    // the sums stay far from overflow; softmax is invariant to the reference,
    // so O / l is unchanged.  A query's maximum exceeds m_run + kLazy exactly
    // when one of its two lane halves' local maxima does, so the cross-half
    // exchange runs only in the (rare) tiles where some lane's does; most
    // tiles skip the rescale and the PV products chain straight onto the
    // previous tile's.
    float mloc = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, s[i]);
    if (__builtin_amdgcn_read_exec() & __ballot(mloc > m_thr)) {
      mloc = fmaxf(mloc, lane_xor32(mloc));
      const bool move = mloc > m_thr;  // false while the query is fully masked
      const float m_new = move ? mloc : m_run;
      // lanes that keep their reference multiply by exactly 1
      const float alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] *= alpha;
        o1[i] *= alpha;
      }
      m_run = m_new;
      m_use = m_run == -INFINITY ? 0.0f : m_run;
      m_thr = m_run + kLazy;
    }
    // v_exp_f32 directly: every argument is <= kLazy (or -inf -> 0), where
    // the hardware exp2 is accurate to about 1 ulp; results below 2^-126
    // flush to zero, far under the weight of any unmasked key.
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = __builtin_amdgcn_exp2f(s[i] - m_use);
      psum += s[i];
    }
    l_run += psum;
    // O^T += V^T P^T: register i supplies k index key_h(i) for lane half h.
    const float* vt = vcol + buf * KT * kLD;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* vrow = vt + ((i >> 2) * 8 + (i & 3)) * kLD;
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[0], s[i], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32], s[i], o1, 0, 0, 0);
    }
  };
  // Only a block that crosses Tk or (causal) the wave's first query needs
  // masking; the test is uniform across the wave.
  auto needs_mask = [&](int kb) { return kb + 32 > Tk || (causal && kb + 31 > q_offset + q0); };

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();
  if constexpr (DB && QS * KS == 4) {
    // Tile t sits in buffer t & 1; the next tile is fetched at the top and
    // stored into the other buffer at the bottom, one barrier per tile.
    auto tile = [&](int t, auto mask_c, auto buf_c) {
      constexpr bool MASK = decltype(mask_c)::value;
      constexpr int B = decltype(buf_c)::value;
      if (t + 1 < ntiles) gload(t + 1);
      const int kb = t * KT + ks * 32;  // first key of this wave's part of the tile
      if (!MASK) {
        block(std::false_type{}, B, kb);
      } else if (kb < kend) {
        if (needs_mask(kb))
          block(std::true_type{}, B, kb);
        else
          block(std::false_type{}, B, kb);
      }
      if (t + 1 < ntiles) sstore(B ^ 1);
      __syncthreads();
    };
    // Tiles before t_plain need no key bounds in any wave of the workgroup
    // (all keys below Tk and, causal, at or before its first query); they run
    // unrolled by two so that the buffer index is a constant.  The rest (a
    // partial last tile, the diagonal tiles) test per wave.
    const int t_full = Tk / KT;
    const int t_diag = causal ? (q_offset + qt0 + 1) / KT : t_full;
    const int t_plain = min(min(t_full, t_diag), ntiles) & ~1;
    int t = 0;
    for (; t < t_plain; t += 2) {
      tile(t, std::false_type{}, std::integral_constant<int, 0>{});
      tile(t + 1, std::false_type{}, std::integral_constant<int, 1>{});
    }
    for (; t < ntiles; t += 2) {
      tile(t, std::true_type{}, std::integral_constant<int, 0>{});
      if (t + 1 < ntiles) tile(t + 1, std::true_type{}, std::integral_constant<int, 1>{});
    }
  } else {
    // Two waves per SIMD (or a single buffer): the loop with the softmax
    // inline and a runtime buffer index, which measures faster there than
    // the restructured block above (T = 3000: 774 vs 838 us).
    for (int t = 0; t < ntiles; ++t) {
      const int buf = DB ? (t & 1) : 0;
      if (t + 1 < ntiles) gload(t + 1);
      const int kb = t * KT + ks * 32;  // first key of this wave's part of the tile
      if (kb < kend) {
        const float* krow = Ks + (buf * KT + ks * 32 + r) * kLD + h * 32;
        floatx16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const floatx4 kv = *reinterpret_cast<const floatx4*>(krow + 4 * j);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[e], qf[j][e], s, 0, 0, 0);
        }
        // S^T register i of lane half h is key kb + (i/4)*8 + h*4 + i%4 for query r.
        // Only a block that crosses Tk or (causal) the wave's first query needs
        // masking; the test is uniform across the wave.
        if (kb + 32 > Tk || (causal && kb + 31 > q_offset + q0)) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb + (i >> 2) * 8 + h * 4 + (i & 3);
            const bool ok = key < Tk && (!causal || key <= my_q);
            s[i] = ok ? s[i] : -INFINITY;
          }
        }
        float mloc = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, s[i]);
        mloc = fmaxf(mloc, lane_xor32(mloc));
        // Lazy rescaling: m_run is the softmax reference, not necessarily the
        // running maximum.  It moves (and O, l are rescaled) only when a lane's
        // maximum exceeds it by more than kLazy (log2 units), so p <= 2^kLazy
        // and the sums stay far from overflow; softmax is invariant to the
        // reference, so O / l is unchanged.  Most tiles skip the rescale and the
        // PV products chain straight onto the previous tile's.
        const bool move = mloc > m_run + kLazy;  // false while the lane is fully masked
        if (__builtin_amdgcn_read_exec() & __ballot(move)) {
          const float m_new = move ? mloc : m_run;
          // lanes that keep their reference multiply by exactly 1
          const float alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
          l_run *= alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            o0[i] *= alpha;
            o1[i] *= alpha;
          }
          m_run = m_new;
        }
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;  // fully masked so far
        // v_exp_f32 directly: every argument is <= kLazy (or -inf -> 0), where
        // the hardware exp2 is accurate to about 1 ulp; results below 2^-126
        // flush to zero, far under the weight of any unmasked key.
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[i] = __builtin_amdgcn_exp2f(s[i] - m_use);
          psum += s[i];
        }
        l_run += psum;
        // O^T += V^T P^T: register i supplies k index key_h(i) for lane half h.
        const float* vt = Vs + (buf * KT + ks * 32) * kLD;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float* vrow = vt + ((i >> 2) * 8 + h * 4 + (i & 3)) * kLD;
          o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[r], s[i], o0, 0, 0, 0);
          o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 + r], s[i], o1, 0, 0, 0);
        }
      }
      if (DB) {
        if (t + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
      } else {
        __syncthreads();  // every wave is done with the tile before it is replaced
        if (t + 1 < ntiles) sstore(0);
        __syncthreads();
      }
    }
  }

  const float l_tot = l_run + lane_xor32(l_run);
  if constexpr (KS == 2) {
    // Two key parts: each wave finalises one half of the 64 channels (part 0
    // channels 0-31, part 1 channels 32-63).  Both publish (m, l) and the
    // half they do not own, then combine their own half with the partner's
    // in part order (part 0's terms first) and store it straight from the
    // registers: register i of lane (r, h) holds channels (i/4)*8 + h*4 +
    // i%4 of query r, four consecutive channels per float4.
    static_assert(QS * 2 * 18 * 64 <= 2 * (DB ? 2 : 1) * KT * kLD, "exchange space");
    float* pub = lds + (qs * 2 + ks) * (18 * 64);
    const floatx16& give = ks == 0 ? o1 : o0;
#pragma unroll
    for (int i = 0; i < 16; ++i) pub[i * 64 + lane] = give[i];
    pub[16 * 64 + lane] = m_run;
    pub[17 * 64 + lane] = l_tot;
    __syncthreads();
    const float* part = lds + (qs * 2 + (ks ^ 1)) * (18 * 64);
    const float m_o = part[16 * 64 + lane], l_o = part[17 * 64 + lane];
    const float m = fmaxf(m_run, m_o);
    const float a_s = exp2f(m_run - m), a_o = exp2f(m_o - m);
    const float l = ks == 0 ? l_tot * a_s + l_o * a_o : l_o * a_o + l_tot * a_s;
    const float inv = 1.0f / l;
    const floatx16& keep = ks == 0 ? o0 : o1;
    const int qi = q0 + r;
    if (qi < Tq) {
      float* orow = o + ((long)b * Tq + qi) * ldo + head * kHD + ks * 32 + h * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = g * 4 + e;
          const float mine = keep[i] * a_s, other = part[i * 64 + lane] * a_o;
          w[e] = (ks == 0 ? mine + other : other + mine) * inv;
        }
        store_o4(orow + g * 8, w, opk);
      }
    }
    return;
  }
  // Merge the key parts: ks > 0 publish (m, l, O^T) per lane, ks = 0 combines
  // them in part order.
  float* xch = lds + qs * ((KS - 1) * 64 * 34);  // per query sub-tile (QS of them)
  if (ks > 0) {
    float* mine = xch + (ks - 1) * (64 * 34);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mine[i * 64 + lane] = o0[i];
      mine[(16 + i) * 64 + lane] = o1[i];
    }
    mine[32 * 64 + lane] = m_run;
    mine[33 * 64 + lane] = l_tot;
  }
  __syncthreads();
  float* otile = lds + QS * (KS - 1) * 64 * 34;   // transposed output tiles [QS][32 q][kLD]
  float* ot = otile + qs * (32 * kLD);
  if (ks == 0) {
    float m = m_run;
#pragma unroll
    for (int p = 0; p < KS - 1; ++p) m = fmaxf(m, xch[p * (64 * 34) + 32 * 64 + lane]);
    const float a0 = exp2f(m_run - m);
    float l = l_tot * a0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] *= a0;
      o1[i] *= a0;
    }
#pragma unroll
    for (int p = 0; p < KS - 1; ++p) {
      const float* other = xch + p * (64 * 34);
      const float ap = exp2f(other[32 * 64 + lane] - m);
      l += other[33 * 64 + lane] * ap;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] += other[i * 64 + lane] * ap;
        o1[i] += other[(16 + i) * 64 + lane] * ap;
      }
    }
    const float inv = 1.0f / l;
    // register i of tile t is channel t*32 + (i/4)*8 + h*4 + i%4 of query r
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = (i >> 2) * 8 + h * 4 + (i & 3);
      ot[r * kLD + d] = o0[i] * inv;
      ot[r * kLD + 32 + d] = o1[i] * inv;
    }
  }
  __syncthreads();
  // coalesced store of the sub-tiles: kQT queries x 16 float4
  for (int idx = tid; idx < kQT * 16; idx += NT) {
    const int row = idx >> 4, c = (idx & 15) * 4;  // row = qs*32 + local row
    const int qi = qt0 + row;
    if (qi < Tq) {
      const float* src = otile + (row >> 5) * (32 * kLD) + (row & 31) * kLD + c;
      store_o4(o + ((long)b * Tq + qi) * ldo + head * kHD + c,
               *reinterpret_cast<const floatx4*>(src), opk);
    }
  }
}


// ---- fp32 attention on the bf16 matrix cores (split operands) ----
//
// Every fp32 operand x is split into three bf16 parts, x = x0 + x1 + x2
// (x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1)), exact for
// normal values: the three parts carry 24 significant bits.  A product
// a * b is then sum_ij a_i b_j; each a_i b_j is exact in the fp32
// accumulator of v_mfma_f32_32x32x16_bf16, and the six terms with
// i + j <= 2 are kept (the dropped a1 b2, a2 b1, a2 b2 are below 2^-23 |ab|,
// under fp32's own rounding of the product).  Sums accumulate in fp32.  Six
// bf16 MFMAs of 32 cycles replace eight fp32 32x32x2 MFMAs of 64 cycles for
// the same 32 x 32 x 16 block, and the VALU work of the split runs beside the
// matrix pipe.
//
// Same work split, merge and output as attn_flash_kernel; S^T = K Q^T and
// O^T += V^T P^T keep the accumulator layouts of the fp32 kernel.  Operands of
// v_mfma_f32_32x32x16_bf16: lane l supplies row (column) l % 32 and the eight k
// values of its half h = l / 32.  For S^T the k index is the head channel
// (K and Q rows, channels s*16 + h*8 + j).  For O^T it is the key: lane half
// h's register j of P^T (S^T register 8u + j) holds key 16u + key16(h, j),
// key16 = (j/4)*8 + h*4 + j%4, so V^T is staged in LDS with the keys of each
// 16-key group permuted to that order (positions h*8 + j), and each lane
// reads its eight keys as one 16-byte vector.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx8 __attribute__((ext_vector_type(8)));

typedef unsigned uintx2 __attribute__((ext_vector_type(2)));
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));

// fp32 value of packed bf16 parts: element 2i is the low half of word i,
// element 2i + 1 the high half (one shift or mask each; the back-conversion
// written this way keeps every rounding a packed two-element v_cvt_pk_bf16_f32)
__device__ __forceinline__ floatx4 bf16x4_to_f32(bf16x4 x) {
  const uintx2 u = __builtin_bit_cast(uintx2, x);
  floatx4 f;
  f[0] = __uint_as_float(u[0] << 16);
  f[1] = __uint_as_float(u[0] & 0xffff0000u);
  f[2] = __uint_as_float(u[1] << 16);
  f[3] = __uint_as_float(u[1] & 0xffff0000u);
  return f;
}
__device__ __forceinline__ floatx8 bf16x8_to_f32(bf16x8 x) {
  const uintx4 u = __builtin_bit_cast(uintx4, x);
  floatx8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
  return f;
}
__device__ __forceinline__ void split3(floatx4 v, bf16x4& x0, bf16x4& x1, bf16x4& x2) {
  x0 = __builtin_convertvector(v, bf16x4);
  const floatx4 r = v - bf16x4_to_f32(x0);
  x1 = __builtin_convertvector(r, bf16x4);
  x2 = __builtin_convertvector(r - bf16x4_to_f32(x1), bf16x4);
}
// The two bf16 parts of a packed group (pack2_bf16) loaded as 16 bytes.
__device__ __forceinline__ void unpack2(floatx4 v, bf16x4* x) {
  const uintx4 u = __builtin_bit_cast(uintx4, v);
  x[0] = __builtin_bit_cast(bf16x4, uintx2{u[0], u[1]});
  x[1] = __builtin_bit_cast(bf16x4, uintx2{u[2], u[3]});
  x[2] = x[1];
}
__device__ __forceinline__ void split3(floatx8 v, bf16x8& x0, bf16x8& x1, bf16x8& x2) {
  x0 = __builtin_convertvector(v, bf16x8);
  const floatx8 r = v - bf16x8_to_f32(x0);
  x1 = __builtin_convertvector(r, bf16x8);
  x2 = __builtin_convertvector(r - bf16x8_to_f32(x1), bf16x8);
}

// acc += sum of the NP split products (smallest first): six a_i b_j with
// i + j <= 2 of three-part splits, or three (a1 b0 + a0 b1 + a0 b0) of
// two-part splits
template <int NP>
__device__ __forceinline__ floatx16 mfma_split(const bf16x8* a, const bf16x8* b, floatx16 acc) {
  if (NP == 3) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  }
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
}

// LDS of the split kernel, two buffers each of K planes [NPL][KT keys][kKP]
// and V^T planes [NPL][64 channels][KT + 8] (bf16; NPL = 3 parts for six
// products, 2 for three); the merge reuses it.
constexpr int kKP = kHD + 8;  // bf16 per K plane row (144 bytes: conflict-free 16-byte reads)
template <int QS, int KS, int NP = 6>
constexpr size_t bx_lds() {
  constexpr int KT = 32 * KS;
  constexpr int NPL = NP == 6 ? 3 : 2;
  constexpr size_t planes = (size_t)2 * 2 * NPL * (KT * kKP + kHD * (KT + 8));
  constexpr size_t merge = KS == 2 ? (size_t)QS * 2 * 18 * 64 * 4
                                   : (size_t)(QS * (KS - 1) * 64 * 34 + QS * 32 * kLD) * 4;
  return planes > merge ? planes : merge;
}

// position of key k (within a tile) in the permuted V^T rows
__device__ __forceinline__ int vt_pos(int k) {
  return (k & ~15) + ((k >> 2) & 1) * 8 + ((k >> 3) & 1) * 4 + (k & 3);
}

// Software pipelined over the key tiles: iteration t issues the score MFMAs
// of tile t + 1 first, then runs the softmax of tile t (VALU, beside those
// MFMAs), splits P and issues O^T += V^T P^T of tile t, then splits and stores
// the tiles fetched during the iteration (K of tile t + 2, V of tile t + 1)
// beside the PV MFMAs.  K and V rotate through two LDS buffers each: K of
// tile t + 2 replaces K of tile t (its scores were formed in iteration t - 1),
// V of tile t + 1 replaces V of tile t - 1, so one barrier per tile suffices.
// KVP: K and V arrive as two-part packed rows (their producer split them
// once; three products), so staging stores the parts without splitting.
template <int QS, int KS, bool BUF, int NP, bool KVP = false>
__global__ __launch_bounds__(64 * QS * KS) void attn_bx_kernel(
    const float* __restrict__ q, int ldq, const float* __restrict__ k, int ldk,
    const float* __restrict__ v, int ldv, float* __restrict__ o, int ldo, int Tq, int Tk,
    int n_heads, int rep, float qscale, int causal, int q_offset, int opk) {
  constexpr int kQT = 32 * QS;
  constexpr int KT = 32 * KS;
  constexpr int NT = 64 * QS * KS;
  constexpr int LPT = KT * 16 / NT;  // K float4 per thread per tile
  constexpr int LPV = LPT / 2;       // V key pairs (two float4) per thread per tile
  constexpr int VP = KT + 8;         // bf16 per V^T plane row
  constexpr int NPL = NP == 6 ? 3 : 2;  // bf16 parts per operand
  constexpr int KBUF = NPL * KT * kKP;  // bf16 per K buffer
  constexpr int VBUF = NPL * kHD * VP;  // bf16 per V buffer
  static_assert(LPT * NT == KT * 16 && LPV * 2 == LPT, "operand tile must split evenly");
  static_assert(bx_lds<QS, KS, NP>() <= 160 * 1024, "LDS of one CU");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __bf16* Kp = reinterpret_cast<__bf16*>(lds);  // [2][NPL][KT][kKP]
  __bf16* Vt = Kp + 2 * KBUF;                    // [2][NPL][64][VP]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qs = wave % QS, ks = wave / QS;
  const int lane = tid & 63, r = lane & 31, h = lane >> 5;
  const int nq = (Tq + kQT - 1) / kQT;
  int work;
  {
    const int n = gridDim.x, x = blockIdx.x & 7, per = n >> 3, rem = n & 7;
    work = x * per + min(x, rem) + (blockIdx.x >> 3);
  }
  const int qtile = work % nq, bh = work / nq;
  const int head = bh % n_heads, b = bh / n_heads, g = head / rep;
  const int qt0 = qtile * kQT;
  const int q0 = qt0 + qs * 32;

  // Q rows of this lane (scaled and split below, once the first K/V tiles'
  // loads are in flight behind them)
  floatx4 qraw[8];
  {
    const float* qrow = q + ((long)b * Tq + min(q0 + r, Tq - 1)) * ldq + head * kHD + h * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qraw[2 * s] = *reinterpret_cast<const floatx4*>(qrow + s * 16);
      qraw[2 * s + 1] = *reinterpret_cast<const floatx4*>(qrow + s * 16 + 4);
    }
  }
  bf16x8 qb[4][3];
  const int my_q = q_offset + q0 + r;
  const int kend = causal ? min(Tk, q_offset + min(qt0 + kQT - 1, Tq - 1) + 1) : Tk;
  const int ntiles = (kend + KT - 1) / KT;

  // K/V tile loaders (as attn_flash_kernel).  K: float4 (row, c) per step;
  // V: two float4 of keys (2 pi, 2 pi + 1) at channels c..c+3, so that each
  // V^T row receives the key pair as one 4-byte store.
  const float* kbase = k + (long)b * Tk * ldk + g * kHD;
  const float* vbase = v + (long)b * Tk * ldv + g * kHD;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)kbase, (short)0, BUF ? (int)(((long)(Tk - 1) * ldk + kHD) * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)vbase, (short)0, BUF ? (int)(((long)(Tk - 1) * ldv + kHD) * 4) : 0, 0x00020000);
  floatx4 rk[LPT], rv[LPV][2];
  auto gload_k_to = [&](int t, floatx4* dst) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int idx = tid + NT * j;
      const int row = idx >> 4, c = (idx & 15) * 4;
      if (BUF) {
        dst[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, (row * ldk + c) * 4, t * KT * ldk * 4, 0);
      } else {
        const int key = min(t * KT + row, Tk - 1);
        dst[j] = *reinterpret_cast<const floatx4*>(kbase + (long)key * ldk + c);
      }
    }
  };
  auto gload_k = [&](int t) { gload_k_to(t, rk); };
  // V key pair pr, channels c..c+3 of step idx: a wave's 64 steps cover 16
  // consecutive pairs x 16 channels, so its V^T stores (rows c+e, 16 key
  // pairs per row, rows 4 apart) fall on 64 distinct LDS banks.
  auto v_map = [](int idx, int& pr, int& c) {
    constexpr int PG = KT / 32;  // groups of 16 pairs
    const int hi = idx >> 6;
    pr = (idx & 15) + 16 * (hi % PG);
    c = 4 * (((idx >> 4) & 3) + 4 * (hi / PG));
  };
  auto gload_v = [&](int t) {
#pragma unroll
    for (int j = 0; j < LPV; ++j) {
      const int idx = tid + NT * j;
      int pr, c;
      v_map(idx, pr, c);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int row = 2 * pr + e;
        if (BUF) {
          rv[j][e] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (row * ldv + c) * 4,
                                                           t * KT * ldv * 4, 0);
        } else {
          const int key = min(t * KT + row, Tk - 1);
          rv[j][e] = *reinterpret_cast<const floatx4*>(vbase + (long)key * ldv + c);
        }
      }
    }
  };
  // split a loaded tile and store its parts into LDS buffer `buf`
  auto stage_k_from = [&](int buf, const floatx4* src) {
    __bf16* dst = Kp + buf * KBUF;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int idx = tid + NT * j;
      const int row = idx >> 4, c = (idx & 15) * 4;
      bf16x4 x[3];
      if constexpr (KVP)
        unpack2(src[j], x);
      else
        split3(src[j], x[0], x[1], x[2]);  // (the third part is dead code with two)
#pragma unroll
      for (int p = 0; p < NPL; ++p)
        *reinterpret_cast<bf16x4*>(dst + (p * KT + row) * kKP + c) = x[p];
    }
  };
  auto stage_k = [&](int buf) { stage_k_from(buf, rk); };
  auto stage_v = [&](int buf) {
    __bf16* dst = Vt + buf * VBUF;
#pragma unroll
    for (int j = 0; j < LPV; ++j) {
      const int idx = tid + NT * j;
      int pr, c;
      v_map(idx, pr, c);
      const int pos = vt_pos(2 * pr);
      bf16x4 x0[3], x1[3];
      if constexpr (KVP) {
        unpack2(rv[j][0], x0);
        unpack2(rv[j][1], x1);
      } else {
        split3(rv[j][0], x0[0], x0[1], x0[2]);
        split3(rv[j][1], x1[0], x1[1], x1[2]);
      }
#pragma unroll
      for (int p = 0; p < NPL; ++p)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bf16x2 pair;
          pair[0] = x0[p][e];
          pair[1] = x1[p][e];
          *reinterpret_cast<bf16x2*>(dst + (p * kHD + c + e) * VP + pos) = pair;
        }
    }
  };
  // S^T of this wave's 32 keys of the tile in K buffer `buf`
  const __bf16* kfrag = Kp + (ks * 32 + r) * kKP + h * 8;
  auto scores = [&](int buf) {
    floatx16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 ka[3];
#pragma unroll
      for (int p = 0; p < NPL; ++p)
        ka[p] = *reinterpret_cast<const bf16x8*>(kfrag + buf * KBUF + p * KT * kKP + st * 16);
      s = mfma_split<NP>(ka, qb[st], s);
    }
    return s;
  };

  floatx16 o0, o1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o0[i] = 0.0f;
    o1[i] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;
  const __bf16* vfrag = Vt + r * VP + ks * 32 + h * 8;

  // Prologue: Q, K and V of tile 0 and K of tile 1 are requested together (one
  // memory round trip), then Q is split while the tiles are in flight.
  // Tile 1's loads are clamped into range (or zero-filled by the buffer
  // descriptor) when there is no tile 1; no later iteration reads its buffer.
  if (ntiles > 0) {
    floatx4 rk1[LPT];
    gload_k(0);
    gload_v(0);
    gload_k_to(1, rk1);
    // Q^T operand, split: qb[s][p] holds part p of Q[q0 + r][s*16 + h*8 + j] *
    // scale * log2(e), j = 0..7.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const floatx4 lo4 = qraw[2 * s] * qscale;
      const floatx4 hi4 = qraw[2 * s + 1] * qscale;
      floatx8 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = lo4[e];
        x[4 + e] = hi4[e];
      }
      split3(x, qb[s][0], qb[s][1], qb[s][2]);
    }
    stage_k(0);
    stage_v(0);
    stage_k_from(1, rk1);
  }
  __syncthreads();
  // iteration t: s_in holds the scores of tile t, s_out receives tile t + 1's
  auto iter = [&](int t, const floatx16& s_in, floatx16& s_out) {
    const bool ld_k = t + 2 < ntiles, ld_v = t + 1 < ntiles;
    if (ld_k) gload_k(t + 2);
    if (ld_v) gload_v(t + 1);
    const int kb = t * KT + ks * 32;  // first key of this wave's part of tile t
    if (t + 1 < ntiles && kb + KT < kend) s_out = scores((t + 1) & 1);
    if (kb < kend) {
      floatx16 s = s_in;
      // S^T register i of lane half h is key kb + (i/4)*8 + h*4 + i%4 for query r.
      if (kb + 32 > Tk || (causal && kb + 31 > q_offset + q0)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + (i >> 2) * 8 + h * 4 + (i & 3);
          const bool ok = key < Tk && (!causal || key <= my_q);
          s[i] = ok ? s[i] : -INFINITY;
        }
      }
      float mloc = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, s[i]);
      mloc = fmaxf(mloc, lane_xor32(mloc));
      // Lazy rescaling, as attn_flash_kernel: the reference moves only when a
      // query's maximum exceeds it by more than kLazy (log2 units).
      const bool move = mloc > m_run + kLazy;  // false while the lane is fully masked
      if (__builtin_amdgcn_read_exec() & __ballot(move)) {
        const float m_new = move ? mloc : m_run;
        const float alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          o0[i] *= alpha;
          o1[i] *= alpha;
        }
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;  // fully masked so far
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] = __builtin_amdgcn_exp2f(s[i] - m_use);
        psum += s[i];
      }
      l_run += psum;
      // O^T += V^T P^T over the two 16-key steps of the block
      const __bf16* vb = vfrag + (t & 1) * VBUF;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        floatx8 pv;
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = s[8 * u + j];
        bf16x8 pb[3];
        split3(pv, pb[0], pb[1], pb[2]);
        bf16x8 va[3], vc[3];
#pragma unroll
        for (int p = 0; p < NPL; ++p) {
          va[p] = *reinterpret_cast<const bf16x8*>(vb + p * kHD * VP + u * 16);
          vc[p] = *reinterpret_cast<const bf16x8*>(vb + (p * kHD + 32) * VP + u * 16);
        }
        o0 = mfma_split<NP>(va, pb, o0);
        o1 = mfma_split<NP>(vc, pb, o1);
      }
    }
    if (ld_k) stage_k(t & 1);
    if (ld_v) stage_v((t + 1) & 1);
    __syncthreads();
  };
  // Iteration over a tile that no wave masks (all keys below Tk and, causal,
  // at or before the workgroup's first query), without branches around the
  // scores, the softmax and the staging, so that the compiler schedules the
  // score MFMAs of tile t + 1, the softmax of tile t, its P V MFMAs and the
  // splits and stores of the staged tiles as one block (T = 1000 59.7 -> 53.8
  // us, T = 3000 450 -> 410).  Loads and stores run unconditionally (tile
  // index clamped into range; a surplus tile lands in a buffer no later
  // iteration reads); only the accumulator rescale keeps its branch.
  auto iter_plain = [&](int t, const floatx16& s_in, floatx16& s_out) {
    const int tl = ntiles - 1;
    gload_k(min(t + 2, tl));
    gload_v(min(t + 1, tl));
    s_out = scores((t + 1) & 1);
    floatx16 s = s_in;
    float mloc = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, s[i]);
    mloc = fmaxf(mloc, lane_xor32(mloc));
    const bool move = mloc > m_run + kLazy;
    const float m_new = move ? mloc : m_run;
    const float alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
      psum += s[i];
    }
    l_run = l_run * alpha + psum;
    bf16x8 pb[2][3];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      floatx8 pv;
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = s[8 * u + j];
      split3(pv, pb[u][0], pb[u][1], pb[u][2]);
    }
    if (__builtin_amdgcn_read_exec() & __ballot(move)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] *= alpha;
        o1[i] *= alpha;
      }
    }
    const __bf16* vb = vfrag + (t & 1) * VBUF;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bf16x8 va[3], vc[3];
#pragma unroll
      for (int p = 0; p < NPL; ++p) {
        va[p] = *reinterpret_cast<const bf16x8*>(vb + p * kHD * VP + u * 16);
        vc[p] = *reinterpret_cast<const bf16x8*>(vb + (p * kHD + 32) * VP + u * 16);
      }
      o0 = mfma_split<NP>(va, pb[u], o0);
      o1 = mfma_split<NP>(vc, pb[u], o1);
    }
    stage_k(t & 1);
    stage_v((t + 1) & 1);
    __syncthreads();
  };
  floatx16 sa, sb;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    sa[i] = 0.0f;
    sb[i] = 0.0f;
  }
  if (ntiles > 0 && ks * 32 < kend) sa = scores(0);
  // tiles before t_plain need no key bounds in any wave
  const int t_plain =
      min(min(Tk / KT, causal ? (q_offset + qt0 + 1) / KT : ntiles), ntiles);
  int t = 0;
  for (; t + 1 < t_plain; t += 2) {
    iter_plain(t, sa, sb);
    iter_plain(t + 1, sb, sa);
  }
  bool in_a = true;
  if (t < t_plain) {
    iter_plain(t, sa, sb);
    ++t;
    in_a = false;
  }
  for (; t < ntiles; ++t) {
    if (in_a)
      iter(t, sa, sb);
    else
      iter(t, sb, sa);
    in_a = !in_a;
  }
  const float l_tot = l_run + lane_xor32(l_run);
  if constexpr (KS == 2) {
    // Two key parts: each wave finalises one half of the 64 channels (part 0
    // channels 0-31, part 1 channels 32-63).  Both publish (m, l) and the
    // half they do not own, then combine their own half with the partner's
    // in part order (part 0's terms first) and store it straight from the
    // registers: register i of lane (r, h) holds channels (i/4)*8 + h*4 +
    // i%4 of query r, four consecutive channels per float4.
    static_assert(QS * 2 * 18 * 64 * 4 <= bx_lds<QS, KS, NP>(), "exchange space");
    float* pub = lds + (qs * 2 + ks) * (18 * 64);
    const floatx16& give = ks == 0 ? o1 : o0;
#pragma unroll
    for (int i = 0; i < 16; ++i) pub[i * 64 + lane] = give[i];
    pub[16 * 64 + lane] = m_run;
    pub[17 * 64 + lane] = l_tot;
    __syncthreads();
    const float* part = lds + (qs * 2 + (ks ^ 1)) * (18 * 64);
    const float m_o = part[16 * 64 + lane], l_o = part[17 * 64 + lane];
    const float m = fmaxf(m_run, m_o);
    const float a_s = exp2f(m_run - m), a_o = exp2f(m_o - m);
    const float l = ks == 0 ? l_tot * a_s + l_o * a_o : l_o * a_o + l_tot * a_s;
    const float inv = 1.0f / l;
    const floatx16& keep = ks == 0 ? o0 : o1;
    const int qi = q0 + r;
    if (qi < Tq) {
      float* orow = o + ((long)b * Tq + qi) * ldo + head * kHD + ks * 32 + h * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = g * 4 + e;
          const float mine = keep[i] * a_s, other = part[i * 64 + lane] * a_o;
          w[e] = (ks == 0 ? mine + other : other + mine) * inv;
        }
        store_o4(orow + g * 8, w, opk);
      }
    }
    return;
  }
  // Merge the key parts: ks > 0 publish (m, l, O^T) per lane, ks = 0 combines
  // them in part order.
  float* xch = lds + qs * ((KS - 1) * 64 * 34);  // per query sub-tile (QS of them)
  if (ks > 0) {
    float* mine = xch + (ks - 1) * (64 * 34);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mine[i * 64 + lane] = o0[i];
      mine[(16 + i) * 64 + lane] = o1[i];
    }
    mine[32 * 64 + lane] = m_run;
    mine[33 * 64 + lane] = l_tot;
  }
  __syncthreads();
  float* otile = lds + QS * (KS - 1) * 64 * 34;   // transposed output tiles [QS][32 q][kLD]
  float* ot = otile + qs * (32 * kLD);
  if (ks == 0) {
    float m = m_run;
#pragma unroll
    for (int p = 0; p < KS - 1; ++p) m = fmaxf(m, xch[p * (64 * 34) + 32 * 64 + lane]);
    const float a0 = exp2f(m_run - m);
    float l = l_tot * a0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] *= a0;
      o1[i] *= a0;
    }
#pragma unroll
    for (int p = 0; p < KS - 1; ++p) {
      const float* other = xch + p * (64 * 34);
      const float ap = exp2f(other[32 * 64 + lane] - m);
      l += other[33 * 64 + lane] * ap;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] += other[i * 64 + lane] * ap;
        o1[i] += other[(16 + i) * 64 + lane] * ap;
      }
    }
    const float inv = 1.0f / l;
    // register i of tile t is channel t*32 + (i/4)*8 + h*4 + i%4 of query r
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = (i >> 2) * 8 + h * 4 + (i & 3);
      ot[r * kLD + d] = o0[i] * inv;
      ot[r * kLD + 32 + d] = o1[i] * inv;
    }
  }
  __syncthreads();
  // coalesced store of the sub-tiles: kQT queries x 16 float4
  for (int idx = tid; idx < kQT * 16; idx += NT) {
    const int row = idx >> 4, c = (idx & 15) * 4;  // row = qs*32 + local row
    const int qi = qt0 + row;
    if (qi < Tq) {
      const float* src = otile + (row >> 5) * (32 * kLD) + (row & 31) * kLD + c;
      store_o4(o + ((long)b * Tq + qi) * ldo + head * kHD + c,
               *reinterpret_cast<const floatx4*>(src), opk);
    }
  }
}

}  // namespace
// Layout of a launch: 0 small grids (32-query workgroups), 1 64-query, 2
// 128-query; and whether the split-operand kernel runs it (see attention()).
static int attention_layout(int B, int Tq, int n_heads, int products, bool* split) {
  const long wg64 = (long)((Tq + 63) / 64) * n_heads * B;
  const long wg128 = (long)((Tq + 127) / 128) * n_heads * B;
  const int layout = wg64 < 256 ? 0 : (wg128 % 256 == 0 ? 2 : 1);  // small / 64-query / wide
  *split = layout == 2 || (layout == 1 && (wg64 <= 256 || products == 3));
  return layout;
}

bool attention_takes_packed_kv(int B, int Tq, int n_heads, int products) {
  bool split = false;
  attention_layout(B, Tq, n_heads, products, &split);
  return split && products == 3;
}

int attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv, float* o,
              int ldo, int B, int Tq, int Tk, int n_heads, int n_kv_heads, int head_dim,
              float scale, int causal, int q_offset, int products, int out_packed,
              hipStream_t stream, int kv_packed) {
  LX_REQUIRE(products == 3 || products == 6, "attention: %d products (3 or 6)", products);
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
  LX_REQUIRE(ldv % 4 == 0 && (uintptr_t)v % 16 == 0, "attention: v rows must be 16-byte aligned");
  LX_REQUIRE(q_offset >= 0, "attention: q_offset < 0");
  if (causal) LX_REQUIRE(q_offset + Tq <= Tk, "attention: causal needs q_offset + Tq <= Tk");
  const int rep = n_heads / n_kv_heads;
  const float log2e = 1.4426950408889634f;
  // Buffer loads need every K/V byte offset (up to the last tile's rows past
  // Tk) below 2^31.
  const long lim = 1L << 31;
  const bool buf = ((long)(Tk + 128) * ldk + kHD) * 4 < lim && ((long)(Tk + 128) * ldv + kHD) * 4 < lim;
  // Three layouts.  64-query workgroups (2 query sub-tiles x 2 key parts, 64-key
  // tiles double buffered, 70 KB of LDS) whenever they cover the CUs (DiT at
  // T = 500: 256 workgroups, 24.9 us; T = 3000: 1504).  A grid smaller than
  // the device (the Qwen2 prefill at L = 256: 56 workgroups) takes 32-query
  // workgroups of 4 key parts over single-buffered 128-key tiles instead:
  // twice the workgroups, four waves each (13.9 -> 9.8 us).  At T = 500 that
  // layout is slower (27.8 us: the 4-part merge and two barriers per tile
  // cost more than the second resident workgroup per CU returns).
  // The third, 128-query workgroups of 4 query sub-tiles x 2 key parts (512
  // threads: every K/V tile feeds twice the queries), replaces the
  // 64-query layout when its grid is a whole number of workgroups per CU (fp32
  // kernel: T = 3000, 768 workgroups, 612 -> 571 us; T = 2000 283 -> 262; T = 1000
  // 75.9 -> 73.8).  Grids that
  // leave a partial round (T = 1500: 384 workgroups; 2500: 640) run slower
  // than the 64-query layout and keep it.
  bool split = false;
  const int layout = attention_layout(B, Tq, n_heads, products, &split);
  // The split-operand kernel (attn_bx_kernel) runs the 128-query layout and
  // the 64-query layout when its grid fits the CUs in one round (T = 500: 23.6
  // vs 26.2 us; T = 1000: 59.7 vs 81.2; T = 2000: 210 vs 275; T = 3000: 450
  // vs 571).  With 108 KB of LDS it keeps one workgroup per CU, so a 64-query
  // grid of several rounds (T = 1500: 181 vs 170 us) and the small grids stay
  // on the fp32 kernel, whose 70 KB (or single-buffered) LDS lets two
  // workgroups share a CU.
  // With three products (two bf16 parts per operand) the split kernel's K/V
  // planes take 72 KB (64-query layout), so two of its workgroups share a CU
  // and it also runs the 64-query grids of several rounds (T = 1500: 157 ->
  // 99 us; T = 2500: 416 -> 263 us against the fp32 kernel).
  const bool np3 = products == 3;
  // K / V as packed rows: the three-product split kernel only.
  LX_REQUIRE(!kv_packed || (split && np3),
             "attention: packed K/V need the three-product split kernel (B=%d Tq=%d)", B, Tq);
  auto pick = [&]() {
    if (split && np3 && kv_packed) {
      if (layout == 2)
        return buf ? attn_bx_kernel<4, 2, true, 3, true> : attn_bx_kernel<4, 2, false, 3, true>;
      return buf ? attn_bx_kernel<2, 2, true, 3, true> : attn_bx_kernel<2, 2, false, 3, true>;
    }
    if (split && np3) {
      if (layout == 2)
        return buf ? attn_bx_kernel<4, 2, true, 3> : attn_bx_kernel<4, 2, false, 3>;
      return buf ? attn_bx_kernel<2, 2, true, 3> : attn_bx_kernel<2, 2, false, 3>;
    }
    if (split) {
      if (layout == 2)
        return buf ? attn_bx_kernel<4, 2, true, 6> : attn_bx_kernel<4, 2, false, 6>;
      return buf ? attn_bx_kernel<2, 2, true, 6> : attn_bx_kernel<2, 2, false, 6>;
    }
    if (layout == 0)
      return buf ? attn_flash_kernel<1, 4, false, true> : attn_flash_kernel<1, 4, false, false>;
    return buf ? attn_flash_kernel<2, 2, true, true> : attn_flash_kernel<2, 2, true, false>;
  };
  auto kern = pick();
  const int qt = layout == 0 ? 32 : layout == 1 ? 64 : 128;
  const int threads = layout == 2 ? 512 : 256;
  const size_t lds =
      split ? (np3 ? (layout == 2 ? bx_lds<4, 2, 3>() : bx_lds<2, 2, 3>())
                   : (layout == 2 ? bx_lds<4, 2, 6>() : bx_lds<2, 2, 6>()))
            : (layout == 0 ? flash_lds<1, 4, false>() : flash_lds<2, 2, true>());
  const int variant = split ? 2 + (layout == 2) + 2 * np3 + 2 * (kv_packed != 0) : layout;
  static LdsLimit once[8][2];  // [kernel variant][buf]
  const int rc = raise_lds_limit((const void*)kern, lds, once[variant][buf], "attention");
  if (rc) return rc;
  const long nwg = (long)((Tq + qt - 1) / qt) * n_heads * B;
  LX_REQUIRE(nwg < (1L << 31), "attention: %ld workgroups exceed the grid limit", nwg);
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(threads), lds, stream, q, ldq, k, ldk, v, ldv,
                     o, ldo, Tq, Tk, n_heads, rep, scale * log2e, causal, q_offset,
                     out_packed ? 1 : 0);
  return check_launch("attn_flash_kernel");
}

}  // namespace lx

using namespace lx;

extern "C" int lx_attention_f32(const float* q, int ldq, const float* k, int ldk,
                                const float* v, int ldv, float* o, int ldo, int B, int Tq,
                                int Tk, int n_heads, int n_kv_heads, int head_dim, float scale,
                                int causal, int q_offset, hipStream_t stream) {
  return attention(q, ldq, k, ldk, v, ldv, o, ldo, B, Tq, Tk, n_heads, n_kv_heads, head_dim,
                   scale, causal, q_offset, 6, 0, stream, 0);
}

extern "C" int lx_attention_np_f32(const float* q, int ldq, const float* k, int ldk,
                                   const float* v, int ldv, float* o, int ldo, int B, int Tq,
                                   int Tk, int n_heads, int n_kv_heads, int head_dim, float scale,
                                   int causal, int q_offset, int products, int out_packed,
                                   int kv_packed, hipStream_t stream) {
  return attention(q, ldq, k, ldk, v, ldv, o, ldo, B, Tq, Tk, n_heads, n_kv_heads, head_dim,
                   scale, causal, q_offset, products, out_packed, stream, kv_packed);
}
