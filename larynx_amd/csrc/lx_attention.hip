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

template <int QS, int KS, bool DB, bool BUF>
__global__ __launch_bounds__(64 * QS * KS) void attn_flash_kernel(
    const float* __restrict__ q, int ldq, const float* __restrict__ k, int ldk,
    const float* __restrict__ v, int ldv, float* __restrict__ o, int ldo, int Tq, int Tk,
    int n_heads, int rep, float qscale, int causal, int q_offset) {
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
        *reinterpret_cast<floatx4*>(orow + g * 8) = w;
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
      *reinterpret_cast<floatx4*>(o + ((long)b * Tq + qi) * ldo + head * kHD + c) =
          *reinterpret_cast<const floatx4*>(src);
    }
  }
}

}  // namespace
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
  // threads, 70 KB: every K/V tile feeds twice the queries), replaces the
  // 64-query layout when its grid is a whole number of workgroups per CU: T = 3000 (768 workgroups)
  // 612 -> 571 us, T = 2000 283 -> 262, T = 1000 75.9 -> 73.8.  Grids that
  // leave a partial round (T = 1500: 384 workgroups; 2500: 640) run slower
  // than the 64-query layout and keep it.
  const long wg64 = (long)((Tq + 63) / 64) * n_heads * B;
  const long wg128 = (long)((Tq + 127) / 128) * n_heads * B;
  const int layout = wg64 < 256 ? 0 : (wg128 % 256 == 0 ? 2 : 1);  // small / 64-query / wide
  auto pick = [&]() {
    if (layout == 0)
      return buf ? attn_flash_kernel<1, 4, false, true> : attn_flash_kernel<1, 4, false, false>;
    if (layout == 2)
      return buf ? attn_flash_kernel<4, 2, true, true> : attn_flash_kernel<4, 2, true, false>;
    return buf ? attn_flash_kernel<2, 2, true, true> : attn_flash_kernel<2, 2, true, false>;
  };
  auto kern = pick();
  const int qt = layout == 0 ? 32 : layout == 1 ? 64 : 128;
  const int threads = layout == 2 ? 512 : 256;
  const size_t lds = layout == 0   ? flash_lds<1, 4, false>()
                     : layout == 1 ? flash_lds<2, 2, true>()
                                   : flash_lds<4, 2, true>();
  static LdsLimit once[3][2];  // [layout][buf]
  const int rc = raise_lds_limit((const void*)kern, lds, once[layout][buf], "attention");
  if (rc) return rc;
  const long nwg = (long)((Tq + qt - 1) / qt) * n_heads * B;
  LX_REQUIRE(nwg < (1L << 31), "attention: %ld workgroups exceed the grid limit", nwg);
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(threads), lds, stream, q, ldq, k, ldk, v, ldv,
                     o, ldo, Tq, Tk, n_heads, rep, scale * log2e, causal, q_offset);
  return check_launch("attn_flash_kernel");
}
