// Split-operand GEMM with the weights in MFMA fragment order.
//
// y = epi(x @ W^T + bias) as fp32 arithmetic on the bf16 matrix cores: every
// operand is three bf16 parts (x = x0 + x1 + x2, x0 = bf16(x), x1 = bf16(x -
// x0), x2 = bf16(x - x0 - x1)), each element pair is the six products a_i b_j
// with i + j <= 2 on v_mfma_f32_32x32x16_bf16, accumulated in fp32 (the same
// arithmetic as gemm_split_kernel).  The layout halves the per-CU LDS traffic
// of a tile:
//   - 4 waves per workgroup split the tile's 128 columns: wave w owns columns
//     n0 + 32 w .. n0 + 32 w + 31 for all BM rows (BM / 32 accumulators of
//     32 x 32).
//   - The A tile (BM rows x 32 k per slab) is split into its three bf16 planes
//     as it is staged, once, in LDS, and read by all four waves.  LDS rows are
//     64 bytes with the four 16-byte chunks XOR-swizzled by (row / 8) % 4
//     (conflict-free staging stores and fragment reads), four slab buffers.
//   - W is re-packed once (wfrag_pack) into fragment order: for each 32-row
//     block of W, 16-wide k step and plane, the 64 lanes' 16-byte B fragments
//     are one contiguous 1 KB.  Each wave streams its own columns' fragments
//     straight into registers three slabs ahead with coalesced loads; W never
//     passes through LDS.
//   - One barrier per slab, between its two k steps; the fragment reads,
//     staging stores and global loads are interleaved one per MFMA.
// Outputs: the fp32 epilogues of lx_linear_f32 (through an LDS tile, float4
// stores), or raw fp32 partial tiles of K slices (the consumer sums the slices
// in order).  With stream-K scratch, one workgroup per CU takes an equal share
// of the (tile, slab pair) work, so launches whose tiles do not fill the CUs
// in whole rounds still use all of them.
#include <algorithm>

#include "lx_common.hpp"
#include "lx_gemm_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {

constexpr int kBxWaves = 4;
constexpr int kBxThreads = 64 * kBxWaves;
constexpr int kBxBN = 32 * kBxWaves;  // columns per workgroup
constexpr int kBxBK = 32;             // k per slab: two 16-wide MFMA k steps
constexpr int kBxBufs = 4;            // A slab buffers (six products)

// NP products per element pair: 6 (three parts each, i + j <= 2) or 3 (two
// parts each: a0 b0 + a0 b1 + a1 b0); NP / 2 + 1 bf16 planes per operand.
#ifndef LX_BX_PD3
#define LX_BX_PD3 4
#endif
#ifndef LX_BX_NG3
#define LX_BX_NG3 2
#endif
template <int BMB, int NP>
struct BxCfg {
  static constexpr int BM = 32 * BMB;
  static constexpr int NPL = NP == 6 ? 3 : 2;
  // pipeline depth: PD slab buffers and W register sets, NG A staging sets
  static constexpr int PD = NP == 6 ? kBxBufs : LX_BX_PD3;
  static constexpr int NG = NP == 6 ? 2 : LX_BX_NG3;
  static_assert(PD % NG == 0 && PD >= NG + 2 && PD % 2 == 0, "pipeline depth");
  static constexpr int ABUF = NPL * BM * kBxBK;  // bf16 per A slab buffer (NPL planes)
  static constexpr size_t lds_k = (size_t)PD * ABUF * 2;
  static constexpr size_t lds_c = (size_t)BM * (kBxBN + 4) * 4;
  static constexpr size_t lds = lds_k > lds_c ? lds_k : lds_c;
};

struct BxArgs {
  const float* A;  // (M, lda)
  long lda;
  const __bf16* Wf;  // W (N, K) in fragment order (wfrag_pack)
  const float* bias;
  float* Y;  // fp32 output rows (ldy), or partial slices slice_stride floats apart
  long ldy;
  long slice_stride;
  int M, N, K, kslice, tiles_m, tiles_n, slices;
  int streamk;          // 1: stream-K over `grid` workgroups; 2: split tail (ws and counters set)
  int grid;
  float* ws;            // partial tiles: stream-K 2 per workgroup, split tail 1 per split
                        // workgroup, BM * 128 floats each
  int ws_bytes;
  unsigned* counters;   // arrival counts, one per tile, zero between launches
  int split_full;       // split tail: tiles [0, split_full) run whole, one workgroup each;
  int split_s;          // every later tile runs as split_s workgroups of consecutive k ranges
};

enum { BX_OUT_F32 = LX_BX_OUT_F32, BX_OUT_PARTIAL = LX_BX_OUT_PARTIAL, BX_OUT_PACKED = LX_BX_OUT_PACKED };

// Fragments are held as 32-bit vectors (uintx4_t) and reinterpreted as bf16
// only at the MFMA (loop-carried bf16 vectors are otherwise rebuilt element by
// element).
__device__ __forceinline__ sbf16x8 as_bf16x8(uintx4_t v) { return __builtin_bit_cast(sbf16x8, v); }

// Three bf16 parts of four fp32 values.
__device__ __forceinline__ void split3(floatx4 v, bf16x4_t& x0, bf16x4_t& x1, bf16x4_t& x2) {
  x0 = __builtin_convertvector(v, bf16x4_t);
  const floatx4 r = v - bf16x4_back(x0);
  x1 = __builtin_convertvector(r, bf16x4_t);
  x2 = __builtin_convertvector(r - bf16x4_back(x1), bf16x4_t);
}

// Stream-K partial tiles: a launch of G workgroups over `tiles` output tiles
// of npt slab pairs each gives workgroup w the units [w U / G, (w + 1) U / G)
// of the U = tiles * npt (tile, pair) units.  A tile that several workgroups
// share is finished by the last one to arrive: each publishes its partial
// tile (slot 2 w for its first segment, 2 w + 1 for its last) and counts its
// arrival; the last sums the contributors' partials in k order (workgroup
// order), adds the epilogue, and clears the count for the next launch.  No
// workgroup waits for another.
__device__ __forceinline__ int bx_owner(long p, long U, int G) {
  return (int)(((p + 1) * G - 1) / U);
}

// 128-row tiles run one wave per SIMD: the register budget holds two k steps
// of A fragments and four slabs of W fragments, so the scheduler must not
// trade them away for a second wave.  64-row tiles fit two waves per SIMD (two
// workgroups per CU), which cover each other's waits.
#ifndef LX_BX_WAVES64
#define LX_BX_WAVES64 2
#endif
// AP: A holds two-part packed rows (pack2_bf16; three products): the staging
// stores its parts without splitting them.  OUT = BX_OUT_PACKED: the fp32
// epilogue's result is stored as packed rows for the next such GEMM.
template <int EPI, int BMB, int OUT, int NP, int AP = 0>
__global__ __launch_bounds__(kBxThreads) __attribute__((amdgpu_waves_per_eu(
    BMB == 2 ? LX_BX_WAVES64 : 1, BMB == 2 ? LX_BX_WAVES64 : 1))) void
gemm_bx_kernel(BxArgs a, EpiArgs ep) {
  using Cfg = BxCfg<BMB, NP>;
  constexpr int BM = Cfg::BM, ABUF = Cfg::ABUF, NPL = Cfg::NPL;
  constexpr int LA = 8 * BM / kBxThreads;  // A float4 per thread per slab
  static_assert(LA * kBxThreads == 8 * BM, "staging slots");
  constexpr int SLOTS = BM * kBxBN / 4 / kBxThreads;  // epilogue float4 slots per thread
  extern __shared__ __attribute__((aligned(16))) __bf16 sm[];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int tiles = a.tiles_m * a.tiles_n * a.slices;
  const int npt = a.kslice / (2 * kBxBK);  // slab pairs per tile
  const int G = gridDim.x;
  int w = blockIdx.x;
  {
    // the dispatcher deals workgroups round-robin over the 8 XCDs: give each
    // XCD a contiguous run of work (tiles ordered (slice, N tile, M tile)) so
    // that its L2 holds a few W column blocks and the A rows they meet
    const int full = G / 8 * 8;
    if (w < full) w = (w % 8) * (full / 8) + w / 8;
  }
  const long U = (long)tiles * npt;
  // data-parallel: one tile per workgroup, its slice's slab pairs (the last
  // slice may hold fewer); stream-K (one slice): an equal share of all of them
  const int tile_pairs =
      min(npt, a.K / (2 * kBxBK) - (w / (a.tiles_m * a.tiles_n)) * npt);
  long u0 = a.streamk == 1 ? (long)w * U / G : (long)w * npt;
  long u1 = a.streamk == 1 ? (long)(w + 1) * U / G : u0 + tile_pairs;
  // Split tail (one slice): each XCD's first split_full / 8 workgroups take
  // whole tiles, its next ones the k ranges of the later tiles (split_s per
  // tile, consecutive), so the dispatcher's first round puts one whole tile
  // and its second at most one part of a split tile on every CU.  sid numbers
  // the split workgroups (their partial tile slot).
  int sid = -1;
  if (a.streamk == 2) {
    const int x = blockIdx.x & 7, i = blockIdx.x >> 3;
    const int fx = a.split_full >> 3, sx = (G - a.split_full) >> 3;
    if (i < fx) {
      u0 = (long)(x * fx + i) * npt;
      u1 = u0 + npt;
    } else {
      sid = x * sx + (i - fx);
      const int t = a.split_full + sid / a.split_s, p = sid % a.split_s;
      u0 = (long)t * npt + p * npt / a.split_s;
      u1 = (long)t * npt + (p + 1) * npt / a.split_s;
    }
  }
  constexpr int SLAB_BYTES = kBxBK * 4;  // A bytes per row per slab
  // A fragments: row block i, plane p, k step st of a slab buffer
  const int aoff = fr * kBxBK;
  const int fc0 = split_col(fr, fh * 8), fc1 = split_col(fr, 16 + fh * 8);
  // The products (A part, W part), the small terms first: six as in
  // mfma_split6x, or the three of the two-part splits.
  constexpr int kPa6[6] = {2, 1, 0, 1, 0, 0}, kPw6[6] = {0, 1, 2, 0, 1, 0};
  constexpr int kPa3[3] = {1, 0, 0}, kPw3[3] = {0, 1, 0};
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(a.ws, (short)0, a.ws_bytes, 0x00020000);
  constexpr int kSc1 = 16;  // cache-policy bits: sc1 = device scope
  floatx16 acc[BMB];
  bool first_seg = true;
  for (long u = u0; u < u1;) {
    const int t = (int)(u / npt);
    const int q0 = (int)(u - (long)t * npt);
    const long uend = min(u1, (long)(t + 1) * npt);
    const int q1 = (int)(uend - (long)t * npt);
    u = uend;
    const int slot = a.streamk == 2 ? sid : first_seg ? 2 * w : 2 * w + 1;
    if (!first_seg) __syncthreads();  // the last segment's epilogue is done with the LDS
    first_seg = false;
    const int mt = t % a.tiles_m;
    const int rest = t / a.tiles_m;
    const int nt = rest % a.tiles_n;
    const int slice = rest / a.tiles_n;
    const int m0 = mt * BM, n0 = nt * kBxBN;
    const int kb = slice * a.kslice + q0 * 2 * kBxBK;
    const int nk = (q1 - q0) * 2;

    // A staging sources and LDS destinations (bf16 units)
    // (rows past M repeat the last row; they only reach unstored outputs).
    // Byte offsets from a workgroup-uniform base: A stays below 2 GiB.
    const char* abase = reinterpret_cast<const char*>(a.A + kb);
    int pa[LA], sa[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + kBxThreads * i;
      const int row = idx / 8, c = (idx % 8) * 4;
      pa[i] = (min(m0 + row, a.M - 1) * (int)a.lda + c) * 4;
      sa[i] = row * kBxBK + split_col(row, c);
    }
    auto load_a = [&](floatx4* g, int s) {
#pragma unroll
      for (int i = 0; i < LA; ++i)
        g[i] = *reinterpret_cast<const floatx4*>(abase + pa[i] + s * SLAB_BYTES);
    };
    auto store_a = [&](const floatx4* g, int buf) {
      __bf16* base = sm + buf * ABUF;
#pragma unroll
      for (int i = 0; i < LA; ++i) {
        bf16x4_t x0, x1, x2;
        if (AP) {  // already split by the producer
          const uintx4_t u = __builtin_bit_cast(uintx4_t, g[i]);
          x0 = __builtin_bit_cast(bf16x4_t, uintx2_t{u[0], u[1]});
          x1 = __builtin_bit_cast(bf16x4_t, uintx2_t{u[2], u[3]});
          x2 = x1;
        } else {
          split3(g[i], x0, x1, x2);  // (x2 is dead code with two planes)
        }
        *reinterpret_cast<bf16x4_t*>(base + sa[i]) = x0;
        *reinterpret_cast<bf16x4_t*>(base + BM * kBxBK + sa[i]) = x1;
        if (NPL == 3) *reinterpret_cast<bf16x4_t*>(base + 2 * BM * kBxBK + sa[i]) = x2;
      }
    };
    // W fragments of this wave's 32 columns: k step ks, plane p at wf + (ks * 3 + p) * 512;
    // the three planes of k step st of slab s
    const int nks = a.K / 16;
    const char* wf = reinterpret_cast<const char*>(
        a.Wf + ((long)(n0 / 32 + wave) * nks + kb / 16) * 3 * 512);  // wave-uniform
    const int wl = lane * 16;
    auto load_w = [&](uintx4_t* wv, int s, int st) {
#pragma unroll
      for (int j = 0; j < NPL; ++j)
        wv[j] = *reinterpret_cast<const uintx4_t*>(wf + wl + (s * 6 + st * 3 + j) * 1024);
    };
    auto read_a = [&](uintx4_t (*f)[3], int buf, int st) {
      const __bf16* base = sm + buf * ABUF + aoff + (st ? fc1 : fc0);
#pragma unroll
      for (int i = 0; i < BMB; ++i)
#pragma unroll
        for (int p = 0; p < NPL; ++p)
          f[i][p] = *reinterpret_cast<const uintx4_t*>(base + p * BM * kBxBK + i * 32 * kBxBK);
    };
#pragma unroll
    for (int i = 0; i < BMB; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    auto mul = [&](uintx4_t (*f)[3], const uintx4_t* wv) {
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int i = 0; i < BMB; ++i)
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(f[i][NP == 6 ? kPa6[q] : kPa3[q]]),
              as_bf16x8(wv[NP == 6 ? kPw6[q] : kPw3[q]]), acc[i], 0, 0, 0);
    };
    // Registers: A fragments of the two k steps (fa0, fa1); the W fragments of
    // PD slabs (slab s in set s % PD: k step 0's planes, then k step 1's); NG A
    // staging sets (slab s uses set s % NG).  LDS: PD slab buffers (slab s in
    // buffer s % PD).  At slab s the A tile of slab s + PD - 1 is split into
    // LDS (from the staging set, loaded NG slabs earlier) and the A tile of
    // slab s + PD - 1 + NG is loaded into it; the W fragments of slab s + PD - 1
    // are loaded into the set slab s - 1 has finished with.  Latency cover:
    // A NG slabs of MFMAs, W PD - 1.  Both product counts run PD = 4, NG = 2:
    // with three products (half the MFMAs per slab) the deeper PD = 6, NG = 3
    // fits the registers but measured slower (T = 500 FF0 20.5 -> 21.3 us,
    // Euler step 2.82 -> 2.86 ms), so the loads are not waiting on latency.
    constexpr int PD = Cfg::PD, NG = Cfg::NG;
    uintx4_t fa0[BMB][3], fa1[BMB][3];
    uintx4_t wv[PD][6];
    floatx4 gst[NG][LA];
    auto load_ws = [&](uintx4_t* w, int s) {
      load_w(w, s, 0);
      load_w(w + 3, s, 1);
    };
    // Every prefetch is unconditional (indices clamped to the last slab; the
    // surplus slabs go to buffers nobody reads), so each body issues its
    // global loads in one fixed order: slab j issues A(j + PD - 1 + NG), then
    // W(j + PD - 1).  The prologue first loads and stores A(0 .. PD - 2) and
    // loads W(0 .. PD - 2 - NG), then issues the loads of the virtual slabs
    // j = -NG .. -1 in that same order, so the waits the compiler derives
    // (from the merge of both paths into the loop) never stall on a recent
    // load.
    const int last = nk - 1;
    {
      floatx4 pre[PD - 1][LA];  // A(0 .. PD - 2) in flight together: one memory latency
#pragma unroll
      for (int i = 0; i < PD - 1; ++i) load_a(pre[i], min(i, last));
#pragma unroll
      for (int i = 0; i <= PD - 2 - NG; ++i) load_ws(wv[i], min(i, last));
#pragma unroll
      for (int i = 0; i < PD - 1; ++i) store_a(pre[i], i);
#pragma unroll
      for (int j = -NG; j < 0; ++j) {
        load_a(gst[(j + NG) % NG], min(j + PD - 1 + NG, last));
        load_ws(wv[(j + PD - 1 + PD) % PD], min(j + PD - 1, last));
      }
    }
    __syncthreads();
    read_a(fa0, 0, 0);
    // Slab s.  k step 0: its MFMAs, beside them the fragment reads of k step
    // 1, the staging of slab s + PD - 1 (into slab s - 1's buffer) and the loads
    // of slab s + PD - 1 + NG (into the staging set just stored).  Then the
    // barrier (k step 1's fragments and slab s + PD - 1 are in LDS; every wave
    // is past its reads of slab s - 1's buffer).  k step 1: its MFMAs, beside
    // them the next slab's k step 0 fragment reads and the W of slab s + PD - 1
    // (into slab s - 1's register set).  The group barriers interleave one
    // memory instruction per MFMA so that the matrix pipe keeps issuing while
    // they go out.
    constexpr int NM = NP * BMB;           // MFMAs per k step
    constexpr int NR = NPL * BMB;          // fragment reads per k step
    constexpr int NW = NPL * LA;           // staging LDS stores
    // i = s % PD (a compile-time constant in every call)
    auto body = [&](int s, int i) {
      const int b = i;
      uintx4_t* wc = wv[i];
      uintx4_t* wn = wv[(i + PD - 1) % PD];
      floatx4* g = gst[i % NG];
      read_a(fa1, b, 1);
      store_a(g, (b + PD - 1) % PD);
      load_a(g, min(s + PD - 1 + NG, last));
      mul(fa0, wc);
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      }
#pragma unroll
      for (int k = 0; k < LA; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (A)
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
      __builtin_amdgcn_sched_barrier(0);  // k step 1's MFMAs stay below the barrier
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      read_a(fa0, (b + 1) % PD, 0);
      load_ws(wn, min(s + PD - 1, last));
      mul(fa1, wc + 3);
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      }
#pragma unroll
      for (int k = 0; k < 2 * NPL; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);  // VMEM read (W)
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NM, 1);
      __builtin_amdgcn_sched_barrier(0);
    };
    int s = 0;
    for (; s + PD <= nk; s += PD) {
#pragma unroll
      for (int i = 0; i < PD; ++i) body(s + i, i);
    }
    // nk is even: the rest is an even number of slabs below PD
#pragma unroll
    for (int i = 0; i + 2 < PD; i += 2) {
      if (s + i < nk) {
        body(s + i, i);
        body(s + i + 1, i + 1);
      }
    }
    __syncthreads();

    // Accumulator element e of lane l in row block i is row 32 i + (e / 4) * 8
    // + (l / 32) * 4 + e % 4, column 32 wave + l % 32.
    if (OUT == BX_OUT_PARTIAL) {
      float* P = a.Y + slice * a.slice_stride + n0 + 32 * wave + fr;
#pragma unroll
      for (int i = 0; i < BMB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + 32 * i + (e >> 2) * 8 + fh * 4 + (e & 3);
          if (m < a.M) P[(long)m * a.ldy] = acc[i][e];
        }
      continue;
    }
    if (q0 != 0 || q1 != npt) {
      // Shared tile: publish this segment's partial products (fragment order,
      // 1 KB per store instruction, device-scope stores: the contributors run
      // on different XCDs) and count the arrival.
      const int pbase = slot * (BM * kBxBN) * 4 + ((wave * BMB) * 4 * 64 + lane) * 16;
#pragma unroll
      for (int i = 0; i < BMB; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 v = {acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2],
                             acc[i][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(v, prs, pbase + (i * 4 + q) * 64 * 16, 0, kSc1);
        }
      __builtin_amdgcn_s_waitcnt(0);  // the stores are performed before the count
      const long tu0 = (long)t * npt;
      // the tile's contributors, in k order: stream-K workgroups cf..cl, or
      // split workgroups (sid) cf..cl
      const int cf = a.streamk == 2 ? (t - a.split_full) * a.split_s : bx_owner(tu0, U, G);
      const int cl = a.streamk == 2 ? cf + a.split_s - 1 : bx_owner(tu0 + npt - 1, U, G);
      const int own = a.streamk == 2 ? sid : w;
      __syncthreads();
      if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.counters + t, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(cl - cf);
      __syncthreads();
      if (!s_last) continue;
      // Last to arrive: the contributors' partials in workgroup (= k) order,
      // two contributors' loads in flight at a time.
      floatx16 tot[BMB];
      auto part = [&](floatx16* pv, int c) {
        if (c == own) {
#pragma unroll
          for (int i = 0; i < BMB; ++i) pv[i] = acc[i];
          return;
        }
        // c's first segment starts inside this tile, else this tile is its last
        // (a split workgroup has one slot)
        const int cs = a.streamk == 2 ? c : (long)c * U / G >= tu0 ? 2 * c : 2 * c + 1;
        const int cb = cs * (BM * kBxBN) * 4 + ((wave * BMB) * 4 * 64 + lane) * 16;
#pragma unroll
        for (int i = 0; i < BMB; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const floatx4 v =
                __builtin_amdgcn_raw_buffer_load_b128(prs, cb + (i * 4 + q) * 64 * 16, 0, kSc1);
            pv[i][4 * q] = v[0];
            pv[i][4 * q + 1] = v[1];
            pv[i][4 * q + 2] = v[2];
            pv[i][4 * q + 3] = v[3];
          }
      };
      for (int c = cf; c <= cl; c += 2) {
        floatx16 p0[BMB], p1[BMB];
        part(p0, c);
        if (c + 1 <= cl) part(p1, c + 1);
#pragma unroll
        for (int i = 0; i < BMB; ++i) {
          tot[i] = c == cf ? p0[i] : tot[i] + p0[i];
          if (c + 1 <= cl) tot[i] += p1[i];
        }
      }
#pragma unroll
      for (int i = 0; i < BMB; ++i) acc[i] = tot[i];
      if (tid == 0)
        __hip_atomic_store(a.counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Epilogue: its per-row global operands (residual, gate, position) are
    // loaded first, then the tile goes through LDS into row-contiguous float4
    // slots.  The bias (one 512-byte row per tile) is read where it is used.
    // (64-row tiles, two waves per SIMD, load them in the slot loop instead:
    // the prefetch would not fit their register budget.)
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    constexpr bool PRE = BMB == 4;
    float4 eg[SLOTS], ey[SLOTS];
    // Rotary epilogue: only tiles that hold rotated columns read positions.
    bool rot = false;
    if (EPI == LX_EPI_ROPE_PARTIAL)
      for (int k = 0; k < ep.sections; ++k)
        rot |= n0 < k * ep.section + ep.rot_dim && n0 + kBxBN > k * ep.section;
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      if (!PRE) break;
      const int idx = tid + j * kBxThreads;
      const int row = idx / (kBxBN / 4), c = (idx % (kBxBN / 4)) * 4;
      const int m = min(m0 + row, a.M - 1), n = n0 + c;
      eg[j] = ey[j] = z4;
      if (OUT != BX_OUT_PARTIAL) {
        if (EPI == LX_EPI_GATED_RESID)
          eg[j] = *reinterpret_cast<const float4*>(ep.gate + (long)(m / ep.rows_per_batch) *
                                                                 ep.gate_stride + n);
        if (EPI == LX_EPI_GATED_RESID || EPI == LX_EPI_RESID)
          ey[j] = *reinterpret_cast<const float4*>(a.Y + (long)m * a.ldy + n);
      }
    }
    constexpr int LDC = kBxBN + 4;
    float* Cs = reinterpret_cast<float*>(sm);
#pragma unroll
    for (int i = 0; i < BMB; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * i + (e >> 2) * 8 + fh * 4 + (e & 3);
        Cs[row * LDC + 32 * wave + fr] = acc[i][e];
      }
    __syncthreads();
    // The slot addresses are formed here from an opaque copy of the thread
    // id: hoisted to the kernel's entry they would stay live through the main
    // loop, past the register budget of the 64-row tiles.
    int etid = tid;
    asm volatile("" : "+v"(etid));
    // A thread's slots share their 4 columns (kBxThreads is a multiple of the
    // 32 float4 per row): the bias is one float4, loaded once before the first
    // store (reloaded after each store to Y, it waited for a round trip).
    const int ec = (etid % (kBxBN / 4)) * 4;
    const float4 eb = a.bias ? *reinterpret_cast<const float4*>(a.bias + n0 + ec) : z4;
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int idx = etid + j * kBxThreads;
      const int row = idx / (kBxBN / 4);
      const int m = m0 + row, n = n0 + ec;
      if (m >= a.M) continue;
      const float4 v = *reinterpret_cast<const float4*>(Cs + row * LDC + ec);
      if (!PRE) {
        eg[j] = ey[j] = z4;
        if (EPI == LX_EPI_GATED_RESID)
          eg[j] = *reinterpret_cast<const float4*>(ep.gate + (long)(m / ep.rows_per_batch) *
                                                                 ep.gate_stride + n);
        if (EPI == LX_EPI_GATED_RESID || EPI == LX_EPI_RESID)
          ey[j] = *reinterpret_cast<const float4*>(a.Y + (long)m * a.ldy + n);
      }
      const int posm = rot ? ep.pos[m % ep.rows_per_batch] : 0;
      epilogue4v<EPI, OUT == BX_OUT_PACKED>(a.Y, (int)a.ldy, m, n, v, eb, eg[j], ey[j], posm, ep);
    }
  }
}

// W (N, K) fp32 -> fragment order: Wf[((nb * nks + ks) * 3 + p) * 512 + l * 8 + j]
// = part p of W[nb * 32 + l % 32][ks * 16 + (l / 32) * 8 + j] (nks = K / 16),
// the B operand of v_mfma_f32_32x32x16_bf16 for lane l.  The parts are the
// rounding of split_planes.
__global__ void wfrag_pack_kernel(const float* __restrict__ W, __bf16* __restrict__ Wf, int N,
                                  int K) {
  const int nks = K / 16;
  const long total = (long)(N / 32) * nks * 64;
  const long t = blockIdx.x * 256L + threadIdx.x;
  if (t >= total) return;
  const int l = (int)(t % 64);
  const long r = t / 64;
  const int ks = (int)(r % nks);
  const long nb = r / nks;
  const float* src = W + (nb * 32 + l % 32) * (long)K + ks * 16 + (l / 32) * 8;
  __bf16* dst = Wf + (nb * nks + ks) * 3 * 512 + l * 8;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(src + 4 * h);
    bf16x4_t x0, x1, x2;
    split3(v, x0, x1, x2);
    *reinterpret_cast<bf16x4_t*>(dst + 4 * h) = x0;
    *reinterpret_cast<bf16x4_t*>(dst + 512 + 4 * h) = x1;
    *reinterpret_cast<bf16x4_t*>(dst + 1024 + 4 * h) = x2;
  }
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int EPI, int BMB, int OUT, int NP, int AP>
int launch_bx(const BxArgs& a, const EpiArgs& ep, hipStream_t stream) {
  auto kern = gemm_bx_kernel<EPI, BMB, OUT, NP, AP>;
  static LdsLimit once;
  const size_t lds = BxCfg<BMB, NP>::lds;
  int rc = raise_lds_limit((const void*)kern, lds, once, "linear_bx");
  if (rc) return rc;
  const long nwg = a.streamk ? a.grid : (long)a.tiles_m * a.tiles_n * a.slices;
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(kBxThreads), lds, stream, a, ep);
  return check_launch("gemm_bx_kernel");
}

// Packed operands exist for three products (AP = 1 on 64- and 128-row tiles,
// BX_OUT_PACKED on 64-row tiles; the host checks this).
template <int BMB, int NP, int AP = 0>
int dispatch_bx(const BxArgs& a, int out, const EpiArgs& ep, hipStream_t s) {
  if (out == BX_OUT_PARTIAL) return launch_bx<LX_EPI_NONE, BMB, BX_OUT_PARTIAL, NP, AP>(a, ep, s);
  if constexpr (BMB == 2 && NP == 3) {
    if (out == BX_OUT_PACKED) {
      if (ep.kind == LX_EPI_GELU_TANH)
        return launch_bx<LX_EPI_GELU_TANH, BMB, BX_OUT_PACKED, NP, AP>(a, ep, s);
      if (ep.kind == LX_EPI_ROPE_PARTIAL)
        return launch_bx<LX_EPI_ROPE_PARTIAL, BMB, BX_OUT_PACKED, NP, AP>(a, ep, s);
      return launch_bx<LX_EPI_NONE, BMB, BX_OUT_PACKED, NP, AP>(a, ep, s);
    }
  }
  switch (ep.kind) {
    case LX_EPI_NONE: return launch_bx<LX_EPI_NONE, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    case LX_EPI_GELU_TANH: return launch_bx<LX_EPI_GELU_TANH, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    case LX_EPI_GATED_RESID:
      return launch_bx<LX_EPI_GATED_RESID, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    case LX_EPI_ROPE_PARTIAL:
      return launch_bx<LX_EPI_ROPE_PARTIAL, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    case LX_EPI_RESID: return launch_bx<LX_EPI_RESID, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    case LX_EPI_SWIGLU_PAIRED:
      return launch_bx<LX_EPI_SWIGLU_PAIRED, BMB, BX_OUT_F32, NP, AP>(a, ep, s);
    default: break;
  }
  set_error("linear_bx: epilogue kind %d not available", ep.kind);
  return LX_ERR_ARG;
}

}  // namespace

int bx_split_parts(int M, int N, int K, int bm) {
  // S: the most parts per split tile (at most 8, at most K / 64) with the split
  // workgroups filling at most the CUs' second round in whole XCD shares
  const int cus = device_cus();
  const int tiles = ((M + bm - 1) / bm) * (N / kBxBN);
  const int npt = K / (2 * kBxBK);
  if (cus % 8 || tiles <= cus || tiles >= 2 * cus) return 0;
  for (int sp = std::min(8, cus / (tiles - cus)); sp >= 2; --sp)
    if ((tiles - cus) * sp % 8 == 0 && npt >= sp) return sp;
  return 0;
}

size_t bx_split_ws_floats(int bm) { return (size_t)device_cus() * bm * kBxBN; }

int wfrag_pack(const float* W, void* Wf, int N, int K, hipStream_t stream) {
  LX_REQUIRE(W && Wf && N > 0 && K > 0 && N % 32 == 0 && K % 16 == 0,
             "wfrag_pack: bad shape N=%d K=%d", N, K);
  LX_REQUIRE(((uintptr_t)W | (uintptr_t)Wf) % 16 == 0, "wfrag_pack: unaligned");
  const long total = (long)(N / 32) * (K / 16) * 64;
  hipLaunchKernelGGL(wfrag_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     stream, W, static_cast<__bf16*>(Wf), N, K);
  return check_launch("wfrag_pack_kernel");
}

int linear_bx(const lx_linear_bx& g, hipStream_t stream) {
  LX_REQUIRE(g.A && g.Wf, "linear_bx: null operand");
  LX_REQUIRE(g.M > 0 && g.N > 0 && g.K > 0 && g.N % kBxBN == 0 && g.K % (2 * kBxBK) == 0,
             "linear_bx: bad shape M=%d N=%d K=%d (N %% 128, K %% 64)", g.M, g.N, g.K);
  LX_REQUIRE(g.bm == 64 || g.bm == 128, "linear_bx: bm=%d must be 64 or 128", g.bm);
  LX_REQUIRE(g.products == 0 || g.products == 3 || g.products == 6,
             "linear_bx: products=%d must be 3 or 6 (0: 6)", g.products);
  LX_REQUIRE(g.lda >= g.K && g.lda % 4 == 0 && (long)g.M * g.lda * 4 < (1L << 31),
             "linear_bx: lda=%ld (K=%d), A must stay below 2 GiB", g.lda, g.K);
  LX_REQUIRE(((uintptr_t)g.A | (uintptr_t)g.Wf) % 16 == 0,
             "linear_bx: operands must be 16-byte aligned");
  LX_REQUIRE(g.out == BX_OUT_F32 || g.out == BX_OUT_PARTIAL || g.out == BX_OUT_PACKED,
             "linear_bx: unknown output %d", g.out);
  LX_REQUIRE(g.a_packed == 0 || g.a_packed == 1, "linear_bx: a_packed=%d must be 0 or 1",
             g.a_packed);
  LX_REQUIRE((!g.a_packed || g.products == 3) && (g.out != BX_OUT_PACKED ||
                                                   (g.products == 3 && g.bm == 64)),
             "linear_bx: packed operands need three products (the packed output 64-row tiles)");
  const int slices = g.slices < 1 ? 1 : g.slices;
  int kslice = g.K;
  if (slices > 1) {
    LX_REQUIRE(g.out == BX_OUT_PARTIAL, "linear_bx: K slices need the partial output");
    // slices of ceil(pairs / slices) 64-wide steps, the last one the rest
    const int pairs = g.K / (2 * kBxBK), per = (pairs + slices - 1) / slices;
    LX_REQUIRE((slices - 1) * per < pairs,
               "linear_bx: K=%d leaves slice %d of %d empty (slices of %d 64-wide steps)", g.K,
               slices - 1, slices, per);
    kslice = per * 2 * kBxBK;
  }
  EpiArgs ep;
  int rc = make_epi(g.epi, g.N, &ep);
  if (rc) return rc;
  if (g.out == BX_OUT_PARTIAL) {
    LX_REQUIRE(g.Y && g.ldy >= g.N && (slices == 1 || g.slice_stride >= (long)g.M * g.ldy),
               "linear_bx: bad partial output");
  } else {
    LX_REQUIRE(g.out != BX_OUT_PACKED || ep.kind == LX_EPI_NONE || ep.kind == LX_EPI_GELU_TANH ||
                   ep.kind == LX_EPI_ROPE_PARTIAL,
               "linear_bx: the packed output takes no epilogue, GELU or rotary (kind %d)",
               ep.kind);
    LX_REQUIRE(g.pack_from >= 0 && g.pack_from % 4 == 0 && (g.pack_from == 0 || g.out == BX_OUT_PACKED),
               "linear_bx: pack_from=%d must be a multiple of 4 (packed output)", g.pack_from);
    ep.pack_from = g.pack_from;
    LX_REQUIRE(g.Y && g.ldy >= (ep.kind == LX_EPI_SWIGLU_PAIRED ? g.N / 2 : g.N) &&
                   g.ldy < (1L << 31),
               "linear_bx: bad output");
    ep.vec = epi_vec_ok(ep, g.Y, (int)g.ldy, g.bias);
    LX_REQUIRE(ep.vec, "linear_bx: y, bias and gate must be 16-byte aligned");
  }
  BxArgs a;
  a.A = g.A;
  a.lda = g.lda;
  a.Wf = static_cast<const __bf16*>(g.Wf);
  a.bias = g.bias;
  a.Y = g.Y;
  a.ldy = g.ldy;
  a.slice_stride = g.slice_stride;
  a.M = g.M;
  a.N = g.N;
  a.K = g.K;
  a.kslice = kslice;
  a.tiles_m = (g.M + g.bm - 1) / g.bm;
  a.tiles_n = g.N / kBxBN;
  a.slices = slices;
  LX_REQUIRE((long)a.tiles_m * a.tiles_n * slices < (1L << 31), "linear_bx: too many tiles");
  a.streamk = 0;
  a.grid = 0;
  a.ws = nullptr;
  a.ws_bytes = 0;
  a.counters = nullptr;
  a.split_full = 0;
  a.split_s = 0;
  LX_REQUIRE(g.split_tail == 0 || g.split_tail == 1, "linear_bx: split_tail=%d must be 0 or 1",
             g.split_tail);
  if (g.split_tail && g.ws && g.counters && slices == 1 && g.out != BX_OUT_PARTIAL) {
    // whole tiles on the first round of CUs, the rest split along K onto the
    // second, so that no CU holds two whole tiles
    const int cus = device_cus();
    const int tiles = a.tiles_m * a.tiles_n;
    const int S = bx_split_parts(g.M, g.N, g.K, g.bm);
    const int G = cus + (tiles - cus) * S;
    const size_t need = (size_t)(G - cus) * g.bm * kBxBN;
    if (S && tiles <= g.n_counters && need <= g.ws_floats && need * 4 < (1u << 31)) {
      a.streamk = 2;
      a.grid = G;
      a.split_full = cus;
      a.split_s = S;
      a.ws = g.ws;
      a.ws_bytes = (int)(need * 4);
      a.counters = g.counters;
    }
  } else if (g.ws && g.counters && g.out == BX_OUT_F32 && !g.a_packed) {
    // Stream-K over one workgroup per CU (at most one per slab pair of work):
    // every CU gets the same number of slab pairs whatever the tile count.
    const int tiles = a.tiles_m * a.tiles_n;
    const long units = (long)tiles * (g.K / (2 * kBxBK));
#ifndef LX_BX_SK_SLOTS64
#define LX_BX_SK_SLOTS64 1
#endif
    const int G = (int)std::min<long>(device_cus() * (g.bm == 64 ? LX_BX_SK_SLOTS64 : 1), units);
    const size_t need = (size_t)2 * G * g.bm * kBxBN;
    if (tiles <= g.n_counters && need <= g.ws_floats && need * 4 < (1u << 31)) {
      a.streamk = 1;
      a.grid = G;
      a.ws = g.ws;
      a.ws_bytes = (int)(need * 4);
      a.counters = g.counters;
    }
  }
  if (g.a_packed)
    return g.bm == 128 ? dispatch_bx<4, 3, 1>(a, g.out, ep, stream)
                       : dispatch_bx<2, 3, 1>(a, g.out, ep, stream);
  if (g.products == 3)
    return g.bm == 128 ? dispatch_bx<4, 3>(a, g.out, ep, stream)
                       : dispatch_bx<2, 3>(a, g.out, ep, stream);
  return g.bm == 128 ? dispatch_bx<4, 6>(a, g.out, ep, stream)
                     : dispatch_bx<2, 6>(a, g.out, ep, stream);
}

}  // namespace lx

using namespace lx;

extern "C" int lx_wfrag_pack_f32(const float* W, void* Wf, int N, int K, hipStream_t stream) {
  return wfrag_pack(W, Wf, N, K, stream);
}

extern "C" int lx_linear_bx_f32(const lx_linear_bx* g, hipStream_t stream) {
  LX_REQUIRE(g, "linear_bx: null argument");
  return linear_bx(*g, stream);
}
