// fp32 projection GEMM on the CDNA4 matrix cores: y = epi(x @ W^T + bias).
//
//   - v_mfma_f32_32x32x2f32, fp32 in / fp32 accumulate (no reduced-precision
//     shortcut: the reference pins fp32 GEMMs, cf. its TF32 ADR).
//   - Output tiles of BM x BN per workgroup, 32x32 accumulators per wave64; K
//     staged through LDS in BK-wide slabs, double buffered, the next slab's
//     global loads in flight during the current slab's MFMAs.
//   - Intra-workgroup split-K (KS groups of waves on disjoint K slabs, reduced
//     through LDS in a fixed order) raises the waves per SIMD for the small-M
//     DiT shapes (M = 2 x 500 rows gives only 256 tiles of 64 x 64 for N = 1024,
//     one per CU) without atomics, so results stay bit-reproducible.
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
#include "lx_gemm_common.hpp"
#include "lx_internal.hpp"

namespace lx {
namespace {


// Split tail: when a launch's tiles leave a partial last round over the CUs,
// the first n_full tiles run whole and each of the remaining tiles runs as
// `splits` K slices of `ksplit` columns (workgroups n_full + tile * splits +
// slice).  A slice publishes its partial tile to ws[tile][slice] and counts its
// arrival; the slice that arrives last sums the slices in slice order and runs
// the epilogue, then clears the count for the next launch.  No workgroup waits
// for another.  splits <= 1: no tail split.
constexpr int kMaxTailSplits = 8;  // K slices per tail tile
struct TailArgs {
  int n_full = 0;
  int splits = 0;
  int ksplit = 0;
  float* ws = nullptr;
  unsigned* arrivals = nullptr;
};


// Shared epilogue of the tiled kernels: 4 consecutive columns n..n+3 of row m.
template <int EPI>
__device__ __forceinline__ void epilogue4(float* Y, int ldy, int m, int n, int N,
                                          const float* __restrict__ bias, float4 v,
                                          const EpiArgs& ep) {
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
    return;
  }
  if (EPI == LX_EPI_GELU_TANH) {
#pragma unroll
    for (int e = 0; e < 4; ++e) vv[e] = gelu_tanh(vv[e]);
  }
  if (EPI == LX_EPI_ROPE_PARTIAL) {
    const int cs = n % ep.section;
    if (n < ep.sections * ep.section && cs < ep.rot_dim) {
      const float p = (float)ep.pos[m % ep.rows_per_batch];
      const int i0 = cs >> 1;
      rotate_pair(vv[0], vv[1], p * ep.inv_freq[i0]);
      rotate_pair(vv[2], vv[3], p * ep.inv_freq[i0 + 1]);
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


// Pipelined NT GEMM for 64 x 64 output tiles, 4 waves (2 x 2) per k-group
// (KS k-groups split the K slabs of one tile between them and are reduced
// through LDS in a fixed order, so results are deterministic).  Global loads
// run two 32-wide slabs ahead of the MFMAs in two register stages, statically
// indexed by unrolling the slab loop by 2; LDS is double buffered.
// Cross-barrier slabs: the barrier sits inside the slab.  The first three
// quarters of a slab's MFMAs run alongside the LDS writes of the next slab and
// the global loads (scheduling-group barriers spread them between the MFMAs),
// then the barrier, then the next slab's fragment reads are issued and the last
// quarter (operands already in registers) covers their latency, so the matrix
// pipe does not drain at every barrier.
// Operand rows past M (or N) read as zeros (buffer loads) or repeat the last
// valid row (64-bit loads); either way they only reach output rows (columns)
// the epilogue never stores.  With KMASK (K not a multiple of BK) the columns
// past K are stored to LDS as zeros.  MF16 selects the wave's 32 x 32 output
// as four independent 16 x 16 accumulator chains on v_mfma_f32_16x16x4f32
// instead of one v_mfma_f32_32x32x2f32 chain.
template <int EPI, int KS, bool KMASK, bool BUF = true, bool MF16 = false>
__global__ __launch_bounds__(256 * KS) void gemm_pipe_kernel(
    const float* X, int ldx, const float* W, int ldw,
    const float* __restrict__ bias, float* Y, int ldy, int M, int N, int K, int ksplit,
    EpiArgs ep, TailArgs ta) {
  constexpr int BM = 64, BN = 64, BK = 32, GT = 256, NT = GT * KS;
  constexpr int LDA = BK + 4;
  constexpr int A4 = BM * BK / 4;          // float4 per operand slab
  constexpr int L = A4 / GT;               // float4 per thread per operand
  static_assert(A4 % GT == 0, "bad slab");
  extern __shared__ __attribute__((aligned(16))) float smem[];

  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int nwg = tiles_m * tiles_n;
  int id = blockIdx.x;
  int slice = blockIdx.y;  // K slice: split-K partial planes, or a tail tile's slice
  int tail = -1;           // tail tile index (split tail), else -1
  if (ta.splits > 1 && id >= ta.n_full) {
    const int j = id - ta.n_full;
    tail = j / ta.splits;
    slice = j - tail * ta.splits;
    id = ta.n_full + tail;
  } else {
    const int nperm = ta.splits > 1 ? ta.n_full : nwg;
    const int full = (nperm / 8) * 8;
    if (id < full) id = (id % 8) * (full / 8) + id / 8;
  }
  // Runs of 8 M-tiles with N fastest across a run: the contiguous id range of
  // one XCD covers a compact block of A rows and W rows (fewer L2 refills).
  int mt, nt;
  {
    const int grp = id / (8 * tiles_n);
    const int gs = min(8, tiles_m - grp * 8);
    const int in = id - grp * 8 * tiles_n;
    mt = grp * 8 + in % gs;
    nt = in / gs;
  }
  const int m0 = mt * BM, n0 = nt * BN;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int kg = wave >> 2;
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;
  const int gtid = tid & (GT - 1);
  // LDS slab layout.  32x32x2 chains: row-major rows of LDA floats.  16x16x4
  // chains (MF16): lanes l and l + 16 of a fragment read share a row and sit
  // 8 floats apart, which two-way conflicts in the row-major layout (the
  // 128-bit reads serve 32 lanes per pass, one 16-byte slot each over 512
  // bytes).  So each row is split in halves: k groups 0 and 2 (columns 0-7,
  // 16-23) in rows of 20 floats, k groups 1 and 3 in a second block kH1
  // floats on, kH1 = 64 mod 128, which puts the two lane halves on disjoint
  // slots (conflict-free reads); the staging stores, eight lanes per pass over
  // 128 bytes, write the same row's k groups 0 and 1 in different passes.
  constexpr int kRow16 = 20, kH1 = 1344;
  constexpr int SLAB = MF16 ? kH1 + BM * kRow16 : BM * LDA;  // floats per operand buffer
  static_assert(!MF16 || (kH1 % 128 == 64 && kH1 >= BM * kRow16), "MF16 slab layout");
  float* As = smem + kg * 2 * 2 * SLAB;
  float* Ws = As + 2 * SLAB;
  // K slice of this workgroup (one slice unless split-K partials or a tail
  // tile's slice)
  {
    const int kl = tail >= 0 ? ta.ksplit : ksplit;
    X += (long)slice * kl;
    W += (long)slice * kl;
    if (tail < 0) Y += (long)slice * M * ldy;
    K = min(kl, K - slice * kl);
  }

  // Operand loads.  BUF: through buffer descriptors over the K slice, each
  // lane's byte offset fixed for the whole loop and the slab advancing through
  // the scalar offset, so the loop carries no address arithmetic; rows past M
  // (N) lie beyond the descriptor's range and read as zeros (the host keeps
  // every offset below 2^31).  Otherwise: 64-bit addresses with rows clamped
  // into range.  Columns past K (KMASK) are zeroed when stored to LDS.
  const float* pa[L];
  const float* pw[L];
  int oa[L], ow[L];
  int cc[L], rr[L];
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)X, (short)0, BUF ? (int)(((long)(M - 1) * ldx + K) * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)W, (short)0, BUF ? (int)(((long)(N - 1) * ldw + K) * 4) : 0, 0x00020000);
  int so[L];  // LDS offset of the thread's float4 within a slab
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int idx = gtid + i * GT;
    if (MF16) {
      // wave w, stage i covers rows 8 w + 32 i .. +7; pass p of eight lanes
      // writes rows (p / 2, p / 2 + 4) at the four chunks of k-group parity
      // p & 1, so its eight 16-byte stores land on distinct slots
      const int w = gtid >> 6, ln = gtid & 63, p = ln >> 3, j = ln & 7;
      rr[i] = 8 * w + 32 * i + (p >> 1) + 4 * (j >> 2);
      const int c = (j & 1) + ((j >> 1) & 1) * 4 + (p & 1) * 2;  // float4 chunk 0..7
      cc[i] = 4 * c;
      so[i] = ((c >> 1) & 1) * kH1 + rr[i] * kRow16 + (c >> 2) * 8 + (c & 1) * 4;
    } else {
      rr[i] = idx / (BK / 4);
      cc[i] = (idx % (BK / 4)) * 4;
      so[i] = rr[i] * LDA + cc[i];
    }
    oa[i] = ((m0 + rr[i]) * ldx + cc[i]) * 4;
    ow[i] = ((n0 + rr[i]) * ldw + cc[i]) * 4;
    pa[i] = X + (long)min(m0 + rr[i], M - 1) * ldx;
    pw[i] = W + (long)min(n0 + rr[i], N - 1) * ldw;
  }
  floatx4 sa0[L], sw0[L], sa1[L], sw1[L];  // two register stages
#define LX_GLOAD(SA, SW, KT)                                                            \
  do {                                                                                  \
    _Pragma("unroll") for (int i = 0; i < L; ++i) {                                      \
      if (BUF) {                                                                        \
        SA[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, oa[i], (KT) * (BK * 4), 0);  \
        SW[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ow[i], (KT) * (BK * 4), 0);  \
      } else {                                                                          \
        SA[i] = *reinterpret_cast<const floatx4*>(pa[i] + min((KT) * BK + cc[i], K - 4)); \
        SW[i] = *reinterpret_cast<const floatx4*>(pw[i] + min((KT) * BK + cc[i], K - 4)); \
      }                                                                                 \
    }                                                                                   \
  } while (0)
#define LX_SSTORE(SA, SW, BUF, KT)                                                   \
  do {                                                                               \
    _Pragma("unroll") for (int i = 0; i < L; ++i) {                                   \
      floatx4 va = SA[i], vw = SW[i];                                                \
      if (KMASK) {                                                                   \
        const bool kin = (KT) * BK + cc[i] < K;                                      \
        _Pragma("unroll") for (int e = 0; e < 4; ++e) {                               \
          va[e] = kin ? va[e] : 0.0f;                                                \
          vw[e] = kin ? vw[e] : 0.0f;                                                \
        }                                                                            \
      }                                                                              \
      *reinterpret_cast<floatx4*>(As + (BUF) * SLAB + so[i]) = va;                  \
      *reinterpret_cast<floatx4*>(Ws + (BUF) * SLAB + so[i]) = vw;                  \
    }                                                                                \
  } while (0)

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  const int iters = (nk + KS - 1) / KS;
  // slab of iteration it for this k-group
#define LX_KT(IT) ((IT) * KS + kg)
  // Loads and stores are unconditional (slab index clamped into range; the
  // stored values are zero-masked by k), so the loop body is straight-line and
  // the compiler's vmcnt waits count exactly the two stages in flight.
#define LX_KC(IT) min(LX_KT(IT), nk - 1)
  // The empty asm statements keep the two stages' loads in order, so the
  // outstanding-load order at the loop entry matches the one at the back edge
  // and the loop's vmcnt waits count exactly one stage.
  // slab 1 is requested before slab 0 is waited for, so the first two
  // slabs' latencies overlap
  LX_GLOAD(sa0, sw0, LX_KC(0));
  asm volatile("" ::: "memory");
  LX_GLOAD(sa1, sw1, LX_KC(1));
  asm volatile("" ::: "memory");
  LX_SSTORE(sa0, sw0, 0, LX_KT(0));
  asm volatile("" ::: "memory");
  LX_GLOAD(sa0, sw0, LX_KC(2));
  asm volatile("" ::: "memory");
  __syncthreads();

  // Cross-barrier slab (XB): fragments FA/FB of this slab are in registers on
  // entry; the next slab's go to NA/NB after the barrier.
#define LX_SLAB_XB(IT, BUF, SNA, SNW, FA, FB, NA, NB)                                  \
  do {                                                                                 \
    _Pragma("unroll") for (int j = 0; j < 3; ++j)                                       \
      _Pragma("unroll") for (int e = 0; e < 4; ++e)                                     \
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(FA[j][e], FB[j][e], acc, 0, 0, 0);   \
    LX_SSTORE(SNA, SNW, (BUF) ^ 1, LX_KT((IT) + 1));                                   \
    LX_GLOAD(SNA, SNW, LX_KC((IT) + 3));                                               \
    /* 12 MFMAs with the 2L DS writes and 2L global loads between them */           \
    _Pragma("unroll") for (int q = 0; q < 2 * L; ++q) {                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                               \
    }                                                                                  \
    _Pragma("unroll") for (int q = 0; q < 2 * L; ++q) {                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                               \
    }                                                                                  \
    __builtin_amdgcn_sched_group_barrier(0x008, 12 - 4 * L, 0);                        \
    __syncthreads();                                                                   \
    {                                                                                  \
      const float* nab = As + ((BUF) ^ 1) * SLAB + (wm * 32 + r) * LDA + h * 16;        \
      const float* nwb = Ws + ((BUF) ^ 1) * SLAB + (wn * 32 + r) * LDA + h * 16;        \
      _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                   \
        NA[j] = *reinterpret_cast<const floatx4*>(nab + 4 * j);                        \
        NB[j] = *reinterpret_cast<const floatx4*>(nwb + 4 * j);                        \
      }                                                                                \
    }                                                                                  \
    _Pragma("unroll") for (int e = 0; e < 4; ++e)                                       \
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(FA[3][e], FB[3][e], acc, 0, 0, 0);     \
    /* the 8 fragment reads first, then the 4 MFMAs that cover them */              \
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);                                 \
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                 \
  } while (0)

  // Cross-barrier slab (XB) on 16x16x4 MFMAs: the wave's 32 x 32 output is
  // 2 x 2 independent 16 x 16 blocks (four accumulator chains).  Lane l feeds
  // row/column l % 16 of a block and k group g = l / 16, which owns k = g*8 .. g*8+7
  // of the slab: MFMA step s (0..7) sums k = {0, 8, 16, 24} + s, so each lane's
  // operands for a slab are 8 contiguous floats (two ds_read_b128) per block row.
  // Steps 0-5 (24 MFMAs) run before the barrier with the DS writes and global
  // loads between them; steps 6-7 (8 MFMAs) run after it and cover the next
  // slab's fragment reads.
#define LX_MF16(FA, FB, S)                                                             \
  _Pragma("unroll") for (int bi = 0; bi < 2; ++bi)                                      \
    _Pragma("unroll") for (int bj = 0; bj < 2; ++bj)                                    \
      acc4[bi][bj] = __builtin_amdgcn_mfma_f32_16x16x4f32(FA[bi][(S) >> 2][(S) & 3],     \
                                                          FB[bj][(S) >> 2][(S) & 3],     \
                                                          acc4[bi][bj], 0, 0, 0)
#define LX_SLAB_XB16(IT, BUF, SNA, SNW, FA, FB, NA, NB)                                  \
  do {                                                                                 \
    _Pragma("unroll") for (int s_ = 0; s_ < 6; ++s_) { LX_MF16(FA, FB, s_); }             \
    LX_SSTORE(SNA, SNW, (BUF) ^ 1, LX_KT((IT) + 1));                                   \
    LX_GLOAD(SNA, SNW, LX_KC((IT) + 3));                                               \
    _Pragma("unroll") for (int q = 0; q < 2 * L; ++q) {                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                               \
    }                                                                                  \
    _Pragma("unroll") for (int q = 0; q < 2 * L; ++q) {                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                               \
    }                                                                                  \
    __builtin_amdgcn_sched_group_barrier(0x008, 24 - 8 * L, 0);                        \
    __syncthreads();                                                                   \
    LX_FRAG16(NA, NB, (BUF) ^ 1);                                                      \
    LX_MF16(FA, FB, 6);                                                                \
    LX_MF16(FA, FB, 7);                                                                \
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);                                 \
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                                 \
  } while (0)
#define LX_FRAG16(NA, NB, BUF)                                                         \
  do {                                                                                 \
    const int f16 = ((lane >> 4) & 1) * kH1 + (lane & 15) * kRow16 + (lane >> 5) * 8;    \
    const float* nab = As + (BUF) * SLAB + wm * 32 * kRow16 + f16;                      \
    const float* nwb = Ws + (BUF) * SLAB + wn * 32 * kRow16 + f16;                      \
    _Pragma("unroll") for (int b_ = 0; b_ < 2; ++b_)                                    \
      _Pragma("unroll") for (int q_ = 0; q_ < 2; ++q_) {                                \
        NA[b_][q_] = *reinterpret_cast<const floatx4*>(nab + b_ * 16 * kRow16 + 4 * q_); \
        NB[b_][q_] = *reinterpret_cast<const floatx4*>(nwb + b_ * 16 * kRow16 + 4 * q_); \
      }                                                                                \
  } while (0)

  floatx4 acc4[2][2];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc4[bi][bj][i] = 0.0f;

  // Both slabs of an iteration run unconditionally (a surplus slab multiplies
  // the zeros it holds; the launcher sets KMASK whenever the slab count is not
  // a multiple of 2 KS), so the loop has a single back-edge state for the waits.
  if (MF16) {
    floatx4 fa0[2][2], fb0[2][2], fa1[2][2], fb1[2][2];
    LX_FRAG16(fa0, fb0, 0);
    for (int it = 0; it < iters; it += 2) {
      LX_SLAB_XB16(it, 0, sa1, sw1, fa0, fb0, fa1, fb1);
      LX_SLAB_XB16(it + 1, 1, sa0, sw0, fa1, fb1, fa0, fb0);
    }
  } else {
    floatx4 fa0[4], fb0[4], fa1[4], fb1[4];
    {
      const float* ab = As + (wm * 32 + r) * LDA + h * 16;
      const float* wb = Ws + (wn * 32 + r) * LDA + h * 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        fa0[j] = *reinterpret_cast<const floatx4*>(ab + 4 * j);
        fb0[j] = *reinterpret_cast<const floatx4*>(wb + 4 * j);
      }
    }
    for (int it = 0; it < iters; it += 2) {
      LX_SLAB_XB(it, 0, sa1, sw1, fa0, fb0, fa1, fb1);
      LX_SLAB_XB(it + 1, 1, sa0, sw0, fa1, fb1, fa0, fb0);
    }
  }
#undef LX_SLAB_XB
#undef LX_SLAB_XB16
#undef LX_FRAG16
#undef LX_MF16
#undef LX_KC
#undef LX_KT
#undef LX_GLOAD
#undef LX_SSTORE

  // Epilogue operands of this thread's output float4s (bias, gate, residual,
  // rotary position) are loaded before the k-group reduction, so their
  // latency overlaps it.
  constexpr int SLOTS = BM * BN / 4 / NT;
  float4 eb[SLOTS], eg[SLOTS], ey[SLOTS];
  int epos[SLOTS];
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  // Loads read an in-range address unconditionally and the value is selected
  // afterwards (a selected address would fall back to flat loads with a stack
  // copy of the zero vector); with ep.vec every pointer involved is 16-byte
  // aligned.
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    eb[j] = z4;
    eg[j] = z4;
    ey[j] = z4;
    epos[j] = 0;
  }
  if (ep.vec) {
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int idx = tid + j * NT;
      const int m = m0 + idx / (BN / 4), n = n0 + (idx % (BN / 4)) * 4;
      const bool ok = m < M && n + 4 <= N;
      const int mc = ok ? m : 0, nc = ok ? n : 0;
      if (bias) {
        const float4 t = *reinterpret_cast<const float4*>(bias + nc);
        eb[j] = ok ? t : z4;
      }
      if (EPI == LX_EPI_GATED_RESID) {
        const float4 t = *reinterpret_cast<const float4*>(
            ep.gate + (long)(mc / ep.rows_per_batch) * ep.gate_stride + nc);
        eg[j] = ok ? t : z4;
      }
      if (EPI == LX_EPI_GATED_RESID || EPI == LX_EPI_RESID) {
        const float4 t = *reinterpret_cast<const float4*>(Y + (long)mc * ldy + nc);
        ey[j] = ok ? t : z4;
      }
      if (EPI == LX_EPI_ROPE_PARTIAL) epos[j] = ep.pos[mc % ep.rows_per_batch];
    }
  }

  constexpr int LDC = BN + 4;
  float* Cs = smem;
#pragma unroll
  for (int g = KS - 1; g >= 0; --g) {
    if (kg == g) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // 32x32x2: register i of lane (r, h) is row (i/4)*8 + h*4 + i%4, col r;
        // 16x16x4 blocks: register v of block (bi, bj), lane l is row
        // bi*16 + 4*(l/16) + v, col bj*16 + l%16
        constexpr bool B16 = MF16;
        const int bi = i >> 3, bj = (i >> 2) & 1, v4 = i & 3;
        const int row = B16 ? wm * 32 + bi * 16 + 4 * (lane >> 4) + v4
                            : wm * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        const int col = B16 ? wn * 32 + bj * 16 + (lane & 15) : wn * 32 + r;
        float v = B16 ? acc4[bi][bj][v4] : acc[i];
        if (g < KS - 1) v += Cs[row * LDC + col];
        Cs[row * LDC + col] = v;
      }
    }
    __syncthreads();
  }
  if (tail >= 0) {
    // Publish this slice's partial tile, count the arrival, and let the last
    // slice sum all of them in slice order.  The slices of a tile run on
    // different XCDs, so the partials are written and read with device-scope
    // (sc1) 16-byte buffer accesses.  Each thread only touches its own float4
    // slots of Cs, the ones its epilogue stores below.
    constexpr int kSc1 = 16;  // cache-policy bits: sc1 = device scope
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        ta.ws + (long)tail * ta.splits * (BM * BN), (short)0, ta.splits * (BM * BN) * 4,
        0x00020000);
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int idx = tid + j * NT;
      const int row = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const floatx4*>(Cs + row * LDC + c),
                                             prs, (slice * (BM * BN) + row * BN + c) * 4, 0, kSc1);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stores are performed before the count
    __shared__ int last;
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(ta.arrivals + tail, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ta.splits - 1);
    __syncthreads();
    if (!last) return;
    // every slice's float4 of a slot is loaded before the first add (slices
    // past `splits` re-read slice 0 and are not added)
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int idx = tid + j * NT;
      const int row = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
      floatx4 pv[kMaxTailSplits];
#pragma unroll
      for (int sl = 0; sl < kMaxTailSplits; ++sl)
        pv[sl] = __builtin_amdgcn_raw_buffer_load_b128(
            prs, ((sl < ta.splits ? sl : 0) * (BM * BN) + row * BN + c) * 4, 0, kSc1);
      floatx4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
      const floatx4 own = *reinterpret_cast<const floatx4*>(Cs + row * LDC + c);
#pragma unroll
      for (int sl = 0; sl < kMaxTailSplits; ++sl)
        if (sl < ta.splits) sum += sl == slice ? own : pv[sl];
      *reinterpret_cast<floatx4*>(Cs + row * LDC + c) = sum;
    }
    if (tid == 0)
      __hip_atomic_store(ta.arrivals + tail, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    const int idx = tid + j * NT;
    const int row = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
    const int m = m0 + row, n = n0 + c;
    if (m < M && n < N) {
      const float4 v = *reinterpret_cast<const float4*>(Cs + row * LDC + c);
      if (ep.vec && n + 4 <= N)
        epilogue4v<EPI>(Y, ldy, m, n, v, eb[j], eg[j], ey[j], epos[j], ep);
      else
        epilogue4<EPI>(Y, ldy, m, n, N, bias, v, ep);
    }
  }
}

template <int KS>
struct PipeCfg {
  static constexpr int BK = 32;
  static constexpr int threads = 256 * KS;
  // KS k-groups x 2 operands x 2 buffers of one slab (the split-half MF16
  // layout: 1344 + 64 x 20 floats; otherwise 64 rows of BK + 4), or the
  // epilogue's 64 x 68 tile if larger
  static size_t lds(bool mf16) {
    const size_t slab = mf16 ? 1344 + 64 * 20 : 64 * (BK + 4);
    size_t a = (size_t)KS * 2 * 2 * slab * sizeof(float);
    size_t c = (size_t)64 * (64 + 4) * sizeof(float);
    return a > c ? a : c;
  }
};

// Launch geometry shared by the launchers: `splits` K slices of `ksplit`
// columns each (blockIdx.y); a single slice covers all of K.
struct Split {
  int splits = 1;
  int ksplit = 0;
  int ldw = 0;
  TailArgs tail;  // split tail (tail.splits > 1), with splits == 1
};

template <int EPI, int KS, bool KMASK, bool BUF, bool MF16>
int launch_pipe_k(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
                  int M, int N, int K, const EpiArgs& ep, hipStream_t stream,
                  const Split& sp) {
  auto kern = gemm_pipe_kernel<EPI, KS, KMASK, BUF, MF16>;
  const size_t lds = PipeCfg<KS>::lds(MF16);
  if (lds > 64 * 1024) {
    static LdsLimit once;  // per instantiation
    const int rc = raise_lds_limit((const void*)kern, lds, once, "linear");
    if (rc) return rc;
  }
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  const long wgs =
      sp.tail.splits > 1 ? sp.tail.n_full + (tiles - sp.tail.n_full) * sp.tail.splits : tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)wgs, sp.splits), dim3(PipeCfg<KS>::threads), lds,
                     stream, x, ldx, W, sp.ldw, bias, y, ldy, M, N, K, sp.ksplit, ep, sp.tail);
  return check_launch("gemm_pipe_kernel");
}

// Buffer-descriptor loads need every operand byte offset, including the rows
// of the last tile past M (N), below 2^31.
inline bool buffer_loads_fit(int M, int ldx, int N, int ldw) {
  const long lim = 1L << 31;
  return ((long)(M + 64) * ldx + 64) * 4 < lim && ((long)(N + 64) * ldw + 64) * 4 < lim;
}

// The unmasked kernel needs every K slice to be whole slabs and its slab
// count a multiple of 2 KS (the loop runs two slabs per k-group per iteration).
template <int EPI, int KS, bool MF16 = false>
int launch_pipe(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
                int M, int N, int K, const EpiArgs& ep, hipStream_t stream, Split sp = Split()) {
  if (sp.ksplit <= 0) sp.ksplit = K;
  if (sp.ldw <= 0) sp.ldw = K;
  const int step = 2 * KS * PipeCfg<KS>::BK;
  bool exact = sp.ksplit % step == 0 && (K % sp.ksplit) % step == 0;
  if (sp.tail.splits > 1)
    exact = exact && sp.tail.ksplit % step == 0 && (K % sp.tail.ksplit) % step == 0;
  if (!buffer_loads_fit(M, ldx, N, sp.ldw))  // operands past 2 GiB: 64-bit addressing
    return launch_pipe_k<EPI, KS, true, false, MF16>(x, ldx, W, bias, y, ldy, M, N, K, ep,
                                                     stream, sp);
  return exact ? launch_pipe_k<EPI, KS, false, true, MF16>(x, ldx, W, bias, y, ldy, M, N, K, ep,
                                                           stream, sp)
               : launch_pipe_k<EPI, KS, true, true, MF16>(x, ldx, W, bias, y, ldy, M, N, K, ep,
                                                          stream, sp);
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

}  // namespace

// float4 epilogue: output rows, bias and gate rows 16-byte aligned (the
// paired SwiGLU output stores float2: 8-byte alignment suffices for it, and
// 16 bytes is asked anyway).
bool epi_vec_ok(const EpiArgs& ep, const float* y, int ldy, const float* bias) {
  const bool swi = ep.kind == LX_EPI_SWIGLU_PAIRED;
  bool ok = ((uintptr_t)y % 16 == 0) && (swi ? ldy % 2 == 0 : ldy % 4 == 0) &&
            ((uintptr_t)bias % 16 == 0);
  if (ep.kind == LX_EPI_GATED_RESID)
    ok = ok && (uintptr_t)ep.gate % 16 == 0 && ep.gate_stride % 4 == 0;
  return ok;
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

namespace {


// ---- fp32 GEMM on the bf16 matrix cores (split operands), for large M ----
//
// y = epi(x @ W^T + bias) with every product formed from three-part bf16
// splits: x = x0 + x1 + x2 (x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 -
// x1), exact for normal values), the six products a_i b_j with i + j <= 2 on
// v_mfma_f32_32x32x16_bf16, fp32 accumulation.  W arrives pre-split (three
// planes of (N, K) bf16, made once by split_planes); x is split as it is
// staged into LDS.  128 x 128 workgroup tiles of 8 waves (2 x 4, each 64 x 32:
// two 32 x 32 accumulators), K in 32-wide slabs, LDS double buffered (three
// planes per operand, 64-byte rows with an XOR chunk swizzle: conflict-free
// staging stores and 16-byte fragment reads), the next two slabs' global loads
// in flight.  The epilogue stages the tile in LDS
// and runs the fp32 kernel's float4 epilogue.  N must be a multiple of 128, K
// of 32, all epilogue pointers 16-byte aligned.

// WM x WN waves, each (32 BI) x 32 outputs: workgroup tile (32 BI WM) x (32 WN).
template <int WM, int WN, int BI>
struct SplitCfg {
  static constexpr int NT = 64 * WM * WN, BM = 32 * BI * WM, BN = 32 * WN;
  static constexpr size_t lds = (size_t)2 * 3 * (BM + BN) * kSplitRS * 2;
};

template <int EPI, int WM, int WN, int BI>
__global__ __launch_bounds__(64 * WM * WN) void gemm_split_kernel(
    const float* __restrict__ X, int ldx, const __bf16* __restrict__ Wp, long wplane,
    const float* __restrict__ bias, float* Y, int ldy, int M, int N, int K, EpiArgs ep) {
  using Cfg = SplitCfg<WM, WN, BI>;
  constexpr int NT = Cfg::NT, BM = Cfg::BM, BN = Cfg::BN, BK = kSplitBK;
  constexpr int RS = kSplitRS;
  constexpr int APL = BM * RS, WPL = BN * RS;  // bf16 per plane
  constexpr int BUFSZ = 3 * APL + 3 * WPL;     // bf16 per buffer
  constexpr int LAT = BM * BK / 4, LWT = 3 * BN * BK / 8;  // x float4, W chunks per slab
  constexpr int LA = (LAT + NT - 1) / NT;      // per thread (a surplus step repeats the
  constexpr int LW = (LWT + NT - 1) / NT;      // last one: same value to the same place)
  static_assert((size_t)BM * (BN + 4) * 4 <= Cfg::lds, "epilogue tile");
  static_assert(BM * BN / 4 % NT == 0, "epilogue slots");
  extern __shared__ __attribute__((aligned(16))) __bf16 sm[];
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  const int nwg = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int full = (nwg / 8) * 8;
    if (id < full) id = (id % 8) * (full / 8) + id / 8;
  }
  // runs of 8 M-tiles with N fastest across a run (as gemm_pipe_kernel)
  int mt, nt;
  {
    const int grp = id / (8 * tiles_n);
    const int gs = min(8, tiles_m - grp * 8);
    const int in = id - grp * 8 * tiles_n;
    mt = grp * 8 + in % gs;
    nt = in / gs;
  }
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int nk = K / BK;
  // x: float4 (row, c); rows past M repeat the last row (never stored)
  const float* pa[LA];
  int sa[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int idx = min(tid + NT * i, LAT - 1);
    const int row = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
    pa[i] = X + (long)min(m0 + row, M - 1) * ldx + c;
    sa[i] = row * RS + split_col(row, c);
  }
  // W: 16-byte chunk (plane, row, c)
  const __bf16* pw[LW];
  int sw[LW];
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    const int idx = min(tid + NT * i, LWT - 1);
    const int p = idx / (BN * BK / 8), rem = idx % (BN * BK / 8);
    const int row = rem / (BK / 8), c = (rem % (BK / 8)) * 8;
    pw[i] = Wp + p * wplane + (long)(n0 + row) * K + c;
    sw[i] = 3 * APL + p * WPL + row * RS + split_col(row, c);
  }
  floatx4 ga0[LA], gw0[LW], ga1[LA], gw1[LW];
#define LX_SGL(GA, GW, KT)                                                                    \
  {                                                                                           \
    const int kk = min(KT, nk - 1) * BK;                                                      \
    _Pragma("unroll") for (int i = 0; i < LA; ++i)                                            \
      GA[i] = *reinterpret_cast<const floatx4*>(pa[i] + kk);                                  \
    _Pragma("unroll") for (int i = 0; i < LW; ++i)                                            \
      GW[i] = *reinterpret_cast<const floatx4*>(pw[i] + kk);                                  \
  }
#define LX_SST(GA, GW, B)                                                                     \
  {                                                                                           \
    __bf16* base = sm + (B) * BUFSZ;                                                          \
    _Pragma("unroll") for (int i = 0; i < LA; ++i) {                                          \
      const bf16x4_t x0 = __builtin_convertvector(GA[i], bf16x4_t);                           \
      const floatx4 r = GA[i] - bf16x4_back(x0);                                              \
      const bf16x4_t x1 = __builtin_convertvector(r, bf16x4_t);                               \
      const bf16x4_t x2 = __builtin_convertvector(r - bf16x4_back(x1), bf16x4_t);             \
      *reinterpret_cast<bf16x4_t*>(base + sa[i]) = x0;                                        \
      *reinterpret_cast<bf16x4_t*>(base + APL + sa[i]) = x1;                                  \
      *reinterpret_cast<bf16x4_t*>(base + 2 * APL + sa[i]) = x2;                              \
    }                                                                                         \
    _Pragma("unroll") for (int i = 0; i < LW; ++i)                                            \
      *reinterpret_cast<floatx4*>(base + sw[i]) = GW[i];                                      \
  }
  floatx16 acc[BI];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
  const int fr = lane & 31, fh = lane >> 5;
  // fragment rows are wm * 32 BI + i * 32 + fr (A) and wn * 32 + fr (W): their
  // chunk swizzle is (fr / 8) % 4, the same for every block
  const int aoff = (wm * 32 * BI + fr) * RS;
  const int woff = 3 * APL + (wn * 32 + fr) * RS;
  const int fc[2] = {split_col(fr, fh * 8), split_col(fr, 16 + fh * 8)};
  // The six products of mfma_split6x as (A part, W part), in its order.
  constexpr int kPa[6] = {2, 1, 0, 1, 0, 0}, kPw[6] = {0, 1, 2, 0, 1, 0};
#define LX_SRD(FA, FB, B, ST)                                                                 \
  {                                                                                           \
    const __bf16* base = sm + (B) * BUFSZ;                                                    \
    _Pragma("unroll") for (int i = 0; i < BI; ++i)                                            \
      _Pragma("unroll") for (int p = 0; p < 3; ++p)                                           \
        FA[i][p] = *reinterpret_cast<const sbf16x8*>(base + aoff + p * APL + i * 32 * RS +    \
                                                     fc[ST]);                                 \
    _Pragma("unroll") for (int p = 0; p < 3; ++p)                                             \
      FB[p] = *reinterpret_cast<const sbf16x8*>(base + woff + p * WPL + fc[ST]);              \
  }
#define LX_SMUL(FA, FB, P0, P1)                                                               \
  _Pragma("unroll") for (int q = P0; q < P1; ++q)                                             \
    _Pragma("unroll") for (int i = 0; i < BI; ++i)                                            \
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FA[i][kPa[q]], FB[kPw[q]], acc[i], 0, 0, 0);
  // Each slab is two 16-wide k steps, fragment sets F0 and F1.  Two
  // accumulators per wave (BI = 2) pipeline across the barrier: F1's reads
  // issue under F0's MFMAs, the next slab's staging and global loads under F0's
  // and the first four of F1's six products, and after the barrier the next
  // slab's F0 reads issue under F1's last two products, so the matrix pipe
  // does not drain at each barrier (QKV at 6000 rows 255 -> 242 us).  With one
  // accumulator (BI = 1) the two live fragment sets would take the kernel past
  // 128 VGPRs and one of its two workgroups per CU (out / FF2 at 6000 rows
  // 127 -> 136 us), so it multiplies each slab between the barriers.
#define LX_HALF(B, GA, GW, KT)                                                                \
  {                                                                                           \
    LX_SRD(fa1, fb1, B, 1);                                                                   \
    LX_SMUL(fa0, fb0, 0, 6);                                                                  \
    LX_SST(GA, GW, 1 - (B));                                                                  \
    LX_SGL(GA, GW, (KT) + 3);                                                                 \
    LX_SMUL(fa1, fb1, 0, 4);                                                                  \
    __syncthreads();                                                                          \
    if ((KT) + 1 < nk) LX_SRD(fa0, fb0, 1 - (B), 0);                                          \
    LX_SMUL(fa1, fb1, 4, 6);                                                                  \
  }
#define LX_SMM(B)                                                                             \
  _Pragma("unroll") for (int st = 0; st < 2; ++st) {                                          \
    sbf16x8 fa[BI][3], fb[3];                                                                 \
    LX_SRD(fa, fb, B, st);                                                                    \
    LX_SMUL(fa, fb, 0, 6);                                                                    \
  }
  LX_SGL(ga0, gw0, 0);
  LX_SGL(ga1, gw1, 1);
  LX_SST(ga0, gw0, 0);
  LX_SGL(ga0, gw0, 2);
  __syncthreads();
  if constexpr (BI >= 2) {
    sbf16x8 fa0[BI][3], fb0[3], fa1[BI][3], fb1[3];
    LX_SRD(fa0, fb0, 0, 0);
    // slab kt in buffer 0 (its F0 in registers) and kt + 1 in ga1 on entry;
    // the last slab stages a repeat of itself, never multiplied
    for (int kt = 0; kt < nk; kt += 2) {
      LX_HALF(0, ga1, gw1, kt);
      if (kt + 1 < nk) LX_HALF(1, ga0, gw0, kt + 1);
    }
  } else {
    // slab kt in buffer 0 and kt + 1 in ga1 on entry; an odd slab count runs
    // a surplus slab of the last one's repeat into buffer 1, never multiplied
    for (int kt = 0; kt < nk; kt += 2) {
      LX_SMM(0);
      LX_SST(ga1, gw1, 1);
      LX_SGL(ga1, gw1, kt + 3);
      __syncthreads();
      if (kt + 1 < nk) LX_SMM(1);
      LX_SST(ga0, gw0, 0);
      LX_SGL(ga0, gw0, kt + 4);
      __syncthreads();
    }
  }
#undef LX_SGL
#undef LX_SST
#undef LX_SRD
#undef LX_SMUL
#undef LX_HALF
#undef LX_SMM
  // epilogue: the tile through LDS, then float4 slots with the fp32 kernel's
  // epilogue operations
  constexpr int LDC = BN + 4;
  float* Cs = reinterpret_cast<float*>(sm);
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = wm * 32 * BI + i * 32 + (e >> 2) * 8 + fh * 4 + (e & 3);
      Cs[row * LDC + wn * 32 + fr] = acc[i][e];
    }
  __syncthreads();
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < BM * BN / 4 / NT; ++j) {
    const int idx = tid + j * NT;
    const int row = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
    const int m = m0 + row, n = n0 + c;
    if (m < M) {
      const float4 v = *reinterpret_cast<const float4*>(Cs + row * LDC + c);
      const float4 b = bias ? *reinterpret_cast<const float4*>(bias + n) : z4;
      float4 g = z4, yo = z4;
      int posm = 0;
      if (EPI == LX_EPI_GATED_RESID)
        g = *reinterpret_cast<const float4*>(ep.gate + (long)(m / ep.rows_per_batch) *
                                                           ep.gate_stride + n);
      if (EPI == LX_EPI_GATED_RESID || EPI == LX_EPI_RESID)
        yo = *reinterpret_cast<const float4*>(Y + (long)m * ldy + n);
      if (EPI == LX_EPI_ROPE_PARTIAL) posm = ep.pos[m % ep.rows_per_batch];
      epilogue4v<EPI>(Y, ldy, m, n, v, b, g, yo, posm, ep);
    }
  }
}

__global__ void split_planes_kernel(const float* __restrict__ w, __bf16* __restrict__ out,
                                    long n4) {
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const floatx4 x = reinterpret_cast<const floatx4*>(w)[i];
  const bf16x4_t x0 = __builtin_convertvector(x, bf16x4_t);
  const floatx4 r = x - bf16x4_back(x0);
  const bf16x4_t x1 = __builtin_convertvector(r, bf16x4_t);
  const bf16x4_t x2 = __builtin_convertvector(r - bf16x4_back(x1), bf16x4_t);
  reinterpret_cast<bf16x4_t*>(out)[i] = x0;
  reinterpret_cast<bf16x4_t*>(out + 4 * n4)[i] = x1;
  reinterpret_cast<bf16x4_t*>(out + 8 * n4)[i] = x2;
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

// Configurations: 7 = one k-group (4 waves), 8 = as 7 with intra-workgroup
// split-K 2, 9 = as 7 on four 16x16x4 accumulator chains.
template <int EPI>
int dispatch_cfg(int cfg, const float* x, int ldx, const float* W, const float* bias, float* y,
                 int ldy, int M, int N, int K, const EpiArgs& ep, hipStream_t s,
                 const Split& sp) {
  switch (cfg) {
    case 7: return launch_pipe<EPI, 1>(x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case 8: return launch_pipe<EPI, 2>(x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case 9:
      return launch_pipe<EPI, 1, true>(x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
  }
  set_error("linear: unknown tile configuration %d", cfg);
  return LX_ERR_ARG;
}

int dispatch_gemm(int kind, int cfg, const float* x, int ldx, const float* W, const float* bias,
                  float* y, int ldy, int M, int N, int K, const EpiArgs& ep, hipStream_t s,
                  const Split& sp = Split()) {
  switch (kind) {
    case LX_EPI_NONE:
      return dispatch_cfg<LX_EPI_NONE>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case LX_EPI_GELU_TANH:
      return dispatch_cfg<LX_EPI_GELU_TANH>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case LX_EPI_GATED_RESID:
      return dispatch_cfg<LX_EPI_GATED_RESID>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case LX_EPI_ROPE_PARTIAL:
      return dispatch_cfg<LX_EPI_ROPE_PARTIAL>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case LX_EPI_RESID:
      return dispatch_cfg<LX_EPI_RESID>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
    case LX_EPI_SWIGLU_PAIRED:
      return dispatch_cfg<LX_EPI_SWIGLU_PAIRED>(cfg, x, ldx, W, bias, y, ldy, M, N, K, ep, s, sp);
  }
  set_error("linear: unknown epilogue kind %d", kind);
  return LX_ERR_ARG;
}

// Tile configuration by shape, from an on-device sweep over the estimator's
// projections at B*T = 1000 and 6000 rows (MI355X, graph-replayed launches
// under continuous load, buffer-descriptor loads).  Cross-barrier slabs win
// everywhere.  With one tile per CU (256 tiles: out, FF2 at B*T = 1000)
// intra-workgroup split-K 2 gives each SIMD a second wave (19.2 / 33.8 us).
// From 512 tiles up the unsplit 4-wave kernel wins: several of its workgroups
// fit on a CU at once (37 KB of LDS each), so a 768-tile launch (QKV at
// B*T = 1000: 50.6 us = 124 TFLOP/s) is resident in one round, whereas the
// split-K 2 kernel (74 KB) runs it in two and the paired workgroups of a CU,
// finishing together, can be re-placed two to a CU in the partial second round
// (65 us).  K <= 512 has too few slabs to split.  From 768 tiles (three or
// more workgroups per CU) four 16x16x4 accumulator chains per wave beat one
// 32x32x2 chain (QKV at B*T = 1000: 51.5 vs 52.2 us; the T = 3000 step 4%
// faster); below that the single chain is equal or ahead.
// Split-K partial GEMMs aim for this many workgroups (two per CU).
constexpr long kSplitTargetWgs = 512;

int pick_config(int M, int N, int K) {
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  if (tiles >= 768) return 9;
  return (K <= 512 || tiles >= 512) ? 7 : 8;
}

int gemm_splitk_partials(const float* x, int ldx, const float* W, int ldw, float* ws, int M,
                         int N, int K, int splits, int ksplit, hipStream_t stream) {
  LX_REQUIRE(x && W && ws && M > 0 && N > 0 && K > 0 && splits >= 1 && ksplit > 0 &&
                 ksplit % 4 == 0 && (long)(splits - 1) * ksplit < K && (long)splits * ksplit >= K &&
                 ldx % 4 == 0 && ldw % 4 == 0 && ldx >= K && ldw >= K,
             "gemm_splitk_partials: bad shape M=%d N=%d K=%d splits=%d ksplit=%d", M, N, K,
             splits, ksplit);
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)W) % 16 == 0, "gemm_splitk_partials: misaligned operand");
  EpiArgs ep;
  int rc = make_epi(nullptr, N, &ep);
  if (rc) return rc;
  ep.vec = epi_vec_ok(ep, ws, N, nullptr);
  Split sp;
  sp.splits = splits;
  sp.ksplit = ksplit;
  sp.ldw = ldw;
  return launch_pipe<LX_EPI_NONE, 1>(x, ldx, W, nullptr, ws, N, M, N, K, ep, stream,
                                                     sp);
}

// Split-tail plan for a one-k-group launch whose tiles leave a partial last
// round over the 256 CUs (at most half a round): n_full tiles run whole, the
// rest as `splits` K slices of `ksplit` columns (a multiple of 64, at least
// 128), the slice count chosen so that the slices spread most evenly over the
// CUs.  Qwen2 prefill gate/up at L = 256: 608 tiles = 512 + 96, the 96 as 5
// slices of 192 (480 workgroups: at most 2 slices = 0.4 of a tile more on a
// CU, against a whole third tile on 96 CUs unsplit).
bool split_tail_plan(int M, int N, int K, int* n_full, int* splits, int* ksplit) {
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  if (pick_config(M, N, K) != 7 || tiles <= 256) return false;
  const long nf = tiles / 256 * 256, tail = tiles - nf;
  if (tail == 0 || tail > 128) return false;
  double best = 1.0;  // unsplit: one more whole tile on `tail` CUs
  int bs = 0, bk = 0;
  for (int s = 2; s <= kMaxTailSplits; ++s) {
    int ks = (K + s - 1) / s;
    ks = (ks + 63) / 64 * 64;
    if (ks < 128) continue;
    const int sp = (K + ks - 1) / ks;
    if (sp < 2) continue;
    const double cost = (double)((tail * sp + 255) / 256) / sp;
    if (cost < best - 1e-9) {
      best = cost;
      bs = sp;
      bk = ks;
    }
  }
  if (bs < 2) return false;
  *n_full = (int)nf;
  *splits = bs;
  *ksplit = bk;
  return true;
}

size_t split_tail_ws_floats(int M, int N, int K, int* tail_tiles) {
  int nf = 0, sp = 0, ks = 0;
  *tail_tiles = 0;
  if (!split_tail_plan(M, N, K, &nf, &sp, &ks)) return 0;
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  *tail_tiles = (int)(tiles - nf);
  return (size_t)(tiles - nf) * sp * 64 * 64;
}

int gemm_splitk_plan(int M, int N, int K, int* ksplit) {
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  int s = (int)((kSplitTargetWgs + tiles - 1) / tiles);
  int max_s = K / 128 > 0 ? K / 128 : 1;  // at least four 32-wide slabs per slice
  if (max_s > 9) max_s = 9;                   // the reduce passes sum at most 9 slices
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  int ks = (K + s - 1) / s;
  ks = (ks + 63) / 64 * 64;  // whole slab pairs
  s = (K + ks - 1) / ks;
  *ksplit = ks;
  return s;
}

}  // namespace lx

using namespace lx;

namespace lx {

// lx_linear_f32, optionally with a split tail over caller-owned scratch.
int linear_impl(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
                int M, int N, int K, const lx_epilogue* epi, float* ws, size_t ws_floats,
                unsigned* arrivals, int n_arrivals, hipStream_t stream) {
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
  ep.vec = epi_vec_ok(ep, y, ldy, bias);
  const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  LX_REQUIRE(tiles < (1L << 31), "linear: too many tiles");
  Split sp;
  int nf = 0, tsp = 0, tks = 0;
  if (ws && arrivals && split_tail_plan(M, N, K, &nf, &tsp, &tks) &&
      (size_t)(tiles - nf) * tsp * 64 * 64 <= ws_floats && tiles - nf <= n_arrivals) {
    sp.tail.n_full = nf;
    sp.tail.splits = tsp;
    sp.tail.ksplit = tks;
    sp.tail.ws = ws;
    sp.tail.arrivals = arrivals;
  }
  return dispatch_gemm(kind, pick_config(M, N, K), x, ldx, W, bias, y, ldy, M, N, K, ep, stream,
                       sp);
}

int split_planes(const float* w, void* planes, long n, hipStream_t stream) {
  LX_REQUIRE(w && planes && n > 0 && n % 4 == 0, "split_planes: bad arguments");
  LX_REQUIRE(((uintptr_t)w | (uintptr_t)planes) % 16 == 0, "split_planes: unaligned");
  const long n4 = n / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                     w, static_cast<__bf16*>(planes), n4);
  return check_launch("split_planes_kernel");
}

int linear_split(const float* x, int ldx, const void* Wp, const float* bias, float* y, int ldy,
                 int M, int N, int K, const lx_epilogue* epi, int narrow, hipStream_t stream) {
  const int BN = narrow ? SplitCfg<4, 2, 1>::BN : SplitCfg<2, 4, 2>::BN;
  const int BM = narrow ? SplitCfg<4, 2, 1>::BM : SplitCfg<2, 4, 2>::BM;
  LX_REQUIRE(x && Wp && y, "linear_split: null pointer");
  LX_REQUIRE(M > 0 && N > 0 && N % BN == 0 && K > 0 && K % kSplitBK == 0 && ldx % 4 == 0 &&
                 ldx >= K,
             "linear_split: bad shape M=%d N=%d K=%d", M, N, K);
  const int kind = epi ? epi->kind : LX_EPI_NONE;
  LX_REQUIRE(ldy >= (kind == LX_EPI_SWIGLU_PAIRED ? N / 2 : N), "linear_split: ldy too small");
  LX_REQUIRE(((uintptr_t)x | (uintptr_t)Wp) % 16 == 0, "linear_split: x and W must be aligned");
  EpiArgs ep;
  int rc = make_epi(epi, N, &ep);
  if (rc) return rc;
  ep.vec = epi_vec_ok(ep, y, ldy, bias);
  LX_REQUIRE(ep.vec, "linear_split: y, bias and gate must be 16-byte aligned");
  const long tiles = (long)((M + BM - 1) / BM) * (N / BN);
  LX_REQUIRE(tiles < (1L << 31), "linear_split: too many tiles");
  const long wplane = (long)N * K;
  auto launch = [&](auto kern, size_t lds, int threads, LdsLimit& once) {
    int r = raise_lds_limit((const void*)kern, lds, once, "linear_split");
    if (r) return r;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(threads), lds, stream, x, ldx,
                       static_cast<const __bf16*>(Wp), wplane, bias, y, ldy, M, N, K, ep);
    return check_launch("gemm_split_kernel");
  };
#define LX_SPLIT_CASE(E)                                                                   \
  case E: {                                                                                \
    static LdsLimit once_w, once_n;                                                        \
    if (narrow)                                                                            \
      return launch(gemm_split_kernel<E, 4, 2, 1>, SplitCfg<4, 2, 1>::lds,                 \
                    SplitCfg<4, 2, 1>::NT, once_n);                                        \
    return launch(gemm_split_kernel<E, 2, 4, 2>, SplitCfg<2, 4, 2>::lds,                   \
                  SplitCfg<2, 4, 2>::NT, once_w);                                          \
  }
  switch (kind) {
    LX_SPLIT_CASE(LX_EPI_NONE)
    LX_SPLIT_CASE(LX_EPI_GELU_TANH)
    LX_SPLIT_CASE(LX_EPI_GATED_RESID)
    LX_SPLIT_CASE(LX_EPI_ROPE_PARTIAL)
    LX_SPLIT_CASE(LX_EPI_RESID)
    LX_SPLIT_CASE(LX_EPI_SWIGLU_PAIRED)
    default:
      break;
  }
#undef LX_SPLIT_CASE
  set_error("linear_split: unknown epilogue kind %d", kind);
  return LX_ERR_ARG;
}

int linear_split_tail(const float* x, int ldx, const float* W, const float* bias, float* y,
                      int ldy, int M, int N, int K, const lx_epilogue* epi, float* ws,
                      size_t ws_floats, unsigned* arrivals, int n_arrivals, hipStream_t stream) {
  return linear_impl(x, ldx, W, bias, y, ldy, M, N, K, epi, ws, ws_floats, arrivals, n_arrivals,
                     stream);
}

}  // namespace lx

extern "C" int lx_split_planes_f32(const float* W, void* planes, long n, hipStream_t stream) {
  return split_planes(W, planes, n, stream);
}

extern "C" int lx_linear_split_f32(const float* x, int ldx, const void* planes,
                                   const float* bias, float* y, int ldy, int M, int N, int K,
                                   const lx_epilogue* epi, int tile, hipStream_t stream) {
  LX_REQUIRE(tile == 0 || tile == 1, "linear_split: tile must be 0 or 1, got %d", tile);
  return linear_split(x, ldx, planes, bias, y, ldy, M, N, K, epi, tile, stream);
}

extern "C" int lx_linear_f32(const float* x, int ldx, const float* W, const float* bias,
                             float* y, int ldy, int M, int N, int K, const lx_epilogue* epi,
                             hipStream_t stream) {
  return lx::linear_impl(x, ldx, W, bias, y, ldy, M, N, K, epi, nullptr, 0, nullptr, 0, stream);
}
