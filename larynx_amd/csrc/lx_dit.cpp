// CosyVoice3 Flow DiT estimator and CFM Euler/CFG loop, device resident.
//
// Host-side counterpart of build_dit / dit_block (src/flow/dit.cpp:34-145) and
// of the CFM loop of FlowDecoder::infer (src/flow/flow.cpp:202-274).  Instead
// of a ~8000-node ggml graph the forward is ~10 launches per block:
//
//   adaln(x) -> QKV GEMM (+bias, +partial rotary epilogue) -> flash attention
//   -> out GEMM (+bias, gated-residual epilogue into x) -> adaln(x)
//   -> FF0 GEMM (+bias, tanh-GELU epilogue) -> FF2 GEMM (+bias, gated residual)
//
// and per Euler step the 22 AdaLN modulation linears plus norm_out's are one
// stacked weight-streaming GEMV (t is shared by both CFG rows and all frames).
// Nothing crosses PCIe inside the loop: the timestep is written by a fill
// kernel and the CFG combine + Euler update reads the proj_out rows directly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "lx_common.hpp"
#include "lx_internal.hpp"

using namespace lx;

namespace {

constexpr int kFreqDim = 256;      // SinusPositionEmbedding(256)
constexpr int kConvK = 31;         // CONV_POS_KERNEL (src/flow/internal.h:32)
constexpr int kConvG = 16;         // CONV_POS_GROUPS (src/flow/internal.h:33)
constexpr float kLnEps = 1e-6f;    // LN_EPS (src/flow/internal.h:34)
constexpr float kRopeBase = 10000.0f;  // ROPE_FREQ_BASE (src/flow/internal.h:35)
constexpr int kRotDim = 64;        // ROT_DIM (src/flow/internal.h:25)
constexpr int kProjSplitMax = 9;   // K slices of the proj_out split-K (gemm_splitk_plan's cap)
constexpr int kSolveChunk = 16;    // solve steps whose modulations one GEMV computes
// Up to this many rows (B * T) the out and FF2 projections run as two K slices
// whose sum is folded into the next modulated LayerNorm: at B * T = 1000 their
// 64-row tiles number 128, half the CUs.
constexpr int kPartialRows = 1024;

}  // namespace

struct lx_dit {
  Arena arena;
  int B = 0, max_T = 0;
  int D = 0, depth = 0, heads = 0, hd = 0, F = 0, mel = 0;
  long NA = 0;  // stacked AdaLN rows: depth * 6D + 2D

  // packed weights
  float *tm0_w, *tm0_b, *tm2_w, *tm2_b;
  float *in_w, *in_b;
  // conv_pos weights in MFMA fragment order (conv_frag_pack: 3 * D * 64 * K bf16)
  void *conv1_wf, *conv2_wf;
  float *conv1_b, *conv2_b;
  float *ada_w, *ada_b;                 // (NA, D), (NA)
  // Block projections: with `frag` the weights are kept only in MFMA
  // fragment order (wfrag_pack: three bf16 parts, 3 * N * K bf16) for the
  // split-operand GEMM; otherwise (a width the fragment tiles do not cover)
  // as fp32 for lx_linear_f32.  QKV is fused into one (3D, D) matrix.
  bool frag = false;
  int products = 3;  // split-operand products per element pair (3 or 6)
  std::vector<void*> qkv_wf, out_wf, ff0_wf, ff2_wf;
  std::vector<float*> qkv_w, out_w, ff0_w, ff2_w;
  std::vector<float*> qkv_b, out_b, ff0_b, ff2_b;
  float *proj_w, *proj_b;

  // activations (sized for B x max_T)
  float *temb, *tmlp_work, *emb;
  // A CFM solve's modulations, one row per step for up to kSolveChunk steps
  float *temb_steps, *tmlp_steps, *emb_steps;
  float *A0, *xe, *c1, *h, *xn, *qkv, *att, *ff, *P;
  float* Pws;          // split-K slices of proj_out (kProjSplitMax x rows x mel)
  float* Rws;          // K slices of the out / FF2 projections (2 x kPartialRows x D)
  // The projections' split tail (lx_linear_bx.split_tail): partial tiles of
  // the split workgroups (CUs x 64 x 128 floats) and one arrival count per tile
  // of the widest projection (zeroed here, left zeroed by every launch).
  float* qkv_ws = nullptr;
  size_t qkv_ws_floats = 0;
  unsigned* qkv_cnt = nullptr;
  int qkv_ncnt = 0;
  int proj_splits = 1; // slices of the last forward's proj_out
  long proj_slice = 0; // floats between slices
  int* pos;

  lx_dit_capture cap{};
  hipStream_t create_stream = nullptr;
};

namespace {

int copy_d2d(float* dst, const float* src, size_t n, hipStream_t s) {
  if (!src) {
    set_error("dit_create: missing weight tensor");
    return LX_ERR_ARG;
  }
  if (hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s) != hipSuccess) {
    set_error("dit_create: device copy failed");
    return LX_ERR_LAUNCH;
  }
  return LX_OK;
}

// Everything up to the proj_out rows: their split-K slices in Pws
// (m->proj_splits slices, m->proj_slice floats apart; the bias is added by
// whoever sums them).  x of batch b starts at x + b * x_bstride; with cfg set,
// mu / cond / spks are the conditional row's and the unconditional row gets
// zeros.  t is read from device memory (tdev) or, when tdev is null, from the
// host array thost.
int forward_core(lx_dit* m, const float* x, long x_bstride, const float* mu, const float* cond,
                 const float* spks, int cfg, const float* tdev, const float* thost, int T,
                 hipStream_t s, const float* emb_pre = nullptr, long emb_bstride = 0) {
  const int B = m->B, D = m->D, mel = m->mel;
  const int rows = B * T;
  // The AdaLN modulations of this step: batch row b's at emb + b * NA (NA
  // floats: 22 blocks x 6 chunks, then norm_out's 2).  emb_pre: computed by
  // the caller (a CFM solve computes all its steps' at once; both CFG rows
  // share one, emb_bstride 0); otherwise the time embedding (a6) and every
  // modulation of this step in one GEMV.
  const float* emb = m->emb;
  long NA = m->NA;
  if (emb_pre) {
    emb = emb_pre;
    NA = emb_bstride;
  } else {
    LX_TRY(time_mlp(tdev, thost, B, m->tm0_w, m->tm0_b, m->tm2_w, m->tm2_b, D, m->tmlp_work,
                    m->temb, s));
    LX_TRY(gemv(m->temb, B, D, m->ada_w, m->ada_b, m->emb, m->NA, m->NA, /*silu in*/ 1, 0, s));
    if (m->cap.time_embed)
      (void)hipMemcpyAsync(m->cap.time_embed, m->temb, sizeof(float) * B * D,
                           hipMemcpyDeviceToDevice, s);
  }

  // InputEmbedding: proj(concat[x, cond, mu, spks]) + conv_pos_embed.
  LX_TRY(dit_pack_input(x, x_bstride, cond, mu, spks, cfg, m->A0, B, T, mel, s));
  LX_TRY(lx_linear_f32(m->A0, 4 * mel, m->in_w, m->in_b, m->xe, D, rows, D, 4 * mel, nullptr, s));
  // conv_pos on the split-operand conv with the estimator's product count.
  LX_TRY(conv_pos_mish_bx(m->xe, m->conv1_wf, m->conv1_b, nullptr, m->c1, B, T, D, kConvG, kConvK,
                          m->products, s));
  // h = xe + mish(conv2(c1)); c1 doubles as the conv_pos capture source below.
  LX_TRY(conv_pos_mish_bx(m->c1, m->conv2_wf, m->conv2_b, m->xe, m->h, B, T, D, kConvG, kConvK,
                          m->products, s));
  if (m->cap.input_proj)
    (void)hipMemcpyAsync(m->cap.input_proj, m->xe, sizeof(float) * rows * D,
                         hipMemcpyDeviceToDevice, s);
  if (m->cap.conv_pos) {
    // conv_pos = h - xe is not recomputed; re-run conv2 without the residual.
    LX_TRY(conv_pos_mish_bx(m->c1, m->conv2_wf, m->conv2_b, nullptr, m->xn, B, T, D, kConvG,
                            kConvK, m->products, s));
    (void)hipMemcpyAsync(m->cap.conv_pos, m->xn, sizeof(float) * rows * D,
                         hipMemcpyDeviceToDevice, s);
  }
  if (m->cap.input_embed)
    (void)hipMemcpyAsync(m->cap.input_embed, m->h, sizeof(float) * rows * D,
                         hipMemcpyDeviceToDevice, s);

  // Block projections on the split-operand GEMM with fragment-order weights
  // (64-row tiles, two workgroups per CU).  Up to kPartialRows rows the out
  // and FF2 projections (N = D: 128 tiles at B * T = 1000, half the CUs) run
  // as two K slices of 64-row tiles; their sum, bias and gate go into the
  // residual stream inside the next modulated LayerNorm (lx_adaln_resid_f32),
  // which replaces the gated-residual epilogue.
  struct Pending {
    const float* bias = nullptr;
    const float* gate = nullptr;
  } pend;
  bool pending = false;
  const bool partial = m->frag && rows <= kPartialRows && D % 128 == 0 && m->F % 128 == 0;
  // With three products the block's activations (the modulated LayerNorms'
  // output, attention's output, FF0's GELU output) pass to the projections
  // that read them as two-part packed rows: each producer splits its output
  // once, with the roundings the GEMM would apply (bit-identical results),
  // instead of every column tile of the consumer splitting it again.
  const bool pk = m->frag && m->products == 3;
  auto adaln = [&](const float* shift, const float* scale, float* y, bool packed) -> int {
    if (!pending && !packed)
      return lx_adaln_modulate_f32(m->h, shift, scale, NA, y, B, T, D, kLnEps, s);
    const int S = pending ? 2 : 0;
    pending = false;
    return adaln_resid(m->h, S ? m->Rws : nullptr, S, (long)rows * D, S ? pend.bias : nullptr,
                       S ? pend.gate : nullptr, NA, shift, scale, NA, y, B, T, D, kLnEps,
                       packed ? 1 : 0, s);
  };
  // K and V leave the QKV projection packed too where attention runs on the
  // three-product split kernel (it then stages them without splitting; q
  // stays fp32: attention scales it before its own split).
  const bool pk_kv = pk && attention_takes_packed_kv(B, T, m->heads, 3);
  // Every projection on the fragment-order GEMM asks for the split tail: it
  // applies where the launch's tiles number between one and two per CU (T = 500:
  // the QKV projection's 384 tiles run 256 whole and 128 in two k ranges).
  auto proj = [&](const float* x, int ldx, const void* Wf, const float* W, const float* bias,
                  float* y, int ldy, int N, int K, const lx_epilogue* epi,
                  bool pack_out = false, int pack_from = 0) -> int {
    if (!m->frag) return lx_linear_f32(x, ldx, W, bias, y, ldy, rows, N, K, epi, s);
    lx_linear_bx g{};
    if (m->qkv_ws) {
      g.split_tail = 1;
      g.ws = m->qkv_ws;
      g.ws_floats = m->qkv_ws_floats;
      g.counters = m->qkv_cnt;
      g.n_counters = m->qkv_ncnt;
    }
    g.a_packed = pk ? 1 : 0;
    g.pack_from = pack_out && pk ? pack_from : 0;
    g.A = x;
    g.lda = ldx;
    g.Wf = Wf;
    g.bias = bias;
    g.epi = epi;
    g.out = pack_out && pk ? LX_BX_OUT_PACKED : LX_BX_OUT_F32;
    g.Y = y;
    g.ldy = ldy;
    g.M = rows;
    g.N = N;
    g.K = K;
    g.bm = 64;
    g.slices = 1;
    g.products = m->products;
    return linear_bx(g, s);
  };
  // y (the residual stream h) += gate * (x W^T + bias), directly or as pending K slices
  auto proj_gated = [&](const float* x, int ldx, const void* Wf, const float* W, const float* bias,
                        const float* gate, int K) -> int {
    if (!partial) {
      lx_epilogue gated{};
      gated.kind = LX_EPI_GATED_RESID;
      gated.rows_per_batch = T;
      gated.gate = gate;
      gated.gate_stride = NA;
      return proj(x, ldx, Wf, W, bias, m->h, D, D, K, &gated);
    }
    lx_linear_bx g{};
    g.a_packed = pk ? 1 : 0;
    g.A = x;
    g.lda = ldx;
    g.Wf = Wf;
    g.out = LX_BX_OUT_PARTIAL;
    g.Y = m->Rws;
    g.ldy = D;
    g.slice_stride = (long)rows * D;
    g.M = rows;
    g.N = D;
    g.K = K;
    g.bm = 64;
    g.slices = 2;
    g.products = m->products;
    LX_TRY(linear_bx(g, s));
    pend.bias = bias;
    pend.gate = gate;
    pending = true;
    return LX_OK;
  };
  for (int i = 0; i < m->depth; ++i) {
    const float* e = emb + (long)i * 6 * D;  // chunk order: shift, scale, gate (msa), (mlp)
    const float* shift_msa = e;
    const float* scale_msa = e + D;
    const float* gate_msa = e + 2 * D;
    const float* shift_mlp = e + 3 * D;
    const float* scale_mlp = e + 4 * D;
    const float* gate_mlp = e + 5 * D;
    const void* wf0 = m->frag ? m->qkv_wf[i] : nullptr;
    const void* wf1 = m->frag ? m->out_wf[i] : nullptr;
    const void* wf2 = m->frag ? m->ff0_wf[i] : nullptr;
    const void* wf3 = m->frag ? m->ff2_wf[i] : nullptr;
    const float* w0 = m->frag ? nullptr : m->qkv_w[i];
    const float* w1 = m->frag ? nullptr : m->out_w[i];
    const float* w2 = m->frag ? nullptr : m->ff0_w[i];
    const float* w3 = m->frag ? nullptr : m->ff2_w[i];

    LX_TRY(adaln(shift_msa, scale_msa, m->xn, pk));
    lx_epilogue rope{};
    rope.kind = LX_EPI_ROPE_PARTIAL;
    rope.rows_per_batch = T;
    rope.pos = m->pos;
    rope.rot_dim = kRotDim;
    rope.rope_section = D;   // q occupies columns [0, D), k [D, 2D)
    rope.rope_sections = 2;
    rope.rope_base = kRopeBase;
    LX_TRY(proj(m->xn, D, wf0, w0, m->qkv_b[i], m->qkv, 3 * D, 3 * D, D, &rope, pk_kv,
                /*pack_from*/ D));
    LX_TRY(attention(m->qkv, 3 * D, m->qkv + D, 3 * D, m->qkv + 2 * D, 3 * D, m->att, D, B, T,
                     T, m->heads, m->heads, m->hd, 1.0f / std::sqrt((float)m->hd), 0, 0,
                     m->products, pk ? 1 : 0, s, pk_kv ? 1 : 0));
    LX_TRY(proj_gated(m->att, D, wf1, w1, m->out_b[i], gate_msa, D));

    LX_TRY(adaln(shift_mlp, scale_mlp, m->xn, pk));
    lx_epilogue gelu{};
    gelu.kind = LX_EPI_GELU_TANH;
    LX_TRY(proj(m->xn, D, wf2, w2, m->ff0_b[i], m->ff, m->F, m->F, D, &gelu, /*pack_out*/ true));
    LX_TRY(proj_gated(m->ff, m->F, wf3, w3, m->ff2_b[i], gate_mlp, m->F));
    if (m->cap.blocks) {
      if (pending) {  // the block's output: fold the FF2 slices into h now
        pending = false;
        LX_TRY(lx_adaln_resid_f32(m->h, m->Rws, 2, (long)rows * D, pend.bias, pend.gate, NA,
                                  emb, emb, NA, nullptr, B, T, D, kLnEps, s));
      }
      (void)hipMemcpyAsync(m->cap.blocks + (long)i * rows * D, m->h, sizeof(float) * rows * D,
                           hipMemcpyDeviceToDevice, s);
    }
  }
  // norm_out (AdaLayerNormZero_Final): chunk order scale, shift (src/flow/dit.cpp:134-135).
  const float* ef = emb + (long)m->depth * 6 * D;
  LX_TRY(adaln(/*shift*/ ef + D, /*scale*/ ef, m->xn, /*packed*/ false));
  if (m->cap.norm_out)
    (void)hipMemcpyAsync(m->cap.norm_out, m->xn, sizeof(float) * rows * D, hipMemcpyDeviceToDevice,
                         s);
  // proj_out (N = mel = 80 columns, 2 x 16 tiles at B*T = 1000): split-K slices
  // fill the device; the slice sum + bias is fused into the consumer.
  int ks = 0;
  const int splits = gemm_splitk_plan(rows, mel, D, &ks);
  LX_REQUIRE(splits <= kProjSplitMax, "dit_forward: proj_out plan of %d slices", splits);
  LX_TRY(gemm_splitk_partials(m->xn, D, m->proj_w, D, m->Pws, rows, mel, D, splits, ks, s));
  m->proj_splits = splits;
  m->proj_slice = (long)rows * mel;
  return check_launch("dit forward");
}

// P = the proj_out rows of the last forward (slice sum + bias).
int proj_rows(lx_dit* m, int T, hipStream_t s) {
  return proj_reduce(m->Pws, m->proj_splits, m->proj_slice, m->proj_b, m->P, m->B * T, m->mel, s);
}

}  // namespace

extern "C" int lx_dit_create(const lx_dit_weights* w, int B, int max_T, lx_dit** out) {
  LX_REQUIRE(w && out, "dit_create: null argument");
  *out = nullptr;
  LX_REQUIRE(B >= 1 && B <= 8 && max_T >= 1, "dit_create: B=%d max_T=%d", B, max_T);
  LX_REQUIRE(w->dim > 0 && w->dim % 64 == 0 && w->depth >= 1 && w->heads >= 1 &&
                 w->head_dim == 64 && w->heads * w->head_dim == w->dim && w->ff_inner > 0 &&
                 w->ff_inner % 4 == 0 && w->mel_dim > 0 && w->mel_dim % 4 == 0,
             "dit_create: unsupported geometry dim=%d heads=%d head_dim=%d ff=%d mel=%d",
             w->dim, w->heads, w->head_dim, w->ff_inner, w->mel_dim);
  LX_REQUIRE(w->dim / kConvG == 64, "dit_create: conv_pos needs dim/16 == 64");
  LX_REQUIRE(w->blocks, "dit_create: blocks array is NULL");
  lx_dit* m = new (std::nothrow) lx_dit();
  if (!m) return LX_ERR_ALLOC;
  m->B = B;
  m->max_T = max_T;
  m->D = w->dim;
  m->depth = w->depth;
  m->heads = w->heads;
  m->hd = w->head_dim;
  m->F = w->ff_inner;
  m->mel = w->mel_dim;
  const int D = m->D, F = m->F, mel = m->mel, depth = m->depth;
  m->NA = (long)depth * 6 * D + 2 * D;
  Arena& a = m->arena;
  bool ok = true;
  auto A = [&](size_t n) {
    float* p = a.alloc<float>(n);
    ok = ok && p;
    return p;
  };
  m->tm0_w = A((size_t)D * kFreqDim);
  m->tm0_b = A(D);
  m->tm2_w = A((size_t)D * D);
  m->tm2_b = A(D);
  m->in_w = A((size_t)D * 4 * mel);
  m->in_b = A(D);
  m->conv1_wf = a.alloc<unsigned short>((size_t)3 * D * 64 * kConvK);
  m->conv1_b = A(D);
  m->conv2_wf = a.alloc<unsigned short>((size_t)3 * D * 64 * kConvK);
  m->conv2_b = A(D);
  ok = ok && m->conv1_wf && m->conv2_wf;
  m->ada_w = A((size_t)m->NA * D);
  m->ada_b = A(m->NA);
  const size_t rows = (size_t)B * max_T;
  // the fragment-order GEMM needs N % 128, K % 64 and each activation below 2 GiB
  m->frag = D % 128 == 0 && F % 128 == 0 && rows * F * 4 < (1ull << 31);
  for (int i = 0; i < depth; ++i) {
    if (m->frag) {
      m->qkv_wf.push_back(a.alloc<unsigned short>((size_t)3 * 3 * D * D));
      m->out_wf.push_back(a.alloc<unsigned short>((size_t)3 * D * D));
      m->ff0_wf.push_back(a.alloc<unsigned short>((size_t)3 * F * D));
      m->ff2_wf.push_back(a.alloc<unsigned short>((size_t)3 * D * F));
      ok = ok && m->qkv_wf.back() && m->out_wf.back() && m->ff0_wf.back() && m->ff2_wf.back();
    } else {
      m->qkv_w.push_back(A((size_t)3 * D * D));
      m->out_w.push_back(A((size_t)D * D));
      m->ff0_w.push_back(A((size_t)F * D));
      m->ff2_w.push_back(A((size_t)D * F));
    }
    m->qkv_b.push_back(A((size_t)3 * D));
    m->out_b.push_back(A(D));
    m->ff0_b.push_back(A(F));
    m->ff2_b.push_back(A(D));
  }
  m->proj_w = A((size_t)mel * D);
  m->proj_b = A(mel);
  m->temb = A((size_t)B * D);
  m->tmlp_work = A((size_t)B * D);
  m->emb = A((size_t)B * m->NA);
  m->temb_steps = A((size_t)kSolveChunk * D);
  m->tmlp_steps = A((size_t)kSolveChunk * D);
  m->emb_steps = A((size_t)kSolveChunk * m->NA);
  m->A0 = A(rows * 4 * mel);
  m->xe = A(rows * D);
  m->c1 = A(rows * D);
  m->h = A(rows * D);
  m->xn = A(rows * D);
  m->qkv = A(rows * 3 * D);
  m->att = A(rows * D);
  m->ff = A(rows * F);
  m->P = A(rows * mel);
  m->Pws = A(rows * mel * kProjSplitMax);
  m->Rws = m->frag ? A((size_t)2 * std::min<size_t>(rows, kPartialRows) * D) : nullptr;
  if (m->frag) {
    m->qkv_ws_floats = bx_split_ws_floats(64);
    m->qkv_ws = A(m->qkv_ws_floats);
    m->qkv_ncnt = (int)((rows + 63) / 64) * (std::max(3 * D, F) / 128);
    m->qkv_cnt = a.alloc<unsigned>(m->qkv_ncnt);
    ok = ok && m->qkv_cnt;
  }
  m->pos = a.alloc<int>(max_T);
  ok = ok && m->pos;
  if (!ok) {
    delete m;
    set_error("dit_create: device allocation failed");
    return LX_ERR_ALLOC;
  }

  hipStream_t s = nullptr;
  if (hipStreamCreate(&s) != hipSuccess) {
    delete m;
    set_error("dit_create: stream creation failed");
    return LX_ERR_LAUNCH;
  }
  int rc = LX_OK;
  auto C = [&](float* dst, const float* src, size_t n) {
    if (rc == LX_OK) rc = copy_d2d(dst, src, n, s);
  };
  // fragment-order packing straight from the caller's (N, K) weight; a source
  // that is not 16-byte aligned goes through an aligned staging copy first
  float* stage = nullptr;
  auto P = [&](const float* src, void* dst, int N, int K) {
    if (rc != LX_OK) return;
    if (!src) {
      rc = LX_ERR_ARG;
      return;
    }
    if ((uintptr_t)src % 16) {
      if (!stage && hipMalloc(&stage, sizeof(float) * (size_t)std::max(D, F) * std::max(D, F)) !=
                        hipSuccess) {
        rc = LX_ERR_ALLOC;
        return;
      }
      rc = copy_d2d(stage, src, (size_t)N * K, s);
      src = stage;
    }
    if (rc == LX_OK) rc = wfrag_pack(src, dst, N, K, s);
  };
  C(m->tm0_w, w->time_mlp_0_w, (size_t)D * kFreqDim);
  C(m->tm0_b, w->time_mlp_0_b, D);
  C(m->tm2_w, w->time_mlp_2_w, (size_t)D * D);
  C(m->tm2_b, w->time_mlp_2_b, D);
  C(m->in_w, w->input_proj_w, (size_t)D * 4 * mel);
  C(m->in_b, w->input_proj_b, D);
  C(m->conv1_b, w->conv_pos_1_b, D);
  C(m->conv2_b, w->conv_pos_2_b, D);
  if (rc == LX_OK) rc = (w->conv_pos_1_w && w->conv_pos_2_w) ? LX_OK : LX_ERR_ARG;
  if (rc == LX_OK) rc = conv_frag_pack(w->conv_pos_1_w, m->conv1_wf, D, kConvG, kConvK, s);
  if (rc == LX_OK) rc = conv_frag_pack(w->conv_pos_2_w, m->conv2_wf, D, kConvG, kConvK, s);
  for (int i = 0; i < depth && rc == LX_OK; ++i) {
    const lx_dit_block_weights& bw = w->blocks[i];
    C(m->ada_w + (size_t)i * 6 * D * D, bw.attn_norm_w, (size_t)6 * D * D);
    C(m->ada_b + (size_t)i * 6 * D, bw.attn_norm_b, (size_t)6 * D);
    C(m->qkv_b[i], bw.to_q_b, D);
    C(m->qkv_b[i] + D, bw.to_k_b, D);
    C(m->qkv_b[i] + 2 * D, bw.to_v_b, D);
    C(m->out_b[i], bw.to_out_b, D);
    C(m->ff0_b[i], bw.ff0_b, F);
    C(m->ff2_b[i], bw.ff2_b, D);
    if (m->frag) {
      // the fused QKV matrix in fragment order: q, k and v are whole 32-row
      // blocks of it, 3 D D bf16 apart
      unsigned short* q = static_cast<unsigned short*>(m->qkv_wf[i]);
      P(bw.to_q_w, q, D, D);
      P(bw.to_k_w, q + (size_t)3 * D * D, D, D);
      P(bw.to_v_w, q + (size_t)6 * D * D, D, D);
      P(bw.to_out_w, m->out_wf[i], D, D);
      P(bw.ff0_w, m->ff0_wf[i], F, D);
      P(bw.ff2_w, m->ff2_wf[i], D, F);
    } else {
      C(m->qkv_w[i], bw.to_q_w, (size_t)D * D);
      C(m->qkv_w[i] + (size_t)D * D, bw.to_k_w, (size_t)D * D);
      C(m->qkv_w[i] + (size_t)2 * D * D, bw.to_v_w, (size_t)D * D);
      C(m->out_w[i], bw.to_out_w, (size_t)D * D);
      C(m->ff0_w[i], bw.ff0_w, (size_t)F * D);
      C(m->ff2_w[i], bw.ff2_w, (size_t)D * F);
    }
  }
  C(m->ada_w + (size_t)depth * 6 * D * D, w->norm_out_w, (size_t)2 * D * D);
  C(m->ada_b + (size_t)depth * 6 * D, w->norm_out_b, (size_t)2 * D);
  C(m->proj_w, w->proj_out_w, (size_t)mel * D);
  C(m->proj_b, w->proj_out_b, mel);
  if (rc == LX_OK) rc = iota_i32(m->pos, max_T, s);
  if (rc == LX_OK && m->qkv_cnt &&
      hipMemsetAsync(m->qkv_cnt, 0, sizeof(unsigned) * m->qkv_ncnt, s) != hipSuccess)
    rc = LX_ERR_LAUNCH;
  if (rc == LX_OK && hipStreamSynchronize(s) != hipSuccess) {
    set_error("dit_create: weight packing failed");
    rc = LX_ERR_LAUNCH;
  }
  (void)hipStreamDestroy(s);
  if (stage) (void)hipFree(stage);
  if (rc != LX_OK) {
    if (rc == LX_ERR_ARG) set_error("dit_create: missing weight tensor");
    delete m;
    return rc;
  }
  *out = m;
  return LX_OK;
}

extern "C" void lx_dit_destroy(lx_dit* dit) {
  if (!dit) return;
  (void)hipDeviceSynchronize();
  delete dit;
}

extern "C" int lx_dit_set_capture(lx_dit* dit, const lx_dit_capture* cap) {
  LX_REQUIRE(dit, "dit_set_capture: null estimator");
  if (cap)
    dit->cap = *cap;
  else
    dit->cap = lx_dit_capture{};
  return LX_OK;
}

extern "C" int lx_dit_set_products(lx_dit* dit, int products) {
  LX_REQUIRE(dit, "dit_set_products: null estimator");
  LX_REQUIRE(products == 3 || products == 6, "dit_set_products: %d products (3 or 6)", products);
  dit->products = products;
  return LX_OK;
}

extern "C" int lx_dit_forward(lx_dit* m, const float* x, const float* mu, const float* cond,
                              const float* spks, const float* t, float* dphi, int T,
                              hipStream_t s) {
  LX_REQUIRE(m && x && mu && cond && spks && t && dphi, "dit_forward: null argument");
  LX_REQUIRE(T >= 1 && T <= m->max_T, "dit_forward: T=%d outside [1, %d]", T, m->max_T);
  LX_TRY(forward_core(m, x, (long)m->mel * T, mu, cond, spks, 0, t, nullptr, T, s));
  LX_TRY(proj_rows(m, T, s));
  return dit_unpack_output(m->P, dphi, m->B, T, m->mel, s);
}

extern "C" int lx_cfm_step(lx_dit* m, float* x, const float* mu, const float* cond,
                           const float* spks, int T, float t, float dt, float cfg_rate,
                           hipStream_t s) {
  LX_REQUIRE(m && x && mu && cond && spks, "cfm_step: null argument");
  LX_REQUIRE(m->B == 2, "cfm_step: the estimator must be built with B == 2 (CFG pair)");
  LX_REQUIRE(T >= 1 && T <= m->max_T, "cfm_step: T=%d outside [1, %d]", T, m->max_T);
  // Batch-2 inputs (src/flow/flow.cpp:215-224): both rows read x (batch stride
  // 0); mu, cond and spks feed the conditional row, zeros the unconditional one.
  const float tt[2] = {t, t};
  LX_TRY(forward_core(m, x, 0, mu, cond, spks, 1, nullptr, tt, T, s));
  // combined = (1+cfg) dphi_cond - cfg dphi_uncond; x += dt * combined (flow.cpp:256-259)
  return cfm_euler_update(x, m->Pws, m->proj_splits, m->proj_slice, m->proj_b, T, m->mel, dt,
                          1.0f + cfg_rate, cfg_rate, s);
}

extern "C" int lx_cfm_solve(lx_dit* m, float* x, const float* mu, const float* cond,
                            const float* spks, int T, int n_steps, float cfg_rate,
                            hipStream_t s) {
  LX_REQUIRE(m && x && mu && cond && spks, "cfm_solve: null argument");
  LX_REQUIRE(n_steps >= 1 && n_steps <= 1000, "cfm_solve: n_steps=%d", n_steps);
  LX_REQUIRE(m->B == 2, "cfm_solve: the estimator must be built with B == 2 (CFG pair)");
  LX_REQUIRE(T >= 1 && T <= m->max_T, "cfm_solve: T=%d outside [1, %d]", T, m->max_T);
  // t_span = 1 - cos(linspace(0, 1, n+1) * pi/2), evaluated as src/flow/flow.cpp:203-207.
  const float PI = 3.14159265358979323846f;
  std::vector<float> t_span(n_steps + 1);
  for (int i = 0; i <= n_steps; ++i) {
    float tt = (float)i / (float)n_steps;
    t_span[i] = 1.0f - cosf(tt * 0.5f * PI);
  }
  // The t and dt of every step, by the recurrence of src/flow/flow.cpp:240-276 (t += dt).
  std::vector<float> ts(n_steps), dts(n_steps);
  float t = t_span[0];
  float dt = t_span[1] - t_span[0];
  for (int step = 1; step <= n_steps; ++step) {
    ts[step - 1] = t;
    dts[step - 1] = dt;
    t += dt;
    if (step < n_steps) dt = t_span[step + 1] - t;
  }
  // t does not depend on x, so the time embeddings and AdaLN modulations of up
  // to kSolveChunk steps come from one time MLP and one stacked GEMV (one
  // stream of the modulation weights instead of one per step).  Each step's
  // row is computed with the arithmetic of the per-step GEMV, and both rows of
  // the CFG pair share it, so the solve matches a sequence of lx_cfm_step.
  // With a time-embedding capture set, steps run one by one (the capture
  // records each step's embedding).
  for (int c0 = 0; c0 < n_steps; c0 += kSolveChunk) {
    const int nc = std::min(kSolveChunk, n_steps - c0);
    const bool batched = !m->cap.time_embed;
    if (batched) {
      LX_TRY(time_mlp(nullptr, ts.data() + c0, nc, m->tm0_w, m->tm0_b, m->tm2_w, m->tm2_b, m->D,
                      m->tmlp_steps, m->temb_steps, s));
      LX_TRY(gemv(m->temb_steps, nc, m->D, m->ada_w, m->ada_b, m->emb_steps, m->NA, m->NA,
                  /*silu in*/ 1, 0, s));
    }
    for (int j = 0; j < nc; ++j) {
      const float tt[2] = {ts[c0 + j], ts[c0 + j]};
      LX_TRY(forward_core(m, x, 0, mu, cond, spks, 1, nullptr, tt, T, s,
                          batched ? m->emb_steps + (long)j * m->NA : nullptr, 0));
      LX_TRY(cfm_euler_update(x, m->Pws, m->proj_splits, m->proj_slice, m->proj_b, T, m->mel,
                              dts[c0 + j], 1.0f + cfg_rate, cfg_rate, s));
    }
  }
  return LX_OK;
}
