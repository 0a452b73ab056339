// Flow decoder: the whole-sequence FlowDecoder::infer (src/flow/flow.cpp:111-290)
// on the device.  The frontend graph the reference runs once per utterance
// (flow.cpp:139-170: speaker affine, token embedding, PreLookaheadLayer,
// repeat-interleave to mel rate, prompt-mel conditioning) becomes a handful of
// launches: one gather, two im2col + matrix-core GEMMs for the PreLookahead
// convolutions (conv2's bias and residual fused in the GEMM epilogue) and one
// packing pass.  The CFM solve then runs on the B = 2 estimator (lx_dit) with
// the start noise copied in, and the output frames past the prompt are copied
// out.  Nothing crosses PCIe except the token ids.
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
#include <vector>

#include "lx_common.hpp"
#include "lx_internal.hpp"

using namespace lx;

namespace {

constexpr int kPreLookahead = 3;   // PRE_LOOKAHEAD (src/flow/internal.h:28): conv1 k = 4
constexpr int kConv2K = 3;         // PreLookaheadLayer.conv2 kernel (prelookahead.cpp:16)
constexpr int kTokenMelRatio = 2;  // TOKEN_MEL_RATIO (src/flow/internal.h:29)
constexpr int kSteps = 10;         // N_TIMESTEPS (src/flow/internal.h:30)
constexpr float kCfgRate = 0.7f;   // CFG_RATE (src/flow/internal.h:31)

}  // namespace

struct lx_flow {
  Arena arena;
  lx_dit* dit = nullptr;
  int mel = 0, vocab = 0, spk_in = 0, ch = 0, max_tokens = 0;
  // weights (frontend, re-packed)
  float *emb = nullptr, *spk_w = nullptr, *spk_b = nullptr;
  float *w1p = nullptr, *b1 = nullptr, *w2p = nullptr, *b2 = nullptr;
  // per-call buffers (max_tokens rows)
  float *spk = nullptr, *tok = nullptr, *a1 = nullptr, *y1 = nullptr, *a2 = nullptr,
        *pre = nullptr, *mu = nullptr, *cond = nullptr, *x = nullptr;
  std::vector<int32_t> ids;  // host staging of the clamped token ids
  lx_flow_capture cap{};

  ~lx_flow() {
    if (dit) lx_dit_destroy(dit);
  }
};

extern "C" int lx_flow_create(const lx_dit_weights* dw, const lx_flow_frontend_weights* fw,
                              int max_tokens, lx_flow** out) {
  LX_REQUIRE(dw && fw && out, "flow_create: null argument");
  *out = nullptr;
  LX_REQUIRE(max_tokens >= 1 && max_tokens <= 32768, "flow_create: max_tokens=%d", max_tokens);
  const int mel = dw->mel_dim;
  LX_REQUIRE(fw->vocab > 0 && fw->spk_in > 0 && fw->spk_in <= 1024 && fw->channels > 0 &&
                 fw->channels % 4 == 0 && mel > 0 && mel % 4 == 0,
             "flow_create: unsupported frontend geometry vocab=%d spk_in=%d channels=%d mel=%d",
             fw->vocab, fw->spk_in, fw->channels, mel);
  LX_REQUIRE(fw->input_embedding && fw->spk_affine_w && fw->spk_affine_b && fw->pre_conv1_w &&
                 fw->pre_conv1_b && fw->pre_conv2_w && fw->pre_conv2_b,
             "flow_create: missing frontend tensor");
  lx_flow* f = new (std::nothrow) lx_flow();
  if (!f) return LX_ERR_ALLOC;
  f->mel = mel;
  f->vocab = fw->vocab;
  f->spk_in = fw->spk_in;
  f->ch = fw->channels;
  f->max_tokens = max_tokens;
  int rc = lx_dit_create(dw, 2, kTokenMelRatio * max_tokens, &f->dit);
  if (rc != LX_OK) {
    delete f;
    return rc;
  }
  const int K1 = kPreLookahead + 1, ch = f->ch;
  const size_t Tm = (size_t)max_tokens, MT = (size_t)kTokenMelRatio * max_tokens;
  Arena& a = f->arena;
  bool ok = true;
  auto A = [&](size_t n) {
    float* p = a.alloc<float>(n);
    ok = ok && p;
    return p;
  };
  f->emb = A((size_t)f->vocab * mel);
  f->spk_w = A((size_t)mel * f->spk_in);
  f->spk_b = A(mel);
  f->w1p = A((size_t)ch * K1 * mel);
  f->b1 = A(ch);
  f->w2p = A((size_t)mel * kConv2K * ch);
  f->b2 = A(mel);
  f->spk = A(mel);
  f->tok = A(Tm * mel);
  f->a1 = A(Tm * K1 * mel);
  f->y1 = A(Tm * ch);
  f->a2 = A(Tm * kConv2K * ch);
  f->pre = A(Tm * mel);
  f->mu = A((size_t)mel * MT);
  f->cond = A((size_t)mel * MT);
  f->x = A((size_t)mel * MT);
  if (!ok) {
    delete f;
    set_error("flow_create: device allocation failed");
    return LX_ERR_ALLOC;
  }
  hipStream_t s = nullptr;
  if (hipStreamCreate(&s) != hipSuccess) {
    delete f;
    set_error("flow_create: stream creation failed");
    return LX_ERR_LAUNCH;
  }
  auto C = [&](float* dst, const float* src, size_t n) {
    if (rc == LX_OK && hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                           hipSuccess) {
      set_error("flow_create: device copy failed");
      rc = LX_ERR_LAUNCH;
    }
  };
  C(f->emb, fw->input_embedding, (size_t)f->vocab * mel);
  C(f->spk_w, fw->spk_affine_w, (size_t)mel * f->spk_in);
  C(f->spk_b, fw->spk_affine_b, mel);
  C(f->b1, fw->pre_conv1_b, ch);
  C(f->b2, fw->pre_conv2_b, mel);
  if (rc == LX_OK) rc = conv_kmajor_pack(fw->pre_conv1_w, ch, mel, K1, f->w1p, s);
  if (rc == LX_OK) rc = conv_kmajor_pack(fw->pre_conv2_w, mel, ch, kConv2K, f->w2p, s);
  if (rc == LX_OK && hipStreamSynchronize(s) != hipSuccess) {
    set_error("flow_create: weight packing failed");
    rc = LX_ERR_LAUNCH;
  }
  (void)hipStreamDestroy(s);
  if (rc != LX_OK) {
    delete f;
    return rc;
  }
  f->ids.resize(max_tokens);
  *out = f;
  return LX_OK;
}

extern "C" void lx_flow_destroy(lx_flow* f) {
  if (!f) return;
  (void)hipDeviceSynchronize();
  delete f;
}

extern "C" lx_dit* lx_flow_estimator(lx_flow* f) { return f ? f->dit : nullptr; }

extern "C" int lx_flow_set_capture(lx_flow* f, const lx_flow_capture* cap) {
  LX_REQUIRE(f, "flow_set_capture: null decoder");
  f->cap = cap ? *cap : lx_flow_capture{};
  return LX_OK;
}

namespace {

int copy_out(float* dst, const float* src, size_t n, hipStream_t s) {
  if (!dst) return LX_OK;
  if (hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s) != hipSuccess) {
    set_error("flow: capture copy failed");
    return LX_ERR_LAUNCH;
  }
  return LX_OK;
}

}  // namespace

extern "C" int lx_flow_infer(lx_flow* f, const int32_t* prompt_tokens, int n_prompt,
                             const int32_t* tokens, int n_tokens, const float* prompt_feat,
                             int mel_len1, const float* spk_embedding, const float* noise_z,
                             float* mel_out, hipStream_t s) {
  LX_REQUIRE(f && spk_embedding && noise_z && mel_out, "flow_infer: null argument");
  LX_REQUIRE(n_prompt >= 0 && n_tokens >= 0 && (prompt_tokens || n_prompt == 0) &&
                 (tokens || n_tokens == 0),
             "flow_infer: bad token arrays");
  const int Tseq = n_prompt + n_tokens;
  LX_REQUIRE(Tseq >= 1 && Tseq <= f->max_tokens, "flow_infer: %d tokens outside [1, %d]", Tseq,
             f->max_tokens);
  const int mel = f->mel, ch = f->ch, K1 = kPreLookahead + 1;
  const int MT = kTokenMelRatio * Tseq;
  LX_REQUIRE(mel_len1 >= 0 && mel_len1 < MT && (prompt_feat || mel_len1 == 0),
             "flow_infer: prompt_feat of %d frames for %d mel frames", mel_len1, MT);
  // token.clamp(min=0) (src/flow/flow.cpp:128-130); ids past the table are errors
  for (int i = 0; i < Tseq; ++i) {
    const int32_t v = i < n_prompt ? prompt_tokens[i] : tokens[i - n_prompt];
    f->ids[i] = v < 0 ? 0 : v;
  }
  // spk = Linear(l2_normalize(spk_embedding))
  LX_TRY(flow_spk_affine(spk_embedding, f->spk_in, f->spk_w, f->spk_b, f->spk, mel, s));
  // token_embed = input_embedding[ids]  (LX_ERR_RANGE before any work on a bad id)
  LX_TRY(lx_embed_gather_f32(f->emb, f->vocab, mel, f->ids.data(), Tseq, f->tok, s));
  // PreLookahead: conv1 over [x; 0 0 0] (right pad 3), leaky_relu, conv2 over
  // [0 0; y] (left pad 2), + x; the residual is pre's initial content.
  LX_TRY(flow_im2col(f->tok, Tseq, mel, K1, 0, 0, f->a1, s));
  LX_TRY(lx_linear_f32(f->a1, K1 * mel, f->w1p, f->b1, f->y1, ch, Tseq, ch, K1 * mel, nullptr, s));
  LX_TRY(flow_im2col(f->y1, Tseq, ch, kConv2K, kConv2K - 1, 1, f->a2, s));
  if (hipMemcpyAsync(f->pre, f->tok, sizeof(float) * Tseq * mel, hipMemcpyDeviceToDevice, s) !=
      hipSuccess) {
    set_error("flow_infer: device copy failed");
    return LX_ERR_LAUNCH;
  }
  lx_epilogue resid{};
  resid.kind = LX_EPI_RESID;
  LX_TRY(lx_linear_f32(f->a2, kConv2K * ch, f->w2p, f->b2, f->pre, mel, Tseq, mel, kConv2K * ch,
                       &resid, s));
  // mu = repeat_interleave(pre, 2)^T, cond = [prompt_feat^T | 0]
  LX_TRY(flow_pack_mu_cond(f->pre, Tseq, kTokenMelRatio, prompt_feat, mel_len1, mel, f->mu,
                           f->cond, s));
  LX_TRY(copy_out(f->cap.spk, f->spk, mel, s));
  LX_TRY(copy_out(f->cap.token_embed, f->tok, (size_t)Tseq * mel, s));
  LX_TRY(copy_out(f->cap.prelookahead, f->pre, (size_t)Tseq * mel, s));
  LX_TRY(copy_out(f->cap.mu, f->mu, (size_t)mel * MT, s));
  LX_TRY(copy_out(f->cap.cond, f->cond, (size_t)mel * MT, s));
  // CFM solve from the caller's noise (the reference's noise_z argument)
  if (hipMemcpyAsync(f->x, noise_z, sizeof(float) * mel * MT, hipMemcpyDeviceToDevice, s) !=
      hipSuccess) {
    set_error("flow_infer: device copy failed");
    return LX_ERR_LAUNCH;
  }
  LX_TRY(lx_cfm_solve(f->dit, f->x, f->mu, f->cond, f->spk, MT, kSteps, kCfgRate, s));
  // feat[:, :, mel_len1:]
  const int out_frames = MT - mel_len1;
  if (hipMemcpy2DAsync(mel_out, sizeof(float) * out_frames, f->x + mel_len1, sizeof(float) * MT,
                       sizeof(float) * out_frames, mel, hipMemcpyDeviceToDevice, s) !=
      hipSuccess) {
    set_error("flow_infer: output copy failed");
    return LX_ERR_LAUNCH;
  }
  return check_launch("flow_infer");
}
