// larynx::flow::FlowDecoder and larynx::llm::LLM over liblxops: the binding a
// maintainer of the reference would add in src/flow/flow.cpp and
// src/llm/llm.cpp (the ggml backend, graph build and per-step uploads replaced
// by the lx_flow / lx_qwen2 objects of include/lx_ops.h).  Host vectors in and
// out, staged through device buffers; errors as bool false plus a message on
// stderr, as the reference reports them (src/flow/flow.cpp:117, 127).
#include "larynx_dropin.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <string>
#include <vector>

#include "lx_ops.h"

namespace {

// One device allocation, freed with its owner.
struct DevBuf {
  void* p = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  bool alloc(size_t bytes) {
    if (p) (void)hipFree(p);
    p = nullptr;
    return hipMalloc(&p, bytes ? bytes : 4) == hipSuccess;
  }
  float* f() const { return static_cast<float*>(p); }
};

bool up(DevBuf& d, const void* src, size_t bytes) {
  return d.alloc(bytes) && (bytes == 0 || hipMemcpy(d.p, src, bytes, hipMemcpyHostToDevice) ==
                                              hipSuccess);
}

bool down(std::vector<float>& dst, const float* src, size_t n) {
  dst.resize(n);
  return n == 0 ||
         hipMemcpy(dst.data(), src, n * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess;
}

bool lx_ok(int rc, const char* what) {
  if (rc == LX_OK) return true;
  std::fprintf(stderr, "%s: %s\n", what, lx_last_error());
  return false;
}

// Shape of a tensor in a GGUF file (torch order), read without a device copy.
std::vector<int64_t> gguf_shape(lx_gguf* g, const std::string& name) {
  const int i = lx_gguf_find(g, name.c_str());
  if (i < 0) return {};
  int nd = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  if (lx_gguf_tensor_info(g, i, nullptr, nullptr, &nd, ne, nullptr) != LX_OK) return {};
  std::vector<int64_t> s;
  for (int d = nd - 1; d >= 0; --d) s.push_back(ne[d]);
  return s;
}

}  // namespace

namespace larynx::flow {

struct FlowDecoder::Impl {
  lx_flow* flow = nullptr;
  int mel = 0, spk_in = 0, dim = 0, depth = 0;
};

FlowDecoder::FlowDecoder() : impl_(new Impl) {}

FlowDecoder::~FlowDecoder() {
  if (impl_->flow) lx_flow_destroy(impl_->flow);
  delete impl_;
}

bool FlowDecoder::load(const std::string& gguf_path, int max_tokens) {
  lx_gguf* g = nullptr;
  if (!lx_ok(lx_gguf_open(gguf_path.c_str(), LX_GGUF_HOST_ONLY, &g), "flow: load")) return false;
  const auto spk = gguf_shape(g, "spk_embed_affine_layer.weight");              // (80, 192)
  const auto proj = gguf_shape(g, "decoder.estimator.input_embed.proj.weight");  // (D, 320)
  int depth = 0;
  while (lx_gguf_find(g, ("decoder.estimator.transformer_blocks." + std::to_string(depth) +
                          ".attn.to_q.weight").c_str()) >= 0)
    ++depth;
  lx_gguf_close(g);
  if (spk.size() != 2 || proj.size() != 2 || depth == 0) {
    std::fprintf(stderr, "flow: %s is not a flow checkpoint\n", gguf_path.c_str());
    return false;
  }
  impl_->mel = (int)spk[0];
  impl_->spk_in = (int)spk[1];
  impl_->dim = (int)proj[0];
  impl_->depth = depth;
  if (impl_->flow) lx_flow_destroy(impl_->flow);
  impl_->flow = nullptr;
  return lx_ok(lx_flow_load(gguf_path.c_str(), max_tokens, &impl_->flow), "flow: load");
}

bool FlowDecoder::infer(const std::vector<int32_t>& prompt_tokens,
                        const std::vector<int32_t>& tokens, const std::vector<float>& prompt_feat,
                        const std::vector<float>& spk_embedding,
                        const std::vector<float>& noise_z, std::vector<float>& mel_out,
                        FlowDebug* debug) {
  if (!impl_->flow) {
    std::fprintf(stderr, "flow: infer before load\n");
    return false;
  }
  const int mel = impl_->mel, D = impl_->dim;
  const int Tseq = (int)(prompt_tokens.size() + tokens.size());
  const int MT = 2 * Tseq;
  const int mel_len1 = (int)(prompt_feat.size() / mel);
  if (noise_z.size() != (size_t)MT * mel || prompt_feat.size() % mel ||
      spk_embedding.size() != (size_t)impl_->spk_in) {
    std::fprintf(stderr, "flow: noise_z / prompt_feat / spk_embedding size mismatch\n");
    return false;
  }
  DevBuf pf, spk, z, out;
  if (!up(pf, prompt_feat.data(), prompt_feat.size() * 4) ||
      !up(spk, spk_embedding.data(), spk_embedding.size() * 4) ||
      !up(z, noise_z.data(), noise_z.size() * 4) ||
      !out.alloc(sizeof(float) * mel * (size_t)(MT > mel_len1 ? MT - mel_len1 : 1))) {
    std::fprintf(stderr, "flow: device staging failed\n");
    return false;
  }
  DevBuf c_spk, c_tok, c_pre, c_mu, c_cond;
  lx_flow_capture cap{};
  if (debug) {
    if (!c_spk.alloc(4L * mel) || !c_tok.alloc(4L * Tseq * mel) || !c_pre.alloc(4L * Tseq * mel) ||
        !c_mu.alloc(4L * mel * MT) || !c_cond.alloc(4L * mel * MT)) {
      std::fprintf(stderr, "flow: device staging failed\n");
      return false;
    }
    cap = {c_spk.f(), c_tok.f(), c_pre.f(), c_mu.f(), c_cond.f()};
  }
  lx_flow_set_capture(impl_->flow, debug ? &cap : nullptr);
  const int rc = lx_flow_infer(impl_->flow, prompt_tokens.data(), (int)prompt_tokens.size(),
                               tokens.data(), (int)tokens.size(), pf.f(), mel_len1, spk.f(),
                               z.f(), out.f(), nullptr);
  lx_flow_set_capture(impl_->flow, nullptr);
  if (!lx_ok(rc, "flow: infer")) return false;
  if (!down(mel_out, out.f(), (size_t)mel * (MT - mel_len1))) return false;
  if (!debug) return true;

  debug->feat = mel_out;
  bool ok = down(debug->spk, c_spk.f(), mel) && down(debug->token_embed, c_tok.f(), (size_t)Tseq * mel) &&
            down(debug->prelookahead, c_pre.f(), (size_t)Tseq * mel) &&
            down(debug->mu, c_mu.f(), (size_t)mel * MT) && down(debug->cond, c_cond.f(), (size_t)mel * MT);
  if (!ok) return false;
  // DiT internals at CFM step 1: x_in = [z; z], mu/cond/spks = [cond row; 0],
  // t = t_span[0] = 0 (src/flow/flow.cpp:215-250, captured at :261-270).
  lx_dit* est = lx_flow_estimator(impl_->flow);
  const size_t n = (size_t)mel * MT, rows = 2 * (size_t)MT;
  DevBuf x2, mu2, cond2, spks2, t2, dphi, te, ip, cp, ie, bl, no;
  const float t0[2] = {0.0f, 0.0f};
  ok = x2.alloc(8 * n) && mu2.alloc(8 * n) && cond2.alloc(8 * n) && spks2.alloc(8L * mel) &&
       up(t2, t0, sizeof t0) && dphi.alloc(8 * n) && te.alloc(8L * D) && ip.alloc(4 * rows * D) &&
       cp.alloc(4 * rows * D) && ie.alloc(4 * rows * D) &&
       bl.alloc(4 * rows * D * (size_t)impl_->depth) && no.alloc(4 * rows * D);
  ok = ok && hipMemcpy(x2.f(), z.f(), 4 * n, hipMemcpyDeviceToDevice) == hipSuccess &&
       hipMemcpy(x2.f() + n, z.f(), 4 * n, hipMemcpyDeviceToDevice) == hipSuccess &&
       hipMemcpy(mu2.f(), c_mu.f(), 4 * n, hipMemcpyDeviceToDevice) == hipSuccess &&
       hipMemset(mu2.f() + n, 0, 4 * n) == hipSuccess &&
       hipMemcpy(cond2.f(), c_cond.f(), 4 * n, hipMemcpyDeviceToDevice) == hipSuccess &&
       hipMemset(cond2.f() + n, 0, 4 * n) == hipSuccess &&
       hipMemcpy(spks2.f(), c_spk.f(), 4L * mel, hipMemcpyDeviceToDevice) == hipSuccess &&
       hipMemset(spks2.f() + mel, 0, 4L * mel) == hipSuccess;
  if (!ok) {
    std::fprintf(stderr, "flow: device staging failed\n");
    return false;
  }
  lx_dit_capture dc = {te.f(), ip.f(), cp.f(), ie.f(), bl.f(), no.f()};
  lx_dit_set_capture(est, &dc);
  const int rc2 = lx_dit_forward(est, x2.f(), mu2.f(), cond2.f(), spks2.f(), t2.f(), dphi.f(), MT,
                                 nullptr);
  lx_dit_set_capture(est, nullptr);
  if (!lx_ok(rc2, "flow: step-1 estimator capture")) return false;
  ok = down(debug->time_embed, te.f(), 2L * D) && down(debug->input_proj, ip.f(), rows * D) &&
       down(debug->conv_pos, cp.f(), rows * D) && down(debug->input_embed, ie.f(), rows * D) &&
       down(debug->norm_out, no.f(), rows * D) && down(debug->dphi, dphi.f(), 2 * n);
  debug->blocks.resize(impl_->depth);
  for (int i = 0; ok && i < impl_->depth; ++i)
    ok = down(debug->blocks[i], bl.f() + (size_t)i * rows * D, rows * D);
  return ok;
}

}  // namespace larynx::flow

namespace larynx::llm {

struct LLM::Impl {
  lx_qwen2* m = nullptr;
  int H = 0, V = 0, NL = 0, KV = 0;
  mutable std::vector<std::vector<float>> k, v;
};

LLM::LLM() : impl_(new Impl) {}

LLM::~LLM() {
  release();
  delete impl_;
}

void LLM::release() {
  if (impl_->m) lx_qwen2_destroy(impl_->m);
  impl_->m = nullptr;
}

int LLM::hidden() const { return impl_->H; }
int LLM::speech_vocab() const { return impl_->V; }
int LLM::n_layers() const { return impl_->NL; }
int LLM::kv_width() const { return impl_->KV; }

bool LLM::load(const std::string& path, int max_ctx) {
  lx_gguf* g = nullptr;
  if (!lx_ok(lx_gguf_open(path.c_str(), LX_GGUF_HOST_ONLY, &g), "llm: load")) return false;
  const std::string M = "llm.model.model.";
  const auto emb = gguf_shape(g, M + "embed_tokens.weight");
  const auto spe = gguf_shape(g, "speech_embedding.weight");
  const auto kw = gguf_shape(g, M + "layers.0.self_attn.k_proj.weight");
  int nl = 0;
  while (lx_gguf_find(g, (M + "layers." + std::to_string(nl) + ".self_attn.q_proj.weight")
                             .c_str()) >= 0)
    ++nl;
  lx_gguf_close(g);
  if (emb.size() != 2 || spe.size() != 2 || kw.size() != 2 || nl == 0) {
    std::fprintf(stderr, "llm: %s is not an LLM checkpoint\n", path.c_str());
    return false;
  }
  release();
  impl_->H = (int)emb[1];
  impl_->V = (int)spe[0];
  impl_->KV = (int)kw[0];
  impl_->NL = nl;
  impl_->k.assign(nl, {});
  impl_->v.assign(nl, {});
  return lx_ok(lx_qwen2_load(path.c_str(), max_ctx, &impl_->m), "llm: load");
}

bool LLM::build_lm_input(const std::vector<int>& text_tokens,
                         const std::vector<int>& prompt_speech_token,
                         std::vector<float>& lm_input, int* L_out) {
  if (!impl_->m) return false;
  const int L = 2 + (int)text_tokens.size() + (int)prompt_speech_token.size();
  DevBuf out;
  if (!out.alloc(sizeof(float) * L * impl_->H)) return false;
  int Lr = 0;
  if (!lx_ok(lx_qwen2_build_lm_input(impl_->m, text_tokens.data(), (int)text_tokens.size(),
                                     prompt_speech_token.data(),
                                     (int)prompt_speech_token.size(), out.f(), &Lr, nullptr),
             "llm: build_lm_input"))
    return false;
  if (L_out) *L_out = Lr;
  return down(lm_input, out.f(), (size_t)Lr * impl_->H);
}

bool LLM::prefill(const std::vector<float>& lm_input, int L, LLMDebug* debug) {
  if (!impl_->m || L < 1 || lm_input.size() != (size_t)L * impl_->H) {
    std::fprintf(stderr, "llm: prefill: bad input (L=%d)\n", L);
    return false;
  }
  const size_t H = impl_->H;
  DevBuf x, logits, hid, fin;
  if (!up(x, lm_input.data(), lm_input.size() * 4) || !logits.alloc(4 * (size_t)L * impl_->V) ||
      (debug && (!hid.alloc(4 * (size_t)impl_->NL * L * H) || !fin.alloc(4 * (size_t)L * H))))
    return false;
  if (!lx_ok(lx_qwen2_prefill(impl_->m, x.f(), L, logits.f(), debug ? hid.f() : nullptr,
                              debug ? fin.f() : nullptr, nullptr),
             "llm: prefill"))
    return false;
  if (!debug) return hipDeviceSynchronize() == hipSuccess;
  debug->hidden_states.resize(impl_->NL);
  bool ok = true;
  for (int i = 0; ok && i < impl_->NL; ++i)
    ok = down(debug->hidden_states[i], hid.f() + (size_t)i * L * H, (size_t)L * H);
  return ok && down(debug->final_norm, fin.f(), (size_t)L * H) &&
         down(debug->logits, logits.f(), (size_t)L * impl_->V);
}

bool LLM::decode(int token, std::vector<float>& logits, std::vector<float>* final_norm) {
  if (!impl_->m) return false;
  DevBuf lg, fn;
  if (!lg.alloc(4L * impl_->V) || !fn.alloc(4L * impl_->H)) return false;
  if (!lx_ok(lx_qwen2_decode(impl_->m, token, lg.f(), final_norm ? fn.f() : nullptr, nullptr),
             "llm: decode"))
    return false;
  return down(logits, lg.f(), impl_->V) && (!final_norm || down(*final_norm, fn.f(), impl_->H));
}

int LLM::cache_len() const { return impl_->m ? lx_qwen2_cache_len(impl_->m) : 0; }

const std::vector<float>& LLM::cache_key(int layer) const {
  std::vector<float>& dst = impl_->k.at(layer);
  if (!down(dst, lx_qwen2_cache_key(impl_->m, layer), (size_t)cache_len() * impl_->KV))
    dst.clear();
  return dst;
}

const std::vector<float>& LLM::cache_value(int layer) const {
  std::vector<float>& dst = impl_->v.at(layer);
  if (!down(dst, lx_qwen2_cache_value(impl_->m, layer), (size_t)cache_len() * impl_->KV))
    dst.clear();
  return dst;
}

}  // namespace larynx::llm
