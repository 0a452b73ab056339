// The reference's dump utilities (tests/flow_dump.cpp, tests/llm_dump.cpp) as
// C entry points over the drop-in classes: the same load -> infer / prefill
// sequence through the public C++ interfaces, with every stage written to
// caller-owned host buffers instead of raw .f32 files, so a test can call them
// in-process (ctypes) and compare against the oracle.
#include <cstdint>
#include <cstring>
#include <vector>

#include "larynx_dropin.h"

namespace {

void put(float* dst, const std::vector<float>& v) {
  if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(float));
}

}  // namespace

extern "C" {

// Stage buffers (host, caller-sized from the case's shapes); any may be NULL.
typedef struct dropin_flow_out {
  float *spk, *token_embed, *prelookahead, *mu, *cond;
  float *time_embed, *input_proj, *conv_pos, *input_embed, *blocks, *norm_out, *dphi;
  float* feat;
} dropin_flow_out;

// tests/flow_dump.cpp:86-136: FlowDecoder::load, then infer with FlowDebug.
int dropin_flow_dump(const char* gguf, int max_tokens, const int32_t* prompt_tokens, int n_prompt,
                     const int32_t* tokens, int n_tokens, const float* prompt_feat, int mel_len1,
                     const float* spk_embedding, int spk_len, const float* noise_z, int mel_t,
                     dropin_flow_out* out) {
  larynx::flow::FlowDecoder dec;
  if (!dec.load(gguf, max_tokens)) return 1;
  std::vector<int32_t> pt(prompt_tokens, prompt_tokens + n_prompt), tk(tokens, tokens + n_tokens);
  std::vector<float> pf(prompt_feat, prompt_feat + (size_t)mel_len1 * 80);
  std::vector<float> spk(spk_embedding, spk_embedding + spk_len);
  std::vector<float> z(noise_z, noise_z + (size_t)mel_t * 80);
  std::vector<float> mel;
  larynx::flow::FlowDebug dbg;
  if (!dec.infer(pt, tk, pf, spk, z, mel, &dbg)) return 1;
  put(out->spk, dbg.spk);
  put(out->token_embed, dbg.token_embed);
  put(out->prelookahead, dbg.prelookahead);
  put(out->mu, dbg.mu);
  put(out->cond, dbg.cond);
  put(out->time_embed, dbg.time_embed);
  put(out->input_proj, dbg.input_proj);
  put(out->conv_pos, dbg.conv_pos);
  put(out->input_embed, dbg.input_embed);
  put(out->norm_out, dbg.norm_out);
  put(out->dphi, dbg.dphi);
  if (out->blocks)
    for (size_t i = 0; i < dbg.blocks.size(); ++i)
      std::memcpy(out->blocks + i * dbg.blocks[i].size(), dbg.blocks[i].data(),
                  dbg.blocks[i].size() * sizeof(float));
  put(out->feat, mel);
  return 0;
}

typedef struct dropin_llm_out {
  float* lm_input;        // (L, hidden)
  float* hidden;          // (n_layers, L, hidden)
  float* final_norm;      // (L, hidden)
  float* logits;          // (L, speech_vocab)
  float* dec_logits;      // (n_dec, speech_vocab)
  float* dec_final_norm;  // (n_dec, hidden)
  float* cache_k;         // (n_layers, L + n_dec, kv)
  float* cache_v;
  int L;
  int cache_len;
} dropin_llm_out;

// tests/llm_dump.cpp:59-100 (LLM::load, prefill with LLMDebug), extended by
// build_lm_input in front and n_dec decode steps plus the cache read-back after.
int dropin_llm_dump(const char* gguf, int max_ctx, const int* text, int n_text, const int* speech,
                    int n_speech, const int* dec_tokens, int n_dec, dropin_llm_out* out) {
  larynx::llm::LLM llm;
  if (!llm.load(gguf, max_ctx)) return 1;
  std::vector<int> tt(text, text + n_text), sp(speech, speech + n_speech);
  std::vector<float> lm_input;
  int L = 0;
  if (!llm.build_lm_input(tt, sp, lm_input, &L)) return 1;
  larynx::llm::LLMDebug dbg;
  if (!llm.prefill(lm_input, L, &dbg)) return 1;
  out->L = L;
  put(out->lm_input, lm_input);
  if (out->hidden)
    for (size_t i = 0; i < dbg.hidden_states.size(); ++i)
      std::memcpy(out->hidden + i * dbg.hidden_states[i].size(), dbg.hidden_states[i].data(),
                  dbg.hidden_states[i].size() * sizeof(float));
  put(out->final_norm, dbg.final_norm);
  put(out->logits, dbg.logits);
  const int V = llm.speech_vocab(), H = llm.hidden();
  for (int i = 0; i < n_dec; ++i) {
    std::vector<float> lg, fn;
    if (!llm.decode(dec_tokens[i], lg, &fn)) return 1;
    if (out->dec_logits) std::memcpy(out->dec_logits + (size_t)i * V, lg.data(), V * sizeof(float));
    if (out->dec_final_norm)
      std::memcpy(out->dec_final_norm + (size_t)i * H, fn.data(), H * sizeof(float));
  }
  out->cache_len = llm.cache_len();
  const size_t per = (size_t)out->cache_len * llm.kv_width();
  for (int l = 0; l < llm.n_layers(); ++l) {
    const std::vector<float>& k = llm.cache_key(l);
    const std::vector<float>& v = llm.cache_value(l);
    if (k.size() != per || v.size() != per) return 1;
    if (out->cache_k) std::memcpy(out->cache_k + l * per, k.data(), per * sizeof(float));
    if (out->cache_v) std::memcpy(out->cache_v + l * per, v.data(), per * sizeof(float));
  }
  return 0;
}

}  // extern "C"
