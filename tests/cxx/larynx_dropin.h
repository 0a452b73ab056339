// The reference's public C++ interfaces for the Flow decoder and the Qwen2 LM,
// re-implemented over liblxops (include/lx_ops.h) as a maintainer would bind
// them: the class and struct shapes of include/larynx/flow/flow.h:15-82 and
// include/larynx/llm/llm.h:16-104 (host std::vector inputs and outputs, bool
// returns with the message on stderr), with the ggml backend replaced by the
// lx_flow / lx_qwen2 objects.  Built into tests/cxx/libdropin.so and driven by
// tests/test_gpu_dropin_cxx.py.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace larynx::flow {

// Per-stage captures (include/larynx/flow/flow.h:15-34), PyTorch layouts.
struct FlowDebug {
  std::vector<float> spk;           // (1, 80)
  std::vector<float> token_embed;   // (1, Tseq, 80)
  std::vector<float> prelookahead;  // (1, Tseq, 80)
  std::vector<float> mu;            // (1, 80, MEL_T)
  std::vector<float> cond;          // (1, 80, MEL_T)
  std::vector<float> time_embed;    // (2, 1024)          DiT at CFM step 1
  std::vector<float> input_proj;    // (2, MEL_T, 1024)
  std::vector<float> conv_pos;      // (2, MEL_T, 1024)
  std::vector<float> input_embed;   // (2, MEL_T, 1024)
  std::vector<std::vector<float>> blocks;  // depth x (2, MEL_T, 1024)
  std::vector<float> norm_out;      // (2, MEL_T, 1024)
  std::vector<float> dphi;          // (2, 80, MEL_T)
  std::vector<float> feat;          // (1, 80, MEL_T - mel_len1)
};

class FlowDecoder {
 public:
  FlowDecoder();
  ~FlowDecoder();
  FlowDecoder(const FlowDecoder&) = delete;
  FlowDecoder& operator=(const FlowDecoder&) = delete;

  // flow.gguf -> device (src/flow/flow.cpp:49-61).  max_tokens bounds
  // prompt + tokens per call (the reference sizes its noise bank for 7500).
  bool load(const std::string& gguf_path, int max_tokens = 7500);

  // token -> mel (src/flow/flow.cpp:111-290), 7-argument form with explicit
  // noise_z (1, 80, MEL_T).
  bool infer(const std::vector<int32_t>& prompt_tokens, const std::vector<int32_t>& tokens,
             const std::vector<float>& prompt_feat, const std::vector<float>& spk_embedding,
             const std::vector<float>& noise_z, std::vector<float>& mel, FlowDebug* debug);

 private:
  struct Impl;
  Impl* impl_;
};

}  // namespace larynx::flow

namespace larynx::llm {

// include/larynx/llm/llm.h:16-27
struct LLMDebug {
  std::vector<std::vector<float>> hidden_states;  // n_layers x (L * hidden)
  std::vector<float> final_norm;                  // L * hidden
  std::vector<float> logits;                      // L * speech_vocab
};

class LLM {
 public:
  LLM();
  ~LLM();
  LLM(const LLM&) = delete;
  LLM& operator=(const LLM&) = delete;

  bool load(const std::string& path, int max_ctx = 4096);
  bool prefill(const std::vector<float>& lm_input, int L, LLMDebug* debug = nullptr);
  bool build_lm_input(const std::vector<int>& text_tokens,
                      const std::vector<int>& prompt_speech_token, std::vector<float>& lm_input,
                      int* L_out = nullptr);
  bool decode(int token, std::vector<float>& logits, std::vector<float>* final_norm = nullptr);
  int cache_len() const;
  // ROPED keys / raw values of `layer`, GGML layout [HEAD_DIM, KV_HEADS, cache_len]
  const std::vector<float>& cache_key(int layer) const;
  const std::vector<float>& cache_value(int layer) const;
  void release();

  int hidden() const;
  int speech_vocab() const;
  int n_layers() const;
  int kv_width() const;

 private:
  struct Impl;
  Impl* impl_;
};

}  // namespace larynx::llm
