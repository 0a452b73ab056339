// GGUF v3 weight files (the reference's on-disk format, docs/WEIGHT_FORMAT.md
// §1-3, read by ggml's gguf_init_from_file + upload_gguf_weights,
// include/larynx/backend.h:48-87) and the model loaders over them
// (FlowDecoder::load / LLM::load, src/flow/gguf.cpp:24-135,
// src/llm/gguf.cpp:30-100).
//
// The reader validates every length, count and offset against the file size
// before using it (the file is untrusted input), then streams the whole data
// blob into one device allocation through two pinned staging buffers, so the
// disk read of one chunk overlaps the host-to-device copy of the previous one.
// Tensor names are the PyTorch state_dict keys; `ne` is the torch shape
// reversed (fastest dimension first).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "lx_common.hpp"
#include "lx_internal.hpp"

using namespace lx;

namespace {

constexpr uint64_t kMaxString = 1u << 20;  // longest key / name / string value accepted
constexpr int64_t kMaxCount = 1 << 24;     // tensors, KV entries, array elements
constexpr size_t kChunk = 64u << 20;       // staging chunk for the device upload

enum GgufType {
  T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
  T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

int scalar_size(int t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
  }
  return 0;
}

// Element size of the plain (non-block-quantised) ggml tensor types.
int ggml_type_size(int t) {
  switch (t) {
    case 0: return 4;   // F32
    case 1: return 2;   // F16
    case 24: return 1;  // I8
    case 25: return 2;  // I16
    case 26: return 4;  // I32
    case 27: return 8;  // I64
    case 28: return 8;  // F64
    case 30: return 2;  // BF16
  }
  return 0;
}

struct Reader {
  FILE* f = nullptr;
  uint64_t pos = 0, size = 0;
  bool ok = true;
  bool read(void* dst, uint64_t n) {
    if (!ok || n > size - pos || (n && std::fread(dst, 1, n, f) != n)) return ok = false;
    pos += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (!ok || n > size - pos || std::fseek(f, (long)(pos + n), SEEK_SET) != 0) return ok = false;
    pos += n;
    return true;
  }
  template <typename T>
  bool get(T* v) { return read(v, sizeof(T)); }
  bool str(std::string* s) {
    uint64_t n = 0;
    if (!get(&n) || n > kMaxString || n > size - pos) return ok = false;
    s->resize(n);
    return read(&(*s)[0], n);
  }
};

}  // namespace

struct lx_gguf {
  struct Tensor {
    std::string name;
    int type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
  };
  uint32_t version = 0;
  uint64_t alignment = 32, data_offset = 0, blob = 0;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int> index;
  std::unordered_map<std::string, std::string> strings;  // string-valued metadata
  void* dev = nullptr;
  ~lx_gguf() {
    if (dev) (void)hipFree(dev);
  }
};

namespace {

int fail(const char* path, const char* what) {
  set_error("gguf: %s: %s", path, what);
  return LX_ERR_ARG;
}

int parse(const char* path, Reader& r, lx_gguf* g) {
  char magic[4];
  if (!r.read(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail(path, "not a GGUF file");
  if (!r.get(&g->version) || g->version != 3)
    return fail(path, "unsupported GGUF version (3 is read)");
  int64_t n_tensors = 0, n_kv = 0;
  if (!r.get(&n_tensors) || !r.get(&n_kv) || n_tensors < 0 || n_tensors > kMaxCount || n_kv < 0 ||
      n_kv > kMaxCount)
    return fail(path, "bad tensor / metadata counts");
  for (int64_t i = 0; i < n_kv; ++i) {
    std::string key;
    int32_t type = 0;
    if (!r.str(&key) || !r.get(&type)) return fail(path, "truncated metadata");
    if (type == T_STRING) {
      std::string v;
      if (!r.str(&v)) return fail(path, "truncated metadata string");
      g->strings[key] = v;
    } else if (type == T_ARRAY) {
      int32_t et = 0;
      uint64_t count = 0;
      if (!r.get(&et) || !r.get(&count) || count > (uint64_t)kMaxCount)
        return fail(path, "bad metadata array");
      if (et == T_STRING) {
        for (uint64_t j = 0; j < count; ++j) {
          std::string v;
          if (!r.str(&v)) return fail(path, "truncated metadata array");
        }
      } else {
        const int sz = scalar_size(et);
        if (!sz || !r.skip(count * (uint64_t)sz)) return fail(path, "bad metadata array");
      }
    } else if (key == "general.alignment" && type == T_U32) {
      uint32_t a = 0;
      if (!r.get(&a) || a == 0 || (a & (a - 1)) != 0) return fail(path, "bad general.alignment");
      g->alignment = a;
    } else {
      const int sz = scalar_size(type);
      if (!sz || !r.skip((uint64_t)sz)) return fail(path, "bad metadata value");
    }
  }
  g->tensors.resize((size_t)n_tensors);
  for (int64_t i = 0; i < n_tensors; ++i) {
    lx_gguf::Tensor& t = g->tensors[(size_t)i];
    uint32_t nd = 0;
    if (!r.str(&t.name) || !r.get(&nd) || nd < 1 || nd > 4) return fail(path, "bad tensor info");
    uint64_t nel = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      int64_t v = 0;
      if (!r.get(&v) || v < 1 || (uint64_t)v > (1ull << 40) / nel)
        return fail(path, "bad tensor dimensions");
      t.ne[d] = v;
      nel *= (uint64_t)v;
    }
    t.n_dims = (int)nd;
    int32_t type = 0;
    if (!r.get(&type) || !r.get(&t.offset)) return fail(path, "truncated tensor info");
    t.type = type;
    const int es = ggml_type_size(type);
    if (!es) {
      set_error("gguf: %s: tensor '%s' has ggml type %d (only unquantised types are read)", path,
                t.name.c_str(), type);
      return LX_ERR_ARG;
    }
    t.nbytes = nel * (uint64_t)es;
    if (!g->index.emplace(t.name, (int)i).second) {
      set_error("gguf: %s: duplicate tensor '%s'", path, t.name.c_str());
      return LX_ERR_ARG;
    }
  }
  if (!r.ok) return fail(path, "truncated header");
  g->data_offset = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
  if (g->data_offset > r.size) return fail(path, "truncated before the data section");
  g->blob = r.size - g->data_offset;
  for (const lx_gguf::Tensor& t : g->tensors) {
    if (t.offset % g->alignment != 0 || t.offset > g->blob || t.nbytes > g->blob - t.offset) {
      set_error("gguf: %s: tensor '%s' lies outside the data section", path, t.name.c_str());
      return LX_ERR_ARG;
    }
  }
  return LX_OK;
}

int upload(const char* path, Reader& r, lx_gguf* g) {
  if (g->blob == 0) return LX_OK;
  if (hipMalloc(&g->dev, g->blob) != hipSuccess) {
    g->dev = nullptr;
    set_error("gguf: %s: cannot allocate %llu bytes of device memory", path,
              (unsigned long long)g->blob);
    return LX_ERR_ALLOC;
  }
  void* host[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  hipStream_t s = nullptr;
  int rc = LX_OK;
  if (hipHostMalloc(&host[0], kChunk, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc(&host[1], kChunk, hipHostMallocDefault) != hipSuccess ||
      hipEventCreateWithFlags(&ev[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) != hipSuccess ||
      hipStreamCreate(&s) != hipSuccess) {
    set_error("gguf: %s: cannot set up the staging buffers", path);
    rc = LX_ERR_ALLOC;
  }
  if (rc == LX_OK && std::fseek(r.f, (long)g->data_offset, SEEK_SET) != 0) rc = fail(path, "seek");
  r.pos = g->data_offset;
  for (uint64_t off = 0, i = 0; rc == LX_OK && off < g->blob; off += kChunk, ++i) {
    const int b = (int)(i & 1);
    const size_t n = (size_t)std::min<uint64_t>(kChunk, g->blob - off);
    if (i >= 2 && hipEventSynchronize(ev[b]) != hipSuccess) {
      rc = fail(path, "staging copy failed");
      break;
    }
    if (!r.read(host[b], n)) {
      rc = fail(path, "short read in the data section");
      break;
    }
    if (hipMemcpyAsync(static_cast<char*>(g->dev) + off, host[b], n, hipMemcpyHostToDevice, s) !=
            hipSuccess ||
        hipEventRecord(ev[b], s) != hipSuccess) {
      set_error("gguf: %s: host-to-device copy failed", path);
      rc = LX_ERR_LAUNCH;
    }
  }
  if (s && hipStreamSynchronize(s) != hipSuccess && rc == LX_OK) {
    set_error("gguf: %s: host-to-device copy failed", path);
    rc = LX_ERR_LAUNCH;
  }
  for (int b = 0; b < 2; ++b) {
    if (ev[b]) (void)hipEventDestroy(ev[b]);
    if (host[b]) (void)hipHostFree(host[b]);
  }
  if (s) (void)hipStreamDestroy(s);
  return rc;
}

}  // namespace

extern "C" int lx_gguf_open(const char* path, int flags, lx_gguf** out) {
  LX_REQUIRE(path && out, "gguf_open: null argument");
  *out = nullptr;
  Reader r;
  r.f = std::fopen(path, "rb");
  if (!r.f) {
    set_error("gguf: cannot open '%s'", path);
    return LX_ERR_ARG;
  }
  int rc = LX_OK;
  if (std::fseek(r.f, 0, SEEK_END) != 0) rc = fail(path, "seek");
  if (rc == LX_OK) {
    const long sz = std::ftell(r.f);
    if (sz < 0 || std::fseek(r.f, 0, SEEK_SET) != 0) rc = fail(path, "seek");
    r.size = (uint64_t)(sz < 0 ? 0 : sz);
  }
  lx_gguf* g = rc == LX_OK ? new (std::nothrow) lx_gguf() : nullptr;
  if (rc == LX_OK && !g) rc = LX_ERR_ALLOC;
  if (rc == LX_OK) rc = parse(path, r, g);
  if (rc == LX_OK && !(flags & LX_GGUF_HOST_ONLY)) rc = upload(path, r, g);
  std::fclose(r.f);
  if (rc != LX_OK) {
    delete g;
    return rc;
  }
  *out = g;
  return LX_OK;
}

extern "C" void lx_gguf_close(lx_gguf* g) { delete g; }

extern "C" int lx_gguf_n_tensors(const lx_gguf* g) { return g ? (int)g->tensors.size() : 0; }

extern "C" int lx_gguf_find(const lx_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->index.find(name);
  return it == g->index.end() ? -1 : it->second;
}

extern "C" int lx_gguf_tensor_info(const lx_gguf* g, int i, const char** name, int* type,
                                   int* n_dims, int64_t* ne, uint64_t* nbytes) {
  LX_REQUIRE(g && i >= 0 && i < (int)g->tensors.size(), "gguf_tensor_info: bad index %d", i);
  const lx_gguf::Tensor& t = g->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (type) *type = t.type;
  if (n_dims) *n_dims = t.n_dims;
  if (ne)
    for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
  if (nbytes) *nbytes = t.nbytes;
  return LX_OK;
}

extern "C" const void* lx_gguf_tensor_data(const lx_gguf* g, int i) {
  if (!g || !g->dev || i < 0 || i >= (int)g->tensors.size()) return nullptr;
  return static_cast<const char*>(g->dev) + g->tensors[(size_t)i].offset;
}

extern "C" const char* lx_gguf_get_string(const lx_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->strings.find(key);
  return it == g->strings.end() ? nullptr : it->second.c_str();
}

// ---- model loaders -------------------------------------------------------------

namespace {

// Device pointer of an F32 tensor whose torch shape is `shape` (ne reversed).
struct Resolver {
  const lx_gguf* g;
  const char* path;
  int rc = LX_OK;
  const float* get(const std::string& name, std::initializer_list<int64_t> shape) {
    if (rc != LX_OK) return nullptr;
    const int i = lx_gguf_find(g, name.c_str());
    if (i < 0) {
      set_error("gguf: %s: missing tensor '%s'", path, name.c_str());
      rc = LX_ERR_ARG;
      return nullptr;
    }
    const lx_gguf::Tensor& t = g->tensors[(size_t)i];
    bool ok = t.type == 0 && t.n_dims == (int)shape.size();
    int d = (int)shape.size() - 1;
    for (int64_t s : shape) ok = ok && t.ne[d--] == s;
    if (!ok) {
      set_error("gguf: %s: tensor '%s' is not F32 of the expected shape", path, name.c_str());
      rc = LX_ERR_ARG;
      return nullptr;
    }
    return static_cast<const float*>(lx_gguf_tensor_data(g, i));
  }
  int64_t dim(const std::string& name, int d) {  // ne[d] of a tensor, 0 if absent
    const int i = lx_gguf_find(g, name.c_str());
    return i < 0 ? 0 : g->tensors[(size_t)i].ne[d];
  }
  bool has(const std::string& name) { return lx_gguf_find(g, name.c_str()) >= 0; }
};

}  // namespace

extern "C" int lx_flow_load(const char* path, int max_tokens, lx_flow** out) {
  LX_REQUIRE(path && out, "flow_load: null argument");
  *out = nullptr;
  lx_gguf* g = nullptr;
  LX_TRY(lx_gguf_open(path, 0, &g));
  Resolver R{g, path};
  // Geometry from the tensors (src/flow/internal.h:18-35 fixes it for CosyVoice3).
  const std::string E = "decoder.estimator.";
  const int64_t mel = R.dim("input_embedding.weight", 0);
  const int64_t vocab = R.dim("input_embedding.weight", 1);
  const int64_t spk_in = R.dim("spk_embed_affine_layer.weight", 0);
  const int64_t ch = R.dim("pre_lookahead_layer.conv1.weight", 2);
  const int64_t D = R.dim(E + "input_embed.proj.weight", 1);
  const int64_t F = R.dim(E + "transformer_blocks.0.ff.ff.0.0.weight", 1);
  const int64_t freq = R.dim(E + "time_embed.time_mlp.0.weight", 0);
  int depth = 0;
  while (R.has(E + "transformer_blocks." + std::to_string(depth) + ".attn_norm.linear.weight"))
    ++depth;
  if (!mel || !vocab || !spk_in || !ch || !D || !F || !depth || freq != 256 || D % 64 != 0) {
    const char* arch = lx_gguf_get_string(g, "general.architecture");
    set_error("gguf: %s: not a CosyVoice3 flow checkpoint (general.architecture '%s')", path,
              arch ? arch : "");
    lx_gguf_close(g);
    return LX_ERR_ARG;
  }
  lx_flow_frontend_weights fw{};
  fw.vocab = (int)vocab;
  fw.spk_in = (int)spk_in;
  fw.channels = (int)ch;
  fw.input_embedding = R.get("input_embedding.weight", {vocab, mel});
  fw.spk_affine_w = R.get("spk_embed_affine_layer.weight", {mel, spk_in});
  fw.spk_affine_b = R.get("spk_embed_affine_layer.bias", {mel});
  fw.pre_conv1_w = R.get("pre_lookahead_layer.conv1.weight", {ch, mel, 4});
  fw.pre_conv1_b = R.get("pre_lookahead_layer.conv1.bias", {ch});
  fw.pre_conv2_w = R.get("pre_lookahead_layer.conv2.weight", {mel, ch, 3});
  fw.pre_conv2_b = R.get("pre_lookahead_layer.conv2.bias", {mel});
  lx_dit_weights dw{};
  dw.dim = (int)D;
  dw.depth = depth;
  dw.heads = (int)(D / 64);
  dw.head_dim = 64;
  dw.ff_inner = (int)F;
  dw.mel_dim = (int)mel;
  const int64_t cg = D / 16;
  dw.time_mlp_0_w = R.get(E + "time_embed.time_mlp.0.weight", {D, 256});
  dw.time_mlp_0_b = R.get(E + "time_embed.time_mlp.0.bias", {D});
  dw.time_mlp_2_w = R.get(E + "time_embed.time_mlp.2.weight", {D, D});
  dw.time_mlp_2_b = R.get(E + "time_embed.time_mlp.2.bias", {D});
  dw.input_proj_w = R.get(E + "input_embed.proj.weight", {D, 4 * mel});
  dw.input_proj_b = R.get(E + "input_embed.proj.bias", {D});
  dw.conv_pos_1_w = R.get(E + "input_embed.conv_pos_embed.conv1.0.weight", {D, cg, 31});
  dw.conv_pos_1_b = R.get(E + "input_embed.conv_pos_embed.conv1.0.bias", {D});
  dw.conv_pos_2_w = R.get(E + "input_embed.conv_pos_embed.conv2.0.weight", {D, cg, 31});
  dw.conv_pos_2_b = R.get(E + "input_embed.conv_pos_embed.conv2.0.bias", {D});
  dw.norm_out_w = R.get(E + "norm_out.linear.weight", {2 * D, D});
  dw.norm_out_b = R.get(E + "norm_out.linear.bias", {2 * D});
  dw.proj_out_w = R.get(E + "proj_out.weight", {mel, D});
  dw.proj_out_b = R.get(E + "proj_out.bias", {mel});
  std::vector<lx_dit_block_weights> blocks((size_t)depth);
  for (int i = 0; i < depth; ++i) {
    const std::string p = E + "transformer_blocks." + std::to_string(i) + ".";
    lx_dit_block_weights& b = blocks[(size_t)i];
    b.attn_norm_w = R.get(p + "attn_norm.linear.weight", {6 * D, D});
    b.attn_norm_b = R.get(p + "attn_norm.linear.bias", {6 * D});
    b.to_q_w = R.get(p + "attn.to_q.weight", {D, D});
    b.to_q_b = R.get(p + "attn.to_q.bias", {D});
    b.to_k_w = R.get(p + "attn.to_k.weight", {D, D});
    b.to_k_b = R.get(p + "attn.to_k.bias", {D});
    b.to_v_w = R.get(p + "attn.to_v.weight", {D, D});
    b.to_v_b = R.get(p + "attn.to_v.bias", {D});
    b.to_out_w = R.get(p + "attn.to_out.0.weight", {D, D});
    b.to_out_b = R.get(p + "attn.to_out.0.bias", {D});
    b.ff0_w = R.get(p + "ff.ff.0.0.weight", {F, D});
    b.ff0_b = R.get(p + "ff.ff.0.0.bias", {F});
    b.ff2_w = R.get(p + "ff.ff.2.weight", {D, F});
    b.ff2_b = R.get(p + "ff.ff.2.bias", {D});
  }
  dw.blocks = blocks.data();
  int rc = R.rc;
  if (rc == LX_OK) rc = lx_flow_create(&dw, &fw, max_tokens, out);
  lx_gguf_close(g);  // the decoder holds its own (re-packed) copies
  return rc;
}

extern "C" int lx_qwen2_load(const char* path, int max_ctx, lx_qwen2** out) {
  LX_REQUIRE(path && out, "qwen2_load: null argument");
  *out = nullptr;
  lx_gguf* g = nullptr;
  LX_TRY(lx_gguf_open(path, 0, &g));
  Resolver R{g, path};
  // Names of src/llm/gguf.cpp:44-83; geometry from the tensors, eps / theta from
  // src/llm/internal.h:27-28.
  const std::string M = "llm.model.model.";
  const int64_t H = R.dim(M + "embed_tokens.weight", 0);
  const int64_t text_vocab = R.dim(M + "embed_tokens.weight", 1);
  const int64_t speech_vocab = R.dim("speech_embedding.weight", 1);
  const int64_t I = R.dim(M + "layers.0.mlp.gate_proj.weight", 1);
  const int64_t KV = R.dim(M + "layers.0.self_attn.k_proj.weight", 1);
  int n_layers = 0;
  while (R.has(M + "layers." + std::to_string(n_layers) + ".self_attn.q_proj.weight")) ++n_layers;
  if (!H || !text_vocab || !speech_vocab || !I || !KV || !n_layers || H % 64 || KV % 64) {
    lx_gguf_close(g);
    set_error("gguf: %s: not a CosyVoice3 Qwen2 checkpoint", path);
    return LX_ERR_ARG;
  }
  lx_qwen2_weights w{};
  w.hidden = (int)H;
  w.intermediate = (int)I;
  w.head_dim = 64;
  w.n_heads = (int)(H / 64);
  w.n_kv_heads = (int)(KV / 64);
  w.n_layers = n_layers;
  w.text_vocab = (int)text_vocab;
  w.speech_vocab = (int)speech_vocab;
  w.rms_eps = 1e-6f;
  w.rope_theta = 1e6f;
  w.embed_tokens = R.get(M + "embed_tokens.weight", {text_vocab, H});
  w.speech_embedding = R.get("speech_embedding.weight", {speech_vocab, H});
  w.final_norm = R.get(M + "norm.weight", {H});
  w.llm_decoder = R.get("llm_decoder.weight", {speech_vocab, H});
  std::vector<lx_qwen2_layer_weights> layers((size_t)n_layers);
  for (int i = 0; i < n_layers; ++i) {
    const std::string p = M + "layers." + std::to_string(i) + ".";
    lx_qwen2_layer_weights& l = layers[(size_t)i];
    l.q_w = R.get(p + "self_attn.q_proj.weight", {H, H});
    l.q_b = R.get(p + "self_attn.q_proj.bias", {H});
    l.k_w = R.get(p + "self_attn.k_proj.weight", {KV, H});
    l.k_b = R.get(p + "self_attn.k_proj.bias", {KV});
    l.v_w = R.get(p + "self_attn.v_proj.weight", {KV, H});
    l.v_b = R.get(p + "self_attn.v_proj.bias", {KV});
    l.o_w = R.get(p + "self_attn.o_proj.weight", {H, H});
    l.gate_w = R.get(p + "mlp.gate_proj.weight", {I, H});
    l.up_w = R.get(p + "mlp.up_proj.weight", {I, H});
    l.down_w = R.get(p + "mlp.down_proj.weight", {H, I});
    l.in_norm = R.get(p + "input_layernorm.weight", {H});
    l.post_norm = R.get(p + "post_attention_layernorm.weight", {H});
  }
  w.layers = layers.data();
  int rc = R.rc;
  if (rc == LX_OK) rc = lx_qwen2_create(&w, max_ctx, out);
  if (rc != LX_OK) {
    lx_gguf_close(g);
    return rc;
  }
  // create copied every layer; the two embedding tables it referenced in place
  // move into the model's memory too, and the file's device copy is released
  rc = qwen2_own_tables(*out);
  lx_gguf_close(g);
  if (rc != LX_OK) {
    lx_qwen2_destroy(*out);
    *out = nullptr;
  }
  return rc;
}
