// Qwen2 backbone of CosyVoice3LM, device resident.
//
// Host-side counterpart of LLM::build_lm_input / prefill / decode
// (src/llm/llm.cpp:63-327).  Differences from the reference by design:
//   - the KV cache lives on the device (the reference reads it back to host
//     vectors after prefill and re-uploads the whole cache as graph constants
//     on every decode step, src/llm/llm.cpp:200-204, 269-275);
//   - q/k/v are one fused GEMM, gate/up one GEMM with interleaved rows whose
//     epilogue applies silu(gate)*up, and o_proj / down_proj add into the
//     residual stream in their epilogues;
//   - GQA never materialises repeated K/V (the attention kernel maps query
//     head h to kv head h / 7, as HF repeat_kv's consecutive layout).
#include <hip/hip_runtime.h>

#include <cmath>
#include <new>
#include <vector>

#include "lx_common.hpp"
#include "lx_internal.hpp"

using namespace lx;

namespace {

constexpr int kSosToken = 6561;     // SOS_TOKEN (src/llm/internal.h:33)
constexpr int kTaskIdToken = 6563;  // TASK_ID_TOKEN (src/llm/internal.h:34)

struct Layer {
  float *qkv_w, *qkv_b, *o_w, *gu_w, *down_w, *in_norm, *post_norm;
  float *k_cache, *v_cache;  // (max_ctx, KV)
  // the prefill projections' weights in MFMA fragment order (wfrag_pack), for
  // the split-operand GEMM; decode streams the fp32 copies above
  void *qkv_wf = nullptr, *o_wf = nullptr, *gu_wf = nullptr, *down_wf = nullptr;
};

// K slices of a prefill projection on the fragment-order GEMM (64-row tiles):
// as many as the reduce passes take (9) while tiles x slices stay within one
// workgroup per CU, then the fewest that keep the same longest slice (slices
// of ceil(steps / slices) 64-wide steps).  L = 256: q|k|v 7 slices of 2 steps
// (252 workgroups), o_proj 7 of 2 (196), down_proj 9 of 9 (252); L = 1024:
// 1 / 2 / 2.
int prefill_bx_slices(int rows, int N, int K) {
  const int steps = K / 64;
  const long tiles = (long)((rows + 63) / 64) * (N / 128);
  int most = (int)std::min<long>(std::min(9, steps), std::max<long>(1, 256 / tiles));
  const int per = (steps + most - 1) / most;
  return (steps + per - 1) / per;
}

}  // namespace

struct lx_qwen2 {
  Arena arena;
  int H = 0, I = 0, NH = 0, NKV = 0, HD = 0, NL = 0, text_vocab = 0, speech_vocab = 0;
  int KV = 0, QKV = 0;
  float eps = 0.0f, theta = 0.0f;
  int max_ctx = 0;
  int cache_len = 0;
  const float* embed_tokens = nullptr;
  const float* speech_embedding = nullptr;
  float *final_norm, *llm_decoder;
  std::vector<Layer> layers;
  // activations, sized for max_ctx rows
  float *x, *hn, *qkv, *att, *act;
  float* ws = nullptr;  // split-K partial sums, and the gate/up split tail's partial tiles
  size_t ws_floats = 0;
  bool frag = false;    // prefill projections on the fragment-order split-operand GEMM
  int products = 3;     // its products per element pair (3 or 6)
  unsigned* arrivals = nullptr;  // split-tail arrival counters (zeroed at creation)
  int n_arrivals = 0;
  int* pos;     // pos[i] = i
  // single-token decode state (lx_decode.hip kernels)
  int* d_pos = nullptr;       // position of the token being decoded
  float* part = nullptr;      // attention split partials
  long part_stride = 0;       // floats per kv head in `part`
  int max_splits = 0;
  float* rope_tab = nullptr;  // device copy of the rotary inverse frequencies
  bool use_graph = true;      // replay the layer stack as one HIP graph
  hipStream_t cap_stream = nullptr;
  // [0]: the cache fits one attention split; [1 + c]: split class c
  hipGraphExec_t graph[1 + kDecAttnClasses] = {};
  ~lx_qwen2() {
    for (hipGraphExec_t g : graph)
      if (g) (void)hipGraphExecDestroy(g);
    if (cap_stream) (void)hipStreamDestroy(cap_stream);
  }
};

int lx::qwen2_own_tables(lx_qwen2* m) {
  const size_t nt = (size_t)m->text_vocab * m->H, ns = (size_t)m->speech_vocab * m->H;
  float* et = m->arena.alloc<float>(nt);
  float* se = m->arena.alloc<float>(ns);
  if (!et || !se) {
    set_error("qwen2_load: device allocation failed for the embedding tables");
    return LX_ERR_ALLOC;
  }
  if (hipMemcpy(et, m->embed_tokens, nt * sizeof(float), hipMemcpyDeviceToDevice) != hipSuccess ||
      hipMemcpy(se, m->speech_embedding, ns * sizeof(float), hipMemcpyDeviceToDevice) !=
          hipSuccess) {
    set_error("qwen2_load: embedding table copy failed");
    return LX_ERR_LAUNCH;
  }
  m->embed_tokens = et;
  m->speech_embedding = se;
  return LX_OK;
}

namespace {

// Width of the split-K partial workspace: the largest splits * rows * N over
// the three split projections, and the gate/up launch's split-tail partials,
// at every prefill length up to max_ctx; *tails = the most tail tiles.
size_t splitk_ws_floats(int max_ctx, int H, int QKV, int I, int* tails) {
  size_t best = 0;
  *tails = 0;
  // splits depend on M only through the tile count, so the largest M of each
  // 64-row band (and max_ctx itself) bounds every length
  for (int M = 64;; M += 64) {
    const int rows = M < max_ctx ? M : max_ctx;
    const int shapes[3][2] = {{QKV, H}, {H, H}, {H, I}};
    for (const auto& sh : shapes) {
      int ks = 0;
      const int splits = gemm_splitk_plan(rows, sh[0], sh[1], &ks);
      const int bx = prefill_bx_slices(rows, sh[0], sh[1]);
      const size_t n = (size_t)std::max(splits, bx) * rows * sh[0];
      if (n > best) best = n;
    }
    int t = 0;
    const size_t nt = split_tail_ws_floats(rows, 2 * I, H, &t);
    if (nt > best) best = nt;
    if (t > *tails) *tails = t;
    if (M >= max_ctx) break;
  }
  return best;
}

// q|k|v, o_proj or down_proj as K-slice partial products into m->ws; returns the
// slice count through *splits.
int prefill_partials(lx_qwen2* m, const float* x, int ldx, const void* wf, const float* w,
                     int rows, int N, int K, int* splits, hipStream_t s, bool x_packed = false) {
  if (m->frag) {
    const int sl = prefill_bx_slices(rows, N, K);
    lx_linear_bx g{};
    g.A = x;
    g.lda = ldx;
    g.Wf = wf;
    g.out = LX_BX_OUT_PARTIAL;
    g.Y = m->ws;
    g.ldy = N;
    g.slice_stride = (long)rows * N;
    g.M = rows;
    g.N = N;
    g.K = K;
    g.bm = 64;
    g.slices = sl;
    g.products = m->products;
    g.a_packed = x_packed ? 1 : 0;
    *splits = sl;
    return linear_bx(g, s);
  }
  int ks = 0;
  *splits = gemm_splitk_plan(rows, N, K, &ks);
  return gemm_splitk_partials(x, ldx, w, K, m->ws, rows, N, K, *splits, ks, s);
}

// Prefill layer (src/llm/llm.cpp:141-173) over L rows at positions m->pos[0..L).
// On entry m->hn holds input_layernorm(x); on exit x is the layer output and
// m->hn holds next_norm(x) (the next layer's input_layernorm or the final norm).
//   q/k/v: K-slice partials, then bias + NEOX rotary + cache append in one pass;
//   attention (causal, GQA) reads q and the cache;
//   o_proj: K-slice partials, then residual + post_attention_layernorm;
//   gate/up with the SwiGLU epilogue;
//   down_proj: K-slice partials, then residual + next_norm.
// Every projection runs on the fragment-order split-operand GEMM when the
// geometry allows (m->frag: N multiples of 128, K of 64), else on the fp32 GEMMs.
// With three products on the fragment-order GEMM, the GEMM inputs written by
// this layer's kernels (attention's output, the RMSNorm outputs) are two-part
// packed rows (bit-identical products, no split per column tile); hn_packed:
// m->hn arrives packed (written by the previous layer), pack_next: write the
// next norm packed (not the final norm, which the fp32 logits GEMM reads).
int prefill_layer(lx_qwen2* m, Layer& L, int rows, const float* next_norm, hipStream_t s,
                  bool hn_packed, bool pack_next) {
  const int H = m->H, KV = m->KV, QKV = m->QKV;
  const bool pk = m->frag && m->products == 3;
  int sp = 0;
  LX_TRY(prefill_partials(m, m->hn, H, L.qkv_wf, L.qkv_w, rows, QKV, H, &sp, s, pk && hn_packed));
  LX_TRY(splitk_qkv_rope_cache(m->ws, sp, rows, L.qkv_b, m->NH, m->NKV, m->pos, m->rope_tab,
                               m->qkv, QKV, L.k_cache, L.v_cache, 0, s));
  const float scale = 1.0f / std::sqrt((float)m->HD);
  LX_TRY(attention(m->qkv, QKV, L.k_cache, KV, L.v_cache, KV, m->att, H, 1, rows, rows, m->NH,
                   m->NKV, m->HD, scale, /*causal*/ 1, /*q_offset*/ 0, /*products*/ 6,
                   /*out_packed*/ pk ? 1 : 0, s));
  LX_TRY(prefill_partials(m, m->att, H, L.o_wf, L.o_w, rows, H, H, &sp, s, pk));
  LX_TRY(splitk_resid_rmsnorm(m->ws, sp, rows, H, nullptr, m->x, L.post_norm, m->eps, m->hn, s,
                              pk));
  lx_epilogue swiglu{};
  swiglu.kind = LX_EPI_SWIGLU_PAIRED;
  if (m->frag) {
    // gate/up + SwiGLU: 64-row tiles with the split tail where it applies (L =
    // 256: 304 tiles, 256 whole and 48 in five k ranges; 24.3 vs 25.3 us on
    // 128-row tiles with cold weights), else 128-row tiles while they fit one
    // round over the CUs, else 64-row tiles (L = 1024: 95 vs 116 us)
    const bool split = bx_split_parts(rows, 2 * m->I, H, 64) > 0;
    lx_linear_bx g{};
    if (split) {
      g.split_tail = 1;
      g.ws = m->ws;
      g.ws_floats = m->ws_floats;
      g.counters = m->arrivals;
      g.n_counters = m->n_arrivals;
    }
    g.A = m->hn;
    g.a_packed = pk ? 1 : 0;
    g.lda = H;
    g.Wf = L.gu_wf;
    g.epi = &swiglu;
    g.out = LX_BX_OUT_F32;
    g.Y = m->act;
    g.ldy = m->I;
    g.M = rows;
    g.N = 2 * m->I;
    g.K = H;
    g.bm = split ? 64 : (long)((rows + 127) / 128) * (2 * m->I / 128) <= 256 ? 128 : 64;
    g.slices = 1;
    g.products = m->products;
    LX_TRY(linear_bx(g, s));
  } else {
    LX_TRY(linear_split_tail(m->hn, H, L.gu_w, nullptr, m->act, m->I, rows, 2 * m->I, H,
                             &swiglu, m->ws, m->ws_floats, m->arrivals, m->n_arrivals, s));
  }
  LX_TRY(prefill_partials(m, m->act, m->I, L.down_wf, L.down_w, rows, H, m->I, &sp, s));
  return splitk_resid_rmsnorm(m->ws, sp, rows, H, nullptr, m->x, next_norm, m->eps, m->hn, s,
                              pk && pack_next);
}

// One decode layer (src/llm/llm.cpp:254-289): RMSNorm + QKV + rotary + cache
// append; attention; o_proj + residual; RMSNorm + gate/up + SwiGLU;
// down_proj + residual.  While the cache fits one split (cls 0) the attention
// is one launch writing its output and o_proj a launch of its own; past it
// (cls = 1 + split class) the split partials are merged inside the o_proj
// launch: five launches per layer either way.  The position is read from
// m->d_pos.
int decode_layer(lx_qwen2* m, Layer& L, int cls, hipStream_t s) {
  const int H = m->H, KV = m->KV;
  DecGemvArgs q;
  q.x = m->x;
  q.norm_w = L.in_norm;
  q.eps = m->eps;
  q.W = L.qkv_w;
  q.bias = L.qkv_b;
  q.y = m->hn;  // roped q row
  q.N = m->QKV;
  q.K = H;
  q.pos = m->d_pos;
  q.q_cols = H;
  q.kv_cols = KV;
  q.rope_heads = m->NH + m->NKV;
  q.k_cache = L.k_cache;
  q.v_cache = L.v_cache;
  q.inv_freq = m->rope_tab;
  LX_TRY(dec_gemv(DEC_QKV_ROPE, q, s));
  DecAttnArgs at;
  at.q = m->hn;
  at.k_cache = L.k_cache;
  at.v_cache = L.v_cache;
  at.ld = KV;
  at.pos = m->d_pos;
  at.scale = 1.0f / std::sqrt((float)m->HD);
  at.rep = m->NH / m->NKV;
  at.n_heads = m->NH;
  at.max_rows = m->max_ctx;
  at.part = m->part;
  at.part_group_stride = m->part_stride;
  at.out = m->att;
  DecGemvArgs o;
  o.x = m->att;
  o.W = L.o_w;
  o.y = m->x;
  o.N = H;
  o.K = H;
  if (cls == 0) {
    LX_TRY(dec_attention(at, m->NKV, s));
    LX_TRY(dec_gemv(DEC_RESID, o, s));
  } else {
    LX_TRY(dec_attention_o(at, m->NKV, cls - 1, o, s));
  }
  DecGemvArgs gu;
  gu.x = m->x;
  gu.norm_w = L.post_norm;
  gu.eps = m->eps;
  gu.W = L.gu_w;
  gu.y = m->act;
  gu.N = 2L * m->I;
  gu.K = H;
  LX_TRY(dec_gemv(DEC_SWIGLU, gu, s));
  DecGemvArgs d;
  d.x = m->act;
  d.W = L.down_w;
  d.y = m->x;
  d.N = H;
  d.K = m->I;
  return dec_gemv(DEC_RESID, d, s);
}

int decode_stack(lx_qwen2* m, int cls, hipStream_t s) {
  for (auto& L : m->layers) LX_TRY(decode_layer(m, L, cls, s));
  return LX_OK;
}

// Launch class of the token decoded at position `pos`: 0 while keys [0, pos]
// fit one attention split, else 1 + the split class of their split count.
int decode_class(int pos) {
  const int n_split = (pos + 1 + dec_attention_split_keys() - 1) / dec_attention_split_keys();
  return n_split == 1 ? 0 : 1 + dec_attention_class(n_split);
}

// Captures the decode layer stack into a HIP graph on the library's own
// stream (capture needs a stream other than the legacy default stream); one
// graph per launch class (decode_class).
int capture_decode(lx_qwen2* m, int cls) {
  if (!m->cap_stream &&
      hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking) != hipSuccess) {
    set_error("qwen2_decode: stream creation failed");
    return LX_ERR_LAUNCH;
  }
  if (hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
    set_error("qwen2_decode: hipStreamBeginCapture failed");
    return LX_ERR_LAUNCH;
  }
  int rc = decode_stack(m, cls, m->cap_stream);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(m->cap_stream, &g);
  if (rc == LX_OK && (e != hipSuccess || !g)) {
    set_error("qwen2_decode: hipStreamEndCapture failed");
    rc = LX_ERR_LAUNCH;
  }
  hipGraphExec_t& exec = m->graph[cls];
  if (rc == LX_OK && hipGraphInstantiate(&exec, g, nullptr, nullptr, 0) != hipSuccess) {
    set_error("qwen2_decode: hipGraphInstantiate failed");
    exec = nullptr;
    rc = LX_ERR_LAUNCH;
  }
  if (g) (void)hipGraphDestroy(g);
  return rc;
}

}  // namespace

extern "C" int lx_qwen2_create(const lx_qwen2_weights* w, int max_ctx, lx_qwen2** out) {
  LX_REQUIRE(w && out, "qwen2_create: null argument");
  *out = nullptr;
  LX_REQUIRE(w->hidden > 0 && w->hidden % 4 == 0 && w->head_dim == 64 && w->n_heads > 0 &&
                 w->n_kv_heads > 0 && w->n_heads % w->n_kv_heads == 0 &&
                 w->n_heads * w->head_dim == w->hidden && w->intermediate > 0 &&
                 w->intermediate % 4 == 0 && w->n_layers > 0,
             "qwen2_create: unsupported geometry");
  LX_REQUIRE(max_ctx >= 1 && max_ctx <= dec_attention_max_ctx(),
             "qwen2_create: max_ctx=%d outside [1, %d]", max_ctx, dec_attention_max_ctx());
  LX_REQUIRE(dec_supported(w->hidden, w->intermediate) && w->n_heads / w->n_kv_heads <= 8,
             "qwen2_create: decode kernels need hidden <= 2048, intermediate <= 6144 and "
             "at most 8 query heads per kv head");
  // the prefill's fused q|k|v reduce pass holds one projected row per workgroup
  LX_REQUIRE(w->hidden + 2 * w->n_kv_heads * w->head_dim <= 2048,
             "qwen2_create: fused q|k|v row of %d floats exceeds 2048 (hidden %d, %d kv heads)",
             w->hidden + 2 * w->n_kv_heads * w->head_dim, w->hidden, w->n_kv_heads);
  LX_REQUIRE(w->embed_tokens && w->speech_embedding && w->final_norm && w->llm_decoder &&
                 w->layers,
             "qwen2_create: missing tables");
  LX_REQUIRE(w->speech_vocab > kTaskIdToken, "qwen2_create: speech vocab too small");
  lx_qwen2* m = new (std::nothrow) lx_qwen2();
  if (!m) return LX_ERR_ALLOC;
  m->H = w->hidden;
  m->I = w->intermediate;
  m->NH = w->n_heads;
  m->NKV = w->n_kv_heads;
  m->HD = w->head_dim;
  m->NL = w->n_layers;
  m->KV = m->NKV * m->HD;
  m->QKV = m->H + 2 * m->KV;
  m->text_vocab = w->text_vocab;
  m->speech_vocab = w->speech_vocab;
  m->eps = w->rms_eps;
  m->theta = w->rope_theta;
  m->max_ctx = max_ctx;
  m->embed_tokens = w->embed_tokens;
  m->speech_embedding = w->speech_embedding;
  const int H = m->H, I = m->I, KV = m->KV, QKV = m->QKV;
  // the fragment-order GEMM needs N multiples of 128 and K of 64 in every
  // prefill projection, and each activation below 2 GiB
  m->frag = QKV % 128 == 0 && H % 128 == 0 && (2 * I) % 128 == 0 && I % 64 == 0 &&
            (size_t)max_ctx * I * 4 < (1ull << 31);
  Arena& a = m->arena;
  bool ok = true;
  auto A = [&](size_t n) {
    float* p = a.alloc<float>(n);
    ok = ok && p;
    return p;
  };
  m->final_norm = A(H);
  m->llm_decoder = A((size_t)m->speech_vocab * H);
  m->layers.resize(m->NL);
  for (auto& L : m->layers) {
    L.qkv_w = A((size_t)QKV * H);
    L.qkv_b = A(QKV);
    L.o_w = A((size_t)H * H);
    L.gu_w = A((size_t)2 * I * H);
    L.down_w = A((size_t)H * I);
    if (m->frag) {
      L.qkv_wf = a.alloc<unsigned short>((size_t)3 * QKV * H);
      L.o_wf = a.alloc<unsigned short>((size_t)3 * H * H);
      L.gu_wf = a.alloc<unsigned short>((size_t)3 * 2 * I * H);
      L.down_wf = a.alloc<unsigned short>((size_t)3 * H * I);
      ok = ok && L.qkv_wf && L.o_wf && L.gu_wf && L.down_wf;
    }
    L.in_norm = A(H);
    L.post_norm = A(H);
    L.k_cache = A((size_t)max_ctx * KV);
    L.v_cache = A((size_t)max_ctx * KV);
  }
  const size_t rows = max_ctx;
  m->x = A(rows * H);
  m->hn = A(rows * H);
  m->qkv = A(rows * QKV);
  m->att = A(rows * H);
  m->act = A(rows * I);
  int tails = 0;
  m->ws_floats = std::max(splitk_ws_floats(max_ctx, H, QKV, I, &tails), bx_split_ws_floats(64));
  m->ws = A(m->ws_floats);
  // counters of the fp32 split tail, and one per tile of the gate/up split tail
  // (fewer than 2 x CUs tiles where it applies)
  m->n_arrivals = std::max(tails, 1024);
  m->arrivals = a.alloc<unsigned>(m->n_arrivals);
  ok = ok && m->arrivals;
  m->max_splits = dec_attention_splits(max_ctx);
  m->part_stride = dec_attention_part_floats(max_ctx, m->NH / m->NKV);
  m->part = A((size_t)m->part_stride * m->NKV);
  m->pos = a.alloc<int>(max_ctx);
  m->d_pos = a.alloc<int>(1);
  m->rope_tab = A(m->HD / 2);
  ok = ok && m->pos && m->d_pos;
  if (!ok) {
    delete m;
    set_error("qwen2_create: device allocation failed");
    return LX_ERR_ALLOC;
  }
  hipStream_t s = nullptr;
  if (hipStreamCreate(&s) != hipSuccess) {
    delete m;
    set_error("qwen2_create: stream creation failed");
    return LX_ERR_LAUNCH;
  }
  int rc = LX_OK;
  auto C = [&](float* dst, const float* src, size_t n) {
    if (rc != LX_OK) return;
    if (!src) {
      set_error("qwen2_create: missing weight tensor");
      rc = LX_ERR_ARG;
      return;
    }
    if (hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s) != hipSuccess) {
      set_error("qwen2_create: device copy failed");
      rc = LX_ERR_LAUNCH;
    }
  };
  C(m->final_norm, w->final_norm, H);
  C(m->llm_decoder, w->llm_decoder, (size_t)m->speech_vocab * H);
  for (int l = 0; l < m->NL && rc == LX_OK; ++l) {
    const lx_qwen2_layer_weights& lw = w->layers[l];
    Layer& L = m->layers[l];
    C(L.qkv_w, lw.q_w, (size_t)H * H);
    C(L.qkv_w + (size_t)H * H, lw.k_w, (size_t)KV * H);
    C(L.qkv_w + (size_t)(H + KV) * H, lw.v_w, (size_t)KV * H);
    C(L.qkv_b, lw.q_b, H);
    C(L.qkv_b + H, lw.k_b, KV);
    C(L.qkv_b + H + KV, lw.v_b, KV);
    C(L.o_w, lw.o_w, (size_t)H * H);
    C(L.down_w, lw.down_w, (size_t)H * I);
    C(L.in_norm, lw.in_norm, H);
    C(L.post_norm, lw.post_norm, H);
    if (rc == LX_OK) rc = (lw.gate_w && lw.up_w) ? LX_OK : LX_ERR_ARG;
    if (rc == LX_OK) rc = interleave_rows(lw.gate_w, lw.up_w, L.gu_w, I, H, s);
    if (m->frag) {
      if (rc == LX_OK) rc = wfrag_pack(L.qkv_w, L.qkv_wf, QKV, H, s);
      if (rc == LX_OK) rc = wfrag_pack(L.o_w, L.o_wf, H, H, s);
      if (rc == LX_OK) rc = wfrag_pack(L.gu_w, L.gu_wf, 2 * I, H, s);
      if (rc == LX_OK) rc = wfrag_pack(L.down_w, L.down_wf, H, I, s);
    }
  }
  if (rc == LX_OK) rc = iota_i32(m->pos, max_ctx, s);
  // the split tail's arrival counters start at zero; every launch leaves them so
  if (rc == LX_OK &&
      hipMemsetAsync(m->arrivals, 0, sizeof(unsigned) * m->n_arrivals, s) != hipSuccess) {
    set_error("qwen2_create: counter initialisation failed");
    rc = LX_ERR_LAUNCH;
  }
  FreqTable inv{};
  rope_inv_freq(m->theta, m->HD, inv.v);
  if (rc == LX_OK && hipMemcpyAsync(m->rope_tab, inv.v, sizeof(float) * (m->HD / 2),
                                    hipMemcpyHostToDevice, s) != hipSuccess) {
    set_error("qwen2_create: rotary table upload failed");
    rc = LX_ERR_LAUNCH;
  }
  if (rc == LX_OK && hipStreamSynchronize(s) != hipSuccess) {
    set_error("qwen2_create: weight packing failed");
    rc = LX_ERR_LAUNCH;
  }
  (void)hipStreamDestroy(s);
  if (rc != LX_OK) {
    delete m;
    return rc;
  }
  *out = m;
  return LX_OK;
}

extern "C" void lx_qwen2_destroy(lx_qwen2* m) {
  if (!m) return;
  (void)hipDeviceSynchronize();
  delete m;
}

extern "C" int lx_qwen2_build_lm_input(lx_qwen2* m, const int* text_tokens, int n_text,
                                       const int* prompt_speech, int n_speech, float* out,
                                       int* L_out, hipStream_t s) {
  LX_REQUIRE(m && out, "qwen2_build_lm_input: null argument");
  LX_REQUIRE(n_text >= 0 && n_speech >= 0 && (text_tokens || n_text == 0) &&
                 (prompt_speech || n_speech == 0),
             "qwen2_build_lm_input: bad token arrays");
  if (L_out) *L_out = 0;
  // Validate every id before writing anything (src/llm/llm.cpp:71-72).
  for (int i = 0; i < n_text; ++i)
    if (text_tokens[i] < 0 || text_tokens[i] >= m->text_vocab) {
      set_error("qwen2_build_lm_input: text id %d at %d outside [0, %d)", text_tokens[i], i,
                m->text_vocab);
      return LX_ERR_RANGE;
    }
  for (int i = 0; i < n_speech; ++i)
    if (prompt_speech[i] < 0 || prompt_speech[i] >= m->speech_vocab) {
      set_error("qwen2_build_lm_input: speech id %d at %d outside [0, %d)", prompt_speech[i], i,
                m->speech_vocab);
      return LX_ERR_RANGE;
    }
  const int H = m->H;
  float* p = out;
  const int sos = kSosToken, task = kTaskIdToken;
  LX_TRY(lx_embed_gather_f32(m->speech_embedding, m->speech_vocab, H, &sos, 1, p, s));
  p += H;
  if (n_text) LX_TRY(lx_embed_gather_f32(m->embed_tokens, m->text_vocab, H, text_tokens, n_text, p, s));
  p += (long)n_text * H;
  LX_TRY(lx_embed_gather_f32(m->speech_embedding, m->speech_vocab, H, &task, 1, p, s));
  p += H;
  if (n_speech)
    LX_TRY(lx_embed_gather_f32(m->speech_embedding, m->speech_vocab, H, prompt_speech, n_speech, p,
                               s));
  if (L_out) *L_out = 1 + n_text + 1 + n_speech;
  return LX_OK;
}

extern "C" int lx_qwen2_prefill(lx_qwen2* m, const float* lm_input, int L, float* logits,
                                float* hidden, float* final_norm, hipStream_t s) {
  LX_REQUIRE(m && lm_input, "qwen2_prefill: null argument");
  LX_REQUIRE(L >= 1 && L <= m->max_ctx, "qwen2_prefill: L=%d outside [1, %d]", L, m->max_ctx);
  const int H = m->H;
  if (hipMemcpyAsync(m->x, lm_input, sizeof(float) * (size_t)L * H, hipMemcpyDeviceToDevice, s) !=
      hipSuccess) {
    set_error("qwen2_prefill: copy failed");
    return LX_ERR_LAUNCH;
  }
  m->cache_len = 0;
  LX_TRY(lx_rmsnorm_f32(m->x, m->layers[0].in_norm, m->hn, L, H, m->eps, s));
  for (int l = 0; l < m->NL; ++l) {
    const float* next_norm = l + 1 < m->NL ? m->layers[l + 1].in_norm : m->final_norm;
    LX_TRY(prefill_layer(m, m->layers[l], L, next_norm, s, /*hn_packed*/ l > 0,
                         /*pack_next*/ l + 1 < m->NL));
    if (hidden)
      (void)hipMemcpyAsync(hidden + (size_t)l * L * H, m->x, sizeof(float) * (size_t)L * H,
                           hipMemcpyDeviceToDevice, s);
  }
  if (final_norm)
    (void)hipMemcpyAsync(final_norm, m->hn, sizeof(float) * (size_t)L * H, hipMemcpyDeviceToDevice,
                         s);
  if (logits)
    LX_TRY(lx_linear_f32(m->hn, H, m->llm_decoder, nullptr, logits, m->speech_vocab, L,
                         m->speech_vocab, H, nullptr, s));
  m->cache_len = L;
  return check_launch("qwen2_prefill");
}

extern "C" int lx_qwen2_decode(lx_qwen2* m, int token, float* logits, float* final_norm,
                               hipStream_t s) {
  LX_REQUIRE(m && logits, "qwen2_decode: null argument");
  if (token < 0 || token >= m->speech_vocab) {
    set_error("qwen2_decode: token %d outside [0, %d)", token, m->speech_vocab);
    return LX_ERR_RANGE;
  }
  if (m->cache_len <= 0) {
    set_error("qwen2_decode: decode before prefill");
    return LX_ERR_STATE;
  }
  if (m->cache_len >= m->max_ctx) {
    set_error("qwen2_decode: KV cache full (%d)", m->max_ctx);
    return LX_ERR_STATE;
  }
  const int H = m->H;
  // speech_embedding row of the token (src/llm/llm.cpp:226-230) and its position
  LX_TRY(dec_begin(m->speech_embedding, token, H, m->x, m->d_pos, m->cache_len, s));
  // one captured layer stack per launch class of the position
  const int cls = decode_class(m->cache_len);
  LX_REQUIRE(cls >= 0, "qwen2_decode: position %d past the attention merge", m->cache_len);
  if (m->use_graph) {
    if (!m->graph[cls]) LX_TRY(capture_decode(m, cls));
    if (hipGraphLaunch(m->graph[cls], s) != hipSuccess) {
      set_error("qwen2_decode: hipGraphLaunch failed");
      return LX_ERR_LAUNCH;
    }
  } else {
    LX_TRY(decode_stack(m, cls, s));
  }
  // final norm + llm_decoder head (src/llm/llm.cpp:291-300)
  DecGemvArgs h;
  h.x = m->x;
  h.norm_w = m->final_norm;
  h.eps = m->eps;
  h.W = m->llm_decoder;
  h.y = logits;
  h.y2 = final_norm;
  h.N = m->speech_vocab;
  h.K = H;
  LX_TRY(dec_gemv(DEC_HEAD, h, s));
  m->cache_len += 1;
  return LX_OK;
}

extern "C" int lx_qwen2_cache_len(const lx_qwen2* m) { return m ? m->cache_len : 0; }

extern "C" const float* lx_qwen2_cache_key(const lx_qwen2* m, int layer) {
  if (!m || layer < 0 || layer >= m->NL) return nullptr;
  return m->layers[layer].k_cache;
}

extern "C" const float* lx_qwen2_cache_value(const lx_qwen2* m, int layer) {
  if (!m || layer < 0 || layer >= m->NL) return nullptr;
  return m->layers[layer].v_cache;
}

extern "C" int lx_qwen2_set_products(lx_qwen2* m, int products) {
  LX_REQUIRE(m, "qwen2_set_products: null model");
  LX_REQUIRE(products == 3 || products == 6, "qwen2_set_products: %d products (3 or 6)",
             products);
  m->products = products;
  return LX_OK;
}

extern "C" int lx_qwen2_set_decode_graph(lx_qwen2* m, int enable) {
  LX_REQUIRE(m, "qwen2_set_decode_graph: null model");
  m->use_graph = enable != 0;  // graphs already captured are kept for a later switch back
  return LX_OK;
}

extern "C" int lx_qwen2_set_cache_len(lx_qwen2* m, int len) {
  LX_REQUIRE(m, "qwen2_set_cache_len: null model");
  LX_REQUIRE(len >= 0 && len <= m->max_ctx, "qwen2_set_cache_len: %d outside [0, %d]", len,
             m->max_ctx);
  m->cache_len = len;
  return LX_OK;
}
