"""Qwen2 backbone of CosyVoice3LM on liblxops (host glue).

The `lx_qwen2` object is the drop-in for LLM (include/larynx/llm/llm.h:31-104):
build_lm_input, prefill, decode and the KV-cache accessors, with the cache kept
on the device.  Parameter names are those of the reference GGUF
(src/llm/gguf.cpp:44-83) without the "llm.model.model." prefix, i.e. the
transformers Qwen2Model state_dict keys plus speech_embedding / llm_decoder.
"""
import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import Qwen2LayerWeights, Qwen2Weights, check, lib
from .ops import stream


@dataclass(frozen=True)
class Qwen2Config:
    """src/llm/internal.h:18-34 (CosyVoice-BlankEN config.json)."""
    hidden: int = 896
    intermediate: int = 4864
    n_heads: int = 14
    n_kv_heads: int = 2
    head_dim: int = 64
    n_layers: int = 24
    text_vocab: int = 151936
    speech_vocab: int = 6761
    rms_eps: float = 1e-6
    rope_theta: float = 1e6


SOS_TOKEN = 6561      # src/llm/internal.h:33
TASK_ID_TOKEN = 6563  # src/llm/internal.h:34


def qwen2_param_shapes(cfg: Qwen2Config):
    H, I, KV = cfg.hidden, cfg.intermediate, cfg.n_kv_heads * cfg.head_dim
    out = [
        ("embed_tokens.weight", (cfg.text_vocab, H)),
        ("speech_embedding.weight", (cfg.speech_vocab, H)),
        ("norm.weight", (H,)),
        ("llm_decoder.weight", (cfg.speech_vocab, H)),
    ]
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (H, H)), (p + "self_attn.q_proj.bias", (H,)),
            (p + "self_attn.k_proj.weight", (KV, H)), (p + "self_attn.k_proj.bias", (KV,)),
            (p + "self_attn.v_proj.weight", (KV, H)), (p + "self_attn.v_proj.bias", (KV,)),
            (p + "self_attn.o_proj.weight", (H, H)),
            (p + "mlp.gate_proj.weight", (I, H)),
            (p + "mlp.up_proj.weight", (I, H)),
            (p + "mlp.down_proj.weight", (H, I)),
            (p + "input_layernorm.weight", (H,)),
            (p + "post_attention_layernorm.weight", (H,)),
        ]
    return out


_LAYER_KEYS = {
    "q_w": "self_attn.q_proj.weight", "q_b": "self_attn.q_proj.bias",
    "k_w": "self_attn.k_proj.weight", "k_b": "self_attn.k_proj.bias",
    "v_w": "self_attn.v_proj.weight", "v_b": "self_attn.v_proj.bias",
    "o_w": "self_attn.o_proj.weight", "gate_w": "mlp.gate_proj.weight",
    "up_w": "mlp.up_proj.weight", "down_w": "mlp.down_proj.weight",
    "in_norm": "input_layernorm.weight", "post_norm": "post_attention_layernorm.weight",
}


def _ptr(params, name, shape):
    t = params[name]
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)} != {tuple(shape)}")
    if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise ValueError(f"{name}: must be a contiguous CUDA float32 tensor")
    return C.c_void_p(t.data_ptr())


class Qwen2LM:
    """Device-resident Qwen2 LM.  The embedding tables stay referenced (keep `params`
    alive); layer weights are re-packed into library memory at construction."""

    def __init__(self, params, cfg: Qwen2Config = Qwen2Config(), max_ctx: int = 4096):
        self.cfg, self.max_ctx = cfg, max_ctx
        self._params = params
        shapes = dict(qwen2_param_shapes(cfg))
        layers = (Qwen2LayerWeights * cfg.n_layers)()
        for i in range(cfg.n_layers):
            for field, key in _LAYER_KEYS.items():
                name = f"layers.{i}.{key}"
                setattr(layers[i], field, _ptr(params, name, shapes[name]))
        w = Qwen2Weights()
        for f in ("hidden", "intermediate", "n_heads", "n_kv_heads", "head_dim", "n_layers",
                  "text_vocab", "speech_vocab", "rms_eps", "rope_theta"):
            setattr(w, f, getattr(cfg, f))
        w.embed_tokens = _ptr(params, "embed_tokens.weight", shapes["embed_tokens.weight"])
        w.speech_embedding = _ptr(params, "speech_embedding.weight",
                                  shapes["speech_embedding.weight"])
        w.final_norm = _ptr(params, "norm.weight", shapes["norm.weight"])
        w.llm_decoder = _ptr(params, "llm_decoder.weight", shapes["llm_decoder.weight"])
        w.layers = layers
        torch.cuda.synchronize()
        h = C.c_void_p()
        check(lib.lx_qwen2_create(C.byref(w), max_ctx, C.byref(h)))
        self._h = h

    @classmethod
    def load(cls, path, max_ctx: int = 4096):
        """LLM::load: an llm.gguf checkpoint (geometry from its tensors; the model
        copies every tensor into its own device memory)."""
        from .gguf import GgufFile
        hdr = GgufFile(path, device=False)
        shape = {n: s for n, _, s, _ in hdr.tensors()}
        hdr.close()
        M = "llm.model.model."
        n_layers = 0
        while f"{M}layers.{n_layers}.self_attn.q_proj.weight" in shape:
            n_layers += 1
        text_vocab, H = shape.get(M + "embed_tokens.weight", (0, 0))
        cfg = Qwen2Config(hidden=H, intermediate=shape.get(M + "layers.0.mlp.gate_proj.weight",
                                                           (0, 0))[0],
                          n_heads=H // 64,
                          n_kv_heads=shape.get(M + "layers.0.self_attn.k_proj.weight",
                                               (0, 0))[0] // 64,
                          n_layers=n_layers, text_vocab=text_vocab,
                          speech_vocab=shape.get("speech_embedding.weight", (0, 0))[0])
        self = cls.__new__(cls)
        self.cfg, self.max_ctx, self._params = cfg, max_ctx, None
        h = C.c_void_p()
        check(lib.lx_qwen2_load(str(path).encode(), max_ctx, C.byref(h)))
        self._h = h
        return self

    def close(self):
        if getattr(self, "_h", None):
            lib.lx_qwen2_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone already
            pass

    def build_lm_input(self, text_tokens, prompt_speech_tokens, device="cuda"):
        """lm_input (L, H) = [sos; embed_tokens(text); task_id; speech_emb(prompt)]."""
        t = [int(v) for v in text_tokens]
        s = [int(v) for v in prompt_speech_tokens]
        L = 2 + len(t) + len(s)
        out = torch.empty(L, self.cfg.hidden, device=device, dtype=torch.float32)
        ta = (C.c_int * max(1, len(t)))(*t)
        sa = (C.c_int * max(1, len(s)))(*s)
        Lo = C.c_int()
        check(lib.lx_qwen2_build_lm_input(self._h, ta, len(t), sa, len(s), out.data_ptr(),
                                          C.byref(Lo), stream()))
        assert Lo.value == L
        return out

    def prefill(self, lm_input, want_logits=True, capture=False):
        """Causal pass over lm_input (L, H); fills the KV cache.  Returns logits
        (L, speech_vocab) or None, plus (hidden (n_layers, L, H), final_norm (L, H))
        when capture is set."""
        L = lm_input.shape[0]
        dev = lm_input.device
        logits = (torch.empty(L, self.cfg.speech_vocab, device=dev) if want_logits else None)
        hidden = final = None
        if capture:
            hidden = torch.empty(self.cfg.n_layers, L, self.cfg.hidden, device=dev)
            final = torch.empty(L, self.cfg.hidden, device=dev)
        check(lib.lx_qwen2_prefill(self._h, lm_input.data_ptr(), L,
                                   logits.data_ptr() if logits is not None else None,
                                   hidden.data_ptr() if hidden is not None else None,
                                   final.data_ptr() if final is not None else None, stream()))
        if capture:
            return logits, hidden, final
        return logits

    def decode(self, token, final_norm=False, device="cuda"):
        """One speech token at position cache_len; returns logits (speech_vocab)
        [and the final-norm row]."""
        logits = torch.empty(self.cfg.speech_vocab, device=device)
        fn = torch.empty(self.cfg.hidden, device=device) if final_norm else None
        check(lib.lx_qwen2_decode(self._h, int(token), logits.data_ptr(),
                                  fn.data_ptr() if fn is not None else None, stream()))
        return (logits, fn) if final_norm else logits

    @property
    def cache_len(self):
        return lib.lx_qwen2_cache_len(self._h)

    def set_cache_len(self, n):
        check(lib.lx_qwen2_set_cache_len(self._h, int(n)))

    def set_decode_graph(self, enable):
        """Replay decode as a captured HIP graph (True, the default) or launch it
        eagerly (False)."""
        check(lib.lx_qwen2_set_decode_graph(self._h, 1 if enable else 0))

    def set_products(self, products):
        """Split-operand products of the prefill projections: 3 (the default) or 6."""
        check(lib.lx_qwen2_set_products(self._h, int(products)))

    def cache_views(self, layer):
        """(k, v) device views (max_ctx, KV) of the layer's cache (roped keys, raw values)."""
        KV = self.cfg.n_kv_heads * self.cfg.head_dim
        out = []
        for fn in (lib.lx_qwen2_cache_key, lib.lx_qwen2_cache_value):
            ptr = fn(self._h, layer)
            if not ptr:
                raise IndexError(layer)
            out.append(_device_view(ptr, (self.max_ctx, KV)))
        return tuple(out)


def _device_view(ptr, shape):
    """Wrap a library-owned device pointer as a torch tensor (no copy, no ownership)."""
    n = 1
    for s in shape:
        n *= s

    class _Iface:
        __cuda_array_interface__ = {
            "shape": tuple(shape), "typestr": "<f4", "data": (int(ptr), False), "version": 2,
            "strides": None,
        }

    return torch.as_tensor(_Iface(), device="cuda")
