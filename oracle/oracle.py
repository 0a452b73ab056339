"""ctypes front end of the CPU oracle (liblxoracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the test oracle / CPU baseline.  Never used by the
product path.  Arrays are numpy float32 (C-contiguous).
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblxoracle.so")

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
vp = C.c_void_p


class OrcDitBlock(C.Structure):
    _fields_ = [(n, vp) for n in (
        "attn_norm_w", "attn_norm_b", "to_q_w", "to_q_b", "to_k_w", "to_k_b", "to_v_w",
        "to_v_b", "to_out_w", "to_out_b", "ff0_w", "ff0_b", "ff2_w", "ff2_b")]


class OrcDit(C.Structure):
    _fields_ = [
        ("dim", C.c_int), ("depth", C.c_int), ("heads", C.c_int), ("head_dim", C.c_int),
        ("ff_inner", C.c_int), ("mel_dim", C.c_int),
        ("time_mlp_0_w", vp), ("time_mlp_0_b", vp), ("time_mlp_2_w", vp), ("time_mlp_2_b", vp),
        ("input_proj_w", vp), ("input_proj_b", vp),
        ("conv_pos_1_w", vp), ("conv_pos_1_b", vp), ("conv_pos_2_w", vp), ("conv_pos_2_b", vp),
        ("blocks", C.POINTER(OrcDitBlock)),
        ("norm_out_w", vp), ("norm_out_b", vp), ("proj_out_w", vp), ("proj_out_b", vp),
    ]


class OrcDitCapture(C.Structure):
    _fields_ = [(n, vp) for n in
                ("time_embed", "input_proj", "conv_pos", "input_embed", "blocks", "norm_out")]


class OrcQwenLayer(C.Structure):
    _fields_ = [(n, vp) for n in ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "gate_w",
                                  "up_w", "down_w", "in_norm", "post_norm")]


class OrcQwen(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("intermediate", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_layers", C.c_int),
        ("text_vocab", C.c_int), ("speech_vocab", C.c_int),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("embed_tokens", vp), ("speech_embedding", vp), ("final_norm", vp), ("llm_decoder", vp),
        ("layers", C.POINTER(OrcQwenLayer)),
    ]


class OrcFlowFront(C.Structure):
    _fields_ = [("vocab", C.c_int), ("spk_in", C.c_int), ("mel", C.c_int), ("channels", C.c_int)] + [
        (n, vp) for n in ("input_embedding", "spk_affine_w", "spk_affine_b", "pre_conv1_w",
                          "pre_conv1_b", "pre_conv2_w", "pre_conv2_b")]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} not built (make -C oracle)")
    lib = C.CDLL(LIB_PATH)
    sig = {
        "orc_set_threads": (None, [C.c_int]),
        "orc_get_threads": (C.c_int, []),
        "orc_fill_normal": (None, [f32p, C.c_long, C.c_uint64, C.c_uint64, C.c_float]),
        "orc_adaln": (None, [f32p, vp, vp, C.c_long, f32p, C.c_int, C.c_int, C.c_int, C.c_float]),
        "orc_linear": (None, [f32p, C.c_int, f32p, vp, f32p, C.c_int, C.c_int, C.c_int, C.c_int]),
        "orc_gelu_tanh": (None, [f32p, f32p, C.c_long]),
        "orc_gated_residual": (None, [f32p, f32p, vp, C.c_long, C.c_int, C.c_int, C.c_int]),
        "orc_rope_inv_freq": (None, [C.c_float, C.c_int, f32p]),
        "orc_rope_partial": (None, [f32p, i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
        "orc_timestep_embed": (None, [f32p, C.c_int, C.c_int, C.c_float, f32p]),
        "orc_time_mlp": (None, [f32p, C.c_int, f32p, f32p, f32p, f32p, C.c_int, f32p]),
        "orc_rmsnorm": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]),
        "orc_rope_neox": (None, [f32p, i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
        "orc_swiglu": (None, [f32p, f32p, f32p, C.c_long]),
        "orc_embed_gather": (C.c_int, [f32p, C.c_long, C.c_int, i32p, C.c_int, f32p]),
        "orc_attention": (None, [vp, C.c_int, vp, C.c_int, vp, C.c_int, vp, C.c_int, C.c_int,
                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int,
                                 C.c_int]),
        "orc_conv_pos_mish": (None, [f32p, f32p, f32p, vp, f32p, C.c_int, C.c_int, C.c_int,
                                     C.c_int, C.c_int]),
        "orc_dit_forward": (C.c_int, [C.POINTER(OrcDit), C.c_int, C.c_int, f32p, f32p, f32p,
                                      f32p, f32p, f32p, C.POINTER(OrcDitCapture)]),
        "orc_cfm_step": (C.c_int, [C.POINTER(OrcDit), C.c_int, f32p, f32p, f32p, f32p, C.c_float,
                                   C.c_float, C.c_float]),
        "orc_cfm_solve": (C.c_int, [C.POINTER(OrcDit), C.c_int, f32p, f32p, f32p, f32p, C.c_int,
                                    C.c_float]),
        "orc_flow_frontend": (C.c_int, [C.POINTER(OrcFlowFront), i32p, C.c_int, vp, C.c_int, f32p,
                                        f32p, vp, vp, f32p, f32p]),
        "orc_qwen2_build_lm_input": (C.c_int, [C.POINTER(OrcQwen), i32p, C.c_int, i32p, C.c_int,
                                               f32p]),
        "orc_qwen2_forward": (C.c_int, [C.POINTER(OrcQwen), f32p, C.c_int, C.c_int, f32p, f32p,
                                        C.c_int, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _vp(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def normal(shape, seed, stream, std=1.0):
    """Deterministic N(0, std^2) float32 array for (seed, stream)."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib.orc_fill_normal(out, n, seed, stream, std)
    return out.reshape(shape)


def make_params(shapes, seed, std=0.02):
    """name -> array for an ordered (name, shape) list; tensor i uses stream i."""
    return {name: normal(shape, seed, i, std) for i, (name, shape) in enumerate(shapes)}


# ---- per-op ----------------------------------------------------------------
def adaln(x, scale, shift, eps=1e-6):
    """x (B, T, D); scale/shift (B, D) arrays (contiguous rows)."""
    x = c32(x)
    B, T, D = x.shape
    scale, shift = c32(scale), c32(shift)
    y = np.empty_like(x)
    lib.orc_adaln(x, _vp(shift), _vp(scale), scale.shape[-1], y, B, T, D, eps)
    return y


def linear(x, W, b=None):
    x, W = c32(x), c32(W)
    M, K = x.shape
    N = W.shape[0]
    b = None if b is None else c32(b)
    y = np.empty((M, N), dtype=np.float32)
    lib.orc_linear(x, K, W, _vp(b), y, N, M, N, K)
    return y


def gelu_tanh(h):
    h = c32(h)
    y = np.empty_like(h)
    lib.orc_gelu_tanh(h, y, h.size)
    return y


def gated_residual(x, y, gate):
    x = c32(x).copy()
    B, T, D = x.shape
    gate = c32(gate)
    lib.orc_gated_residual(x, c32(y), _vp(gate), gate.shape[-1], B, T, D)
    return x


def rope_inv_freq(base, dim):
    out = np.empty(dim // 2, dtype=np.float32)
    lib.orc_rope_inv_freq(base, dim, out)
    return out


def rope_partial(q, pos, rot_dim=64, base=10000.0):
    q = c32(q).copy()
    B, T, ld = q.shape
    lib.orc_rope_partial(q, np.ascontiguousarray(pos, dtype=np.int32), B, T, ld, rot_dim, base)
    return q


def timestep_embed(t, half_dim=128, scale=1000.0):
    t = c32(t)
    out = np.empty((t.shape[0], 2 * half_dim), dtype=np.float32)
    lib.orc_timestep_embed(t, t.shape[0], half_dim, scale, out)
    return out


def time_mlp(t, w0, b0, w2, b2):
    t = c32(t)
    D = w0.shape[0]
    out = np.empty((t.shape[0], D), dtype=np.float32)
    lib.orc_time_mlp(t, t.shape[0], c32(w0), c32(b0), c32(w2), c32(b2), D, out)
    return out


def rmsnorm(x, w, eps=1e-6):
    x = c32(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib.orc_rmsnorm(x, c32(w), y, x.size // D, D, eps)
    return y


def rope_neox(qk, pos, n_heads, head_dim=64, theta=1e6):
    qk = c32(qk).copy()
    rows, ld = qk.shape
    lib.orc_rope_neox(qk, np.ascontiguousarray(pos, dtype=np.int32), rows, n_heads, head_dim, ld,
                      theta)
    return qk


def swiglu(g, u):
    g = c32(g)
    y = np.empty_like(g)
    lib.orc_swiglu(g, c32(u), y, g.size)
    return y


def embed_gather(table, ids):
    table = c32(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((len(ids), table.shape[1]), dtype=np.float32)
    rc = lib.orc_embed_gather(table, table.shape[0], table.shape[1], ids, len(ids), out)
    if rc != 0:
        raise IndexError("token id out of range")
    return out


def attention(q, k, v, n_heads, n_kv_heads=None, scale=None, causal=False, q_offset=0,
              head_dim=64):
    """q (B, Tq, ldq), k/v (B, Tk, ld) arrays; heads packed from column 0."""
    q, k, v = c32(q), c32(k), c32(v)
    n_kv_heads = n_kv_heads or n_heads
    B, Tq, ldq = q.shape
    Tk = k.shape[1]
    scale = head_dim ** -0.5 if scale is None else scale
    o = np.empty((B, Tq, n_heads * head_dim), dtype=np.float32)
    lib.orc_attention(_vp(q), ldq, _vp(k), k.shape[2], _vp(v), v.shape[2], _vp(o), o.shape[2], B,
                      Tq, Tk, n_heads, n_kv_heads, head_dim, scale, int(causal), q_offset)
    return o


def conv_pos_mish(x, w, b, resid=None, groups=16):
    x = c32(x)
    B, T, Cc = x.shape
    K = w.shape[2]
    y = np.empty_like(x)
    r = None if resid is None else c32(resid)
    lib.orc_conv_pos_mish(x, c32(w), c32(b), _vp(r), y, B, T, Cc, groups, K)
    return y


# ---- composites --------------------------------------------------------------
_BLOCK_KEYS = {
    "attn_norm_w": "attn_norm.linear.weight", "attn_norm_b": "attn_norm.linear.bias",
    "to_q_w": "attn.to_q.weight", "to_q_b": "attn.to_q.bias",
    "to_k_w": "attn.to_k.weight", "to_k_b": "attn.to_k.bias",
    "to_v_w": "attn.to_v.weight", "to_v_b": "attn.to_v.bias",
    "to_out_w": "attn.to_out.0.weight", "to_out_b": "attn.to_out.0.bias",
    "ff0_w": "ff.ff.0.0.weight", "ff0_b": "ff.ff.0.0.bias",
    "ff2_w": "ff.ff.2.weight", "ff2_b": "ff.ff.2.bias",
}
_TOP_KEYS = {
    "time_mlp_0_w": "time_embed.time_mlp.0.weight", "time_mlp_0_b": "time_embed.time_mlp.0.bias",
    "time_mlp_2_w": "time_embed.time_mlp.2.weight", "time_mlp_2_b": "time_embed.time_mlp.2.bias",
    "input_proj_w": "input_embed.proj.weight", "input_proj_b": "input_embed.proj.bias",
    "conv_pos_1_w": "input_embed.conv_pos_embed.conv1.0.weight",
    "conv_pos_1_b": "input_embed.conv_pos_embed.conv1.0.bias",
    "conv_pos_2_w": "input_embed.conv_pos_embed.conv2.0.weight",
    "conv_pos_2_b": "input_embed.conv_pos_embed.conv2.0.bias",
    "norm_out_w": "norm_out.linear.weight", "norm_out_b": "norm_out.linear.bias",
    "proj_out_w": "proj_out.weight", "proj_out_b": "proj_out.bias",
}


class Dit:
    """Oracle DiT over a dict of numpy params (names as larynx_amd.flow.dit_param_shapes)."""

    def __init__(self, params, dim=1024, depth=22, heads=16, head_dim=64, ff_inner=2048,
                 mel_dim=80):
        self._keep = {k: c32(v) for k, v in params.items()}
        self.blocks = (OrcDitBlock * depth)()
        for i in range(depth):
            for f, key in _BLOCK_KEYS.items():
                setattr(self.blocks[i], f, _vp(self._keep[f"transformer_blocks.{i}.{key}"]))
        w = OrcDit()
        w.dim, w.depth, w.heads, w.head_dim, w.ff_inner, w.mel_dim = (
            dim, depth, heads, head_dim, ff_inner, mel_dim)
        for f, key in _TOP_KEYS.items():
            setattr(w, f, _vp(self._keep[key]))
        w.blocks = self.blocks
        self.w = w
        self.mel = mel_dim
        self.dim = dim
        self.depth = depth

    def forward(self, x, mu, cond, spks, t, capture=None):
        x, mu, cond, spks, t = map(c32, (x, mu, cond, spks, t))
        B, mel, T = x.shape
        dphi = np.empty_like(x)
        cap = OrcDitCapture()
        if capture is not None:
            shapes = {"time_embed": (B, self.dim), "input_proj": (B, T, self.dim),
                      "conv_pos": (B, T, self.dim), "input_embed": (B, T, self.dim),
                      "blocks": (self.depth, B, T, self.dim), "norm_out": (B, T, self.dim)}
            for k in list(capture):
                capture[k] = np.empty(shapes[k], dtype=np.float32)
                setattr(cap, k, _vp(capture[k]))
        rc = lib.orc_dit_forward(C.byref(self.w), B, T, x, mu, cond, spks, t, dphi, C.byref(cap))
        assert rc == 0, rc
        return dphi

    def cfm_step(self, x, mu, cond, spks, t, dt, cfg_rate=0.7):
        x = c32(x).copy()
        rc = lib.orc_cfm_step(C.byref(self.w), x.shape[-1], x, c32(mu), c32(cond), c32(spks),
                              t, dt, cfg_rate)
        assert rc == 0, rc
        return x

    def cfm_solve(self, z, mu, cond, spks, n_steps=10, cfg_rate=0.7):
        x = c32(z).copy()
        rc = lib.orc_cfm_solve(C.byref(self.w), x.shape[-1], x, c32(mu), c32(cond), c32(spks),
                               n_steps, cfg_rate)
        assert rc == 0, rc
        return x


_FRONT_KEYS = {
    "input_embedding": "input_embedding.weight",
    "spk_affine_w": "spk_embed_affine_layer.weight", "spk_affine_b": "spk_embed_affine_layer.bias",
    "pre_conv1_w": "pre_lookahead_layer.conv1.weight", "pre_conv1_b": "pre_lookahead_layer.conv1.bias",
    "pre_conv2_w": "pre_lookahead_layer.conv2.weight", "pre_conv2_b": "pre_lookahead_layer.conv2.bias",
}


class Flow:
    """Oracle FlowDecoder::infer (frontend + CFM solve) over numpy params: the
    frontend names of larynx_amd.flow.flow_frontend_param_shapes plus the
    estimator's (Dit) names."""

    def __init__(self, front_params, dit_params, mel=80, **dit_kw):
        self._keep = {k: c32(v) for k, v in front_params.items()}
        w = OrcFlowFront()
        emb = self._keep["input_embedding.weight"]
        w.vocab, w.mel = emb.shape
        w.spk_in = self._keep["spk_embed_affine_layer.weight"].shape[1]
        w.channels = self._keep["pre_lookahead_layer.conv1.weight"].shape[0]
        for f, key in _FRONT_KEYS.items():
            setattr(w, f, _vp(self._keep[key]))
        self.w = w
        self.mel = mel
        self.dit = Dit(dit_params, mel_dim=mel, **dit_kw) if dit_params is not None else None

    def frontend(self, prompt_tokens, tokens, prompt_feat, spk_embedding):
        """-> dict spk (mel,), token_embed (Tseq, mel), prelookahead (Tseq, mel),
        mu (mel, MEL_T), cond (mel, MEL_T)."""
        ids = np.concatenate([np.asarray(prompt_tokens, np.int64), np.asarray(tokens, np.int64)])
        ids = np.ascontiguousarray(np.maximum(ids, 0), dtype=np.int32)  # token.clamp(min=0)
        T = len(ids)
        pf = c32(prompt_feat).reshape(-1, self.mel)
        out = {"spk": np.empty(self.mel, np.float32),
               "token_embed": np.empty((T, self.mel), np.float32),
               "prelookahead": np.empty((T, self.mel), np.float32),
               "mu": np.empty((self.mel, 2 * T), np.float32),
               "cond": np.empty((self.mel, 2 * T), np.float32)}
        rc = lib.orc_flow_frontend(C.byref(self.w), ids, T, _vp(pf), pf.shape[0],
                                   c32(spk_embedding).reshape(-1), out["spk"],
                                   _vp(out["token_embed"]), _vp(out["prelookahead"]), out["mu"],
                                   out["cond"])
        if rc == -3:
            raise IndexError("token id out of range")
        assert rc == 0, rc
        return out

    def infer(self, prompt_tokens, tokens, prompt_feat, spk_embedding, noise_z, n_steps=10,
              cfg_rate=0.7):
        """-> mel (mel, MEL_T - mel_len1), the frontend then the CFG Euler solve."""
        st = self.frontend(prompt_tokens, tokens, prompt_feat, spk_embedding)
        x = self.dit.cfm_solve(noise_z, st["mu"], st["cond"], st["spk"], n_steps, cfg_rate)
        mel_len1 = c32(prompt_feat).reshape(-1, self.mel).shape[0]
        return x[:, mel_len1:], st


_QKEYS = {
    "q_w": "self_attn.q_proj.weight", "q_b": "self_attn.q_proj.bias",
    "k_w": "self_attn.k_proj.weight", "k_b": "self_attn.k_proj.bias",
    "v_w": "self_attn.v_proj.weight", "v_b": "self_attn.v_proj.bias",
    "o_w": "self_attn.o_proj.weight", "gate_w": "mlp.gate_proj.weight",
    "up_w": "mlp.up_proj.weight", "down_w": "mlp.down_proj.weight",
    "in_norm": "input_layernorm.weight", "post_norm": "post_attention_layernorm.weight",
}


class Qwen2:
    """Oracle Qwen2 over numpy params (names as larynx_amd.llm.qwen2_param_shapes)."""

    def __init__(self, params, cfg, cap=4096):
        self._keep = {k: c32(v) for k, v in params.items()}
        self.cfg = cfg
        self.layers = (OrcQwenLayer * cfg.n_layers)()
        for i in range(cfg.n_layers):
            for f, key in _QKEYS.items():
                setattr(self.layers[i], f, _vp(self._keep[f"layers.{i}.{key}"]))
        w = OrcQwen()
        for f in ("hidden", "intermediate", "n_heads", "n_kv_heads", "head_dim", "n_layers",
                  "text_vocab", "speech_vocab", "rms_eps", "rope_theta"):
            setattr(w, f, getattr(cfg, f))
        w.embed_tokens = _vp(self._keep["embed_tokens.weight"])
        w.speech_embedding = _vp(self._keep["speech_embedding.weight"])
        w.final_norm = _vp(self._keep["norm.weight"])
        w.llm_decoder = _vp(self._keep["llm_decoder.weight"])
        w.layers = self.layers
        self.w = w
        self.cap = cap
        KV = cfg.n_kv_heads * cfg.head_dim
        self.k_cache = np.zeros((cfg.n_layers, cap, KV), dtype=np.float32)
        self.v_cache = np.zeros((cfg.n_layers, cap, KV), dtype=np.float32)
        self.cache_len = 0

    def build_lm_input(self, text, speech):
        text = np.ascontiguousarray(text, dtype=np.int32)
        speech = np.ascontiguousarray(speech, dtype=np.int32)
        L = 2 + len(text) + len(speech)
        out = np.empty((L, self.cfg.hidden), dtype=np.float32)
        rc = lib.orc_qwen2_build_lm_input(C.byref(self.w), text, len(text), speech, len(speech),
                                          out)
        if rc < 0:
            raise IndexError("token id out of range")
        return out

    def forward(self, x, past, want_logits=True, capture=False):
        x = c32(x)
        L = x.shape[0]
        cfg = self.cfg
        logits = np.empty((L, cfg.speech_vocab), np.float32) if want_logits else None
        hidden = np.empty((cfg.n_layers, L, cfg.hidden), np.float32) if capture else None
        final = np.empty((L, cfg.hidden), np.float32) if capture else None
        rc = lib.orc_qwen2_forward(C.byref(self.w), x, L, past, self.k_cache, self.v_cache,
                                   self.cap, _vp(logits), _vp(hidden), _vp(final))
        assert rc == 0, rc
        self.cache_len = past + L
        return logits, hidden, final

    def prefill(self, lm_input, capture=False):
        return self.forward(lm_input, 0, capture=capture)

    def decode(self, token):
        emb = self._keep["speech_embedding.weight"][int(token)][None, :]
        logits, _, final = self.forward(emb, self.cache_len, capture=True)
        return logits[0], final[0]


def rel_err(a, ref):
    """max|a - ref| / max|ref| (the reference's metric, tests/verify_flow.py:60-69)."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max()
    return float(np.abs(a - ref).max() / (den if den > 0 else 1.0))
