"""CosyVoice3 Flow DiT estimator + CFM Euler loop on liblxops (host glue).

The estimator object (`lx_dit` in the C-ABI) is the drop-in for the reference's
DiTGraph (src/flow/internal.h:104-120, built by build_dit src/flow/dit.cpp:83-145)
and the CFM loop of FlowDecoder::infer (src/flow/flow.cpp:184-274).  Parameter
names are the estimator's state_dict keys, i.e. the GGUF tensor names of
src/flow/gguf.cpp:56-90 without the "decoder.estimator." prefix.
"""
import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import (DitBlockWeights, DitCapture, DitWeights, FlowCapture, FlowFrontendWeights,
                   check, lib)
from .ops import stream


@dataclass(frozen=True)
class DiTConfig:
    """Architecture constants of src/flow/internal.h:18-41 (cosyvoice3.yaml)."""
    dim: int = 1024
    depth: int = 22
    heads: int = 16
    head_dim: int = 64
    ff_inner: int = 2048
    mel_dim: int = 80
    freq_dim: int = 256
    conv_kernel: int = 31
    conv_groups: int = 16
    n_timesteps: int = 10
    cfg_rate: float = 0.7


def dit_param_shapes(cfg: DiTConfig):
    """Ordered (name, shape) list of the estimator's parameters (torch layouts)."""
    D, F, mel = cfg.dim, cfg.ff_inner, cfg.mel_dim
    cg = D // cfg.conv_groups
    out = [
        ("time_embed.time_mlp.0.weight", (D, cfg.freq_dim)),
        ("time_embed.time_mlp.0.bias", (D,)),
        ("time_embed.time_mlp.2.weight", (D, D)),
        ("time_embed.time_mlp.2.bias", (D,)),
        ("input_embed.proj.weight", (D, 4 * mel)),
        ("input_embed.proj.bias", (D,)),
        ("input_embed.conv_pos_embed.conv1.0.weight", (D, cg, cfg.conv_kernel)),
        ("input_embed.conv_pos_embed.conv1.0.bias", (D,)),
        ("input_embed.conv_pos_embed.conv2.0.weight", (D, cg, cfg.conv_kernel)),
        ("input_embed.conv_pos_embed.conv2.0.bias", (D,)),
    ]
    for i in range(cfg.depth):
        p = f"transformer_blocks.{i}."
        out += [
            (p + "attn_norm.linear.weight", (6 * D, D)),
            (p + "attn_norm.linear.bias", (6 * D,)),
            (p + "attn.to_q.weight", (D, D)), (p + "attn.to_q.bias", (D,)),
            (p + "attn.to_k.weight", (D, D)), (p + "attn.to_k.bias", (D,)),
            (p + "attn.to_v.weight", (D, D)), (p + "attn.to_v.bias", (D,)),
            (p + "attn.to_out.0.weight", (D, D)), (p + "attn.to_out.0.bias", (D,)),
            (p + "ff.ff.0.0.weight", (F, D)), (p + "ff.ff.0.0.bias", (F,)),
            (p + "ff.ff.2.weight", (D, F)), (p + "ff.ff.2.bias", (D,)),
        ]
    out += [
        ("norm_out.linear.weight", (2 * D, D)),
        ("norm_out.linear.bias", (2 * D,)),
        ("proj_out.weight", (mel, D)),
        ("proj_out.bias", (mel,)),
    ]
    return out


_BLOCK_KEYS = {
    "attn_norm_w": "attn_norm.linear.weight", "attn_norm_b": "attn_norm.linear.bias",
    "to_q_w": "attn.to_q.weight", "to_q_b": "attn.to_q.bias",
    "to_k_w": "attn.to_k.weight", "to_k_b": "attn.to_k.bias",
    "to_v_w": "attn.to_v.weight", "to_v_b": "attn.to_v.bias",
    "to_out_w": "attn.to_out.0.weight", "to_out_b": "attn.to_out.0.bias",
    "ff0_w": "ff.ff.0.0.weight", "ff0_b": "ff.ff.0.0.bias",
    "ff2_w": "ff.ff.2.weight", "ff2_b": "ff.ff.2.bias",
}


def _ptr(params, name, shape):
    t = params[name]
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)} != {tuple(shape)}")
    if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise ValueError(f"{name}: must be a contiguous CUDA float32 tensor")
    return C.c_void_p(t.data_ptr())


_TOP_KEYS = {
    "time_mlp_0_w": "time_embed.time_mlp.0.weight",
    "time_mlp_0_b": "time_embed.time_mlp.0.bias",
    "time_mlp_2_w": "time_embed.time_mlp.2.weight",
    "time_mlp_2_b": "time_embed.time_mlp.2.bias",
    "input_proj_w": "input_embed.proj.weight",
    "input_proj_b": "input_embed.proj.bias",
    "conv_pos_1_w": "input_embed.conv_pos_embed.conv1.0.weight",
    "conv_pos_1_b": "input_embed.conv_pos_embed.conv1.0.bias",
    "conv_pos_2_w": "input_embed.conv_pos_embed.conv2.0.weight",
    "conv_pos_2_b": "input_embed.conv_pos_embed.conv2.0.bias",
    "norm_out_w": "norm_out.linear.weight",
    "norm_out_b": "norm_out.linear.bias",
    "proj_out_w": "proj_out.weight",
    "proj_out_b": "proj_out.bias",
}


def _dit_weights(params, cfg):
    """lx_dit_weights over a dict of CUDA tensors (the block array is kept
    alive as an attribute of the returned struct)."""
    shapes = dict(dit_param_shapes(cfg))
    blocks = (DitBlockWeights * cfg.depth)()
    for i in range(cfg.depth):
        for field, key in _BLOCK_KEYS.items():
            name = f"transformer_blocks.{i}.{key}"
            setattr(blocks[i], field, _ptr(params, name, shapes[name]))
    w = DitWeights()
    w.dim, w.depth, w.heads, w.head_dim = cfg.dim, cfg.depth, cfg.heads, cfg.head_dim
    w.ff_inner, w.mel_dim = cfg.ff_inner, cfg.mel_dim
    for field, name in _TOP_KEYS.items():
        setattr(w, field, _ptr(params, name, shapes[name]))
    w.blocks = blocks
    w._keep = blocks
    return w


class DiTEstimator:
    """Device-resident DiT estimator for batches of B rows and up to max_T frames.

    `params` maps dit_param_shapes() names to CUDA fp32 tensors; they are copied
    (and re-packed) into library-owned memory at construction.
    """

    def __init__(self, params, cfg: DiTConfig = DiTConfig(), B: int = 2, max_T: int = 500):
        self.cfg, self.B, self.max_T = cfg, B, max_T
        w = _dit_weights(params, cfg)
        torch.cuda.synchronize()  # parameters must be materialised before the copy stream
        h = C.c_void_p()
        check(lib.lx_dit_create(C.byref(w), B, max_T, C.byref(h)))
        self._h = h
        self._capture = None

    def close(self):
        if getattr(self, "_h", None):
            lib.lx_dit_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone already
            pass

    @property
    def handle(self):
        return self._h

    def set_capture(self, capture):
        """capture: dict with any of time_embed, input_proj, conv_pos, input_embed, blocks,
        norm_out -> preallocated CUDA tensors (FlowDebug, include/larynx/flow/flow.h:15-34);
        None disables."""
        cap = DitCapture()
        if capture:
            for k, v in capture.items():
                setattr(cap, k, C.c_void_p(v.data_ptr()))
        self._capture = capture
        check(lib.lx_dit_set_capture(self._h, C.byref(cap)))

    def set_products(self, products):
        """Split-operand products of the block projections: 3 (the default, about
        5e-6 relative error per projection) or 6 (fp32-GEMM level, slower)."""
        check(lib.lx_dit_set_products(self._h, int(products)))

    def forward(self, x, mu, cond, spks, t):
        """dphi = DiT(x, mu, t, spks, cond); x/mu/cond (B, mel, T), spks (B, mel), t (B)."""
        B, mel, T = x.shape
        if B != self.B or mel != self.cfg.mel_dim:
            raise ValueError(f"x shape {tuple(x.shape)} does not match B={self.B} mel={mel}")
        dphi = torch.empty_like(x)
        check(lib.lx_dit_forward(self._h, x.data_ptr(), mu.data_ptr(), cond.data_ptr(),
                                 spks.data_ptr(), t.data_ptr(), dphi.data_ptr(), T, stream()))
        return dphi

    def cfm_step(self, x, mu, cond, spks, t, dt, cfg_rate=None):
        """One Euler step with CFG on x (mel, T) in place."""
        cfg_rate = self.cfg.cfg_rate if cfg_rate is None else cfg_rate
        T = x.shape[-1]
        check(lib.lx_cfm_step(self._h, x.data_ptr(), mu.data_ptr(), cond.data_ptr(),
                              spks.data_ptr(), T, float(t), float(dt), float(cfg_rate), stream()))
        return x

    def cfm_solve(self, z, mu, cond, spks, n_steps=None, cfg_rate=None):
        """CausalConditionalCFM.solve_euler from noise z (mel, T); returns the solution."""
        n_steps = self.cfg.n_timesteps if n_steps is None else n_steps
        cfg_rate = self.cfg.cfg_rate if cfg_rate is None else cfg_rate
        x = z.clone()
        T = x.shape[-1]
        check(lib.lx_cfm_solve(self._h, x.data_ptr(), mu.data_ptr(), cond.data_ptr(),
                               spks.data_ptr(), T, n_steps, float(cfg_rate), stream()))
        return x


@dataclass(frozen=True)
class FlowConfig:
    """Frontend constants of src/flow/internal.h:19-29 (cosyvoice3.yaml)."""
    vocab: int = 6561
    spk_in: int = 192
    channels: int = 1024
    pre_lookahead: int = 3
    token_mel_ratio: int = 2


def flow_frontend_param_shapes(cfg: DiTConfig = DiTConfig(), fcfg: FlowConfig = FlowConfig()):
    """Ordered (name, shape) list of the frontend parameters (torch layouts;
    the GGUF names of src/flow/gguf.cpp:45-53)."""
    mel = cfg.mel_dim
    return [
        ("input_embedding.weight", (fcfg.vocab, mel)),
        ("spk_embed_affine_layer.weight", (mel, fcfg.spk_in)),
        ("spk_embed_affine_layer.bias", (mel,)),
        ("pre_lookahead_layer.conv1.weight", (fcfg.channels, mel, fcfg.pre_lookahead + 1)),
        ("pre_lookahead_layer.conv1.bias", (fcfg.channels,)),
        ("pre_lookahead_layer.conv2.weight", (mel, fcfg.channels, 3)),
        ("pre_lookahead_layer.conv2.bias", (mel,)),
    ]


_FRONT_FIELDS = {
    "input_embedding": "input_embedding.weight",
    "spk_affine_w": "spk_embed_affine_layer.weight",
    "spk_affine_b": "spk_embed_affine_layer.bias",
    "pre_conv1_w": "pre_lookahead_layer.conv1.weight",
    "pre_conv1_b": "pre_lookahead_layer.conv1.bias",
    "pre_conv2_w": "pre_lookahead_layer.conv2.weight",
    "pre_conv2_b": "pre_lookahead_layer.conv2.bias",
}


class FlowDecoder:
    """FlowDecoder (include/larynx/flow/flow.h:37-82) on liblxops: the frontend
    (speaker affine, token embedding, PreLookaheadLayer, mel-rate mu and prompt
    cond), then the 10-step CFG Euler solve of the 22-block estimator.

    `front_params` maps flow_frontend_param_shapes() names and `dit_params`
    dit_param_shapes() names to CUDA fp32 tensors (copied at construction).
    """

    def __init__(self, front_params, dit_params, cfg: DiTConfig = DiTConfig(),
                 fcfg: FlowConfig = FlowConfig(), max_tokens: int = 250):
        self.cfg, self.fcfg, self.max_tokens = cfg, fcfg, max_tokens
        dw = _dit_weights(dit_params, cfg)
        shapes = dict(flow_frontend_param_shapes(cfg, fcfg))
        fw = FlowFrontendWeights()
        fw.vocab, fw.spk_in, fw.channels = fcfg.vocab, fcfg.spk_in, fcfg.channels
        for field, name in _FRONT_FIELDS.items():
            setattr(fw, field, _ptr(front_params, name, shapes[name]))
        torch.cuda.synchronize()
        h = C.c_void_p()
        check(lib.lx_flow_create(C.byref(dw), C.byref(fw), max_tokens, C.byref(h)))
        self._h = h
        self._capture = None

    @classmethod
    def load(cls, path, max_tokens: int = 250):
        """FlowDecoder::load: a flow.gguf checkpoint (geometry from its tensors)."""
        from .gguf import GgufFile
        hdr = GgufFile(path, device=False)
        shape = {n: s for n, _, s, _ in hdr.tensors()}
        hdr.close()
        E = "decoder.estimator."
        depth = 0
        while f"{E}transformer_blocks.{depth}.attn_norm.linear.weight" in shape:
            depth += 1
        vocab, mel = shape.get("input_embedding.weight", (0, 0))
        dim = shape.get(E + "input_embed.proj.weight", (0, 0))[0]
        ff = shape.get(E + "transformer_blocks.0.ff.ff.0.0.weight", (0, 0))[0]
        cfg = DiTConfig(dim=dim, depth=depth, heads=max(dim // 64, 1), ff_inner=ff, mel_dim=mel)
        fcfg = FlowConfig(vocab=vocab,
                          spk_in=shape.get("spk_embed_affine_layer.weight", (0, 0))[1],
                          channels=shape.get("pre_lookahead_layer.conv1.weight", (0,))[0])
        self = cls.__new__(cls)
        self.cfg, self.fcfg, self.max_tokens = cfg, fcfg, max_tokens
        h = C.c_void_p()
        check(lib.lx_flow_load(str(path).encode(), max_tokens, C.byref(h)))
        self._h = h
        self._capture = None
        return self

    def close(self):
        if getattr(self, "_h", None):
            lib.lx_flow_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone already
            pass

    def set_capture(self, capture):
        """capture: dict with any of spk, token_embed, prelookahead, mu, cond ->
        preallocated CUDA tensors (FlowDebug, include/larynx/flow/flow.h:15-22)."""
        cap = FlowCapture()
        if capture:
            for k, v in capture.items():
                setattr(cap, k, C.c_void_p(v.data_ptr()))
        self._capture = capture
        check(lib.lx_flow_set_capture(self._h, C.byref(cap)))

    def set_products(self, products):
        """Split-operand products of the estimator's block projections (3 or 6)."""
        check(lib.lx_dit_set_products(lib.lx_flow_estimator(self._h), int(products)))

    def infer(self, prompt_tokens, tokens, prompt_feat, spk_embedding, noise_z):
        """Speech tokens -> mel frames past the prompt, (mel, MEL_T - mel_len1).

        prompt_tokens / tokens: int sequences (host); prompt_feat (mel_len1, mel),
        spk_embedding (spk_in,), noise_z (mel, MEL_T): CUDA fp32 tensors, with
        MEL_T = token_mel_ratio * (len(prompt_tokens) + len(tokens))."""
        import numpy as np
        pt = np.ascontiguousarray(prompt_tokens, dtype=np.int32)
        tk = np.ascontiguousarray(tokens, dtype=np.int32)
        mel = self.cfg.mel_dim
        MT = self.fcfg.token_mel_ratio * (len(pt) + len(tk))
        pf = prompt_feat.reshape(-1, mel)
        if tuple(noise_z.shape[-2:]) != (mel, MT) or noise_z.numel() != mel * MT:
            raise ValueError(f"noise_z {tuple(noise_z.shape)} must be ({mel}, {MT})")
        if spk_embedding.numel() != self.fcfg.spk_in:
            raise ValueError(f"spk_embedding must have {self.fcfg.spk_in} values")
        for t in (pf, spk_embedding, noise_z):
            if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
                raise ValueError("prompt_feat, spk_embedding and noise_z must be contiguous "
                                 "CUDA float32 tensors")
        out = torch.empty(mel, MT - pf.shape[0], device=noise_z.device, dtype=torch.float32)
        check(lib.lx_flow_infer(self._h, C.c_void_p(pt.ctypes.data), len(pt),
                                C.c_void_p(tk.ctypes.data), len(tk), C.c_void_p(pf.data_ptr()),
                                pf.shape[0], C.c_void_p(spk_embedding.data_ptr()),
                                C.c_void_p(noise_z.data_ptr()), C.c_void_p(out.data_ptr()),
                                stream()))
        return out


def cfm_t_span(n_steps=10):
    """t_span = 1 - cos(linspace(0,1,n+1) pi/2) as src/flow/flow.cpp:203-207 forms it."""
    import numpy as np
    pi = np.float32(3.14159265358979323846)
    out = []
    for i in range(n_steps + 1):
        tt = np.float32(i) / np.float32(n_steps)
        out.append(np.float32(1.0) - np.float32(np.cos(np.float32(tt * np.float32(0.5) * pi))))
    return out
