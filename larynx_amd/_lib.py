"""ctypes binding of liblxops.so (the C-ABI declared in include/lx_ops.h).

The library is loaded from the package directory.  There is no fallback: if
the shared object is missing or fails to load, importing this module raises,
so nothing can silently run on another code path.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblxops.so")

LX_OK = 0
LX_ERR_ARG = -1
LX_ERR_LAUNCH = -2
LX_ERR_RANGE = -3
LX_ERR_ALLOC = -4
LX_ERR_STATE = -5

LX_GGUF_HOST_ONLY = 1

LX_EPI_NONE = 0
LX_EPI_GELU_TANH = 1
LX_EPI_GATED_RESID = 2
LX_EPI_ROPE_PARTIAL = 3
LX_EPI_RESID = 4
LX_EPI_SWIGLU_PAIRED = 5

LX_BX_OUT_F32 = 0
LX_BX_OUT_PARTIAL = 1
LX_BX_OUT_PACKED = 2

fp = C.c_void_p  # device pointer
ip = C.c_void_p
stream_t = C.c_void_p


class LxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"liblxops error {code}: {msg}")
        self.code = code


class Epilogue(C.Structure):
    _fields_ = [
        ("kind", C.c_int),
        ("rows_per_batch", C.c_int),
        ("gate", fp),
        ("gate_stride", C.c_long),
        ("pos", ip),
        ("rot_dim", C.c_int),
        ("rope_section", C.c_int),
        ("rope_sections", C.c_int),
        ("rope_base", C.c_float),
    ]


class LinearBx(C.Structure):
    _fields_ = [
        ("A", fp), ("lda", C.c_long), ("Wf", C.c_void_p), ("bias", fp),
        ("epi", C.POINTER(Epilogue)), ("out", C.c_int), ("Y", fp), ("ldy", C.c_long),
        ("slice_stride", C.c_long), ("M", C.c_int), ("N", C.c_int), ("K", C.c_int),
        ("bm", C.c_int), ("slices", C.c_int), ("ws", fp), ("ws_floats", C.c_size_t),
        ("counters", C.c_void_p), ("n_counters", C.c_int), ("products", C.c_int),
        ("a_packed", C.c_int), ("pack_from", C.c_int), ("split_tail", C.c_int),
    ]


_DIT_BLOCK_FIELDS = [
    "attn_norm_w", "attn_norm_b", "to_q_w", "to_q_b", "to_k_w", "to_k_b", "to_v_w", "to_v_b",
    "to_out_w", "to_out_b", "ff0_w", "ff0_b", "ff2_w", "ff2_b",
]


class DitBlockWeights(C.Structure):
    _fields_ = [(n, fp) for n in _DIT_BLOCK_FIELDS]


class DitWeights(C.Structure):
    _fields_ = [
        ("dim", C.c_int), ("depth", C.c_int), ("heads", C.c_int), ("head_dim", C.c_int),
        ("ff_inner", C.c_int), ("mel_dim", C.c_int),
        ("time_mlp_0_w", fp), ("time_mlp_0_b", fp), ("time_mlp_2_w", fp), ("time_mlp_2_b", fp),
        ("input_proj_w", fp), ("input_proj_b", fp),
        ("conv_pos_1_w", fp), ("conv_pos_1_b", fp), ("conv_pos_2_w", fp), ("conv_pos_2_b", fp),
        ("blocks", C.POINTER(DitBlockWeights)),
        ("norm_out_w", fp), ("norm_out_b", fp), ("proj_out_w", fp), ("proj_out_b", fp),
    ]


class DitCapture(C.Structure):
    _fields_ = [(n, fp) for n in
                ("time_embed", "input_proj", "conv_pos", "input_embed", "blocks", "norm_out")]


class FlowFrontendWeights(C.Structure):
    _fields_ = [("vocab", C.c_int), ("spk_in", C.c_int), ("channels", C.c_int)] + [
        (n, fp) for n in ("input_embedding", "spk_affine_w", "spk_affine_b", "pre_conv1_w",
                          "pre_conv1_b", "pre_conv2_w", "pre_conv2_b")]


class FlowCapture(C.Structure):
    _fields_ = [(n, fp) for n in ("spk", "token_embed", "prelookahead", "mu", "cond")]


_QWEN_LAYER_FIELDS = ["q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "gate_w", "up_w",
                      "down_w", "in_norm", "post_norm"]


class Qwen2LayerWeights(C.Structure):
    _fields_ = [(n, fp) for n in _QWEN_LAYER_FIELDS]


class Qwen2Weights(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("intermediate", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("n_layers", C.c_int),
        ("text_vocab", C.c_int), ("speech_vocab", C.c_int),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("embed_tokens", fp), ("speech_embedding", fp), ("final_norm", fp), ("llm_decoder", fp),
        ("layers", C.POINTER(Qwen2LayerWeights)),
    ]


# (name, restype, argtypes) for every symbol of include/lx_ops.h
SIGNATURES = [
    ("lx_version", C.c_char_p, []),
    ("lx_last_error", C.c_char_p, []),
    ("lx_adaln_modulate_f32", C.c_int,
     [fp, fp, fp, C.c_long, fp, C.c_int, C.c_int, C.c_int, C.c_float, stream_t]),
    ("lx_adaln_resid_f32", C.c_int,
     [fp, fp, C.c_int, C.c_long, fp, fp, C.c_long, fp, fp, C.c_long, fp, C.c_int, C.c_int,
      C.c_int, C.c_float, stream_t]),
    ("lx_adaln_resid_packed_f32", C.c_int,
     [fp, fp, C.c_int, C.c_long, fp, fp, C.c_long, fp, fp, C.c_long, fp, C.c_int, C.c_int,
      C.c_int, C.c_float, stream_t]),
    ("lx_adaln_emb_f32", C.c_int, [fp, fp, fp, fp, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_rope_partial_interleaved_f32", C.c_int,
     [fp, fp, ip, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, stream_t]),
    ("lx_gelu_tanh_f32", C.c_int, [fp, fp, C.c_long, stream_t]),
    ("lx_gated_residual_f32", C.c_int,
     [fp, fp, fp, C.c_long, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_timestep_embed_f32", C.c_int, [fp, C.c_int, C.c_int, C.c_float, fp, stream_t]),
    ("lx_time_mlp_f32", C.c_int, [fp, C.c_int, fp, fp, fp, fp, C.c_int, fp, fp, stream_t]),
    ("lx_time_mlp_f32_noalloc", C.c_int, [fp, C.c_int, fp, fp, fp, fp, C.c_int, fp, stream_t]),
    ("lx_rmsnorm_f32", C.c_int, [fp, fp, fp, C.c_int, C.c_int, C.c_float, stream_t]),
    ("lx_rope_neox_f32", C.c_int,
     [fp, ip, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, stream_t]),
    ("lx_swiglu_f32", C.c_int, [fp, fp, fp, C.c_long, stream_t]),
    ("lx_embed_gather_f32", C.c_int,
     [fp, C.c_long, C.c_int, C.POINTER(C.c_int), C.c_int, fp, stream_t]),
    ("lx_linear_f32", C.c_int,
     [fp, C.c_int, fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(Epilogue),
      stream_t]),
    ("lx_split_planes_f32", C.c_int, [fp, C.c_void_p, C.c_long, stream_t]),
    ("lx_linear_split_f32", C.c_int,
     [fp, C.c_int, C.c_void_p, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int,
      C.POINTER(Epilogue), C.c_int, stream_t]),
    ("lx_wfrag_pack_f32", C.c_int, [fp, C.c_void_p, C.c_int, C.c_int, stream_t]),
    ("lx_linear_bx_f32", C.c_int, [C.POINTER(LinearBx), stream_t]),
    ("lx_attention_f32", C.c_int,
     [fp, C.c_int, fp, C.c_int, fp, C.c_int, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
      C.c_int, C.c_int, C.c_float, C.c_int, C.c_int, stream_t]),
    ("lx_attention_np_f32", C.c_int,
     [fp, C.c_int, fp, C.c_int, fp, C.c_int, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
      C.c_int, C.c_int, C.c_float, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_conv_pos_mish_f32", C.c_int,
     [fp, fp, fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_conv_pack_weight_f32", C.c_int, [fp, fp, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_conv_pos_mish_bx_f32", C.c_int,
     [fp, C.c_void_p, fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
      stream_t]),
    ("lx_conv_frag_pack_f32", C.c_int, [fp, C.c_void_p, C.c_int, C.c_int, C.c_int, stream_t]),
    ("lx_dit_create", C.c_int,
     [C.POINTER(DitWeights), C.c_int, C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_dit_destroy", None, [C.c_void_p]),
    ("lx_dit_forward", C.c_int, [C.c_void_p, fp, fp, fp, fp, fp, fp, C.c_int, stream_t]),
    ("lx_dit_set_capture", C.c_int, [C.c_void_p, C.POINTER(DitCapture)]),
    ("lx_dit_set_products", C.c_int, [C.c_void_p, C.c_int]),
    ("lx_cfm_solve", C.c_int,
     [C.c_void_p, fp, fp, fp, fp, C.c_int, C.c_int, C.c_float, stream_t]),
    ("lx_cfm_step", C.c_int,
     [C.c_void_p, fp, fp, fp, fp, C.c_int, C.c_float, C.c_float, C.c_float, stream_t]),
    ("lx_flow_create", C.c_int,
     [C.POINTER(DitWeights), C.POINTER(FlowFrontendWeights), C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_flow_destroy", None, [C.c_void_p]),
    ("lx_flow_estimator", C.c_void_p, [C.c_void_p]),
    ("lx_flow_set_capture", C.c_int, [C.c_void_p, C.POINTER(FlowCapture)]),
    ("lx_flow_infer", C.c_int,
     [C.c_void_p, ip, C.c_int, ip, C.c_int, fp, C.c_int, fp, fp, fp, stream_t]),
    ("lx_gguf_open", C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_gguf_close", None, [C.c_void_p]),
    ("lx_gguf_n_tensors", C.c_int, [C.c_void_p]),
    ("lx_gguf_find", C.c_int, [C.c_void_p, C.c_char_p]),
    ("lx_gguf_tensor_info", C.c_int,
     [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int),
      C.POINTER(C.c_int64), C.POINTER(C.c_uint64)]),
    ("lx_gguf_tensor_data", C.c_void_p, [C.c_void_p, C.c_int]),
    ("lx_gguf_get_string", C.c_char_p, [C.c_void_p, C.c_char_p]),
    ("lx_flow_load", C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_qwen2_load", C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_qwen2_create", C.c_int,
     [C.POINTER(Qwen2Weights), C.c_int, C.POINTER(C.c_void_p)]),
    ("lx_qwen2_destroy", None, [C.c_void_p]),
    ("lx_qwen2_build_lm_input", C.c_int,
     [C.c_void_p, C.POINTER(C.c_int), C.c_int, C.POINTER(C.c_int), C.c_int, fp,
      C.POINTER(C.c_int), stream_t]),
    ("lx_qwen2_prefill", C.c_int, [C.c_void_p, fp, C.c_int, fp, fp, fp, stream_t]),
    ("lx_qwen2_decode", C.c_int, [C.c_void_p, C.c_int, fp, fp, stream_t]),
    ("lx_qwen2_cache_len", C.c_int, [C.c_void_p]),
    ("lx_qwen2_cache_key", C.c_void_p, [C.c_void_p, C.c_int]),
    ("lx_qwen2_cache_value", C.c_void_p, [C.c_void_p, C.c_int]),
    ("lx_qwen2_set_cache_len", C.c_int, [C.c_void_p, C.c_int]),
    ("lx_qwen2_set_decode_graph", C.c_int, [C.c_void_p, C.c_int]),
    ("lx_qwen2_set_products", C.c_int, [C.c_void_p, C.c_int]),
]


def _load():
    # torch first: liblxops.so must bind to the HIP runtime torch already
    # carries (its bundled libamdhip64, soname libamdhip64.so.7), which the
    # dynamic linker then reuses.  Loaded the other way round, liblxops.so pulls
    # in the system copy and torch later loads its own beside it: two runtimes in
    # one process, and device allocations fail.
    import torch  # noqa: F401
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C larynx_amd/csrc`")
    lib = C.CDLL(LIB_PATH)
    for name, res, args in SIGNATURES:
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def check(rc):
    """Raise LxError for a non-zero status, with the library's message."""
    if rc != LX_OK:
        raise LxError(rc, lib.lx_last_error().decode(errors="replace"))
    return rc
