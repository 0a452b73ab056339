"""The boundary from C++: the reference's FlowDecoder and LLM interfaces
(include/larynx/flow/flow.h:39-82, include/larynx/llm/llm.h:31-104) bound to
liblxops in tests/cxx (compiled by build() into tests/cxx/libdropin.so against
include/lx_ops.h), driven in-process through the dump entry points that mirror
the reference's tests/flow_dump.cpp:86-136 and tests/llm_dump.cpp:59-100.

- FlowDecoder::load of a 22-block flow.gguf written with the reference's
  names, then infer of the reference's validation case with FlowDebug: the
  pre-DiT stages and the final mel against the golden vectors written from the
  reference's own modules, the DiT stages at CFM step 1 (time_embed,
  input_proj, conv_pos, input_embed, every block, norm_out, dphi) against the
  oracle;
- LLM::load of a 24-layer llm.gguf with the full tables, build_lm_input,
  prefill with LLMDebug (every hidden state, final norm, logits), 8 greedy
  decode steps and the cache read-back, against the oracle.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import GOLDEN, ROOT, announce
from gguf_writer import write_gguf
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
LIB = os.path.join(ROOT, "tests", "cxx", "libdropin.so")
TOL = 1e-4
TOL_22 = 1e-3

FLOW_FIELDS = ("spk", "token_embed", "prelookahead", "mu", "cond", "time_embed", "input_proj",
               "conv_pos", "input_embed", "blocks", "norm_out", "dphi", "feat")
LLM_FIELDS = ("lm_input", "hidden", "final_norm", "logits", "dec_logits", "dec_final_norm",
              "cache_k", "cache_v")


class FlowOut(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in FLOW_FIELDS]


class LlmOut(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in LLM_FIELDS] + [("L", C.c_int), ("cache_len", C.c_int)]


@pytest.fixture(scope="module")
def dropin(gpu):
    import larynx_amd  # noqa: F401  (torch, then liblxops.so: one HIP runtime)
    assert os.path.exists(LIB), "tests/cxx/libdropin.so is not built (make -C tests/cxx)"
    lib = C.CDLL(LIB)
    i32p = C.POINTER(C.c_int32)
    vp = C.c_void_p
    lib.dropin_flow_dump.restype = C.c_int
    lib.dropin_flow_dump.argtypes = [C.c_char_p, C.c_int, i32p, C.c_int, i32p, C.c_int, vp, C.c_int,
                                     vp, C.c_int, vp, C.c_int, C.POINTER(FlowOut)]
    lib.dropin_llm_dump.restype = C.c_int
    lib.dropin_llm_dump.argtypes = [C.c_char_p, C.c_int, i32p, C.c_int, i32p, C.c_int, i32p,
                                    C.c_int, C.POINTER(LlmOut)]
    return lib


def _i32(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(C.POINTER(C.c_int32))


def test_flow_decoder_from_cxx(gpu, dropin, tmp_path_factory):
    from larynx_amd.flow import DiTConfig, dit_param_shapes, flow_frontend_param_shapes
    g = np.load(os.path.join(GOLDEN, "flow_infer_T24.npz"))
    cfg = DiTConfig()
    announce("C++ FlowDecoder: writing a 22-block flow.gguf")
    dit = orc.make_params(dit_param_shapes(cfg), int(g["weight_seed"]))
    front = orc.make_params(flow_frontend_param_shapes(cfg), int(g["front_seed"]))
    front["input_embedding.weight"] = orc.normal((6561, 80), int(g["front_seed"]), 100)
    path = tmp_path_factory.mktemp("cxx") / "flow.gguf"
    write_gguf(path, list(front.items()) + [("decoder.estimator." + k, v) for k, v in dit.items()],
               arch="cosyvoice3.flow")
    Tseq, MT, D = 12, 24, cfg.dim
    mel_len1 = g["prompt_feat"].shape[0]
    shapes = {"spk": (80,), "token_embed": (Tseq, 80), "prelookahead": (Tseq, 80),
              "mu": (80, MT), "cond": (80, MT), "time_embed": (2, D), "input_proj": (2, MT, D),
              "conv_pos": (2, MT, D), "input_embed": (2, MT, D), "blocks": (cfg.depth, 2, MT, D),
              "norm_out": (2, MT, D), "dphi": (2, 80, MT), "feat": (80, MT - mel_len1)}
    res = {k: np.full(s, np.nan, np.float32) for k, s in shapes.items()}
    out = FlowOut(**{k: res[k].ctypes.data for k in FLOW_FIELDS})
    pt, ptp = _i32(g["prompt_tokens"])
    tk, tkp = _i32(g["tokens"])
    pf, spk, z = (orc.c32(g[k]) for k in ("prompt_feat", "spk_embedding", "noise"))
    announce("C++ FlowDecoder: load + infer with FlowDebug")
    rc = dropin.dropin_flow_dump(str(path).encode(), 64, ptp, len(pt), tkp, len(tk),
                                 pf.ctypes.data, mel_len1, spk.ctypes.data, spk.size,
                                 z.ctypes.data, MT, C.byref(out))
    os.remove(path)
    assert rc == 0
    # pre-DiT stages and the mel against the reference modules' goldens
    assert orc.rel_err(res["spk"], g["spk"]) < TOL
    assert np.array_equal(res["token_embed"], g["token_embed"])
    assert orc.rel_err(res["prelookahead"], g["prelookahead"]) < TOL
    assert orc.rel_err(res["mu"], g["mu"]) < TOL
    assert np.array_equal(res["cond"], g["cond"])
    assert orc.rel_err(res["feat"], g["feat"]) < TOL_22
    # DiT stages at CFM step 1 against the oracle over the same inputs
    x2 = np.stack([z, z])
    mu2 = np.stack([g["mu"], np.zeros_like(g["mu"])])
    cond2 = np.stack([g["cond"], np.zeros_like(g["cond"])])
    spks2 = np.stack([g["spk"], np.zeros_like(g["spk"])])
    cap = {k: None for k in ("time_embed", "input_proj", "conv_pos", "input_embed", "blocks",
                             "norm_out")}
    ref = orc.Dit(dit).forward(x2, mu2, cond2, spks2, np.zeros(2, np.float32), capture=cap)
    for k in ("time_embed", "input_proj", "conv_pos", "input_embed"):
        assert orc.rel_err(res[k], cap[k]) < TOL, k
    for i in range(cfg.depth):
        assert orc.rel_err(res["blocks"][i], cap["blocks"][i]) < TOL_22, i
    assert orc.rel_err(res["norm_out"], cap["norm_out"]) < TOL_22
    assert orc.rel_err(res["dphi"], ref) < TOL_22


def test_llm_from_cxx_full_geometry(gpu, dropin, tmp_path_factory):
    from larynx_amd.llm import Qwen2Config, qwen2_param_shapes
    cfg = Qwen2Config()
    announce("C++ LLM: writing a 24-layer llm.gguf with the full tables")
    params = orc.make_params(qwen2_param_shapes(cfg), 4242)
    for k in params:
        if k.endswith("layernorm.weight") or k == "norm.weight":
            params[k] = (params[k] + 1.0).astype(np.float32)
    rename = {"embed_tokens.weight": "llm.model.model.embed_tokens.weight",
              "norm.weight": "llm.model.model.norm.weight"}
    tensors = [(rename.get(k, "llm.model.model." + k if k.startswith("layers.") else k), v)
               for k, v in params.items()]
    path = tmp_path_factory.mktemp("cxx") / "llm.gguf"
    write_gguf(path, tensors, arch="cosyvoice3.llm")
    del tensors
    rng = np.random.default_rng(4242)
    text, tp = _i32(rng.integers(0, cfg.text_vocab, 160))
    speech, sp = _i32(rng.integers(0, 6564, 94))
    # the oracle first: its greedy tokens are the ones both sides decode
    o = orc.Qwen2(params, cfg, cap=512)
    ref_in = o.build_lm_input(text, speech)
    L = ref_in.shape[0]
    rl, rh, rf = o.prefill(ref_in, capture=True)
    n_dec = 8
    toks, rdl, rdf = [int(np.argmax(rl[-1]))], [], []
    for _ in range(n_dec):
        lg, fn = o.decode(toks[-1])
        rdl.append(lg)
        rdf.append(fn)
        toks.append(int(np.argmax(lg)))
    dec, dp = _i32(toks[:n_dec])
    H, V, KV, NL, n = cfg.hidden, cfg.speech_vocab, 128, cfg.n_layers, L + n_dec
    shapes = {"lm_input": (L, H), "hidden": (NL, L, H), "final_norm": (L, H), "logits": (L, V),
              "dec_logits": (n_dec, V), "dec_final_norm": (n_dec, H), "cache_k": (NL, n, KV),
              "cache_v": (NL, n, KV)}
    res = {k: np.full(s, np.nan, np.float32) for k, s in shapes.items()}
    out = LlmOut(**{k: res[k].ctypes.data for k in LLM_FIELDS})
    announce("C++ LLM: load, build_lm_input, prefill L=256, 8 decode steps")
    rc = dropin.dropin_llm_dump(str(path).encode(), 512, tp, len(text), sp, len(speech), dp,
                                n_dec, C.byref(out))
    os.remove(path)
    assert rc == 0 and out.L == L and out.cache_len == n
    assert np.array_equal(res["lm_input"].view(np.uint32), ref_in.view(np.uint32))
    for i in range(NL):
        assert orc.rel_err(res["hidden"][i], rh[i]) < TOL, i
    assert orc.rel_err(res["final_norm"], rf) < TOL
    assert orc.rel_err(res["logits"], rl) < TOL
    for i in range(n_dec):
        assert orc.rel_err(res["dec_logits"][i], rdl[i]) < TOL, i
        assert orc.rel_err(res["dec_final_norm"][i], rdf[i]) < TOL, i
        assert int(np.argmax(res["dec_logits"][i])) == toks[i + 1], i
    for layer in range(NL):
        assert orc.rel_err(res["cache_k"][layer], o.k_cache[layer, :n]) < TOL, layer
        assert orc.rel_err(res["cache_v"][layer], o.v_cache[layer, :n]) < TOL, layer
