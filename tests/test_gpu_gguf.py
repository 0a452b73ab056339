"""Model loaders over GGUF v3 files on the GPU (FlowDecoder::load, LLM::load).

Checkpoints are written with the reference's tensor names and layout
(tests/gguf_writer.py); a model loaded from the file must give bit-identical
results to the same model built from the in-memory tensors, and a file with a
missing or mis-shaped tensor must be refused with a message naming it.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from gguf_writer import write_gguf
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def to_dev(params, gpu):
    return {k: torch.from_numpy(v).to(gpu) for k, v in params.items()}


@pytest.fixture(scope="module")
def flow_file(gpu, tmp_path_factory):
    from larynx_amd.flow import DiTConfig, dit_param_shapes, flow_frontend_param_shapes
    cfg = DiTConfig(depth=2)
    dit = orc.make_params(dit_param_shapes(cfg), 5150)
    front = orc.make_params(flow_frontend_param_shapes(cfg), 5151)
    front["input_embedding.weight"] = orc.normal((6561, 80), 5151, 100)
    path = tmp_path_factory.mktemp("gguf") / "flow.gguf"
    tensors = list(front.items()) + [("decoder.estimator." + k, v) for k, v in dit.items()]
    write_gguf(path, tensors, arch="cosyvoice3.flow")
    return cfg, dit, front, path


def test_flow_load_matches_in_memory_build(gpu, flow_file):
    from larynx_amd.flow import FlowDecoder
    cfg, dit, front, path = flow_file
    announce("flow.gguf load (2 blocks) vs in-memory build")
    a = FlowDecoder.load(path, max_tokens=64)
    assert a.cfg.depth == 2 and a.cfg.mel_dim == 80 and a.fcfg.vocab == 6561
    b = FlowDecoder(to_dev(front, gpu), to_dev(dit, gpu), cfg, max_tokens=64)
    rng = np.random.default_rng(3)
    pt, tk = rng.integers(0, 6561, 10), rng.integers(0, 6561, 30)
    pf = torch.from_numpy(orc.normal((20, 80), 8, 1)).to(gpu)
    spk = torch.from_numpy(orc.normal((192,), 8, 2)).to(gpu)
    z = torch.from_numpy(orc.normal((80, 80), 8, 3)).to(gpu)
    ma = a.infer(pt, tk, pf, spk, z)
    mb = b.infer(pt, tk, pf, spk, z)
    torch.cuda.synchronize()
    assert tuple(ma.shape) == (80, 60)
    assert torch.equal(ma, mb)
    a.close()
    b.close()


def test_flow_load_refuses_bad_files(gpu, flow_file, tmp_path):
    from larynx_amd._lib import LX_ERR_ARG, LxError
    from larynx_amd.flow import FlowDecoder
    cfg, dit, front, _ = flow_file
    announce("flow.gguf with a missing / mis-shaped tensor")
    drop = [(k, v) for k, v in front.items() if k != "pre_lookahead_layer.conv2.bias"]
    p1 = tmp_path / "missing.gguf"
    write_gguf(p1, drop + [("decoder.estimator." + k, v) for k, v in dit.items()])
    with pytest.raises(LxError) as e:
        FlowDecoder.load(p1)
    assert e.value.code == LX_ERR_ARG and "pre_lookahead_layer.conv2.bias" in str(e.value)
    bad = dict(dit)
    bad["transformer_blocks.1.attn.to_v.bias"] = np.zeros(1000, np.float32)
    p2 = tmp_path / "shape.gguf"
    write_gguf(p2, list(front.items()) + [("decoder.estimator." + k, v) for k, v in bad.items()])
    with pytest.raises(LxError) as e:
        FlowDecoder.load(p2)
    assert e.value.code == LX_ERR_ARG and "to_v.bias" in str(e.value)


def test_qwen2_load_matches_in_memory_build(gpu, tmp_path):
    from larynx_amd.llm import Qwen2Config, Qwen2LM, qwen2_param_shapes
    announce("llm.gguf load (2 layers) vs in-memory build")
    cfg = Qwen2Config(n_layers=2, text_vocab=1000)
    params = orc.make_params(qwen2_param_shapes(cfg), 6161)
    for k in params:
        if k.endswith("layernorm.weight") or k == "norm.weight":
            params[k] = (params[k] + 1.0).astype(np.float32)
    # the reference's llm.gguf names (src/llm/gguf.cpp:44-83)
    rename = {"embed_tokens.weight": "llm.model.model.embed_tokens.weight",
              "norm.weight": "llm.model.model.norm.weight"}
    tensors = [(rename.get(k, "llm.model.model." + k if k.startswith("layers.") else k), v)
               for k, v in params.items()]
    path = tmp_path / "llm.gguf"
    write_gguf(path, tensors, arch="cosyvoice3.llm")
    a = Qwen2LM.load(path, max_ctx=512)
    assert (a.cfg.n_layers, a.cfg.text_vocab, a.cfg.hidden) == (2, 1000, 896)
    dp = to_dev(params, gpu)
    b = Qwen2LM(dp, cfg, max_ctx=512)
    rng = np.random.default_rng(4)
    text, speech = rng.integers(0, 1000, 40), rng.integers(0, 6564, 20)
    ia, ib = a.build_lm_input(text, speech), b.build_lm_input(text, speech)
    assert torch.equal(ia, ib)
    la = a.prefill(ia)
    lb = b.prefill(ib)
    torch.cuda.synchronize()
    assert torch.equal(la, lb)
    for tok in (5, 6560):
        da = a.decode(tok)
        db = b.decode(tok)
        torch.cuda.synchronize()
        assert torch.equal(da, db)
    a.close()
    b.close()
