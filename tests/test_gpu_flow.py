"""FlowDecoder::infer parity on the GPU (frontend + estimator + CFM solve).

- the reference's validation case (4 prompt + 8 tokens, one negative id, 8
  prompt frames -> 16 output frames) against the golden vectors written from
  the reference's own modules: every frontend stage (FlowDebug captures) and
  the final mel;
- a 10 s utterance (250 tokens -> 500 mel frames, 100 prompt frames) against
  the oracle: frontend stages at 1e-4, the mel after 10 Euler steps of the
  22-block estimator at 1e-3;
- error paths: an id past the table, a prompt as long as the utterance, more
  tokens than the decoder was built for.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL_22 = 1e-3


def to_dev(params, gpu):
    return {k: torch.from_numpy(v).to(gpu) for k, v in params.items()}


def front_params(seed):
    from larynx_amd.flow import DiTConfig, flow_frontend_param_shapes
    p = orc.make_params(flow_frontend_param_shapes(DiTConfig()), seed)
    p["input_embedding.weight"] = orc.normal((6561, 80), seed, 100)
    return p


@pytest.fixture(scope="module")
def flow_setup(gpu):
    from larynx_amd.flow import DiTConfig, FlowDecoder, dit_param_shapes
    g = np.load(os.path.join(GOLDEN, "flow_infer_T24.npz"))
    dparams = orc.make_params(dit_param_shapes(DiTConfig()), int(g["weight_seed"]))
    fparams = front_params(int(g["front_seed"]))
    dec = FlowDecoder(to_dev(fparams, gpu), to_dev(dparams, gpu), max_tokens=250)
    yield g, dparams, fparams, dec
    dec.close()


def test_flow_infer_golden_T24(gpu, flow_setup):
    g, _, _, dec = flow_setup
    announce("flow infer golden (4 + 8 tokens, 24 mel frames)")
    Tseq, MT = 12, 24
    cap = {"spk": torch.empty(80, device=gpu),
           "token_embed": torch.empty(Tseq, 80, device=gpu),
           "prelookahead": torch.empty(Tseq, 80, device=gpu),
           "mu": torch.empty(80, MT, device=gpu),
           "cond": torch.empty(80, MT, device=gpu)}
    dec.set_capture(cap)
    mel = dec.infer(g["prompt_tokens"], g["tokens"], torch.from_numpy(g["prompt_feat"]).to(gpu),
                    torch.from_numpy(g["spk_embedding"]).to(gpu),
                    torch.from_numpy(g["noise"]).to(gpu))
    torch.cuda.synchronize()
    dec.set_capture(None)
    assert orc.rel_err(cap["spk"].cpu().numpy(), g["spk"]) < 1e-4
    assert np.array_equal(cap["token_embed"].cpu().numpy(), g["token_embed"])  # bit-exact gather
    assert orc.rel_err(cap["prelookahead"].cpu().numpy(), g["prelookahead"]) < 1e-4
    assert orc.rel_err(cap["mu"].cpu().numpy(), g["mu"]) < 1e-4
    assert np.array_equal(cap["cond"].cpu().numpy(), g["cond"])
    assert tuple(mel.shape) == (80, 16)
    assert orc.rel_err(mel.cpu().numpy(), g["feat"]) < TOL_22


def test_flow_infer_T500_vs_oracle(gpu, flow_setup):
    _, dparams, fparams, dec = flow_setup
    announce("flow infer 250 tokens (500 mel frames) vs oracle")
    rng = np.random.default_rng(11)
    prompt_tokens = rng.integers(0, 6561, 50).astype(np.int32)
    tokens = rng.integers(-2, 6561, 200).astype(np.int32)  # a few negatives: clamped to 0
    prompt_feat = orc.normal((100, 80), 77, 1)
    spk = orc.normal((192,), 77, 2)
    noise = orc.normal((80, 500), 77, 3)
    flow = orc.Flow(fparams, dparams)
    ref_mel, ref_st = flow.infer(prompt_tokens, tokens, prompt_feat, spk, noise)
    cap = {"spk": torch.empty(80, device=gpu), "prelookahead": torch.empty(250, 80, device=gpu),
           "mu": torch.empty(80, 500, device=gpu), "cond": torch.empty(80, 500, device=gpu)}
    dec.set_capture(cap)
    mel = dec.infer(prompt_tokens, tokens, torch.from_numpy(prompt_feat).to(gpu),
                    torch.from_numpy(spk).to(gpu), torch.from_numpy(noise).to(gpu))
    torch.cuda.synchronize()
    dec.set_capture(None)
    assert orc.rel_err(cap["spk"].cpu().numpy(), ref_st["spk"]) < 1e-4
    assert orc.rel_err(cap["prelookahead"].cpu().numpy(), ref_st["prelookahead"]) < 1e-4
    assert orc.rel_err(cap["mu"].cpu().numpy(), ref_st["mu"]) < 1e-4
    assert np.array_equal(cap["cond"].cpu().numpy(), ref_st["cond"])
    assert tuple(mel.shape) == (80, 400)
    assert orc.rel_err(mel.cpu().numpy(), ref_mel) < TOL_22


def test_flow_infer_errors(gpu, flow_setup):
    from larynx_amd._lib import LX_ERR_ARG, LX_ERR_RANGE, LxError
    g, _, _, dec = flow_setup
    announce("flow infer error paths")
    pf = torch.from_numpy(g["prompt_feat"]).to(gpu)
    spk = torch.from_numpy(g["spk_embedding"]).to(gpu)
    noise = torch.from_numpy(g["noise"]).to(gpu)
    with pytest.raises(LxError) as e:
        dec.infer([1, 2, 3, 4], [5, 6, 6561, 7, 8, 9, 10, 11], pf, spk, noise)
    assert e.value.code == LX_ERR_RANGE
    with pytest.raises(LxError) as e:  # 24 prompt frames leave no output frame
        dec.infer([1, 2, 3, 4], [5, 6, 7, 8, 9, 10, 11, 12],
                  torch.zeros(24, 80, device=gpu), spk, noise)
    assert e.value.code == LX_ERR_ARG
    big = torch.zeros(80, 502, device=gpu)
    with pytest.raises(LxError) as e:  # 251 tokens, built for 250
        dec.infer(list(range(51)), list(range(200)), pf, spk, big)
    assert e.value.code == LX_ERR_ARG
    # the decoder still works after rejected calls
    mel = dec.infer(g["prompt_tokens"], g["tokens"], pf, spk, noise)
    torch.cuda.synchronize()
    assert orc.rel_err(mel.cpu().numpy(), g["feat"]) < TOL_22
