"""Pins the oracle's composites (no GPU).

Flow: against the golden vectors that tests/golden/make_flow_golden.py wrote
from the reference's own PyTorch modules (tests/flow_reference.py of Larynx):
22-block DiT.forward at T=24, the 10-step CFG Euler solve, the whole
FlowDecoder inference with its frontend stages (speaker affine, token
embedding, PreLookaheadLayer, mu, cond), the rotary at T=3000 and the timestep
sinusoid.

Qwen2: against a transformers Qwen2Model built locally from a hand-written
config with the oracle's synthetic weights (an independent implementation of
the same layer: RMSNorm, NEOX rotary theta 1e6, GQA 7:1, SwiGLU), for prefill
and KV-cache decode.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import oracle as orc

from larynx_amd.flow import DiTConfig, dit_param_shapes, flow_frontend_param_shapes
from larynx_amd.llm import Qwen2Config, qwen2_param_shapes


@pytest.fixture(scope="module")
def dit_golden():
    g = np.load(os.path.join(GOLDEN, "flow_dit_T24.npz"))
    params = orc.make_params(dit_param_shapes(DiTConfig()), int(g["weight_seed"]))
    return g, orc.Dit(params)


def test_dit_forward_matches_reference_modules(dit_golden):
    g, dit = dit_golden
    cap = {"time_embed": None, "input_embed": None, "blocks": None, "norm_out": None}
    dphi = dit.forward(g["x"], g["mu"], g["cond"], g["spks"], g["t"], capture=cap)
    assert orc.rel_err(cap["time_embed"], g["time_embed"]) < 1e-5
    assert orc.rel_err(cap["input_embed"], g["input_embed"]) < 1e-5
    assert orc.rel_err(cap["blocks"][0], g["block0"]) < 1e-5
    assert orc.rel_err(cap["blocks"][21], g["block21"]) < 1e-5
    assert orc.rel_err(cap["norm_out"], g["norm_out"]) < 1e-5
    assert orc.rel_err(dphi, g["dphi"]) < 1e-5


def test_cfm_solve_matches_reference_modules(dit_golden):
    _, dit = dit_golden
    c = np.load(os.path.join(GOLDEN, "flow_cfm_T24.npz"))
    feat = dit.cfm_solve(c["z"][0], c["mu"][0], c["cond"][0], c["spks"][0], 10, 0.7)
    assert orc.rel_err(feat, c["feat"][0]) < 1e-5


def flow_front_params(g):
    """Frontend weights of flow_infer_T24.npz, regenerated from its seed."""
    front = orc.make_params(flow_frontend_param_shapes(DiTConfig()), int(g["front_seed"]))
    front["input_embedding.weight"] = orc.normal((6561, 80), int(g["front_seed"]), 100)
    return front


def test_flow_infer_matches_reference_modules(dit_golden):
    """CausalMaskedDiffWithDiT.inference: 4 prompt + 8 tokens (one negative id,
    clamped to 0), 8 prompt frames, 16 output frames; every frontend stage and
    the final mel against the reference's own modules."""
    _, dit = dit_golden
    g = np.load(os.path.join(GOLDEN, "flow_infer_T24.npz"))
    flow = orc.Flow(flow_front_params(g), None)
    flow.dit = dit
    mel, st = flow.infer(g["prompt_tokens"], g["tokens"], g["prompt_feat"], g["spk_embedding"],
                         g["noise"])
    assert orc.rel_err(st["spk"], g["spk"]) < 1e-6
    assert np.array_equal(st["token_embed"], g["token_embed"])  # a gather: bit-exact
    assert orc.rel_err(st["prelookahead"], g["prelookahead"]) < 1e-6
    assert orc.rel_err(st["mu"], g["mu"]) < 1e-6
    assert np.array_equal(st["cond"], g["cond"])  # a copy + zero pad
    assert mel.shape == (80, 16)
    assert orc.rel_err(mel, g["feat"]) < 1e-5


def test_flow_frontend_closed_forms():
    """Invariants the frontend math fixes, independently of the reference import:
    the speaker projection is scale-invariant (l2-normalised input) and an all-zero
    embedding hits the 1e-12 clamp (output = bias); PreLookahead with zero conv
    weights is the identity (residual only) plus the conv2 bias; a token's mu
    frames are its two repeats; cond is the transposed prompt then zeros."""
    rng = np.random.default_rng(5)
    mel, ch, spk_in, vocab = 80, 32, 192, 50
    p = {"input_embedding.weight": rng.standard_normal((vocab, mel)).astype(np.float32),
         "spk_embed_affine_layer.weight": rng.standard_normal((mel, spk_in)).astype(np.float32),
         "spk_embed_affine_layer.bias": rng.standard_normal(mel).astype(np.float32),
         "pre_lookahead_layer.conv1.weight": np.zeros((ch, mel, 4), np.float32),
         "pre_lookahead_layer.conv1.bias": np.zeros(ch, np.float32),
         "pre_lookahead_layer.conv2.weight": np.zeros((mel, ch, 3), np.float32),
         "pre_lookahead_layer.conv2.bias": rng.standard_normal(mel).astype(np.float32)}
    flow = orc.Flow(p, None)
    spk = rng.standard_normal(spk_in).astype(np.float32)
    pf = rng.standard_normal((3, mel)).astype(np.float32)
    a = flow.frontend([1, 2], [3, 4, 5], pf, spk)
    b = flow.frontend([1, 2], [3, 4, 5], pf, 7.0 * spk)
    assert np.abs(a["spk"] - b["spk"]).max() < 1e-5
    z = flow.frontend([1], [2], pf[:1], np.zeros(spk_in, np.float32))
    assert np.array_equal(z["spk"], p["spk_embed_affine_layer.bias"])
    ids = [1, 2, 3, 4, 5]
    emb = p["input_embedding.weight"][ids]
    np.testing.assert_allclose(a["prelookahead"], emb + p["pre_lookahead_layer.conv2.bias"],
                               rtol=0, atol=1e-6)
    assert np.array_equal(a["mu"][:, 0::2], a["prelookahead"].T)
    assert np.array_equal(a["mu"][:, 1::2], a["prelookahead"].T)
    assert np.array_equal(a["cond"][:, :3], pf.T) and not a["cond"][:, 3:].any()
    with pytest.raises(IndexError):
        flow.frontend([1], [vocab], pf[:1], spk)


def test_flow_prelookahead_matches_torch_conv():
    """PreLookahead against torch.nn.functional.conv1d / leaky_relu in float64 at a
    length where both paddings and interior frames matter."""
    import torch.nn.functional as F
    rng = np.random.default_rng(6)
    mel, ch, vocab, T = 80, 48, 40, 17
    p = {"input_embedding.weight": rng.standard_normal((vocab, mel)).astype(np.float32),
         "spk_embed_affine_layer.weight": np.zeros((mel, 192), np.float32),
         "spk_embed_affine_layer.bias": np.zeros(mel, np.float32),
         "pre_lookahead_layer.conv1.weight": (0.1 * rng.standard_normal((ch, mel, 4))).astype(np.float32),
         "pre_lookahead_layer.conv1.bias": (0.1 * rng.standard_normal(ch)).astype(np.float32),
         "pre_lookahead_layer.conv2.weight": (0.1 * rng.standard_normal((mel, ch, 3))).astype(np.float32),
         "pre_lookahead_layer.conv2.bias": (0.1 * rng.standard_normal(mel)).astype(np.float32)}
    ids = rng.integers(0, vocab, T)
    out = orc.Flow(p, None).frontend([], ids, np.zeros((0, mel), np.float32),
                                     np.ones(192, np.float32))
    x = torch.from_numpy(p["input_embedding.weight"][ids].T[None].astype(np.float64))
    w1 = torch.from_numpy(p["pre_lookahead_layer.conv1.weight"].astype(np.float64))
    b1 = torch.from_numpy(p["pre_lookahead_layer.conv1.bias"].astype(np.float64))
    w2 = torch.from_numpy(p["pre_lookahead_layer.conv2.weight"].astype(np.float64))
    b2 = torch.from_numpy(p["pre_lookahead_layer.conv2.bias"].astype(np.float64))
    y = F.leaky_relu(F.conv1d(F.pad(x, (0, 3)), w1, b1), 0.01)
    y = F.conv1d(F.pad(y, (2, 0)), w2, b2) + x
    assert orc.rel_err(out["prelookahead"], y[0].T.numpy()) < 1e-6
    # planted mistakes the pin must see: lookahead padding on the wrong side,
    # conv2 padded symmetrically, and the residual dropped
    bad1 = F.conv1d(F.pad(F.leaky_relu(F.conv1d(F.pad(x, (3, 0)), w1, b1), 0.01), (2, 0)), w2,
                    b2) + x
    bad2 = F.conv1d(F.pad(F.leaky_relu(F.conv1d(F.pad(x, (0, 3)), w1, b1), 0.01), (1, 1)), w2,
                    b2) + x
    for bad in (bad1, bad2, y - x):
        assert orc.rel_err(out["prelookahead"], bad[0].T.numpy()) > 1e-2


def test_rotary_T3000_matches_reference_modules():
    r = np.load(os.path.join(GOLDEN, "flow_rope_T3000.npz"))
    assert np.array_equal(orc.rope_inv_freq(10000.0, 64), r["inv_freq"])
    T = int(r["T"])
    q = orc.normal((1, T, 64), int(r["q_seed"]), int(r["q_stream"]))
    out = orc.rope_partial(q, np.arange(T, dtype=np.int32), 64, 10000.0)
    assert np.abs(out[0, r["sel"]] - r["out"]).max() < 1e-6


def test_sinusoid_matches_reference_modules():
    s = np.load(os.path.join(GOLDEN, "flow_sinus.npz"))
    out = orc.timestep_embed(s["t"])
    # |angle| <= 1000 rad: one fp32 ulp of the angle is 6e-5, torch's exp may
    # round the coefficient one ulp apart from expf.
    assert np.abs(out - s["out"]).max() < 2e-5


SMALL_QWEN = Qwen2Config(n_layers=2, text_vocab=1000)


@pytest.fixture(scope="module")
def qwen_pair():
    from transformers import Qwen2Config as HFConfig
    from transformers import Qwen2Model
    cfg = SMALL_QWEN
    params = orc.make_params(qwen2_param_shapes(cfg), 99)
    # RMSNorm weights around 1 so the check is not degenerate
    for k in params:
        if k.endswith("layernorm.weight") or k == "norm.weight":
            params[k] = (params[k] + 1.0).astype(np.float32)
    hf_cfg = HFConfig(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                      num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
                      num_hidden_layers=cfg.n_layers, rms_norm_eps=cfg.rms_eps,
                      rope_theta=cfg.rope_theta, vocab_size=cfg.text_vocab,
                      max_position_embeddings=4096, attn_implementation="eager",
                      use_sliding_window=False, tie_word_embeddings=True)
    hf = Qwen2Model(hf_cfg).double().eval()
    sd = {k: torch.from_numpy(v).double() for k, v in params.items()
          if k not in ("speech_embedding.weight", "llm_decoder.weight")}
    res = hf.load_state_dict(sd, strict=False)
    assert not res.unexpected_keys
    assert all("rotary_emb" in k for k in res.missing_keys), res.missing_keys
    return params, hf


def test_qwen2_prefill_and_decode_match_transformers(qwen_pair):
    params, hf = qwen_pair
    cfg = SMALL_QWEN
    o = orc.Qwen2(params, cfg, cap=64)
    rng = np.random.default_rng(3)
    text = rng.integers(0, cfg.text_vocab, 20).astype(np.int32)
    speech = rng.integers(0, 6561, 14).astype(np.int32)
    lm_input = o.build_lm_input(text, speech)
    L = lm_input.shape[0]
    assert L == 36
    # bit-exact assembly: [sos; text; task_id; speech] rows of the tables
    emb, sp = params["embed_tokens.weight"], params["speech_embedding.weight"]
    ref_in = np.concatenate([sp[[6561]], emb[text], sp[[6563]], sp[speech]])
    assert np.array_equal(lm_input, ref_in)

    logits, hidden, final = o.prefill(lm_input, capture=True)
    with torch.no_grad():
        out = hf(inputs_embeds=torch.from_numpy(lm_input).double()[None], use_cache=True,
                 output_hidden_states=True)
    hs = out.hidden_states
    assert orc.rel_err(hidden[0], hs[1][0].numpy()) < 2e-6
    assert orc.rel_err(final, out.last_hidden_state[0].numpy()) < 2e-6
    ref_logits = out.last_hidden_state[0].numpy() @ params["llm_decoder.weight"].astype(np.float64).T
    assert orc.rel_err(logits, ref_logits) < 2e-6

    # two decode steps through the KV cache
    past = out.past_key_values
    for step, tok in enumerate([123, 4567]):
        lg, fn = o.decode(tok)
        with torch.no_grad():
            e = torch.from_numpy(params["speech_embedding.weight"][tok]).double()[None, None]
            pos = torch.tensor([[L + step]])
            out = hf(inputs_embeds=e, past_key_values=past, use_cache=True, position_ids=pos)
        past = out.past_key_values
        assert orc.rel_err(fn, out.last_hidden_state[0, 0].numpy()) < 2e-6
        ref_lg = out.last_hidden_state[0, 0].numpy() @ params["llm_decoder.weight"].astype(
            np.float64).T
        assert orc.rel_err(lg, ref_lg) < 2e-6
