#!/usr/bin/env python3
"""Writes the Flow golden vectors under tests/golden/ from the reference's own
PyTorch modules (Larynx tests/flow_reference.py), imported from
/root/reference in the build container only.

What is pinned here, and why an import is needed: the composed DiT.forward
(flow_reference.py:355-400), CausalConditionalCFM.solve_euler (:476-501), the
whole CausalMaskedDiffWithDiT inference with its frontend stages
(PreLookaheadLayer :406-431, manual_inference :597-665), and torch's exact fp32
rounding of SinusPositionEmbedding (:125-137) and RotaryEmbedding /
apply_rotary_pos_emb (:52-106).  Per-op semantics are pinned
by closed forms and library routines in tests/test_oracle_*.py instead.

Weights and inputs come from the oracle's counter-based generator
(oracle.normal(shape, seed, stream)), so the fixtures hold only seeds, small
inputs and outputs; the tests regenerate the weights bit-identically.

Usage (build container):  python tests/golden/make_flow_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
REF_TESTS = "/root/reference/tests"
sys.path.insert(0, REF_TESTS)

import flow_reference as fr  # noqa: E402  (reference module, build container only)

from larynx_amd.flow import DiTConfig, dit_param_shapes, flow_frontend_param_shapes  # noqa: E402
from oracle import oracle as orc  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
WEIGHT_SEED = 20260101
INPUT_SEED = 1234
FRONT_SEED = 20260202


def build_dit(cfg, seed):
    est = fr.DiT(dim=cfg.dim, depth=cfg.depth, heads=cfg.heads, dim_head=cfg.head_dim,
                 ff_mult=cfg.ff_inner / cfg.dim, mel_dim=cfg.mel_dim, mu_dim=cfg.mel_dim,
                 spk_dim=cfg.mel_dim, out_channels=cfg.mel_dim, static_chunk_size=50,
                 num_decoding_left_chunks=-1)
    params = orc.make_params(dit_param_shapes(cfg), seed)
    sd = {k: torch.from_numpy(v) for k, v in params.items()}
    res = est.load_state_dict(sd, strict=False)
    # inv_freq is a buffer the module computes itself (flow_reference.py:79-80)
    assert list(res.missing_keys) == ["rotary_embed.inv_freq"], res.missing_keys
    assert not res.unexpected_keys, res.unexpected_keys
    est.eval()
    return est


def dit_inputs(T, seed):
    x = orc.normal((2, 80, T), seed, 1)
    mu = orc.normal((2, 80, T), seed, 2)
    cond = orc.normal((2, 80, T), seed, 3)
    spks = orc.normal((2, 80), seed, 4) / np.sqrt(80.0)
    # classifier-free-guidance row: mu / cond / spks are zero (src/flow/flow.cpp:215-224)
    x[1] = x[0]
    mu[1] = 0.0
    cond[1] = 0.0
    spks[1] = 0.0
    return x.astype(np.float32), mu, cond, spks.astype(np.float32)


def main():
    torch.set_num_threads(8)
    cfg = DiTConfig()
    T = 24  # the reference's own validation length (flow_reference.py:42-47)
    est = build_dit(cfg, WEIGHT_SEED)
    x, mu, cond, spks = dit_inputs(T, INPUT_SEED)
    t = np.array([0.3, 0.3], dtype=np.float32)
    cap = {}
    with torch.no_grad():
        mask = torch.ones(2, 1, T)
        dphi = est(torch.from_numpy(x), mask, torch.from_numpy(mu), torch.from_numpy(t),
                   spks=torch.from_numpy(spks), cond=torch.from_numpy(cond), capture=cap)
    np.savez_compressed(
        os.path.join(OUT, "flow_dit_T24.npz"),
        weight_seed=np.int64(WEIGHT_SEED), input_seed=np.int64(INPUT_SEED),
        x=x, mu=mu, cond=cond, spks=spks, t=t,
        time_embed=cap["time_embed"].numpy(),
        input_embed=cap["input_embed"].numpy(),
        block0=cap["blocks"][0].numpy(),
        block21=cap["blocks"][21].numpy(),
        norm_out=cap["norm_out"].numpy(),
        dphi=dphi.numpy())
    print("flow_dit_T24.npz written")

    # 10-step CFM solve with CFG 0.7 (CausalConditionalCFM.solve_euler).
    cfm_params = fr._CFMParams()
    dec = fr.CausalConditionalCFM(in_channels=240, n_spks=1, spk_emb_dim=80,
                                  cfm_params=cfm_params, estimator=est)
    z = orc.normal((1, 80, T), INPUT_SEED, 10)
    mu1 = orc.normal((1, 80, T), INPUT_SEED, 11)
    cond1 = orc.normal((1, 80, T), INPUT_SEED, 12)
    spk1 = (orc.normal((1, 80), INPUT_SEED, 13) / np.sqrt(80.0)).astype(np.float32)
    t_span = torch.linspace(0, 1, 11, dtype=torch.float32)
    t_span = 1 - torch.cos(t_span * 0.5 * torch.pi)
    with torch.no_grad():
        feat = dec.solve_euler(torch.from_numpy(z), t_span=t_span, mu=torch.from_numpy(mu1),
                               mask=torch.ones(1, 1, T), spks=torch.from_numpy(spk1),
                               cond=torch.from_numpy(cond1))
    np.savez_compressed(os.path.join(OUT, "flow_cfm_T24.npz"),
                        weight_seed=np.int64(WEIGHT_SEED), z=z, mu=mu1, cond=cond1, spks=spk1,
                        t_span=t_span.numpy(), feat=feat.numpy())
    print("flow_cfm_T24.npz written")

    # Whole FlowDecoder inference (CausalMaskedDiffWithDiT.inference, finalize=True) through
    # the reference's step-by-step replica with stage captures (flow_reference.py:597-665):
    # the validation case of include/larynx/flow/flow.h:12-14 (4 prompt + 8 tokens -> 24 mel
    # frames, 8 prompt frames -> 16 output frames).  Frontend weights ~N(0, 0.02) except the
    # token embedding table ~N(0, 1); the CFM start noise replaces the module's seed bank.
    model = fr.CausalMaskedDiffWithDiT(
        input_size=80, output_size=80, spk_embed_dim=192, output_type="mel", vocab_size=fr.VOCAB,
        input_frame_rate=25, token_mel_ratio=2, pre_lookahead_len=3,
        pre_lookahead_layer=fr.PreLookaheadLayer(in_channels=80, channels=1024,
                                                 pre_lookahead_len=3),
        decoder=dec)
    front = orc.make_params(flow_frontend_param_shapes(cfg), FRONT_SEED)
    front["input_embedding.weight"] = orc.normal((fr.VOCAB, 80), FRONT_SEED, 100)
    res = model.load_state_dict({k: torch.from_numpy(v) for k, v in front.items()},
                                strict=False)
    assert not res.unexpected_keys, res.unexpected_keys
    assert all(k.startswith("decoder.") for k in res.missing_keys), res.missing_keys
    model.eval()
    prompt_tokens = np.array([[3, 1500, 6560, 42]], dtype=np.int64)
    tokens = np.array([[7, -1, 4095, 6000, 12, 0, 3333, 999]], dtype=np.int64)  # -1: clamp
    prompt_feat = orc.normal((1, 8, 80), INPUT_SEED, 30)
    spk_embedding = orc.normal((1, 192), INPUT_SEED, 31)
    noise = orc.normal((1, 80, 24), INPUT_SEED, 32)
    dec.rand_noise = torch.from_numpy(noise)
    cap = {}
    with torch.no_grad():
        feat = fr.manual_inference(model, torch.from_numpy(prompt_tokens),
                                   torch.from_numpy(tokens), torch.from_numpy(prompt_feat),
                                   torch.from_numpy(spk_embedding), cap)
        # the module's own inference() agrees with the step-by-step replica
        ref_feat, _ = model.inference(torch.from_numpy(tokens), torch.tensor([8]),
                                      torch.from_numpy(prompt_tokens), torch.tensor([4]),
                                      torch.from_numpy(prompt_feat), torch.tensor([8]),
                                      torch.from_numpy(spk_embedding), streaming=False,
                                      finalize=True)
    assert torch.allclose(feat, ref_feat, rtol=0, atol=1e-5), (feat - ref_feat).abs().max()
    np.savez_compressed(os.path.join(OUT, "flow_infer_T24.npz"),
                        weight_seed=np.int64(WEIGHT_SEED), front_seed=np.int64(FRONT_SEED),
                        prompt_tokens=prompt_tokens[0].astype(np.int32),
                        tokens=tokens[0].astype(np.int32), prompt_feat=prompt_feat[0],
                        spk_embedding=spk_embedding[0], noise=noise[0],
                        spk=cap["spk"][0].numpy(), token_embed=cap["token_embed"][0].numpy(),
                        prelookahead=cap["prelookahead"][0].numpy(), mu=cap["mu"][0].numpy(),
                        cond=cap["cond"][0].numpy(), feat=feat[0].numpy())
    print("flow_infer_T24.npz written")

    # Rotary at the long-utterance length: fp32 angle rounding matters at T=3000.
    T_long = 3000
    rot = fr.RotaryEmbedding(64)
    freqs, _ = rot.forward_from_seq_len(T_long)
    q = orc.normal((1, T_long, 64), INPUT_SEED, 20)
    with torch.no_grad():
        qr = fr.apply_rotary_pos_emb(torch.from_numpy(q), freqs, 1.0)
    sel = np.unique(np.concatenate([np.arange(10), np.arange(10, T_long, 97),
                                    np.arange(T_long - 10, T_long)])).astype(np.int64)
    np.savez_compressed(os.path.join(OUT, "flow_rope_T3000.npz"), q_seed=np.int64(INPUT_SEED),
                        q_stream=np.int64(20), T=np.int64(T_long), sel=sel,
                        inv_freq=rot.inv_freq.numpy(), freqs=freqs[0, sel].numpy(),
                        out=qr[0, sel].numpy())
    print("flow_rope_T3000.npz written")

    # Sinusoid at the cosine t_span points and a spread of t in [0, 1].
    ts = np.concatenate([t_span.numpy(), np.linspace(0, 1, 37, dtype=np.float32),
                         np.array([1e-3, 0.123456, 0.999], dtype=np.float32)]).astype(np.float32)
    with torch.no_grad():
        sin = fr.SinusPositionEmbedding(256)(torch.from_numpy(ts), scale=1000)
    np.savez_compressed(os.path.join(OUT, "flow_sinus.npz"), t=ts, out=sin.numpy())
    print("flow_sinus.npz written")


if __name__ == "__main__":
    main()
