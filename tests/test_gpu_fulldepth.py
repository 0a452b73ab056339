"""Full-depth parity on the GPU against the oracle, at the configs' real sizes.

Qwen2-0.5B (24 layers, the 151936-row text table and the 6761-row speech
table, the reference's shapes; src/llm/internal.h:18-34):
- prefill at L = 256 over the build_lm_input layout [sos; 160 text ids; task;
  94 speech ids]: lm_input bit-exact, every layer's hidden state h0..h23, the
  final norm, the logits and all 48 KV-cache tensors (src/llm/llm.cpp:141-180;
  the reference's own checks tests/verify_llm.py:34-40);
- a 24-step decode trajectory after that prefill, each step fed the oracle's
  greedy token (the injected-token form of tests/verify_llm_decode_seq.py:
  97-107), with logits, final norm and argmax agreement at every step and the
  whole cache compared afterwards;
- decode through all 24 layers against synthetic caches of length 1, 256,
  1024 and 2048.

DiT estimator at the long-utterance size (B = 2, T = 3000, 22 blocks;
src/flow/dit.cpp:83-145): every block's residual stream, norm_out and dphi
against the oracle (the reference pins every block, tests/verify_flow.py:
37-50), with the CFG pair as the Euler loop forms it (row 1 with zero mu, cond
and spks, src/flow/flow.cpp:216-224).

Bars: gather bit-exact; 1e-4 relative (max|d| / max|ref|) for Qwen2 stages;
1e-3 relative after the 22-block estimator.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4
TOL_22 = 1e-3


@pytest.fixture(scope="module")
def qwen_full(gpu):
    from larynx_amd.llm import Qwen2Config, Qwen2LM, qwen2_param_shapes
    cfg = Qwen2Config()
    announce("qwen2 full geometry: generating 24-layer weights and full tables")
    params = orc.make_params(qwen2_param_shapes(cfg), 2024)
    for k in params:
        if k.endswith("layernorm.weight") or k == "norm.weight":
            params[k] = (params[k] + 1.0).astype(np.float32)
    dparams = {k: torch.from_numpy(v).to(gpu) for k, v in params.items()}
    lm = Qwen2LM(dparams, cfg, max_ctx=2304)
    yield cfg, params, dparams, lm
    lm.close()


def _prefill_inputs(cfg):
    rng = np.random.default_rng(2024)
    text = rng.integers(0, cfg.text_vocab, 160)   # uniform over the whole text table
    speech = rng.integers(0, 6564, 94)             # the config's speech id range
    return text, speech


def test_full_prefill_L256_and_decode_trajectory(gpu, qwen_full):
    cfg, params, _, lm = qwen_full
    text, speech = _prefill_inputs(cfg)
    announce("qwen2 24 layers: build_lm_input + prefill L=256")
    o = orc.Qwen2(params, cfg, cap=2304)
    lm_in = lm.build_lm_input(text, speech)
    ref_in = o.build_lm_input(text, speech)
    assert lm_in.shape == (256, cfg.hidden)
    assert np.array_equal(lm_in.cpu().numpy().view(np.uint32), ref_in.view(np.uint32))
    logits, hidden, final = lm.prefill(lm_in, capture=True)
    torch.cuda.synchronize()
    rl, rh, rf = o.prefill(ref_in, capture=True)
    errs = [orc.rel_err(hidden[i].cpu().numpy(), rh[i]) for i in range(cfg.n_layers)]
    print("hidden rel err per layer:", " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert max(errs) < TOL, errs
    e_final = orc.rel_err(final.cpu().numpy(), rf)
    e_logits = orc.rel_err(logits.cpu().numpy(), rl)
    print(f"final_norm {e_final:.2e} logits {e_logits:.2e}", flush=True)
    assert e_final < TOL and e_logits < TOL
    assert np.array_equal(logits.argmax(-1).cpu().numpy(), rl.argmax(-1))
    assert lm.cache_len == 256
    kv_errs = []
    for layer in range(cfg.n_layers):
        k, v = lm.cache_views(layer)
        kv_errs.append(orc.rel_err(k[:256].cpu().numpy(), o.k_cache[layer, :256]))
        kv_errs.append(orc.rel_err(v[:256].cpu().numpy(), o.v_cache[layer, :256]))
    print(f"kv cache (48 tensors) max rel err {max(kv_errs):.2e}", flush=True)
    assert max(kv_errs) < TOL, kv_errs

    # greedy trajectory: both sides are fed the oracle's argmax (injected tokens)
    tok = int(np.argmax(rl[-1]))
    worst = 0.0
    for step in range(24):
        announce(f"qwen2 24 layers: decode step {step} token {tok} at position {256 + step}")
        lg, fn = lm.decode(tok, final_norm=True)
        torch.cuda.synchronize()
        rlg, rfn = o.decode(tok)
        e = max(orc.rel_err(lg.cpu().numpy(), rlg), orc.rel_err(fn.cpu().numpy(), rfn))
        worst = max(worst, e)
        assert e < TOL, (step, e)
        assert int(lg.argmax()) == int(np.argmax(rlg)), step
        tok = int(np.argmax(rlg))
    print(f"decode trajectory (24 steps) worst rel err {worst:.2e}", flush=True)
    n = 256 + 24
    assert lm.cache_len == n
    for layer in range(cfg.n_layers):
        k, v = lm.cache_views(layer)
        assert orc.rel_err(k[:n].cpu().numpy(), o.k_cache[layer, :n]) < TOL, layer
        assert orc.rel_err(v[:n].cpu().numpy(), o.v_cache[layer, :n]) < TOL, layer


@pytest.mark.parametrize("cache_len", [1, 256, 1024, 2048])
def test_full_decode_against_synthetic_cache(gpu, qwen_full, cache_len):
    """The decode config at full depth: KV cache lengths 1..2048 with random
    ~N(0, 0.02) contents in all 24 layers."""
    cfg, params, _, lm = qwen_full
    announce(f"qwen2 24 layers: decode against a synthetic cache of {cache_len}")
    o = orc.Qwen2(params, cfg, cap=2304)
    for layer in range(cfg.n_layers):
        kc = orc.normal((cache_len, 128), 700 + layer, 1, 0.02)
        vc = orc.normal((cache_len, 128), 700 + layer, 2, 0.02)
        o.k_cache[layer, :cache_len] = kc
        o.v_cache[layer, :cache_len] = vc
        kd, vd = lm.cache_views(layer)
        kd[:cache_len].copy_(torch.from_numpy(kc))
        vd[:cache_len].copy_(torch.from_numpy(vc))
    o.cache_len = cache_len
    lm.set_cache_len(cache_len)
    torch.cuda.synchronize()
    for tok in (4321, 6561):
        lg, fn = lm.decode(tok, final_norm=True)
        torch.cuda.synchronize()
        rlg, rfn = o.decode(tok)
        assert orc.rel_err(fn.cpu().numpy(), rfn) < TOL
        assert orc.rel_err(lg.cpu().numpy(), rlg) < TOL
        assert int(lg.argmax()) == int(np.argmax(rlg))


@pytest.mark.timeout(900)
def test_dit_T3000_22_blocks_vs_oracle(gpu):
    """Long-utterance estimator: B = 2 (the CFG pair), T = 3000, 22 blocks."""
    from larynx_amd.flow import DiTConfig, DiTEstimator, dit_param_shapes
    cfg = DiTConfig()
    T, D = 3000, cfg.dim
    announce("dit T=3000 22 blocks: weights")
    params = orc.make_params(dit_param_shapes(cfg), 3000)
    dparams = {k: torch.from_numpy(v).to(gpu) for k, v in params.items()}
    est = DiTEstimator(dparams, cfg, B=2, max_T=T)
    x1 = orc.normal((80, T), 3001, 1)
    mu = np.zeros((2, 80, T), np.float32)
    cond = np.zeros((2, 80, T), np.float32)
    spks = np.zeros((2, 80), np.float32)
    mu[0] = orc.normal((80, T), 3001, 2)
    cond[0] = orc.normal((80, T), 3001, 3)
    spks[0] = orc.normal((80,), 3001, 4, 1.0 / np.sqrt(80.0))
    x = np.stack([x1, x1])
    t = np.array([0.42, 0.42], np.float32)
    cap = {"blocks": torch.empty(cfg.depth, 2, T, D, device=gpu),
           "norm_out": torch.empty(2, T, D, device=gpu)}
    est.set_capture(cap)
    announce("dit T=3000 22 blocks: device forward")
    dphi = est.forward(*(torch.from_numpy(a).to(gpu) for a in (x, mu, cond, spks, t)))
    torch.cuda.synchronize()
    est.set_capture(None)
    est.close()
    announce("dit T=3000 22 blocks: oracle forward")
    rcap = {"blocks": None, "norm_out": None}
    ref = orc.Dit(params).forward(x, mu, cond, spks, t, capture=rcap)
    errs = [orc.rel_err(cap["blocks"][i].cpu().numpy(), rcap["blocks"][i])
            for i in range(cfg.depth)]
    e_norm = orc.rel_err(cap["norm_out"].cpu().numpy(), rcap["norm_out"])
    e_dphi = orc.rel_err(dphi.cpu().numpy(), ref)
    print("block rel err:", " ".join(f"{e:.1e}" for e in errs), flush=True)
    print(f"norm_out {e_norm:.2e} dphi {e_dphi:.2e}", flush=True)
    assert max(errs) < TOL_22, errs
    assert e_norm < TOL_22 and e_dphi < TOL_22


@pytest.mark.timeout(900)
def test_cfm_solve_T3000_vs_oracle(gpu):
    """The long-utterance workload's whole CFM solve (src/flow/flow.cpp:240-274 at
    T = 3000): 10 CFG Euler steps on the cosine t-schedule, CFG rate 0.7, the CFG
    pair as B = 2, through a 2-block estimator, against the oracle's solve at the
    per-op bar."""
    from larynx_amd.flow import DiTConfig, DiTEstimator, dit_param_shapes
    cfg = DiTConfig(depth=2)
    T = 3000
    announce("cfm solve T=3000 2 blocks: weights")
    params = orc.make_params(dit_param_shapes(cfg), 3010)
    est = DiTEstimator({k: torch.from_numpy(v).to(gpu) for k, v in params.items()}, cfg, B=2,
                       max_T=T)
    z = orc.normal((80, T), 3011, 1)
    mu = orc.normal((80, T), 3011, 2)
    cond = orc.normal((80, T), 3011, 3)
    spks = orc.normal((80,), 3011, 4, 1.0 / np.sqrt(80.0))
    announce("cfm solve T=3000 2 blocks: device solve")
    feat = est.cfm_solve(*(torch.from_numpy(a).to(gpu) for a in (z, mu, cond, spks)),
                         n_steps=10, cfg_rate=0.7)
    torch.cuda.synchronize()
    est.close()
    announce("cfm solve T=3000 2 blocks: oracle solve")
    ref = orc.Dit(params, depth=2).cfm_solve(z, mu, cond, spks, n_steps=10, cfg_rate=0.7)
    err = orc.rel_err(feat.cpu().numpy(), ref)
    print(f"solve rel err {err:.2e}", flush=True)
    assert err < TOL
