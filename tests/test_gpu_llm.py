"""Qwen2 LM parity on the GPU against the oracle (which is itself pinned to
transformers' Qwen2Model in test_oracle_golden.py).

Full hidden size / heads / intermediate, fewer layers (4) and a reduced text
vocabulary to keep the oracle fast; the full-size tables are exercised by the
gather tests.  Prefill at L=256 (160 text + 96 speech-prompt rows, the config's
mix), decode steps through the device KV cache, and decode against synthetic
caches of length 1 / 256 / 1024 / 2048.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def qwen(gpu):
    from larynx_amd.llm import Qwen2Config, Qwen2LM, qwen2_param_shapes
    cfg = Qwen2Config(n_layers=4, text_vocab=2000)
    params = orc.make_params(qwen2_param_shapes(cfg), 77)
    for k in params:
        if k.endswith("layernorm.weight") or k == "norm.weight":
            params[k] = (params[k] + 1.0).astype(np.float32)
    dparams = {k: torch.from_numpy(v).to(gpu) for k, v in params.items()}
    lm = Qwen2LM(dparams, cfg, max_ctx=2304)
    yield cfg, params, dparams, lm
    lm.close()


def test_prefill_then_decode(gpu, qwen):
    cfg, params, _, lm = qwen
    rng = np.random.default_rng(5)
    text = rng.integers(0, cfg.text_vocab, 160)
    speech = rng.integers(0, 6564, 94)
    announce("qwen2 build_lm_input + prefill L=256")
    lm_in = lm.build_lm_input(text, speech)
    o = orc.Qwen2(params, cfg, cap=2304)
    ref_in = o.build_lm_input(text, speech)
    assert lm_in.shape[0] == 256
    assert np.array_equal(lm_in.cpu().numpy().view(np.uint32), ref_in.view(np.uint32))
    logits, hidden, final = lm.prefill(lm_in, capture=True)
    torch.cuda.synchronize()
    rl, rh, rf = o.prefill(ref_in, capture=True)
    for layer in range(cfg.n_layers):
        assert orc.rel_err(hidden[layer].cpu().numpy(), rh[layer]) < TOL, layer
    assert orc.rel_err(final.cpu().numpy(), rf) < TOL
    assert orc.rel_err(logits.cpu().numpy(), rl) < TOL
    assert lm.cache_len == 256
    k0, v0 = lm.cache_views(0)
    assert orc.rel_err(k0[:256].cpu().numpy(), o.k_cache[0, :256]) < TOL
    assert orc.rel_err(v0[:256].cpu().numpy(), o.v_cache[0, :256]) < TOL
    for step, tok in enumerate([17, 6560, 3000]):
        announce(f"qwen2 decode step {step}")
        lg, fn = lm.decode(tok, final_norm=True)
        torch.cuda.synchronize()
        rlg, rfn = o.decode(tok)
        assert orc.rel_err(fn.cpu().numpy(), rfn) < TOL
        assert orc.rel_err(lg.cpu().numpy(), rlg) < TOL
        assert int(lg.argmax()) == int(np.argmax(rlg))
    assert lm.cache_len == 259


@pytest.mark.parametrize("cache_len", [1, 256, 1024, 2048])
def test_decode_against_synthetic_cache(gpu, qwen, cache_len):
    """The decode config: KV cache lengths 1..2048 with random ~N(0, 0.02) contents."""
    cfg, params, _, lm = qwen
    announce(f"qwen2 decode cache_len={cache_len}")
    o = orc.Qwen2(params, cfg, cap=2304)
    for layer in range(cfg.n_layers):
        kc = orc.normal((cache_len, 128), 60 + layer, 1, 0.02)
        vc = orc.normal((cache_len, 128), 60 + layer, 2, 0.02)
        o.k_cache[layer, :cache_len] = kc
        o.v_cache[layer, :cache_len] = vc
        kd, vd = lm.cache_views(layer)
        kd[:cache_len].copy_(torch.from_numpy(kc))
        vd[:cache_len].copy_(torch.from_numpy(vc))
    o.cache_len = cache_len
    lm.set_cache_len(cache_len)
    torch.cuda.synchronize()
    lg, fn = lm.decode(4321, final_norm=True)
    torch.cuda.synchronize()
    rlg, rfn = o.decode(4321)
    assert orc.rel_err(fn.cpu().numpy(), rfn) < TOL
    assert orc.rel_err(lg.cpu().numpy(), rlg) < TOL


def test_errors(gpu, qwen):
    from larynx_amd import LxError
    from larynx_amd._lib import LX_ERR_RANGE, LX_ERR_STATE
    cfg, params, dparams, _ = qwen
    from larynx_amd.llm import Qwen2LM
    announce("qwen2 error paths")
    lm = Qwen2LM(dparams, cfg, max_ctx=64)
    with pytest.raises(LxError) as e:
        lm.decode(5)  # before prefill
    assert e.value.code == LX_ERR_STATE
    with pytest.raises(LxError) as e:
        lm.build_lm_input([0, cfg.text_vocab], [])
    assert e.value.code == LX_ERR_RANGE
    with pytest.raises(LxError) as e:
        lm.build_lm_input([0], [6761])
    assert e.value.code == LX_ERR_RANGE
    x = lm.build_lm_input([1, 2], [3])
    lm.prefill(x, want_logits=False)
    with pytest.raises(LxError) as e:
        lm.decode(6761)
    assert e.value.code == LX_ERR_RANGE
    lm.close()


def test_decode_graph_matches_eager_and_crosses_splits(gpu, qwen):
    """The decode layer stack replayed as a HIP graph and launched eagerly
    (set_decode_graph(False)) give bit-identical logits; sequential decode steps
    across the 64-key attention split boundary (cache 62 -> 67) track the
    oracle, including its device-side position and split counters."""
    from larynx_amd.llm import Qwen2LM
    cfg, params, dparams, _ = qwen
    announce("qwen2 decode graph vs eager, cache 62..67")
    eager = Qwen2LM(dparams, cfg, max_ctx=128)
    eager.set_decode_graph(False)
    graph = Qwen2LM(dparams, cfg, max_ctx=128)
    o = orc.Qwen2(params, cfg, cap=128)
    n0 = 62
    for layer in range(cfg.n_layers):
        kc = orc.normal((n0, 128), 90 + layer, 1, 0.02)
        vc = orc.normal((n0, 128), 90 + layer, 2, 0.02)
        o.k_cache[layer, :n0] = kc
        o.v_cache[layer, :n0] = vc
        for lm in (eager, graph):
            kd, vd = lm.cache_views(layer)
            kd[:n0].copy_(torch.from_numpy(kc))
            vd[:n0].copy_(torch.from_numpy(vc))
    o.cache_len = n0
    eager.set_cache_len(n0)
    graph.set_cache_len(n0)
    torch.cuda.synchronize()
    for step, tok in enumerate([5, 6561, 77, 6000, 1234]):
        announce(f"qwen2 decode step {step} at position {n0 + step}")
        lg_e, fn_e = eager.decode(tok, final_norm=True)
        lg_g, fn_g = graph.decode(tok, final_norm=True)
        torch.cuda.synchronize()
        assert torch.equal(lg_e, lg_g) and torch.equal(fn_e, fn_g), step
        rlg, rfn = o.decode(tok)
        assert orc.rel_err(fn_g.cpu().numpy(), rfn) < TOL, step
        assert orc.rel_err(lg_g.cpu().numpy(), rlg) < TOL, step
    assert graph.cache_len == n0 + 5
    for layer in range(cfg.n_layers):
        kd, vd = graph.cache_views(layer)
        assert orc.rel_err(kd[:n0 + 5].cpu().numpy(), o.k_cache[layer, :n0 + 5]) < TOL
        assert orc.rel_err(vd[:n0 + 5].cpu().numpy(), o.v_cache[layer, :n0 + 5]) < TOL
    eager.close()
    graph.close()


@pytest.mark.parametrize("max_ctx,n0", [(300, 253), (1100, 1021)])
def test_decode_crosses_split_classes(gpu, qwen, max_ctx, n0):
    """Past one split, the attention splits are merged inside the o_proj launch,
    which reads the split states of its split class (up to 4, 8, 12, ...
    splits; one captured graph per class): sequential steps across a class
    boundary (cache 253 -> 258: 4 -> 5 splits; 1021 -> 1026: 16 -> 17) stay
    bit-identical between graph replay and eager launches and track the oracle.
    With max_ctx 300 the cache holds 5 splits, fewer than the 8 the second class
    covers, so the merge clamps to the splits that exist."""
    from larynx_amd.llm import Qwen2LM
    cfg, params, dparams, _ = qwen
    announce(f"qwen2 decode across split classes, max_ctx {max_ctx}, cache {n0}..{n0 + 5}")
    eager = Qwen2LM(dparams, cfg, max_ctx=max_ctx)
    eager.set_decode_graph(False)
    graph = Qwen2LM(dparams, cfg, max_ctx=max_ctx)
    o = orc.Qwen2(params, cfg, cap=max_ctx)
    for layer in range(cfg.n_layers):
        kc = orc.normal((n0, 128), 70 + layer, 1, 0.02)
        vc = orc.normal((n0, 128), 70 + layer, 2, 0.02)
        o.k_cache[layer, :n0] = kc
        o.v_cache[layer, :n0] = vc
        for lm in (eager, graph):
            kd, vd = lm.cache_views(layer)
            kd[:n0].copy_(torch.from_numpy(kc))
            vd[:n0].copy_(torch.from_numpy(vc))
    o.cache_len = n0
    eager.set_cache_len(n0)
    graph.set_cache_len(n0)
    torch.cuda.synchronize()
    for step, tok in enumerate([11, 6562, 4000, 2, 6563]):
        announce(f"qwen2 decode step {step} at position {n0 + step}")
        lg_e, fn_e = eager.decode(tok, final_norm=True)
        lg_g, fn_g = graph.decode(tok, final_norm=True)
        torch.cuda.synchronize()
        assert torch.equal(lg_e, lg_g) and torch.equal(fn_e, fn_g), step
        rlg, rfn = o.decode(tok)
        assert orc.rel_err(fn_g.cpu().numpy(), rfn) < TOL, step
        assert orc.rel_err(lg_g.cpu().numpy(), rlg) < TOL, step
        assert int(np.argmax(lg_g.cpu().numpy())) == int(np.argmax(rlg)), step
    eager.close()
    graph.close()


@pytest.mark.parametrize("L", [1, 37, 200, 300])
def test_prefill_ragged_lengths(gpu, qwen, L):
    """Prefill at lengths that leave partial 64-row tiles and change the
    split-K plan (1 row: one tile per column band; 300 rows: five bands).  At
    200 and 300 rows the gate/up launch runs the split tail on 64-row tiles (4
    row bands x 76 column tiles = 256 whole + 48 in five k ranges; 5 x 76 = 256
    whole + 124 in two), with the last row band partial."""
    cfg, params, _, lm = qwen
    announce(f"qwen2 prefill L={L}")
    lm_in = torch.from_numpy(orc.normal((L, cfg.hidden), 300 + L, 1, 0.5)).to(gpu)
    logits, hidden, final = lm.prefill(lm_in, capture=True)
    torch.cuda.synchronize()
    o = orc.Qwen2(params, cfg, cap=2304)
    rl, rh, rf = o.prefill(lm_in.cpu().numpy(), capture=True)
    for layer in range(cfg.n_layers):
        assert orc.rel_err(hidden[layer].cpu().numpy(), rh[layer]) < TOL, layer
    assert orc.rel_err(final.cpu().numpy(), rf) < TOL
    assert orc.rel_err(logits.cpu().numpy(), rl) < TOL
    assert lm.cache_len == L
    for layer in (0, cfg.n_layers - 1):
        k, v = lm.cache_views(layer)
        assert orc.rel_err(k[:L].cpu().numpy(), o.k_cache[layer, :L]) < TOL
        assert orc.rel_err(v[:L].cpu().numpy(), o.v_cache[layer, :L]) < TOL


def test_prefill_split_tail_is_deterministic(gpu, qwen):
    """The gate/up launch at L=256 (split tail: 256 whole tiles, 48 in five k
    ranges) sums the parts of its split tiles in k order whichever part arrives
    last: two prefills of the same input give bit-identical hidden states,
    logits and caches."""
    cfg, params, _, lm = qwen
    announce("qwen2 prefill L=256 twice (split tail determinism)")
    lm_in = torch.from_numpy(orc.normal((256, cfg.hidden), 4040, 1, 0.5)).to(gpu)
    runs = []
    for _ in range(2):
        logits, hidden, final = lm.prefill(lm_in, capture=True)
        k, v = lm.cache_views(cfg.n_layers - 1)
        torch.cuda.synchronize()
        runs.append([t.cpu().numpy().copy() for t in (*hidden, final, logits, k[:256], v[:256])])
    for a, b in zip(*runs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
