"""The fp32 CPU baseline (the reference's ggml DiT graph restated node by node,
oracle/lx_ggml_cpu.c) computes the same function as the reference (no GPU).

It is what bench.py times as the reference's CPU path, so it has to be right:
- the 22-block DiT.forward at T=24 against the golden vectors written from the
  reference's own PyTorch modules;
- the same forward at a ragged length (T=37, per-row t) and one CFG Euler step
  at T=48 against the oracle;
- both SIMD builds (AVX2 and, where the host has it, AVX-512) load and agree.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import ggml_cpu
from oracle import oracle as orc

from larynx_amd.flow import DiTConfig, dit_param_shapes

TOL = 1e-4


@pytest.fixture(scope="module")
def golden_params():
    g = np.load(os.path.join(GOLDEN, "flow_dit_T24.npz"))
    params = orc.make_params(dit_param_shapes(DiTConfig()), int(g["weight_seed"]))
    return g, params


def test_forward_matches_reference_modules(golden_params):
    g, params = golden_params
    base = ggml_cpu.GgmlCpuDit(params, B=2, max_T=64)
    dphi = base.forward(g["x"], g["mu"], g["cond"], g["spks"], g["t"])
    base.close()
    assert orc.rel_err(dphi, g["dphi"]) < TOL


def test_forward_and_cfm_step_match_oracle(golden_params):
    _, params = golden_params
    base = ggml_cpu.GgmlCpuDit(params, B=2, max_T=64)
    T = 37
    x, mu, cond = (orc.normal((2, 80, T), 21, s) for s in (1, 2, 3))
    spks = orc.normal((2, 80), 21, 4, 0.1)
    t = np.array([0.15, 0.85], np.float32)  # distinct rows: per-batch modulation
    ref = orc.Dit(params).forward(x, mu, cond, spks, t)
    assert orc.rel_err(base.forward(x, mu, cond, spks, t), ref) < TOL

    T = 48
    x1 = orc.normal((80, T), 22, 1)
    mu1, c1 = orc.normal((80, T), 22, 2), orc.normal((80, T), 22, 3)
    s1 = orc.normal((80,), 22, 4, 0.1)
    ref = orc.Dit(params).cfm_step(x1, mu1, c1, s1, 0.3, 0.07)
    xs = x1.copy()
    base.cfm_step(xs, *base.cfm_inputs(mu1, c1, s1), 0.3, 0.07)
    base.close()
    assert orc.rel_err(xs, ref) < TOL


def test_both_simd_builds_agree(golden_params):
    g, params = golden_params
    here = os.path.dirname(ggml_cpu.__file__)
    builds = ["liblxggmlcpu_avx2.so"] + (["liblxggmlcpu_avx512.so"]
                                         if ggml_cpu.host_has_avx512() else [])
    outs = []
    dit = orc.Dit(params)
    for name in builds:
        lib = C.CDLL(os.path.join(here, name))
        lib.gcpu_ws_create.restype = C.c_void_p
        lib.gcpu_ws_create.argtypes = [C.c_int, C.c_int]
        lib.gcpu_ws_destroy.argtypes = [C.c_void_p]
        lib.gcpu_dit_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int] + \
            [C.c_void_p] * 6
        ws = lib.gcpu_ws_create(2, 24)
        arrs = [orc.c32(g[k]) for k in ("x", "mu", "cond", "spks", "t")]
        out = np.empty_like(arrs[0])
        rc = lib.gcpu_dit_forward(ws, C.addressof(dit.w), 2, 24,
                                  *[a.ctypes.data for a in arrs], out.ctypes.data)
        lib.gcpu_ws_destroy(ws)
        assert rc == 0
        outs.append(out)
    for out in outs:
        assert orc.rel_err(out, g["dphi"]) < TOL
    if len(outs) == 2:
        assert orc.rel_err(outs[0], outs[1]) < 1e-5


def test_rejects_bad_shapes(golden_params):
    _, params = golden_params
    base = ggml_cpu.GgmlCpuDit(params, B=2, max_T=16)
    x = np.zeros((2, 80, 17), np.float32)
    with pytest.raises(AssertionError):
        base.forward(x, x, x, np.zeros((2, 80), np.float32), np.zeros(2, np.float32))
    base.close()
