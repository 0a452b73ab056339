"""ctypes front end of the fp32 ggml-graph CPU baseline (liblxggmlcpu_*.so).

TEST / MEASUREMENT INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it,
tests/ check it against the oracle.  It restates the reference's CPU-backend
graph for one CFG Euler step of the DiT estimator (see lx_ggml_cpu.c); it is
never used by the product path.  Weights reuse the oracle's Dit struct.
"""
import ctypes as C
import os

import numpy as np

from .oracle import Dit, c32, f32p

_HERE = os.path.dirname(os.path.abspath(__file__))


def host_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512vl"} <= flags
    except OSError:
        pass
    return False


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _load():
    name = "liblxggmlcpu_avx512.so" if host_has_avx512() else "liblxggmlcpu_avx2.so"
    path = os.path.join(_HERE, name)
    if not os.path.exists(path):
        raise ImportError(f"{path} not built (make -C oracle)")
    lib = C.CDLL(path)
    from .oracle import OrcDit
    sig = {
        "gcpu_isa": (C.c_char_p, []),
        "gcpu_threads": (C.c_int, []),
        "gcpu_set_threads": (None, [C.c_int]),
        "gcpu_ws_create": (C.c_void_p, [C.c_int, C.c_int]),
        "gcpu_ws_destroy": (None, [C.c_void_p]),
        "gcpu_dit_forward": (C.c_int, [C.c_void_p, C.POINTER(OrcDit), C.c_int, C.c_int, f32p,
                                       f32p, f32p, f32p, f32p, f32p]),
        "gcpu_cfm_step": (C.c_int, [C.c_void_p, C.POINTER(OrcDit), C.c_int, f32p, f32p, f32p,
                                    f32p, C.c_float, C.c_float, C.c_float]),
    }
    for fn_name, (res, args) in sig.items():
        fn = getattr(lib, fn_name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class GgmlCpuDit:
    """The reference's DiT graph on the CPU for batch B and up to max_T frames."""

    def __init__(self, params, B=2, max_T=500, depth=22):
        self.dit = Dit(params, depth=depth)
        self.B, self.max_T = B, max_T
        self._ws = lib.gcpu_ws_create(B, max_T)
        if not self._ws:
            raise MemoryError("gcpu_ws_create")

    def close(self):
        if getattr(self, "_ws", None):
            lib.gcpu_ws_destroy(self._ws)
            self._ws = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, x, mu, cond, spks, t):
        x, mu, cond, spks, t = map(c32, (x, mu, cond, spks, t))
        B, _, T = x.shape
        dphi = np.empty_like(x)
        rc = lib.gcpu_dit_forward(self._ws, C.byref(self.dit.w), B, T, x, mu, cond, spks, t,
                                  dphi)
        assert rc == 0, rc
        return dphi

    def cfm_inputs(self, mu, cond, spks):
        """The batch-2 graph inputs of the CFG loop: row 0 the condition, row 1 zeros
        (src/flow/flow.cpp:216-224)."""
        mel, T = np.shape(mu)
        mu2 = np.zeros((2, mel, T), np.float32)
        cond2 = np.zeros((2, mel, T), np.float32)
        spks2 = np.zeros((2, mel), np.float32)
        mu2[0], cond2[0], spks2[0] = mu, cond, spks
        return mu2, cond2, spks2

    def cfm_step(self, x, mu2, cond2, spks2, t, dt, cfg_rate=0.7):
        """x (mel, T) updated in place."""
        assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
        rc = lib.gcpu_cfm_step(self._ws, C.byref(self.dit.w), x.shape[-1], x, mu2, cond2, spks2,
                               t, dt, cfg_rate)
        assert rc == 0, rc
        return x


def isa():
    return lib.gcpu_isa().decode()


def threads():
    return lib.gcpu_threads()
