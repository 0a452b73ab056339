"""larynx_amd — MI355X (gfx950) fused-op library for Larynx's CosyVoice3 Flow DiT
estimator and Qwen2 LM.

The compute lives in liblxops.so (hand-written HIP kernels behind the C-ABI of
include/lx_ops.h, plus the host C++ estimator / CFM loop / Qwen2 layer code).
This package is the Python front end: `ops` (per-op calls on torch tensors),
`flow` (DiTEstimator), `llm` (Qwen2LM).  Importing it loads liblxops.so and
fails if the library is not built.
"""
from ._lib import LIB_PATH, LxError, lib  # noqa: F401  (loads liblxops.so or raises)

__version__ = "0.1.0"


def version():
    return lib.lx_version().decode()
