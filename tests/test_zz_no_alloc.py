"""lx_time_mlp_f32_noalloc (the allocation-free variant of lx_time_mlp_f32,
whose hidden layer lives in a library-owned device array) against the
workspace entry point, through the C-ABI: two calls in a row, the second with
a smaller input, each bit-identical to lx_time_mlp_f32 on the same inputs and
within 1e-4 of the oracle; sizes past the array are refused before any launch."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _case(gpu, B, D, seed):
    from larynx_amd._lib import lib
    from larynx_amd.ops import stream
    t = torch.from_numpy(np.linspace(0.05, 0.95, B).astype(np.float32)).to(gpu)
    w0 = torch.from_numpy(orc.normal((D, 256), seed, 1, 0.02)).to(gpu)
    b0 = torch.from_numpy(orc.normal((D,), seed, 2, 0.02)).to(gpu)
    w2 = torch.from_numpy(orc.normal((D, D), seed, 3, 0.02)).to(gpu)
    b2 = torch.from_numpy(orc.normal((D,), seed, 4, 0.02)).to(gpu)
    work = torch.empty(B * (256 + D), device=gpu)
    ref_out = torch.empty(B, D, device=gpu)
    out = torch.full((B, D), float("nan"), device=gpu)
    args = [t.data_ptr(), B, w0.data_ptr(), b0.data_ptr(), w2.data_ptr(), b2.data_ptr(), D]
    assert lib.lx_time_mlp_f32(*args, work.data_ptr(), ref_out.data_ptr(), stream()) == 0
    assert lib.lx_time_mlp_f32_noalloc(*args, out.data_ptr(), stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)
    ref = orc.time_mlp(t.cpu().numpy(), *(a.cpu().numpy() for a in (w0, b0, w2, b2)))
    assert orc.rel_err(out.cpu().numpy(), ref) < 1e-4


def test_noalloc_matches_workspace_entry_point(gpu):
    announce("time_mlp_noalloc: B=8 D=2048 then B=2 D=1024")
    _case(gpu, 8, 2048, 51)   # fills the whole 16384-float array
    _case(gpu, 2, 1024, 52)   # smaller, after the larger call


def test_noalloc_rejects_sizes_past_the_array(gpu):
    from larynx_amd._lib import LX_ERR_ARG, lib
    announce("time_mlp_noalloc: oversize refused")
    buf = torch.zeros(16, device=gpu)
    p = buf.data_ptr()
    assert lib.lx_time_mlp_f32_noalloc(p, 8, p, p, p, p, 4096, p, None) == LX_ERR_ARG
    assert b"exceeds" in lib.lx_last_error()
