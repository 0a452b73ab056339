"""C-ABI boundary checks that need no GPU: the library loads, exports every
function include/lx_ops.h declares, and rejects bad arguments before any
device work is enqueued."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "lx_ops.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(lx_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_path():
    names = declared_functions()
    for must in ["lx_adaln_modulate_f32", "lx_rope_partial_interleaved_f32", "lx_gelu_tanh_f32",
                 "lx_gated_residual_f32", "lx_timestep_embed_f32", "lx_rmsnorm_f32",
                 "lx_rope_neox_f32", "lx_swiglu_f32", "lx_embed_gather_f32", "lx_linear_f32",
                 "lx_attention_f32", "lx_dit_forward", "lx_cfm_solve", "lx_qwen2_prefill",
                 "lx_qwen2_decode"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    from larynx_amd._lib import LIB_PATH, SIGNATURES
    lib = C.CDLL(LIB_PATH)
    names = declared_functions()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    bound = {s[0] for s in SIGNATURES}
    assert set(names) == bound, (set(names) ^ bound)


def test_version_string():
    import larynx_amd
    assert "gfx950" in larynx_amd.version()


def test_argument_errors_need_no_device():
    from larynx_amd._lib import LX_ERR_ARG, LX_ERR_RANGE, lib
    # null pointers
    assert lib.lx_adaln_modulate_f32(None, None, None, 1024, None, 2, 500, 1024, 1e-6,
                                     None) == LX_ERR_ARG
    assert b"null" in lib.lx_last_error()
    assert lib.lx_linear_f32(None, 4, None, None, None, 4, 1, 1, 4, None, None) == LX_ERR_ARG
    # a bad token id is rejected on the host before any launch
    fake = C.c_void_p(16)
    ids = (C.c_int * 3)(1, 7000, 2)
    assert lib.lx_embed_gather_f32(fake, 6761, 896, ids, 3, fake, None) == LX_ERR_RANGE
    assert b"7000" in lib.lx_last_error()
    ids = (C.c_int * 1)(-1)
    assert lib.lx_embed_gather_f32(fake, 6761, 896, ids, 1, fake, None) == LX_ERR_RANGE
    # unsupported head dim / misaligned shapes
    assert lib.lx_attention_f32(fake, 1024, fake, 1024, fake, 1024, fake, 1024, 1, 4, 4, 8, 8, 128,
                                0.1, 0, 0, None) == LX_ERR_ARG
    assert lib.lx_linear_f32(fake, 6, fake, None, fake, 6, 8, 8, 6, None, None) == LX_ERR_ARG
    assert lib.lx_conv_pos_mish_f32(fake, fake, fake, None, fake, 1, 8, 1024, 8, 31,
                                    None) == LX_ERR_ARG  # 128 channels per group
    assert lib.lx_conv_pos_mish_bx_f32(fake, fake, fake, None, fake, 1, 8, 1024, 16, 31, 4,
                                       None) == LX_ERR_ARG  # products 3 or 6
    assert lib.lx_conv_frag_pack_f32(fake, fake, 1024, 16, 33, None) == LX_ERR_ARG
    # fragment-order GEMM: N not a multiple of 128, an empty last K slice (18
    # steps of 64 as 7 slices of 3), a tile height other than 64 / 128, a
    # product count other than 3 / 6
    from larynx_amd._lib import LX_BX_OUT_PARTIAL, LinearBx
    g = LinearBx()
    g.A, g.lda, g.Wf, g.Y, g.ldy, g.M, g.N, g.K, g.bm, g.slices = (16, 1024, 16, 16, 1000,
                                                                   8, 1000, 1024, 64, 1)
    assert lib.lx_linear_bx_f32(C.byref(g), None) == LX_ERR_ARG
    assert b"N %" in lib.lx_last_error() or b"bad shape" in lib.lx_last_error()
    g.N, g.ldy, g.out, g.slices, g.K, g.lda = 1024, 1024, LX_BX_OUT_PARTIAL, 7, 1152, 1152
    assert lib.lx_linear_bx_f32(C.byref(g), None) == LX_ERR_ARG
    assert b"empty" in lib.lx_last_error()
    g.bm, g.slices = 96, 1
    assert lib.lx_linear_bx_f32(C.byref(g), None) == LX_ERR_ARG
    g.bm, g.products = 64, 4
    assert lib.lx_linear_bx_f32(C.byref(g), None) == LX_ERR_ARG
    assert b"products" in lib.lx_last_error()
    g.products, g.split_tail = 3, 2  # split_tail is a 0 / 1 switch
    assert lib.lx_linear_bx_f32(C.byref(g), None) == LX_ERR_ARG
    assert b"split_tail" in lib.lx_last_error()
    # the folded residual takes at most four partial slices
    assert lib.lx_adaln_resid_f32(fake, fake, 5, 1 << 20, None, fake, 1024, fake, fake, 1024,
                                  fake, 2, 8, 1024, 1e-6, None) == LX_ERR_ARG
    # composite objects: null handles and empty token lists are refused on the host
    assert lib.lx_flow_infer(None, None, 0, None, 0, None, 0, None, None, None,
                             None) == LX_ERR_ARG
    out = C.c_void_p()
    assert lib.lx_flow_load(b"/nonexistent/flow.gguf", 250, C.byref(out)) == LX_ERR_ARG
    assert b"cannot open" in lib.lx_last_error() and not out.value
    # a Qwen2 geometry whose fused q|k|v row the prefill cannot hold is refused
    # at create time (hidden 2048 with 4 kv heads: 2560 floats)
    from larynx_amd._lib import Qwen2Weights
    w = Qwen2Weights()
    (w.hidden, w.intermediate, w.n_heads, w.n_kv_heads, w.head_dim, w.n_layers, w.text_vocab,
     w.speech_vocab, w.rms_eps, w.rope_theta) = (2048, 4864, 32, 4, 64, 1, 100, 6761, 1e-6, 1e6)
    assert lib.lx_qwen2_create(C.byref(w), 16, C.byref(out)) == LX_ERR_ARG
    assert b"2560" in lib.lx_last_error() and not out.value


def _c_layout(struct, fields):
    """sizeof / offsetof of a header struct, as the C compiler lays it out."""
    import shutil
    import subprocess
    import tempfile
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no C compiler")
    prints = "".join(f'printf("%zu\\n", offsetof({struct}, {f}));' for f in fields)
    src = (f'#include <stddef.h>\n#include <stdio.h>\n#include "lx_ops.h"\n'
           f'int main(void){{printf("%zu\\n", sizeof({struct})); {prints} return 0;}}\n')
    with tempfile.TemporaryDirectory() as d:
        c_file, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(c_file, "w").write(src)
        subprocess.run([cc, "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                        "-I", "/opt/rocm/include", c_file, "-o", exe], check=True,
                       capture_output=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    return [int(v) for v in out]


@pytest.mark.parametrize("struct,cls", [
    ("lx_epilogue", "Epilogue"), ("lx_dit_block_weights", "DitBlockWeights"),
    ("lx_dit_weights", "DitWeights"), ("lx_dit_capture", "DitCapture"),
    ("lx_qwen2_layer_weights", "Qwen2LayerWeights"), ("lx_qwen2_weights", "Qwen2Weights"),
    ("lx_flow_frontend_weights", "FlowFrontendWeights"), ("lx_flow_capture", "FlowCapture"),
    ("lx_linear_bx", "LinearBx")])
def test_struct_layouts_match_header(struct, cls):
    import larynx_amd._lib as L
    py = getattr(L, cls)
    fields = [f[0] for f in py._fields_]
    got = _c_layout(struct, fields)
    assert got[0] == C.sizeof(py)
    assert got[1:] == [getattr(py, f).offset for f in fields]


def test_product_path_does_not_reference_the_oracle():
    """The shipped package and library never load or name the oracle."""
    pkg = os.path.join(ROOT, "larynx_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "lxoracle" not in text and "import oracle" not in text, f
                assert "from oracle" not in text, f


def test_one_hip_runtime_whatever_the_import_order():
    """Importing the package before torch must still leave one HIP runtime in
    the process (torch's), or allocations made through liblxops.so and
    through torch land in different runtimes."""
    import subprocess
    import sys
    code = ("import larynx_amd, torch\n"
            "maps = open('/proc/self/maps').read().splitlines()\n"
            "print(len({l.split()[-1] for l in maps if 'libamdhip64' in l}))\n")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == "1"
