"""Torch-tensor front end of the liblxops C-ABI.

Function names follow the reference's op builders (src/flow/ops.cpp,
src/llm/ops.cpp): ada_ln, rope_partial, gelu_tanh, linear, attention,
rms_norm, rope_full, ...  Tensors are CUDA (HIP) fp32 tensors in PyTorch row-major
layout; work is enqueued on torch's current stream.  Every call goes through
liblxops.so; a failing call raises LxError (no fallback path exists).
"""
import ctypes as C

import torch

from ._lib import (LX_BX_OUT_F32, LX_BX_OUT_PACKED, LX_BX_OUT_PARTIAL, LX_EPI_GATED_RESID,
                   LX_EPI_GELU_TANH, LX_EPI_NONE, LX_EPI_RESID, LX_EPI_ROPE_PARTIAL,
                   LX_EPI_SWIGLU_PAIRED, Epilogue, LinearBx, check, lib)

__all__ = [
    "stream", "ada_ln", "adaln_resid", "adaln_emb", "rope_partial", "gelu_tanh", "gated_residual",
    "timestep_embed", "time_mlp", "rms_norm", "rope_full", "swiglu", "embed_gather", "linear",
    "attention", "conv_pos_mish", "conv_pack_weight", "conv_frag_pack", "conv_pos_mish_bx",
    "Epilogue", "split_planes", "linear_split", "wfrag_pack", "linear_bx", "bx_scratch",
    "LX_EPI_NONE", "LX_EPI_GELU_TANH", "LX_EPI_GATED_RESID", "LX_EPI_ROPE_PARTIAL",
    "LX_EPI_RESID", "LX_EPI_SWIGLU_PAIRED", "LX_BX_OUT_F32", "LX_BX_OUT_PARTIAL",
    "LX_BX_OUT_PACKED",
]


def stream():
    """hipStream_t handle of torch's current stream."""
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("liblxops ops take device tensors")
    return C.c_void_p(t.data_ptr())


def _f32(t, name):
    if t.dtype != torch.float32 or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA float32 tensor")


def ada_ln(x, scale, shift, eps=1e-6, out=None):
    """LN(x) * (1 + scale[b]) + shift[b]; x (B, T, D), scale/shift (B, D) possibly strided
    rows (views into the chunked AdaLN embedding).  src/flow/ops.cpp:94-104."""
    _f32(x, "x")
    B, T, D = x.shape
    if scale.stride(-1) != 1 or shift.stride(-1) != 1 or scale.stride(0) != shift.stride(0):
        raise ValueError("scale/shift rows must be contiguous with a common row stride")
    y = torch.empty_like(x) if out is None else out
    check(lib.lx_adaln_modulate_f32(_p(x), _p(shift), _p(scale), scale.stride(0), _p(y), B, T, D,
                                    eps, stream()))
    return y


def adaln_resid(h, partials, bias, gate, shift, scale, out=None, eps=1e-6, packed=False):
    """h += gate * (sum of the K-slice partials (S, B*T, D) + bias), in place; then,
    unless out is False, LN(h) * (1 + scale) + shift into out (B, T, D).
    gate/shift/scale: (B, D) views (row stride = their stride(0)).  packed: out
    receives two-part packed rows (linear_bx's a_packed operand) in its fp32 bytes.
    src/flow/dit.cpp:71,77 + src/flow/ops.cpp:94-104."""
    B, T, D = h.shape
    S = 0 if partials is None else partials.shape[0]
    y = None
    if out is not False:
        y = torch.empty_like(h) if out is None else out
    fn = lib.lx_adaln_resid_packed_f32 if packed else lib.lx_adaln_resid_f32
    check(fn(_p(h), _p(partials), S, partials.stride(0) if S else 0, _p(bias), _p(gate),
             gate.stride(0) if gate is not None else 0, _p(shift), _p(scale), shift.stride(0),
             _p(y), B, T, D, eps, stream()))
    return y


def adaln_emb(c, W, b):
    """W @ silu(c[b]) + bias, c (B, D), W (n_out, D).  src/flow/dit.cpp:56."""
    B, D = c.shape
    n_out = W.shape[0]
    emb = torch.empty(B, n_out, device=c.device, dtype=torch.float32)
    check(lib.lx_adaln_emb_f32(_p(c), _p(W), _p(b), _p(emb), B, D, n_out, stream()))
    return emb


def rope_partial(q, k, pos, rot_dim=64, base=10000.0):
    """In-place partial interleaved rotary on q and k (B, T, ld).  src/flow/ops.cpp:85-92."""
    B, T, ld = q.shape
    if k is not None and k.shape != q.shape:
        raise ValueError("q and k shapes differ")
    check(lib.lx_rope_partial_interleaved_f32(_p(q), _p(k), _p(pos), B, T, q.stride(1), rot_dim,
                                              base, stream()))
    return q, k


def gelu_tanh(h, out=None):
    """tanh-GELU.  src/flow/ops.cpp:73-83."""
    y = torch.empty_like(h) if out is None else out
    check(lib.lx_gelu_tanh_f32(_p(h), _p(y), h.numel(), stream()))
    return y


def gated_residual(x, y, gate):
    """x += gate[b] * y in place; gate (B, D) rows may be strided.  src/flow/dit.cpp:71, 77."""
    B, T, D = x.shape
    check(lib.lx_gated_residual_f32(_p(x), _p(y), _p(gate), gate.stride(0), B, T, D, stream()))
    return x


def timestep_embed(t, half_dim=128, scale=1000.0):
    """Sinusoid of SinusPositionEmbedding.  src/flow/flow_matching.cpp:13-20."""
    B = t.shape[0]
    out = torch.empty(B, 2 * half_dim, device=t.device, dtype=torch.float32)
    check(lib.lx_timestep_embed_f32(_p(t), B, half_dim, scale, _p(out), stream()))
    return out


def time_mlp(t, w0, b0, w2, b2):
    """TimestepEmbedding (sinusoid -> Linear -> SiLU -> Linear).
    src/flow/flow_matching.cpp:10-42."""
    B = t.shape[0]
    D = w0.shape[0]
    work = torch.empty(B * (256 + D), device=t.device, dtype=torch.float32)
    out = torch.empty(B, D, device=t.device, dtype=torch.float32)
    check(lib.lx_time_mlp_f32(_p(t), B, _p(w0), _p(b0), _p(w2), _p(b2), D, _p(work), _p(out),
                              stream()))
    return out


def rms_norm(x, w, eps=1e-6, out=None):
    """x / sqrt(mean(x^2) + eps) * w.  src/llm/ops.cpp:7-11."""
    D = x.shape[-1]
    rows = x.numel() // D
    y = torch.empty_like(x) if out is None else out
    check(lib.lx_rmsnorm_f32(_p(x), _p(w), _p(y), rows, D, eps, stream()))
    return y


def rope_full(qk, pos, n_heads, head_dim=64, theta=1e6):
    """In-place NEOX rotary on (rows, ld) with heads packed from column 0.
    src/llm/ops.cpp:21-30."""
    rows = qk.shape[0]
    check(lib.lx_rope_neox_f32(_p(qk), _p(pos), rows, n_heads, head_dim, qk.stride(0), theta,
                               stream()))
    return qk


def swiglu(gate, up, out=None):
    """silu(gate) * up.  src/llm/llm.cpp:167-169."""
    y = torch.empty_like(gate) if out is None else out
    check(lib.lx_swiglu_f32(_p(gate), _p(up), _p(y), gate.numel(), stream()))
    return y


def embed_gather(table, ids, out=None):
    """table[ids] (bit-exact).  ids: host int sequence.  src/llm/llm.cpp:63-100."""
    ids = [int(i) for i in ids]
    n_rows, D = table.shape
    arr = (C.c_int * max(1, len(ids)))(*ids)
    y = torch.empty(len(ids), D, device=table.device, dtype=table.dtype) if out is None else out
    check(lib.lx_embed_gather_f32(_p(table), n_rows, D, arr, len(ids), _p(y), stream()))
    return y


def linear(x, W, b=None, epilogue=None, out=None):
    """epi(x @ W^T + b) on the matrix cores; x (M, K) (row stride may exceed K),
    W (N, K).  `epilogue` is an Epilogue (kind LX_EPI_*) or None.
    src/flow/ops.cpp:20-26."""
    M, K = x.shape
    N = W.shape[0]
    kind = epilogue.kind if epilogue is not None else LX_EPI_NONE
    if out is None:
        if kind in (LX_EPI_GATED_RESID, LX_EPI_RESID):
            raise ValueError("residual epilogues need out= (the residual stream)")
        ncol = N // 2 if kind == LX_EPI_SWIGLU_PAIRED else N
        out = torch.empty(M, ncol, device=x.device, dtype=torch.float32)
    check(lib.lx_linear_f32(_p(x), x.stride(0), _p(W), _p(b), _p(out), out.stride(0), M, N, K,
                            C.byref(epilogue) if epilogue is not None else None, stream()))
    return out


def split_planes(W):
    """The three bf16 planes (3, N, K) of an fp32 weight W (N, K), w = w0 + w1 + w2,
    that linear_split reads."""
    N, K = W.shape
    planes = torch.empty(3, N, K, device=W.device, dtype=torch.bfloat16)
    check(lib.lx_split_planes_f32(_p(W), planes.data_ptr(), N * K, stream()))
    return planes


def linear_split(x, planes, b=None, epilogue=None, out=None, tile=0):
    """epi(x @ W^T + b) with fp32 arithmetic on the bf16 matrix cores (six exact
    bf16 partial products per element pair), W given as split_planes(W); tile 0:
    128 x 128 output tiles, 1: 128 x 64.  src/flow/ops.cpp:20-26."""
    M, K = x.shape
    N = planes.shape[1]
    kind = epilogue.kind if epilogue is not None else LX_EPI_NONE
    if out is None:
        if kind in (LX_EPI_GATED_RESID, LX_EPI_RESID):
            raise ValueError("residual epilogues need out= (the residual stream)")
        ncol = N // 2 if kind == LX_EPI_SWIGLU_PAIRED else N
        out = torch.empty(M, ncol, device=x.device, dtype=torch.float32)
    check(lib.lx_linear_split_f32(_p(x), x.stride(0), planes.data_ptr(), _p(b), _p(out),
                                  out.stride(0), M, N, K,
                                  C.byref(epilogue) if epilogue is not None else None, tile,
                                  stream()))
    return out


def wfrag_pack(W):
    """W (N, K) fp32 in MFMA fragment order (3 * N * K bf16) for linear_bx."""
    N, K = W.shape
    wf = torch.empty(3 * N * K, device=W.device, dtype=torch.bfloat16)
    check(lib.lx_wfrag_pack_f32(_p(W), wf.data_ptr(), N, K, stream()))
    return wf


def linear_bx(a, wf, N, b=None, epilogue=None, out=None, out_kind=LX_BX_OUT_F32, bm=128,
              slices=1, scratch=None, products=6, a_packed=False, pack_from=0, split_tail=False):
    """epi(a @ W^T + b) with fp32 arithmetic on the bf16 matrix cores, W given as
    wfrag_pack(W) (N rows), a fp32 (M, K).  out_kind LX_BX_OUT_F32: (M, N) (out= the
    residual stream for residual epilogues); LX_BX_OUT_PARTIAL: (slices, M, N) raw
    K-slice products; LX_BX_OUT_PACKED: (M, N) as two-part packed rows.  a_packed: a
    holds two-part packed rows (three products, bm 64).  scratch = bx_scratch(): the
    launch runs stream-K over the CUs, or with split_tail the tiles past one per CU
    split along K (when the tile count allows).  src/flow/ops.cpp:20-26."""
    M, K = a.shape
    g = LinearBx()
    g.A, g.lda = a.data_ptr(), a.stride(0)
    g.Wf = wf.data_ptr()
    g.bias = _p(b)
    if epilogue is not None:
        g.epi = C.pointer(epilogue)
    g.out = out_kind
    g.M, g.N, g.K, g.bm, g.slices, g.products = M, N, K, bm, slices, products
    g.a_packed = int(a_packed)
    g.pack_from = pack_from
    g.split_tail = int(split_tail)
    if out_kind == LX_BX_OUT_PARTIAL:
        if out is None:
            out = torch.empty(slices, M, N, device=a.device, dtype=torch.float32)
        g.Y, g.ldy, g.slice_stride = out.data_ptr(), out.stride(1), out.stride(0)
    else:
        kind = epilogue.kind if epilogue is not None else LX_EPI_NONE
        if out is None:
            if kind in (LX_EPI_GATED_RESID, LX_EPI_RESID):
                raise ValueError("residual epilogues need out= (the residual stream)")
            ncol = N // 2 if kind == LX_EPI_SWIGLU_PAIRED else N
            out = torch.empty(M, ncol, device=a.device, dtype=torch.float32)
        g.Y, g.ldy = out.data_ptr(), out.stride(0)
    if scratch is not None:
        ws, cnt = scratch
        g.ws, g.ws_floats = ws.data_ptr(), ws.numel()
        g.counters, g.n_counters = cnt.data_ptr(), cnt.numel()
    check(lib.lx_linear_bx_f32(C.byref(g), stream()))
    return out


def bx_scratch(device, bm=128, max_tiles=4096):
    """Stream-K scratch for linear_bx: partial tiles and zeroed arrival counters."""
    ws = torch.empty(2 * 256 * bm * 128, device=device, dtype=torch.float32)
    cnt = torch.zeros(max_tiles, device=device, dtype=torch.int32)
    return ws, cnt


def attention(q, k, v, n_heads, n_kv_heads=None, scale=None, causal=False, q_offset=0,
              out=None, head_dim=64, products=6, out_packed=False, kv_packed=False):
    """softmax(scale q k^T) v per head; q (B, Tq, *), k/v (B, Tk, *) with heads packed from
    column 0 (row strides may exceed the head span); products: the split-operand kernel's
    bf16 products per fp32 product (6 or 3); out_packed: the output as two-part packed
    rows (linear_bx's a_packed operand); kv_packed: k and v given as packed rows (three
    products, the split kernel's layouts).  src/flow/dit.cpp:34-51."""
    n_kv_heads = n_kv_heads or n_heads
    B, Tq = q.shape[0], q.shape[1]
    Tk = k.shape[1]
    scale = scale if scale is not None else head_dim ** -0.5
    if out is None:
        out = torch.empty(B, Tq, n_heads * head_dim, device=q.device, dtype=torch.float32)
    check(lib.lx_attention_np_f32(_p(q), q.stride(1), _p(k), k.stride(1), _p(v), v.stride(1),
                                  _p(out), out.stride(1), B, Tq, Tk, n_heads, n_kv_heads,
                                  head_dim, scale, int(causal), q_offset, products,
                                  int(out_packed), int(kv_packed), stream()))
    return out


def conv_pack_weight(w, groups=16):
    """torch Conv1d weight (C, C/G, K) -> tap-major packed copy."""
    Cc, cg, K = w.shape
    wp = torch.empty_like(w)
    check(lib.lx_conv_pack_weight_f32(_p(w), _p(wp), Cc, groups, K, stream()))
    return wp


def conv_pos_mish(x, wp, bias, resid=None, groups=16, kernel=31):
    """mish(causal grouped conv1d(x)) (+ resid); x (B, T, C), wp packed weight.
    src/flow/dit.cpp:113-122."""
    B, T, Cc = x.shape
    y = torch.empty_like(x)
    check(lib.lx_conv_pos_mish_f32(_p(x), _p(wp), _p(bias), _p(resid), _p(y), B, T, Cc, groups,
                                   kernel, stream()))
    return y


def conv_frag_pack(w, groups=16):
    """torch Conv1d weight (C, 64, K) -> MFMA fragment order (3 * C * 64 * K bf16) for
    conv_pos_mish_bx."""
    Cc, cg, K = w.shape
    wf = torch.empty(3 * Cc * cg * K, device=w.device, dtype=torch.bfloat16)
    check(lib.lx_conv_frag_pack_f32(_p(w), wf.data_ptr(), Cc, groups, K, stream()))
    return wf


def conv_pos_mish_bx(x, wf, bias, resid=None, groups=16, kernel=31, products=3):
    """conv_pos_mish as fp32 arithmetic on the bf16 matrix cores (split operands, 3 or 6
    products per fp32 product); wf = conv_frag_pack(w).  src/flow/dit.cpp:113-122."""
    B, T, Cc = x.shape
    y = torch.empty_like(x)
    check(lib.lx_conv_pos_mish_bx_f32(_p(x), wf.data_ptr(), _p(bias), _p(resid), _p(y), B, T, Cc,
                                      groups, kernel, products, stream()))
    return y
