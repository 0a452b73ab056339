"""Parity of the fragment-order split-operand GEMM (lx_linear_bx_f32) and of the
gated residual folded into the modulated LayerNorm (lx_adaln_resid_f32).

The GEMM forms every fp32 product from three bf16 parts per operand (six exact
partial products, fp32 accumulation), so its error against float64 products is
at the fp32 level: the bound 4e-6 of the output's largest magnitude is the one
the fp32 matrix-core kernel meets (bf16 arithmetic alone would give ~4e-3).
Epilogues and the fused LayerNorm are checked against the oracle at the per-op
bar (1e-4).
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4
FP32_LEVEL = 4e-6
# Three products of two-part splits: each product within about 2^-16 of a * b;
# measured 3.5e-6 - 5.6e-6 over the estimator's and the Qwen2 prefill's shapes.
THREE_PRODUCT_LEVEL = 2e-5


def rnd(shape, stream, std=1.0, seed=23):
    return orc.normal(shape, seed, stream, std)


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.fixture(scope="module")
def ops(gpu):
    from larynx_amd import ops as o
    return o


def bf16_rne(f):
    """bfloat16 bits of float32 values, rounded to nearest even (finite inputs)."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def pack2_np(x):
    """Two-part packed rows on the host: each aligned group of four fp32 values as
    the four bf16(x) then the four bf16(x - bf16(x)), in the group's 16 bytes."""
    x = np.ascontiguousarray(x, np.float32)
    h0 = bf16_rne(x)
    x0 = (h0.astype(np.uint32) << 16).view(np.float32)
    h1 = bf16_rne(x - x0)
    sh = x.shape[:-1] + (x.shape[-1] // 4, 1, 4)
    both = np.concatenate([h0.reshape(sh), h1.reshape(sh)], axis=-2)
    return np.ascontiguousarray(both).reshape(x.shape[:-1] + (2 * x.shape[-1],)).view(np.float32)


def same_bits(a, b):
    a = a.cpu().numpy() if isinstance(a, torch.Tensor) else a
    b = b.cpu().numpy() if isinstance(b, torch.Tensor) else b
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                          np.ascontiguousarray(b).view(np.uint32))


def unpack_wfrag(wf, N, K):
    """W rebuilt on the host from its fragment order: part p of W[nb*32 + l % 32,
    ks*16 + (l // 32)*8 + j] sits at ((nb*(K/16) + ks)*3 + p)*512 + l*8 + j."""
    parts = wf.view(torch.int16).cpu().numpy().astype(np.int32)
    f = (parts.astype(np.uint32) << 16).view(np.float32).reshape(N // 32, K // 16, 3, 2, 32, 8)
    # axes: nb, ks, part, lane half h, row r, j  ->  W[nb*32 + r, ks*16 + h*8 + j]
    tot = (f[:, :, 0].astype(np.float64) + f[:, :, 1]) + f[:, :, 2]
    return tot.transpose(0, 3, 1, 2, 4).reshape(N, K)


def test_wfrag_layout_and_parts_exact(gpu, ops):
    """The fragment order places every weight where the MFMA B operand expects
    it, and its three bf16 parts sum back to the fp32 weight exactly."""
    announce("wfrag layout")
    N, K = 256, 192
    W = rnd((N, K), 1, 0.05)
    wf = ops.wfrag_pack(dev(W, gpu))
    assert wf.numel() == 3 * N * K
    assert np.array_equal(unpack_wfrag(wf, N, K), W.astype(np.float64))


@pytest.mark.parametrize("products", [6, 3])
@pytest.mark.parametrize("M,N,K,bm,sk", [
    (1000, 3072, 1024, 128, False), (1000, 1024, 1024, 64, False), (1000, 2048, 1024, 64, True),
    (37, 128, 64, 64, False), (6000, 1024, 2048, 64, False), (6000, 3072, 1024, 128, True),
    (300, 256, 192, 128, True), (48, 3072, 1024, 64, False)])
def test_linear_bx_fp32_level(gpu, ops, M, N, K, bm, sk, products):
    announce(f"linear_bx M={M} N={N} K={K} bm={bm} streamk={sk} products={products}")
    x, W, b = rnd((M, K), 2), rnd((N, K), 3, 0.03), rnd((N,), 4)
    scr = ops.bx_scratch(gpu, bm=bm) if sk else None
    y = ops.linear_bx(dev(x, gpu), ops.wfrag_pack(dev(W, gpu)), N, dev(b, gpu), bm=bm,
                      scratch=scr, products=products).cpu().numpy()
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b.astype(np.float64)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    assert err < (FP32_LEVEL if products == 6 else THREE_PRODUCT_LEVEL), err
    if sk:  # every arrival count is left at zero for the next call
        assert int(scr[1].abs().sum()) == 0


@pytest.mark.parametrize("T,bm,sk,products", [
    (500, 64, False, 3), (500, 64, False, 6), (500, 128, True, 3), (24, 64, False, 3),
    (3, 128, False, 6), (1500, 64, True, 6)])
def test_linear_bx_epilogues(gpu, ops, T, bm, sk, products):
    """QKV + partial rotary, FF0 + GELU and out / FF2 + gated residual at the
    estimator's shapes, against the oracle."""
    announce(f"linear_bx epilogues T={T} bm={bm} streamk={sk} products={products}")
    B, D, F = 2, 1024, 2048
    scr = ops.bx_scratch(gpu, bm=bm) if sk else None
    x, W, b = rnd((B * T, D), 5), rnd((3 * D, D), 6, 0.03), rnd((3 * D,), 7)
    pos = torch.arange(T, dtype=torch.int32, device=gpu)
    ep = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                      rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
    y = ops.linear_bx(dev(x, gpu), ops.wfrag_pack(dev(W, gpu)), 3 * D, dev(b, gpu), ep, bm=bm,
                      scratch=scr, products=products).cpu().numpy()
    ref = orc.linear(x, W, b).reshape(B, T, 3 * D)
    p = np.arange(T, dtype=np.int32)
    q = orc.rope_partial(np.ascontiguousarray(ref[..., :D]), p)
    k = orc.rope_partial(np.ascontiguousarray(ref[..., D:2 * D]), p)
    ref = np.concatenate([q, k, ref[..., 2 * D:]], -1).reshape(B * T, 3 * D)
    assert orc.rel_err(y, ref) < TOL

    W1, b1 = rnd((F, D), 8, 0.03), rnd((F,), 9)
    g = ops.Epilogue(kind=ops.LX_EPI_GELU_TANH)
    y1 = ops.linear_bx(dev(x, gpu), ops.wfrag_pack(dev(W1, gpu)), F, dev(b1, gpu), g, bm=bm,
                       scratch=scr, products=products).cpu().numpy()
    assert orc.rel_err(y1, orc.gelu_tanh(orc.linear(x, W1, b1))) < TOL

    xf, W2, b2 = rnd((B * T, F), 10), rnd((D, F), 11, 0.03), rnd((D,), 12)
    h = rnd((B, T, D), 13)
    emb = rnd((B, 6 * D), 14, 0.3)
    hd, ed = dev(h, gpu), dev(emb, gpu)
    gate = ed[:, 5 * D:]
    epg = ops.Epilogue(kind=ops.LX_EPI_GATED_RESID, rows_per_batch=T, gate=gate.data_ptr(),
                       gate_stride=6 * D)
    ops.linear_bx(dev(xf, gpu), ops.wfrag_pack(dev(W2, gpu)), D, dev(b2, gpu), epg,
                  out=hd.view(B * T, D), bm=bm, scratch=scr, products=products)
    refg = orc.gated_residual(h, orc.linear(xf, W2, b2).reshape(B, T, D), emb[:, 5 * D:])
    assert orc.rel_err(hd.cpu().numpy(), refg) < TOL


@pytest.mark.parametrize("M,N,K,slices,bm", [
    (1000, 1024, 1024, 2, 64), (1000, 1024, 2048, 2, 64), (1000, 1024, 2048, 4, 128),
    (45, 1024, 1024, 2, 64),
    # the Qwen2 L=256 prefill plans: o_proj 14 steps as 7 x 2, down_proj 76 steps
    # as 8 x 9 + 4 (ragged last slice), and 3 steps over 2 slices
    (256, 896, 896, 7, 64), (256, 896, 4864, 9, 64), (70, 128, 192, 2, 128)])
def test_linear_bx_partial_slices(gpu, ops, M, N, K, slices, bm):
    """K slices written as raw partial products: slice s is the product over its
    K range (ceil(K / 64 / slices) 64-wide steps each, the last the rest), and
    their sum is the whole one."""
    announce(f"linear_bx partial M={M} N={N} K={K} slices={slices} bm={bm}")
    x, W = rnd((M, K), 15), rnd((N, K), 16, 0.03)
    P = ops.linear_bx(dev(x, gpu), ops.wfrag_pack(dev(W, gpu)), N,
                      out_kind=ops.LX_BX_OUT_PARTIAL, slices=slices, bm=bm).cpu().numpy()
    ks = -(-(K // 64) // slices) * 64
    assert (slices - 1) * ks < K
    x64, W64 = x.astype(np.float64), W.astype(np.float64)
    for s in range(slices):
        ref = x64[:, s * ks:min(K, (s + 1) * ks)] @ W64[:, s * ks:min(K, (s + 1) * ks)].T
        assert np.abs(P[s] - ref).max() / np.abs(ref).max() < FP32_LEVEL
    ref = x64 @ W64.T
    assert np.abs(P.astype(np.float64).sum(0) - ref).max() / np.abs(ref).max() < FP32_LEVEL


def test_linear_bx_streamk_is_deterministic(gpu, ops):
    """Stream-K sums a shared tile's partials in k order whatever the arrival
    order: repeated calls are bit-identical (QKV at T=500: 192 tiles over 256
    workgroups, every tile shared by two)."""
    announce("linear_bx stream-K determinism")
    x, W = dev(rnd((1000, 1024), 17), gpu), dev(rnd((3072, 1024), 18, 0.03), gpu)
    wf = ops.wfrag_pack(W)
    scr = ops.bx_scratch(gpu)
    y0 = ops.linear_bx(x, wf, 3072, scratch=scr)
    for _ in range(4):
        assert torch.equal(ops.linear_bx(x, wf, 3072, scratch=scr), y0)


@pytest.mark.parametrize("N,S", [(3072, 2), (2560, 4)])
def test_linear_bx_split_tail(gpu, ops, N, S):
    """Split tail at B*T = 1000 (16 row tiles of 64): N = 3072 gives 384 tiles, 256
    run whole and 128 as two k ranges each; N = 2560 gives 320, 256 whole and 64 as
    four.  In the QKV form (packed A, rotary epilogue, fp32 or packed k / v output):
    the whole tiles (columns below 2048) are bit-identical to the data-parallel
    launch, the split ones sum their parts in k order (within the per-op bar of the
    oracle, bit-identical over repeated calls), and the arrival counts are left at
    zero."""
    announce(f"linear_bx split tail N={N} S={S}")
    M, D, T = 1000, 1024, 500
    x, W, b = rnd((M, D), 60), rnd((N, D), 61, 0.03), rnd((N,), 62)
    xp, wf, bd = dev(pack2_np(x), gpu), ops.wfrag_pack(dev(W, gpu)), dev(b, gpu)
    pos = torch.arange(T, dtype=torch.int32, device=gpu)
    ep = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                      rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
    scr = ops.bx_scratch(gpu, bm=64)
    kw = dict(bm=64, products=3, a_packed=True)
    y_dp = ops.linear_bx(xp, wf, N, bd, ep, **kw)
    y_st = ops.linear_bx(xp, wf, N, bd, ep, scratch=scr, split_tail=True, **kw)
    assert same_bits(y_st[:, :2048], y_dp[:, :2048])
    assert not same_bits(y_st[:, 2048:], y_dp[:, 2048:])  # the split tiles summed their parts
    ref = orc.linear(x, W, b).reshape(2, T, N)
    p = np.arange(T, dtype=np.int32)
    q = orc.rope_partial(np.ascontiguousarray(ref[..., :D]), p)
    k = orc.rope_partial(np.ascontiguousarray(ref[..., D:2 * D]), p)
    ref = np.concatenate([q, k, ref[..., 2 * D:]], -1).reshape(M, N)
    assert orc.rel_err(y_st.cpu().numpy(), ref) < TOL
    assert orc.rel_err(y_dp.cpu().numpy(), ref) < TOL
    for _ in range(3):
        assert torch.equal(ops.linear_bx(xp, wf, N, bd, ep, scratch=scr, split_tail=True, **kw),
                           y_st)
    pk = dict(out_kind=ops.LX_BX_OUT_PACKED, pack_from=D, **kw)
    yp_dp = ops.linear_bx(xp, wf, N, bd, ep, **pk)
    yp_st = ops.linear_bx(xp, wf, N, bd, ep, scratch=scr, split_tail=True, **pk)
    assert same_bits(yp_st[:, :2048], yp_dp[:, :2048])
    assert same_bits(yp_st, pack2_np_from(y_st.cpu().numpy(), D))
    # raw partial products have no epilogue to finish a split tile: the same launch
    # as without scratch
    Pd = ops.linear_bx(xp, wf, N, out_kind=ops.LX_BX_OUT_PARTIAL, **kw)
    Ps = ops.linear_bx(xp, wf, N, out_kind=ops.LX_BX_OUT_PARTIAL, scratch=scr, split_tail=True,
                       **kw)
    assert same_bits(Ps, Pd)
    assert int(scr[1].abs().sum()) == 0


def pack2_np_from(y, c0):
    """Columns [c0, ...) of fp32 rows as two-part packed groups, the rest unchanged."""
    out = np.array(y, np.float32, copy=True)
    out[:, c0:] = pack2_np(np.ascontiguousarray(y[:, c0:]))
    return out


def test_linear_bx_rejects_bad_arguments(gpu, ops):
    from larynx_amd import LxError
    announce("linear_bx bad arguments")
    x = torch.zeros(64, 128, device=gpu)
    wf = ops.wfrag_pack(torch.zeros(192, 128, device=gpu))
    with pytest.raises(LxError):
        ops.linear_bx(x, wf, 192)  # N not a multiple of 128
    wf = ops.wfrag_pack(torch.zeros(128, 128, device=gpu))
    with pytest.raises(LxError):
        ops.linear_bx(x, wf, 128, bm=32)
    with pytest.raises(LxError):  # 2 steps of 64 leave a third slice empty
        ops.linear_bx(x, wf, 128, out_kind=ops.LX_BX_OUT_PARTIAL, slices=3)
    with pytest.raises(LxError):  # K slices only with the partial output
        ops.linear_bx(x, wf, 128, slices=2)
    with pytest.raises(LxError):
        ops.linear_bx(x[:, :96], ops.wfrag_pack(torch.zeros(128, 96, device=gpu)), 128)
    with pytest.raises(LxError):  # packed operands: three products
        ops.linear_bx(x, wf, 128, bm=64, products=6, a_packed=True)
    with pytest.raises(LxError):  # the packed output: 64-row tiles
        ops.linear_bx(x, wf, 128, out_kind=ops.LX_BX_OUT_PACKED, bm=128, products=3)
    with pytest.raises(LxError):  # the packed output takes no epilogue but GELU
        ops.linear_bx(x, wf, 128, epilogue=ops.Epilogue(kind=ops.LX_EPI_SWIGLU_PAIRED),
                      out_kind=ops.LX_BX_OUT_PACKED, bm=64, products=3)


@pytest.mark.parametrize("B,T,S", [(2, 500, 2), (2, 500, 0), (2, 24, 4), (2, 3, 1), (1, 7, 2),
                                   (2, 3000, 2), (3, 1999, 2), (3, 1999, 4), (3, 1999, 0)])
def test_adaln_resid(gpu, ops, B, T, S):
    """h += gate * (sum of the K-slice partials + bias), then the modulated
    LayerNorm of the updated h, against the oracle (gated residual, then ada_ln)."""
    announce(f"adaln_resid B={B} T={T} S={S}")
    D = 1024
    h = rnd((B, T, D), 19) * 2 + 0.1
    P = rnd((max(S, 1), B * T, D), 20)
    bias = rnd((D,), 21, 0.1)
    emb = rnd((B, 6 * D), 22, 0.2)
    hd, ed = dev(h, gpu), dev(emb, gpu)
    Pd = dev(P[:S], gpu) if S else None
    y = ops.adaln_resid(hd, Pd, dev(bias, gpu), ed[:, 2 * D:3 * D], ed[:, :D], ed[:, D:2 * D])
    if S:
        acc = P[:S].astype(np.float64).sum(0).reshape(B, T, D) + bias
        h_ref = orc.gated_residual(h, acc.astype(np.float32), emb[:, 2 * D:3 * D])
    else:
        h_ref = h
    assert orc.rel_err(hd.cpu().numpy(), h_ref) < TOL
    ref = orc.adaln(h_ref, emb[:, D:2 * D], emb[:, :D])
    assert orc.rel_err(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("T", [500, 3000])
def test_adaln_resid_reduce_only_matches_fused(gpu, ops, T):
    """The reduce-only form (no LayerNorm output) leaves h bit-identical to the
    fused one: the estimator uses it for block captures."""
    announce(f"adaln_resid reduce-only T={T}")
    B, D = 2, 1024
    h = dev(rnd((B, T, D), 23), gpu)
    P = dev(rnd((2, B * T, D), 24), gpu)
    bias, emb = dev(rnd((D,), 25), gpu), dev(rnd((B, 6 * D), 26, 0.2), gpu)
    h1, h2 = h.clone(), h.clone()
    ops.adaln_resid(h1, P, bias, emb[:, 2 * D:3 * D], emb[:, :D], emb[:, D:2 * D])
    ops.adaln_resid(h2, P, bias, emb[:, 2 * D:3 * D], emb[:, :D], emb[:, D:2 * D], out=False)
    assert torch.equal(h1, h2)


def test_split_operand_nonfinite_inputs(gpu, ops):
    """The contract of the split-operand kernels for non-finite operands: an
    infinite element, a NaN, or a finite value above the largest bf16 magnitude
    (3.3895e38; its leading part rounds to infinity) turns every output it
    reaches into NaN (the parts x - bf16(x) of an infinity are NaN), where the
    fp32 kernel gives +-inf or a finite product; every other output is
    unaffected.  GEMM: the rows of A holding such an element.  Attention: the
    query row of such a q element, and every query of the (batch, head) whose
    keys hold one.  conv_pos: the channels of its group at the frames whose
    causal window holds it."""
    announce("split-operand kernels: non-finite inputs")
    M, N, K = 1000, 1024, 1024
    x = rnd((M, K), 40)
    W = rnd((N, K), 41, 0.02)
    bad = {3: np.inf, 5: np.nan, 7: 3.3999e38, 9: -np.inf}
    for r, v in bad.items():
        x[r, 17] = v
    xd, Wd = dev(x, gpu), dev(W, gpu)
    clean = np.ones(M, bool)
    clean[list(bad)] = False
    ref = x[clean].astype(np.float64) @ W.astype(np.float64).T
    for y, lvl in ((ops.linear_bx(xd, ops.wfrag_pack(Wd), N, bm=64).cpu().numpy(), FP32_LEVEL),
                   (ops.linear_bx(xd, ops.wfrag_pack(Wd), N, bm=64, products=3).cpu().numpy(),
                    THREE_PRODUCT_LEVEL),
                   (ops.linear_split(xd, ops.split_planes(Wd), tile=0).cpu().numpy(), FP32_LEVEL)):
        for r in bad:
            assert np.isnan(y[r]).all(), r
        assert np.abs(y[clean] - ref).max() / np.abs(ref).max() < lvl
    y32 = ops.linear(xd, Wd).cpu().numpy()  # the fp32 kernel, for contrast
    assert np.isfinite(y32[7]).all() and not np.isfinite(y32[3]).any()

    B, T, D = 2, 500, 1024  # 64-query split-operand layout
    qkv = rnd((B, T, 3 * D), 42, 0.5)
    qkv[0, 10, 3 * 64 + 5] = np.nan         # q of batch 0, query 10, head 3
    qkv[1, 20, D + 5 * 64 + 7] = np.inf     # k of batch 1, key 20, head 5
    qd = dev(qkv, gpu)
    hit = np.zeros((B, T, 16), bool)
    hit[0, 10, 3] = True
    hit[1, :, 5] = True
    for products in (6, 3):
        o = ops.attention(qd[..., :D], qd[..., D:2 * D], qd[..., 2 * D:], 16,
                          products=products).cpu().numpy()
        oh = o.reshape(B, T, 16, 64)
        assert np.isnan(oh[hit]).all(), products
        assert np.isfinite(oh[~hit]).all(), products

    # conv_pos: an infinite input element reaches the 64 outputs of its group at
    # the K frames whose causal window holds it
    T, Kc = 100, 31
    xc = rnd((1, T, D), 43)
    wc, bc = rnd((D, 64, Kc), 44, 0.03), rnd((D,), 45, 0.03)
    xc[0, 10, 3 * 64 + 5] = np.inf
    hitc = np.zeros((1, T, D), bool)
    hitc[0, 10:10 + Kc, 3 * 64:4 * 64] = True
    x0 = xc.copy()
    x0[0, 10, 3 * 64 + 5] = 0.0
    refc = orc.conv_pos_mish(x0, wc, bc)
    wf = ops.conv_frag_pack(dev(wc, gpu))
    for products in (6, 3):
        yc = ops.conv_pos_mish_bx(dev(xc, gpu), wf, dev(bc, gpu), products=products).cpu().numpy()
        assert np.isnan(yc[hitc]).all(), products
        assert orc.rel_err(yc[~hitc], refc[~hitc]) < TOL, products


@pytest.mark.parametrize("M", [1000, 45])
def test_linear_bx_packed_operands_bit_identical(gpu, ops, M):
    """A given as two-part packed rows (the roundings the GEMM applies itself)
    gives bit-identical results to the fp32 A it packs, for every epilogue the
    estimator uses and for K-slice partials; the packed output (none / GELU) is
    the packing of the fp32 output."""
    announce(f"linear_bx packed operands M={M}")
    D, F = 1024, 2048
    T = max(1, M // 2)
    x = rnd((M, D), 50)
    xd, xp = dev(x, gpu), dev(pack2_np(x), gpu)
    W, b = rnd((3 * D, D), 51, 0.03), rnd((3 * D,), 52)
    pos = torch.arange(T, dtype=torch.int32, device=gpu)
    gate = dev(rnd((M // T + 1, D), 53, 0.3), gpu)
    h = dev(rnd((M, D), 54), gpu)
    cases = {
        "rope": (ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                              rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0),
                 3 * D),
        "gelu": (ops.Epilogue(kind=ops.LX_EPI_GELU_TANH), F),
        "none": (None, D),
        "gated": (ops.Epilogue(kind=ops.LX_EPI_GATED_RESID, rows_per_batch=T,
                               gate=gate.data_ptr(), gate_stride=D), D),
    }
    for name, (ep, N) in cases.items():
        wf = ops.wfrag_pack(dev(W[:N], gpu))
        bd = dev(b[:N], gpu)
        outs = []
        for a, packed in ((xd, False), (xp, True)):
            out = h.clone() if name == "gated" else None
            outs.append(ops.linear_bx(a, wf, N, bd, ep, out=out, bm=64, products=3,
                                      a_packed=packed))
        assert same_bits(outs[0], outs[1]), name
        if name in ("gelu", "none"):
            yp = ops.linear_bx(xp, wf, N, bd, ep, out_kind=ops.LX_BX_OUT_PACKED, bm=64,
                               products=3, a_packed=True)
            assert same_bits(yp, pack2_np(outs[0].cpu().numpy())), name
    wf = ops.wfrag_pack(dev(W[:D], gpu))
    P = [ops.linear_bx(a, wf, D, out_kind=ops.LX_BX_OUT_PARTIAL, slices=2, bm=64, products=3,
                       a_packed=packed) for a, packed in ((xd, False), (xp, True))]
    assert same_bits(P[0], P[1])
    # 128-row tiles (the Qwen2 prefill's gate/up) read packed rows too
    wf2 = ops.wfrag_pack(dev(W[:2 * D], gpu))
    sw = ops.Epilogue(kind=ops.LX_EPI_SWIGLU_PAIRED)
    Y = [ops.linear_bx(a, wf2, 2 * D, dev(b[:2 * D], gpu), sw, bm=128, products=3,
                       a_packed=packed) for a, packed in ((xd, False), (xp, True))]
    assert same_bits(Y[0], Y[1])


def test_packed_producers_match_host_packing(gpu, ops):
    """The producers' packed outputs are the host packing of their fp32 outputs:
    the modulated LayerNorm with folded K slices, and attention on the
    split-operand layouts (T = 500, 1000) and the fp32 kernel's small grid
    (T = 24), with three and six products."""
    announce("packed producers")
    B, T, D = 2, 500, 1024
    h = rnd((B, T, D), 60)
    parts = rnd((2, B * T, D), 61, 0.1)
    emb = rnd((B, 6 * D), 62, 0.3)
    ed = dev(emb, gpu)
    args = (dev(parts, gpu), dev(rnd((D,), 63), gpu), ed[:, 2 * D:3 * D], ed[:, :D],
            ed[:, D:2 * D])
    y = ops.adaln_resid(dev(h, gpu), *args)
    yp = ops.adaln_resid(dev(h, gpu), *args, packed=True)
    assert same_bits(yp, pack2_np(y.cpu().numpy()))
    y0 = ops.adaln_resid(dev(h, gpu), None, None, None, ed[:, :D], ed[:, D:2 * D])
    y0p = ops.adaln_resid(dev(h, gpu), None, None, None, ed[:, :D], ed[:, D:2 * D], packed=True)
    assert same_bits(y0p, pack2_np(y0.cpu().numpy()))
    for Tq in (500, 1000, 24):
        qkv = dev(rnd((B, Tq, 3 * D), 64), gpu)
        q, k, v = qkv[..., :D], qkv[..., D:2 * D], qkv[..., 2 * D:]
        for products in (3, 6):
            o = ops.attention(q, k, v, 16, products=products)
            op = ops.attention(q, k, v, 16, products=products, out_packed=True)
            assert same_bits(op, pack2_np(o.cpu().numpy())), (Tq, products)


def test_packed_kv_into_attention_bit_identical(gpu, ops):
    """The QKV projection with its rotary epilogue writes q fp32 and k, v as packed
    rows (pack_from = D); attention reading them packed (three products, the split
    kernel's layouts: T = 500 and 1500 on 64-query workgroups, 1000 on 128-query)
    gives bit-identical output to attention on the fp32 q, k, v; the fp32 kernel's
    small grids refuse packed K/V."""
    from larynx_amd import LxError
    announce("packed K/V into attention")
    B, D = 2, 1024
    for T in (500, 1500, 1000):
        M = B * T
        x = dev(rnd((M, D), 70), gpu)
        wf = ops.wfrag_pack(dev(rnd((3 * D, D), 71, 0.03), gpu))
        bq = dev(rnd((3 * D,), 72), gpu)
        pos = torch.arange(T, dtype=torch.int32, device=gpu)
        rope = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                            rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
        y = ops.linear_bx(x, wf, 3 * D, bq, rope, bm=64, products=3)
        yp = ops.linear_bx(x, wf, 3 * D, bq, rope, out_kind=ops.LX_BX_OUT_PACKED, bm=64,
                           products=3, pack_from=D)
        yc = y.cpu().numpy()
        assert same_bits(yp[:, :D], yc[:, :D])
        assert same_bits(yp[:, D:], pack2_np(yc[:, D:]))
        q3, p3 = y.view(B, T, 3 * D), yp.view(B, T, 3 * D)
        o = ops.attention(q3[..., :D], q3[..., D:2 * D], q3[..., 2 * D:], 16, products=3)
        op = ops.attention(p3[..., :D], p3[..., D:2 * D], p3[..., 2 * D:], 16, products=3,
                           kv_packed=True)
        assert same_bits(o, op), T
    q = torch.zeros(2, 24, D, device=gpu)
    with pytest.raises(LxError):
        ops.attention(q, q, q, 16, products=3, kv_packed=True)
