"""Pins the CPU oracle op by op (no GPU).

Each oracle function is checked against something that is NOT a retyping of
its own formula: a float64 torch / transformers library routine with the same
semantics, a closed-form special case, or an invariant — chosen so that a
dropped term, a wrong sign or index, or a transposed operand fails.  A
planted-mistake test at the end shows the checks have teeth.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

RTOL = 2e-6  # fp32 storage of an fp64 evaluation


def rnd(shape, stream, std=1.0, seed=7):
    return orc.normal(shape, seed, stream, std)


# --- a1/a2 AdaLN -------------------------------------------------------------
def test_adaln_matches_torch_layer_norm():
    B, T, D = 2, 37, 1024
    x = rnd((B, T, D), 1) * 3 + 0.5
    sc, sh = rnd((B, D), 2, 0.1), rnd((B, D), 3, 0.1)
    y = orc.adaln(x, sc, sh)
    xt = torch.from_numpy(x).double()
    ref = F.layer_norm(xt, (D,), eps=1e-6) * (1 + torch.from_numpy(sc).double()[:, None]) \
        + torch.from_numpy(sh).double()[:, None]
    assert orc.rel_err(y, ref.numpy()) < RTOL


def test_adaln_invariants():
    B, T, D = 2, 8, 1024
    x = rnd((B, T, D), 4) * 5 + 2
    z = np.zeros((B, D), np.float32)
    y = orc.adaln(x, z, z).astype(np.float64)
    assert np.abs(y.mean(-1)).max() < 1e-6
    assert np.abs(y.var(-1) - 1.0).max() < 1e-5          # biased variance
    # a constant row normalises to 0, so the output is exactly the shift
    xc = np.full((1, 3, D), 4.25, np.float32)
    sh = rnd((1, D), 5)
    yc = orc.adaln(xc, rnd((1, D), 6), sh)
    assert np.array_equal(yc[0, 1], sh[0])
    # batch b uses row b of scale/shift (not row 0)
    sc2 = np.stack([np.zeros(D), np.ones(D)]).astype(np.float32)
    y2 = orc.adaln(x, sc2, z)
    assert np.allclose(y2[1], 2 * y[1], atol=1e-5) and np.allclose(y2[0], y[0], atol=1e-6)


# --- linear ------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 80, 1024), (37, 67, 320), (130, 257, 96)])
def test_linear_matches_float64_matmul(M, N, K):
    x, W, b = rnd((M, K), 1), rnd((N, K), 2, 0.05), rnd((N,), 3)
    y = orc.linear(x, W, b)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b
    assert orc.rel_err(y, ref) < RTOL


# --- a4 GELU -----------------------------------------------------------------
def test_gelu_matches_torch_tanh_gelu():
    h = np.concatenate([rnd((4096,), 1) * 4, np.array([0.0, -30.0, 30.0, 1e-3, -1e-3], np.float32)])
    y = orc.gelu_tanh(h)
    ref = F.gelu(torch.from_numpy(h).double(), approximate="tanh").numpy()
    assert np.abs(y - ref).max() < 1e-6 * np.abs(ref).max()
    assert y[-5] == 0.0 and y[-4] == 0.0 and y[-3] == 30.0


# --- a5 gated residual --------------------------------------------------------
def test_gated_residual_exact():
    B, T, D = 2, 5, 1024
    x, y, g = rnd((B, T, D), 1), rnd((B, T, D), 2), rnd((B, D), 3)
    out = orc.gated_residual(x, y, g)
    ref = x.astype(np.float64) + g[:, None, :].astype(np.float64) * y
    assert np.abs(out - ref).max() <= np.abs(ref).max() * 2 ** -23


# --- a3 partial rotary ---------------------------------------------------------
def test_rope_inv_freq_is_torch_bitwise():
    for base in (10000.0, 1e6):
        ref = 1.0 / (base ** (torch.arange(0, 64, 2).float() / 64))
        assert np.array_equal(orc.rope_inv_freq(base, 64), ref.numpy())


def test_rope_partial_complex_form_and_invariants():
    B, T, D = 2, 300, 1024
    q = rnd((B, T, D), 1)
    pos = np.arange(T, dtype=np.int32)
    out = orc.rope_partial(q, pos, 64, 10000.0)
    # channels >= 64 untouched, position 0 is the identity
    assert np.array_equal(out[..., 64:], q[..., 64:])
    assert np.array_equal(out[:, 0], q[:, 0]) or orc.rel_err(out[:, 0], q[:, 0]) < 1e-7
    # complex form: (x0 + i x1) * exp(i theta), theta = fp32(pos * inv_freq)
    inv = orc.rope_inv_freq(10000.0, 64)
    theta = (pos[:, None].astype(np.float32) * inv[None, :]).astype(np.float32).astype(np.float64)
    z = q[..., 0:64:2].astype(np.float64) + 1j * q[..., 1:64:2]
    zr = z * np.exp(1j * theta)[None]
    assert np.abs(out[..., 0:64:2] - zr.real).max() < 1e-6
    assert np.abs(out[..., 1:64:2] - zr.imag).max() < 1e-6
    # pair norms preserved; relative-position property q(m).k(n) depends on m - n
    n0 = np.hypot(q[..., 0:64:2], q[..., 1:64:2])
    n1 = np.hypot(out[..., 0:64:2], out[..., 1:64:2])
    assert np.abs(n0 - n1).max() < 1e-5
    v = np.tile(rnd((1, 1, D), 9), (1, T, 1))
    rv = orc.rope_partial(v, pos, 64, 10000.0)[0, :, :64].astype(np.float64)
    d1 = rv[10] @ rv[3]
    d2 = rv[107] @ rv[100]
    assert abs(d1 - d2) < 1e-4 * abs(d1)


# --- a6 sinusoid + time MLP ----------------------------------------------------
def test_timestep_embed_closed_forms():
    out = orc.timestep_embed(np.array([0.0, 0.5], np.float32))
    assert np.array_equal(out[0, :128], np.zeros(128, np.float32))
    assert np.array_equal(out[0, 128:], np.ones(128, np.float32))
    # j = 0: coefficient exactly 1 -> sin(500), cos(500)
    assert abs(out[1, 0] - np.sin(500.0)) < 1e-6 and abs(out[1, 128] - np.cos(500.0)) < 1e-6
    # last coefficient is 1e-4 (exp(-127 ln(1e4)/127)) -> angle 0.05
    assert abs(out[1, 127] - np.sin(0.05)) < 1e-6


def test_time_mlp_matches_torch_modules():
    D = 1024
    w0, b0 = rnd((D, 256), 1, 0.02), rnd((D,), 2, 0.02)
    w2, b2 = rnd((D, D), 3, 0.02), rnd((D,), 4, 0.02)
    t = np.array([0.0, 0.3, 0.97], np.float32)
    out = orc.time_mlp(t, w0, b0, w2, b2)
    s = torch.from_numpy(orc.timestep_embed(t)).double()
    h = F.silu(s @ torch.from_numpy(w0).double().T + torch.from_numpy(b0).double())
    ref = h @ torch.from_numpy(w2).double().T + torch.from_numpy(b2).double()
    assert orc.rel_err(out, ref.numpy()) < RTOL


# --- a10 RMSNorm ---------------------------------------------------------------
def test_rmsnorm_matches_transformers():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    x, w = rnd((33, 896), 1) * 2, rnd((896,), 2) + 1
    y = orc.rmsnorm(x, w)
    m = Qwen2RMSNorm(896, eps=1e-6).double()
    with torch.no_grad():
        m.weight.copy_(torch.from_numpy(w).double())
        ref = m(torch.from_numpy(x).double()).numpy()
    assert orc.rel_err(y, ref) < RTOL
    # scale invariance (up to eps)
    y4 = orc.rmsnorm(4 * x, w)
    assert orc.rel_err(y4, y) < 1e-6


# --- a11 NEOX rotary -------------------------------------------------------------
def test_rope_neox_matches_transformers():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    rows, H, hd = 40, 14, 64
    pos = (np.arange(rows) * 37 + 5).astype(np.int32)  # up to ~1500
    q = rnd((rows, H * hd), 1)
    out = orc.rope_neox(q, pos, H, hd, 1e6)
    inv = torch.from_numpy(orc.rope_inv_freq(1e6, hd))
    freqs = (torch.from_numpy(pos).float()[:, None] * inv[None, :])  # fp32 angles, as HF
    emb = torch.cat([freqs, freqs], -1).double()
    qt = torch.from_numpy(q).double().view(1, rows, H, hd).transpose(1, 2)
    qr, _ = apply_rotary_pos_emb(qt, qt, emb.cos()[None], emb.sin()[None])
    ref = qr.transpose(1, 2).reshape(rows, H * hd).numpy()
    assert np.abs(out - ref).max() < 1e-6


# --- a12 SwiGLU ------------------------------------------------------------------
def test_swiglu_matches_torch():
    g, u = rnd((4864 * 3,), 1) * 3, rnd((4864 * 3,), 2)
    y = orc.swiglu(g, u)
    ref = (F.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    assert orc.rel_err(y, ref) < RTOL


# --- a13 gather ----------------------------------------------------------------
def test_gather_bitexact_and_range_checked():
    table = rnd((6761, 896), 1)
    ids = np.array([6561, 0, 6760, 17, 17, 6563], np.int32)
    out = orc.embed_gather(table, ids)
    assert np.array_equal(out.view(np.uint32), table[ids].view(np.uint32))
    with pytest.raises(IndexError):
        orc.embed_gather(table, np.array([0, 6761], np.int32))
    with pytest.raises(IndexError):
        orc.embed_gather(table, np.array([-1], np.int32))


# --- attention ---------------------------------------------------------------------
@pytest.mark.parametrize("causal,H,Hkv,Tq,Tk,off", [
    (False, 16, 16, 45, 45, 0), (True, 14, 2, 33, 33, 0), (True, 14, 2, 1, 70, 69),
    (True, 14, 2, 5, 40, 35)])
def test_attention_matches_torch_sdpa(causal, H, Hkv, Tq, Tk, off):
    B, hd = 2, 64
    q = rnd((B, Tq, H * hd), 1)
    k = rnd((B, Tk, Hkv * hd), 2)
    v = rnd((B, Tk, Hkv * hd), 3)
    o = orc.attention(q, k, v, H, Hkv, causal=causal, q_offset=off)
    qt = torch.from_numpy(q).double().view(B, Tq, H, hd).transpose(1, 2)
    kt = torch.from_numpy(k).double().view(B, Tk, Hkv, hd).transpose(1, 2)
    vt = torch.from_numpy(v).double().view(B, Tk, Hkv, hd).transpose(1, 2)
    kt = kt.repeat_interleave(H // Hkv, dim=1)
    vt = vt.repeat_interleave(H // Hkv, dim=1)
    mask = None
    if causal:
        qi = torch.arange(Tq)[:, None] + off
        kj = torch.arange(Tk)[None, :]
        mask = kj <= qi
    ref = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    ref = ref.transpose(1, 2).reshape(B, Tq, H * hd).numpy()
    assert orc.rel_err(o, ref) < RTOL


# --- conv_pos ------------------------------------------------------------------------
def test_conv_pos_matches_torch_grouped_conv():
    B, T, Cc, G, K = 2, 50, 1024, 16, 31
    x = rnd((B, T, Cc), 1)
    w, b = rnd((Cc, Cc // G, K), 2, 0.05), rnd((Cc,), 3, 0.05)
    r = rnd((B, T, Cc), 4)
    y = orc.conv_pos_mish(x, w, b, r)
    xt = torch.from_numpy(x).double().permute(0, 2, 1)
    c = F.conv1d(F.pad(xt, (K - 1, 0)), torch.from_numpy(w).double(),
                 torch.from_numpy(b).double(), groups=G)
    ref = (F.mish(c).permute(0, 2, 1) + torch.from_numpy(r).double()).numpy()
    assert orc.rel_err(y, ref) < RTOL


# --- the checks have teeth ---------------------------------------------------------
def test_planted_mistakes_are_caught():
    """Plausible oracle mistakes, applied on the CPU, fail the pins above."""
    B, T, D = 1, 64, 1024
    q = rnd((B, T, D), 1)
    pos = np.arange(T, dtype=np.int32)
    good = orc.rope_partial(q, pos, 64, 10000.0)
    # NEOX pairing instead of interleaved pairs
    neox = orc.rope_neox(q[0], pos, 1, 64, 10000.0)[None]
    assert orc.rel_err(neox[..., :64], good[..., :64]) > 1e-2
    # wrong rotation direction (sin sign)
    flipped = orc.rope_partial(q, -pos, 64, 10000.0)
    assert orc.rel_err(flipped, good) > 1e-2
    # scale/shift chunks swapped (the norm_out order trap)
    x = rnd((2, 8, D), 2)
    sc, sh = rnd((2, D), 3, 0.3), rnd((2, D), 4, 0.3)
    assert orc.rel_err(orc.adaln(x, sh, sc), orc.adaln(x, sc, sh)) > 1e-2
    # unbiased variance instead of biased
    xt = torch.from_numpy(x).double()
    unb = (xt - xt.mean(-1, keepdim=True)) / torch.sqrt(xt.var(-1, keepdim=True) + 1e-6)
    z = np.zeros((2, D), np.float32)
    assert np.abs(orc.adaln(x, z, z) - unb.numpy()).max() > 1e-4
