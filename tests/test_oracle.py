"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so a plausible mistake (dropped term, wrong index, wrong
sign, transposed operand) fails it: fp64 brute force written independently of
the oracle's loops, closed forms, invariants, torch CPU as an independent
implementation, and bit-equality of the blocked loops with the literal
reference loop order.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import pyoracle as O

RNG = np.random.default_rng(1234)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- Linear


@pytest.mark.parametrize("M,K,N", [(4, 8, 6), (37, 64, 129), (8, 257, 33)])
def test_linear_fp64_bruteforce(M, K, N):
    x, W, b = rnd(M, K), rnd(N, K, scale=0.1), rnd(N)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b
    y = O.linear(x, W, b)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("M,K,N", [(3, 5, 7), (19, 64, 300), (9, 33, 257)])
def test_linear_blocked_equals_reference_loop(M, K, N, layout):
    x, W, b = rnd(M, K), rnd(N, K, scale=0.1), rnd(N)
    np.testing.assert_array_equal(O.linear(x, W, b, layout), O.linear(x, W, b, layout, naive=True))
    np.testing.assert_array_equal(O.linear(x, W, None, layout),
                                  O.linear(x, W, None, layout, naive=True))


def test_linear_literal_layout_identity():
    # D1: the reference CPU path reads the [out,in] buffer as [in,out]:
    # literal(W) == standard(reshape(W, [K, N])^T), bit for bit.
    M, K, N = 7, 12, 20
    x, W, b = rnd(M, K), rnd(N, K), rnd(N)
    lit = O.linear(x, W, b, layout=1)
    std = O.linear(x, np.ascontiguousarray(W.reshape(K, N).T), b, layout=0)
    np.testing.assert_array_equal(lit, std)
    # and it is NOT x W^T (the quirk is real)
    assert not np.allclose(lit, O.linear(x, W, b, layout=0), atol=1e-3)


def test_linear_identity_and_zero_weights():
    x = rnd(5, 16)
    np.testing.assert_array_equal(O.linear(x, np.eye(16, dtype=np.float32)), x)
    b = rnd(9)
    np.testing.assert_array_equal(O.linear(x, np.zeros((9, 16), np.float32), b),
                                  np.broadcast_to(b, (5, 9)))


def test_linear_torch():
    x, W, b = rnd(33, 128), rnd(96, 128, scale=0.05), rnd(96)
    ref = F.linear(torch.from_numpy(x), torch.from_numpy(W), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(O.linear(x, W, b), ref, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- LayerNorm


def test_layernorm_closed_form_two_values():
    a, c, eps = 3.0, -1.0, 1e-6
    x = np.array([[a, c]], np.float32)
    y = O.layernorm(x, np.ones(2, np.float32), np.zeros(2, np.float32), eps)
    # mean = 1, var = 4 -> (x - 1)/sqrt(4 + eps)
    np.testing.assert_allclose(y, [[2 / np.sqrt(4 + eps), -2 / np.sqrt(4 + eps)]], rtol=1e-6)


def test_layernorm_constant_row_gives_beta_and_affine():
    D = 64
    g, b = rnd(D), rnd(D)
    y = O.layernorm(np.full((3, D), 7.25, np.float32), g, b, 1e-6)
    np.testing.assert_array_equal(y, np.broadcast_to(b, (3, D)))
    x = rnd(50, D, scale=3.0) + 5
    y1 = O.layernorm(x, np.ones(D, np.float32), np.zeros(D, np.float32), 1e-6)
    np.testing.assert_allclose(y1.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y1.var(-1), 1, atol=1e-4)
    ref = F.layer_norm(torch.from_numpy(x), (D,), torch.from_numpy(g), torch.from_numpy(b), 1e-6)
    np.testing.assert_allclose(O.layernorm(x, g, b, 1e-6), ref.numpy(), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- GELU


def test_gelu_known_values_and_torch():
    x = np.array([0.0, 3.0, -3.0, 1.0], np.float32)
    y = O.gelu(x)
    assert y[0] == 0.0
    # gelu(x) - gelu(-x) == x for the tanh form
    np.testing.assert_allclose(y[1] - y[2], 3.0, rtol=1e-6)
    # tanh-form value at 1: 0.5*(1+tanh(sqrt(2/pi)*1.044715)) = 0.8411920
    np.testing.assert_allclose(y[3], 0.8411920, rtol=2e-6)
    z = rnd(1000, scale=3)
    ref = F.gelu(torch.from_numpy(z), approximate="tanh").numpy()
    np.testing.assert_allclose(O.gelu(z), ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- attention


def sdpa64(q, k, v, scale):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    s = np.exp(s - s.max(-1, keepdims=True))
    s /= s.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", s, v)


@pytest.mark.parametrize("Nq,Nkv,hd", [(5, 5, 8), (4, 6, 8), (33, 70, 64)])
def test_sdpa_fp64_and_torch(Nq, Nkv, hd):
    q, k, v = rnd(2, 3, Nq, hd), rnd(2, 3, Nkv, hd), rnd(2, 3, Nkv, hd)
    sc = 1.0 / np.sqrt(hd)
    o = O.sdpa(q, k, v)
    np.testing.assert_allclose(o, sdpa64(q, k, v, sc), rtol=1e-5, atol=1e-5)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                         torch.from_numpy(v)).numpy()
    np.testing.assert_allclose(o, ref, rtol=1e-4, atol=1e-5)


def test_sdpa_zero_query_is_mean_and_dominant_is_onehot():
    k, v = rnd(1, 2, 9, 16), rnd(1, 2, 9, 16)
    o = O.sdpa(np.zeros((1, 2, 3, 16), np.float32), k, v)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(2, keepdims=True), o.shape), atol=1e-6)
    kd = np.zeros((1, 1, 5, 16), np.float32)
    kd[0, 0, 3, 0] = 1.0
    q = np.zeros((1, 1, 1, 16), np.float32)
    q[0, 0, 0, 0] = 400.0
    vd = rnd(1, 1, 5, 16)
    np.testing.assert_allclose(O.sdpa(q, kd, vd)[0, 0, 0], vd[0, 0, 3], atol=1e-6)


# ---------------------------------------------------------------- RoPE 2D


def test_rope_identity_at_origin_and_norm_preserving():
    H, gw = 2, 3
    t = rnd(1, 6, H * 64)
    r = O.rope2d(t, H, gw, 100.0)
    np.testing.assert_array_equal(r[0, 0], t[0, 0])  # token 0 sits at (0, 0)
    # each rotated pair (j, j+16) of each axis-half keeps its norm
    tt = t.reshape(1, 6, H, 2, 2, 16)
    rr = r.reshape(1, 6, H, 2, 2, 16)
    np.testing.assert_allclose((rr ** 2).sum(4), (tt ** 2).sum(4), rtol=1e-5)


def test_rope_relative_position_invariance():
    # q.k after rotation depends only on the position difference.
    gw, gh = 5, 4
    H = 1
    q, k = rnd(64), rnd(64)

    def rot_at(vec, y, x):
        t = np.zeros((1, gh * gw, 64), np.float32)
        t[0, y * gw + x] = vec
        return O.rope2d(t, H, gw, 100.0)[0, y * gw + x].astype(np.float64)

    d1 = rot_at(q, 1, 1) @ rot_at(k, 2, 3)
    d2 = rot_at(q, 2, 2) @ rot_at(k, 3, 4)
    d3 = rot_at(q, 0, 0) @ rot_at(k, 1, 2)
    np.testing.assert_allclose([d1, d2], [d3, d3], rtol=1e-4, atol=1e-5)


def test_rope_frequency_schedule_known_answer():
    # unit vector in pair j=1 of the y half at row y=1: angle = 100^(-2/32)
    gw = 2
    t = np.zeros((1, 4, 64), np.float32)
    t[0, 2, 1] = 1.0  # token 2 = (y=1, x=0), dim 1 (pair (1, 17))
    r = O.rope2d(t, 1, gw, 100.0)[0, 2]
    th = 100.0 ** (-2.0 / 32.0)
    np.testing.assert_allclose([r[1], r[17]], [np.cos(th), np.sin(th)], rtol=1e-6)
    # x half: dim 32+3 at column x=1 (token 1), angle = 100^(-6/32)
    t = np.zeros((1, 4, 64), np.float32)
    t[0, 1, 35] = 1.0
    r = O.rope2d(t, 1, gw, 100.0)[0, 1]
    th = 100.0 ** (-6.0 / 32.0)
    np.testing.assert_allclose([r[35], r[51]], [np.cos(th), np.sin(th)], rtol=1e-6)


def test_rope_brute_force_2x3():
    # complex-multiplication statement of the rotation on a 2x3 grid
    H, gh, gw = 1, 2, 3
    t = rnd(1, gh * gw, 64)
    r = O.rope2d(t, H, gw, 100.0)
    for n in range(gh * gw):
        y, x = divmod(n, gw)
        for ax, pos in ((0, y), (1, x)):
            u = t[0, n, ax * 32:(ax + 1) * 32].astype(np.float64)
            z = (u[:16] + 1j * u[16:]) * np.exp(1j * pos * 100.0 ** (-np.arange(16) * 2 / 32))
            np.testing.assert_allclose(r[0, n, ax * 32:ax * 32 + 16], z.real, atol=2e-6)
            np.testing.assert_allclose(r[0, n, ax * 32 + 16:(ax + 1) * 32], z.imag, atol=2e-6)


def test_rope_ref_token_known_cases():
    # reference token RoPE (src/mastr/encoder_v2.cr:204-254): identity at (0,0)
    x = rnd(1, 4, 128)
    y = O.rope_ref_token(x, 2, 2, 2, 100.0)
    np.testing.assert_array_equal(y[0, 0], x[0, 0])
    # token (y=1, x=0), head 0, dim 0: x0*cos(f0) - x32*sin(f0), f0 = 1
    np.testing.assert_allclose(y[0, 2, 0], x[0, 2, 0] * np.cos(1.0) - x[0, 2, 32] * np.sin(1.0),
                               rtol=1e-5)
    # x-half of token (0, 1), dim 32+1: x1*sin(f1) + x33*cos(f1), f1 = 100^(-2/64)
    f1 = 100.0 ** (-2.0 / 64.0)
    np.testing.assert_allclose(y[0, 1, 33], x[0, 1, 1] * np.sin(f1) + x[0, 1, 33] * np.cos(f1),
                               rtol=1e-5)


# ---------------------------------------------------------------- conv & resampling


@pytest.mark.parametrize("k,s,p", [(3, 1, 1), (3, 2, 1), (1, 1, 0), (4, 4, 0)])
def test_conv_blocked_equals_reference_loop_and_torch(k, s, p):
    x, w, b = rnd(2, 9, 11, 32), rnd(40, 32, k, k, scale=0.1), rnd(40)
    y = O.conv2d(x, w, b, s, p)
    np.testing.assert_array_equal(y, O.conv2d(x, w, b, s, p, naive=True))
    ref = F.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w),
                   torch.from_numpy(b), stride=s, padding=p).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("kh,kw,s,p", [(1, 3, 1, 1), (3, 1, 2, 1), (2, 5, 1, 2), (5, 2, 3, 0)])
def test_conv_nonsquare_kernel_reference_loop_and_torch(kh, kw, s, p):
    """kh x kw kernels (the GPU conv2d_forward reads kernel_h and kernel_w
    separately): blocked == literal loop bit for bit, and torch conv2d; a
    transposed kernel (kw x kh) changes the output grid or the values."""
    x, w, b = rnd(2, 9, 11, 32), rnd(24, 32, kh, kw, scale=0.1), rnd(24)
    y = O.conv2d(x, w, b, s, p)
    np.testing.assert_array_equal(y, O.conv2d(x, w, b, s, p, naive=True))
    ref = F.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w),
                   torch.from_numpy(b), stride=s, padding=p).permute(0, 2, 3, 1).numpy()
    assert y.shape == ref.shape
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)


def test_conv_1x1_is_linear_and_delta_kernel_is_identity():
    x, w, b = rnd(1, 5, 7, 32), rnd(24, 32, 1, 1), rnd(24)
    np.testing.assert_array_equal(O.conv2d(x, w, b),
                                  O.linear(x.reshape(-1, 32), w.reshape(24, 32), b).reshape(1, 5, 7, 24))
    d = np.zeros((32, 32, 3, 3), np.float32)
    d[np.arange(32), np.arange(32), 1, 1] = 1.0
    np.testing.assert_array_equal(O.conv2d(x, d, None, 1, 1), x)


@pytest.mark.parametrize("k", [2, 4])
def test_conv_transpose_torch_and_gemm_identity(k):
    x, w, b = rnd(2, 3, 5, 32), rnd(32, 48, k, k, scale=0.1), rnd(48)
    y = O.conv_transpose(x, w, b, k)
    ref = F.conv_transpose2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w),
                             torch.from_numpy(b), stride=k).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)
    g = x.reshape(-1, 32).astype(np.float64) @ w.reshape(32, -1).astype(np.float64)
    g = g.reshape(2, 3, 5, 48, k, k).transpose(0, 1, 4, 2, 5, 3).reshape(2, 3 * k, 5 * k, 48) + b
    np.testing.assert_allclose(y, g, rtol=1e-5, atol=1e-5)


def test_upsample_exact_fields_and_torch():
    H, W, Cc = 5, 7, 8
    const = np.full((1, H, W, Cc), 2.5, np.float32)
    np.testing.assert_array_equal(O.upsample2x(const), np.full((1, 2 * H, 2 * W, Cc), 2.5))
    yy, xx = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    aff = (0.5 * yy - 0.25 * xx + 1.0).astype(np.float32)[None, :, :, None].repeat(Cc, 3)
    up = O.upsample2x(aff)
    oy, ox = np.meshgrid(np.arange(2 * H) * (H - 1) / (2 * H - 1),
                         np.arange(2 * W) * (W - 1) / (2 * W - 1), indexing="ij")
    np.testing.assert_allclose(up[0, :, :, 0], 0.5 * oy - 0.25 * ox + 1.0, atol=1e-5)
    x = rnd(2, H, W, Cc)
    u = O.upsample2x(x)
    for (a, b) in ((0, 0), (0, -1), (-1, 0), (-1, -1)):
        np.testing.assert_array_equal(u[:, a, b], x[:, a, b])
    ref = F.interpolate(torch.from_numpy(x).permute(0, 3, 1, 2), scale_factor=2, mode="bilinear",
                        align_corners=True).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(u, ref, rtol=1e-5, atol=1e-6)


def test_pixel_shuffle_and_unfold_torch():
    h, w, r, Cout = 3, 4, 4, 5
    f = rnd(2, h * w, (Cout + 1) * r * r)
    ps = O.pixel_shuffle(f, h, w, r, Cout)
    t = torch.from_numpy(f).reshape(2, h, w, -1).permute(0, 3, 1, 2)
    ref = F.pixel_shuffle(t, r).permute(0, 2, 3, 1).numpy()[..., :Cout]
    np.testing.assert_array_equal(ps, ref)
    img = rnd(2, 3, 32, 48)
    u = O.unfold(img, 16)
    ref = F.unfold(torch.from_numpy(img), 16, stride=16).transpose(1, 2).numpy()
    np.testing.assert_array_equal(u, ref)


# ---------------------------------------------------------------- composites


def torch_rope(z, H, gw):
    """2D RoPE on q or k [B, N, H*64] from torch ops: per 64-wide head, dims
    [0,32) rotate by the token's row and [32,64) by its column; pairs (j, j+16)
    with inv_freq_j = 100^(-2j/32)."""
    B, N, D = z.shape
    z = z.reshape(B, N, H, 2, 2, 16).clone()
    n = torch.arange(N)
    pos = torch.stack([n // gw, n % gw], 1).double()  # (y, x)
    inv = 100.0 ** (-torch.arange(16).double() * 2 / 32)
    ang = pos[:, :, None] * inv  # N, 2, 16
    c, s = torch.cos(ang).float(), torch.sin(ang).float()
    a, b = z[..., 0, :], z[..., 1, :]
    c = c[None, :, None]
    s = s[None, :, None]
    out = torch.stack([a * c - b * s, b * c + a * s], -2)
    return out.reshape(B, N, D)


def torch_mha(q, k, v, H):
    """Heads of 64 split from token-major [B, N, H*64], SDPA, merged back."""
    B, Nq, D = q.shape
    sh = lambda z: z.reshape(B, z.shape[1], H, D // H).transpose(1, 2)
    return F.scaled_dot_product_attention(sh(q), sh(k), sh(v)).transpose(1, 2).reshape(B, Nq, D)


def _mods(w, eps):
    t = torch.from_numpy
    ln = lambda z, n: F.layer_norm(z, (z.shape[-1],), t(w[n + ".weight"]), t(w[n + ".bias"]), eps)
    lin = lambda z, n: F.linear(z, t(w[n + ".weight"]), t(w[n + ".bias"]))
    return ln, lin


def torch_block(x, w, p, H, gw, eps):
    """Encoder block composed from torch CPU ops (independent of the oracle),
    src/mastr/encoder_v2.cr:38-48 with RoPE on q and k."""
    ln, lin = _mods(w, eps)
    D = x.shape[-1]
    xx = torch.from_numpy(x)
    q, k, v = lin(ln(xx, p + ".norm1"), p + ".attn.qkv").split(D, -1)
    xx = xx + lin(torch_mha(torch_rope(q, H, gw), torch_rope(k, H, gw), v, H), p + ".attn.proj")
    m = F.gelu(lin(ln(xx, p + ".norm2"), p + ".mlp.fc1"), approximate="tanh")
    return (xx + lin(m, p + ".mlp.fc2")).numpy()


def torch_decoder_block(x, mem, w, p, H, gw, eps, rope=True):
    """One MASt3RDecoderBlock from torch CPU ops, written from
    src/mastr/decoder_v2.cr:47-63 (reference role names: norm3 before the
    cross-attention query, norm_y on the memory, norm2 before the MLP) with
    RoPE2D on q and k of both attentions (the memory tokens sit on the same
    grid). x, mem: torch [B, N, D]."""
    ln, lin = _mods(w, eps)
    D = x.shape[-1]
    r = (lambda z: torch_rope(z, H, gw)) if rope else (lambda z: z)
    q, k, v = lin(ln(x, p + ".norm1"), p + ".attn.qkv").split(D, -1)
    x = x + lin(torch_mha(r(q), r(k), v, H), p + ".attn.proj")
    hq, hm = ln(x, p + ".norm3"), ln(mem, p + ".norm_y")
    q = lin(hq, p + ".cross_attn.projq")
    k, v = lin(hm, p + ".cross_attn.projk"), lin(hm, p + ".cross_attn.projv")
    x = x + lin(torch_mha(r(q), r(k), v, H), p + ".cross_attn.proj")
    m = F.gelu(lin(ln(x, p + ".norm2"), p + ".mlp.fc1"), approximate="tanh")
    return x + lin(m, p + ".mlp.fc2")


def torch_decoder(e1, e2, w, cfg, gw, states=False):
    """MASt3RDecoder#forward_pair (src/mastr/decoder_v2.cr:170-191) from torch
    ops: decoder_embed, then per layer l chain 1 (dec_blocks) and chain 2
    (dec_blocks2). composite 0: each chain's cross-attention memory is the
    other chain's state before layer l; composite 1: its own view's
    decoder_embed output, fixed (176-184). Returns dec_norm of both; with
    states=True also each chain's state after every layer (index l = after
    l layers, so index 0 is the decoder_embed output)."""
    comp = cfg.get("composite", 0)
    eps, H = cfg["ln_eps"], cfg["dec_heads"]
    rope = cfg["rope_mode"] == 1
    ln, lin = _mods(w, eps)
    d1, d2 = lin(torch.from_numpy(e1), "decoder_embed"), lin(torch.from_numpy(e2), "decoder_embed")
    m1, m2 = d1, d2
    s1, s2 = [d1.numpy()], [d2.numpy()]
    for l in range(cfg["dec_depth"]):
        if comp == 0:
            m1, m2 = d2, d1
        d1, d2 = (torch_decoder_block(d1, m1, w, f"dec_blocks.{l}", H, gw, eps, rope),
                  torch_decoder_block(d2, m2, w, f"dec_blocks2.{l}", H, gw, eps, rope))
        s1.append(d1.numpy())
        s2.append(d2.numpy())
    n1, n2 = ln(d1, "dec_norm").numpy(), ln(d2, "dec_norm").numpy()
    return (n1, n2, s1, s2) if states else (n1, n2)


def local_features_f64(enc, dec, w, pre, gh, gw, r, C):
    """Local-feature (descriptor) head in float64 numpy: fc2(GELU_tanh(fc1(
    concat(enc, dec)))), then the pixel shuffle by r: desc[b, r*y+i, r*x+j, c]
    = f[b, token (y, x), c*r*r + i*r + j], channels c < C."""
    f64 = lambda a: np.asarray(a, np.float64)
    W = lambda n: (f64(w[n + ".weight"]), f64(w[n + ".bias"]))
    cat = np.concatenate([f64(enc), f64(dec)], -1)
    w1, b1 = W(pre + ".head_local_features.fc1")
    w2, b2 = W(pre + ".head_local_features.fc2")
    h = cat @ w1.T + b1
    h = 0.5 * h * (1 + np.tanh(np.sqrt(2 / np.pi) * (h + 0.044715 * h ** 3)))
    f = h @ w2.T + b2
    B = f.shape[0]
    f = f[..., :C * r * r].reshape(B, gh, gw, C, r, r)
    return f.transpose(0, 1, 4, 2, 5, 3).reshape(B, gh * r, gw * r, C)


def max_excess(got, ref, rtol, atol):
    """Largest |got - ref| / (atol + rtol |ref|): <= 1 means within tolerance."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float((np.abs(got - ref) / (atol + rtol * np.abs(ref))).max())


@pytest.fixture(scope="module")
def tiny_weights(tiny_cfg):
    import gsplat_hip as G
    cfg = G.default_config(**tiny_cfg)
    return G.seeded_weights(cfg, seed=0, bias_std=0.02, ln_std=0.1)


def test_encoder_block_matches_torch_composition(tiny_cfg, tiny_weights):
    gh, gw = 4, 6
    x = rnd(2, gh * gw, tiny_cfg["enc_dim"])
    y = O.encoder_block(tiny_cfg, tiny_weights, "enc_blocks.1", x, gh, gw)
    ref = torch_block(x, tiny_weights, "enc_blocks.1", tiny_cfg["enc_heads"], gw, 1e-6)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)


def test_pair_view_swap_symmetry_and_determinism(tiny_cfg, tiny_weights):
    w = dict(tiny_weights)
    for k in list(w):  # share decoder chain and head weights across the views
        if k.startswith("dec_blocks2."):
            w[k] = w["dec_blocks." + k[len("dec_blocks2."):]]
        if k.startswith("downstream_head2."):
            w[k] = w["downstream_head1." + k[len("downstream_head2."):]]
    i1 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    i2 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    a = O.mastr_pair(tiny_cfg, w, i1, i2)
    b = O.mastr_pair(tiny_cfg, w, i2, i1)
    for k in ("pts", "conf", "desc"):
        np.testing.assert_array_equal(a[k + "1"], b[k + "2"])
        np.testing.assert_array_equal(a[k + "2"], b[k + "1"])
    c = O.mastr_pair(tiny_cfg, w, i1, i2)
    for k in a:
        np.testing.assert_array_equal(a[k], c[k])
    assert np.all(a["conf1"] > 1.0)  # 1 + exp(.)


def test_oracle_thread_count_does_not_change_bits(tiny_cfg, tiny_weights):
    i1 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    O.set_threads(1)
    a = O.mastr_pair(tiny_cfg, tiny_weights, i1, i1[:, :, ::-1].copy())
    O.set_threads(0)
    b = O.mastr_pair(tiny_cfg, tiny_weights, i1, i1[:, :, ::-1].copy())
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])


# Tolerances of the composition pins: oracle (fp32, serial sums) against torch
# CPU (fp32, blocked sums) or float64 numpy, a few layers deep.
COMP_RTOL, COMP_ATOL = 1e-4, 1e-5


def _tiny_imgs(B=1, seed=0):
    r = np.random.default_rng(100 + seed)
    return (r.uniform(-1, 1, (B, 3, 64, 96)).astype(np.float32),
            r.uniform(-1, 1, (B, 3, 64, 96)).astype(np.float32))


@pytest.mark.parametrize("prefix", ["dec_blocks.1", "dec_blocks2.2"])
def test_decoder_block_matches_torch_composition(tiny_cfg, tiny_weights, prefix):
    """One decoder block of either chain (non-trivial LayerNorm affine and
    biases) against the torch composition, with a memory unrelated to x."""
    gh, gw, D = 4, 6, tiny_cfg["dec_dim"]
    x, mem = rnd(2, gh * gw, D), rnd(2, gh * gw, D)
    y = O.decoder_block(tiny_cfg, tiny_weights, prefix, x, mem, gh, gw)
    ref = torch_decoder_block(torch.from_numpy(x), torch.from_numpy(mem), tiny_weights, prefix,
                              tiny_cfg["dec_heads"], gw, 1e-6).numpy()
    assert max_excess(y, ref, COMP_RTOL, COMP_ATOL) <= 1.0


@pytest.mark.parametrize("composite", [0, 1])
def test_decoder_pair_matches_torch_composition(tiny_cfg, tiny_weights, composite):
    """Both decoder chains over all layers, from the oracle's own encoder taps:
    composite 0 (memory = the other chain's previous-layer state) and
    composite 1 (the reference's own-view decoder_embed memory)."""
    cfg = dict(tiny_cfg) if composite == 0 else _ref_cfg(tiny_cfg)
    i1, i2 = _tiny_imgs(2)
    e1, e2, d1, d2 = O.mastr_pair_taps(cfg, tiny_weights, i1, i2)
    r1, r2 = torch_decoder(e1, e2, tiny_weights, cfg, 6)
    assert max_excess(d1, r1, COMP_RTOL, COMP_ATOL) <= 1.0
    assert max_excess(d2, r2, COMP_RTOL, COMP_ATOL) <= 1.0


def test_local_features_match_float64(tiny_cfg, tiny_weights):
    """Descriptor head of the pair (concat(enc, dec_norm) -> fc1 -> GELU ->
    fc2 -> x16 pixel shuffle -> channels 0..23) against float64 numpy, both
    standalone and inside the full pair."""
    i1, i2 = _tiny_imgs(1, 1)
    e1, e2, d1, d2 = O.mastr_pair_taps(tiny_cfg, tiny_weights, i1, i2)
    out = O.mastr_pair(tiny_cfg, tiny_weights, i1, i2, heads=False)
    for v, e, d in ((1, e1, d1), (2, e2, d2)):
        pre = f"downstream_head{v}"
        ref = local_features_f64(e, d, tiny_weights, pre, 4, 6, 16, 24)
        assert max_excess(out[f"desc{v}"], ref, COMP_RTOL, COMP_ATOL) <= 1.0
        got = O.local_features(tiny_cfg, tiny_weights, pre, e, d, 4, 6)
        np.testing.assert_array_equal(got, out[f"desc{v}"])


@pytest.mark.parametrize("mut", [O.MUT_NO_NORM_Y, O.MUT_NO_CROSS_ROPE, O.MUT_NORM_ROLES])
def test_decoder_block_pin_catches_planted_mistakes(tiny_cfg, tiny_weights, mut):
    """The decoder-block pin fails when the oracle drops norm_y, drops RoPE on
    the cross-attention q / k, or swaps the norm2 / norm3 roles (none of which
    the view-swap symmetry can see)."""
    gh, gw, D = 4, 6, tiny_cfg["dec_dim"]
    x, mem = rnd(2, gh * gw, D), rnd(2, gh * gw, D)
    ref = torch_decoder_block(torch.from_numpy(x), torch.from_numpy(mem), tiny_weights,
                              "dec_blocks.1", tiny_cfg["dec_heads"], gw, 1e-6).numpy()
    with O.mutation(mut):
        y = O.decoder_block(tiny_cfg, tiny_weights, "dec_blocks.1", x, mem, gh, gw)
    assert max_excess(y, ref, COMP_RTOL, COMP_ATOL) > 10.0
    assert max_excess(O.decoder_block(tiny_cfg, tiny_weights, "dec_blocks.1", x, mem, gh, gw),
                      ref, COMP_RTOL, COMP_ATOL) <= 1.0  # switch is off again


def _dpt_routing_excess(cfg, w, i1, i2, mut=0):
    """Largest tolerance excess of the pair's full-DPT outputs (pts, conf of
    both views, with mistake mut planted in the pair only) against each
    view's head run standalone on hooks assembled outside the oracle's pair:
    [the view's encoder output, its chain's torch state after layers
    dpt_hooks[1] and dpt_hooks[2], dec_norm of its chain's last state]
    (hook set of MASt3R's DPT adapter, src/mastr/decoder_v2.cr:502-530 for
    the head entry). The standalone head is the float64-golden-pinned
    O.dpt_head."""
    gh, gw = cfg["img_h"] // cfg["patch"], cfg["img_w"] // cfg["patch"]
    hk = cfg["dpt_hooks"]
    e1, e2, _, _ = O.mastr_pair_taps(cfg, w, i1, i2)
    n1, n2, s1, s2 = torch_decoder(e1, e2, w, cfg, gw, states=True)
    with O.mutation(mut):
        out = O.mastr_pair(cfg, w, i1, i2, desc=False)
    worst = 0.0
    for v, e, st, n in ((1, e1, s1, n1), (2, e2, s2, n2)):
        hooks = [e, st[hk[1]], st[hk[2]], n]
        pts, conf = O.dpt_head(cfg, w, f"downstream_head{v}", hooks, gh, gw)
        worst = max(worst, max_excess(out[f"pts{v}"], pts, COMP_RTOL, COMP_ATOL),
                    max_excess(out[f"conf{v}"], conf, COMP_RTOL, COMP_ATOL))
    return worst


@pytest.fixture(scope="module")
def routing_weights(tiny_weights):
    """The tiny weights with every DPT-head weight rescaled to unit gain
    (std 1/sqrt(fan_in) instead of 0.02), so a change in any hook reaches
    pts / conf at full size rather than damped below the biases. Fan-in of
    a conv [out, in, kh, kw] is in*kh*kw; of a ConvTranspose with kernel =
    stride [in, out, k, k] it is in (one tap per output pixel)."""
    w = dict(tiny_weights)
    for n, a in tiny_weights.items():
        if ".dpt." in n and n.endswith(".weight"):
            convt = ".act_postprocess." in n and n.endswith(".1.weight") and a.shape[2] == a.shape[3] \
                and a.shape[2] in (2, 4)
            fan = a.shape[0] if convt else int(np.prod(a.shape[1:]))
            w[n] = (a / (0.02 * np.sqrt(fan))).astype(np.float32)
    return w


def test_pair_dpt_hook_routing(tiny_cfg, routing_weights):
    """Inside the pair, each view's full DPT head reads its own view's
    encoder output, its own chain's states after layers dpt_hooks[1] and
    dpt_hooks[2], and dec_norm of its own chain's final state (non-trivial
    LayerNorm affine, distinct weights per chain and per head)."""
    i1, i2 = _tiny_imgs(1, 4)
    assert _dpt_routing_excess(tiny_cfg, routing_weights, i1, i2) <= 1.0


@pytest.mark.parametrize("mut", [O.MUT_HOOKS_SWAPPED, O.MUT_HEADS_CROSSED, O.MUT_HOOK3_PRE_NORM])
def test_pair_dpt_hook_routing_catches_planted_mistakes(tiny_cfg, routing_weights, mut):
    """The routing pin fails, by more than ten times its tolerance, when the
    two intermediate hooks are swapped, when each head is fed the other
    view's hooks, or when the last hook is taken before dec_norm."""
    i1, i2 = _tiny_imgs(1, 4)
    assert _dpt_routing_excess(tiny_cfg, routing_weights, i1, i2, mut) > 10.0


def test_decoder_pair_pin_catches_fixed_memory(tiny_cfg, tiny_weights):
    """Memory taken from the other view's decoder_embed output (fixed) instead
    of its previous-layer state fails the two-chain pin."""
    i1, i2 = _tiny_imgs(1, 2)
    with O.mutation(O.MUT_MEMORY_FIXED):
        e1, e2, d1, d2 = O.mastr_pair_taps(tiny_cfg, tiny_weights, i1, i2)
    r1, r2 = torch_decoder(e1, e2, tiny_weights, tiny_cfg, 6)
    assert max_excess(d1, r1, COMP_RTOL, COMP_ATOL) > 10.0
    assert max_excess(d2, r2, COMP_RTOL, COMP_ATOL) > 10.0


def test_local_features_pin_catches_swapped_concat(tiny_cfg, tiny_weights):
    """concat(dec, enc) instead of concat(enc, dec) fails the descriptor pin
    (at equal encoder and decoder widths the shapes still fit)."""
    i1, i2 = _tiny_imgs(1, 3)
    e1, _, d1, _ = O.mastr_pair_taps(tiny_cfg, tiny_weights, i1, i2)
    ref = local_features_f64(e1, d1, tiny_weights, "downstream_head1", 4, 6, 16, 24)
    with O.mutation(O.MUT_CONCAT_SWAP):
        got = O.local_features(tiny_cfg, tiny_weights, "downstream_head1", e1, d1, 4, 6)
    assert max_excess(got, ref, COMP_RTOL, COMP_ATOL) > 10.0


def torch_ref_stub_head(dec, w, pre, gh, gw):
    """The reference's stub DPTHead#forward + split_output
    (src/mastr/decoder_v2.cr:502-530, 619-655) from torch CPU ops."""
    t = torch.from_numpy
    B, _, D = dec.shape

    def conv(z, n, pad, bias=True):
        return F.conv2d(z, t(w[n + ".weight"]), t(w[n + ".bias"]) if bias else None, padding=pad)

    x = conv(t(dec).reshape(B, gh, gw, D).permute(0, 3, 1, 2), pre + ".dpt.scratch.layer4_rn", 1,
             bias=False)
    rp = pre + ".dpt.scratch.refinenet4"
    for u in (1, 2):  # ResidualConvUnit: x + conv2(relu(conv1(x)))
        x = x + conv(F.relu(conv(x, f"{rp}.resConfUnit{u}.conv1", 1)),
                     f"{rp}.resConfUnit{u}.conv2", 1)
    x = conv(x, rp + ".out_conv", 0)
    x = conv(F.relu(x), pre + ".dpt.head.0", 1)
    x = conv(F.relu(x), pre + ".dpt.head.2", 1)
    x = conv(x, pre + ".dpt.head.4", 0).permute(0, 2, 3, 1)
    return x[..., :3].numpy(), torch.sigmoid(x[..., 3:]).numpy()


def _ref_cfg(tiny_cfg):
    return dict(tiny_cfg, composite=1, rope_mode=2, ln_eps=1e-5)


def test_ref_composite_stub_head_matches_torch(tiny_cfg, tiny_weights):
    d = _ref_cfg(tiny_cfg)
    i1 = RNG.uniform(-1, 1, (2, 3, 64, 96)).astype(np.float32)
    i2 = RNG.uniform(-1, 1, (2, 3, 64, 96)).astype(np.float32)
    out = O.mastr_pair(d, tiny_weights, i1, i2)
    assert out["pts1"].shape == (2, 4, 6, 3) and out["desc1"] is None
    _, _, d1, d2 = O.mastr_pair_taps(d, tiny_weights, i1, i2)
    for v, dec in ((1, d1), (2, d2)):
        p, c = torch_ref_stub_head(dec, tiny_weights, f"downstream_head{v}", 4, 6)
        np.testing.assert_allclose(out[f"pts{v}"], p, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(out[f"conf{v}"], c, rtol=1e-4, atol=1e-6)
    assert np.all((out["conf1"] > 0) & (out["conf1"] < 1))  # sigmoid


def test_ref_composite_views_are_independent(tiny_cfg, tiny_weights):
    """Reference decoder memory = the view's own decoder_embed output
    (src/mastr/decoder_v2.cr:176-184): view 1 ignores image 2 entirely; the
    MASt3R composition (other view's state) does not."""
    i1 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    i2 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    i3 = RNG.uniform(-1, 1, (1, 3, 64, 96)).astype(np.float32)
    d = _ref_cfg(tiny_cfg)
    a = O.mastr_pair(d, tiny_weights, i1, i2)
    b = O.mastr_pair(d, tiny_weights, i1, i3)
    np.testing.assert_array_equal(a["pts1"], b["pts1"])
    np.testing.assert_array_equal(a["conf1"], b["conf1"])
    assert not np.array_equal(a["pts2"], b["pts2"])
    a = O.mastr_pair(tiny_cfg, tiny_weights, i1, i2, desc=False)
    b = O.mastr_pair(tiny_cfg, tiny_weights, i1, i3, desc=False)
    assert not np.array_equal(a["pts1"], b["pts1"])


# ---- caller-side passes (src/mastr/inference.cr:193-374) -------------------

def test_resize_identity_corners_and_affine_ramp():
    rng = np.random.default_rng(3)
    img = rng.random((7, 11, 3), dtype=np.float32)
    assert np.array_equal(O.resize_image(img, 7, 11), img)  # equal size: identity
    up = O.resize_image(img, 20, 31)
    for (ty, tx), (sy, sx) in {(0, 0): (0, 0), (0, 30): (0, 10), (19, 0): (6, 0),
                               (19, 30): (6, 10)}.items():
        assert np.array_equal(up[ty, tx], img[sy, sx])
    # affine ramp f = 3y + 2x + c on a grid whose steps are exact halves:
    # bilinear reproduces it exactly; a transposed axis or scale would not
    yy, xx = np.meshgrid(np.arange(5), np.arange(9), indexing="ij")
    ramp = np.stack([3 * yy + 2 * xx, yy - xx, 0 * yy + 1], -1).astype(np.float32)
    out = O.resize_image(ramp, 9, 17)
    ty, tx = np.meshgrid(np.arange(9) / 2, np.arange(17) / 2, indexing="ij")
    want = np.stack([3 * ty + 2 * tx, ty - tx, 0 * ty + 1], -1).astype(np.float32)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("sh,sw,th,tw", [(37, 53, 64, 96), (120, 90, 48, 64), (2, 2, 5, 3)])
def test_resize_matches_torch_align_corners(sh, sw, th, tw):
    rng = np.random.default_rng(sh)
    img = rng.random((sh, sw, 3), dtype=np.float32)
    got = O.resize_image(img, th, tw)
    ref = F.interpolate(torch.from_numpy(img).permute(2, 0, 1)[None], size=(th, tw),
                        mode="bilinear", align_corners=True)[0].permute(1, 2, 0).numpy()
    # torch forms the source coordinate as ty * ((sh-1)/(th-1)), the reference
    # as (ty*(sh-1))/(th-1): the fp32 coordinates differ by an ulp or so
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)


def test_preprocess_numpy_and_layout():
    rng = np.random.default_rng(4)
    img = rng.random((2, 5, 7, 3), dtype=np.float32)
    got = O.preprocess_image(img)
    mean = np.array([0.485, 0.456, 0.406], np.float32)
    std = np.array([0.229, 0.224, 0.225], np.float32)
    want = ((img - mean) / std).transpose(0, 3, 1, 2)
    assert got.dtype == np.float32 and np.array_equal(got, want)
    # coded pattern: value encodes (b, y, x, c); the output plane c holds it
    b, y, x, c = np.meshgrid(np.arange(2), np.arange(5), np.arange(7), np.arange(3),
                             indexing="ij")
    code = (1000 * b + 100 * y + 10 * x + c).astype(np.float32)
    back = O.preprocess_image(code) * std[None, :, None, None] + mean[None, :, None, None]
    np.testing.assert_allclose(back, code.transpose(0, 3, 1, 2), rtol=1e-6)


def test_collect_points_mask_order_and_edges():
    rng = np.random.default_rng(5)
    pts = rng.standard_normal((3, 4, 5, 3)).astype(np.float32)
    conf = rng.random((3, 4, 5, 1)).astype(np.float32)
    conf[0, 0, 0, 0] = np.nan
    conf[1, 2, 3, 0] = 0.5  # equal to the threshold: not selected (strict >)
    p, c = O.collect_points(pts, conf, 0.5)
    m = conf.reshape(-1) > 0.5
    assert np.array_equal(p, pts.reshape(-1, 3)[m]) and np.array_equal(c, conf.reshape(-1)[m])
    p, c = O.collect_points(pts, conf, 2.0)
    assert p.shape == (0, 3) and c.shape == (0,)
    p, c = O.collect_points(pts, np.nan_to_num(conf), -1.0)
    assert np.array_equal(p, pts.reshape(-1, 3))
