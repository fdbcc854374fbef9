"""Writes tests/golden/golden.npz: tiny inputs and float64 expected outputs,
computed here from the mathematics in numpy (no oracle, no library kernel),
for the checks in tests/test_golden.py.

    python tests/golden/make_golden.py

Cases: Linear 4x8 -> 6, LayerNorm 3x16, attention 1x2x5x8, conv 1x5x7x3 -> 4
(3x3, pad 1), RoPE2D on a 2x3 grid (one 64-dim head), GELU (tanh form), the
linear / attention / conv cases again at shapes the device kernels take
(K = 32, head dim 64 with 5 queries x 7 keys, Cin = 32), and
one full DPT head, one decoder block (self- and cross-attention with RoPE2D,
norm_y on the memory) and the local-feature head (concat, MLP, x16 pixel
shuffle) on a 2x2 patch grid with the tiny test widths and seed-0 weights of
the library's generator (the generator is pinned separately by a
numpy restatement in tests/test_abi.py). Inputs are stored as float32 (what
the kernels consume), expectations as float64.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "crystal-gausplat_amd"))

TINY = dict(img_h=32, img_w=32, patch=16, enc_dim=128, enc_depth=2, enc_heads=2, enc_mlp=256,
            dec_dim=128, dec_depth=3, dec_heads=2, dec_mlp=256, dpt_feat=64,
            dpt_dims=[32, 64, 96, 128], dpt_hooks=[0, 1, 2, 3], head_mid=32, lf_hidden=256,
            desc_dim=24)


def f64(a):
    return np.asarray(a, np.float64)


def linear(x, w, b):
    return f64(x) @ f64(w).T + f64(b)


def layernorm(x, g, b, eps):
    x = f64(x)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * f64(g) + f64(b)


def attention(q, k, v, scale):
    s = np.einsum("bhqd,bhkd->bhqk", f64(q), f64(k)) * scale
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, f64(v))


def conv2d(x, w, b, stride=1, pad=0):
    """x NHWC, w OIHW."""
    x, w = f64(x), f64(w)
    B, H, W, C = x.shape
    O, _, k, _ = w.shape
    xp = np.zeros((B, H + 2 * pad, W + 2 * pad, C))
    xp[:, pad:pad + H, pad:pad + W] = x
    Ho, Wo = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    y = np.zeros((B, Ho, Wo, O))
    for i in range(k):
        for j in range(k):
            patch = xp[:, i:i + stride * Ho:stride, j:j + stride * Wo:stride, :]
            y += np.einsum("bhwc,oc->bhwo", patch, w[:, :, i, j])
    return y + (f64(b) if b is not None else 0.0)


def conv_transpose(x, w, b, k):
    """k == stride; x NHWC, w [Cin, Cout, k, k]."""
    x, w = f64(x), f64(w)
    B, H, W, _ = x.shape
    Co = w.shape[1]
    y = np.einsum("bhwc,coij->bhiwjo", x, w).reshape(B, H * k, W * k, Co)
    return y + f64(b)


def upsample2x(x):
    """bilinear, align_corners=True, NHWC."""
    x = f64(x)
    B, H, W, C = x.shape

    def axis(n):
        src = np.arange(2 * n) * (n - 1) / (2 * n - 1)
        i0 = np.clip(np.floor(src).astype(int), 0, n - 1)
        i1 = np.minimum(i0 + 1, n - 1)
        return i0, i1, src - i0

    y0, y1, fy = axis(H)
    x0, x1, fx = axis(W)
    top = x[:, y0][:, :, x0] * (1 - fx)[None, None, :, None] + x[:, y0][:, :, x1] * fx[None, None, :, None]
    bot = x[:, y1][:, :, x0] * (1 - fx)[None, None, :, None] + x[:, y1][:, :, x1] * fx[None, None, :, None]
    return top * (1 - fy)[None, :, None, None] + bot * fy[None, :, None, None]


def relu(x):
    return np.maximum(x, 0.0)


def rope2d(t, grid_w, base=100.0):
    """[N, 64] one head: dims [0,32) rotate by row, [32,64) by column; pairs
    (j, j+16), inv_freq_j = base^(-2j/32)."""
    t = f64(t).copy()
    N = t.shape[0]
    out = np.empty_like(t)
    for n in range(N):
        pos = (n // grid_w, n % grid_w)
        for half in range(2):
            for j in range(16):
                th = pos[half] * base ** (-2.0 * j / 32.0)
                a, b = t[n, 32 * half + j], t[n, 32 * half + j + 16]
                out[n, 32 * half + j] = a * np.cos(th) - b * np.sin(th)
                out[n, 32 * half + j + 16] = b * np.cos(th) + a * np.sin(th)
    return out


def gelu(x):
    x = f64(x)
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))


def dpt_head(w, pre, hooks, gh, gw, cfg):
    """Full DPT head (act_postprocess, layer_rn, four fusion blocks, head)."""
    B = hooks[0].shape[0]
    d = cfg["dpt_dims"]
    ap = pre + ".dpt.act_postprocess."
    W = lambda n: w[n + ".weight"]
    Bi = lambda n: w[n + ".bias"]
    grid = lambda h: f64(h).reshape(B, gh, gw, -1)
    a0 = conv_transpose(conv2d(grid(hooks[0]), W(ap + "0.0"), Bi(ap + "0.0")), W(ap + "0.1"),
                        Bi(ap + "0.1"), 4)
    a1 = conv_transpose(conv2d(grid(hooks[1]), W(ap + "1.0"), Bi(ap + "1.0")), W(ap + "1.1"),
                        Bi(ap + "1.1"), 2)
    a2 = conv2d(grid(hooks[2]), W(ap + "2.0"), Bi(ap + "2.0"))
    a3 = conv2d(conv2d(grid(hooks[3]), W(ap + "3.0"), Bi(ap + "3.0")), W(ap + "3.1"),
                Bi(ap + "3.1"), stride=2, pad=1)
    L = [conv2d(a, W(f"{pre}.dpt.scratch.layer{i + 1}_rn"), None, pad=1)
         for i, a in enumerate((a0, a1, a2, a3))]

    def rcu(n, x):
        t = conv2d(relu(x), W(n + ".conv1"), Bi(n + ".conv1"), pad=1)
        return conv2d(relu(t), W(n + ".conv2"), Bi(n + ".conv2"), pad=1) + x

    def fusion(n, x0, x1):
        s = x0 if x1 is None else x0 + rcu(n + ".resConfUnit1", x1)
        s = rcu(n + ".resConfUnit2", s)
        return conv2d(upsample2x(s), W(n + ".out_conv"), Bi(n + ".out_conv"))

    rp = pre + ".dpt.scratch.refinenet"
    r = fusion(rp + "4", L[3], None)
    r = fusion(rp + "3", r, L[2])
    r = fusion(rp + "2", r, L[1])
    r = fusion(rp + "1", r, L[0])
    h = conv2d(r, W(pre + ".dpt.head.0"), Bi(pre + ".dpt.head.0"), pad=1)
    h = relu(conv2d(upsample2x(h), W(pre + ".dpt.head.2"), Bi(pre + ".dpt.head.2"), pad=1))
    out = conv2d(h, W(pre + ".dpt.head.4"), Bi(pre + ".dpt.head.4"))
    return out[..., :3], 1.0 + np.exp(out[..., 3:])


def rope2d_heads(t, grid_w, H):
    """rope2d on each 64-wide head of token-major t [N, H*64]."""
    return np.concatenate([rope2d(t[:, 64 * h:64 * h + 64], grid_w) for h in range(H)], -1)


def decoder_block(w, p, x, mem, H, grid_w, eps):
    """One decoder block (src/mastr/decoder_v2.cr:47-63, reference role names)
    with RoPE2D on q and k of the self- and the cross-attention; x, mem [N, D]
    of one image."""
    x, mem = f64(x), f64(mem)
    D = x.shape[-1]
    ln = lambda z, n: layernorm(z, w[n + ".weight"], w[n + ".bias"], eps)
    lin = lambda z, n: linear(z, w[n + ".weight"], w[n + ".bias"])

    def mha(q, k, v):
        heads = lambda z: z.reshape(z.shape[0], H, D // H).transpose(1, 0, 2)[None]
        o = attention(heads(rope2d_heads(q, grid_w, H)), heads(rope2d_heads(k, grid_w, H)),
                      heads(v), (D // H) ** -0.5)
        return o[0].transpose(1, 0, 2).reshape(-1, D)

    qkv = lin(ln(x, p + ".norm1"), p + ".attn.qkv")
    x = x + lin(mha(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]), p + ".attn.proj")
    hq, hm = ln(x, p + ".norm3"), ln(mem, p + ".norm_y")
    a = mha(lin(hq, p + ".cross_attn.projq"), lin(hm, p + ".cross_attn.projk"),
            lin(hm, p + ".cross_attn.projv"))
    x = x + lin(a, p + ".cross_attn.proj")
    return x + lin(gelu(lin(ln(x, p + ".norm2"), p + ".mlp.fc1")), p + ".mlp.fc2")


def local_features(w, pre, enc, dec, gh, gw, r, C):
    """fc2(GELU(fc1(concat(enc, dec)))) per token, pixel shuffle by r:
    desc[r*y+i, r*x+j, c] = f[token (y, x), c*r*r + i*r + j], c < C."""
    cat = np.concatenate([f64(enc), f64(dec)], -1)
    h = gelu(linear(cat, w[pre + ".head_local_features.fc1.weight"],
                    w[pre + ".head_local_features.fc1.bias"]))
    f = linear(h, w[pre + ".head_local_features.fc2.weight"],
               w[pre + ".head_local_features.fc2.bias"])
    f = f[:, :C * r * r].reshape(gh, gw, C, r, r)
    return f.transpose(0, 3, 1, 4, 2).reshape(gh * r, gw * r, C)


def main():
    rng = np.random.default_rng(20261201)
    r32 = lambda *s: rng.standard_normal(s).astype(np.float32)
    g = {}
    g["lin_x"], g["lin_w"], g["lin_b"] = r32(4, 8), r32(6, 8), r32(6)
    g["lin_y"] = linear(g["lin_x"], g["lin_w"], g["lin_b"])
    g["ln_x"] = (r32(3, 16) * 3 + 1).astype(np.float32)
    g["ln_g"], g["ln_b"] = (1 + 0.1 * r32(16)).astype(np.float32), (0.1 * r32(16)).astype(np.float32)
    g["ln_y"] = layernorm(g["ln_x"], g["ln_g"], g["ln_b"], 1e-6)
    g["att_q"], g["att_k"], g["att_v"] = r32(1, 2, 5, 8), r32(1, 2, 5, 8), r32(1, 2, 5, 8)
    g["att_o"] = attention(g["att_q"], g["att_k"], g["att_v"], 8 ** -0.5)
    g["conv_x"], g["conv_w"], g["conv_b"] = r32(1, 5, 7, 3), (0.3 * r32(4, 3, 3, 3)).astype(np.float32), r32(4)
    g["conv_y"] = conv2d(g["conv_x"], g["conv_w"], g["conv_b"], pad=1)
    g["rope_t"] = r32(6, 64)
    g["rope_y"] = rope2d(g["rope_t"], 3)
    g["gelu_x"] = np.linspace(-4, 4, 17, dtype=np.float32)
    g["gelu_y"] = gelu(g["gelu_x"])
    # the same cases at shapes the device kernels take (K % 32, head dim 64,
    # Cin % 32)
    g["lin32_x"], g["lin32_w"], g["lin32_b"] = r32(4, 32), r32(6, 32), r32(6)
    g["lin32_y"] = linear(g["lin32_x"], g["lin32_w"], g["lin32_b"])
    g["att64_q"], g["att64_k"], g["att64_v"] = r32(1, 2, 5, 64), r32(1, 2, 7, 64), r32(1, 2, 7, 64)
    g["att64_o"] = attention(g["att64_q"], g["att64_k"], g["att64_v"], 0.125)
    g["conv32_x"], g["conv32_w"], g["conv32_b"] = r32(1, 5, 7, 32), (0.1 * r32(4, 32, 3, 3)).astype(np.float32), r32(4)
    g["conv32_y"] = conv2d(g["conv32_x"], g["conv32_w"], g["conv32_b"], pad=1)

    import gsplat_hip as G
    cfg = G.default_config(**TINY)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    gh = gw = 2
    hooks = [r32(1, gh * gw, 128) for _ in range(4)]
    for i in range(4):
        g[f"dpt_hook{i}"] = hooks[i]
    pts, conf = dpt_head(w, "downstream_head1", hooks, gh, gw, cfg.as_dict())
    g["dpt_pts"], g["dpt_conf"] = pts, conf
    # decoder block (both attentions with RoPE, non-trivial LayerNorm affine)
    # and the local-feature head, on the same 2x2 grid
    g["dec_x"], g["dec_mem"] = r32(1, gh * gw, 128), r32(1, gh * gw, 128)
    g["dec_y"] = decoder_block(w, "dec_blocks2.1", g["dec_x"][0], g["dec_mem"][0], 2, gw, 1e-6)[None]
    g["lf_enc"], g["lf_dec"] = r32(1, gh * gw, 128), r32(1, gh * gw, 128)
    g["lf_desc"] = local_features(w, "downstream_head2", g["lf_enc"][0], g["lf_dec"][0], gh, gw,
                                  16, 24)[None]
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **g)
    print({k: v.shape for k, v in g.items()})


if __name__ == "__main__":
    main()
