"""Golden fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py from the mathematics in float64 numpy): the
oracle on the CPU and the device kernels on the GPU against them."""
import os

import numpy as np
import pytest

import gsplat_hip as G
import pyoracle as O

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))

TINY_DPT = dict(img_h=32, img_w=32, patch=16, enc_dim=128, enc_depth=2, enc_heads=2,
                enc_mlp=256, dec_dim=128, dec_depth=3, dec_heads=2, dec_mlp=256, dpt_feat=64,
                dpt_dims=[32, 64, 96, 128], dpt_hooks=[0, 1, 2, 3], head_mid=32,
                lf_hidden=256, desc_dim=24)


def close(got, want, rtol, atol):
    np.testing.assert_allclose(np.asarray(got, np.float64), want, rtol=rtol, atol=atol)


# ---- oracle (CPU) -----------------------------------------------------------

def test_oracle_linear_layernorm_gelu():
    g = GOLD
    close(O.linear(g["lin_x"], g["lin_w"], g["lin_b"]), g["lin_y"], 1e-6, 1e-6)
    close(O.linear(g["lin32_x"], g["lin32_w"], g["lin32_b"]), g["lin32_y"], 1e-6, 2e-6)
    close(O.layernorm(g["ln_x"], g["ln_g"], g["ln_b"], 1e-6), g["ln_y"], 1e-6, 1e-6)
    close(O.gelu(g["gelu_x"]), g["gelu_y"], 1e-6, 1e-7)


def test_oracle_attention_conv_rope():
    g = GOLD
    close(O.sdpa(g["att_q"], g["att_k"], g["att_v"], float(np.float32(8 ** -0.5))), g["att_o"],
          1e-5, 1e-6)
    close(O.sdpa(g["att64_q"], g["att64_k"], g["att64_v"], 0.125), g["att64_o"], 1e-5, 1e-6)
    close(O.conv2d(g["conv_x"], g["conv_w"], g["conv_b"], 1, 1), g["conv_y"], 1e-6, 1e-6)
    close(O.conv2d(g["conv32_x"], g["conv32_w"], g["conv32_b"], 1, 1), g["conv32_y"], 1e-5, 1e-6)
    close(O.rope2d(g["rope_t"][None], 1, 3, 100.0)[0], g["rope_y"], 1e-5, 1e-6)


def test_oracle_dpt_head_2x2_grid():
    cfg = G.default_config(**TINY_DPT)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    hooks = [GOLD[f"dpt_hook{i}"] for i in range(4)]
    pts, conf = O.dpt_head(cfg.as_dict(), w, "downstream_head1", hooks, 2, 2)
    close(pts, GOLD["dpt_pts"], 1e-4, 1e-5)
    close(conf, GOLD["dpt_conf"], 1e-4, 1e-5)


def test_oracle_decoder_block_2x2_grid():
    """Decoder block (RoPE2D on both attentions, norm_y on the memory,
    reference role names) against the float64 golden; each planted
    composition mistake fails it."""
    cfg = G.default_config(**TINY_DPT)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    d = cfg.as_dict()
    run = lambda: O.decoder_block(d, w, "dec_blocks2.1", GOLD["dec_x"], GOLD["dec_mem"], 2, 2)
    close(run(), GOLD["dec_y"], 1e-4, 1e-5)
    for m in (O.MUT_NO_NORM_Y, O.MUT_NO_CROSS_ROPE, O.MUT_NORM_ROLES):
        with O.mutation(m):
            with pytest.raises(AssertionError):
                close(run(), GOLD["dec_y"], 1e-4, 1e-5)


def test_oracle_local_features_2x2_grid():
    """Local-feature head (concat(enc, dec) -> fc1 -> GELU -> fc2 -> x16 pixel
    shuffle -> channels 0..23) against the float64 golden; the swapped concat
    fails it."""
    cfg = G.default_config(**TINY_DPT)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    d = cfg.as_dict()
    run = lambda: O.local_features(d, w, "downstream_head2", GOLD["lf_enc"], GOLD["lf_dec"], 2, 2)
    close(run(), GOLD["lf_desc"], 1e-4, 1e-5)
    with O.mutation(O.MUT_CONCAT_SWAP):
        with pytest.raises(AssertionError):
            close(run(), GOLD["lf_desc"], 1e-4, 1e-5)


# ---- device kernels (GPU) -----------------------------------------------------

@pytest.mark.gpu
def test_device_kernels_against_golden():
    import torch

    from gpu_util import case, dev, empty, host, stream
    case("golden fixtures on the device")
    g, L, p = GOLD, G.lib(), G.ptr
    y = empty(4, 6)
    G.check(L.gs_hip_linear(p(dev(g["lin32_x"])), p(dev(g["lin32_w"])), p(dev(g["lin32_b"])),
                            p(y), 4, 32, 6, 0, 0, None, stream()))
    close(host(y), g["lin32_y"], 1e-3, 1e-4)
    y = empty(3, 16)
    G.check(L.gs_hip_layernorm(p(dev(g["ln_x"])), p(dev(g["ln_g"])), p(dev(g["ln_b"])), p(y), 3,
                               16, 1e-6, stream()))
    close(host(y), g["ln_y"], 1e-5, 1e-6)
    q, k, v = dev(g["att64_q"]), dev(g["att64_k"]), dev(g["att64_v"])
    o = empty(1, 2, 5, 64)
    st = lambda n: (2 * n * 64, n * 64, 64)  # [B, H, N, 64] strides
    G.check(L.gs_hip_attention(p(q), p(k), p(v), p(o), 1, 2, 5, 7, 64, 0.125, *st(5), *st(7),
                               *st(7), *st(5), stream()))
    close(host(o), g["att64_o"], 1e-3, 1e-4)
    y = empty(1, 5, 7, 4)
    G.check(L.gs_hip_conv2d(p(dev(g["conv32_x"])), 1, 5, 7, 32, p(dev(g["conv32_w"])),
                            p(dev(g["conv32_b"])), p(y), 4, 3, 1, 1, 0, 0, None, stream()))
    close(host(y), g["conv32_y"], 1e-3, 1e-4)
    t = dev(g["rope_t"][None])
    G.check(L.gs_hip_rope2d(p(t), 1, 6, 1, 64, 3, 100.0, stream()))
    close(host(t)[0], g["rope_y"], 1e-5, 1e-5)
