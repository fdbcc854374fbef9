"""Model-level parity of the graph entry points (gs_hip_mastr_*) against the
oracle composites: config 0 (one ViT-L block), config 1 (full encoder),
config 2 (full pair) at full size, the reduced TINY pair, and size-independent
properties (batch invariance, determinism) for the batched configs 3/4."""
import numpy as np
import pytest
import torch

import gsplat_hip as G
import pyoracle as O
from gpu_util import assert_close, assert_close_bf16, case, dev, empty, host, stream

pytestmark = pytest.mark.gpu


_W_CACHE, _REF_CACHE = {}, {}


def _cfg_key(cfg, drop=()):
    return tuple((k, tuple(v) if isinstance(v, list) else v) for k, v in sorted(cfg.as_dict().items())
                 if k not in drop)


def weights_for(cfg, seed=0, bias_std=0.0, ln_std=0.0, prefix=None):
    key = (_cfg_key(cfg, ("img_h", "img_w", "precision")), seed, bias_std, ln_std,
           tuple(prefix or ()))
    if key in _W_CACHE:
        return _W_CACHE[key]
    w = {}
    for i, (n, s, k) in enumerate(G.weight_inventory(cfg)):
        if prefix and not any(n.startswith(pf) for pf in prefix):
            continue
        w[n] = G.weight_values(cfg, i, int(np.prod(s)), seed, bias_std, ln_std).reshape(s)
    if prefix is None and bias_std == 0.0 and ln_std == 0.0:
        _W_CACHE.clear()  # keep one full weight set (2.75 GB) at a time
        _W_CACHE[key] = w
    return w


def oracle_pair(cfg, w, i1, i2):
    """O.mastr_pair of full-size seed-0 weights, cached per configuration and
    images (the counter-based generator makes pair 0 of a batch the same
    images as the single-pair tests, so their oracle runs are shared)."""
    import hashlib
    key = (_cfg_key(cfg, ("precision",)), hashlib.sha1(np.ascontiguousarray(i1)).hexdigest(),
           hashlib.sha1(np.ascontiguousarray(i2)).hexdigest())
    if key not in _REF_CACHE:
        O.set_threads(0)
        _REF_CACHE[key] = O.mastr_pair(cfg.as_dict(), w, i1, i2)
    return _REF_CACHE[key]


def load_ctx(cfg, w, max_pairs=1):
    m = G.Mastr(cfg, max_pairs)
    m.init_seeded(0)
    for n, a in w.items():
        m.set_weight(n, a)
    return m


@pytest.mark.parametrize("variant", ["spec", "biased", "literal"])
def test_config0_encoder_block(variant):
    """Config 0: one ViT-L block, 768 tokens on the 24x32 grid, RoPE2D base 100,
    eps 1e-6, N(0,0.02) weights; 'biased' adds nonzero biases and LN affine
    so those epilogues are exercised; 'literal' uses the reference CPU
    path's linear layout (D1)."""
    case(f"config0 block {variant}")
    cfg = G.default_config(enc_depth=1, dec_depth=1, dpt_hooks=[0, 1, 1, 1],
                           linear_layout=1 if variant == "literal" else 0)
    bias_std, ln_std = (0.02, 0.1) if variant == "biased" else (0.0, 0.0)
    w = weights_for(cfg, 0, bias_std, ln_std, prefix=["enc_blocks.0."])
    x = G.seed_normal(0, "tokens", 768 * 1024).reshape(1, 768, 1024)
    ref = O.encoder_block(cfg.as_dict(), w, "enc_blocks.0", x, 24, 32)
    m = load_ctx(cfg, w)
    xd = dev(x)
    m.encoder_block(0, xd, 1, stream())
    err = assert_close(host(xd), ref, name="config0")
    print(f"config0 {variant}: max abs err {err:.3e}")
    m.close()


def test_config1_encoder():
    """Config 1: full ViT-L encoder (24 blocks + enc_norm) on one 384x512 image."""
    case("config1 encoder")
    cfg = G.default_config()
    w = weights_for(cfg, prefix=["patch_embed.", "enc_blocks.", "enc_norm."])
    img = G.seed_uniform(0, "view1", 3 * 384 * 512, -1.0, 1.0).reshape(1, 3, 384, 512)
    ref = O.encoder(cfg.as_dict(), w, img)
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    enc = empty(1, 768, 1024)
    m.encoder(dev(img), 1, enc, stream())
    err = assert_close(host(enc), ref, name="config1")
    print(f"config1: max abs err {err:.3e}")
    m.close()


def run_pair(m, cfg, img1, img2, B):
    H, W = cfg.img_h, cfg.img_w
    out = {}
    for v in (1, 2):
        out[f"pts{v}"] = empty(B, H, W, 3)
        out[f"conf{v}"] = empty(B, H, W, 1)
        out[f"desc{v}"] = empty(B, H, W, cfg.desc_dim)
    m.pair(dev(img1), dev(img2), B, out["pts1"], out["conf1"], out["desc1"], out["pts2"],
           out["conf2"], out["desc2"], stream())
    return {k: host(v) for k, v in out.items()}


def check_pair(got, ref, tag):
    for k in ("pts1", "conf1", "desc1", "pts2", "conf2", "desc2"):
        err = assert_close(got[k], ref[k], name=f"{tag} {k}")
        print(f"{tag} {k}: max abs err {err:.3e}, |ref| max {np.abs(ref[k]).max():.3e}")


def test_tiny_pair_parity_and_taps(tiny_cfg):
    case("tiny pair")
    cfg = G.default_config(**tiny_cfg)
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    B = 2
    n = B * 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(0, "view1", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(0, "view2", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    m = load_ctx(cfg, w, max_pairs=B)
    got = run_pair(m, cfg, i1, i2, B)
    d = cfg.as_dict()
    check_pair(got, O.mastr_pair(d, w, i1, i2), "tiny")
    e1, e2, d1, d2 = O.mastr_pair_taps(d, w, i1, i2)
    N = (cfg.img_h // 16) * (cfg.img_w // 16)
    te = [empty(B, N, cfg.enc_dim) for _ in range(2)]
    td = [empty(B, N, cfg.dec_dim) for _ in range(2)]
    m.pair_taps(B, te[0], te[1], td[0], td[1], stream())
    for got_t, ref_t, nm in zip(te + td, [e1, e2, d1, d2], ["enc1", "enc2", "dec1", "dec2"]):
        assert_close(host(got_t), ref_t, name=nm)
    m.close()


def test_tiny_pair_f32x6_parity(tiny_cfg):
    """Precision 2 (fp32 GEMMs and convolutions through bf16x6 split
    products): the whole pair at the fp32 parity bar against the oracle."""
    case("tiny pair f32x6")
    cfg = G.default_config(**tiny_cfg, precision=2)
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    B = 2
    n = B * 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(0, "view1", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(0, "view2", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    m = load_ctx(cfg, w, max_pairs=B)
    got = run_pair(m, cfg, i1, i2, B)
    m.close()
    check_pair(got, O.mastr_pair(cfg.as_dict(), w, i1, i2), "tiny f32x6")


def test_config2_f32x6_vs_fp32():
    """Config 2 at full size in precision 2 against the fp32 MFMA path (itself
    checked against the oracle at this size): the fp32 parity bar."""
    case("config2 f32x6 vs fp32")
    n = 3 * 384 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, 384, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, 384, 512)
    outs = []
    for prec in (0, 2):
        cfg = G.default_config(precision=prec)
        m = G.Mastr(cfg, 1)
        m.init_seeded(0)
        outs.append(run_pair(m, cfg, i1, i2, 1))
        m.close()
        del m
        torch.cuda.empty_cache()
    for k in outs[0]:
        assert not np.array_equal(outs[0][k], outs[1][k])
    check_pair(outs[1], outs[0], "config2 f32x6")


def test_batched_f32x6_vs_fp32():
    """8 pairs at 384x512 in precision 2, where the launches are large enough
    for the bf16x6 attention kernel as well as the bf16x6 GEMMs: every pair
    against the fp32 MFMA path at the fp32 parity bar."""
    case("8 pairs f32x6 vs fp32")
    B = 8
    n = B * 3 * 384 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(B, 3, 384, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(B, 3, 384, 512)
    outs, kernels = [], None
    for prec in (0, 2):
        cfg = G.default_config(precision=prec)
        m = G.Mastr(cfg, B)
        m.init_seeded(0)
        if prec == 2:
            G.profile_begin()
        outs.append(run_pair(m, cfg, i1, i2, B))
        if prec == 2:
            torch.cuda.synchronize()
            kernels = G.profile_end()
        m.close()
        del m
        torch.cuda.empty_cache()
    assert any(k.startswith("attn_fwd_x6_kernel") for k in kernels), sorted(kernels)
    assert any(k.startswith("gemm_x6_kernel") for k in kernels), sorted(kernels)
    for b in (0, B - 1):
        check_pair({k: v[b] for k, v in outs[1].items()}, {k: v[b] for k, v in outs[0].items()},
                   f"8 pairs f32x6 pair {b}")


def test_ragged_grid_split_paths(tiny_cfg):
    """A 12x26 patch grid (312 tokens) at one pair: the small launches split K
    (GEMMs) and the key range (attention, last range ragged: 312 = 4 x 64 + 56)
    and must still match the oracle."""
    case("ragged grid 192x416 split paths")
    cfg = G.default_config(**dict(tiny_cfg, img_h=192, img_w=416))
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    n = 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(4, "view1", n).reshape(1, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(4, "view2", n).reshape(1, 3, cfg.img_h, cfg.img_w)
    m = load_ctx(cfg, w, max_pairs=1)
    got = run_pair(m, cfg, i1, i2, 1)
    check_pair(got, O.mastr_pair(cfg.as_dict(), w, i1, i2), "ragged")
    again = run_pair(m, cfg, i1, i2, 1)
    for k in got:  # fixed-order merges: deterministic
        np.testing.assert_array_equal(got[k], again[k])
    m.close()


def test_tiny_batch_invariance_and_determinism(tiny_cfg):
    """Pair p of a batch equals the same pair run alone, bit for bit, and a
    rerun is bit-identical (fixed-order reductions, no atomics). Kernel and
    K-split choices follow a launch's tile count, so the batch is sized for
    both batch sizes to pick the same kernel and split for every GEMM and
    conv: at three pairs the full-resolution head convs (3 x 64 x 96 rows,
    two views: 576 tiles of 64 rows) would move to the 64-row kernel."""
    case("tiny batch invariance")
    cfg = G.default_config(**tiny_cfg)
    B = 2
    n = B * 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(1, "view1", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(1, "view2", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    m = G.Mastr(cfg, B)
    m.init_seeded(0, 0.02, 0.1)
    full = run_pair(m, cfg, i1, i2, B)
    again = run_pair(m, cfg, i1, i2, B)
    for k in full:
        np.testing.assert_array_equal(full[k], again[k])
    for b in (0, B - 1):
        one = run_pair(m, cfg, i1[b:b + 1], i2[b:b + 1], 1)
        for k in full:
            np.testing.assert_array_equal(one[k][0], full[k][b], err_msg=f"{k} pair {b}")
    m.close()


def test_config2_full_pair():
    """Config 2: full MASt3R two-view inference at 384x512, seed-0 weights."""
    case("config2 full pair")
    cfg = G.default_config()
    w = weights_for(cfg)
    n = 3 * 384 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, 384, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, 384, 512)
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    got = run_pair(m, cfg, i1, i2, 1)
    m.close()
    del m
    torch.cuda.empty_cache()
    ref = oracle_pair(cfg, w, i1, i2)
    check_pair(got, ref, "config2")


def test_config4_grid_pair():
    """Config 4 geometry: 512x512 images (32x32 grid, 1024 tokens), full model,
    one pair against the oracle; the batched 32-pair run is covered by batch
    invariance below."""
    case("config4 512x512 pair")
    cfg = G.default_config(img_h=512, img_w=512)
    w = weights_for(cfg)
    n = 3 * 512 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, 512, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, 512, 512)
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    got = run_pair(m, cfg, i1, i2, 1)
    m.close()
    del m
    torch.cuda.empty_cache()
    ref = oracle_pair(cfg, w, i1, i2)
    check_pair(got, ref, "config4")


def test_config4_batch_invariance_32_pairs():
    """32 pairs at 512x512 in one launch sequence: pairs 0 and 31 equal the
    same pairs run alone. A single pair leaves CUs idle, so its small GEMMs
    split K (a different fp32 summation order), hence the parity tolerance
    rather than bit equality (measured: <= 2.1e-5 abs on desc, 2.4e-7 on
    conf)."""
    case("config4 32-pair batch invariance")
    cfg = G.default_config(img_h=512, img_w=512)
    B = 32
    n = B * 3 * 512 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(B, 3, 512, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(B, 3, 512, 512)
    m = G.Mastr(cfg, B)
    m.init_seeded(0)
    full = run_pair(m, cfg, i1, i2, B)
    for b in (0, B - 1):
        one = run_pair(m, cfg, i1[b:b + 1], i2[b:b + 1], 1)
        for k in full:
            err = assert_close(one[k][0], full[k][b], name=f"{k} pair {b}")
            print(f"pair {b} {k}: max abs diff single vs batched {err:.2e}")
    m.close()


@pytest.mark.parametrize("precision", [0, 2])
def test_config3_16_pairs(precision):
    """Config 3, the benchmark workload: 16 pairs at 384x512 in one launch
    sequence, fp32 (precision 0) and fp32 through bf16x6 split products
    (precision 2, the bench line's fp32x6 variant). Pairs 0 and 15 against
    the oracle at the fp32 bar (1e-3 relative + 1e-4 absolute per element);
    a rerun is bit-identical. The oracle outputs are cached across the two
    precisions (same weights, same images)."""
    case(f"config3 16 pairs precision {precision}")
    cfg = G.default_config(precision=precision)
    B = 16
    n = 3 * 384 * 512
    i1 = G.seed_uniform(0, "view1", B * n).reshape(B, 3, 384, 512)
    i2 = G.seed_uniform(0, "view2", B * n).reshape(B, 3, 384, 512)
    m = G.Mastr(cfg, B)
    m.init_seeded(0)
    full = run_pair(m, cfg, i1, i2, B)
    again = run_pair(m, cfg, i1, i2, B)
    for k in full:
        np.testing.assert_array_equal(full[k], again[k], err_msg=f"rerun {k}")
    m.close()
    del m, again
    torch.cuda.empty_cache()
    w = weights_for(cfg)
    for b in (0, B - 1):
        ref = oracle_pair(cfg, w, i1[b:b + 1], i2[b:b + 1])
        check_pair({k: v[b:b + 1] for k, v in full.items()}, ref,
                   f"config3 precision {precision} pair {b}")


def test_config4_bf16_32_pairs():
    """Config 4 in the bf16-input / fp32-accumulate variant at its own
    workload: 32 pairs at 512x512 in one launch sequence, pairs 0 and 31
    against the fp32 oracle at 2e-2 relative (norm-wise, worst element within
    2e-2 of the tensor maximum; the element-wise 99.9th-percentile relative
    error is printed)."""
    case("config4 bf16 32 pairs")
    cfg = G.default_config(img_h=512, img_w=512, precision=1)
    B = 32
    n = 3 * 512 * 512
    i1 = G.seed_uniform(0, "view1", B * n).reshape(B, 3, 512, 512)
    i2 = G.seed_uniform(0, "view2", B * n).reshape(B, 3, 512, 512)
    m = G.Mastr(cfg, B)
    m.init_seeded(0)
    full = run_pair(m, cfg, i1, i2, B)
    m.close()
    del m
    torch.cuda.empty_cache()
    w = weights_for(cfg)
    for b in (0, B - 1):
        ref = oracle_pair(cfg, w, i1[b:b + 1], i2[b:b + 1])
        for k in ref:
            rel, worst, p999 = assert_close_bf16(full[k][b:b + 1], ref[k],
                                                 name=f"config4 bf16 pair {b} {k}")
            print(f"config4 bf16 pair {b} {k}: rel {rel:.2e} worst {worst:.2e} "
                  f"p99.9 elementwise {p999:.2e}")


def test_tiny_pair_bf16_variant(tiny_cfg):
    """bf16-input / fp32-accumulate GEMMs and attention vs the fp32 oracle."""
    case("tiny pair bf16")
    cfg = G.default_config(**tiny_cfg, precision=1)
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    n = 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, cfg.img_h, cfg.img_w)
    m = load_ctx(cfg, w)
    got = run_pair(m, cfg, i1, i2, 1)
    m.close()
    ref = O.mastr_pair(cfg.as_dict(), w, i1, i2)
    for k in ref:
        rel, worst, p999 = assert_close_bf16(got[k], ref[k], name=f"tiny bf16 {k}")
        print(f"tiny bf16 {k}: rel {rel:.2e} worst {worst:.2e} p99.9 elementwise {p999:.2e}")


def test_config4_bf16_vs_fp32():
    """Config 4 in the bf16 variant: one 512x512 pair against the fp32 oracle
    outputs at 2e-2 relative (the batched 32-pair run is position-invariant,
    as the fp32 test shows for the shared kernels)."""
    case("config4 bf16 pair")
    cfg = G.default_config(img_h=512, img_w=512, precision=1)
    w = weights_for(cfg)
    n = 3 * 512 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, 512, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, 512, 512)
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    got = run_pair(m, cfg, i1, i2, 1)
    m.close()
    del m
    torch.cuda.empty_cache()
    ref = oracle_pair(cfg, w, i1, i2)
    for k in ref:
        rel, worst, p999 = assert_close_bf16(got[k], ref[k], name=f"config4 bf16 {k}")
        print(f"config4 bf16 {k}: rel {rel:.2e} worst {worst:.2e} p99.9 elementwise {p999:.2e}")


def test_graph_replay_matches_eager(tiny_cfg):
    """hipGraph replay of the pair sequence: several replays, with eager work,
    synchronisation and in-place input changes between them; every replay is
    bit-identical to the eager run on the same inputs."""
    case("graph replay")
    cfg = G.default_config(**tiny_cfg)
    B = 2
    n = B * 3 * cfg.img_h * cfg.img_w
    shape = (B, 3, cfg.img_h, cfg.img_w)
    imgs = [(G.seed_uniform(s, "view1", n).reshape(shape), G.seed_uniform(s, "view2", n).reshape(shape))
            for s in range(3)]
    m = G.Mastr(cfg, B)
    m.init_seeded(0, 0.02, 0.1)
    st = torch.cuda.Stream()
    H, W = cfg.img_h, cfg.img_w
    with torch.cuda.stream(st):
        i1, i2 = dev(imgs[0][0]), dev(imgs[0][1])
        outs = [empty(B, H, W, c) for c in (3, 1, cfg.desc_dim, 3, 1, cfg.desc_dim)]
        eager = []
        for a, b in imgs:
            i1.copy_(torch.from_numpy(a).to("cuda", non_blocking=False))
            i2.copy_(torch.from_numpy(b).to("cuda", non_blocking=False))
            m.pair(i1, i2, B, *outs, stream=st.cuda_stream)
            eager.append([host(o).copy() for o in outs])
        m.set_graph(True)
        for rep in range(2):
            for j, (a, b) in enumerate(imgs):
                i1.copy_(torch.from_numpy(a).to("cuda"))
                i2.copy_(torch.from_numpy(b).to("cuda"))
                junk = torch.randn(1 << 20, device="cuda") * 2  # eager work between replays
                m.pair(i1, i2, B, *outs, stream=st.cuda_stream)
                torch.cuda.synchronize()
                del junk
                for o, e in zip(outs, eager[j]):
                    np.testing.assert_array_equal(host(o), e, err_msg=f"replay {rep} input {j}")
        m.set_graph(False)
    m.close()


def test_view_swap_symmetry_full_size():
    """With the second decoder chain and head sharing the first's weights,
    swapping the views swaps the outputs (bit for bit) at the config-2 size."""
    case("config2 view swap")
    cfg = G.default_config(enc_depth=2, dec_depth=2, dpt_hooks=[0, 1, 2, 2])
    inv = G.weight_inventory(cfg)
    m = G.Mastr(cfg, 1)
    w = {}
    for i, (nme, s, k) in enumerate(inv):
        src = nme.replace("dec_blocks2.", "dec_blocks.").replace("downstream_head2.",
                                                                  "downstream_head1.")
        j = [x[0] for x in inv].index(src)
        a = G.weight_values(cfg, j, int(np.prod(s)), 0, 0.02, 0.1)
        m.set_weight(nme, a)
    n = 3 * 384 * 512
    i1 = G.seed_uniform(3, "view1", n).reshape(1, 3, 384, 512)
    i2 = G.seed_uniform(3, "view2", n).reshape(1, 3, 384, 512)
    a = run_pair(m, cfg, i1, i2, 1)
    b = run_pair(m, cfg, i2, i1, 1)
    for k in ("pts", "conf", "desc"):
        np.testing.assert_array_equal(a[k + "1"], b[k + "2"])
        np.testing.assert_array_equal(a[k + "2"], b[k + "1"])
    m.close()


def test_entry_points_reject_bad_arguments(tiny_cfg):
    """The graph entry points check batch sizes and pointers on the host and
    return an error with its reason before any launch (batch 0, negative,
    above the context's capacity; null images; pts without conf); the
    context stays usable and a valid call afterwards matches the oracle."""
    case("entry point argument checks")
    cfg = G.default_config(**tiny_cfg)
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    m = load_ctx(cfg, w, max_pairs=2)
    H, W = cfg.img_h, cfg.img_w
    n = 3 * H * W
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, H, W)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, H, W)
    d1, d2 = dev(i1), dev(i2)
    pts, conf = empty(3, H, W, 3), empty(3, H, W, 1)
    for B in (0, -1, 3):
        with pytest.raises(G.GsError, match="B exceeds context capacity"):
            m.pair(d1, d2, B, pts, conf, None, pts, conf, None, stream())
    with pytest.raises(G.GsError, match="null image"):
        m.pair(None, d2, 1, pts, conf, None, pts, conf, None, stream())
    with pytest.raises(G.GsError, match="pts and conf must be given together"):
        m.pair(d1, d2, 1, pts, None, None, None, None, None, stream())
    N = (H // cfg.patch) * (W // cfg.patch)
    enc = empty(5, N, cfg.enc_dim)
    for B in (0, 5):
        with pytest.raises(G.GsError, match="encoder: B exceeds context capacity"):
            m.encoder(d1, B, enc, stream())
    with pytest.raises(G.GsError, match="encoder: null argument"):
        m.encoder(None, 1, enc, stream())
    check_pair(run_pair(m, cfg, i1, i2, 1), O.mastr_pair(cfg.as_dict(), w, i1, i2), "after errors")
    m.close()
