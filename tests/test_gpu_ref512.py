"""The reference-literal composition (composite 1, "ref512"): own-view decoder
memory, stub DPT heads on the patch grid, sigmoid confidence
(src/mastr/decoder_v2.cr:170-191, 502-530, 619-655; src/mastr/inference.cr:
92-115), on the device against the oracle's composite 1."""
import numpy as np
import pytest

import gsplat_hip as G
import pyoracle as O
from gpu_util import assert_close, case, dev, empty, host, stream

pytestmark = pytest.mark.gpu


def _pair(m, cfg, i1, i2, B):
    gh, gw = cfg.img_h // cfg.patch, cfg.img_w // cfg.patch
    out = {k: empty(B, gh, gw, c) for k, c in (("pts1", 3), ("conf1", 1), ("pts2", 3),
                                                 ("conf2", 1))}
    m.pair(i1, i2, B, out["pts1"], out["conf1"], None, out["pts2"], out["conf2"], None, stream())
    return {k: host(v) for k, v in out.items()}


def _check(got, ref, tag):
    for k in got:
        err = assert_close(got[k], ref[k], name=f"{tag} {k}")
        print(f"{tag} {k}: max abs err {err:.3e}")


def test_tiny_ref_composite(tiny_cfg):
    case("tiny ref composite")
    cfg = G.default_config(**dict(tiny_cfg, composite=1, rope_mode=2, ln_eps=1e-5))
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    B = 2
    n = B * 3 * cfg.img_h * cfg.img_w
    i1 = G.seed_uniform(2, "view1", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    i2 = G.seed_uniform(2, "view2", n).reshape(B, 3, cfg.img_h, cfg.img_w)
    m = G.Mastr(cfg, B)
    m.init_seeded(0, 0.02, 0.1)
    got = _pair(m, cfg, dev(i1), dev(i2), B)
    ref = O.mastr_pair(cfg.as_dict(), w, i1, i2)
    _check(got, {k: ref[k] for k in got}, "tiny ref")
    with pytest.raises(G.GsError, match="no descriptor head"):
        d = empty(B, cfg.img_h, cfg.img_w, cfg.desc_dim)
        m.pair(dev(i1), dev(i2), B, None, None, d, None, None, None, stream())
    m.close()


def test_ref512_forward_pair_from_unit_images():
    """MASt3RInference#forward_pair literally: [0,1] NHWC images ->
    preprocess_image -> encoder / decoder / stub heads at 512x512."""
    case("ref512 forward_pair")
    cfg = G.ref512_config()
    w = G.seeded_weights(cfg)
    H, W = cfg.img_h, cfg.img_w
    rng = np.random.default_rng(7)
    u1 = rng.random((1, H, W, 3), dtype=np.float32)
    u2 = rng.random((1, H, W, 3), dtype=np.float32)
    p1, p2 = empty(1, 3, H, W), empty(1, 3, H, W)
    for u, p in ((u1, p1), (u2, p2)):
        G.check(G.lib().gs_hip_preprocess_image(G.ptr(dev(u)), 1, H, W, G.ptr(p), stream()))
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    got = _pair(m, cfg, p1, p2, 1)
    ref = O.mastr_pair(cfg.as_dict(), w, O.preprocess_image(u1), O.preprocess_image(u2))
    _check(got, {k: ref[k] for k in got}, "ref512")
    assert got["pts1"].shape == (1, 32, 32, 3)
    m.close()


def test_ref_frames_to_pointcloud(tiny_cfg):
    """frames_to_pointcloud over the reference composition: sigmoid confidences
    make the threshold bite; it is placed in a gap of the oracle's confidences
    at least 1e-3 wide so fp32 rounding cannot flip a point."""
    case("ref frames_to_pointcloud")
    cfg = G.default_config(**dict(tiny_cfg, composite=1, rope_mode=2, ln_eps=1e-5))
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    F = 6
    raw = np.random.default_rng(8).random((F, 50, 70, 3), dtype=np.float32)
    _, rc_all = O.frames_to_pointcloud(cfg.as_dict(), w, list(raw), -1.0)
    sc = np.sort(rc_all)
    mid = len(sc) // 2
    gaps = [(sc[i + 1] - sc[i], i) for i in range(len(sc) - 1) if sc[i + 1] - sc[i] > 1e-3]
    assert gaps, "no confidence gap"
    _, i = min(gaps, key=lambda g: abs(g[1] - mid))
    thr = float((sc[i] + sc[i + 1]) / 2)
    rp, rc = O.frames_to_pointcloud(cfg.as_dict(), w, list(raw), thr)
    m = G.Mastr(cfg, 2)
    m.init_seeded(0, 0.02, 0.1)
    cap = len(rc_all)
    op, oc = empty(cap, 3), empty(cap)
    k = m.frames_to_pointcloud(dev(raw), thr, op, oc, stream())
    assert k == len(rc) and 0 < k < cap
    assert_close(host(op)[:k], rp, name="points")
    assert_close(host(oc)[:k], rc, name="confidences")
    m.close()
