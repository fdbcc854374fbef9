"""Caller-side passes on the device against the oracle: resize_image,
preprocess_image, their fused form, collect_points compaction
(src/mastr/inference.cr:193-374), and the batched frames_to_pointcloud caller
(135-191). Image passes and compaction are bit-exact; the point cloud is
bit-exact against the same compaction of the device pair outputs and within
the fp32 tolerance of the oracle's full composition."""
import numpy as np
import pytest
import torch

import gsplat_hip as G
import pyoracle as O
from gpu_util import KEEP, assert_close, case, dev, empty, host, stream

pytestmark = pytest.mark.gpu


def _frames(F, h, w, seed=0, C=3):
    return np.random.default_rng(seed).random((F, h, w, C), dtype=np.float32)


@pytest.mark.parametrize("F,sh,sw,th,tw,C", [(3, 37, 53, 64, 96, 3), (2, 120, 90, 48, 64, 4),
                                              (1, 2, 2, 5, 3, 3), (2, 384, 512, 512, 512, 3)])
def test_resize_bit_exact(F, sh, sw, th, tw, C):
    case(f"resize {F}x{sh}x{sw}x{C} -> {th}x{tw}")
    fr = _frames(F, sh, sw, seed=sh, C=C)
    out = empty(F, th, tw, C)
    G.check(G.lib().gs_hip_resize_image(G.ptr(dev(fr)), F, sh, sw, C, th, tw, G.ptr(out),
                                        stream()))
    got = host(out)
    for f in range(F):
        np.testing.assert_array_equal(got[f], O.resize_image(fr[f], th, tw), err_msg=f"frame {f}")


def test_preprocess_and_prepare_bit_exact():
    case("preprocess / prepare_frames")
    fr = _frames(4, 64, 96, seed=1)
    out = empty(4, 3, 64, 96)
    G.check(G.lib().gs_hip_preprocess_image(G.ptr(dev(fr)), 4, 64, 96, G.ptr(out), stream()))
    np.testing.assert_array_equal(host(out), O.preprocess_image(fr))
    raw = _frames(3, 50, 70, seed=2)
    prep = empty(3, 3, 64, 96)
    G.check(G.lib().gs_hip_prepare_frames(G.ptr(dev(raw)), 3, 50, 70, 64, 96, G.ptr(prep),
                                          stream()))
    want = np.concatenate([O.preprocess_image(O.resize_image(f, 64, 96)[None]) for f in raw])
    np.testing.assert_array_equal(host(prep), want)


def test_image_pass_validation():
    case("image pass validation")
    x = empty(1, 4, 4, 3)
    with pytest.raises(G.GsError, match=">= 2"):
        G.check(G.lib().gs_hip_resize_image(G.ptr(x), 1, 4, 4, 3, 1, 8, G.ptr(x), stream()))
    with pytest.raises(G.GsError, match="null pointer"):
        G.check(G.lib().gs_hip_prepare_frames(G.ptr(x), 1, 4, 4, 8, 8, None, stream()))
    with pytest.raises(G.GsError, match="null pointer"):
        G.check(G.lib().gs_hip_preprocess_image(G.ptr(x), 1, 4, 4, None, stream()))
    with pytest.raises(G.GsError, match="bad sizes"):
        G.check(G.lib().gs_hip_preprocess_image(G.ptr(x), 1, 0, 4, G.ptr(x), stream()))


def _collect(pts, conf, thr, cap, count, ptsd=None, confd=None):
    n = conf.size
    op, oc = empty(max(cap, 1), 3), empty(max(cap, 1))
    G.check(G.lib().gs_hip_collect_points(G.ptr(ptsd if ptsd is not None else dev(pts)),
                                          G.ptr(confd if confd is not None else dev(conf)), n,
                                          thr, G.ptr(op), G.ptr(oc), cap, G.ptr(count),
                                          stream()))
    return op, oc


@pytest.mark.parametrize("n", [0, 1, 4095, 4096, 3 * 4096 + 5, 32 * 512 * 512])
def test_collect_points_bit_exact(n):
    case(f"collect_points n={n}")
    rng = np.random.default_rng(n)
    pts = rng.standard_normal((n, 3)).astype(np.float32)
    conf = (1 + rng.random(n) * 3).astype(np.float32)
    if n > 10:
        conf[3] = np.nan
        conf[7] = 2.5  # equal to the threshold: not selected
    wp, wc = O.collect_points(pts, conf, 2.5)
    count = torch.zeros(1, dtype=torch.int64, device="cuda")
    KEEP.append(count)
    op, oc = _collect(pts, conf, 2.5, n, count)
    k = int(host(count)[0])
    assert k == len(wc)
    np.testing.assert_array_equal(host(op)[:k], wp)
    np.testing.assert_array_equal(host(oc)[:k], wc)


def test_collect_points_append_and_overflow():
    case("collect_points append / overflow")
    rng = np.random.default_rng(9)
    pts = rng.standard_normal((2, 9000, 3)).astype(np.float32)
    conf = rng.random((2, 9000)).astype(np.float32)
    count = torch.zeros(1, dtype=torch.int64, device="cuda")
    KEEP.append(count)
    cap = 20000
    op, oc = empty(cap, 3), empty(cap)
    for i in range(2):  # appends at the running count
        G.check(G.lib().gs_hip_collect_points(G.ptr(dev(pts[i])), G.ptr(dev(conf[i])), 9000, 0.3,
                                              G.ptr(op), G.ptr(oc), cap, G.ptr(count), stream()))
    wp, wc = O.collect_points(pts, conf, 0.3)
    k = int(host(count)[0])
    assert k == len(wc)
    np.testing.assert_array_equal(host(op)[:k], wp)
    np.testing.assert_array_equal(host(oc)[:k], wc)
    # capacity below the count: the first cap points are written, the count is total
    count.zero_()
    small = 1000
    sp, sc = empty(small, 3), empty(small)
    G.check(G.lib().gs_hip_collect_points(G.ptr(dev(pts)), G.ptr(dev(conf)), 18000, 0.3,
                                          G.ptr(sp), G.ptr(sc), small, G.ptr(count), stream()))
    assert int(host(count)[0]) == len(wc)
    np.testing.assert_array_equal(host(sp), wp[:small])
    np.testing.assert_array_equal(host(sc), wc[:small])


def _tiny_model(tiny_cfg, max_pairs):
    cfg = G.default_config(**tiny_cfg)
    m = G.Mastr(cfg, max_pairs)
    m.init_seeded(0, 0.02, 0.1)
    return cfg, m


def test_frames_to_pointcloud_composition_bit_exact(tiny_cfg):
    """Chunked batched caller == per-pair device pair calls + the oracle's
    compaction of their outputs, bit for bit (5 frames, chunks of 2 pairs)."""
    case("frames_to_pointcloud composition")
    cfg, m = _tiny_model(tiny_cfg, 2)
    H, W = cfg.img_h, cfg.img_w
    F = 5
    raw = _frames(F, 50, 70, seed=3)
    rawd = dev(raw)
    # per-pair reference on the device
    prep = empty(F, 3, H, W)
    G.check(G.lib().gs_hip_prepare_frames(G.ptr(rawd), F, 50, 70, H, W, G.ptr(prep), stream()))
    p1, c1, p2, c2 = empty(1, H, W, 3), empty(1, H, W, 1), empty(1, H, W, 3), empty(1, H, W, 1)
    conf_all = []
    for i in range(F - 1):
        m.pair(prep[i:i + 1], prep[i + 1:i + 2], 1, p1, c1, None, p2, c2, None, stream())
        conf_all.append((host(p1).copy(), host(c1).copy()))
        if i == F - 2:
            conf_all.append((host(p2).copy(), host(c2).copy()))
    allc = np.concatenate([c.reshape(-1) for _, c in conf_all])
    thr = float(np.median(allc))
    wp = np.concatenate([O.collect_points(p, c, thr)[0] for p, c in conf_all])
    wc = np.concatenate([O.collect_points(p, c, thr)[1] for p, c in conf_all])
    cap = F * H * W
    op, oc = empty(cap, 3), empty(cap)
    k = m.frames_to_pointcloud(rawd, thr, op, oc, stream())
    assert k == len(wc) and 0 < k < cap
    np.testing.assert_array_equal(host(op)[:k], wp)
    np.testing.assert_array_equal(host(oc)[:k], wc)
    # fewer than two frames: empty cloud
    assert m.frames_to_pointcloud(rawd[:1], thr, op, oc, stream()) == 0
    m.close()


def test_frames_to_pointcloud_vs_oracle(tiny_cfg):
    """The reference's default threshold 0.3 against the oracle's composition
    (confidence 1+exp(.) > 1 selects every point, so the clouds align)."""
    case("frames_to_pointcloud vs oracle")
    cfg, m = _tiny_model(tiny_cfg, 3)
    F = 4
    raw = _frames(F, 40, 60, seed=4)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    rp, rc = O.frames_to_pointcloud(cfg.as_dict(), w, list(raw), 0.3)
    cap = F * cfg.img_h * cfg.img_w
    op, oc = empty(cap, 3), empty(cap)
    k = m.frames_to_pointcloud(dev(raw), 0.3, op, oc, stream())
    assert k == len(rc) == F * cfg.img_h * cfg.img_w
    assert_close(host(op)[:k], rp, name="points")
    assert_close(host(oc)[:k], rc, name="confidences")
    m.close()
