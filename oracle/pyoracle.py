"""ctypes wrapper of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, always as the checker. Arrays are float32 numpy arrays.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

vp = C.c_void_p


class OrcConfig(C.Structure):
    _fields_ = [
        ("img_h", C.c_int32), ("img_w", C.c_int32), ("patch", C.c_int32),
        ("enc_dim", C.c_int32), ("enc_depth", C.c_int32), ("enc_heads", C.c_int32),
        ("enc_mlp", C.c_int32),
        ("dec_dim", C.c_int32), ("dec_depth", C.c_int32), ("dec_heads", C.c_int32),
        ("dec_mlp", C.c_int32),
        ("dpt_feat", C.c_int32),
        ("dpt_dims", C.c_int32 * 4),
        ("dpt_hooks", C.c_int32 * 4),
        ("head_mid", C.c_int32),
        ("lf_hidden", C.c_int32),
        ("desc_dim", C.c_int32),
        ("ln_eps", C.c_float),
        ("rope_base", C.c_float),
        ("linear_layout", C.c_int32),
        ("rope_mode", C.c_int32),
        ("composite", C.c_int32),
    ]


WEIGHT_FN = C.CFUNCTYPE(vp, C.c_char_p, vp)

_SIGS = [
    ("orc_set_threads", None, [C.c_int32]),
    ("orc_get_threads", C.c_int32, []),
    ("orc_linear", None, [vp, C.c_int64, C.c_int32, vp, vp, C.c_int32, vp, C.c_int32]),
    ("orc_linear_naive", None, [vp, C.c_int64, C.c_int32, vp, vp, C.c_int32, vp, C.c_int32]),
    ("orc_layernorm", None, [vp, C.c_int64, C.c_int32, vp, vp, C.c_float, vp]),
    ("orc_gelu", None, [vp, C.c_int64, vp]),
    ("orc_relu", None, [vp, C.c_int64, vp]),
    ("orc_add", None, [vp, vp, C.c_int64, vp]),
    ("orc_sdpa", None, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                        C.c_float]),
    ("orc_sdpa_naive", None, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                              C.c_int32, C.c_float]),
    ("orc_set_naive", None, [C.c_int32]),
    ("orc_rope_table", None, [C.c_int32, C.c_int32, C.c_float, vp, vp]),
    ("orc_rope2d", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float]),
    ("orc_rope_ref_token", None, [vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_float]),
    ("orc_unfold", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_conv2d", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp, C.c_int32,
                          C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_conv2d_naive", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp, C.c_int32,
                                C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_conv2d_hw", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp, C.c_int32,
                             C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_conv2d_hw_naive", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp,
                                   C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_conv_transpose", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp,
                                  C.c_int32, C.c_int32, vp]),
    ("orc_upsample2x", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_pixel_shuffle", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                 C.c_int32, vp]),
    ("orc_resize_image", None, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_preprocess_image", None, [vp, C.c_int32, C.c_int32, C.c_int32, vp]),
    ("orc_collect_points", C.c_int64, [vp, vp, C.c_int64, C.c_float, vp, vp]),
    ("orc_encoder_block", C.c_int32, [C.POINTER(OrcConfig), C.c_char_p, WEIGHT_FN, vp, vp,
                                      C.c_int32, C.c_int32, C.c_int32]),
    ("orc_encoder", C.c_int32, [C.POINTER(OrcConfig), WEIGHT_FN, vp, vp, C.c_int32, vp]),
    ("orc_mastr_pair", C.c_int32, [C.POINTER(OrcConfig), WEIGHT_FN, vp, vp, vp, C.c_int32, vp, vp,
                                   vp, vp, vp, vp]),
    ("orc_dpt_head", C.c_int32, [C.POINTER(OrcConfig), WEIGHT_FN, vp, C.c_char_p, C.POINTER(vp),
                                 C.c_int32, C.c_int32, C.c_int32, vp, vp]),
    ("orc_mastr_pair_taps", C.c_int32, [C.POINTER(OrcConfig), WEIGHT_FN, vp, vp, vp, C.c_int32,
                                        vp, vp, vp, vp]),
    ("orc_set_mutation", None, [C.c_int32]),
    ("orc_decoder_block", C.c_int32, [C.POINTER(OrcConfig), C.c_char_p, WEIGHT_FN, vp, vp, vp,
                                      C.c_int32, C.c_int32, C.c_int32]),
    ("orc_local_features", C.c_int32, [C.POINTER(OrcConfig), WEIGHT_FN, vp, C.c_char_p, vp, vp,
                                       C.c_int32, C.c_int32, C.c_int32, vp]),
]

# Planted composition mistakes of orc_set_mutation (tests only).
MUT_MEMORY_FIXED, MUT_NO_NORM_Y, MUT_NO_CROSS_ROPE, MUT_CONCAT_SWAP, MUT_NORM_ROLES = 1, 2, 3, 4, 5
MUT_HOOKS_SWAPPED, MUT_HEADS_CROSSED, MUT_HOOK3_PRE_NORM = 6, 7, 8

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle wants contiguous float32"
    return a.ctypes.data_as(vp)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n):
    lib().orc_set_threads(n)


def linear(x, W, b=None, layout=0, naive=False):
    x = f32(x)
    W = f32(W)
    K = x.shape[-1]
    M = x.size // K
    N = W.shape[0] if layout == 0 else W.size // K
    y = np.empty(x.shape[:-1] + (N,), np.float32)
    fn = lib().orc_linear_naive if naive else lib().orc_linear
    fn(_p(x), M, K, _p(W), _p(f32(b) if b is not None else None), N, _p(y), layout)
    return y


def layernorm(x, g, b, eps):
    x = f32(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_layernorm(_p(x), x.size // D, D, _p(f32(g)), _p(f32(b)), eps, _p(y))
    return y


def gelu(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_gelu(_p(x), x.size, _p(y))
    return y


def set_naive(on):
    lib().orc_set_naive(1 if on else 0)


def sdpa(q, k, v, scale=None, naive=False):
    """q [B,H,Nq,hd], k/v [B,H,Nkv,hd]."""
    q, k, v = f32(q), f32(k), f32(v)
    B, H, Nq, hd = q.shape
    Nkv = k.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    o = np.empty_like(q)
    fn = lib().orc_sdpa_naive if naive else lib().orc_sdpa
    fn(_p(q), _p(k), _p(v), _p(o), B, H, Nq, Nkv, hd, scale)
    return o


def rope_table(max_pos, hd, base):
    c = np.empty((max_pos, hd // 4), np.float32)
    s = np.empty((max_pos, hd // 4), np.float32)
    lib().orc_rope_table(max_pos, hd, base, _p(c), _p(s))
    return c, s


def rope2d(t, H, grid_w, base, hd=64):
    """t [B, N, H*hd] -> rotated copy."""
    t = f32(t).copy()
    B, N, _ = t.shape
    lib().orc_rope2d(_p(t), B, N, H, hd, grid_w, base)
    return t


def rope_ref_token(x, grid_h, grid_w, H, base):
    x = f32(x)
    B, N, D = x.shape
    y = np.empty_like(x)
    lib().orc_rope_ref_token(_p(x), _p(y), B, grid_h, grid_w, D, H, base)
    return y


def unfold(img, p):
    img = f32(img)
    B, Cc, H, W = img.shape
    out = np.empty((B, (H // p) * (W // p), Cc * p * p), np.float32)
    lib().orc_unfold(_p(img), B, Cc, H, W, p, _p(out))
    return out


def conv2d(x, w, b=None, stride=1, pad=0, naive=False):
    """x NHWC, w OIHW [Cout, Cin, kh, kw] (kh != kw allowed)."""
    x, w = f32(x), f32(w)
    B, H, W, Cin = x.shape
    Cout, _, kh, kw = w.shape
    Ho = (H + 2 * pad - kh) // stride + 1
    Wo = (W + 2 * pad - kw) // stride + 1
    y = np.empty((B, Ho, Wo, Cout), np.float32)
    bp = _p(f32(b) if b is not None else None)
    if kh == kw:
        fn = lib().orc_conv2d_naive if naive else lib().orc_conv2d
        fn(_p(x), B, H, W, Cin, _p(w), bp, Cout, kh, stride, pad, _p(y))
    else:
        fn = lib().orc_conv2d_hw_naive if naive else lib().orc_conv2d_hw
        fn(_p(x), B, H, W, Cin, _p(w), bp, Cout, kh, kw, stride, pad, _p(y))
    return y


def conv_transpose(x, w, b, k):
    """x NHWC, w [Cin, Cout, k, k]."""
    x, w = f32(x), f32(w)
    B, H, W, Cin = x.shape
    Cout = w.shape[1]
    y = np.empty((B, H * k, W * k, Cout), np.float32)
    lib().orc_conv_transpose(_p(x), B, H, W, Cin, _p(w), _p(f32(b) if b is not None else None),
                             Cout, k, _p(y))
    return y


def upsample2x(x):
    x = f32(x)
    B, H, W, Cc = x.shape
    y = np.empty((B, 2 * H, 2 * W, Cc), np.float32)
    lib().orc_upsample2x(_p(x), B, H, W, Cc, _p(y))
    return y


def pixel_shuffle(f, h, w, r, Cout):
    f = f32(f)
    B, _, Cf = f.shape
    out = np.empty((B, h * r, w * r, Cout), np.float32)
    lib().orc_pixel_shuffle(_p(f), B, h, w, Cf, r, Cout, _p(out))
    return out


def resize_image(img, th, tw):
    """[sh, sw, C] -> [th, tw, C] (src/mastr/inference.cr:330-374)."""
    img = f32(img)
    sh, sw, Cc = img.shape
    out = np.empty((th, tw, Cc), np.float32)
    lib().orc_resize_image(_p(img), sh, sw, Cc, th, tw, _p(out))
    return out


def preprocess_image(img):
    """[B, H, W, 3] -> [B, 3, H, W] (src/mastr/inference.cr:193-229)."""
    img = f32(img)
    B, H, W, _ = img.shape
    out = np.empty((B, 3, H, W), np.float32)
    lib().orc_preprocess_image(_p(img), B, H, W, _p(out))
    return out


def collect_points(pts, conf, threshold):
    """pts [..., 3], conf [...] -> (points [k, 3], confs [k])."""
    pts = f32(pts).reshape(-1, 3)
    conf = f32(conf).reshape(-1)
    assert pts.shape[0] == conf.shape[0]
    op = np.empty_like(pts)
    oc = np.empty_like(conf)
    k = lib().orc_collect_points(_p(pts), _p(conf), conf.shape[0], threshold, _p(op), _p(oc))
    return op[:k].copy(), oc[:k].copy()


def frames_to_pointcloud(cfgd, weights, frames, threshold):
    """frames_to_pointcloud (src/mastr/inference.cr:135-191) composed from the
    oracle's passes: each frame resized to the model size, consecutive pairs
    through the pair path, view-1 points of every pair and view-2 points of
    the last pair collected in that order. frames: list of [h, w, 3]."""
    if len(frames) < 2:
        return np.zeros((0, 3), np.float32), np.zeros((0,), np.float32)
    H, W = cfgd["img_h"], cfgd["img_w"]
    prep = [preprocess_image(resize_image(f, H, W)[None]) for f in frames]
    pts, confs = [], []
    for i in range(len(frames) - 1):
        o = mastr_pair(cfgd, weights, prep[i], prep[i + 1], desc=False)
        p, c = collect_points(o["pts1"], o["conf1"], threshold)
        pts.append(p)
        confs.append(c)
        if i == len(frames) - 2:
            p, c = collect_points(o["pts2"], o["conf2"], threshold)
            pts.append(p)
            confs.append(c)
    return np.concatenate(pts), np.concatenate(confs)


def config_from(d):
    """OrcConfig from a dict with the gs_mastr_config field names."""
    c = OrcConfig()
    for name, _ in OrcConfig._fields_:
        v = d.get(name, 0) if name == "composite" else d[name]
        if isinstance(v, (list, tuple)):
            arr = getattr(c, name)
            for i, x in enumerate(v):
                arr[i] = x
        else:
            setattr(c, name, v)
    return c


class _Weights:
    """Keeps the weight dict and the C callback alive."""

    def __init__(self, weights):
        self.w = {k: f32(v) for k, v in weights.items()}
        self.missing = []

        def cb(name, user):
            key = name.decode()
            a = self.w.get(key)
            if a is None:
                self.missing.append(key)
                return None
            return a.ctypes.data

        self.cb = WEIGHT_FN(cb)


def encoder_block(cfgd, weights, prefix, x, grid_h, grid_w):
    cfg = config_from(cfgd)
    W = _Weights(weights)
    x = f32(x).copy()
    B = x.shape[0]
    rc = lib().orc_encoder_block(C.byref(cfg), prefix.encode(), W.cb, None, _p(x), B, grid_h,
                                 grid_w)
    assert rc == 0 and not W.missing, (rc, W.missing)
    return x


class mutation:
    """Context manager planting composition mistake m in the oracle (tests
    only: shows that a pin fails on that mistake)."""

    def __init__(self, m):
        self.m = m

    def __enter__(self):
        lib().orc_set_mutation(self.m)
        return self

    def __exit__(self, *exc):
        lib().orc_set_mutation(0)
        return False


def decoder_block(cfgd, weights, prefix, x, mem, grid_h, grid_w):
    cfg = config_from(cfgd)
    W = _Weights(weights)
    x = f32(x).copy()
    mem = f32(mem)
    B = x.shape[0]
    rc = lib().orc_decoder_block(C.byref(cfg), prefix.encode(), W.cb, None, _p(x), _p(mem), B,
                                 grid_h, grid_w)
    assert rc == 0 and not W.missing, (rc, W.missing)
    return x


def local_features(cfgd, weights, prefix, enc, dec, gh, gw):
    cfg = config_from(cfgd)
    W = _Weights(weights)
    enc, dec = f32(enc), f32(dec)
    B = enc.shape[0]
    r = cfgd["patch"]
    desc = np.empty((B, gh * r, gw * r, cfgd["desc_dim"]), np.float32)
    rc = lib().orc_local_features(C.byref(cfg), W.cb, None, prefix.encode(), _p(enc), _p(dec), B,
                                  gh, gw, _p(desc))
    assert rc == 0 and not W.missing, (rc, W.missing)
    return desc


def encoder(cfgd, weights, img):
    cfg = config_from(cfgd)
    W = _Weights(weights)
    img = f32(img)
    B = img.shape[0]
    N = (cfgd["img_h"] // cfgd["patch"]) * (cfgd["img_w"] // cfgd["patch"])
    enc = np.empty((B, N, cfgd["enc_dim"]), np.float32)
    rc = lib().orc_encoder(C.byref(cfg), W.cb, None, _p(img), B, _p(enc))
    assert rc == 0 and not W.missing, (rc, W.missing)
    return enc


def mastr_pair(cfgd, weights, img1, img2, heads=True, desc=True):
    """Returns dict pts1, conf1, desc1, pts2, conf2, desc2 (NHWC); with
    composite 1 pts / conf are on the patch grid and desc is None."""
    cfg = config_from(cfgd)
    W = _Weights(weights)
    img1, img2 = f32(img1), f32(img2)
    B = img1.shape[0]
    H, Wd = cfgd["img_h"], cfgd["img_w"]
    if cfgd.get("composite", 0) == 1:  # stub heads on the patch grid, no descriptors
        H, Wd = H // cfgd["patch"], Wd // cfgd["patch"]
        desc = False
    out = {}
    for v in (1, 2):
        out[f"pts{v}"] = np.empty((B, H, Wd, 3), np.float32) if heads else None
        out[f"conf{v}"] = np.empty((B, H, Wd, 1), np.float32) if heads else None
        out[f"desc{v}"] = np.empty((B, H, Wd, cfgd["desc_dim"]), np.float32) if desc else None
    rc = lib().orc_mastr_pair(C.byref(cfg), W.cb, None, _p(img1), _p(img2), B,
                              _p(out["pts1"]), _p(out["conf1"]), _p(out["desc1"]),
                              _p(out["pts2"]), _p(out["conf2"]), _p(out["desc2"]))
    assert rc == 0 and not W.missing, (rc, W.missing)
    return out


def mastr_pair_taps(cfgd, weights, img1, img2):
    cfg = config_from(cfgd)
    W = _Weights(weights)
    img1, img2 = f32(img1), f32(img2)
    B = img1.shape[0]
    N = (cfgd["img_h"] // cfgd["patch"]) * (cfgd["img_w"] // cfgd["patch"])
    e1 = np.empty((B, N, cfgd["enc_dim"]), np.float32)
    e2 = np.empty_like(e1)
    d1 = np.empty((B, N, cfgd["dec_dim"]), np.float32)
    d2 = np.empty_like(d1)
    rc = lib().orc_mastr_pair_taps(C.byref(cfg), W.cb, None, _p(img1), _p(img2), B, _p(e1), _p(e2),
                                   _p(d1), _p(d2))
    assert rc == 0 and not W.missing, (rc, W.missing)
    return e1, e2, d1, d2


def dpt_head(cfgd, weights, prefix, hooks, gh, gw):
    """One full DPT head on hooks (enc [B,N,enc_dim], three [B,N,dec_dim])."""
    cfg = config_from(cfgd)
    W = _Weights(weights)
    hs = [f32(h) for h in hooks]
    B = hs[0].shape[0]
    arr = (vp * 4)(*[h.ctypes.data_as(vp) for h in hs])
    Hi, Wi = gh * cfgd["patch"], gw * cfgd["patch"]
    pts = np.empty((B, Hi, Wi, 3), np.float32)
    conf = np.empty((B, Hi, Wi, 1), np.float32)
    rc = lib().orc_dpt_head(C.byref(cfg), W.cb, None, prefix.encode(), arr, B, gh, gw, _p(pts),
                            _p(conf))
    assert rc == 0 and not W.missing, (rc, W.missing)
    return pts, conf
