"""ctypes binding of libgsplat_hip.so (the C ABI declared in include/gs_hip.h).

Used by the tests and bench.py. Device memory is passed as raw pointers
(torch.Tensor.data_ptr() of CUDA/HIP tensors). The library must be built
(crystal-gausplat_amd/build.py); loading fails loudly when it is missing, there
is no fallback path.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgsplat_hip.so")

c_float_p = C.POINTER(C.c_float)
vp = C.c_void_p


class MastrConfig(C.Structure):
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
        ("precision", C.c_int32),
        ("composite", C.c_int32),
    ]

    def as_dict(self):
        d = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            d[name] = list(v) if hasattr(v, "__len__") else v
        return d


# (name, restype, argtypes)
_SIGS = [
    ("gs_create_buffer", vp, [C.c_int64, C.c_int32]),
    ("gs_release_buffer", None, [vp]),
    ("gs_buffer_contents", vp, [vp]),
    ("gs_buffer_write", None, [vp, vp, C.c_int64]),
    ("gs_buffer_read", None, [vp, vp, C.c_int64]),
    ("gs_buffer_sync", None, [vp]),
    ("gs_buffer_copy", None, [vp, vp, C.c_int64]),
    ("gs_buffer_write_async", C.c_int32, [vp, vp, C.c_int64, C.c_int64, vp]),
    ("gs_buffer_read_async", C.c_int32, [vp, vp, C.c_int64, C.c_int64, vp]),
    ("gs_host_alloc", vp, [C.c_int64]),
    ("gs_host_free", None, [vp]),
    ("gs_stream_synchronize", C.c_int32, [vp]),
    ("gs_init_device", C.c_int32, []),
    ("gs_get_device", vp, []),
    ("gs_get_command_queue", vp, []),
    ("gs_synchronize", None, []),
    ("gs_device_name", C.c_char_p, []),
    ("gs_max_threads_per_threadgroup", C.c_int32, []),
    ("gs_recommended_working_set_size", C.c_int64, []),
    ("gs_has_unified_memory", C.c_int32, []),
    ("gs_hip_last_error", C.c_char_p, []),
    ("gs_seed_normal", None, [C.c_uint64, C.c_char_p, C.c_float, C.c_float, vp, C.c_int64]),
    ("gs_seed_uniform", None, [C.c_uint64, C.c_char_p, C.c_float, C.c_float, vp, C.c_int64]),
    ("gs_hip_linear", C.c_int32, [vp, vp, vp, vp, C.c_int64, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_int32, vp, vp]),
    ("gs_hip_layernorm", C.c_int32, [vp, vp, vp, vp, C.c_int64, C.c_int32, C.c_float, vp]),
    ("gs_hip_attention", C.c_int32, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                     C.c_int32, C.c_float] + [C.c_int64] * 12 + [vp]),
    ("gs_hip_attention_prec", C.c_int32, [vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32,
                                          C.c_int32, C.c_int32, C.c_float] + [C.c_int64] * 12 +
     [C.c_int32, vp]),
    ("gs_hip_rope2d", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int64, C.c_int32,
                                  C.c_float, vp]),
    ("gs_hip_conv2d", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp, vp,
                                  C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_int32, vp, vp]),
    ("gs_hip_conv2d_hw", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp, vp,
                                     C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                     C.c_int32, C.c_int32, vp, vp]),
    ("gs_hip_conv_transpose", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp,
                                          vp, C.c_int32, C.c_int32, vp]),
    ("gs_hip_upsample2x", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp]),
    ("gs_hip_resize_image", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_int32, vp, vp]),
    ("gs_hip_preprocess_image", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, vp, vp]),
    ("gs_hip_prepare_frames", C.c_int32, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                          C.c_int32, vp, vp]),
    ("gs_hip_collect_points", C.c_int32, [vp, vp, C.c_int64, C.c_float, vp, vp, C.c_int64, vp,
                                          vp]),
    ("gs_hip_collect_points_noalloc", C.c_int32, [vp, vp, C.c_int64, C.c_float, vp, vp,
                                                  C.c_int64, vp, vp]),
    ("gs_mastr_default_config", None, [C.POINTER(MastrConfig)]),
    ("gs_mastr_weight_count", C.c_int32, [C.POINTER(MastrConfig)]),
    ("gs_mastr_weight_info", C.c_int32, [C.POINTER(MastrConfig), C.c_int32, C.c_char_p, C.c_int32,
                                         C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
    ("gs_mastr_weight_values", C.c_int32, [C.POINTER(MastrConfig), C.c_int32, C.c_uint64,
                                           C.c_float, C.c_float, vp, C.c_int64]),
    ("gs_hip_mastr_create", C.c_int32, [C.POINTER(MastrConfig), C.c_int32, C.POINTER(vp)]),
    ("gs_hip_mastr_destroy", None, [vp]),
    ("gs_hip_mastr_init_seeded", C.c_int32, [vp, C.c_uint64, C.c_float, C.c_float]),
    ("gs_hip_mastr_set_weight", C.c_int32, [vp, C.c_char_p, vp, C.c_int64]),
    ("gs_hip_mastr_encoder_block", C.c_int32, [vp, C.c_int32, vp, C.c_int32, vp]),
    ("gs_hip_mastr_encoder", C.c_int32, [vp, vp, C.c_int32, vp, vp]),
    ("gs_hip_mastr_pair", C.c_int32, [vp, vp, vp, C.c_int32, vp, vp, vp, vp, vp, vp, vp]),
    ("gs_hip_mastr_pair_taps", C.c_int32, [vp, C.c_int32, vp, vp, vp, vp, vp]),
    ("gs_hip_mastr_set_graph", C.c_int32, [vp, C.c_int32]),
    ("gs_hip_mastr_frames_to_pointcloud", C.c_int32, [vp, vp, C.c_int32, C.c_int32, C.c_int32,
                                                      C.c_float, vp, vp, C.c_int64,
                                                      C.POINTER(C.c_int64), vp]),
    ("gs_safetensors_count", C.c_int32, [C.c_char_p]),
    ("gs_safetensors_info", C.c_int32, [C.c_char_p, C.c_int32, C.c_char_p, C.c_int32, C.c_char_p,
                                        C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
    ("gs_safetensors_read_f32", C.c_int32, [C.c_char_p, C.c_char_p, vp, C.c_int64]),
    ("gs_hip_mastr_load_safetensors", C.c_int32, [vp, C.c_char_p, C.POINTER(C.c_int32),
                                                  C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("gs_hip_profile_begin", C.c_int32, [C.c_int32]),
    ("gs_hip_profile_end", C.c_int32, []),
    ("gs_hip_profile_entry", C.c_int32, [C.c_int32, C.c_char_p, C.c_int32, C.POINTER(C.c_int64),
                                         C.POINTER(C.c_double), C.POINTER(C.c_double),
                                         C.POINTER(C.c_double)]),
]

EPI_GELU, EPI_RESIDUAL, EPI_RELU, EPI_BF16, EPI_F32X6 = 1, 2, 4, 8, 16
CONV_RELU_IN, CONV_RELU_OUT, CONV_F32X6 = 1, 2, 4

_lib = None


def lib():
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built: run crystal-gausplat_amd/build.py")
        # torch carries its own HIP runtime; loading it first makes the library
        # bind to that same runtime (one HIP runtime per process). Loaded the
        # other way round, two runtimes coexist and the second sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_names():
    return [s[0] for s in _SIGS]


class GsError(RuntimeError):
    pass


def check(rc):
    if rc != 0:
        raise GsError(f"rc={rc}: {lib().gs_hip_last_error().decode()}")
    return rc


def ptr(t):
    """Device pointer of a torch tensor (None passes through as NULL)."""
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def default_config(**over):
    cfg = MastrConfig()
    lib().gs_mastr_default_config(C.byref(cfg))
    for k, v in over.items():
        if isinstance(v, (list, tuple)):
            arr = getattr(cfg, k)
            for i, x in enumerate(v):
                arr[i] = x
        else:
            setattr(cfg, k, v)
    return cfg


def ref512_config(**over):
    """The reference's literal MASt3RInference#forward_pair at 512x512
    (src/mastr/inference.cr:25-57, 92-115): token-level RoPE, LayerNorm eps
    1e-5, own-view decoder memory, stub DPT heads on the 32x32 patch grid,
    sigmoid confidence."""
    kw = dict(img_h=512, img_w=512, rope_mode=2, ln_eps=1e-5, composite=1)
    kw.update(over)
    return default_config(**kw)


def weight_inventory(cfg):
    """[(name, shape tuple, kind)] of a configuration."""
    L = lib()
    out = []
    n = L.gs_mastr_weight_count(C.byref(cfg))
    buf = C.create_string_buffer(256)
    shp = (C.c_int64 * 4)()
    kind = C.c_int32()
    for i in range(n):
        check(L.gs_mastr_weight_info(C.byref(cfg), i, buf, 256, shp, C.byref(kind)))
        shape = tuple(int(s) for s in shp if s > 0)
        out.append((buf.value.decode(), shape, kind.value))
    return out


def weight_values(cfg, i, n, seed=0, bias_std=0.0, ln_std=0.0):
    import numpy as np
    a = np.empty(n, dtype=np.float32)
    check(lib().gs_mastr_weight_values(C.byref(cfg), i, seed, bias_std, ln_std,
                                       a.ctypes.data_as(C.c_void_p), n))
    return a


def seeded_weights(cfg, seed=0, bias_std=0.0, ln_std=0.0):
    """dict name -> float32 numpy array (shaped) of the seeded weights. The
    generator is counter-based (each tensor depends only on its name and the
    seed), so the tensors are generated on a few host threads (the ctypes
    call releases the GIL) with the same values as one at a time."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    inv = weight_inventory(cfg)

    def one(i):
        name, shape, kind = inv[i]
        return name, weight_values(cfg, i, int(np.prod(shape)), seed, bias_std,
                                   ln_std).reshape(shape)
    with ThreadPoolExecutor(max_workers=max(1, min(8, os.cpu_count() or 1))) as ex:
        return dict(ex.map(one, range(len(inv))))


def seed_normal(seed, name, n, mean=0.0, std=1.0):
    import numpy as np
    a = np.empty(n, dtype=np.float32)
    lib().gs_seed_normal(seed, name.encode(), mean, std, a.ctypes.data_as(C.c_void_p), n)
    return a


def seed_uniform(seed, name, n, lo=-1.0, hi=1.0):
    import numpy as np
    a = np.empty(n, dtype=np.float32)
    lib().gs_seed_uniform(seed, name.encode(), lo, hi, a.ctypes.data_as(C.c_void_p), n)
    return a


def safetensors_index(path):
    """[(name, dtype, shape tuple)] of a safetensors file, in header order."""
    L = lib()
    p = os.fsencode(path)
    n = L.gs_safetensors_count(p)
    if n < 0:
        check(n)
    name, dt = C.create_string_buffer(512), C.create_string_buffer(8)
    shp, nd = (C.c_int64 * 8)(), C.c_int32()
    out = []
    for i in range(n):
        check(L.gs_safetensors_info(p, i, name, 512, dt, shp, C.byref(nd)))
        out.append((name.value.decode(), dt.value.decode(), tuple(shp[:nd.value])))
    return out


def safetensors_read(path, name, shape):
    """Tensor `name` of a safetensors file as float32 numpy (F32/F16/BF16)."""
    import numpy as np
    a = np.empty(shape, dtype=np.float32)
    check(lib().gs_safetensors_read_f32(os.fsencode(path), name.encode(),
                                        a.ctypes.data_as(C.c_void_p), a.size))
    return a


def profile_begin(per_shape=False):
    check(lib().gs_hip_profile_begin(1 if per_shape else 0))


def profile_end():
    """{kernel: dict(launches, ms, flops, bytes)} of the launches since begin."""
    L = lib()
    n = L.gs_hip_profile_end()
    if n < 0:
        check(n)
    out = {}
    buf = C.create_string_buffer(256)
    la, ms, fl, by = C.c_int64(), C.c_double(), C.c_double(), C.c_double()
    for i in range(n):
        check(L.gs_hip_profile_entry(i, buf, 256, C.byref(la), C.byref(ms), C.byref(fl),
                                     C.byref(by)))
        out[buf.value.decode()] = dict(launches=la.value, ms=ms.value, flops=fl.value,
                                       bytes=by.value)
    return out


class Mastr:
    """A device MASt3R context (weights + workspaces for max_pairs pairs)."""

    def __init__(self, cfg, max_pairs=1):
        self.cfg = cfg
        h = C.c_void_p()
        check(lib().gs_hip_mastr_create(C.byref(cfg), max_pairs, C.byref(h)))
        self.h = h

    def init_seeded(self, seed=0, bias_std=0.0, ln_std=0.0):
        check(lib().gs_hip_mastr_init_seeded(self.h, seed, bias_std, ln_std))

    def set_weight(self, name, arr):
        import numpy as np
        a = np.ascontiguousarray(arr, dtype=np.float32)
        check(lib().gs_hip_mastr_set_weight(self.h, name.encode(), a.ctypes.data_as(C.c_void_p),
                                            a.size))

    def load_safetensors(self, path):
        """Place every inventory weight found in a checkpoint file; returns
        dict(loaded, unexpected, missing) counts."""
        a, b, c = C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().gs_hip_mastr_load_safetensors(self.h, os.fsencode(path), C.byref(a),
                                                  C.byref(b), C.byref(c)))
        return dict(loaded=a.value, unexpected=b.value, missing=c.value)

    def frames_to_pointcloud(self, frames, threshold, out_pts, out_conf, stream=None):
        """frames: device tensor [F, h, w, 3]; out_pts [cap, 3], out_conf [cap]
        device tensors. Returns the total point count (may exceed cap)."""
        F, h, w, c = frames.shape
        assert c == 3 and out_pts.shape[0] == out_conf.shape[0]
        n = C.c_int64()
        check(lib().gs_hip_mastr_frames_to_pointcloud(self.h, ptr(frames), F, h, w, threshold,
                                                      ptr(out_pts), ptr(out_conf),
                                                      out_pts.shape[0], C.byref(n), stream))
        return n.value

    def encoder_block(self, layer, x, B, stream=None):
        check(lib().gs_hip_mastr_encoder_block(self.h, layer, ptr(x), B, stream))

    def encoder(self, img, B, enc, stream=None):
        check(lib().gs_hip_mastr_encoder(self.h, ptr(img), B, ptr(enc), stream))

    def pair(self, img1, img2, B, pts1=None, conf1=None, desc1=None, pts2=None, conf2=None,
             desc2=None, stream=None):
        check(lib().gs_hip_mastr_pair(self.h, ptr(img1), ptr(img2), B, ptr(pts1), ptr(conf1),
                                      ptr(desc1), ptr(pts2), ptr(conf2), ptr(desc2), stream))

    def set_graph(self, enable=True):
        check(lib().gs_hip_mastr_set_graph(self.h, 1 if enable else 0))

    def pair_taps(self, B, enc1=None, enc2=None, dec1=None, dec2=None, stream=None):
        check(lib().gs_hip_mastr_pair_taps(self.h, B, ptr(enc1), ptr(enc2), ptr(dec1), ptr(dec2),
                                           stream))

    def close(self):
        if self.h:
            lib().gs_hip_mastr_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
