"""Per-op parity of the HIP kernels (through the C ABI) against the oracle,
at the shapes the MASt3R configs use and at ragged edge shapes."""
import ctypes as C

import numpy as np
import pytest
import torch

import gsplat_hip as G
import pyoracle as O
from gpu_util import assert_close, assert_close_bf16, case, dev, empty, host, stream

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(7)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def L():
    return G.lib()


def p(t):
    return G.ptr(t)


# ---------------------------------------------------------------- linear

LINEAR_CASES = [
    # config-0 shapes (M = 768 tokens)
    (768, 1024, 3072), (768, 1024, 1024), (768, 1024, 4096), (768, 4096, 1024),
    # decoder / embed / descriptor shapes
    (768, 768, 2304), (768, 3072, 768), (768, 1024, 768), (300, 1792, 7168),
    # ragged
    (1, 32, 32), (37, 64, 100), (129, 96, 130),
]


@pytest.mark.parametrize("M,K,N", LINEAR_CASES)
def test_linear_parity(M, K, N):
    case(f"linear M={M} K={K} N={N}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1)
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, 0, None,
                              stream()))
    assert_close(host(y), O.linear(x, W, b), name="linear")


@pytest.mark.parametrize("epi", ["gelu", "residual", "relu", "nobias"])
def test_linear_epilogues(epi):
    case(f"linear epilogue {epi}")
    M, K, N = 200, 256, 384
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.05), rnd(N, scale=0.1), rnd(M, N)
    ref = O.linear(x, W, None if epi == "nobias" else b)
    flags = 0
    if epi == "gelu":
        flags, ref = G.EPI_GELU, O.gelu(ref)
    elif epi == "relu":
        flags, ref = G.EPI_RELU, np.maximum(ref, 0)
    elif epi == "residual":
        flags, ref = G.EPI_RESIDUAL, r + ref
    y = dev(r) if epi == "residual" else empty(M, N)  # residual in place
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), None if epi == "nobias" else p(dev(b)), p(y),
                              M, K, N, 0, flags, p(y) if epi == "residual" else None, stream()))
    assert_close(host(y), ref, name=epi)


@pytest.mark.parametrize("M,K,N", [(768, 1024, 3072), (768, 4096, 1024), (37, 64, 100)])
def test_linear_bf16_variant(M, K, N):
    case(f"linear bf16 M={M} K={K} N={N}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1)
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, G.EPI_BF16, None,
                              stream()))
    rel, worst = assert_close_bf16(host(y), O.linear(x, W, b), name="linear bf16")
    print(f"bf16 linear: rel {rel:.2e} worst {worst:.2e}")
    assert rel > 1e-5  # it really ran in bf16


@pytest.mark.parametrize("M,K,N", [(256, 1024, 256), (256, 4096, 256), (300, 1792, 7168),
                                   (129, 96, 130)])
def test_linear_f32x6_accuracy_vs_fp64(M, K, N):
    """fp32 through bf16x6 split products against an fp64 product: its error
    is at the level of the fp32 MFMA kernel's (RMS within 1.5x, max within
    2x), it meets the fp32 parity bar against the oracle, and it differs from
    the fp32 kernel in the last bits (it really ran the bf16 matrix cores)."""
    case(f"linear f32x6 M={M} K={K} N={N}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1)
    ref64 = x.astype(np.float64) @ W.astype(np.float64).T + b.astype(np.float64)

    def run(flags):
        y = empty(M, N)
        G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, flags, None,
                                  stream()))
        return host(y)

    y32, y6 = run(0), run(G.EPI_F32X6)
    e32, e6 = y32.astype(np.float64) - ref64, y6.astype(np.float64) - ref64
    rms32, rms6 = np.sqrt(np.mean(e32 ** 2)), np.sqrt(np.mean(e6 ** 2))
    print(f"f32x6 M={M} K={K} N={N}: rms err fp32 {rms32:.3e} x6 {rms6:.3e}; "
          f"max fp32 {np.abs(e32).max():.3e} x6 {np.abs(e6).max():.3e}")
    assert rms6 <= 1.5 * rms32 + 1e-9
    assert np.abs(e6).max() <= 2.0 * np.abs(e32).max() + 1e-9
    assert (y6 != y32).mean() > 0.01
    assert_close(y6, O.linear(x, W, b), name="linear f32x6")


@pytest.mark.parametrize("epi", ["gelu", "residual"])
def test_linear_f32x6_epilogues(epi):
    case(f"linear f32x6 epilogue {epi}")
    M, K, N = 200, 256, 384
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.05), rnd(N, scale=0.1), rnd(M, N)
    ref = O.linear(x, W, b)
    flags = G.EPI_F32X6
    if epi == "gelu":
        flags, ref = flags | G.EPI_GELU, O.gelu(ref)
    else:
        flags, ref = flags | G.EPI_RESIDUAL, r + ref
    y = dev(r) if epi == "residual" else empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, flags,
                              p(y) if epi == "residual" else None, stream()))
    assert_close(host(y), ref, name=f"f32x6 {epi}")


def test_linear_f32x6_validation():
    case("linear f32x6 validation")
    x = empty(4, 32)
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 32, 4, 1, G.EPI_F32X6, None, stream())
    assert rc != 0 and b"w_layout 0" in L().gs_hip_last_error()
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 32, 4, 0, G.EPI_F32X6 | G.EPI_BF16, None,
                           stream())
    assert rc != 0


@pytest.mark.parametrize("M,K,N", [(768, 1024, 1024), (50, 64, 96)])
def test_linear_literal_layout(M, K, N):
    # D1: the reference CPU path's [out,in] buffer read as [in,out]
    case(f"linear literal M={M} K={K} N={N}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1)
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 1, 0, None,
                              stream()))
    assert_close(host(y), O.linear(x, W, b, layout=1), name="literal")


def test_linear_rejects_bad_shapes_without_launch():
    case("linear validation")
    x = empty(4, 33)
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 33, 4, 0, 0, None, stream())
    assert rc != 0 and b"multiple of 32" in L().gs_hip_last_error()
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 32, 4, 2, 0, None, stream())
    assert rc != 0


# ---------------------------------------------------------------- layernorm


@pytest.mark.parametrize("rows,D", [(768, 1024), (1536, 768), (5, 132), (3, 4096)])
def test_layernorm_parity(rows, D):
    case(f"layernorm rows={rows} D={D}")
    x, g, b = rnd(rows, D, scale=2.0) + 0.5, rnd(D, scale=0.2) + 1, rnd(D, scale=0.2)
    y = empty(rows, D)
    G.check(L().gs_hip_layernorm(p(dev(x)), p(dev(g)), p(dev(b)), p(y), rows, D, 1e-6, stream()))
    assert_close(host(y), O.layernorm(x, g, b, 1e-6), name="layernorm")


# ---------------------------------------------------------------- attention


def attn_call(q, k, v, o, B, H, Nq, Nkv, qs, ks, vs, os_):
    G.check(L().gs_hip_attention(p(q), p(k), p(v), p(o), B, H, Nq, Nkv, 64, 0.125, *qs, *ks, *vs,
                                 *os_, stream()))


@pytest.mark.parametrize("B,H,Nq,Nkv", [(2, 16, 768, 768), (1, 12, 768, 768), (1, 2, 100, 77),
                                        (2, 3, 1, 5), (1, 1, 33, 1024)])
def test_attention_token_major(B, H, Nq, Nkv):
    case(f"attention token-major B={B} H={H} Nq={Nq} Nkv={Nkv}")
    D = H * 64
    q, k, v = rnd(B, Nq, D), rnd(B, Nkv, D), rnd(B, Nkv, D)
    o = empty(B, Nq, D)
    attn_call(dev(q), dev(k), dev(v), o, B, H, Nq, Nkv, (Nq * D, 64, D), (Nkv * D, 64, D),
              (Nkv * D, 64, D), (Nq * D, 64, D))
    sh = lambda a, n: a.reshape(B, n, H, 64).transpose(0, 2, 1, 3)
    ref = O.sdpa(sh(q, Nq), sh(k, Nkv), sh(v, Nkv)).transpose(0, 2, 1, 3).reshape(B, Nq, D)
    assert_close(host(o), ref, name="attention")


def test_attention_bhnd_layout_and_large_scores():
    # the reference GPU layout [B*H, N, 64] (src/nn/gpu_ops.cr:200-227) and
    # scores large enough that an unstabilised softmax would overflow
    case("attention BHND layout")
    B, H, N = 2, 3, 130
    q, k, v = rnd(B, H, N, 64, scale=4.0), rnd(B, H, N, 64, scale=4.0), rnd(B, H, N, 64)
    o = empty(B, H, N, 64)
    st = (H * N * 64, N * 64, 64)
    attn_call(dev(q), dev(k), dev(v), o, B, H, N, N, st, st, st, st)
    assert_close(host(o), O.sdpa(q, k, v), name="attention bhnd")


def test_attention_rejects_bad_head_dim():
    case("attention validation")
    x = empty(64)
    rc = L().gs_hip_attention(p(x), p(x), p(x), p(x), 1, 1, 1, 1, 32, 0.1, *([0] * 12), stream())
    assert rc != 0 and b"head_dim" in L().gs_hip_last_error()


def test_elementwise_and_conv_reject_bad_sizes_without_launch():
    # negative or oversized extents are errors on the host, before any grid is
    # formed (a negative element count must not wrap into a huge grid)
    case("elementwise / conv validation")
    x = empty(64)
    assert L().gs_hip_upsample2x(p(x), -1, 2, 2, 4, p(x), stream()) == -1
    assert b"upsample2x" in L().gs_hip_last_error()
    assert L().gs_hip_rope2d(p(x), 1, 4, 0, 64, 2, 100.0, stream()) == -1
    assert b"rope2d" in L().gs_hip_last_error()
    assert L().gs_hip_conv2d(p(x), 70000, 256, 256, 32, p(x), None, p(x), 32, 1, 1, 0, 1, 0, None,
                             stream()) == -1
    assert b"too many output pixels" in L().gs_hip_last_error()
    assert L().gs_hip_conv_transpose(p(x), 70000, 256, 256, 32, p(x), None, p(x), 32, 2,
                                     stream()) == -1
    assert b"too many pixels" in L().gs_hip_last_error()


# ---------------------------------------------------------------- rope


@pytest.mark.parametrize("gh,gw,H", [(24, 32, 16), (3, 5, 2)])
def test_rope2d_parity(gh, gw, H):
    case(f"rope2d {gh}x{gw} H={H}")
    B, N = 2, gh * gw
    ld = 3 * H * 64
    t = rnd(B, N, ld)
    td = dev(t)
    G.check(L().gs_hip_rope2d(p(td), B, N, H, ld, gw, 100.0, stream()))
    ref = t.copy()
    ref[:, :, :H * 64] = O.rope2d(t[:, :, :H * 64].copy(), H, gw, 100.0)
    assert_close(host(td), ref, rtol=1e-6, atol=1e-7, name="rope2d")


# ---------------------------------------------------------------- convolutions

CONV_CASES = [
    # (B, H, W, Cin, Cout, k, s, p, flags, residual)
    (1, 12, 16, 256, 256, 3, 1, 1, 0, False),        # RCU at 1/32
    (1, 24, 32, 768, 768, 3, 2, 1, 0, False),         # act_postprocess 3.1
    (2, 96, 128, 96, 256, 3, 1, 1, 0, False),         # layer1_rn
    (1, 48, 64, 256, 256, 3, 1, 1, G.CONV_RELU_IN | G.CONV_RELU_OUT, False),  # RCU conv1
    (1, 48, 64, 256, 256, 3, 1, 1, 0, True),          # RCU conv2 + residual
    (1, 24, 32, 1024, 96, 1, 1, 0, 0, False),         # act_postprocess 0.0 (1x1)
    (1, 7, 9, 64, 40, 3, 2, 1, 0, False),             # ragged
    (3, 5, 6, 32, 4, 1, 1, 0, 0, False),              # head.4-like tiny Cout
]


@pytest.mark.parametrize("B,H,W,Cin,Cout,k,s,pd,flags,res", CONV_CASES)
def test_conv2d_parity(B, H, W, Cin, Cout, k, s, pd, flags, res):
    case(f"conv2d B={B} {H}x{W} {Cin}->{Cout} k={k} s={s} p={pd} flags={flags} res={res}")
    x, w, b = rnd(B, H, W, Cin), rnd(Cout, Cin, k, k, scale=0.05), rnd(Cout, scale=0.1)
    Ho, Wo = (H + 2 * pd - k) // s + 1, (W + 2 * pd - k) // s + 1
    r = rnd(B, Ho, Wo, Cout)
    xin = np.maximum(x, 0) if flags & G.CONV_RELU_IN else x
    ref = O.conv2d(xin, w, b, s, pd)
    if flags & G.CONV_RELU_OUT:
        ref = np.maximum(ref, 0)
    if res:
        ref = ref + r
    y = empty(B, Ho, Wo, Cout)
    G.check(L().gs_hip_conv2d(p(dev(x)), B, H, W, Cin, p(dev(w)), p(dev(b)), p(y), Cout, k, s, pd,
                              0, flags, p(dev(r)) if res else None, stream()))
    assert_close(host(y), ref, name="conv2d")


@pytest.mark.parametrize("B,H,W,Cin,Cout,k,s,pd,flags,res", [CONV_CASES[i] for i in (0, 2, 3, 4, 6)])
def test_conv2d_f32x6(B, H, W, Cin, Cout, k, s, pd, flags, res):
    """Implicit-GEMM convolution with bf16x6 split products: the fp32 parity
    bar against the oracle, and close to the fp32 MFMA kernel."""
    case(f"conv2d f32x6 B={B} {H}x{W} {Cin}->{Cout} k={k} s={s} p={pd} flags={flags} res={res}")
    x, w, b = rnd(B, H, W, Cin), rnd(Cout, Cin, k, k, scale=0.05), rnd(Cout, scale=0.1)
    Ho, Wo = (H + 2 * pd - k) // s + 1, (W + 2 * pd - k) // s + 1
    r = rnd(B, Ho, Wo, Cout)
    xin = np.maximum(x, 0) if flags & G.CONV_RELU_IN else x
    ref = O.conv2d(xin, w, b, s, pd)
    if flags & G.CONV_RELU_OUT:
        ref = np.maximum(ref, 0)
    if res:
        ref = ref + r
    ys = []
    for extra in (0, G.CONV_F32X6):
        y = empty(B, Ho, Wo, Cout)
        G.check(L().gs_hip_conv2d(p(dev(x)), B, H, W, Cin, p(dev(w)), p(dev(b)), p(y), Cout, k, s,
                                  pd, 0, flags | extra, p(dev(r)) if res else None, stream()))
        ys.append(host(y))
    assert_close(ys[1], ref, name="conv2d f32x6")
    scale = np.abs(ys[0]).max()
    assert np.abs(ys[1] - ys[0]).max() <= 1e-5 * scale + 1e-6


@pytest.mark.parametrize("Cin,Cout,k,H,W", [(96, 96, 4, 24, 32), (192, 192, 2, 24, 32),
                                            (32, 64, 2, 3, 5)])
def test_conv_transpose_parity(Cin, Cout, k, H, W):
    case(f"conv_transpose {Cin}->{Cout} k={k} {H}x{W}")
    B = 2
    x, w, b = rnd(B, H, W, Cin), rnd(Cin, Cout, k, k, scale=0.05), rnd(Cout, scale=0.1)
    y = empty(B, H * k, W * k, Cout)
    G.check(L().gs_hip_conv_transpose(p(dev(x)), B, H, W, Cin, p(dev(w)), p(dev(b)), p(y), Cout, k,
                                      stream()))
    assert_close(host(y), O.conv_transpose(x, w, b, k), name="convT")


@pytest.mark.parametrize("B,H,W,C", [(1, 96, 128, 256), (2, 5, 7, 8)])
def test_upsample_parity(B, H, W, C):
    case(f"upsample2x {B}x{H}x{W}x{C}")
    x = rnd(B, H, W, C)
    y = empty(B, 2 * H, 2 * W, C)
    G.check(L().gs_hip_upsample2x(p(dev(x)), B, H, W, C, p(y), stream()))
    assert_close(host(y), O.upsample2x(x), rtol=1e-6, atol=1e-7, name="upsample")


def test_buffer_api_roundtrip():
    case("gs_* buffer api")
    Lb = L()
    assert Lb.gs_init_device() == 0
    assert Lb.gs_has_unified_memory() == 0
    assert Lb.gs_recommended_working_set_size() > 0
    n = 1000
    a = rnd(n)
    h1 = Lb.gs_create_buffer(4 * n, 0)
    h2 = Lb.gs_create_buffer(4 * n, 0)
    assert h1 and h2
    Lb.gs_buffer_write(h1, a.ctypes.data_as(C.c_void_p), 4 * n)
    Lb.gs_buffer_copy(h1, h2, 4 * n)
    Lb.gs_synchronize()
    out = np.empty_like(a)
    Lb.gs_buffer_read(h2, out.ctypes.data_as(C.c_void_p), 4 * n)
    np.testing.assert_array_equal(out, a)
    assert Lb.gs_buffer_contents(h1)
    Lb.gs_release_buffer(h1)
    Lb.gs_release_buffer(h2)
    assert Lb.gs_create_buffer(0, 0) is None


def test_buffer_async_copies_with_pinned_memory():
    """gs_buffer_write_async / read_async at byte offsets on a caller stream,
    through pinned host memory from gs_host_alloc, and their range checks."""
    case("gs_* async buffer copies")
    Lb = L()
    n = 4096
    a = rnd(n)
    hbuf = Lb.gs_host_alloc(4 * n)
    assert hbuf
    host = np.ctypeslib.as_array((C.c_float * n).from_address(hbuf))
    host[:] = a
    h = Lb.gs_create_buffer(4 * n, 0)
    s = stream()
    # two halves, the second at a byte offset
    G.check(Lb.gs_buffer_write_async(h, C.c_void_p(hbuf), 2 * n, 0, s))
    G.check(Lb.gs_buffer_write_async(h, C.c_void_p(hbuf + 2 * n), 2 * n, 2 * n, s))
    out = np.zeros(n, np.float32)
    G.check(Lb.gs_buffer_read_async(h, out.ctypes.data_as(C.c_void_p), 4 * n, 0, s))
    G.check(Lb.gs_stream_synchronize(s))
    np.testing.assert_array_equal(out, a)
    part = np.zeros(10, np.float32)
    G.check(Lb.gs_buffer_read_async(h, part.ctypes.data_as(C.c_void_p), 40, 400, s))
    G.check(Lb.gs_stream_synchronize(s))
    np.testing.assert_array_equal(part, a[100:110])
    assert Lb.gs_buffer_write_async(h, C.c_void_p(hbuf), 8, 4 * n - 4, s) == -1
    assert Lb.gs_buffer_read_async(h, out.ctypes.data_as(C.c_void_p), 4, -4, s) == -1
    Lb.gs_release_buffer(h)
    Lb.gs_host_free(hbuf)
