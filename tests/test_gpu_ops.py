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


def p_off(t, nbytes):
    """Device pointer nbytes into a tensor (to break 16-byte alignment)."""
    return C.c_void_p(t.data_ptr() + nbytes)


# ---------------------------------------------------------------- linear

LINEAR_CASES = [
    # config-0 shapes (M = 768 tokens)
    (768, 1024, 3072), (768, 1024, 1024), (768, 1024, 4096), (768, 4096, 1024),
    # decoder / embed / descriptor shapes
    (768, 768, 2304), (768, 3072, 768), (768, 1024, 768), (300, 1792, 7168),
    # ragged
    (1, 32, 32), (37, 64, 100), (129, 96, 130),
    # at least one 128 x 256 tile per CU (the one-wave-per-SIMD kernel) with
    # ragged rows and columns
    (5000, 96, 3000), (4099, 1024, 2304),
]


@pytest.mark.parametrize("M,K,N", LINEAR_CASES)
def test_linear_parity(M, K, N):
    case(f"linear M={M} K={K} N={N}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1)
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, 0, None,
                              stream()))
    assert_close(host(y), O.linear(x, W, b), name="linear")


@pytest.mark.parametrize("M", [200, 8200])
@pytest.mark.parametrize("epi", ["gelu", "residual", "relu", "nobias"])
def test_linear_epilogues(epi, M):
    case(f"linear epilogue {epi} M={M}")
    K, N = 256, 4096 if M > 1000 else 384
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
    rel, worst, p999 = assert_close_bf16(host(y), O.linear(x, W, b), name="linear bf16")
    print(f"bf16 linear: rel {rel:.2e} worst {worst:.2e} p99.9 elementwise {p999:.2e}")
    assert rel > 1e-5  # it really ran in bf16


@pytest.mark.parametrize("M,K,N,epi", [(8200, 1024, 3000, "gelu"), (8200, 1024, 3000, "residual"),
                                       (8192, 768, 2304, "nobias"), (16384, 2048, 1024, "residual"),
                                       (16400, 3072, 1000, "gelu"), (8200, 7168, 2000, "residual")])
def test_linear_bf16_large_launches(M, K, N, epi):
    """The bf16 variant on launches large enough for the 256 x 128 kernel in
    its two- and three-stage forms (K >= 6144 takes the latter; ragged M and
    N, the three epilogues), against an fp64 product of
    the bf16-rounded operands: the kernels round x and W to bf16 and
    accumulate in fp32, so the error bound is the fp32 accumulation's."""
    case(f"linear bf16 large M={M} K={K} N={N} {epi}")
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1), rnd(M, N)
    xb = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    Wb = torch.from_numpy(W).to(torch.bfloat16).double().numpy()
    ref = xb @ Wb.T + (0 if epi == "nobias" else b.astype(np.float64))
    flags = G.EPI_BF16
    if epi == "gelu":
        flags |= G.EPI_GELU
        ref = 0.5 * ref * (1 + np.tanh(0.7978845608028654 * (ref + 0.044715 * ref ** 3)))
    elif epi == "residual":
        flags |= G.EPI_RESIDUAL
        ref = ref + r
    y = dev(r) if epi == "residual" else empty(M, N)  # residual in place
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), None if epi == "nobias" else p(dev(b)), p(y),
                              M, K, N, 0, flags, p(y) if epi == "residual" else None, stream()))
    got = host(y)
    # fp32 accumulation of K bf16 products: a few ulp of the partial sums
    assert_close(got, ref, rtol=1e-4, atol=2e-5 * np.sqrt(K / 1024), name=f"bf16 large {epi}")


@pytest.mark.parametrize("M,K,N,epi", [(18440, 6144, 1924, "residual"), (12288, 6144, 4096, "nobias"),
                                       (12288, 7168, 2048, "gelu")])
def test_linear_f32_long_k_large_launches(M, K, N, epi):
    """fp32 launches with K >= 6144 and more than one round of 256 x 128
    tiles run as one launch per round of tiles: 1168 tiles (ragged M and N)
    as a full round and a partial one (96 + 50 tiles per XCD), 1536 tiles as
    two full rounds; 768 tiles stay one launch. Against an fp64 product of the
    same operands."""
    case(f"linear f32 long K M={M} K={K} N={N} {epi}")
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.02), rnd(N, scale=0.1), rnd(M, N)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + (0 if epi == "nobias" else b.astype(np.float64))
    flags = 0
    if epi == "gelu":
        flags |= G.EPI_GELU
        ref = 0.5 * ref * (1 + np.tanh(0.7978845608028654 * (ref + 0.044715 * ref ** 3)))
    elif epi == "residual":
        flags |= G.EPI_RESIDUAL
        ref = ref + r
    y = dev(r) if epi == "residual" else empty(M, N)  # residual in place
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), None if epi == "nobias" else p(dev(b)), p(y),
                              M, K, N, 0, flags, p(y) if epi == "residual" else None, stream()))
    assert_close(host(y), ref, rtol=1e-4, atol=2e-5 * np.sqrt(K / 1024), name=f"f32 long K {epi}")


# The direct-to-LDS kernels wait for their own loads with hand-counted
# s_waitcnt vmcnt immediates, which differ between the first, the steady-state
# and the last K steps. Each kernel here runs K of few and many steps, against
# an fp64 product of the same operands:
# - the fp32 256-, 192-, 64- and 32-row kernels (16-deep steps; gs_hip_linear
#   pads K to a multiple of 32, so K = 16 / 48 / 272 run as 2 / 4 / 18 steps;
#   odd step counts of these kernels are reached through the conv op in
#   test_conv2d_nonsquare_kernel). The 192-row form also at ragged M and N
#   (24500 x 760: 128 x 6 tiles, the last row and column tiles partial). The
#   64-row form takes small launches with at least 432 of its tiles (N = 4096
#   here); the 32-row form smaller ones with at least 768 of its tiles, those
#   of the 64-row form it spreads more evenly over the CUs (N = 3072 at M =
#   1536 / 1400: 1152 / 1056 tiles of 32 rows, at most 5 per CU, against 576 /
#   528 of 64 rows, 3 per CU) and those whose busiest CU it loads no more than
#   the split 128 x 128 kernel (M = 768, N = 1024, K <= 96); ragged M and N
#   too; split in K at 512-767 tiles (M = 768, N = 3072 and the ragged 750 x
#   3000: 576 tiles in three ranges of 4, 7 and 10-11 32-deep steps);
# - the bf16 two- and three-stage kernels (32-deep steps: one, two, three and
#   many; K >= 6144 takes three stages);
# - the 128 x 128 kernel of split small launches (M = 768, N = 1024: K = 672,
#   704 and 736 split in five ranges whose last holds one, two and three
#   32-deep steps; K = 4128 in five of 26).
@pytest.mark.parametrize("M,K,N,bf16", [
    (8192, 16, 3072, False), (8192, 32, 3072, False), (8192, 48, 3072, False),
    (8192, 272, 3072, False),
    (24576, 16, 768, False), (24576, 48, 768, False), (24576, 272, 768, False),
    (8192, 32, 3072, True), (8192, 64, 3072, True), (8192, 96, 3072, True), (8192, 288, 3072, True),
    (8192, 6176, 3072, True), (8192, 6208, 3072, True),
    (768, 32, 1024, False), (768, 64, 1024, False), (768, 96, 1024, False), (768, 4128, 1024, False),
    (768, 672, 1024, False), (768, 704, 1024, False), (768, 736, 1024, False),
    (1536, 16, 3072, False), (1536, 48, 3072, False), (1400, 272, 3072, False),
    (1536, 16, 4096, False), (1536, 48, 4096, False), (1400, 272, 4096, False),
    (8192, 256, 4096, False), (8142, 320, 4000, False), (8192, 1088, 2048, False),
    (768, 16, 4096, False), (768, 48, 4096, False), (768, 1024, 4096, False),
    (750, 272, 4000, False), (24500, 48, 760, False), (24500, 1024, 760, False),
    (768, 384, 3072, False), (750, 672, 3000, False), (768, 1024, 3072, False)])
def test_linear_direct_to_lds_k_classes(M, K, N, bf16):
    case(f"linear K classes M={M} K={K} N={N} bf16={bf16}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.05), rnd(N, scale=0.1)
    xd, Wd = dev(x), dev(W)
    if bf16:
        xr, Wr = xd.to(torch.bfloat16).double(), Wd.to(torch.bfloat16).double()
    else:
        xr, Wr = xd.double(), Wd.double()
    ref = host(torch.mm(xr, Wr.t().contiguous()) + dev(b).double())
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(xd), p(Wd), p(dev(b)), p(y), M, K, N, 0, G.EPI_BF16 if bf16 else 0,
                              None, stream()))
    assert_close(host(y), ref, rtol=1e-4, atol=4e-5 * np.sqrt(max(K, 256) / 1024),
                 name=f"K classes K={K}")


@pytest.mark.parametrize("M,K,N", [(768, 1024, 4096), (750, 288, 4000)])
@pytest.mark.parametrize("epi", ["gelu", "relu", "residual"])
def test_linear_32row_epilogues(M, K, N, epi):
    """The 32-row direct-to-LDS form (launches of 768 or more 32 x 128 tiles
    below 432 of 64 rows: 768 here, the second case ragged in M and N)
    with its one-block epilogue: bias + GELU, bias + ReLU, and a residual
    added in place, against an fp64 product."""
    case(f"linear 32-row M={M} K={K} N={N} {epi}")
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.05), rnd(N, scale=0.1), rnd(M, N)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b.astype(np.float64)
    if epi == "gelu":
        flags = G.EPI_GELU
        ref = 0.5 * ref * (1 + np.tanh(0.7978845608028654 * (ref + 0.044715 * ref ** 3)))
    elif epi == "relu":
        flags = G.EPI_RELU
        ref = np.maximum(ref, 0)
    else:
        flags = G.EPI_RESIDUAL
        ref = ref + r
    y = dev(r) if epi == "residual" else empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, flags,
                              p(y) if epi == "residual" else None, stream()))
    assert_close(host(y), ref, rtol=1e-4, atol=4e-5 * np.sqrt(K / 1024), name=f"32-row {epi}")


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
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 0, 4, 0, 0, None, stream())
    assert rc != 0 and b"positive" in L().gs_hip_last_error()
    rc = L().gs_hip_linear(p(x), p(x), None, p(x), 4, 32, 4, 2, 0, None, stream())
    assert rc != 0
    rc = L().gs_hip_linear(None, p(x), None, p(x), 4, 32, 4, 0, 0, None, stream())
    assert rc != 0 and b"null" in L().gs_hip_last_error()


# The reference's GPUOps.linear_forward takes any in / out width
# (src/nn/gpu_ops.cr:39-78; linear_forward_simple below 64): spec shapes
# (spec/nn/linear_spec.cr:29-38: 64 -> 32 over 8 rows, 16 -> 8 over 2x4 rows),
# the self-test's 512 -> 256 over 256 rows (src/main.cr:860-876) and ragged K
# in both weight layouts.
@pytest.mark.parametrize("M,K,N,layout", [(8, 64, 32, 0), (8, 16, 8, 0), (256, 512, 256, 0),
                                          (37, 33, 100, 0), (5, 1000, 77, 0), (9, 7, 3, 1),
                                          (64, 96, 30, 1), (3, 1, 1, 0)])
def test_linear_any_width(M, K, N, layout):
    case(f"linear any width M={M} K={K} N={N} layout={layout}")
    x, W, b = rnd(M, K), rnd(N, K, scale=0.1), rnd(N, scale=0.1)
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, layout, 0, None,
                              stream()))
    assert_close(host(y), O.linear(x, W, b, layout), name="linear any width")


@pytest.mark.parametrize("epi", ["gelu", "residual", "bf16", "f32x6"])
def test_linear_ragged_k_epilogues_and_variants(epi):
    case(f"linear ragged K {epi}")
    M, K, N = 70, 45, 130
    x, W, b, r = rnd(M, K), rnd(N, K, scale=0.1), rnd(N, scale=0.1), rnd(M, N)
    ref = O.linear(x, W, b)
    flags, res = 0, None
    if epi == "gelu":
        flags, ref = G.EPI_GELU, O.gelu(ref)
    elif epi == "residual":
        flags, res, ref = G.EPI_RESIDUAL, dev(r), ref + r
    elif epi == "bf16":
        flags = G.EPI_BF16
    else:
        flags = G.EPI_F32X6
    y = empty(M, N)
    G.check(L().gs_hip_linear(p(dev(x)), p(dev(W)), p(dev(b)), p(y), M, K, N, 0, flags,
                              p(res) if res is not None else None, stream()))
    if epi == "bf16":
        assert_close_bf16(host(y), ref, name="linear ragged bf16")
    else:
        assert_close(host(y), ref, name=f"linear ragged {epi}")


def test_linear_unaligned_operands():
    # rows starting 4 bytes into an allocation (16-byte alignment broken)
    case("linear unaligned operands")
    M, K, N = 40, 64, 48
    x, W, b = rnd(M, K), rnd(N, K, scale=0.1), rnd(N, scale=0.1)
    xb, wb = dev(np.concatenate([[0.0], x.ravel()])), dev(np.concatenate([[0.0], W.ravel()]))
    y = empty(M * N + 1)
    G.check(L().gs_hip_linear(p_off(xb, 4), p_off(wb, 4), p(dev(b)), p_off(y, 4), M, K, N, 0, 0,
                              None, stream()))
    assert_close(host(y)[1:].reshape(M, N), O.linear(x, W, b), name="linear unaligned")


# ---------------------------------------------------------------- layernorm


@pytest.mark.parametrize("rows,D", [(768, 1024), (1536, 768), (5, 132), (3, 4096)])
def test_layernorm_parity(rows, D):
    case(f"layernorm rows={rows} D={D}")
    x, g, b = rnd(rows, D, scale=2.0) + 0.5, rnd(D, scale=0.2) + 1, rnd(D, scale=0.2)
    y = empty(rows, D)
    G.check(L().gs_hip_layernorm(p(dev(x)), p(dev(g)), p(dev(b)), p(y), rows, D, 1e-6, stream()))
    assert_close(host(y), O.layernorm(x, g, b, 1e-6), name="layernorm")


# LayerNorm of any width (GPUOps.layernorm_forward takes any feature count,
# src/nn/gpu_ops.cr:114-138): the self-test's 256x256 (src/main.cr:878-892),
# odd widths, widths past 4096, and unaligned rows.
@pytest.mark.parametrize("rows,D,off", [(256, 256, 0), (5, 7, 0), (3, 4097, 0), (4, 6000, 0),
                                        (7, 130, 1), (9, 1, 0)])
def test_layernorm_any_width(rows, D, off):
    case(f"layernorm any width rows={rows} D={D} off={off}")
    x, g, b = rnd(rows, D, scale=2.0) + 0.5, rnd(D, scale=0.2) + 1, rnd(D, scale=0.2)
    pad = lambda a: dev(np.concatenate([np.zeros(off, np.float32), a.ravel()]))
    y = empty(rows * D + off)
    G.check(L().gs_hip_layernorm(p_off(pad(x), 4 * off), p_off(pad(g), 4 * off),
                                 p_off(pad(b), 4 * off), p_off(y, 4 * off), rows, D, 1e-5,
                                 stream()))
    assert_close(host(y)[off:].reshape(rows, D), O.layernorm(x, g, b, 1e-5), name="layernorm any")


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
    for hd in (0, -3):
        rc = L().gs_hip_attention(p(x), p(x), p(x), p(x), 1, 1, 1, 1, hd, 0.1, *([0] * 12),
                                  stream())
        assert rc != 0 and b"head_dim" in L().gs_hip_last_error()
    # the bf16 variants exist for the MFMA shapes only (head_dim 64, aligned rows)
    rc = L().gs_hip_attention_prec(p(x), p(x), p(x), p(x), 1, 1, 1, 1, 32, 0.1, *([32] * 12), 1,
                                   stream())
    assert rc != 0 and b"head_dim 64" in L().gs_hip_last_error()
    rc = L().gs_hip_attention_prec(p(x), p(x), p(x), p(x), 1, 1, 1, 1, 64, 0.1, *([64] * 12), 3,
                                   stream())
    assert rc != 0 and b"precision" in L().gs_hip_last_error()


# GPUOps.fused_attention takes any head_dim (src/nn/gpu_ops.cr:200-227); the
# reference's own shapes: the spec's self-attention 2x8 tokens, 4 heads of 16
# (spec/nn/attention_spec.cr:20-25, 49-58), its cross-attention 4 queries over 6
# keys, 2 heads of 16 (:28-37), the self-test's 2x32 tokens, 4 heads of 16
# (src/main.cr:894-909); then other head dims, the reference [B*H, N, hd]
# layout, and unaligned head-dim-64 rows (general kernel).
@pytest.mark.parametrize("B,H,Nq,Nkv,hd,layout", [
    (2, 4, 8, 8, 16, "tok"), (1, 2, 4, 6, 16, "tok"), (2, 4, 32, 32, 16, "tok"),
    (1, 3, 100, 77, 32, "tok"), (2, 2, 70, 70, 128, "tok"), (2, 2, 33, 65, 80, "bhnd"),
    (1, 2, 45, 200, 1, "bhnd"), (2, 3, 50, 40, 64, "odd"),
    # head dims beyond 128: chunks of 128, the last one ragged
    (1, 2, 37, 70, 129, "tok"), (2, 1, 20, 33, 200, "bhnd"), (1, 2, 9, 40, 256, "odd"),
    (1, 1, 5, 64, 1000, "tok")])
def test_attention_any_head_dim(B, H, Nq, Nkv, hd, layout):
    case(f"attention any head_dim B={B} H={H} Nq={Nq} Nkv={Nkv} hd={hd} {layout}")
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    q, k, v = rnd(B, H, Nq, hd, scale=2.0), rnd(B, H, Nkv, hd, scale=2.0), rnd(B, H, Nkv, hd)
    ref = O.sdpa(q, k, v, scale)
    if layout == "bhnd":
        st = lambda n: (H * n * hd, n * hd, hd)
        lay = lambda a: a
    else:  # token-major [B, N, H*hd]; "odd" adds one padding column per row
        extra = 1 if layout == "odd" else 0
        D = H * hd + extra
        st = lambda n: (n * D, hd, D)

        def lay(a):
            t = a.transpose(0, 2, 1, 3).reshape(B, a.shape[2], H * hd)
            return np.concatenate([t, np.zeros((B, a.shape[2], extra), np.float32)], -1)
    o = empty(B * Nq * H * hd + B * Nq * 2)
    G.check(L().gs_hip_attention(p(dev(lay(q))), p(dev(lay(k))), p(dev(lay(v))), p(o), B, H, Nq,
                                 Nkv, hd, scale, *st(Nq), *st(Nkv), *st(Nkv), *st(Nq), stream()))
    got = host(o)
    if layout == "bhnd":
        got = got[:B * H * Nq * hd].reshape(B, H, Nq, hd)
    else:
        D = H * hd + (1 if layout == "odd" else 0)
        got = got[:B * Nq * D].reshape(B, Nq, D)[..., :H * hd].reshape(B, Nq, H, hd)
        got = got.transpose(0, 2, 1, 3)
    assert_close(got, ref, name="attention any head_dim")


def bf16_round(a):
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def attn_prec_call(q, k, v, B, H, N, Nkv, prec, scale=0.125):
    """[B, H, N, 64] operands through gs_hip_attention_prec."""
    o = empty(B, H, N, 64)
    st = lambda n: (H * n * 64, n * 64, 64)
    G.check(L().gs_hip_attention_prec(p(dev(q)), p(dev(k)), p(dev(v)), p(o), B, H, N, Nkv, 64,
                                      scale, *st(N), *st(Nkv), *st(Nkv), *st(N), prec, stream()))
    return host(o)


@pytest.mark.parametrize("B,H,N,Nkv", [(2, 4, 300, 257), (4, 16, 768, 768)])
def test_attention_precision_variants(B, H, N, Nkv):
    """gs_hip_attention_prec: the bf16-input variant against the fp32 oracle
    at the bf16 bar (2e-2 norm-wise), the bf16x6 variant at the fp32 bar."""
    case(f"attention precision variants B={B} H={H} N={N} Nkv={Nkv}")
    q, k, v = rnd(B, H, N, 64, scale=1.5), rnd(B, H, Nkv, 64, scale=1.5), rnd(B, H, Nkv, 64)
    ref = O.sdpa(q, k, v, 0.125)
    got1 = attn_prec_call(q, k, v, B, H, N, Nkv, 1)
    rel, worst, p999 = assert_close_bf16(got1, ref, name="attention bf16")
    print(f"attention bf16: rel {rel:.2e} worst {worst:.2e} p99.9 elementwise {p999:.2e}")
    assert rel > 1e-5  # it really ran in bf16
    assert_close(attn_prec_call(q, k, v, B, H, N, Nkv, 2), ref, name="attention bf16x6")
    np.testing.assert_array_equal(attn_prec_call(q, k, v, B, H, N, Nkv, 0),
                                  attn_prec_call(q, k, v, B, H, N, Nkv, 0))


@pytest.mark.parametrize("kind", ["random", "all_negative"])
def test_attention_bf16_huge_logits(kind):
    """The bf16 flash kernel with scores of order 2^16 in its log2 domain,
    where one bf16 term for the running maximum would be off by up to 256
    and overflow (or underflow) exp2. The output is finite and matches a
    float64 softmax of the same bf16-rounded operands (q pre-scaled by
    scale * log2(e) before rounding, as the kernel does), at the bf16 bar."""
    case(f"attention bf16 huge logits {kind}")
    B, H, N, Nkv = 1, 2, 128, 192
    rng = np.random.default_rng(7)
    if kind == "random":
        q = (rng.standard_normal((B, H, N, 64)) * 128).astype(np.float32)
        k = (rng.standard_normal((B, H, Nkv, 64)) * 128).astype(np.float32)
    else:  # every score near -2^16: keys opposite to a shared query direction
        u = rng.standard_normal(64)
        u /= np.linalg.norm(u)
        q = np.broadcast_to(u * 700.0, (B, H, N, 64)).astype(np.float32)
        q = q + rng.standard_normal((B, H, N, 64)).astype(np.float32)
        k = np.broadcast_to(-u * 700.0, (B, H, Nkv, 64)).astype(np.float32)
        k = k + rng.standard_normal((B, H, Nkv, 64)).astype(np.float32) * 2
    v = rng.standard_normal((B, H, Nkv, 64)).astype(np.float32)
    qs = np.float32(0.125 * 1.4426950408889634)
    q2 = bf16_round(q * qs).astype(np.float64)
    k2, v2 = bf16_round(k).astype(np.float64), bf16_round(v).astype(np.float64)
    s2 = q2 @ k2.transpose(0, 1, 3, 2)
    mx = s2.max(-1, keepdims=True)
    assert np.abs(mx).max() > 2.0 ** 15  # the regime this test is for
    pr = np.exp2(s2 - mx)
    ref = (pr @ v2) / pr.sum(-1, keepdims=True)
    got = attn_prec_call(q, k, v, B, H, N, Nkv, 1)
    assert np.isfinite(got).all(), "non-finite bf16 attention output"
    rel, worst, _ = assert_close_bf16(got, ref, name=f"attention bf16 huge logits {kind}")
    print(f"attention bf16 huge logits {kind}: |m| max {np.abs(mx).max():.0f}, rel {rel:.2e}, "
          f"worst {worst:.2e}")


@pytest.mark.parametrize("B,N,Nkv,E,H", [(2, 8, 8, 64, 4), (1, 4, 6, 32, 2)])
def test_multi_head_attention_module_at_spec_shapes(B, N, Nkv, E, H):
    """MultiHeadAttention#forward (src/nn/attention.cr:49-81) through the op
    seam: q / k / v projections, heads of E/H split from the token-major rows,
    SDPA, output projection; against the oracle's composition of the same."""
    case(f"MHA module B={B} N={N} Nkv={Nkv} E={E} H={H}")
    hd = E // H
    xq, xkv = rnd(B, N, E), rnd(B, Nkv, E)
    Ws = {n: (rnd(E, E, scale=0.2), rnd(E, scale=0.1)) for n in ("q", "k", "v", "o")}
    proj = {}
    for n, src, rows in (("q", xq, N), ("k", xkv, Nkv), ("v", xkv, Nkv)):
        proj[n] = empty(B, rows, E)
        G.check(L().gs_hip_linear(p(dev(src)), p(dev(Ws[n][0])), p(dev(Ws[n][1])), p(proj[n]),
                                  B * rows, E, E, 0, 0, None, stream()))
    a = empty(B, N, E)
    st = lambda n: (n * E, hd, E)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    G.check(L().gs_hip_attention(p(proj["q"]), p(proj["k"]), p(proj["v"]), p(a), B, H, N, Nkv, hd,
                                 scale, *st(N), *st(Nkv), *st(Nkv), *st(N), stream()))
    out = empty(B, N, E)
    G.check(L().gs_hip_linear(p(a), p(dev(Ws["o"][0])), p(dev(Ws["o"][1])), p(out), B * N, E, E, 0,
                              0, None, stream()))
    heads = lambda t, n: t.reshape(B, n, H, hd).transpose(0, 2, 1, 3)
    rq = O.linear(xq.reshape(-1, E), *Ws["q"]).reshape(B, N, E)
    rk = O.linear(xkv.reshape(-1, E), *Ws["k"]).reshape(B, Nkv, E)
    rv = O.linear(xkv.reshape(-1, E), *Ws["v"]).reshape(B, Nkv, E)
    ra = O.sdpa(heads(rq, N), heads(rk, Nkv), heads(rv, Nkv), scale)
    ra = ra.transpose(0, 2, 1, 3).reshape(B * N, E)
    assert_close(host(out), O.linear(ra, *Ws["o"]).reshape(B, N, E), name="MHA module")


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


# GPUOps.conv2d_forward takes any channel count (src/nn/gpu_ops.cr:478-527):
# RGB-like inputs, ragged Cin, OHWI weights, strides and fused flags.
@pytest.mark.parametrize("B,H,W,Cin,Cout,k,s,pd,layout,flags,res", [
    (1, 6, 7, 3, 8, 3, 1, 1, 0, 0, False),
    (2, 5, 5, 40, 16, 1, 1, 0, 1, 0, False),
    (1, 9, 9, 17, 32, 3, 2, 1, 1, G.CONV_RELU_IN | G.CONV_RELU_OUT, True),
    (2, 8, 6, 50, 5, 3, 1, 0, 0, 0, True)])
def test_conv2d_any_channels(B, H, W, Cin, Cout, k, s, pd, layout, flags, res):
    case(f"conv2d any Cin B={B} {H}x{W} {Cin}->{Cout} k={k} s={s} p={pd} layout={layout}")
    x, w, b = rnd(B, H, W, Cin), rnd(Cout, Cin, k, k, scale=0.1), rnd(Cout, scale=0.1)
    Ho, Wo = (H + 2 * pd - k) // s + 1, (W + 2 * pd - k) // s + 1
    r = rnd(B, Ho, Wo, Cout)
    ref = O.conv2d(np.maximum(x, 0) if flags & G.CONV_RELU_IN else x, w, b, s, pd)
    if flags & G.CONV_RELU_OUT:
        ref = np.maximum(ref, 0)
    if res:
        ref = ref + r
    wk = w if layout == 0 else np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    y = empty(B, Ho, Wo, Cout)
    G.check(L().gs_hip_conv2d(p(dev(x)), B, H, W, Cin, p(dev(wk)), p(dev(b)), p(y), Cout, k, s, pd,
                              layout, flags, p(dev(r)) if res else None, stream()))
    assert_close(host(y), ref, name="conv2d any Cin")


# conv2d_forward reads kernel_h and kernel_w separately (src/nn/gpu_ops.cr:
# 491-495): kh x kw kernels through gs_hip_conv2d_hw, on the register-staged
# conv kernel, the bf16x6 kernel, the direct-to-LDS conv kernel (768 tiles of
# 192 rows; K = 96 and 48, six and three 16-deep steps of one tap each) and
# its 64-row form (768 and 576 tiles of 64 rows, the second strided with a
# ReLU epilogue; then 768 and 784 tiles at K = 144 and 48, nine and three
# 16-deep steps: odd step counts end the two-stage loop on either stage).
@pytest.mark.parametrize("B,H,W,Cin,Cout,kh,kw,s,pd,layout,flags", [
    (2, 9, 11, 32, 40, 1, 3, 1, 1, 0, 0),
    (1, 12, 10, 64, 32, 3, 1, 2, 1, 1, G.CONV_RELU_OUT),
    (2, 7, 13, 20, 16, 2, 5, 1, 2, 0, G.CONV_RELU_IN),
    (1, 10, 10, 32, 64, 5, 2, 3, 0, 0, G.CONV_F32X6),
    (1, 192, 382, 32, 256, 3, 1, 1, 1, 0, 0),
    (1, 192, 384, 16, 256, 3, 1, 1, 1, 0, 0),
    (2, 96, 128, 64, 256, 3, 3, 1, 1, 0, 0),
    (32, 24, 32, 64, 768, 3, 3, 2, 1, 0, G.CONV_RELU_OUT),
    (2, 96, 128, 16, 256, 3, 3, 1, 1, 0, 0),
    (2, 96, 128, 16, 256, 1, 3, 1, 1, 1, 0)])
def test_conv2d_nonsquare_kernel(B, H, W, Cin, Cout, kh, kw, s, pd, layout, flags):
    case(f"conv2d_hw B={B} {H}x{W} {Cin}->{Cout} k={kh}x{kw} s={s} p={pd} layout={layout} "
         f"flags={flags}")
    x, w, b = rnd(B, H, W, Cin), rnd(Cout, Cin, kh, kw, scale=0.1), rnd(Cout, scale=0.1)
    Ho, Wo = (H + 2 * pd - kh) // s + 1, (W + 2 * pd - kw) // s + 1
    ref = O.conv2d(np.maximum(x, 0) if flags & G.CONV_RELU_IN else x, w, b, s, pd)
    if flags & G.CONV_RELU_OUT:
        ref = np.maximum(ref, 0)
    assert ref.shape == (B, Ho, Wo, Cout)
    wk = w if layout == 0 else np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    y = empty(B, Ho, Wo, Cout)
    G.check(L().gs_hip_conv2d_hw(p(dev(x)), B, H, W, Cin, p(dev(wk)), p(dev(b)), p(y), Cout, kh,
                                 kw, s, pd, layout, flags, None, stream()))
    assert_close(host(y), ref, name="conv2d_hw")


def test_op_scratch_is_per_stream():
    """Op-level calls whose kernels use scratch (OIHW conv re-layout, ragged
    linear staging, bf16 weight copies, compaction block counts), issued
    back to back on two streams without synchronisation in between, each
    produce their own results: scratch is stream-ordered, not shared."""
    case("op scratch on two streams")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cv, ln_, cp = [], [], []
    for i, st in enumerate(streams):
        B, H, W, C = 1, 24, 32, 96 + 32 * i
        x, w, b = rnd(B, H, W, C), rnd(C, C, 3, 3, scale=0.05), rnd(C, scale=0.1)
        xl, wl = rnd(300, 45 + i), rnd(200, 45 + i, scale=0.1)
        conf = RNG.uniform(0, 1, 50000 + 7000 * i).astype(np.float32)
        pts = rnd(conf.size, 3)
        cv.append((x, w, b, dev(x), dev(w), dev(b), empty(B, H, W, C)))
        ln_.append((xl, wl, dev(xl), dev(wl), empty(300, 200), empty(300, 200)))
        cnt = dev(np.zeros(2, np.float32)).view(torch.int64)
        cnt.zero_()
        cp.append((pts, conf, dev(pts), dev(conf), empty(conf.size, 3), empty(conf.size), cnt))
    torch.cuda.synchronize()
    for _ in range(3):  # repeated, interleaved across the streams
        for i, st in enumerate(streams):
            x, w, b, xd, wd, bd, y = cv[i]
            G.check(L().gs_hip_conv2d(p(xd), 1, 24, 32, x.shape[-1], p(wd), p(bd), p(y), x.shape[-1],
                                      3, 1, 1, 0, 0, None, st.cuda_stream))
            xl, wl, xld, wld, yl, yh = ln_[i]
            K = xl.shape[1]
            G.check(L().gs_hip_linear(p(xld), p(wld), None, p(yl), 300, K, 200, 0, 0, None,
                                      st.cuda_stream))
            G.check(L().gs_hip_linear(p(xld), p(wld), None, p(yh), 300, K, 200, 0, G.EPI_BF16, None,
                                      st.cuda_stream))
    for i, st in enumerate(streams):
        pts, conf, ptd, cfd, op, oc, cnt = cp[i]
        G.check(L().gs_hip_collect_points(p(ptd), p(cfd), conf.size, 0.5, p(op), p(oc), conf.size,
                                          p(cnt), st.cuda_stream))
    torch.cuda.synchronize()
    for i in range(2):
        x, w, b, _, _, _, y = cv[i]
        assert_close(host(y), O.conv2d(x, w, b, 1, 1), name=f"conv stream {i}")
        xl, wl, _, _, yl, yh = ln_[i]
        assert_close(host(yl), O.linear(xl, wl), name=f"linear stream {i}")
        assert_close_bf16(host(yh), O.linear(xl, wl), name=f"linear bf16 stream {i}")
        pts, conf, _, _, op, oc, cnt = cp[i]
        n = int(host(cnt)[0])
        rp, rc = O.collect_points(pts, conf, 0.5)
        assert n == len(rc)
        np.testing.assert_array_equal(host(op)[:n], rp)
        np.testing.assert_array_equal(host(oc)[:n], rc)


@pytest.mark.parametrize("B,H,W,C", [(1, 96, 128, 256), (2, 5, 7, 8), (2, 48, 64, 128),
                                     (1, 3, 37, 12), (1, 1, 1, 4), (1, 3, 5, 2048)])
def test_upsample_parity(B, H, W, C):
    """Channel widths of one and of several workgroup steps, a width that
    leaves threads idle (C / 4 = 3), a 1 x 1 input and rows wider than a
    workgroup (C / 4 > 256)."""
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
