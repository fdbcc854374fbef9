"""MASt3R two-view inference throughput on one MI355X (pairs/s, fp32).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|2|4]
    python bench.py --workload frames|ref512|checkpoint   (secondary lines)

A step is one full forward (ViT-L encoder on both views, ViT-B cross-attention
decoder, two DPT heads, two local-feature heads) over one batch of synthetic
image pairs already resident in HBM. Default workload: config 3 of the
baseline (16 pairs at 3x384x512, U(-1,1) images, seed-0 N(0,0.02) weights).
Prints one JSON line.

Secondary workloads (each its own JSON line, not the headline metric):
  frames      frames_to_pointcloud: 33 synthetic 720x1280 frames resized and
              normalised on the device, 32 consecutive pairs at 512x512 in one
              batched call, confidence compaction; pairs/s end to end, with
              the HBM roofline of the resize / compaction passes.
  ref512      the reference-literal composition at 512x512 (stub DPT heads),
              32 pairs per step; pairs/s.
  checkpoint  gs_hip_mastr_load_safetensors of an fp32 checkpoint of the
              default configuration written to a temporary file; GB/s.
  block       config 0: one ViT-L encoder block, 768 tokens; ms per block.
  encoder     config 1: the full ViT-L encoder on one 384x512 image.
  cpu         the oracle's literal reference loops on the host: config 0 at 1 and
              all threads, config 1 (24 blocks, progress on stderr) at 1 and all
              threads; config 2 extrapolated by FLOPs.
  linear-vs-library
              the config-3 linear shapes (bias epilogue) through gs_hip_linear
              and through torch's fp32 F.linear (the ROCm BLAS libraries) on the
              same device tensors, alternating; TFLOP/s of each and their ratio.
  library-bf16
              the vendor library's bf16 GEMM (torch F.linear on bf16 tensors) on
              the config-4 linear shapes; TFLOP/s per shape (reference point).
  ref-selftest
              the reference's own GPU micro-benchmarks (src/main.cr:860-909):
              Linear 256x512->256, LayerNorm 256x256, MHA 2x32x64 with 4 heads
              of 16, through the op-level C ABI; ms per iteration beside the
              M2 Max figures the reference records (a different machine).
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "crystal-gausplat_amd"))

MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0
# fp32 through bf16x6 split products: six bf16 MFMAs per fp32-equivalent
# product, so its fp32-equivalent ceiling is the bf16 peak / 6
MFMA_X6_PEAK_TFLOPS = MFMA_BF16_PEAK_TFLOPS / 6


def kernel_peak(name):
    """MFMA ceiling of a library kernel in the units bench.py counts its flops:
    bf16 kernels 2.5 PFLOP/s, bf16x6 kernels (fp32-equivalent flops) 2.5/6,
    fp32 kernels 157.3 TFLOP/s."""
    if "bf16" in name:
        return MFMA_BF16_PEAK_TFLOPS
    if "_x6_" in name:
        return MFMA_X6_PEAK_TFLOPS
    return MFMA_FP32_PEAK_TFLOPS
HBM_PEAK_GBS = 8000.0
# Algorithmic work of one 384x512 pair and of one config-0 encoder block
# (GFLOP), from the FLOP model of the path.
PAIR_GFLOP_384x512 = 2037.2
BLOCK_GFLOP = 21.74

CONFIGS = {
    2: dict(pairs=1, img_h=384, img_w=512),
    3: dict(pairs=16, img_h=384, img_w=512),
    4: dict(pairs=32, img_h=512, img_w=512),
}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline():
    """Reference CPU path stand-in, timed on the host: the oracle's literal
    reference loops (Linear i-j-k, attention scores / softmax / PV, conv
    kh-kw-ic) on one full config-2 pair (384x512, seed-0 weights and images)
    on all host threads -- the measured figure -- and one config-0 ViT-L block
    on 1 thread and on all threads; the block's thread ratio extrapolates the
    measured pair to one thread (labelled as extrapolated)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import gsplat_hip as G
    import pyoracle as O

    cfg = G.default_config()
    w = G.seeded_weights(cfg, 0)
    n = 3 * 384 * 512
    i1 = G.seed_uniform(0, "view1", n).reshape(1, 3, 384, 512)
    i2 = G.seed_uniform(0, "view2", n).reshape(1, 3, 384, 512)
    O.set_naive(True)
    O.set_threads(0)
    threads_all = O.lib().orc_get_threads()
    print(f"[cpu] one 384x512 pair through the literal loops on {threads_all} threads",
          file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    out = O.mastr_pair(cfg.as_dict(), w, i1, i2)
    dt_pair = time.perf_counter() - t0
    assert all(np.isfinite(v).all() for v in out.values())
    print(f"[cpu] pair: {dt_pair:.1f} s", file=sys.stderr, flush=True)
    x = G.seed_normal(0, "tokens", 768 * 1024).reshape(1, 768, 1024)
    t0 = time.perf_counter()
    y_all = O.encoder_block(cfg.as_dict(), w, "enc_blocks.0", x, 24, 32)
    dt_all = time.perf_counter() - t0
    O.set_threads(1)
    t0 = time.perf_counter()
    y_one = O.encoder_block(cfg.as_dict(), w, "enc_blocks.0", x, 24, 32)
    dt_one = time.perf_counter() - t0
    O.set_naive(False)
    O.set_threads(0)
    assert np.array_equal(y_one, y_all)  # threads split output rows only: same bits
    thread_ratio = dt_one / dt_all
    s_pair_1t = dt_pair * thread_ratio
    return {
        "value": 1.0 / dt_pair,
        "unit": "pairs/s",
        "cores": threads_all,
        "kind": "port",
        "measured_s_per_pair": round(dt_pair, 2),
        "value_1_thread_extrapolated": 1.0 / s_pair_1t,
        "s_per_pair_1_thread_extrapolated": round(s_pair_1t, 1),
        "cpu": cpu_model(),
        "logical_cpus": os.cpu_count(),
        "extrapolation": f"1-thread figure only: the measured {threads_all}-thread pair x the "
                         f"config-0 block's measured 1-thread / {threads_all}-thread time ratio "
                         f"({dt_one:.2f} s / {dt_all:.3f} s = {thread_ratio:.2f})",
        "sample": (f"one full config-2 pair (two 3x384x512 U(-1,1) images, seed-0 N(0,0.02) "
                   f"weights: ViT-L encoder x2, ViT-B decoder, 2 DPT heads, 2 descriptor heads, "
                   f"2037.2 GFLOP) through the oracle's literal reference loops: {dt_pair:.1f} s "
                   f"measured on {threads_all} threads; one config-0 ViT-L block (21.74 GFLOP): "
                   f"{dt_one:.2f} s on 1 thread, {dt_all:.3f} s on {threads_all} threads "
                   f"(bit-identical); host CPU: {cpu_model()}, {os.cpu_count()} logical CPUs"),
    }


def cpu_table():
    """Oracle (literal reference loops) timings on the host for BASELINE's table."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import gsplat_hip as G
    import pyoracle as O
    cfg = G.default_config(enc_depth=24, dec_depth=1, dpt_hooks=[0, 1, 1, 1])
    inv = G.weight_inventory(cfg)
    w = {n: G.weight_values(cfg, i, int(np.prod(s))).reshape(s)
         for i, (n, s, k) in enumerate(inv) if n.startswith(("enc_blocks.", "patch_embed.", "enc_norm."))}
    nthreads = os.cpu_count()
    O.set_naive(True)
    res = {}
    x = G.seed_normal(0, "tokens", 768 * 1024).reshape(1, 768, 1024)
    for T in (1, nthreads):
        O.set_threads(T)
        t0 = time.perf_counter()
        O.encoder_block(cfg.as_dict(), w, "enc_blocks.0", x, 24, 32)
        res[f"config0_s_{T}t"] = round(time.perf_counter() - t0, 3)
        print(f"[cpu] config 0, {T} threads: {res[f'config0_s_{T}t']} s", file=sys.stderr, flush=True)
    img = G.seed_uniform(0, "view1", 3 * 384 * 512).reshape(1, 3, 384, 512)
    for T in (nthreads, 1):
        O.set_threads(T)
        t0 = time.perf_counter()
        # the encoder block by block (same work as O.encoder), so progress shows
        pe = O.unfold(img, 16)
        h = O.linear(pe.reshape(-1, 768), w["patch_embed.proj.weight"].reshape(1024, -1),
                     w["patch_embed.proj.bias"], naive=True).reshape(1, 768, 1024)
        for l in range(24):
            h = O.encoder_block(cfg.as_dict(), w, f"enc_blocks.{l}", h, 24, 32)
            print(f"[cpu] config 1, {T} threads: block {l} at {time.perf_counter() - t0:.1f} s",
                  file=sys.stderr, flush=True)
        O.layernorm(h, w["enc_norm.weight"], w["enc_norm.bias"], cfg.ln_eps)
        res[f"config1_s_{T}t"] = round(time.perf_counter() - t0, 2)
    O.set_naive(False)
    O.set_threads(0)
    ratio = PAIR_GFLOP_384x512 / 523.0
    return {"metric": "reference CPU path (oracle literal loops) seconds", "unit": "s",
            "cpu": cpu_model(), "threads_all": nthreads, **res,
            "config2_s_per_pair_1t_extrapolated": round(res["config1_s_1t"] * ratio, 1),
            "config2_s_per_pair_all_extrapolated": round(res[f"config1_s_{nthreads}t"] * ratio, 1),
            "extrapolation": f"config 1 x {ratio:.3f} (2037.2 / 523.0 GFLOP)"}


def _timed(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _kernel_rates(prof, steps):
    return {k: {"launches": v["launches"] // steps, "ms_per_step": round(v["ms"] / steps, 3),
                "gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1) if v["bytes"] else None,
                "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2) if v["flops"] else None}
            for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}


# (name, M, N, K) of the config-3 linears: encoder on 2 x 16 images of 768
# tokens, decoder per chain on 16 x 768 tokens, descriptor MLP per head
LIBRARY_SHAPES = [("encoder fc1", 24576, 4096, 1024), ("encoder qkv", 24576, 3072, 1024),
                  ("encoder proj", 24576, 1024, 1024), ("encoder fc2", 24576, 1024, 4096),
                  ("decoder fc1", 12288, 3072, 768), ("decoder fc2", 12288, 768, 3072),
                  ("decoder proj", 12288, 768, 768), ("descriptor fc2", 12288, 6144, 7168)]


def linear_vs_library(args):
    """Our fp32 GEMM against the vendor library on the same shapes and tensors.
    A reference point for the kernels, not a model measurement."""
    import torch

    import gsplat_hip as G
    torch.backends.cuda.matmul.allow_tf32 = False
    L = G.lib()
    stream = torch.cuda.current_stream().cuda_stream
    reps = max(args.steps, 5)

    def timed(f):
        for _ in range(2):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    rows, t_ours, t_lib, flops = [], 0.0, 0.0, 0.0
    for name, M, N, K in LIBRARY_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.rand(M, K, device="cuda", generator=g) * 2 - 1
        w = (torch.rand(N, K, device="cuda", generator=g) * 2 - 1) * 0.02
        b = (torch.rand(N, device="cuda", generator=g) * 2 - 1) * 0.02
        y = torch.empty(M, N, device="cuda")
        ours = lambda: G.check(L.gs_hip_linear(G.ptr(a), G.ptr(w), G.ptr(b), G.ptr(y), M, K, N,
                                               0, 0, None, stream))
        lib = lambda: torch.nn.functional.linear(a, w, b)
        mo, ml = [], []
        for _ in range(2):  # alternate, keep the faster of two rounds each
            mo.append(timed(ours))
            ml.append(timed(lib))
        mo, ml = min(mo), min(ml)
        # both results against an fp64 product of the same tensors
        ref = torch.nn.functional.linear(a.double(), w.double(), b.double())
        ours()
        torch.cuda.synchronize()
        scale = ref.abs().max().item()
        err_o = (y.double() - ref).abs().max().item() / scale
        err_l = (lib().double() - ref).abs().max().item() / scale
        del ref
        fl = 2.0 * M * N * K
        t_ours, t_lib, flops = t_ours + mo, t_lib + ml, flops + fl
        rows.append({"shape": f"{name} M={M} N={N} K={K}", "ours_tflops": round(fl / mo / 1e9, 1),
                     "library_tflops": round(fl / ml / 1e9, 1), "ratio": round(ml / mo, 3),
                     "max_err_vs_fp64": {"ours": float(f"{err_o:.3g}"), "library": float(f"{err_l:.3g}")}})
        del a, w, b, y
    return {"metric": "fp32 linear (bias) throughput, gs_hip_linear vs torch F.linear",
            "value": round(flops / t_ours / 1e9, 1), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": reps, "warmup": 2, "higher_is_better": True, "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "library_tflops": round(flops / t_lib / 1e9, 1),
            "ratio_ours_over_library": round(t_lib / t_ours, 3),
            "config": {"workload": "config-3 linear shapes, one launch each"}, "shapes": rows}


# The reference's self-test micro-benchmarks (src/main.cr:860-909) and the
# timings its TODO.md:111,118 records for them on an Apple M2 Max (a different
# machine: listed beside ours, not a like-for-like comparison).
REF_SELFTEST_M2MAX_MS = {"linear": 1.2, "layernorm": 1.3, "mha": 1.6}


def ref_selftest(args):
    """GPU Linear 512->256 over 256 rows, GPU LayerNorm 256 over 256 rows and
    GPU MultiHeadAttention self-attention (2 x 32 tokens, embed 64, 4 heads of
    16: q / k / v projections, attention, output projection) through the
    op-level C ABI, as src/main.cr:860-909 runs them: one warm-up, then 10
    iterations. Reported per iteration as the reference measures it (loop,
    then one synchronisation) and with a synchronisation after every
    iteration (the reference's Metal ops each wait for completion)."""
    import torch

    import gsplat_hip as G
    L = G.lib()
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(0)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)
    P = G.ptr
    x_lin, w_lin, b_lin = rn(256, 512), rn(256, 512) * 0.05, rn(256) * 0.05
    y_lin = torch.empty(256, 256, device="cuda")
    x_ln, g_ln, b_ln = rn(256, 256), torch.ones(256, device="cuda"), torch.zeros(256, device="cuda")
    y_ln = torch.empty(256, 256, device="cuda")
    B, N, E, H = 2, 32, 64, 4
    x_at = rn(B, N, E)
    Wm = {k: (rn(E, E) * 0.1, rn(E) * 0.1) for k in "qkvo"}
    proj = {k: torch.empty(B, N, E, device="cuda") for k in "qkv"}
    a_at, y_at = torch.empty(B, N, E, device="cuda"), torch.empty(B, N, E, device="cuda")
    hd = E // H
    stt = (N * E, hd, E)

    def linear():
        G.check(L.gs_hip_linear(P(x_lin), P(w_lin), P(b_lin), P(y_lin), 256, 512, 256, 0, 0, None,
                                st))

    def layernorm():
        G.check(L.gs_hip_layernorm(P(x_ln), P(g_ln), P(b_ln), P(y_ln), 256, 256, 1e-5, st))

    def mha():
        for k in "qkv":
            G.check(L.gs_hip_linear(P(x_at), P(Wm[k][0]), P(Wm[k][1]), P(proj[k]), B * N, E, E, 0,
                                    0, None, st))
        G.check(L.gs_hip_attention(P(proj["q"]), P(proj["k"]), P(proj["v"]), P(a_at), B, H, N, N,
                                   hd, float(1.0 / hd ** 0.5), *stt, *stt, *stt, *stt, st))
        G.check(L.gs_hip_linear(P(a_at), P(Wm["o"][0]), P(Wm["o"][1]), P(y_at), B * N, E, E, 0, 0,
                                None, st))

    iters = 10
    res = {}
    for name, fn, what in (("linear", linear, "Linear 256x512 -> 256 (bias)"),
                           ("layernorm", layernorm, "LayerNorm 256 x 256"),
                           ("mha", mha, "MultiHeadAttention self-attention 2 x 32 x 64, 4 heads "
                                        "of 16 (3 projections, attention, output projection)")):
        fn()  # warm-up, as the reference
        torch.cuda.synchronize()
        best_loop, best_sync = float("inf"), float("inf")
        for _ in range(5):  # five repetitions of the reference's 10-iteration loop, best kept
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
            torch.cuda.synchronize()
            best_loop = min(best_loop, (time.perf_counter() - t0) * 1e3 / iters)
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
                torch.cuda.synchronize()
            best_sync = min(best_sync, (time.perf_counter() - t0) * 1e3 / iters)
        G.profile_begin()
        fn()
        torch.cuda.synchronize()
        prof = G.profile_end()
        res[name] = {"what": what, "ms_per_iter": round(best_loop, 4),
                     "ms_per_iter_synced": round(best_sync, 4),
                     "kernel_ms": round(sum(v["ms"] for v in prof.values()), 4),
                     "kernels": sorted(prof),
                     "reference_m2max_ms_per_iter": REF_SELFTEST_M2MAX_MS[name]}
    res["linear"]["tflops"] = round(2.0 * 256 * 512 * 256 / (res["linear"]["ms_per_iter"] * 1e-3)
                                    / 1e12, 3)
    return {"metric": "reference self-test GPU micro-benchmarks (src/main.cr:860-909) through "
                      "the op-level C ABI, ms per iteration",
            "value": round(sum(r["ms_per_iter"] for r in res.values()), 4),
            "unit": "ms (sum of the three, per iteration)", "n_gpus": 1, "steps": iters,
            "warmup": 1, "higher_is_better": False, "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (torch seeded normal)",
            "config": {"workload": "ref-selftest: Linear 256x512->256, LayerNorm 256x256, MHA "
                                   "2x32x64 with 4 heads of 16"},
            "reference_note": "reference_m2max_ms_per_iter are the figures TODO.md:111,118 of the "
                              "reference records on an Apple M2 Max (Metal, one synchronous "
                              "command buffer per op): a different machine, listed beside ours "
                              "for orientation, not a like-for-like claim",
            "ops": res}


# (name, M, N, K) of the config-4 linears (32 pairs at 512x512: encoder on
# 2 x 32 images of 1024 tokens, decoder per chain on 32 x 1024 tokens)
LIBRARY_SHAPES_C4 = [("encoder fc1", 65536, 4096, 1024), ("encoder qkv", 65536, 3072, 1024),
                     ("encoder proj", 65536, 1024, 1024), ("encoder fc2", 65536, 1024, 4096),
                     ("decoder fc1", 32768, 3072, 768), ("decoder qkv", 32768, 2304, 768),
                     ("decoder proj", 32768, 768, 768), ("decoder fc2", 32768, 768, 3072)]


def library_bf16(args):
    """The vendor library's bf16 GEMM (torch F.linear on bf16 tensors, bias
    epilogue) on the config-4 linear shapes: the reference point for the bf16
    kernels, whose per-shape rates in the model come from --precision bf16
    --per-shape."""
    import torch
    reps = max(args.steps, 5)
    rows, t_lib, flops = [], 0.0, 0.0
    for name, M, N, K in LIBRARY_SHAPES_C4:
        g = torch.Generator(device="cuda").manual_seed(0)
        a = (torch.rand(M, K, device="cuda", generator=g) * 2 - 1).bfloat16()
        w = ((torch.rand(N, K, device="cuda", generator=g) * 2 - 1) * 0.02).bfloat16()
        b = ((torch.rand(N, device="cuda", generator=g) * 2 - 1) * 0.02).bfloat16()
        f = lambda: torch.nn.functional.linear(a, w, b)
        for _ in range(2):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        fl = 2.0 * M * N * K
        t_lib, flops = t_lib + ms, flops + fl
        rows.append({"shape": f"{name} M={M} N={N} K={K}", "library_tflops": round(fl / ms / 1e9, 1)})
        del a, w, b
    return {"metric": "vendor bf16 linear (torch F.linear, bias) throughput on the config-4 shapes",
            "value": round(flops / t_lib / 1e9, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps,
            "warmup": 2, "higher_is_better": True, "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic", "config": {"workload": "config-4 linear shapes, one launch each"},
            "shapes": rows}


def secondary(args):
    import torch

    import gsplat_hip as G
    out = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    stream = torch.cuda.current_stream().cuda_stream
    if args.workload == "checkpoint":
        import tempfile

        from safetensors.numpy import save_file
        cfg = G.default_config()
        w = G.seeded_weights(cfg, 0, 0.02, 0.1)
        nbytes = sum(a.nbytes for a in w.values())
        m = G.Mastr(cfg, 1)
        with tempfile.TemporaryDirectory() as td:
            path = os.path.join(td, "mastr.safetensors")
            save_file(w, path)
            del w
            counts = m.load_safetensors(path)  # warm the page cache
            sec = _timed(lambda: m.load_safetensors(path), args.steps, 0)
        m.close()
        out.update(metric="MASt3R fp32 checkpoint ingestion (mmap, convert, re-layout, upload)",
                   value=round(nbytes / sec / 1e9, 3), unit="GB/s", ms_per_step=round(sec * 1e3, 1),
                   config={"workload": f"{counts['loaded']} tensors, {nbytes / 1e9:.2f} GB F32, "
                                       "page-cached file"})
        return out
    if args.workload in ("block", "encoder"):
        cfg = G.default_config()
        m = G.Mastr(cfg, 1)
        m.init_seeded(0)
        if args.workload == "block":  # applied in place, step after step
            x = torch.from_numpy(G.seed_normal(0, "tokens", 768 * 1024).reshape(1, 768, 1024)).cuda()
            fn = lambda: m.encoder_block(0, x, 1, stream=stream)
            gflop, what = BLOCK_GFLOP, "config 0: one ViT-L block, 768 tokens, batch 1"
        else:
            img = torch.from_numpy(G.seed_uniform(0, "view1", 3 * 384 * 512).reshape(1, 3, 384, 512)).cuda()
            enc = torch.empty(1, 768, 1024, device="cuda")
            fn = lambda: m.encoder(img, 1, enc, stream=stream)
            gflop, what = 523.0, "config 1: ViT-L encoder, one 3x384x512 image"
        sec = _timed(fn, args.steps, args.warmup)
        G.profile_begin()
        fn()
        torch.cuda.synchronize()
        prof = G.profile_end()
        if args.per_shape:
            G.profile_begin(per_shape=True)
            fn()
            torch.cuda.synchronize()
            for k, v in sorted(G.profile_end().items(), key=lambda kv: -kv[1]["ms"]):
                tf = v["flops"] / (v["ms"] * 1e-3) / 1e12 if v["flops"] else 0.0
                print(f"{v['ms']:9.3f} ms {v['launches']:4d}x {tf:7.1f} TF/s  {k}", file=sys.stderr)
        m.close()
        mm = [v for k, v in prof.items() if k.startswith(("gemm", "attn"))]
        frac = sum(v["flops"] for v in mm) / (sum(v["ms"] for v in mm) * 1e-3) / 1e12 / MFMA_FP32_PEAK_TFLOPS
        out.update(metric=f"MASt3R {args.workload} forward time, fp32", value=round(sec * 1e3, 4),
                   unit="ms", higher_is_better=False, ms_per_step=round(sec * 1e3, 4),
                   config={"workload": what},
                   achieved_tflops=round(gflop / sec / 1e3, 2),
                   gemm_attn_frac_mfma_peak=round(frac, 4), kernels=_kernel_rates(prof, 1))
        return out
    if args.workload == "cpu":
        return cpu_table()
    if args.workload == "linear-vs-library":
        return linear_vs_library(args)
    if args.workload == "ref-selftest":
        return ref_selftest(args)
    if args.workload == "library-bf16":
        return library_bf16(args)
    if args.workload == "ref512":
        B = args.pairs or 32
        cfg = G.ref512_config()
        m = G.Mastr(cfg, B)
        m.init_seeded(0)
        n = B * 3 * 512 * 512
        i1 = torch.from_numpy(G.seed_uniform(0, "view1", n).reshape(B, 3, 512, 512)).cuda()
        i2 = torch.from_numpy(G.seed_uniform(0, "view2", n).reshape(B, 3, 512, 512)).cuda()
        o = [torch.empty(B, 32, 32, c, device="cuda") for c in (3, 1, 3, 1)]
        fn = lambda: m.pair(i1, i2, B, o[0], o[1], None, o[2], o[3], None, stream=stream)
        sec = _timed(fn, args.steps, args.warmup)
        G.profile_begin()
        fn()
        torch.cuda.synchronize()
        prof = G.profile_end()
        m.close()
        out.update(metric="reference-literal MASt3R forward_pair (ref512) pairs/sec, fp32",
                   value=round(B / sec, 3), unit="pairs/s", ms_per_step=round(sec * 1e3, 3),
                   config={"workload": f"ref512: {B} pairs at 3x512x512, stub DPT heads on the "
                                       "32x32 patch grid"},
                   kernels=_kernel_rates(prof, 1))
        return out
    # frames -> point cloud
    F, sh, sw = 33, 720, 1280
    cfg = G.default_config(img_h=512, img_w=512)
    m = G.Mastr(cfg, F - 1)
    m.init_seeded(0)
    frames = torch.rand(F, sh, sw, 3, device="cuda", generator=torch.Generator("cuda").manual_seed(0))
    cap = F * 512 * 512
    op, oc = torch.empty(cap, 3, device="cuda"), torch.empty(cap, device="cuda")
    npts = []
    fn = lambda: npts.append(m.frames_to_pointcloud(frames, 0.3, op, oc, stream=stream))
    sec = _timed(fn, args.steps, args.warmup)
    G.profile_begin()
    fn()
    torch.cuda.synchronize()
    prof = G.profile_end()
    m.close()
    rates = _kernel_rates(prof, 1)
    passes = {k: v for k, v in rates.items() if k.startswith(("image_prep", "collect_points"))}
    dom = max(passes, key=lambda k: passes[k]["ms_per_step"])
    out.update(metric="MASt3R frames_to_pointcloud, consecutive pairs/sec @512x512 fp32 "
                      "(device resize/normalise + pairs + compaction)",
               value=round((F - 1) / sec, 3), unit="pairs/s", ms_per_step=round(sec * 1e3, 3),
               config={"workload": f"{F} frames 3x{sh}x{sw} -> {F - 1} pairs at 512x512, "
                                   f"threshold 0.3, {npts[-1]} points"},
               roofline={"bound": "hbm", "kernel": dom, "achieved": passes[dom]["gbs"],
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(passes[dom]["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
               caller_passes=passes,
               caller_share_of_step=round(sum(v["ms_per_step"] for v in passes.values())
                                          / (sec * 1e3), 5))
    return out


# Algorithmic work of one 512x512 pair (GFLOP), same FLOP model.
PAIR_GFLOP_512x512 = 2806.4
ENCODER_GFLOP = 523.0
PREC_NAME = {0: "fp32", 1: "bf16", 2: "fp32x6"}
PREC_DTYPE = {0: "f32", 1: "bf16-in/f32-acc", 2: "f32 (bf16x6 split products, f32 acc)"}
# the MFMA ceiling each precision's flops are counted against
PREC_PEAK = {0: MFMA_FP32_PEAK_TFLOPS, 1: MFMA_BF16_PEAK_TFLOPS, 2: MFMA_X6_PEAK_TFLOPS}


def _event_timed(fn, steps, warmup):
    """Seconds per step: W warm-up steps, then K steps between two HIP events
    on the current (launch) stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / steps


def _profiled(fn, steps):
    """Per-kernel launch records (the library's own HIP event pairs) over
    `steps` further steps."""
    import torch

    import gsplat_hip as G
    G.profile_begin()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return G.profile_end()


def _mfma_summary(prof, steps):
    """GEMM+attention fraction of the MFMA peak (each kernel against its own
    precision's ceiling) and the dominant kernel's rate."""
    mm = [(k, v) for k, v in prof.items() if k.startswith(("gemm", "attn"))]
    fl = sum(v["flops"] for k, v in mm)
    cap = sum(v["ms"] * 1e-3 * kernel_peak(k) * 1e12 for k, v in mm)
    dom_name, dom = max(prof.items(), key=lambda kv: kv[1]["ms"])
    tf = dom["flops"] / (dom["ms"] * 1e-3) / 1e12 if dom["flops"] else 0.0
    return {"gemm_attn_frac_mfma_peak": round(fl / cap, 4) if cap else None,
            "dominant_kernel": dom_name,
            "dominant_launches_per_step": dom["launches"] // steps,
            "dominant_tflops": round(tf, 2),
            "dominant_frac": round(tf / kernel_peak(dom_name), 4)}


def pair_variant(args, config, precision, pairs=None):
    """A pair workload besides the headline, timed the same way (W warm-up
    steps, then K steps between events on the launch stream, inputs resident
    in HBM, outputs left there), then K instrumented steps for the per-kernel
    figures. Reported in `variants`, never as `value`."""
    import torch

    import gsplat_hip as G
    wl = CONFIGS[config]
    B, H, W = pairs or wl["pairs"], wl["img_h"], wl["img_w"]
    cfg = G.default_config(img_h=H, img_w=W, precision=precision)
    m = G.Mastr(cfg, B)
    m.init_seeded(0)
    n = B * 3 * H * W
    img1 = torch.from_numpy(G.seed_uniform(0, "view1", n).reshape(B, 3, H, W)).cuda()
    img2 = torch.from_numpy(G.seed_uniform(0, "view2", n).reshape(B, 3, H, W)).cuda()
    outs = [torch.empty(B, H, W, c, device="cuda") for c in (3, 1, cfg.desc_dim) * 2]
    stream = torch.cuda.current_stream().cuda_stream
    step = lambda: m.pair(img1, img2, B, *outs, stream=stream)
    sec = _event_timed(step, args.steps, args.warmup)
    prof = _profiled(step, args.steps)
    m.close()
    del m, img1, img2, outs
    torch.cuda.empty_cache()
    gflop = (PAIR_GFLOP_384x512 if H * W == 384 * 512 else PAIR_GFLOP_512x512) * B
    peak = PREC_PEAK[precision]
    return {"workload": f"config {config}: {B} pair{'s' if B > 1 else ''} at 3x{H}x{W}, "
                        f"{PREC_NAME[precision]}",
            "value": round(B / sec, 3), "unit": "pairs/s", "ms_per_step": round(sec * 1e3, 3),
            "steps": args.steps, "warmup": args.warmup, "dtype": PREC_DTYPE[precision],
            "wall_tflops": round(gflop / sec / 1e3, 2),
            "wall_frac_of_peak": round(gflop / sec / 1e3 / peak, 4), "peak_tflops": peak,
            **_mfma_summary(prof, args.steps)}


def batch1_variant(args, which):
    """Config 0 (one ViT-L block on 768 tokens, applied in place step after
    step) or config 1 (the ViT-L encoder on one 384x512 image): wall time per
    step and its fraction of the fp32 MFMA peak. These launches are small, so
    more steps are timed (10x K for the block, 2x K for the encoder)."""
    import torch

    import gsplat_hip as G
    cfg = G.default_config()
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    stream = torch.cuda.current_stream().cuda_stream
    if which == "block":
        x = torch.from_numpy(G.seed_normal(0, "tokens", 768 * 1024).reshape(1, 768, 1024)).cuda()
        fn = lambda: m.encoder_block(0, x, 1, stream=stream)
        gflop, steps = BLOCK_GFLOP, 10 * args.steps
        what = "config 0: one ViT-L encoder block, 768 tokens (24x32 grid), batch 1, fp32"
    else:
        img = torch.from_numpy(G.seed_uniform(0, "view1", 3 * 384 * 512).reshape(1, 3, 384, 512)).cuda()
        enc = torch.empty(1, 768, 1024, device="cuda")
        fn = lambda: m.encoder(img, 1, enc, stream=stream)
        gflop, steps = ENCODER_GFLOP, 2 * args.steps
        what = "config 1: ViT-L encoder (patch embed, 24 blocks, enc_norm), one 3x384x512 image, fp32"
    sec = _event_timed(fn, steps, args.warmup)
    prof = _profiled(fn, steps)
    m.close()
    return {"workload": what, "value": round(sec * 1e3, 4), "unit": "ms", "higher_is_better": False,
            "steps": steps, "warmup": args.warmup, "dtype": "f32",
            "wall_tflops": round(gflop / sec / 1e3, 2),
            "wall_frac_of_peak": round(gflop / sec / 1e3 / MFMA_FP32_PEAK_TFLOPS, 4),
            "peak_tflops": MFMA_FP32_PEAK_TFLOPS, **_mfma_summary(prof, steps)}


def fp32x6_variant(args, B, H, W):
    """The headline workload in precision 2 (fp32 GEMMs, convolutions and
    attention on bf16 matrix cores through exact three-term splits), timed
    the same way. Reported beside the fp32 headline, never as `value`."""
    v = pair_variant(args, 3 if H * W == 384 * 512 else 4, 2, pairs=B)
    v["precision_note"] = ("error against an fp64 product at or below the fp32 MFMA kernel's "
                           "(tests/test_gpu_ops.py::test_linear_f32x6_accuracy_vs_fp64); pairs 0 "
                           "and 15 of this workload at the fp32 parity bar against the oracle "
                           "(tests/test_gpu_model.py::test_config3_16_pairs[2])")
    return v


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS))
    ap.add_argument("--pairs", type=int, default=0, help="override the config's pair count")
    ap.add_argument("--graph", action="store_true",
                    help="replay the launch sequence as a hipGraph (the per-kernel roofline "
                         "then comes from one extra eager, profiled step)")
    ap.add_argument("--precision", default="fp32", choices=["fp32", "bf16", "fp32x6"],
                    help="fp32: fp32 MFMA (the headline); bf16: bf16-input / fp32-accumulate "
                         "variant; fp32x6: fp32 GEMMs, convolutions and attention on bf16 "
                         "matrix cores through exact three-term bf16 splits (six term "
                         "products, fp32 accumulate; fp32-level accuracy)")
    ap.add_argument("--bf16", action="store_true", help="same as --precision bf16")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the fp32x6 line reported beside the fp32 headline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--per-shape", action="store_true",
                    help="also print a per-shape kernel table (stderr) from a separate step")
    ap.add_argument("--workload", default="pair",
                    choices=["pair", "frames", "ref512", "checkpoint", "block", "encoder", "cpu",
                             "linear-vs-library", "ref-selftest", "library-bf16"])
    ap.add_argument("--e2e", action="store_true",
                    help="pair workload: include the host->device image copies and the "
                         "device->host output copies (pinned host buffers) in the timed step")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device-to-device copies of MIB MiB (the known-size "
                         "kernel that scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.bf16:
        args.precision = "bf16"

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only. MASt3R pairs are independent, so "
              "N GPUs would each run pairs/N with replicated weights and no collectives; "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import gsplat_hip as G

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": 4 * n, "copies": 3}))
        return
    if args.workload != "pair":
        print(json.dumps(secondary(args)), flush=True)
        return
    wl = CONFIGS[args.config]
    B = args.pairs or wl["pairs"]
    cfg = G.default_config(img_h=wl["img_h"], img_w=wl["img_w"],
                           precision={"fp32": 0, "bf16": 1, "fp32x6": 2}[args.precision])
    H, W = cfg.img_h, cfg.img_w

    m = G.Mastr(cfg, B)
    m.init_seeded(0)
    n = B * 3 * H * W
    img1 = torch.from_numpy(G.seed_uniform(0, "view1", n).reshape(B, 3, H, W)).cuda()
    img2 = torch.from_numpy(G.seed_uniform(0, "view2", n).reshape(B, 3, H, W)).cuda()
    outs = [torch.empty(B, H, W, c, device="cuda") for c in (3, 1, cfg.desc_dim) * 2]
    side = torch.cuda.Stream() if args.graph else None  # graph capture needs a non-null stream
    if side is not None:
        torch.cuda.set_stream(side)
        m.set_graph(True)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        m.pair(img1, img2, B, *outs, stream=stream)

    if args.e2e:  # pinned host images in, pinned host outputs back, every step
        h_img = [img1.cpu().pin_memory(), img2.cpu().pin_memory()]
        h_out = [torch.empty(o.shape, pin_memory=True) for o in outs]

        def step():  # noqa: F811
            img1.copy_(h_img[0], non_blocking=True)
            img2.copy_(h_img[1], non_blocking=True)
            m.pair(img1, img2, B, *outs, stream=stream)
            for h, d in zip(h_out, outs):
                h.copy_(d, non_blocking=True)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # The value: exactly K steps with nothing but the path on the stream.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    ms_per_step = ms / args.steps
    value = B * args.steps / (ms / 1000.0)
    # The per-kernel table and the roofline: a second timed pass of the same K
    # steps with the library's HIP event pair around every launch, on the
    # launch stream (the events serialise the dispatches, so this pass runs a
    # little slower; its time per step is reported beside the value). Graph
    # replay has no per-launch events: one eager step is timed instead.
    ms_instr = None
    if args.graph:
        G.profile_begin()  # graph replay runs eagerly while profiling
        step()
        torch.cuda.synchronize()
        prof = G.profile_end()
        for v in prof.values():  # scale the one profiled step to K steps
            v["ms"] *= args.steps
            v["flops"] *= args.steps
            v["bytes"] *= args.steps
            v["launches"] *= args.steps
    else:
        G.profile_begin()
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            step()
        end.record()
        torch.cuda.synchronize()
        prof = G.profile_end()
        ms_instr = start.elapsed_time(end)

    # roofline of the dominant kernel (largest summed event time)
    dom_name, dom = max(prof.items(), key=lambda kv: kv[1]["ms"])
    avg_ms = dom["ms"] / dom["launches"]
    peak = kernel_peak(dom_name)
    if dom["flops"] > 0 and dom_name.startswith(("gemm", "attn")):
        achieved = dom["flops"] / dom["launches"] / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None}
    else:
        achieved = dom["bytes"] / dom["launches"] / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None}
    # HBM traffic per launch of this kernel, from the committed rocprofv3 PMC
    # summary of the same workload (null when the workload has none)
    try:
        tr = json.load(open(os.path.join(ROOT, "profiles", "pmc_traffic.json")))["workloads"]
        key = f"config{args.config}-{'graph' if args.graph else 'eager'}-" \
              f"{ {'fp32': 'f32', 'bf16': 'bf16', 'fp32x6': 'f32x6'}[args.precision]}-{B}"
        t = tr.get(key, {}).get(dom_name)
        if t:
            roof["traffic"] = (t["fetch_kib"] + t["write_kib"]) * 1024
            roof["traffic_source"] = f"profiles/pmc_traffic.json [{key}]"
    except (OSError, ValueError, KeyError):
        pass
    roof["kernel"] = dom_name
    roof["launches_per_step"] = dom["launches"] // args.steps
    roof["avg_launch_ms"] = round(avg_ms, 4)
    mm = [(k, v) for k, v in prof.items() if k.startswith(("gemm", "attn"))]
    mfma_fl = sum(v["flops"] for k, v in mm)
    mfma_cap = sum(v["ms"] * 1e-3 * kernel_peak(k) * 1e12 for k, v in mm)
    kernels = {k: {"launches": v["launches"] // args.steps, "ms_per_step": round(v["ms"] / args.steps, 3),
                   "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2) if v["flops"] else None,
                   "gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1) if v["bytes"] else None}
               for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}

    out = {
        "metric": "MASt3R image pairs/sec @512x384 fp32 on 1 MI355X; GEMM/attn % MFMA peak",
        "value": round(value, 3),
        "unit": "pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp32": "f32", "bf16": "bf16-in/f32-acc",
                  "fp32x6": "f32 (bf16x6 split products, f32 acc)"}[args.precision],
        "data": "synthetic (seeded U(-1,1) images, seeded N(0,0.02) weights)",
        "config": {"workload": f"config {args.config}: {B} image pairs at 3x{H}x{W}, full "
                               f"MASt3R two-view inference (ViT-L encoder x2 views, ViT-B "
                               f"decoder, 2 DPT heads, 2 local-feature heads)",
                   "pairs_per_step": B, "img": [3, H, W], "parallelism": "single GPU",
                   "launch": "hipGraph replay" if args.graph else "eager stream",
                   "timed": "H2D images + pair + D2H outputs (PCIe-inclusive, not the "
                            "headline)" if args.e2e else "device-resident inputs and outputs"},
        "gemm_attn_frac_mfma_peak": round(mfma_fl / mfma_cap, 4),
        "kernel_share_of_step": round(sum(v["ms"] for v in prof.values()) / (ms_instr or ms), 4),
        "instrumented_ms_per_step": round(ms_instr / args.steps, 3) if ms_instr else None,
        "roofline": roof,
        "kernels": kernels,
    }
    if args.per_shape:
        G.profile_begin(per_shape=True)
        step()
        torch.cuda.synchronize()
        shp = G.profile_end()
        for k, v in sorted(shp.items(), key=lambda kv: -kv[1]["ms"]):
            tf = v["flops"] / (v["ms"] * 1e-3) / 1e12 if v["flops"] else 0.0
            print(f"{v['ms']:9.3f} ms {v['launches']:4d}x {tf:7.1f} TF/s  {k}", file=sys.stderr)
    m.close()
    del m, img1, img2, outs
    torch.cuda.empty_cache()
    if args.precision == "fp32" and not (args.graph or args.e2e or args.no_variants):
        # the other configurations of the baseline, each timed the same way
        # in this run: the fp32x6 form of this workload, config 4 in the
        # bf16 variant at its own size, and the batch-1 configs 0 / 1 / 2
        out["variants"] = {
            "fp32x6": fp32x6_variant(args, B, H, W),
            "config4_bf16": pair_variant(args, 4, 1),
            "config2_fp32": pair_variant(args, 2, 0),
            "config1_fp32": batch1_variant(args, "encoder"),
            "config0_fp32": batch1_variant(args, "block"),
        }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
