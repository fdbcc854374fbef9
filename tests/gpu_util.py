"""Helpers for the GPU parity tests (device tensors via torch, checks vs the
oracle)."""
import sys

import numpy as np
import torch

DEV = "cuda"

# fp32 path tolerance of the north star: 1e-3 relative / 1e-4 absolute.
RTOL, ATOL = 1e-3, 1e-4


def case(msg):
    """Name the case before any GPU step, flushed, so a fault names it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


# Device tensors handed to the C ABI as raw pointers must outlive the kernels
# that read them: keep every tensor made here until the test ends (cleared by
# an autouse fixture in conftest.py).
KEEP = []


def dev(a):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)
    KEEP.append(t)
    return t


def empty(*shape):
    t = torch.empty(shape, device=DEV, dtype=torch.float32)
    KEEP.append(t)
    return t


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def assert_close(got, ref, rtol=RTOL, atol=ATOL, name=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{bad.size} elements outside rtol={rtol} atol={atol}; "
            f"worst at {i}: got {got[i]!r} ref {ref[i]!r}; max abs err {err.max():.3e}")
    return float(err.max())


# bf16-input / fp32-accumulate variant: 2e-2 relative (north star), stated
# norm-wise over the tensor, with the worst element bounded by 2e-2 of the
# tensor's largest magnitude.
BF16_RTOL = 2e-2


def assert_close_bf16(got, ref, rtol=BF16_RTOL, name=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    worst = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert rel <= rtol and worst <= rtol, f"{name}: norm-wise rel err {rel:.3e}, worst/max {worst:.3e}"
    # element-wise view (reported, not asserted): the 99.9th percentile of
    # |got - ref| / |ref| over elements with |ref| >= 1e-2 of the tensor maximum
    big = np.abs(ref) >= 1e-2 * np.abs(ref).max()
    p999 = float(np.percentile(np.abs(got - ref)[big] / np.abs(ref)[big], 99.9)) if big.any() else 0.0
    return rel, worst, p999
