"""gs_hip_collect_points_noalloc (scratch in a static device array, no
allocation at call time) against gs_hip_collect_points (stream-ordered
scratch) through the C ABI: bit-identical points, confidences and counts on two
calls in a row, the first at the maximum size (every block slot of the static
array in use), the second smaller (the array still holds the first call's
block counts); sizes past the maximum are refused before any launch."""
import numpy as np
import pytest
import torch

import gsplat_hip as G
from gpu_util import KEEP, case, stream

pytestmark = pytest.mark.gpu

NOALLOC_MAX = 1 << 27


def _run(fn, pts, conf, thr, cap):
    count = torch.zeros(1, dtype=torch.int64, device="cuda")
    op = torch.full((cap, 3), -7.0, device="cuda")
    oc = torch.full((cap,), -7.0, device="cuda")
    KEEP.extend([count, op, oc])
    G.check(fn(G.ptr(pts), G.ptr(conf), conf.numel(), thr, G.ptr(op), G.ptr(oc), cap,
               G.ptr(count), stream()))
    return count, op, oc


def test_noalloc_matches_allocating_entry_point_twice():
    L = G.lib()
    gen = torch.Generator(device="cuda")
    for n, thr, seed in ((NOALLOC_MAX, 0.75, 1), (1_000_003, 0.3, 2)):
        case(f"collect_points noalloc vs allocating n={n} thr={thr}")
        gen.manual_seed(seed)
        conf = torch.rand(n, device="cuda", generator=gen)
        pts = torch.randn(n, 3, device="cuda", generator=gen)
        KEEP.extend([conf, pts])
        cap = n // 2
        want = _run(L.gs_hip_collect_points, pts, conf, thr, cap)
        got = _run(L.gs_hip_collect_points_noalloc, pts, conf, thr, cap)
        torch.cuda.synchronize()
        k = int(want[0].item())
        assert int(got[0].item()) == k and k > 0
        assert torch.equal(got[1], want[1]) and torch.equal(got[2], want[2])
        if n < NOALLOC_MAX:  # the small case is also checked against a host mask
            sel = (conf > thr).cpu().numpy()
            np.testing.assert_array_equal(got[2][:min(k, cap)].cpu().numpy(),
                                          conf.cpu().numpy()[sel][:cap])
        del conf, pts
        KEEP.clear()
        torch.cuda.empty_cache()


def test_noalloc_refuses_sizes_past_its_array():
    case("collect_points noalloc size check")
    L = G.lib()
    x = torch.zeros(4, device="cuda")
    KEEP.append(x)
    rc = L.gs_hip_collect_points_noalloc(G.ptr(x), G.ptr(x), NOALLOC_MAX + 1, 0.5, G.ptr(x),
                                         G.ptr(x), 0, G.ptr(x), stream())
    assert rc == -1 and b"2^27" in L.gs_hip_last_error()
    rc = L.gs_hip_collect_points_noalloc(G.ptr(x), G.ptr(x), -1, 0.5, G.ptr(x), G.ptr(x), 0,
                                         G.ptr(x), stream())
    assert rc == -1
    # n == 0 touches nothing and leaves the count as it was
    count = torch.full((1,), 5, dtype=torch.int64, device="cuda")
    KEEP.append(count)
    G.check(L.gs_hip_collect_points_noalloc(G.ptr(x), G.ptr(x), 0, 0.5, None, None, 0,
                                            G.ptr(count), stream()))
    assert int(count.item()) == 5
