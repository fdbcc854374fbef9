"""The CPU oracle built with address + undefined-behaviour sanitizers
(make -C oracle sanitize) runs every entry point, the two-view pair in both
compositions included, without a report. CPU only."""
import os
import struct
import subprocess

import numpy as np

import gsplat_hip as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")


def test_oracle_under_asan_ubsan(tiny_cfg, tmp_path):
    subprocess.run(["make", "-s", "-C", ORACLE, "sanitize"], check=True)
    cfg = G.default_config(**tiny_cfg)
    w = G.seeded_weights(cfg, 0, 0.02, 0.1)
    path = tmp_path / "weights.bin"
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(w)))
        for name, a in w.items():
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<Q", a.size))
            f.write(np.ascontiguousarray(a, np.float32).tobytes())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    r = subprocess.run([os.path.join(ORACLE, "_san", "check"), str(path)], capture_output=True,
                       text=True, env=env, timeout=600)
    assert r.returncode == 0 and r.stdout.strip() == "OK", (r.returncode, r.stdout, r.stderr[-3000:])
