"""Shared test configuration.

`-m "not gpu"` runs the oracle checks, the host logic and the C-ABI symbol
checks on the CPU; `-m gpu` runs the parity tests of the HIP path against the
oracle on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("crystal-gausplat_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


# A reduced MASt3R configuration with every structural element of the real one
# (two 64-wide heads per attention, both decoder chains, all four DPT hooks,
# both ConvTranspose stages, the stride-2 conv, descriptors) at sizes the oracle
# finishes in well under a second.
TINY = dict(img_h=64, img_w=96, patch=16, enc_dim=128, enc_depth=2, enc_heads=2,
            enc_mlp=256, dec_dim=128, dec_depth=3, dec_heads=2, dec_mlp=256,
            dpt_feat=64, dpt_dims=[32, 64, 96, 128], dpt_hooks=[0, 1, 2, 3],
            head_mid=32, lf_hidden=256, desc_dim=24, ln_eps=1e-6, rope_base=100.0,
            linear_layout=0, rope_mode=1)


@pytest.fixture(autouse=True)
def _release_device_tensors():
    yield
    mod = sys.modules.get("gpu_util")
    if mod is not None:
        import torch
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        mod.KEEP.clear()


@pytest.fixture(scope="session")
def tiny_cfg():
    return dict(TINY)
