"""Checkpoint ingestion on the device: gs_hip_mastr_load_safetensors
(WeightLoader, src/mastr/weight_loader.cr:43-123, over SafetensorsLoader,
src/mastr/weights.cr:30-290). The seeded weights are written to a
safetensors file by the `safetensors` package; loading it must reproduce the
seeded context bit for bit (F32), and a BF16 checkpoint must match the oracle
run on the same bf16-rounded weights."""
import numpy as np
import pytest
import torch

import gsplat_hip as G
import pyoracle as O
from gpu_util import assert_close, case
from test_gpu_model import check_pair, run_pair, weights_for

pytestmark = pytest.mark.gpu


def _images(cfg, B, seed=0):
    n = B * 3 * cfg.img_h * cfg.img_w
    return (G.seed_uniform(seed, "view1", n).reshape(B, 3, cfg.img_h, cfg.img_w),
            G.seed_uniform(seed, "view2", n).reshape(B, 3, cfg.img_h, cfg.img_w))


def test_f32_checkpoint_equals_seeded(tiny_cfg, tmp_path):
    from safetensors.numpy import save_file
    case("checkpoint f32 round trip")
    cfg = G.default_config(**tiny_cfg)
    w = weights_for(cfg, 0, bias_std=0.02, ln_std=0.1)
    extra = {"mask_token": np.zeros((1, 1, cfg.enc_dim), np.float32),
             "downstream_head1.extra.weight": np.ones((4,), np.float32)}
    p = str(tmp_path / "tiny.safetensors")
    save_file({**w, **extra}, p, metadata={"format": "pt"})
    B = 2
    i1, i2 = _images(cfg, B)
    a = G.Mastr(cfg, B)
    a.init_seeded(0, 0.02, 0.1)
    ref = run_pair(a, cfg, i1, i2, B)
    a.close()
    b = G.Mastr(cfg, B)
    counts = b.load_safetensors(p)
    assert counts == dict(loaded=len(w), unexpected=len(extra), missing=0)
    got = run_pair(b, cfg, i1, i2, B)
    for k in ref:
        np.testing.assert_array_equal(got[k], ref[k], err_msg=k)
    b.close()


def test_bf16_checkpoint_vs_oracle(tiny_cfg, tmp_path):
    from safetensors.torch import save_file
    case("checkpoint bf16 vs oracle")
    cfg = G.default_config(**tiny_cfg)
    w = weights_for(cfg, 3, bias_std=0.02, ln_std=0.1)
    wb = {n: torch.from_numpy(a).to(torch.bfloat16) for n, a in w.items()}
    p = str(tmp_path / "tiny_bf16.safetensors")
    save_file(wb, p)
    w_rounded = {n: t.float().numpy() for n, t in wb.items()}
    B = 1
    i1, i2 = _images(cfg, B, seed=5)
    m = G.Mastr(cfg, B)
    assert m.load_safetensors(p)["loaded"] == len(w)
    got = run_pair(m, cfg, i1, i2, B)
    check_pair(got, O.mastr_pair(cfg.as_dict(), w_rounded, i1, i2), "bf16 ckpt")
    m.close()


def test_partial_checkpoint_and_shape_error(tiny_cfg, tmp_path):
    from safetensors.numpy import save_file
    case("checkpoint partial / shape mismatch")
    cfg = G.default_config(**tiny_cfg)
    w = weights_for(cfg, 0)
    part = {n: a for n, a in w.items() if n.startswith("enc_blocks.0.")}
    p = str(tmp_path / "part.safetensors")
    save_file(part, p)
    m = G.Mastr(cfg, 1)
    m.init_seeded(0)
    assert m.load_safetensors(p) == dict(loaded=len(part), unexpected=0,
                                         missing=len(w) - len(part))
    bad = {"enc_blocks.0.mlp.fc1.weight": np.ascontiguousarray(
        w["enc_blocks.0.mlp.fc1.weight"].T)}
    q = str(tmp_path / "bad.safetensors")
    save_file(bad, q)
    with pytest.raises(G.GsError, match="shape of enc_blocks.0.mlp.fc1.weight"):
        m.load_safetensors(q)
    m.close()
