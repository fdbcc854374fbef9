"""Safetensors checkpoint reader (SafetensorsLoader, src/mastr/weights.cr:30-290).

Files are written by the `safetensors` package itself (numpy and torch
writers), so the reader is checked against the format's own producer; the
dtype conversions are checked against numpy (F16, all 65536 bit patterns) and
torch (BF16). Host-only: no GPU needed.
"""
import json
import os
import struct

import numpy as np
import pytest

import gsplat_hip as G


def _raw_file(path, header, data=b""):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


def test_f32_roundtrip_and_metadata(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    t = {"a.weight": rng.standard_normal((3, 5)).astype(np.float32),
         "b": rng.standard_normal((7,)).astype(np.float32),
         "c.scalar": np.array(2.5, dtype=np.float32),
         "d.empty": np.zeros((0, 4), dtype=np.float32),
         "e\"q\\uote": np.arange(6, dtype=np.float32).reshape(1, 2, 3)}
    p = str(tmp_path / "x.safetensors")
    save_file(t, p, metadata={"format": "pt", "note": "x"})
    idx = {n: (dt, s) for n, dt, s in G.safetensors_index(p)}
    assert set(idx) == set(t)  # __metadata__ skipped
    for n, a in t.items():
        assert idx[n] == ("F32", a.shape)
        got = G.safetensors_read(p, n, a.shape)
        assert got.tobytes() == a.tobytes()


def test_f16_all_bit_patterns(tmp_path):
    from safetensors.numpy import save_file
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    p = str(tmp_path / "h.safetensors")
    save_file({"h": h}, p)
    assert G.safetensors_index(p) == [("h", "F16", (65536,))]
    got = G.safetensors_read(p, "h", (65536,))
    want = h.astype(np.float32)
    nan = np.isnan(want)
    # every non-NaN value exact (zeros, subnormals, normals, infinities, signs)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    # closed forms of the binary16 extremes
    assert got[1] == 2.0 ** -24 and got[0x3FF] == 1023 * 2.0 ** -24
    assert got[0x400] == 2.0 ** -14 and got[0x7BFF] == 65504.0
    assert got[0x8001] == -(2.0 ** -24) and np.signbit(got[0x8000])


def test_bf16_matches_torch(tmp_path):
    import torch
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(64, 33, generator=g) * 10).to(torch.bfloat16)
    x[0, :4] = torch.tensor([0.0, -0.0, float("inf"), 1e-40]).to(torch.bfloat16)
    p = str(tmp_path / "b.safetensors")
    save_file({"w": x}, p)
    assert G.safetensors_index(p) == [("w", "BF16", (64, 33))]
    got = G.safetensors_read(p, "w", (64, 33))
    assert got.tobytes() == x.float().numpy().tobytes()


def test_mixed_dtypes_and_unsupported(tmp_path):
    from safetensors.numpy import save_file
    p = str(tmp_path / "m.safetensors")
    save_file({"f": np.ones((2, 2), np.float32), "i": np.arange(4, dtype=np.int64),
               "u8": np.arange(3, dtype=np.uint8)}, p)
    idx = {n: (dt, s) for n, dt, s in G.safetensors_index(p)}
    assert idx == {"f": ("F32", (2, 2)), "i": ("I64", (4,)), "u8": ("U8", (3,))}
    with pytest.raises(G.GsError, match="unsupported dtype I64"):
        G.safetensors_read(p, "i", (4,))
    with pytest.raises(G.GsError, match="no tensor"):
        G.safetensors_read(p, "nope", (1,))
    with pytest.raises(G.GsError, match="numel mismatch"):
        G.safetensors_read(p, "f", (5,))


@pytest.mark.parametrize("case", ["offsets_past_end", "size_vs_shape", "bad_json",
                                  "header_too_long", "unknown_dtype", "missing_field",
                                  "short_file", "float_offset", "bytes_overflow",
                                  "shape_overflow"])
def test_malformed_files_are_errors(tmp_path, case):
    p = str(tmp_path / "bad.safetensors")
    data = np.arange(4, dtype=np.float32).tobytes()
    if case == "offsets_past_end":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}}, data)
    elif case == "size_vs_shape":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, data)
    elif case == "bad_json":
        h = b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]'
        open(p, "wb").write(struct.pack("<Q", len(h)) + h + data)
    elif case == "header_too_long":
        h = b"{}"
        open(p, "wb").write(struct.pack("<Q", 1 << 40) + h)
    elif case == "unknown_dtype":
        _raw_file(p, {"a": {"dtype": "F7", "shape": [4], "data_offsets": [0, 16]}}, data)
    elif case == "missing_field":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [4]}}, data)
    elif case == "short_file":
        open(p, "wb").write(b"\x02\x00")
    elif case == "bytes_overflow":  # (2^62 + 4) x 4 bytes wraps to 16 in int64
        _raw_file(p, {"a": {"dtype": "F32", "shape": [(1 << 62) + 4], "data_offsets": [0, 16]}},
                  data)
    elif case == "shape_overflow":  # 2^32 x 2^32 x 4 wraps the element count
        _raw_file(p, {"a": {"dtype": "F32", "shape": [1 << 32, 1 << 32, 4],
                            "data_offsets": [0, 16]}}, data)
    elif case == "float_offset":
        h = b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16.0]}}'
        open(p, "wb").write(struct.pack("<Q", len(h)) + h + data)
    assert G.lib().gs_safetensors_count(os.fsencode(p)) == -1
    assert G.lib().gs_hip_last_error().decode().startswith("safetensors:")


def test_missing_file():
    with pytest.raises(G.GsError, match="cannot open"):
        G.safetensors_index("/nonexistent/x.safetensors")


def test_header_padding_and_order(tmp_path):
    """Writers may pad the header with spaces; tensor order is header order."""
    data = np.arange(6, dtype=np.float32).tobytes()
    hdr = {"z": {"dtype": "F32", "shape": [2], "data_offsets": [16, 24]},
           "a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}
    h = json.dumps(hdr).encode()
    h += b" " * (8 - len(h) % 8)
    p = str(tmp_path / "pad.safetensors")
    open(p, "wb").write(struct.pack("<Q", len(h)) + h + data)
    assert [n for n, _, _ in G.safetensors_index(p)] == ["z", "a"]
    assert G.safetensors_read(p, "z", (2,)).tolist() == [4.0, 5.0]
    assert G.safetensors_read(p, "a", (2, 2)).tolist() == [[0, 1], [2, 3]]
