"""The .safetensors reader against files written by the `safetensors`
package (an independent writer), and its refusals, after
internal/safetensors/safetensors.go:122-231 and its tests."""
import json
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

from rembed_amd import checkpoint as C


def test_f32_f16_bf16_widen_and_position_ids_skipped(tmp_path):
    rng = np.random.default_rng(1)
    w32 = rng.standard_normal((5, 7), dtype=np.float32)
    # float16 specials: subnormal, max, -0, inf, nan
    w16 = np.array([[1.5, -2.25, 6e-8, 65504.0], [-0.0, np.inf, -np.inf, np.nan]], np.float16)
    bf_vals = rng.standard_normal(9, dtype=np.float32)
    bf_bits = (bf_vals.view(np.uint32) >> 16).astype(np.uint16)
    path = tmp_path / "m.safetensors"
    save_file({"a.weight": w32, "b.weight": w16,
               "embeddings.position_ids": np.arange(4, dtype=np.int64)[None, :]}, str(path))
    # the numpy writer has no bfloat16 type: append a BF16 entry by hand
    raw = path.read_bytes()
    hlen = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + hlen])
    data = raw[8 + hlen:]
    header["c.weight"] = {"dtype": "BF16", "shape": [3, 3],
                          "data_offsets": [len(data), len(data) + 18]}
    hb = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(hb)) + hb + data + bf_bits.tobytes())

    t = C.load(str(path))
    assert set(t) == {"a.weight", "b.weight", "c.weight"}
    assert t["a.weight"].dtype == np.float32 and np.array_equal(t["a.weight"], w32)
    want16 = w16.astype(np.float32)
    got16 = t["b.weight"]
    assert got16.shape == (2, 4)
    assert np.array_equal(got16.view(np.uint32)[~np.isnan(want16)],
                          want16.view(np.uint32)[~np.isnan(want16)])
    assert np.isnan(got16[1, 3])
    assert got16[0, 2] > 0 and np.float32(got16[0, 2]) == np.float32(np.float16(6e-8))
    assert np.array_equal(t["c.weight"].ravel().view(np.uint32),
                          bf_bits.astype(np.uint32) << 16)


def _file(tmp_path, header, data=b"", hlen=None):
    hb = json.dumps(header).encode() if not isinstance(header, bytes) else header
    p = tmp_path / "x.safetensors"
    p.write_bytes(struct.pack("<Q", len(hb) if hlen is None else hlen) + hb + data)
    return str(p)


@pytest.mark.parametrize("case,match", [
    ("short", "too short"),
    ("hlen", "exceeds file size"),
    ("json", "bad JSON header"),
    ("dtype", "has dtype I32"),
    ("offsets", "out of range"),
    ("shape", "does not match byte range"),
    ("negative", "negative dimension"),
])
def test_refusals(tmp_path, case, match):
    if case == "short":
        p = tmp_path / "s.safetensors"
        p.write_bytes(b"\x01\x02")
        path = str(p)
    elif case == "hlen":
        path = _file(tmp_path, {}, hlen=1 << 20)
    elif case == "json":
        path = _file(tmp_path, b"{not json")
    elif case == "dtype":
        path = _file(tmp_path, {"w": {"dtype": "I32", "shape": [1], "data_offsets": [0, 4]}},
                     b"\0" * 4)
    elif case == "offsets":
        path = _file(tmp_path, {"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}},
                     b"\0" * 4)
    elif case == "shape":
        path = _file(tmp_path, {"w": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}},
                     b"\0" * 8)
    else:
        path = _file(tmp_path, {"w": {"dtype": "F32", "shape": [-1, -2], "data_offsets": [0, 8]}},
                     b"\0" * 8)
    with pytest.raises(C.CheckpointError, match=match):
        C.load(path)


def test_metadata_and_empty_tensor(tmp_path):
    path = _file(tmp_path, {"__metadata__": {"format": "pt"},
                            "e": {"dtype": "F32", "shape": [0, 4], "data_offsets": [0, 0]}})
    t = C.load(path)
    assert list(t) == ["e"] and t["e"].shape == (0, 4)
