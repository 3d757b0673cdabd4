"""The .safetensors reader against files written by the `safetensors`
package (an independent writer), and its refusals, after
internal/safetensors/safetensors.go:122-231 and its tests."""
import json
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

import safetensors_files as SF
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
    ("short", "fewer than the 8-byte header length"),
    ("hlen", "the header claims"),
    ("json", "not valid JSON"),
    ("dtype", "stored as I32"),
    ("offsets", "outside the 4-byte data block"),
    ("shape", "needs 12 bytes of F32 but spans 8"),
    ("negative", "negative dimension"),
    ("entry", "lacks a valid shape"),
    ("array", "not a JSON object"),
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
    elif case == "negative":
        path = _file(tmp_path, {"w": {"dtype": "F32", "shape": [-1, -2], "data_offsets": [0, 8]}},
                     b"\0" * 8)
    elif case == "entry":
        path = _file(tmp_path, {"w": {"dtype": "F32", "shape": [2]}}, b"\0" * 8)
    else:
        path = _file(tmp_path, [1, 2])
    with pytest.raises(C.CheckpointError, match=match):
        C.load(path)


def test_metadata_and_empty_tensor(tmp_path):
    path = _file(tmp_path, {"__metadata__": {"format": "pt"},
                            "e": {"dtype": "F32", "shape": [0, 4], "data_offsets": [0, 0]}})
    t = C.load(path)
    assert list(t) == ["e"] and t["e"].shape == (0, 4)


def test_half_widening_known_answers(tmp_path):
    """Hand-checked bit patterns (internal/safetensors/safetensors_test.go:89-118):
    F16 1, -2, 0x3555, the smallest subnormal 2^-24, 0; BF16 1, -3, 0x3EAB."""
    f16 = bytes([0x00, 0x3C, 0x00, 0xC0, 0x55, 0x35, 0x01, 0x00, 0x00, 0x00])
    t = C.load(_file(tmp_path, {"w": {"dtype": "F16", "shape": [5], "data_offsets": [0, 10]}},
                     f16))
    assert t["w"].tolist() == [1.0, -2.0, 0.333251953125, 2.0 ** -24, 0.0]
    bf = bytes([0x80, 0x3F, 0x40, 0xC0, 0xAB, 0x3E])
    t = C.load(_file(tmp_path, {"w": {"dtype": "BF16", "shape": [3], "data_offsets": [0, 6]}},
                     bf))
    assert t["w"].tolist() == [1.0, -3.0, 0.333984375]


@pytest.mark.parametrize("dtype", SF.DTYPES)
def test_round_trip_per_dtype(tmp_path, dtype):
    rng = np.random.default_rng(7)
    x = {"a": rng.standard_normal((17, 9), dtype=np.float32),
         "b": (rng.standard_normal(33, dtype=np.float32) * 1e-3)}
    p = tmp_path / "m.safetensors"
    SF.write_file(p, x, dtype)
    t = C.load(str(p))
    for n, a in x.items():
        want = SF.represented(a, dtype)
        assert t[n].shape == a.shape
        assert np.array_equal(t[n].view(np.uint32), want.view(np.uint32)), n
    if dtype != "F32":
        assert not np.array_equal(t["a"], x["a"])  # really rounded


def _shards(tmp_path, wmap, files):
    for fname, tensors in files.items():
        SF.write_file(tmp_path / fname, tensors, "F32")
    (tmp_path / C.INDEX_NAME).write_text(json.dumps({"weight_map": wmap}))
    return str(tmp_path / "model.safetensors")


def test_load_any_sharded(tmp_path):
    """internal/safetensors/sharded_test.go:35-73: no model.safetensors, an
    index naming two shards; both tensors come back."""
    s1, s2 = "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"
    path = _shards(tmp_path, {"a": s1, "b": s2},
                   {s1: {"a": np.array([1, 2, 3], np.float32)},
                    s2: {"b": np.array([4, 5], np.float32)}})
    t = C.load_any(path)
    assert sorted(t) == ["a", "b"]
    assert t["a"].tolist() == [1, 2, 3] and t["b"].tolist() == [4, 5]
    # a single file beside an index wins (safetensors.go:61-63)
    SF.write_file(tmp_path / "model.safetensors", {"c": np.ones(2, np.float32)}, "F32")
    assert list(C.load_any(path)) == ["c"]


@pytest.mark.parametrize("bad", ["../evil.safetensors", "/etc/passwd", "sub/dir.safetensors",
                                 "..", ".", "", "a\\b.safetensors"])
def test_shard_names_that_are_paths_are_refused(tmp_path, bad):
    """sharded_test.go:76-98: the index is downloaded data."""
    assert not C.valid_shard_name(bad)
    (tmp_path / C.INDEX_NAME).write_text(json.dumps({"weight_map": {"a": bad}}))
    with pytest.raises(C.CheckpointError, match="not a plain file name"):
        C.load_any(str(tmp_path / "model.safetensors"))


def test_valid_shard_name():
    assert C.valid_shard_name("model-00001-of-00002.safetensors")
    assert not C.valid_shard_name(None)


@pytest.mark.parametrize("case,match", [
    ("absent", "no model.safetensors.index.json is beside it"),
    ("empty", "no weight_map entries"),
    ("json", "the index is not valid JSON"),
    ("missing", "mapped to a shard that does not hold it"),
])
def test_sharded_refusals(tmp_path, case, match):
    path = str(tmp_path / "model.safetensors")
    s1 = "model-00001-of-00001.safetensors"
    if case == "empty":
        _shards(tmp_path, {}, {})
    elif case == "json":
        (tmp_path / C.INDEX_NAME).write_text("{weight_map")
    elif case == "missing":
        _shards(tmp_path, {"a": s1, "b": s1}, {s1: {"a": np.zeros(2, np.float32)}})
    with pytest.raises(C.CheckpointError, match=match):
        C.load_any(path)


def test_model_dir_with_dense_head(tmp_path):
    """gemma3.go:144-172: 2_Dense / 3_Dense each hold one [out][in]
    linear.weight; they arrive as 2_Dense.linear.weight / 3_Dense.linear.weight."""
    rng = np.random.default_rng(3)
    H, D = 8, 12
    t = {"embed_tokens.weight": rng.standard_normal((5, H), dtype=np.float32),
         "2_Dense.linear.weight": rng.standard_normal((D, H), dtype=np.float32),
         "3_Dense.linear.weight": rng.standard_normal((H, D), dtype=np.float32)}
    SF.write_model_dir(str(tmp_path), t, "BF16", shards=2, prefix="model.")
    got = C.load_model_dir(str(tmp_path), D, H)
    assert sorted(got) == ["2_Dense.linear.weight", "3_Dense.linear.weight",
                           "model.embed_tokens.weight"]
    for n, a in t.items():
        key = n if "Dense" in n else "model." + n
        assert np.array_equal(got[key], SF.represented(a, "BF16"))
    # no Dense head asked for: the backbone only
    assert list(C.load_model_dir(str(tmp_path))) == ["model.embed_tokens.weight"]
    with pytest.raises(C.CheckpointError, match=r"linear.weight is \[12, 8\], expected \[12, 9\]"):
        C.load_model_dir(str(tmp_path), D, H + 1)
    SF.write_file(tmp_path / "3_Dense" / "model.safetensors", {"weight": np.ones(2, np.float32)},
                  "F32")
    with pytest.raises(C.CheckpointError, match="no linear.weight"):
        C.load_model_dir(str(tmp_path), D, H)


def test_model_dir_without_dense_files_is_refused(tmp_path):
    """EmbeddingGemma requires its Dense head (gemma3.go:144-151)."""
    SF.write_model_dir(str(tmp_path), {"embed_tokens.weight": np.ones((2, 4), np.float32)}, "F32")
    with pytest.raises(C.CheckpointError, match="2_Dense.*needs its Dense head"):
        C.load_model_dir(str(tmp_path), 6, 4)
