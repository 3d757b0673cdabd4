"""Reading .safetensors checkpoints into float32 arrays, as rembed's loader
does (internal/safetensors/safetensors.go:54-231, reader.go:33-73), for
`Model`.

One file: an 8-byte little-endian header length, a JSON header mapping each
tensor name to {dtype, shape, data_offsets}, then the data block; offsets
are relative to the data block. F32, F16 and BF16 tensors are widened to
float32 (BF16 is float32's top 16 bits; F16 widens exactly, subnormals,
infinities and NaN included). The I64 `position_ids` buffer BERT checkpoints
carry is skipped. Refused: any other dtype, a file too small to hold the
header length, a header running past the end of the file, a header that is
not a JSON object, offsets outside the data block, and a shape whose element
count disagrees with its byte range. The data block is memory-mapped, not
read whole.

A sharded checkpoint: where `model.safetensors` is absent, the
`model.safetensors.index.json` beside it maps each tensor to a shard file;
each distinct shard (a plain file name, never a path: the index is
downloaded data) is read once, in sorted order, and every tensor the index
names must come from one of them (LoadAny / loadSharded,
safetensors.go:54-121).

EmbeddingGemma's Dense head ships as two more single files,
`2_Dense/model.safetensors` and `3_Dense/model.safetensors`, each holding
one `linear.weight` [out][in] (loadDenseLinear, gemma3.go:144-172);
`load_model_dir` hands them over as "2_Dense.linear.weight" and
"3_Dense.linear.weight".
"""
import json
import os

import numpy as np


class CheckpointError(ValueError):
    """A malformed or unsupported .safetensors file."""


_ELEM = {"F32": 4, "F16": 2, "BF16": 2}
INDEX_NAME = "model.safetensors.index.json"


def _widen(dtype, raw):
    if dtype == "F32":
        return raw.view("<f4").astype(np.float32)
    if dtype == "F16":
        return raw.view("<f2").astype(np.float32)
    return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)


def load(path):
    """{name: float32 ndarray of the tensor's shape} from one file
    (safetensors.go:122-181)."""
    size = os.path.getsize(path)
    if size < 8:
        raise CheckpointError(f"{path}: {size} bytes, fewer than the 8-byte header length")
    with open(path, "rb") as f:
        header_len = int.from_bytes(f.read(8), "little")
        if header_len > size - 8:
            raise CheckpointError(f"{path}: the header claims {header_len} bytes but only "
                                  f"{size - 8} follow the length field")
        try:
            header = json.loads(f.read(header_len))
        except ValueError as e:
            raise CheckpointError(f"{path}: the header is not valid JSON ({e})") from None
    if not isinstance(header, dict):
        raise CheckpointError(f"{path}: the header is not a JSON object")
    data_len = size - 8 - header_len
    data = (np.memmap(path, np.uint8, "r", offset=8 + header_len, shape=(data_len,))
            if data_len else np.zeros(0, np.uint8))
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(e, dict):
            raise CheckpointError(f"{path}: header entry {name!r} is not an object")
        dtype = e.get("dtype")
        if dtype not in _ELEM:
            if name.endswith("position_ids"):
                continue
            raise CheckpointError(f"{path}: {name!r} is stored as {dtype}, which is not one of "
                                  "F32, F16, BF16")
        try:
            start, end = (int(x) for x in e["data_offsets"])
            shape = [int(d) for d in e["shape"]]
        except (KeyError, TypeError, ValueError):
            raise CheckpointError(f"{path}: header entry {name!r} lacks a valid shape or "
                                  "data_offsets") from None
        if start < 0 or start > end or end > data_len:
            raise CheckpointError(f"{path}: {name!r} spans bytes [{start},{end}) outside the "
                                  f"{data_len}-byte data block")
        if any(d < 0 for d in shape):
            raise CheckpointError(f"{path}: {name!r} has a negative dimension in {shape}")
        n = int(np.prod(shape, dtype=np.int64))
        if n * _ELEM[dtype] != end - start:
            raise CheckpointError(f"{path}: {name!r} of shape {shape} needs {n * _ELEM[dtype]} "
                                  f"bytes of {dtype} but spans {end - start}")
        out[name] = _widen(dtype, np.asarray(data[start:end])).reshape(shape)
    return out


def valid_shard_name(name):
    """A bare file name that is safe to join to the model directory
    (ValidShardName, safetensors.go:42-52): the index is downloaded data, so a
    value like "../x" or "a/b" must not become a path."""
    return isinstance(name, str) and name not in ("", ".", "..") and not any(
        c in name for c in "/\\")


def load_sharded(index_path):
    """Every tensor of the shards an index names (loadSharded,
    safetensors.go:73-121)."""
    try:
        with open(index_path) as f:
            index = json.load(f)
    except ValueError as e:
        raise CheckpointError(f"{index_path}: the index is not valid JSON ({e})") from None
    wmap = index.get("weight_map") if isinstance(index, dict) else None
    if not isinstance(wmap, dict) or not wmap:
        raise CheckpointError(f"{index_path}: the index has no weight_map entries")
    for shard in wmap.values():
        if not valid_shard_name(shard):
            raise CheckpointError(f"{index_path}: shard name {shard!r} is not a plain file name")
    base = os.path.dirname(index_path)
    out = {}
    for shard in sorted(set(wmap.values())):
        out.update(load(os.path.join(base, shard)))
    for name in wmap:
        if name not in out:
            raise CheckpointError(f"{index_path}: {name!r} is mapped to a shard that does not "
                                  "hold it")
    return out


def load_any(path):
    """`path` (a model.safetensors) if it exists, else the sharded set its
    directory's index names (LoadAny, safetensors.go:54-71)."""
    if os.path.exists(path):
        return load(path)
    index = os.path.join(os.path.dirname(path), INDEX_NAME)
    if not os.path.exists(index):
        raise CheckpointError(f"{path} does not exist and no {INDEX_NAME} is beside it")
    return load_sharded(index)


def load_model_dir(directory, dense_hidden=0, hidden=0):
    """A model directory's tensors: model.safetensors or its shards, plus,
    when `dense_hidden` > 0, EmbeddingGemma's Dense head from 2_Dense/ and
    3_Dense/ (each one `linear.weight`, [dense_hidden][hidden] and
    [hidden][dense_hidden]; gemma3.go:144-172)."""
    t = load_any(os.path.join(directory, "model.safetensors"))
    if dense_hidden > 0:
        for sub, shape in (("2_Dense", (dense_hidden, hidden)), ("3_Dense", (hidden, dense_hidden))):
            path = os.path.join(directory, sub, "model.safetensors")
            if not os.path.exists(path):
                raise CheckpointError(f"{path} does not exist: this model needs its Dense head")
            w = load(path).get("linear.weight")
            if w is None:
                raise CheckpointError(f"{path}: no linear.weight")
            if tuple(w.shape) != shape:
                raise CheckpointError(f"{path}: linear.weight is {list(w.shape)}, expected "
                                      f"{list(shape)}")
            t[f"{sub}.linear.weight"] = w
    return t
