"""Reading .safetensors checkpoints into float32 arrays, as rembed's loader
does (internal/safetensors/safetensors.go:122-231), for `Model`.

Layout: an 8-byte little-endian header length, a JSON header mapping each
tensor name to {dtype, shape, data_offsets}, then the data block; offsets
are relative to the data block. F32, F16 and BF16 tensors are widened to
float32 (BF16 is float32's top 16 bits; F16 widens exactly, subnormals,
infinities and NaN included). The I64 `position_ids` buffer BERT checkpoints
carry is skipped; any other dtype is an error, as are a short file, a header
past the end of the file, a bad JSON header, offsets outside the data block
and a shape whose element count does not match its byte range. The data
block is memory-mapped, not read whole.
"""
import json
import os

import numpy as np


class CheckpointError(ValueError):
    """A malformed or unsupported .safetensors file."""


_ELEM = {"F32": 4, "F16": 2, "BF16": 2}


def _widen(dtype, raw):
    if dtype == "F32":
        return raw.view("<f4").astype(np.float32)
    if dtype == "F16":
        return raw.view("<f2").astype(np.float32)
    return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)


def load(path):
    """{name: float32 ndarray of the tensor's shape} (safetensors.go:122-181)."""
    size = os.path.getsize(path)
    if size < 8:
        raise CheckpointError(f"safetensors {path}: file too short for header length")
    with open(path, "rb") as f:
        header_len = int.from_bytes(f.read(8), "little")
        if header_len > size - 8:
            raise CheckpointError(f"safetensors {path}: header length {header_len} exceeds "
                                  f"file size {size}")
        try:
            header = json.loads(f.read(header_len))
        except ValueError as e:
            raise CheckpointError(f"safetensors {path}: bad JSON header: {e}") from None
    if not isinstance(header, dict):
        raise CheckpointError(f"safetensors {path}: bad JSON header: not an object")
    data_len = size - 8 - header_len
    data = (np.memmap(path, np.uint8, "r", offset=8 + header_len, shape=(data_len,))
            if data_len else np.zeros(0, np.uint8))
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(e, dict):
            raise CheckpointError(f"safetensors {path}: bad entry {name!r}")
        dtype = e.get("dtype")
        if dtype not in _ELEM:
            if name.endswith("position_ids"):
                continue
            raise CheckpointError(f"safetensors {path}: tensor {name!r} has dtype {dtype}; "
                                  "supported: F32, F16, BF16")
        try:
            start, end = (int(x) for x in e["data_offsets"])
            shape = [int(d) for d in e["shape"]]
        except (KeyError, TypeError, ValueError):
            raise CheckpointError(f"safetensors {path}: bad entry {name!r}") from None
        if start < 0 or start > end or end > data_len:
            raise CheckpointError(f"safetensors {path}: tensor {name!r} offsets [{start},{end}) "
                                  f"out of range (data size {data_len})")
        if any(d < 0 for d in shape):
            raise CheckpointError(f"safetensors {path}: tensor {name!r} has negative dimension")
        n = int(np.prod(shape, dtype=np.int64))
        if n * _ELEM[dtype] != end - start:
            raise CheckpointError(f"safetensors {path}: tensor {name!r} shape {shape} ({n} elems "
                                  f"x {_ELEM[dtype]} B) does not match byte range {end - start}")
        out[name] = _widen(dtype, np.asarray(data[start:end])).reshape(shape)
    return out
