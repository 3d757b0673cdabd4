"""Writing .safetensors checkpoints for the loader tests: F32, F16 or BF16
files, sharded sets with a model.safetensors.index.json, and
sentence-transformers' 2_Dense/ and 3_Dense/ head files.

The writer is this module's own (the `safetensors` package has no bfloat16
for numpy), so `represented()` gives, independently of the reader, the
float32 values a file of each dtype holds: F16 through numpy's IEEE
conversion, BF16 by round-to-nearest-even on float32's top 16 bits.
"""
import json
import os
import struct

import numpy as np

DTYPES = ("F32", "F16", "BF16")


def bf16_bits(a):
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (finite input)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def represented(a, dtype):
    """The float32 values a `dtype` file stores for float32 input `a`."""
    a = np.ascontiguousarray(a, np.float32)
    if dtype == "F32":
        return a.copy()
    if dtype == "F16":
        return a.astype(np.float16).astype(np.float32)
    return (bf16_bits(a).astype(np.uint32) << 16).view(np.float32)


def _encode(a, dtype):
    a = np.ascontiguousarray(a, np.float32)
    if dtype == "F32":
        return a.astype("<f4").tobytes()
    if dtype == "F16":
        return a.astype("<f2").tobytes()
    return bf16_bits(a).astype("<u2").tobytes()


def write_file(path, tensors, dtype, extra=None):
    """One file; tensors' data in insertion order, 8-byte aligned header.
    `extra`: more header entries with raw data, {name: (dtype, shape, bytes)}."""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    items = [(n, dtype, list(np.shape(a)), _encode(a, dtype)) for n, a in tensors.items()]
    items += [(n, dt, list(sh), raw) for n, (dt, sh, raw) in (extra or {}).items()]
    for name, dt, shape, raw in items:
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hb = json.dumps(header).encode()
    hb += b" " * (-len(hb) % 8)
    os.makedirs(os.path.dirname(str(path)) or ".", exist_ok=True)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for raw in blobs:
            f.write(raw)


def write_model_dir(directory, tensors, dtype, shards=1, prefix=""):
    """A model directory as the hub ships it: the backbone as
    model.safetensors (shards == 1) or as `shards` files
    model-0000i-of-0000n.safetensors named by model.safetensors.index.json,
    each tensor under `prefix` + its name; "2_Dense.linear.weight" and
    "3_Dense.linear.weight" as 2_Dense/ and 3_Dense/model.safetensors holding
    `linear.weight`."""
    os.makedirs(directory, exist_ok=True)
    body = {prefix + n: a for n, a in tensors.items() if not n.endswith("_Dense.linear.weight")}
    for sub in ("2_Dense", "3_Dense"):
        if f"{sub}.linear.weight" in tensors:
            write_file(os.path.join(directory, sub, "model.safetensors"),
                       {"linear.weight": tensors[f"{sub}.linear.weight"]}, dtype)
    if shards == 1:
        write_file(os.path.join(directory, "model.safetensors"), body, dtype)
        return
    names = list(body)
    wmap = {}
    for i in range(shards):
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = names[i::shards]
        write_file(os.path.join(directory, fname), {n: body[n] for n in part}, dtype)
        wmap.update({n: fname for n in part})
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": wmap}, f)
