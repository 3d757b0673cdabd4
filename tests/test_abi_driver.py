"""A C caller of the ABI, built as a cgo binding would be built.

tests/c/abi_driver.c is plain C99 against include/rembed_hip.h and links
librembed_hip.so; it makes the Load / Embed / Close sequence of a Go host
(context, model, every raw tensor by name, finalize, Quantized*, Embed with
int64 ids, destroy). These tests

* compile it with gcc -std=c99 -pedantic -Wall -Wextra -Werror (CPU);
* run it with no GPU and expect the distinct no-device status, the host's
  cue to fall back to its CPU path (CPU);
* run it on the GPU over a synthetic checkpoint and batch and compare its
  vectors with the oracle's forward: fp32 within 1e-4, full int8 cosine
  >= 0.999, weight-only int8 cosine >= 0.9999 (GPU).
"""
import dataclasses
import os
import struct
import subprocess

import numpy as np
import pytest

from rembed_amd import _lib
from rembed_amd.model import QUANT_FULL, QUANT_NONE, QUANT_WEIGHTS, make_config
from rembed_amd.synthetic import (QWEN3_0_6B, BertShape, bert_tensors, decoder_tensors,
                                  token_batch)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c", "abi_driver.c")
LIBDIR = os.path.dirname(_lib.LIB_PATH)


def build_driver(outdir):
    exe = os.path.join(str(outdir), "abi_driver")
    cmd = ["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-O1",
           "-I", os.path.join(ROOT, "include"), SRC, "-o", exe,
           "-L", LIBDIR, "-l:" + os.path.basename(_lib.LIB_PATH), f"-Wl,-rpath,{LIBDIR}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def write_bundle(path, shape, tensors, quant, ids, lens):
    """The Go host's state after reading a checkpoint and tokenizing."""
    c = make_config(shape)
    eps_bits = struct.unpack("<i", struct.pack("<f", c.layer_norm_eps))[0]
    ints = [c.arch, c.hidden, c.layers, c.heads, c.intermediate, c.vocab, c.max_position,
            c.position_offset, c.type_vocab, eps_bits, c.pooling, c.normalize, c.kv_heads,
            c.head_dim, c.sliding_window, c.sliding_pattern, c.query_pre_attn_scalar,
            c.dense_hidden, 0, 0, 0, 0]
    ids = np.ascontiguousarray(ids, np.int64)
    lens = np.ascontiguousarray(lens, np.int32)
    with open(path, "wb") as f:
        f.write(b"RHB1")
        f.write(struct.pack("<22i", *ints))
        f.write(struct.pack("<ddi", c.rope_theta, c.rope_local_theta, quant))
        f.write(struct.pack("<i", len(tensors)))
        for name, arr in tensors.items():
            arr = np.ascontiguousarray(arr, np.float32)
            nb = name.encode()
            f.write(struct.pack("<i", len(nb)) + nb)
            f.write(struct.pack("<i", arr.ndim))
            f.write(struct.pack(f"<{arr.ndim}q", *arr.shape))
            f.write(arr.tobytes())
        f.write(struct.pack("<ii", ids.shape[0], ids.shape[1]))
        f.write(lens.tobytes())
        f.write(ids.tobytes())


def read_out(path):
    raw = open(path, "rb").read()
    st, q, qa, batch, hidden = struct.unpack("<5i", raw[:20])
    vec = np.frombuffer(raw[20:], np.float32).reshape(batch, hidden)
    return st, bool(q), bool(qa), vec


def small_bert():
    return BertShape("abi-bert", layers=2, hidden=384, heads=6, intermediate=1536,
                     vocab=5000, max_position=256, pooling=0)


def test_driver_compiles_as_c99_and_reports_no_device(tmp_path):
    exe = build_driver(tmp_path)
    import ctypes
    n = ctypes.c_int(0)
    if _lib.lib.rh_device_count(ctypes.byref(n)) == _lib.RH_OK:
        pytest.skip("a GPU is present: the GPU test runs the driver")
    shape = small_bert()
    t = bert_tensors(shape, seed=3)
    ids, lens = token_batch(2, 16, 4, 16, vocab=shape.vocab, seed=4)
    bundle = tmp_path / "b.bin"
    write_bundle(bundle, shape, t, QUANT_NONE, ids, lens)
    r = subprocess.run([exe, str(bundle), str(tmp_path / "o.bin")], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == _lib.RH_ERR_NO_DEVICE, (r.returncode, r.stderr)
    assert "no HIP device" in r.stderr


CASES = [("bert-fp32", QUANT_NONE), ("bert-a8w8", QUANT_FULL), ("qwen3-w8", QUANT_WEIGHTS)]


@pytest.mark.gpu
@pytest.mark.parametrize("case,quant", CASES, ids=[c[0] for c in CASES])
def test_driver_embeds_like_the_oracle(tmp_path, case, quant):
    from oracle import oracle as O
    exe = build_driver(tmp_path)
    if case.startswith("bert"):
        shape = small_bert()
        t = bert_tensors(shape, seed=5)
        ids, lens = token_batch(6, 128, 3, 128, vocab=shape.vocab, seed=6)
        orc = O.BertOracle(shape, t, quant)
    else:
        shape = dataclasses.replace(QWEN3_0_6B, name="abi-qwen3", layers=2, vocab=3000,
                                    max_seq=512)
        t = decoder_tensors(shape, seed=7, bf16=True)
        ids, lens = token_batch(4, 96, 8, 96, vocab=shape.vocab, id_lo=0, seed=8)
        orc = O.DecoderOracle(shape, t, quant)
    print(f"{case}: lens {lens.tolist()}", flush=True)
    bundle, out = tmp_path / "b.bin", tmp_path / "o.bin"
    write_bundle(bundle, shape, t, quant, ids, lens)
    r = subprocess.run([exe, str(bundle), str(out)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, (r.returncode, r.stderr)
    st, q, qa, got = read_out(out)
    assert st == 0
    assert q == (quant != QUANT_NONE) and qa == (quant == QUANT_FULL)
    want = orc.embed_batch(ids.astype(np.int32), lens, threads=8)
    if quant == QUANT_NONE:
        err = np.abs(got - want).max()
        print(f"  max abs err {err:.3e}", flush=True)
        assert err <= 1e-4
    else:
        g, w = got.astype(np.float64), want.astype(np.float64)
        cos = np.sum(g * w, 1) / np.linalg.norm(g, axis=1) / np.linalg.norm(w, axis=1)
        print(f"  min cos {cos.min():.7f}", flush=True)
        assert cos.min() >= (0.999 if quant == QUANT_FULL else 0.9999)
