"""Checkpoints on disk, loaded by Model.from_safetensors, against the oracle.

model.Load reads a model directory through LoadAny (bert.go:307-316,
internal/safetensors/safetensors.go:54-121) and, for EmbeddingGemma, the
Dense head from 2_Dense/ and 3_Dense/ (gemma3.go:144-172); every tensor is
widened to float32 on the way in. Each case here writes a synthetic model
directory (F32, F16 or BF16; one file or a sharded set with
model.safetensors.index.json; the backbone's names bare or under "model."),
loads it on the GPU, and compares the pooled vectors with the oracle run on
the float32 values the file represents (computed from the written arrays,
not by the reader): fp32 within 1e-4 absolute, weight-only int8 cosine
>= 0.9999. Gemma's norm weights are stored in checkpoint form (the unit
offset is added at load, gemma3.go:40-50,80-98), so the file route covers it.
"""
import dataclasses

import numpy as np
import pytest

import safetensors_files as SF
from oracle import oracle as O
from rembed_amd.model import QUANT_NONE, QUANT_WEIGHTS, Model
from rembed_amd.synthetic import (GEMMA3_300M, QWEN3_0_6B, BertShape, bert_tensors,
                                  decoder_tensors, token_batch)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def cos_rows(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.sum(a * b, 1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)


def bert_case():
    shape = BertShape("ckpt-bert", layers=2, hidden=384, heads=6, intermediate=1536,
                      vocab=4000, max_position=256, pooling=0)
    ids, lens = token_batch(6, 128, 5, 128, vocab=shape.vocab, seed=31)
    return shape, bert_tensors(shape, seed=32), ids, lens, O.BertOracle


def gemma_case():
    shape = dataclasses.replace(GEMMA3_300M, name="ckpt-gemma", layers=2, vocab=3000,
                                sliding_pattern=2, max_seq=1024)
    ids, lens = token_batch(4, 400, 5, 400, vocab=shape.vocab, id_lo=0, seed=33)
    lens[0] = 400  # past the 257-token window
    return shape, decoder_tensors(shape, seed=34), ids, lens, O.DecoderOracle


def qwen3_case():
    shape = dataclasses.replace(QWEN3_0_6B, name="ckpt-qwen3", layers=2, vocab=3000,
                                max_seq=512)
    ids, lens = token_batch(4, 200, 5, 200, vocab=shape.vocab, id_lo=0, seed=35)
    return shape, decoder_tensors(shape, seed=36), ids, lens, O.DecoderOracle


MAKE = {"bert": bert_case, "gemma3": gemma_case, "qwen3": qwen3_case}
_CACHE = {}


def case(name):
    if name not in _CACHE:
        _CACHE[name] = MAKE[name]()
    return _CACHE[name]


# (model, file dtype, shards, name prefix, quant)
CASES = [
    ("bert", "F32", 1, "", QUANT_NONE),
    ("bert", "F16", 1, "", QUANT_NONE),
    ("bert", "BF16", 2, "bert.", QUANT_NONE),
    ("bert", "F16", 1, "", QUANT_WEIGHTS),
    ("gemma3", "F32", 1, "", QUANT_NONE),
    ("gemma3", "BF16", 1, "", QUANT_NONE),
    ("gemma3", "F16", 2, "model.", QUANT_WEIGHTS),
    ("qwen3", "F16", 3, "model.", QUANT_NONE),
    ("qwen3", "BF16", 3, "", QUANT_WEIGHTS),
]


@pytest.mark.parametrize("model,dtype,shards,prefix,quant", CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}shard-{'w8' if c[4] else 'fp32'}"
                              for c in CASES])
def test_checkpoint_dir_matches_oracle(gpu_ctx, tmp_path, model, dtype, shards, prefix, quant):
    shape, t, ids, lens, Oracle = case(model)
    say(f"{model} {dtype} shards={shards} prefix={prefix!r} quant={quant} "
        f"lens {lens.tolist()}")
    SF.write_model_dir(str(tmp_path), t, dtype, shards=shards, prefix=prefix)
    held = {n: SF.represented(a, dtype) for n, a in t.items()}
    m = Model.from_safetensors(gpu_ctx, shape, str(tmp_path), quant)
    try:
        got = m.embed(ids, lens)
    finally:
        m.close()
    want = Oracle(shape, held, quant).embed_batch(ids, lens, threads=8)
    assert got.shape == want.shape and np.isfinite(got).all()
    if quant == QUANT_NONE:
        err = np.abs(got - want).max()
        say(f"  max abs err {err:.3e}")
        assert err <= 1e-4
    else:
        c = cos_rows(got, want)
        say(f"  min cos {c.min():.7f}")
        assert c.min() >= 0.9999
    if dtype != "F32":
        # the file's rounding is visible: the unrounded model differs
        full = Oracle(shape, t, quant).embed_batch(ids[:1], lens[:1], threads=8)
        assert not np.array_equal(full[0], want[0])

