"""nomic-embed and ModernBERT parity on the GPU (through the C ABI) against
the oracle (oracle/oracle_renc.c, itself pinned by tests/test_oracle_renc.py).

* Full width (hidden 768, 12 heads of 64; nomic SwiGLU 3072, ModernBERT
  GeGLU 1152), nomic two layers, ModernBERT four (global, local, local,
  global with a ±64 window, texts up to 300 tokens so the window cuts):
  fp32 embeddings within 1e-4 of the oracle, weight-only int8 cosine
  >= 0.9999 against the oracle's int8 path, full int8 cosine >= 0.999,
  per-token hidden states, batch == single.
* Every device variant gives identical bits: producer-written planes vs
  split rows, parts on 1-3 streams, gate|up fused into one gated weight vs
  separate GEMMs.
* A missing tensor and an out-of-vocab id are refused.
"""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd import _lib
from rembed_amd.model import QUANT_FULL, QUANT_NONE, QUANT_WEIGHTS, Model
from rembed_amd.synthetic import (MODERNBERT_BASE, NOMIC_V15, rope_encoder_tensors,
                                  token_batch)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def nomic_2l():
    return dataclasses.replace(NOMIC_V15, name="nomic-2l", layers=2, vocab=4000, max_seq=2048)


def modernbert_4l():
    return dataclasses.replace(MODERNBERT_BASE, name="modernbert-4l", layers=4, vocab=4000,
                               max_seq=2048)


MAKES = [nomic_2l, modernbert_4l]
IDS = ["nomic", "modernbert"]
_CACHE = {}


def setup(make):
    if make.__name__ not in _CACHE:
        shape = make()
        _CACHE[make.__name__] = (shape, rope_encoder_tensors(shape, seed=0x5EED0021))
    return _CACHE[make.__name__]


def cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, axis=1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)


def batch(shape, seed, n=5, hi=300):
    ids, lens = token_batch(n, hi, 1, hi, vocab=shape.vocab, id_lo=0, seed=seed)
    lens[0], lens[1] = hi, 1  # one text past the window, one of a single token
    return ids, lens


@pytest.mark.parametrize("make", MAKES, ids=IDS)
def test_renc_fp32_max_abs_1e4(gpu_ctx, make):
    shape, t = setup(make)
    ids, lens = batch(shape, 31)
    say(f"{shape.name} fp32 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_NONE)
    assert not m.quantized()
    got = m.embed(ids, lens)
    want = O.RopeEncoderOracle(shape, t, 0).embed_batch(ids, lens, threads=8)
    err = np.abs(got - want).max()
    say(f"  max abs err {err:.3e}")
    assert err <= 1e-4


@pytest.mark.parametrize("make", MAKES, ids=IDS)
def test_renc_weight_only_int8_cosine(gpu_ctx, make):
    shape, t = setup(make)
    ids, lens = batch(shape, 32)
    say(f"{shape.name} weight-only int8 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    assert m.quantized() and not m.quantized_activations()
    got = m.embed(ids, lens)
    want = O.RopeEncoderOracle(shape, t, 1).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    say(f"  min cos {c.min():.7f}")
    assert c.min() >= 0.9999


@pytest.mark.parametrize("make", MAKES, ids=IDS)
def test_renc_full_int8_cosine(gpu_ctx, make):
    shape, t = setup(make)
    ids, lens = batch(shape, 33)
    say(f"{shape.name} full int8 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_FULL)
    assert m.quantized() and m.quantized_activations()
    got = m.embed(ids, lens)
    want = O.RopeEncoderOracle(shape, t, 2).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    say(f"  min cos {c.min():.6f}")
    assert c.min() >= 0.999


@pytest.mark.parametrize("make", MAKES, ids=IDS)
def test_renc_tokens_match_oracle_hidden(gpu_ctx, make):
    shape, t = setup(make)
    ids, lens = batch(shape, 34, n=3, hi=200)
    m = Model(gpu_ctx, shape, t, QUANT_NONE)
    toks = m.embed_tokens(ids, lens)
    orc = O.RopeEncoderOracle(shape, t, 0)
    for b in range(len(lens)):
        want = orc.encode(ids[b, :lens[b]])
        err = np.abs(toks[b] - want).max() / max(1.0, np.abs(want).max())
        say(f"  text {b} len {lens[b]} rel err {err:.3e}")
        assert err <= 2e-5


@pytest.mark.parametrize("make", MAKES, ids=IDS)
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS, QUANT_FULL],
                         ids=["fp32", "w8", "a8w8"])
def test_renc_batch_matches_single(gpu_ctx, make, quant):
    shape, t = setup(make)
    ids, lens = batch(shape, 35, n=4, hi=200)
    m = Model(gpu_ctx, shape, t, quant)
    full = m.embed(ids, lens)
    for b in range(len(lens)):
        single = m.embed(ids[b:b + 1, :lens[b]], lens[b:b + 1])
        assert np.array_equal(single[0], full[b]), b


@pytest.mark.parametrize("make", MAKES, ids=IDS)
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS], ids=["fp32", "w8"])
def test_renc_producer_planes_identical(gpu_ctx, make, quant):
    """The LayerNorms, attention and the gated epilogue writing the next
    GEMM's bf16 planes directly match, bit for bit, fp32 rows split by each
    GEMM (nomic's post-norm writes x and the planes together)."""
    shape, t = setup(make)
    ids, lens = batch(shape, 36, n=3, hi=150)
    m = Model(gpu_ctx, shape, t, quant)
    direct = m.embed(ids, lens)
    m.set_producer_planes(False)
    split = m.embed(ids, lens)
    assert np.array_equal(direct, split)


@pytest.mark.parametrize("make", MAKES, ids=IDS)
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS, QUANT_FULL],
                         ids=["fp32", "w8", "a8w8"])
def test_renc_parts_on_streams_identical(gpu_ctx, make, quant):
    shape, t = setup(make)
    ids, lens = token_batch(32, 300, 150, 300, vocab=shape.vocab, id_lo=0, seed=37)
    say(f"{shape.name} quant={quant}: {len(lens)} texts, {int(lens.sum())} tokens")
    assert lens.sum() >= 6144
    m = Model(gpu_ctx, shape, t, quant)
    m.set_streams(1)
    one = m.embed(ids, lens)
    for n in (2, 3):
        m.set_streams(n)
        assert np.array_equal(m.embed(ids, lens), one), n


@pytest.mark.parametrize("make", MAKES, ids=IDS)
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS, QUANT_FULL],
                         ids=["fp32", "w8", "a8w8"])
def test_renc_separate_gate_up_identical(gpu_ctx, make, quant):
    """gate|up as one gated weight (act(gate) * up in the epilogue) equals
    two GEMMs and the separate glue pass, bit for bit (nomic: gate = fc12,
    up = fc11; ModernBERT: the two halves of Wi)."""
    shape, t = setup(make)
    ids, lens = batch(shape, 38, n=4, hi=200)
    fused = Model(gpu_ctx, shape, t, quant).embed(ids, lens)
    sep = Model(gpu_ctx, shape, t, quant, fuse_projections=False).embed(ids, lens)
    assert np.array_equal(fused, sep)


@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS], ids=["fp32", "w8"])
def test_modernbert_long_text_window(gpu_ctx, quant):
    """One 1024-token text: the ±64 window of the local layers is crossed
    many times over; fp32 within 1e-4, weight-only int8 cosine >= 0.9999,
    per-token hidden states too."""
    shape, t = setup(modernbert_4l)
    ids, lens = token_batch(1, 1024, 1024, 1024, vocab=shape.vocab, id_lo=0, seed=39)
    m = Model(gpu_ctx, shape, t, quant)
    got = m.embed(ids, lens)
    toks = m.embed_tokens(ids, lens)[0]
    orc = O.RopeEncoderOracle(shape, t, quant)
    want = orc.embed_batch(ids, lens)
    want_tok = orc.encode(ids[0, :1024])
    if quant == QUANT_NONE:
        err = np.abs(got - want).max()
        terr = np.abs(toks - want_tok).max() / max(1.0, np.abs(want_tok).max())
        say(f"  max abs err {err:.3e}, hidden rel err {terr:.3e}")
        assert err <= 1e-4 and terr <= 2e-5
    else:
        c, ct = cos_rows(got, want), cos_rows(toks, want_tok)
        say(f"  cos {c.min():.7f}, per-token min cos {ct.min():.7f}")
        assert c.min() >= 0.9999 and ct.min() >= 0.9999


@pytest.mark.parametrize("make,name", [(nomic_2l, "encoder.layers.1.mlp.fc11.weight"),
                                       (modernbert_4l, "layers.2.attn_norm.weight")], ids=IDS)
def test_renc_model_errors(gpu_ctx, make, name):
    shape, t = setup(make)
    bad = dict(t)
    del bad[name]
    with pytest.raises(_lib.RembedError) as e:
        Model(gpu_ctx, shape, bad, QUANT_NONE)
    assert e.value.code == _lib.RH_ERR_MISSING
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    with pytest.raises(_lib.RembedError) as e:
        m.embed(np.array([[shape.vocab]], np.int32), np.array([1], np.int32))
    assert e.value.code == _lib.RH_ERR_VOCAB
