"""GPU parity of the device-resident encoder against the oracle's per-text,
unpadded forward on identical synthetic weights and token ids.

Contracts: fp32 max |err| <= 1e-4 on final embeddings; weight-only int8
cosine >= 0.9999 against the oracle's int8 path; full int8 cosine against
the oracle's full-int8 path (and >= 0.991 against fp32, the reference's own
floor, rembed_test.go:107-166); batch results equal single-text results.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


SHAPES = {}


def minilm_small():
    from rembed_amd.synthetic import MINILM_L6
    return MINILM_L6


def bert_base():
    from rembed_amd.synthetic import BERT_BASE
    return BERT_BASE


@pytest.fixture(scope="module")
def minilm():
    from rembed_amd.synthetic import bert_tensors, token_batch
    shape = minilm_small()
    t = bert_tensors(shape, seed=0x5EED0001)
    ids, lens = token_batch(12, 128, 16, 128, seed=0x5EED0002)
    return shape, t, ids, lens


def gpu_embed(ctx, shape, t, quant, ids, lens, prec=None):
    from rembed_amd.model import Model
    m = Model(ctx, shape, t, quant)
    if prec:
        m.set_attention_precision(prec)
    out = m.embed(ids, lens)
    return m, out


def cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, 1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


def test_minilm_fp32_max_abs_1e4(gpu_ctx, minilm):
    shape, t, ids, lens = minilm
    say("minilm fp32")
    m, got = gpu_embed(gpu_ctx, shape, t, 0, ids, lens)
    assert not m.quantized()
    want = O.BertOracle(shape, t, 0).embed_batch(ids, lens, threads=8)
    err = np.abs(got - want).max()
    say(f"  max abs err {err:.3e}")
    assert err <= 1e-4


def test_minilm_weight_only_cosine(gpu_ctx, minilm):
    shape, t, ids, lens = minilm
    say("minilm w8")
    m, got = gpu_embed(gpu_ctx, shape, t, 1, ids, lens)
    assert m.quantized() and not m.quantized_activations()
    want = O.BertOracle(shape, t, 1).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    say(f"  min cos {c.min():.7f} max abs {np.abs(got - want).max():.3e}")
    assert c.min() >= 0.9999


def test_minilm_full_int8_cosine(gpu_ctx, minilm):
    shape, t, ids, lens = minilm
    say("minilm a8w8")
    m, got = gpu_embed(gpu_ctx, shape, t, 2, ids, lens)
    assert m.quantized() and m.quantized_activations()
    want = O.BertOracle(shape, t, 2).embed_batch(ids, lens, threads=8)
    fp = O.BertOracle(shape, t, 0).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    c32 = cos_rows(got, fp)
    say(f"  min cos vs oracle int8 {c.min():.6f}, vs fp32 {c32.min():.6f}")
    assert c.min() >= 0.999
    assert c32.min() >= 0.991
    # the int8 path is really active (rembed_test.go:107-174)
    assert np.abs(got - fp).max() >= 1e-4


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_batch_matches_single(gpu_ctx, minilm, quant):
    """TestEmbedBatchMatchesSingle (rembed_test.go:1262-1315): a text's vector
    does not depend on the other texts in the batch."""
    shape, t, ids, lens = minilm
    from rembed_amd.model import Model
    m = Model(gpu_ctx, shape, t, quant)
    batch = m.embed(ids, lens)
    for b in (0, 5, 11):
        single = m.embed(ids[b: b + 1, : lens[b]], lens[b: b + 1])
        assert np.array_equal(single[0], batch[b]), b


def test_fused_ffn1_identical(gpu_ctx, minilm):
    """The fused full-int8 FFN1 (u8 rows written by the GEMM, no fp32
    intermediate) yields the same embeddings, bit for bit, as fp32 GELU rows
    followed by QuantizeRowU8 (bert.go:910-916)."""
    shape, t, ids, lens = minilm
    from rembed_amd.model import Model
    m = Model(gpu_ctx, shape, t, 2)
    m.set_fused_ffn1(0)
    plain = m.embed(ids, lens)
    m.set_fused_ffn1(1)
    fused = m.embed(ids, lens)
    assert np.array_equal(plain, fused)


@pytest.mark.parametrize("model", ["minilm", "bertbase"])
@pytest.mark.parametrize("streams", [1, 2])
def test_onepass_ffn1_identical(gpu_ctx, request, model, streams):
    """The one-pass full-int8 FFN1 (RH_OPT_FUSED_FFN1 2: the GEMM's
    workgroups meet per row block on the GELU rows' |max| and write
    QuantizeRowU8's bytes, bert.go:910-916) gives the same embeddings, bit
    for bit, as fp32 rows followed by the separate GELU + quantize pass.
    Repeated calls and a smaller batch after the full one check that every
    launch leaves its departure counts zero and its row slots empty for the
    next; no wait timed out (rh_model_check)."""
    from rembed_amd.model import Model
    shape, t, ids, lens = request.getfixturevalue(model)
    say(f"{shape.name}: {len(lens)} texts, {int(lens.sum())} rows, {streams} stream(s)")
    m = Model(gpu_ctx, shape, t, 2)
    m.set_streams(streams)
    m.set_fused_ffn1(0)
    plain = m.embed(ids, lens)
    few = m.embed(ids[:5], lens[:5])
    m.set_fused_ffn1(2)
    for rep in range(3):
        assert np.array_equal(m.embed(ids, lens), plain), rep
        assert np.array_equal(m.embed(ids[:5], lens[:5]), few), rep
    m.check()


@pytest.mark.parametrize("model", ["minilm", "bertbase"])
@pytest.mark.parametrize("streams", [1, 2])
def test_fused_ln_identical(gpu_ctx, request, model, streams):
    """The full-int8 attention-output and FFN2 projections finishing the
    residual add, LayerNorm and the next GEMM's u8 rows in their epilogue
    (one kernel per block, whole rows per workgroup) give the same
    embeddings and hidden states, bit for bit, as the projection's fp32
    rows followed by the separate residual + LayerNorm pass
    (bert.go:905-907,916-918): the same float operations in the same
    order. MiniLM (hidden 384, K 384 and 1536) and BERT-base (768; 768 and
    3072), ragged row tails included."""
    from rembed_amd.model import Model
    shape, t, ids, lens = request.getfixturevalue(model)
    say(f"{shape.name}: {len(lens)} texts, {int(lens.sum())} rows, {streams} stream(s)")
    m = Model(gpu_ctx, shape, t, 2)
    m.set_streams(streams)
    m.set_fused_ln(True)
    fused = m.embed(ids, lens)
    tok_fused = m.embed_tokens(ids, lens)
    m.set_fused_ln(False)
    plain = m.embed(ids, lens)
    tok_plain = m.embed_tokens(ids, lens)
    assert np.array_equal(fused, plain)
    for a, b in zip(tok_fused, tok_plain):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("quant", [0, 1], ids=["fp32", "w8"])
def test_producer_planes_identical(gpu_ctx, minilm, quant):
    """Norms, attention and the FFN1 epilogue writing the next GEMM's bf16
    planes directly give the same embeddings and hidden states, bit for bit,
    as fp32 rows split by each GEMM (the same hi = bf16(v), lo = bf16(v - hi)
    of the same values)."""
    shape, t, ids, lens = minilm
    from rembed_amd.model import Model
    m = Model(gpu_ctx, shape, t, quant)
    direct = m.embed(ids, lens)
    tok_direct = m.embed_tokens(ids, lens)
    m.set_producer_planes(False)
    split = m.embed(ids, lens)
    tok_split = m.embed_tokens(ids, lens)
    assert np.array_equal(direct, split)
    for a, b in zip(tok_direct, tok_split):
        assert np.array_equal(a, b)


@pytest.fixture(scope="module")
def minilm_int8_big(gpu_ctx, minilm):
    from rembed_amd.model import Model
    from rembed_amd.synthetic import token_batch
    shape, t, _, _ = minilm
    ids, lens = token_batch(128, 128, 16, 128, seed=0x5EED0003)
    m = Model(gpu_ctx, shape, t, 2)
    m.set_streams(1)
    return m, ids, lens, m.embed(ids, lens), m.embed_tokens(ids, lens)


@pytest.mark.parametrize("quant", [0, 1], ids=["fp32", "w8"])
def test_parts_on_streams_identical_planes(gpu_ctx, minilm, quant):
    """The fp32 / weight-only encoder (the embedding LayerNorm writes the
    first QKV's planes, so no GEMM needs the split workspace) as 2 parts on
    two streams equals one stream bit for bit."""
    from rembed_amd.model import Model
    from rembed_amd.synthetic import token_batch
    shape, t, _, _ = minilm
    ids, lens = token_batch(64, 128, 16, 128, seed=0x5EED0004)
    assert lens.sum() >= 4096
    m = Model(gpu_ctx, shape, t, quant)
    m.set_streams(1)
    one = m.embed(ids, lens)
    m.set_streams(2)
    assert np.array_equal(m.embed(ids, lens), one)


@pytest.mark.parametrize("tile", [3, 7, 9, 10, 11, 12])
def test_full_int8_forward_identical_on_every_tile(gpu_ctx, minilm_int8_big, tile):
    """The full-int8 forward (bf16 q|k|v rows, fp32 O / FFN rows, every
    epilogue the model uses) gives the same embeddings and hidden states, bit
    for bit, whichever int8 GEMM tile runs: the accumulators and the
    dequantization are the same."""
    from rembed_amd._lib import RH_CTX_I8_TILE
    m, ids, lens, one, tok_one = minilm_int8_big
    say(f"tile {tile}: {len(lens)} texts, {int(lens.sum())} tokens")
    gpu_ctx.set_option(RH_CTX_I8_TILE, tile)
    try:
        got = m.embed(ids, lens)
        tok = m.embed_tokens(ids, lens)
    finally:
        gpu_ctx.set_option(RH_CTX_I8_TILE, 0)
    assert np.array_equal(got, one)
    for a, b in zip(tok, tok_one):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("streams", [2, 3, 4])
def test_parts_on_streams_identical(minilm_int8_big, streams):
    """A full-int8 batch (128 texts, >= 8192 tokens: parts of >= 2048 rows)
    run as `streams` parts of whole texts on as many streams gives the same
    embeddings and hidden states, bit for bit, as one stream (every kernel
    computes each row the same way whichever part it belongs to)."""
    m, ids, lens, one, tok_one = minilm_int8_big
    say(f"{streams} streams: {len(lens)} texts, {int(lens.sum())} tokens")
    assert lens.sum() >= 8192
    m.set_streams(streams)
    try:
        got = m.embed(ids, lens)
        tok = m.embed_tokens(ids, lens)
    finally:
        m.set_streams(1)
    assert np.array_equal(got, one)
    for a, b in zip(tok, tok_one):
        assert np.array_equal(a, b)


def test_embed_tokens_matches_oracle_hidden(gpu_ctx, minilm):
    shape, t, ids, lens = minilm
    from rembed_amd.model import Model
    m = Model(gpu_ctx, shape, t, 0)
    toks = m.embed_tokens(ids[:3], lens[:3])
    orc = O.BertOracle(shape, t, 0)
    for b in range(3):
        want = orc.encode(ids[b, : lens[b]])
        assert toks[b].shape == want.shape
        assert np.abs(toks[b] - want).max() <= 1e-4


def test_model_errors(gpu_ctx, minilm):
    from rembed_amd._lib import RembedError, RH_ERR_SEQ, RH_ERR_VOCAB, RH_ERR_MISSING
    from rembed_amd.model import Model
    shape, t, ids, lens = minilm
    m = Model(gpu_ctx, shape, t, 0)
    with pytest.raises(RembedError) as e:
        m.embed([[1, 2, shape.vocab]])
    assert e.value.code == RH_ERR_VOCAB
    with pytest.raises(RembedError) as e:
        m.embed(np.zeros((1, 4), np.int32), np.array([0], np.int32))
    assert e.value.code == RH_ERR_SEQ
    with pytest.raises(RembedError) as e:
        m.embed(np.zeros((1, 600), np.int32), np.array([600], np.int32))
    assert e.value.code == RH_ERR_SEQ
    t2 = dict(t)
    del t2["encoder.layer.3.output.dense.bias"]
    with pytest.raises(RembedError) as e:
        Model(gpu_ctx, shape, t2, 0)
    assert e.value.code == RH_ERR_MISSING


@pytest.fixture(scope="module")
def bertbase():
    from rembed_amd.synthetic import bert_tensors, token_batch
    shape = bert_base()
    t = bert_tensors(shape, seed=0x5EED0001)
    ids, lens = token_batch(64, 256, 64, 256, seed=0x5EED0002)
    return shape, t, ids, lens


@pytest.mark.parametrize("quant", [0, 2])
def test_bert_base_full_batch_parity(gpu_ctx, bertbase, quant):
    """The benchmark workload (64 texts x up to 256 tokens) on the GPU; a
    sample of texts re-run on the oracle."""
    shape, t, ids, lens = bertbase
    say(f"bert-base quant={quant}")
    m, got = gpu_embed(gpu_ctx, shape, t, quant, ids, lens)
    assert np.all(np.abs(np.linalg.norm(got.astype(np.float64), axis=1) - 1) < 1e-5)
    sample = [0, 17, 63]
    want = O.BertOracle(shape, t, quant).embed_batch(ids[sample], lens[sample], threads=8)
    if quant == 0:
        err = np.abs(got[sample] - want).max()
        say(f"  max abs err {err:.3e}")
        assert err <= 1e-4
    else:
        c = cos_rows(got[sample], want)
        say(f"  min cos {c.min():.6f}")
        assert c.min() >= 0.999


def _write_safetensors(path, tensors, bf16):
    """A .safetensors file of the tensors as F32, or as BF16 (top 16 bits)."""
    import json
    import struct
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr, np.float32)
        raw = (a.view(np.uint32) >> 16).astype("<u2").tobytes() if bf16 else a.astype("<f4").tobytes()
        header[name] = {"dtype": "BF16" if bf16 else "F32", "shape": list(a.shape),
                        "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"".join(blobs))


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_model_from_safetensors_identical(gpu_ctx, minilm, tmp_path, bf16):
    """Model.from_safetensors (the checkpoint read as safetensors.go:122-181
    widens it) embeds bit for bit as the model built from the same float32
    tensors in memory; a BF16 file equals its widened values."""
    from rembed_amd.model import Model
    shape, t, ids, lens = minilm
    path = str(tmp_path / "m.safetensors")
    _write_safetensors(path, t, bf16)
    if bf16:
        t = {k: ((np.ascontiguousarray(v, np.float32).view(np.uint32) >> 16) << 16).view(np.float32)
             for k, v in t.items()}
    for quant in (0, 2):
        want = Model(gpu_ctx, shape, t, quant).embed(ids, lens)
        got = Model.from_safetensors(gpu_ctx, shape, path, quant).embed(ids, lens)
        assert np.array_equal(got, want), quant
