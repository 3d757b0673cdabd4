"""Decoder-family parity on the GPU (through the C ABI) against the oracle.

* Gated GEMM (rh_pack_weight_gated + rh_linear with SwiGLU, tanh-GeGLU or
  erf-GeGLU): the fp32 values of gate and up come out of the same epilogue
  arithmetic as MatMulPacked/MatMulPacked8/MatMulPackedVNNI, then
  act(gate)*up as the model loops compute it (qwen3.go:530-539,
  gemma3.go:365-374, modernbert.go:292-301). Full int8 is compared
  element-wise within 1e-6 relative for SiLU / GELUTanh (the int32
  accumulators and dequantization are exact; the device evaluates them in
  float32, a few ulp from the reference's float64-then-rounded values) and
  bit for bit for the erf-GELU (the reference's float32 geluAVX2); fp32 and
  weight-only int8 within the GEMM tolerances.
* Qwen3- and EmbeddingGemma-shaped models at full width (hidden 1024 /
  16 Q, 8 KV heads of 128; hidden 768 / 3 Q, 1 KV head of 256, window 257,
  Dense 3072), two layers: fp32 embeddings within 1e-4 of the oracle,
  weight-only int8 cosine >= 0.9999 against the oracle's int8 path, full
  int8 cosine >= 0.999, batch == single, per-token hidden states.
* The same at the configurations' full length: Qwen3 one 512-token text,
  EmbeddingGemma one 2048-token text with window 512 / pattern 2.
"""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd import _lib
from rembed_amd import tensor as T
from rembed_amd.model import QUANT_FULL, QUANT_NONE, QUANT_WEIGHTS, Model
from rembed_amd.synthetic import GEMMA3_300M, QWEN3_0_6B, decoder_tensors, token_batch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def oracle_dense(mode, bT, a):
    """applyDense of the oracle for one weight (bert.go:282-301)."""
    n, k = bT.shape
    if mode == _lib.RH_MODE_F32:
        return O.matmul_f32(a, bT)
    if mode == _lib.RH_MODE_W8:
        st, q, sc = O.pack_b8(bT, k, n)
        assert st == 0
        return O.matmul_w8(a, q, sc)
    st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
    assert st == 0
    return O.matmul_vnni(a, q, cs, sc)[0]


# bf: the weight-only int8 / fp32 GEMM on pre-split bf16 planes (0) or with
# the split in its main loop (1); full int8 has one path
@pytest.mark.parametrize("mode,bf,tile", [(_lib.RH_MODE_F32, 0, 0), (_lib.RH_MODE_F32, 1, 0),
                                          (_lib.RH_MODE_W8, 0, 0), (_lib.RH_MODE_W8, 1, 0),
                                          (_lib.RH_MODE_W8, 0, 6), (_lib.RH_MODE_W8, 0, 10),
                                          (_lib.RH_MODE_A8W8, 0, 0)],
                         ids=["f32", "f32-inloop", "w8", "w8-inloop", "w8-tile6", "w8-tile10",
                              "a8w8"])
@pytest.mark.parametrize("act", [_lib.RH_ACT_SWIGLU, _lib.RH_ACT_GEGLU, _lib.RH_ACT_GEGLU_ERF],
                         ids=["swiglu", "geglu-tanh", "geglu-erf"])
def test_gated_linear_matches_oracle(gpu_ctx, mode, bf, tile, act):
    """Gated linear against the oracle; tile forces a planes tile (6 and 10
    are the two the automatic choice gives large one-term GLU linears)."""
    ctx = gpu_ctx
    rng = np.random.default_rng(10 * mode + act)
    m, k, i = 301, 384, 528
    say(f"gated linear mode={mode} bf_algo={bf} tile={tile} act={act} m={m} k={k} i={i}")
    a = rng.standard_normal((m, k)).astype(np.float32)
    gate = (rng.standard_normal((i, k)) * 0.05).astype(np.float32)
    up = (rng.standard_normal((i, k)) * 0.05).astype(np.float32)
    pw = T.PackedGated(ctx, mode, gate, up, k, i)
    a_d = ctx.upload(a)
    out = ctx.alloc(m * i * 4)
    ldq = T.ldq_for(k)
    qa, rs = ctx.alloc(m * ldq), ctx.alloc(m * 4)
    ctx.set_bf_algo(bf)
    ctx.set_option(_lib.RH_CTX_BF_TILE, tile)
    try:
        T.Linear(ctx, out, a_d, pw, m, act, qa, ldq, rs)
        ctx.sync()
    finally:
        ctx.set_bf_algo(0)
        ctx.set_option(_lib.RH_CTX_BF_TILE, 0)
    got = out.download(np.float32, (m, i))
    g = oracle_dense(mode, gate, a)
    u = oracle_dense(mode, up, a)
    # ModernBERT's tensor.GELU runs geluAVX2 over rows of i (a multiple of 8)
    # values: gelu_ref over the flattened rows takes the same path
    fn = {_lib.RH_ACT_SWIGLU: O.silu, _lib.RH_ACT_GEGLU: O.gelu_tanh,
          _lib.RH_ACT_GEGLU_ERF: O.gelu_ref}[act]
    want = (fn(g.ravel()).reshape(m, i) * u).astype(np.float32)
    err = np.abs(got.astype(np.float64) - want) / (1 + np.abs(want))
    say(f"  max rel err {err.max():.3e}")
    if mode == _lib.RH_MODE_A8W8 and act == _lib.RH_ACT_GEGLU_ERF:
        # exact accumulators, dequantization and erf-GELU: bit for bit
        assert np.array_equal(got, want)
    elif mode == _lib.RH_MODE_A8W8:
        assert err.max() <= 1e-6
    elif mode == _lib.RH_MODE_W8:
        # one bf16 activation term: |dg| <= 2^-9 sum|a·w| per half (2x
        # margin); the gated product moves by at most 1.2|dg||u| + |act(g)||du|
        # (|act'| <= 1.2 for SiLU, GELUTanh and erf-GELU)
        _, qg, sg = O.pack_b8(gate, k, i)
        _, qu, su = O.pack_b8(up, k, i)
        aa = np.abs(a.astype(np.float64))
        dg = 2.0 ** -8 * aa @ (np.abs(qg.astype(np.float64)) * sg[:, None]).T
        du = 2.0 ** -8 * aa @ (np.abs(qu.astype(np.float64)) * su[:, None]).T
        fg = np.abs(fn(g.ravel()).reshape(m, i).astype(np.float64))
        bound = 1.2 * dg * np.abs(u) + fg * du + 2e-4 * (1 + np.abs(want))
        assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    else:
        assert err.max() <= 2e-4
    # the gated weight refuses non-gated acts, and each half must pass the
    # packers' shape rule (pack.go:29-37)
    with pytest.raises(_lib.RembedError):
        T.Linear(ctx, out, a_d, pw, m, _lib.RH_ACT_NONE, qa, ldq, rs)
    with pytest.raises(_lib.RembedError) as e:
        T.PackedGated(ctx, mode, gate[:520], up[:520], k, 520)
    assert e.value.code == _lib.RH_ERR_SHAPE


def qwen3_2l():
    return dataclasses.replace(QWEN3_0_6B, name="qwen3-2l", layers=2, vocab=4000, max_seq=2048)


def gemma3_2l():
    # pattern 2: layer 0 sliding-window (257), layer 1 global
    return dataclasses.replace(GEMMA3_300M, name="gemma3-2l", layers=2, vocab=4000,
                               sliding_pattern=2, max_seq=2048)


_CACHE = {}


def setup(make, bf16):
    key = (make.__name__, bf16)
    if key not in _CACHE:
        shape = make()
        t = decoder_tensors(shape, seed=0x5EED0011, bf16=bf16)
        _CACHE[key] = (shape, t)
    return _CACHE[key]


def cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, axis=1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)


CASES = [(qwen3_2l, True, 6, 5, 300), (gemma3_2l, False, 4, 5, 600)]


@pytest.mark.parametrize("make,bf16,batch,lo,hi", CASES, ids=["qwen3", "gemma3"])
def test_decoder_fp32_max_abs_1e4(gpu_ctx, make, bf16, batch, lo, hi):
    shape, t = setup(make, bf16)
    ids, lens = token_batch(batch, hi, lo, hi, vocab=shape.vocab, id_lo=0, seed=21)
    lens[0] = hi  # one text spans the window / several 64-key blocks
    say(f"{shape.name} fp32 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_NONE)
    assert not m.quantized()
    got = m.embed(ids, lens)
    want = O.DecoderOracle(shape, t, 0).embed_batch(ids, lens, threads=8)
    err = np.abs(got - want).max()
    say(f"  max abs err {err:.3e}")
    assert err <= 1e-4


@pytest.mark.parametrize("make,bf16,batch,lo,hi", CASES, ids=["qwen3", "gemma3"])
def test_decoder_weight_only_int8_cosine(gpu_ctx, make, bf16, batch, lo, hi):
    shape, t = setup(make, bf16)
    ids, lens = token_batch(batch, hi, lo, hi, vocab=shape.vocab, id_lo=0, seed=22)
    say(f"{shape.name} weight-only int8 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    assert m.quantized() and not m.quantized_activations()
    got = m.embed(ids, lens)
    want = O.DecoderOracle(shape, t, 1).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    say(f"  min cos {c.min():.7f}")
    assert c.min() >= 0.9999


@pytest.mark.parametrize("make,bf16,batch,lo,hi", CASES, ids=["qwen3", "gemma3"])
def test_decoder_full_int8_cosine(gpu_ctx, make, bf16, batch, lo, hi):
    shape, t = setup(make, bf16)
    ids, lens = token_batch(batch, hi, lo, hi, vocab=shape.vocab, id_lo=0, seed=23)
    say(f"{shape.name} full int8 lens {lens.tolist()}")
    m = Model(gpu_ctx, shape, t, QUANT_FULL)
    assert m.quantized() and m.quantized_activations()
    got = m.embed(ids, lens)
    want = O.DecoderOracle(shape, t, 2).embed_batch(ids, lens, threads=8)
    c = cos_rows(got, want)
    say(f"  min cos {c.min():.6f}")
    assert c.min() >= 0.999


@pytest.mark.parametrize("shape,bf16", [(QWEN3_0_6B, True), (GEMMA3_300M, False)],
                         ids=["qwen3-28L", "gemma3-24L"])
def test_decoder_full_depth_weight_only_cosine(gpu_ctx, shape, bf16):
    """All 28 / 24 layers (errors compound with depth), weight-only int8 with
    one bf16 activation term (the default) and with two, against the
    oracle's int8 path: cosine >= 0.9999 for both."""
    from rembed_amd._lib import RH_CTX_W8_TERMS
    t = decoder_tensors(shape, seed=0x5EED0003, bf16=bf16)
    ids, lens = token_batch(4, 48, 24, 48, vocab=shape.vocab, id_lo=0, seed=7)
    want = O.DecoderOracle(shape, t, 1).embed_batch(ids, lens, threads=8)
    for terms in (1, 2):
        gpu_ctx.set_option(RH_CTX_W8_TERMS, terms)
        try:
            m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
            got = m.embed(ids, lens)
        finally:
            gpu_ctx.set_option(RH_CTX_W8_TERMS, 1)
        c = cos_rows(got, want)
        say(f"{shape.name} {terms}-term min cos {c.min():.7f}")
        assert c.min() >= 0.9999


@pytest.mark.parametrize("make,bf16", [(qwen3_2l, True), (gemma3_2l, False)], ids=["qwen3", "gemma3"])
def test_decoder_batch_matches_single(gpu_ctx, make, bf16):
    shape, t = setup(make, bf16)
    ids, lens = token_batch(4, 200, 3, 200, vocab=shape.vocab, id_lo=0, seed=24)
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    batch = m.embed(ids, lens)
    for b in range(len(lens)):
        single = m.embed(ids[b:b + 1, :lens[b]], lens[b:b + 1])
        assert np.array_equal(single[0], batch[b]), b


@pytest.mark.parametrize("make,bf16", [(qwen3_2l, True), (gemma3_2l, False)], ids=["qwen3", "gemma3"])
def test_decoder_tokens_match_oracle_hidden(gpu_ctx, make, bf16):
    shape, t = setup(make, bf16)
    ids, lens = token_batch(3, 140, 1, 140, vocab=shape.vocab, id_lo=0, seed=25)
    m = Model(gpu_ctx, shape, t, QUANT_NONE)
    toks = m.embed_tokens(ids, lens)
    orc = O.DecoderOracle(shape, t, 0)
    for b in range(len(lens)):
        want = orc.encode(ids[b, :lens[b]])
        err = np.abs(toks[b] - want).max() / max(1.0, np.abs(want).max())
        say(f"  text {b} len {lens[b]} rel err {err:.3e}")
        assert err <= 2e-5


@pytest.mark.parametrize("make,bf16", [(qwen3_2l, True), (gemma3_2l, False)], ids=["qwen3", "gemma3"])
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS], ids=["fp32", "w8"])
def test_decoder_producer_planes_identical(gpu_ctx, make, bf16, quant):
    """RMSNorm, attention and the gated epilogue writing the next GEMM's bf16
    planes directly match, bit for bit, fp32 rows split by each GEMM."""
    shape, t = setup(make, bf16)
    ids, lens = token_batch(3, 150, 20, 150, vocab=shape.vocab, id_lo=0, seed=26)
    m = Model(gpu_ctx, shape, t, quant)
    direct = m.embed(ids, lens)
    m.set_producer_planes(False)
    split = m.embed(ids, lens)
    assert np.array_equal(direct, split)


@pytest.mark.parametrize("make,bf16", [(qwen3_2l, True), (gemma3_2l, False)], ids=["qwen3", "gemma3"])
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS, QUANT_FULL], ids=["fp32", "w8", "a8w8"])
def test_decoder_parts_on_streams_identical(gpu_ctx, make, bf16, quant):
    """A batch of >= 6144 tokens run as 2 or 3 parts of whole texts on as
    many streams gives the same embeddings and hidden states, bit for bit,
    as one stream (the producers write every GEMM's planes, so no part
    touches the context's split workspace)."""
    shape, t = setup(make, bf16)
    ids, lens = token_batch(32, 300, 150, 300, vocab=shape.vocab, id_lo=0, seed=27)
    say(f"{shape.name} quant={quant}: {len(lens)} texts, {int(lens.sum())} tokens")
    assert lens.sum() >= 6144
    m = Model(gpu_ctx, shape, t, quant)
    m.set_streams(1)
    one = m.embed(ids, lens)
    tok_one = m.embed_tokens(ids, lens)
    for n in (2, 3):
        m.set_streams(n)
        got = m.embed(ids, lens)
        tok = m.embed_tokens(ids, lens)
        assert np.array_equal(got, one), n
        for a, b in zip(tok, tok_one):
            assert np.array_equal(a, b), n


@pytest.mark.parametrize("make,bf16", [(qwen3_2l, True), (gemma3_2l, False)], ids=["qwen3", "gemma3"])
def test_decoder_qk_epilogue_identical(gpu_ctx, make, bf16):
    """Weight-only int8 with QK-norm + RoPE in the q|k|v GEMM's epilogue
    (bf16 rows straight to attention) equals the GEMM's fp32 rows plus the
    separate pass, bit for bit: same values, same per-element arithmetic,
    same sum-of-squares order. The batch (~7000 rows) gives the fused tile
    at least 128 tiles; texts of one token and ragged row tails are
    included."""
    shape, t = setup(make, bf16)
    ids, lens = token_batch(48, 300, 1, 300, vocab=shape.vocab, id_lo=0, seed=28)
    lens[0], lens[1] = 1, 300
    say(f"{shape.name} qk epilogue: {len(lens)} texts, {int(lens.sum())} tokens")
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    m.set_streams(1)
    m.set_qk_epilogue(True)
    fused = m.embed(ids, lens)
    tok_fused = m.embed_tokens(ids, lens)
    m.set_qk_epilogue(False)
    sep = m.embed(ids, lens)
    tok_sep = m.embed_tokens(ids, lens)
    assert np.array_equal(fused, sep)
    for a, b in zip(tok_fused, tok_sep):
        assert np.array_equal(a, b)


def gemma3_2l_w512():
    # the benchmark's attention: layer 0 sliding window 512, layer 1 global
    return dataclasses.replace(GEMMA3_300M, name="gemma3-2l-w512", layers=2, vocab=4000,
                               sliding_window=512, sliding_pattern=2, max_seq=2048)


# Qwen3 at the benchmark's 512 tokens, EmbeddingGemma at 2048 with window 512:
# one full-length text each, two layers, against the oracle's forward
FULL_LENGTH = [(qwen3_2l, True, 512), (gemma3_2l_w512, False, 2048)]


@pytest.mark.parametrize("make,bf16,length", FULL_LENGTH, ids=["qwen3-512", "gemma3-2048-w512"])
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS], ids=["fp32", "w8"])
def test_decoder_full_config_length(gpu_ctx, make, bf16, length, quant):
    """The configurations' full text length: every key block of the causal
    mask (qwen3.go:319-390) and of the |i-j| < 512 window (gemma3.go:339-347)
    is crossed. fp32 embeddings within 1e-4 of the oracle, weight-only int8
    cosine >= 0.9999 against the oracle's int8 path; per-token hidden states
    checked too."""
    shape, t = setup(make, bf16)
    ids, lens = token_batch(1, length, length, length, vocab=shape.vocab, id_lo=0, seed=29)
    say(f"{shape.name} quant={quant} one text of {length} tokens, window {shape.sliding_window}")
    m = Model(gpu_ctx, shape, t, quant)
    got = m.embed(ids, lens)
    toks = m.embed_tokens(ids, lens)[0]
    orc = O.DecoderOracle(shape, t, quant)
    want = orc.embed_batch(ids, lens)
    want_tok = orc.encode(ids[0, :length])
    if quant == QUANT_NONE:
        err = np.abs(got - want).max()
        terr = np.abs(toks - want_tok).max() / max(1.0, np.abs(want_tok).max())
        say(f"  max abs err {err:.3e}, hidden rel err {terr:.3e}")
        assert err <= 1e-4
        assert terr <= 2e-5
    else:
        c = cos_rows(got, want)
        ct = cos_rows(toks, want_tok)
        say(f"  cos {c.min():.7f}, per-token min cos {ct.min():.7f}")
        assert c.min() >= 0.9999
        assert ct.min() >= 0.9999


def test_decoder_model_errors(gpu_ctx):
    shape, t = setup(qwen3_2l, True)
    bad = dict(t)
    del bad["layers.1.mlp.up_proj.weight"]
    with pytest.raises(_lib.RembedError) as e:
        Model(gpu_ctx, shape, bad, QUANT_NONE)
    assert e.value.code == _lib.RH_ERR_MISSING
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    with pytest.raises(_lib.RembedError) as e:
        m.embed(np.array([[shape.vocab]], np.int32), np.array([1], np.int32))
    assert e.value.code == _lib.RH_ERR_VOCAB
