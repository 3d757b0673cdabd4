"""The seam and the boundary contract on the GPU, through the C ABI.

newDense (internal/model/bert.go:263-278) picks each matrix's mode on its
own: the requested one unless the packer refuses the matrix (PackB*'s
n % 16 rule, pack.go:29-37; a NaN/Inf weight, pack8.go:43-48), then the
next, down to the unpacked fp32 weights. Quantized / QuantizedActivations
(bert.go:526-644) report whether every matrix took an int8 path. The
decoders pack q, k, v, gate and up one matrix at a time
(qwen3.go:479-481,528-529; gemma3.go:297-299,363-364), so a refusal moves
only that matrix.

* A NaN weight under full int8: the load succeeds with that matrix in fp32,
  the introspection reports it, and the forward's NaN pattern matches the
  oracle built with the same fallback (a NaN weight reaches every output
  row, in the reference as here).
* A shape every packer refuses (intermediate 1000, not a multiple of 16):
  those matrices run on unpacked fp32 weights, the rest stay int8; the
  embeddings match the oracle's forward with the same fallback (full int8
  cosine >= 0.999, weight-only >= 0.9999).
* q, k, v, gate and up as separate weights (the reference's packing) give
  the same embeddings, bit for bit, as the fused weights, in every mode.
* The ABI's contract: a host allocation failure returns RH_ERR_OOM and the
  process carries on; a weight is refused on a context that did not pack
  it; rh_linear_u8 refuses a gated weight; int64 ids outside [0, vocab)
  return RH_ERR_VOCAB.
"""
import ctypes
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd import _lib
from rembed_amd import tensor as T
from rembed_amd._lib import lib
from rembed_amd.model import QUANT_FULL, QUANT_NONE, QUANT_WEIGHTS, Model, make_config
from rembed_amd.synthetic import (GEMMA3_300M, QWEN3_0_6B, BertShape, bert_tensors,
                                  decoder_tensors, token_batch)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def cos_rows(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.sum(a * b, 1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)


def bert_small(intermediate=1536):
    return BertShape("seam-bert", layers=2, hidden=384, heads=6, intermediate=intermediate,
                     vocab=4000, max_position=256, pooling=0)


def qwen3_small(intermediate=3072):
    return dataclasses.replace(QWEN3_0_6B, name="seam-qwen3", layers=2, vocab=3000,
                               max_seq=512, intermediate=intermediate)


def gemma3_small():
    return dataclasses.replace(GEMMA3_300M, name="seam-gemma3", layers=2, vocab=3000,
                               sliding_window=100, sliding_pattern=2, max_seq=512)


def oracle_for(shape, t, quant):
    if isinstance(shape, BertShape):
        return O.BertOracle(shape, t, quant)
    return O.DecoderOracle(shape, t, quant)


def tensors_for(shape, seed):
    if isinstance(shape, BertShape):
        return bert_tensors(shape, seed=seed)
    return decoder_tensors(shape, seed=seed, bf16=shape.arch == _lib.RH_ARCH_QWEN3)


# (shape maker, name of the matrix that gets a NaN weight)
NAN_CASES = [
    (bert_small, "encoder.layer.1.intermediate.dense.weight"),
    (qwen3_small, "layers.0.self_attn.k_proj.weight"),
    (gemma3_small, "layers.1.mlp.up_proj.weight"),
]


@pytest.mark.parametrize("make,name", NAN_CASES, ids=["bert-ffn1", "qwen3-k", "gemma3-up"])
def test_nan_weight_falls_back_to_fp32_for_that_matrix(gpu_ctx, make, name):
    shape = make()
    t = dict(tensors_for(shape, 31))
    w = t[name].copy()
    w[5, 7] = np.nan
    t[name] = w
    ids, lens = token_batch(3, 40, 5, 40, vocab=shape.vocab, id_lo=0, seed=32)
    say(f"{shape.name}: NaN in {name}")
    # the same matrix refused alone: every other matrix keeps full int8, so
    # the model is neither Quantized nor QuantizedActivations
    m = Model(gpu_ctx, shape, t, QUANT_FULL)
    assert not m.quantized() and not m.quantized_activations()
    got = m.embed(ids, lens)
    want = oracle_for(shape, t, QUANT_FULL).embed_batch(ids, lens)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # without the NaN every matrix is int8 again
    clean = tensors_for(shape, 31)
    m2 = Model(gpu_ctx, shape, clean, QUANT_FULL)
    assert m2.quantized() and m2.quantized_activations()
    m3 = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    assert not m3.quantized()


SHAPE_CASES = [
    (lambda: bert_small(1000), QUANT_FULL), (lambda: bert_small(1000), QUANT_WEIGHTS),
    (lambda: qwen3_small(1000), QUANT_FULL), (lambda: qwen3_small(1000), QUANT_WEIGHTS),
]


@pytest.mark.parametrize("make,quant", SHAPE_CASES,
                         ids=["bert-i1000-a8w8", "bert-i1000-w8", "qwen3-i1000-a8w8",
                              "qwen3-i1000-w8"])
def test_shape_refusal_runs_unpacked_fp32(gpu_ctx, make, quant):
    """intermediate = 1000: the matrices with 1000 output channels (BERT's
    FFN1; the decoders' gate and up) are refused by every packer and run on
    unpacked fp32 weights; the down projections (1000 inputs) stay int8."""
    shape = make()
    t = tensors_for(shape, 33)
    ids, lens = token_batch(4, 64, 8, 64, vocab=shape.vocab, id_lo=0, seed=34)
    m = Model(gpu_ctx, shape, t, quant)
    assert not m.quantized() and not m.quantized_activations()
    got = m.embed(ids, lens)
    want = oracle_for(shape, t, quant).embed_batch(ids, lens)
    c = cos_rows(got, want)
    say(f"{shape.name} quant={quant}: min cos {c.min():.7f}")
    assert c.min() >= (0.999 if quant == QUANT_FULL else 0.9999)
    # and the fp32 model of the same shape meets the fp32 bound
    if quant == QUANT_WEIGHTS:
        m0 = Model(gpu_ctx, shape, t, QUANT_NONE)
        err = np.abs(m0.embed(ids, lens) - oracle_for(shape, t, QUANT_NONE).embed_batch(ids, lens))
        say(f"  fp32 max abs err {err.max():.3e}")
        assert err.max() <= 1e-4


@pytest.mark.parametrize("make", [qwen3_small, gemma3_small], ids=["qwen3", "gemma3"])
@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS, QUANT_FULL],
                         ids=["fp32", "w8", "a8w8"])
def test_separate_projections_identical(gpu_ctx, make, quant):
    """q, k, v and gate, up packed as separate weights (three and two GEMMs,
    the glue kernel for act(gate)*up) equal the fused weights bit for bit:
    each output column is the same dot product, and the gated product is
    the same float32 expression."""
    shape = make()
    t = tensors_for(shape, 35)
    ids, lens = token_batch(5, 120, 1, 120, vocab=shape.vocab, id_lo=0, seed=36)
    fused = Model(gpu_ctx, shape, t, quant)
    sep = Model(gpu_ctx, shape, t, quant, fuse_projections=False)
    assert fused.quantized() == sep.quantized() == (quant != QUANT_NONE)
    assert sep.quantized_activations() == (quant == QUANT_FULL)
    a, b = fused.embed(ids, lens), sep.embed(ids, lens)
    assert np.array_equal(a, b)
    for x, y in zip(fused.embed_tokens(ids, lens), sep.embed_tokens(ids, lens)):
        assert np.array_equal(x, y)


def _model_handle(gpu_ctx, shape):
    cfg = make_config(shape)
    h = ctypes.c_void_p()
    _lib.check(lib.rh_model_create(gpu_ctx.h, ctypes.byref(cfg), QUANT_NONE, ctypes.byref(h)))
    return h


def test_host_allocation_failure_is_a_status(gpu_ctx):
    """A tensor too large for host memory (2^48 floats): the copy's
    allocation fails inside the library and comes back as RH_ERR_OOM; the
    process and the model handle stay usable."""
    shape = bert_small()
    h = _model_handle(gpu_ctx, shape)
    try:
        small = np.zeros(16, np.float32)
        dims = (ctypes.c_int64 * 2)(1 << 24, 1 << 24)
        st = lib.rh_model_set_tensor(h, b"embeddings.word_embeddings.weight",
                                     small.ctypes.data, dims, 2)
        assert st == _lib.RH_ERR_OOM, (st, lib.rh_last_error())
        assert b"allocation" in lib.rh_last_error()
        # the handle still works: a normal tensor is accepted
        dims1 = (ctypes.c_int64 * 1)(16)
        assert lib.rh_model_set_tensor(h, b"x", small.ctypes.data, dims1, 1) == 0
    finally:
        lib.rh_model_destroy(h)


def test_weight_of_another_context_is_refused(gpu_ctx):
    rng = np.random.default_rng(37)
    k, n, m = 64, 32, 8
    bT = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    with T.Context(0) as other:
        w = T.PackB(other, bT, k, n)
        a = gpu_ctx.upload(rng.standard_normal((m, k)).astype(np.float32))
        dst = gpu_ctx.alloc(m * n * 4)
        with pytest.raises(_lib.RembedError) as e:
            T.Linear(gpu_ctx, dst, a, w, m)
        assert e.value.code == _lib.RH_ERR_INVALID
        assert "another context" in str(e.value)
        # on its own context the same call runs
        a2 = other.upload(rng.standard_normal((m, k)).astype(np.float32))
        d2 = other.alloc(m * n * 4)
        T.Linear(other, d2, a2, w, m)
        other.sync()
        w.close()


def test_linear_u8_refuses_gated_weights(gpu_ctx):
    rng = np.random.default_rng(38)
    k, i, m = 64, 32, 16
    gate = (rng.standard_normal((i, k)) * 0.1).astype(np.float32)
    up = (rng.standard_normal((i, k)) * 0.1).astype(np.float32)
    pw = T.PackedGated(gpu_ctx, _lib.RH_MODE_A8W8, gate, up, k, i)
    ldq = T.ldq_for(k)
    qa, rs = gpu_ctx.alloc(m * ldq), gpu_ctx.alloc(m * 4)
    qo, ro, amx = gpu_ctx.alloc(m * 2 * i), gpu_ctx.alloc(m * 4), gpu_ctx.alloc(m * 4)
    for act in (_lib.RH_ACT_SWIGLU, _lib.RH_ACT_NONE):
        with pytest.raises(_lib.RembedError) as e:
            T.LinearU8(gpu_ctx, qa, ldq, rs, pw, m, act, qo, T.ldq_for(2 * i), ro, amx)
        assert e.value.code == _lib.RH_ERR_INVALID


def test_int64_ids_are_range_checked(gpu_ctx):
    """Ids arrive as int64 (bert.go:649); one outside [0, vocab) -- negative,
    or past 2^31 where an int32 narrowing would wrap -- is RH_ERR_VOCAB, and
    in-range int64 ids give the device path's vectors."""
    shape = bert_small()
    t = tensors_for(shape, 39)
    m = Model(gpu_ctx, shape, t, QUANT_WEIGHTS)
    ids, lens = token_batch(3, 20, 5, 20, vocab=shape.vocab, seed=40)
    want = m.embed(ids, lens)
    ids64 = ids.astype(np.int64)
    assert np.array_equal(m.embed(ids64, lens), want)
    for bad in (-1, shape.vocab, (1 << 32) + 5, 1 << 40):
        b = ids64.copy()
        b[1, 2] = bad
        with pytest.raises(_lib.RembedError) as e:
            m.embed(b, lens)
        assert e.value.code == _lib.RH_ERR_VOCAB, bad
    # ids past a text's length are never read
    b = ids64.copy()
    b[0, lens[0]:] = 1 << 40
    assert np.array_equal(m.embed(b, lens), want)
    with pytest.raises(ValueError):
        m.embed(ids64, lens[:2])
