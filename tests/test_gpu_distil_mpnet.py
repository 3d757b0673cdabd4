"""DistilBERT and MPNet device forwards against the oracle (the reference's
multi-qa-distilbert-cos-v1 and all-mpnet-base-v2 architectures: bert.go:399-470
tensor names, no token-type table, MPNet's relative-position bias added to the
scaled scores, bert.go:816-830,876-890, and its position offset).

Contracts, as for BERT: fp32 max |err| <= 1e-4 on final embeddings;
weight-only int8 cosine >= 0.9999 against the oracle's int8 path; full int8
cosine >= 0.999 against the oracle's full-int8 path; with RH_OPT_EXACT the
full-int8 vectors and hidden states equal the oracle's bit for bit. Texts
reach MPNet's longest relative positions (bucket saturation past 128) and the
full 512-token table.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, 1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


SHAPES = {}


def workload(which):
    from rembed_amd import synthetic as S
    if which not in SHAPES:
        shape = S.DISTILBERT_BASE if which == "distilbert" else S.MPNET_BASE
        t = S.bert_tensors(shape, seed=0x5EED0011)
        ids, lens = S.token_batch(6, 512, 8, 300, vocab=shape.vocab, id_lo=3, seed=0x5EED0012)
        if which == "mpnet":  # one text at the table's full length (514 - 2)
            lens[0] = 512
            ids[0, :512] = np.random.default_rng(5).integers(3, shape.vocab, 512)
        SHAPES[which] = (shape, t, ids, lens)
    return SHAPES[which]


@pytest.mark.parametrize("which", ["distilbert", "mpnet"])
@pytest.mark.parametrize("quant", [0, 1, 2], ids=["fp32", "w8", "int8"])
def test_forward_against_oracle(gpu_ctx, which, quant):
    from rembed_amd.model import Model
    shape, t, ids, lens = workload(which)
    say(f"{which} quant={quant} lens={lens.tolist()}")
    m = Model(gpu_ctx, shape, t, quant)
    got = m.embed(ids, lens)
    assert m.quantized() == (quant > 0) and m.quantized_activations() == (quant == 2)
    m.close()
    orc = O.BertOracle(shape, t, quant)
    want = orc.embed_batch(ids, lens, threads=8)
    orc.close()
    if quant == 0:
        err = np.abs(got - want).max()
        say(f"  fp32 max err {err:.2e}")
        assert err <= 1e-4
    else:
        c = cos_rows(got, want)
        say(f"  min cosine {c.min():.7f}")
        assert c.min() >= (0.9999 if quant == 1 else 0.999)


@pytest.mark.parametrize("which", ["distilbert", "mpnet"])
def test_exact_full_int8_byte_identical(gpu_ctx, which):
    from rembed_amd.model import Model
    shape, t, ids, lens = workload(which)
    orc = O.BertOracle(shape, t, 2)
    want_v = orc.embed_batch(ids, lens, threads=8)
    want_h = [orc.encode(ids[b, :lens[b]]) for b in range(len(lens))]
    orc.close()
    m = Model(gpu_ctx, shape, t, 2)
    m.set_exact(True)
    vec = m.embed(ids, lens)
    toks = m.embed_tokens(ids, lens)
    m.close()
    assert np.array_equal(vec.view(np.uint32), want_v.view(np.uint32))
    for b in range(len(lens)):
        assert np.array_equal(toks[b].view(np.uint32), want_h[b].view(np.uint32)), b


def test_attention_precisions_agree_with_bias(gpu_ctx):
    """MPNet at bf16 and fp32-grade attention: both within the weight-only
    contract of the oracle, and the bias is observable at that resolution
    (a zero table breaks the contract)."""
    from rembed_amd.model import Model
    shape, t, ids, lens = workload("mpnet")
    orc = O.BertOracle(shape, t, 1)
    want = orc.embed_batch(ids, lens, threads=8)
    orc.close()
    m = Model(gpu_ctx, shape, t, 1)
    for prec in (1, 3):
        m.set_attention_precision(prec)
        c = cos_rows(m.embed(ids, lens), want)
        say(f"  mpnet w8 precision {prec}: min cosine {c.min():.7f}")
        assert c.min() >= 0.9999
    m.close()
    t0 = dict(t)
    t0["encoder.relative_attention_bias.weight"] = np.zeros_like(
        t["encoder.relative_attention_bias.weight"])
    m0 = Model(gpu_ctx, shape, t0, 1)
    c0 = cos_rows(m0.embed(ids, lens), want)
    m0.close()
    say(f"  without the bias table: min cosine {c0.min():.7f}")
    assert c0.min() < 0.9999, "dropping the relative-position bias stays within the contract"


def test_distilbert_has_no_token_type_and_mpnet_offsets_positions(gpu_ctx):
    """Loading refuses what the architecture does not have: a DistilBERT
    checkpoint missing its renamed FFN is RH_ERR_MISSING; MPNet texts past
    max_position - 2 are RH_ERR_SEQ (config.go:91-95)."""
    from rembed_amd._lib import RembedError
    from rembed_amd.model import Model
    shape, t, ids, lens = workload("distilbert")
    t1 = {k: v for k, v in t.items() if "ffn.lin1.weight" not in k}
    with pytest.raises(RembedError):
        Model(gpu_ctx, shape, t1, 0)
    shape, t, ids, lens = workload("mpnet")
    m = Model(gpu_ctx, shape, t, 0)
    long_ids = np.full((1, 513), 5, np.int32)
    with pytest.raises(RembedError):
        m.embed(long_ids, np.array([513], np.int32))
    m.close()
