"""Pins of the oracle's DistilBERT and MPNet forwards (bert.go:378-522 names,
bert.go:816-830,876-890 MPNet's relative-position bias).

* relPosBucket (bert.go:123-150) against the reference's own known answers,
  TestRelPosBucket (internal/model/mpnet_test.go:18-38), its range check,
  and HF's relative_position_bucket computed with float32 logs, which the
  reference states picks identical buckets for every |distance| <= 1000.
* Both forwards against an independent float64 numpy composition written
  from bert.go: DistilBERT's renamed tensors and absent token-type row,
  MPNet's position offset (config.go:84-89) and the bias of bucket(j - i)
  added to the scaled scores. A planted wrong sign of the relative position
  (bucket(i - j)) is shown to move the result past the tolerance, so the
  check separates it.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

# internal/model/mpnet_test.go:20-26 — (relative position, bucket) at 32 buckets
REL_POS_KATS = [(-513, 15), (-512, 15), (-129, 15), (-128, 15), (-127, 15),
                (-64, 14), (-17, 10), (-16, 10), (-9, 8), (-8, 8), (-7, 7),
                (-1, 1), (0, 0), (1, 17), (7, 23), (8, 24), (9, 24),
                (16, 26), (17, 26), (64, 30), (127, 31), (128, 31), (129, 31),
                (512, 31), (513, 31)]


def hf_bucket_f32(rel, num_buckets=32, max_distance=128):
    """HF MPNetEncoder.relative_position_bucket with float32 logs."""
    n = -rel
    half = num_buckets // 2
    ret = half if n < 0 else 0
    n = abs(n)
    max_exact = half // 2
    if n < max_exact:
        return ret + n
    f = np.float32
    val = max_exact + int(f(f(np.log(f(n) / f(max_exact))) / f(np.log(f(max_distance / max_exact))))
                          * f(half - max_exact))
    return ret + min(val, half - 1)


def test_rel_pos_bucket_known_answers_and_range():
    for rel, want in REL_POS_KATS:
        assert O.rel_pos_bucket(rel, 32) == want, rel
    for d in range(-1000, 1001):
        b = O.rel_pos_bucket(d, 32)
        assert 0 <= b < 32
        assert b == hf_bucket_f32(d), d


def np_forward(shape, t, ids, rel_sign=1):
    """DistilBERT / MPNet forward in float64 (bert.go:796-918)."""
    from rembed_amd.synthetic import ARCH_MPNET, layer_names
    H, nh = shape.hidden, shape.heads
    dh = H // nh
    L = len(ids)
    g = lambda n: t[n].astype(np.float64)

    def ln(x, gam, bet):
        mu = x.mean(axis=1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
        return (x - mu) / np.sqrt(var + shape.eps) * gam + bet

    off = shape.position_offset
    x = g("embeddings.word_embeddings.weight")[ids] + \
        g("embeddings.position_embeddings.weight")[off:off + L]
    x = ln(x, g("embeddings.LayerNorm.weight"), g("embeddings.LayerNorm.bias"))
    bias = None
    if shape.arch == ARCH_MPNET:
        tab = g("encoder.relative_attention_bias.weight")  # [buckets][heads]
        i = np.arange(L)[:, None]
        j = np.arange(L)[None, :]
        bk = np.vectorize(lambda d: O.rel_pos_bucket(int(d), shape.rel_buckets))(
            rel_sign * (j - i))
        bias = tab[bk]  # [L][L][heads]
    erf = np.vectorize(math.erf)
    for l in range(shape.layers):
        n = layer_names(shape.arch, l)
        q = x @ g(n[0]).T + g(n[1])
        k = x @ g(n[2]).T + g(n[3])
        v = x @ g(n[4]).T + g(n[5])
        ctx = np.zeros_like(x)
        for h in range(nh):
            sl = slice(h * dh, (h + 1) * dh)
            s = q[:, sl] @ k[:, sl].T / math.sqrt(dh)
            if bias is not None:
                s = s + bias[:, :, h]
            s = np.exp(s - s.max(axis=1, keepdims=True))
            s /= s.sum(axis=1, keepdims=True)
            ctx[:, sl] = s @ v[:, sl]
        x = ln(x + ctx @ g(n[6]).T + g(n[7]), g(n[8]), g(n[9]))
        hdn = x @ g(n[10]).T + g(n[11])
        hdn = 0.5 * hdn * (1 + erf(hdn / math.sqrt(2)))
        x = ln(x + hdn @ g(n[12]).T + g(n[13]), g(n[14]), g(n[15]))
    pooled = x.mean(axis=0) if shape.pooling == 0 else x[0]
    return x, pooled / np.linalg.norm(pooled)


def tiny(arch):
    from rembed_amd.synthetic import ARCH_DISTILBERT, BertShape
    if arch == ARCH_DISTILBERT:
        return BertShape("tiny-distil", 2, 64, 2, 128, vocab=500, max_position=64,
                         type_vocab=0, pooling=1, arch=arch)
    return BertShape("tiny-mpnet", 2, 64, 2, 128, vocab=500, max_position=66, type_vocab=0,
                     eps=1e-5, pooling=0, arch=arch, position_offset=2, rel_buckets=32)


@pytest.mark.parametrize("arch", [5, 6], ids=["distilbert", "mpnet"])
def test_oracle_matches_float64_composition(arch):
    from rembed_amd.synthetic import bert_tensors
    shape = tiny(arch)
    t = bert_tensors(shape, seed=30 + arch)
    orc = O.BertOracle(shape, t, 0)
    rng = np.random.default_rng(arch)
    planted_seen = False
    for L in (1, 7, 33, 64):
        ids = rng.integers(0, shape.vocab, size=L).astype(np.int32)
        hid_ref, vec_ref = np_forward(shape, t, ids)
        hid = orc.encode(ids)
        assert np.max(np.abs(hid - hid_ref)) < 2e-5, L
        vec = orc.forward(ids)
        assert np.max(np.abs(vec - vec_ref)) < 1e-5, L
        if arch == 6 and L > 1:
            wrong, _ = np_forward(shape, t, ids, rel_sign=-1)
            planted_seen |= np.max(np.abs(hid - wrong)) > 1e-3
    assert arch != 6 or planted_seen, "the bias direction is not observable"
    orc.close()


def test_mpnet_max_length_is_table_minus_offset():
    from rembed_amd.synthetic import bert_tensors
    shape = tiny(6)
    orc = O.BertOracle(shape, bert_tensors(shape, seed=2), 0)
    ok = orc.encode(np.zeros(shape.max_position - 2, np.int32))
    assert ok.shape[0] == shape.max_position - 2
    with pytest.raises(RuntimeError):
        orc.encode(np.zeros(shape.max_position - 1, np.int32))
    orc.close()
