"""Pins the nomic-embed / ModernBERT oracle (oracle/oracle_renc.c) without
the Go binary or real checkpoints (the reference's goldens for these two,
testdata/golden-nomic-embed-text-v1.5.json and
golden-modernbert-embed-base.json, need the real weights).

* Both forwards against independent float64 numpy compositions written from
  internal/model/nomic.go:113-250 and internal/model/modernbert.go:148-311
  (exact erf / exp, no fast math), with texts longer than ModernBERT's
  local window so the mask matters.
* Planted variants of that float64 composition — the mistakes a restatement
  could plausibly make (fc11 / fc12 swapped, the GeGLU halves swapped,
  the segment row dropped, interleaved RoPE pairs, the window bound
  exclusive, the global-layer schedule shifted, the RoPE thetas swapped,
  layer 0's identity attention norm replaced by a LayerNorm) — must each
  disagree with the oracle far beyond the tolerance.
* Mode agreement, batch policy and input refusal as for the other oracles.
"""
import dataclasses
import math

import numpy as np
import pytest
from scipy.special import erf

from oracle import oracle as O
from rembed_amd.synthetic import (ARCH_MODERNBERT, MODERNBERT_BASE, NOMIC_V15,
                                  rope_encoder_tensors, token_batch)


def np_ln(x, g, b, eps):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def np_rope(x, pos, dh, theta, interleaved=False):
    h = dh // 2
    inv = theta ** (-2.0 * np.arange(h) / dh)
    ang = pos[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    if interleaved:
        x1, x2 = x[:, 0::2], x[:, 1::2]
        out = np.empty_like(x)
        out[:, 0::2] = x1 * c - x2 * s
        out[:, 1::2] = x2 * c + x1 * s
        return out
    x1, x2 = x[:, :h], x[:, h:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=1)


def gelu(v):
    return 0.5 * v * (1 + erf(v / math.sqrt(2)))


def silu(v):
    return v / (1 + np.exp(-v))


def np_attention(qkv, H, heads, theta, window, interleaved=False):
    """Bidirectional softmax attention with RoPE on q and k; window w keeps
    keys with |i - j| <= w (None: all keys)."""
    L = qkv.shape[0]
    dh = H // heads
    pos = np.arange(L, dtype=np.float64)
    ctx = np.zeros((L, H))
    i, j = np.meshgrid(np.arange(L), np.arange(L), indexing="ij")
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        q = np_rope(qkv[:, sl], pos, dh, theta, interleaved)
        k = np_rope(qkv[:, H:][:, sl], pos, dh, theta, interleaved)
        v = qkv[:, 2 * H:][:, sl]
        s = q @ k.T / math.sqrt(dh)
        if window is not None:
            s[np.abs(i - j) > window] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ctx[:, sl] = p @ v
    return ctx


def np_nomic(shape, t, ids, mistake=None):
    """nomic-embed in float64, from nomic.go:113-250 and bert.go:657-689."""
    g = lambda n: t[n].astype(np.float64)
    H, I, eps = shape.hidden, shape.intermediate, shape.eps
    x = g("embeddings.word_embeddings.weight")[ids]
    if mistake != "no_segment_row":
        x = x + g("embeddings.token_type_embeddings.weight")[0]
    x = np_ln(x, g("emb_ln.weight"), g("emb_ln.bias"), eps)
    for l in range(shape.layers):
        p = f"encoder.layers.{l}."
        qkv = x @ g(p + "attn.Wqkv.weight").T
        ctx = np_attention(qkv, H, shape.heads, shape.rope_theta, None,
                           interleaved=mistake == "interleaved_rope")
        x = np_ln(x + ctx @ g(p + "attn.out_proj.weight").T, g(p + "norm1.weight"),
                  g(p + "norm1.bias"), eps)
        f11 = x @ g(p + "mlp.fc11.weight").T
        f12 = x @ g(p + "mlp.fc12.weight").T
        act = f12 * silu(f11) if mistake == "swap_fc11_fc12" else f11 * silu(f12)
        x = np_ln(x + act @ g(p + "mlp.fc2.weight").T, g(p + "norm2.weight"),
                  g(p + "norm2.bias"), eps)
    return x


def np_modernbert(shape, t, ids, mistake=None):
    """ModernBERT in float64, from modernbert.go:148-311."""
    g = lambda n: t[n].astype(np.float64)
    H, I, eps = shape.hidden, shape.intermediate, shape.eps
    zero = np.zeros(H)
    x = np_ln(g("embeddings.tok_embeddings.weight")[ids], g("embeddings.norm.weight"), zero, eps)
    w = shape.local_attention // 2 - (1 if mistake == "exclusive_window" else 0)
    for l in range(shape.layers):
        p = f"layers.{l}."
        sched = l + 1 if mistake == "shifted_schedule" else l
        glob = sched % shape.global_every == 0
        thetas = (shape.rope_theta, shape.rope_local_theta)
        if mistake == "swapped_thetas":
            thetas = thetas[::-1]
        theta = thetas[0] if glob else thetas[1]
        if l:
            n = np_ln(x, g(p + "attn_norm.weight"), zero, eps)
        elif mistake == "layer0_norm":
            n = np_ln(x, np.ones(H), zero, eps)
        else:
            n = x
        ctx = np_attention(n @ g(p + "attn.Wqkv.weight").T, H, shape.heads, theta,
                           None if glob else w)
        x = x + ctx @ g(p + "attn.Wo.weight").T
        wi = np_ln(x, g(p + "mlp_norm.weight"), zero, eps) @ g(p + "mlp.Wi.weight").T
        a, b = wi[:, :I], wi[:, I:]
        act = gelu(b) * a if mistake == "swap_geglu" else gelu(a) * b
        x = x + act @ g(p + "mlp.Wo.weight").T
    return np_ln(x, g("final_norm.weight"), zero, eps)


def tiny_nomic():
    return dataclasses.replace(NOMIC_V15, name="tiny-nomic", layers=2, hidden=64, heads=4,
                               intermediate=96, vocab=300)


def tiny_modernbert():
    # four layers so global_every 3 gives global 0, 3 and local 1, 2; window ±4
    return dataclasses.replace(MODERNBERT_BASE, name="tiny-modernbert", layers=4, hidden=64,
                               heads=4, intermediate=80, vocab=300, local_attention=8)


def np_forward(shape, t, ids, mistake=None):
    f = np_modernbert if shape.arch == ARCH_MODERNBERT else np_nomic
    x = f(shape, t, ids, mistake)
    pooled = x.mean(axis=0)
    return x, pooled / np.linalg.norm(pooled)


LENGTHS = (1, 5, 17, 40)
STD = 0.1  # weights large enough on hidden 64 that every sublayer moves the output


@pytest.mark.parametrize("make", [tiny_nomic, tiny_modernbert])
def test_renc_oracle_matches_float64_composition(make):
    shape = make()
    t = rope_encoder_tensors(shape, seed=3, std=STD)
    orc = O.RopeEncoderOracle(shape, t, 0)
    rng = np.random.default_rng(4)
    for L in LENGTHS:
        ids = rng.integers(0, shape.vocab, size=L).astype(np.int32)
        hid_ref, vec_ref = np_forward(shape, t, ids)
        hid = orc.encode(ids)
        assert np.max(np.abs(hid - hid_ref)) < 5e-5 * max(1.0, np.abs(hid_ref).max()), L
        vec = orc.forward(ids)
        assert np.max(np.abs(vec - vec_ref)) < 2e-5, L


PLANTED = {
    "nomic": ["swap_fc11_fc12", "no_segment_row", "interleaved_rope"],
    "modernbert": ["exclusive_window", "shifted_schedule", "swapped_thetas", "swap_geglu",
                   "layer0_norm"],
}


@pytest.mark.parametrize("make,mistake",
                         [(tiny_nomic, m) for m in PLANTED["nomic"]] +
                         [(tiny_modernbert, m) for m in PLANTED["modernbert"]])
def test_renc_planted_mistakes_are_caught(make, mistake):
    """Each plausible restatement mistake moves the float64 forward far past
    the tolerance the oracle is held to above."""
    shape = make()
    t = rope_encoder_tensors(shape, seed=3, std=STD)
    orc = O.RopeEncoderOracle(shape, t, 0)
    ids = np.random.default_rng(6).integers(0, shape.vocab, size=40).astype(np.int32)
    bad, _ = np_forward(shape, t, ids, mistake)
    hid = orc.encode(ids)
    assert np.max(np.abs(hid - bad)) > 50 * 5e-5 * max(1.0, np.abs(bad).max()), mistake


@pytest.mark.parametrize("make", [tiny_nomic, tiny_modernbert])
def test_renc_oracle_modes_and_batch_policy(make):
    shape = make()
    t = rope_encoder_tensors(shape, seed=8, std=STD)
    ids, lens = token_batch(5, 40, 2, 40, vocab=shape.vocab, id_lo=0, seed=9)
    outs = {}
    for quant in (0, 1, 2):
        orc = O.RopeEncoderOracle(shape, t, quant)
        assert orc.quantized_kind() == quant
        b1 = orc.embed_batch(ids, lens, threads=1)
        b4 = orc.embed_batch(ids, lens, threads=4)
        assert np.array_equal(b1, b4)
        single = np.stack([orc.forward(ids[b, :lens[b]]) for b in range(len(lens))])
        assert np.array_equal(b1, single)
        outs[quant] = b1
    for quant, floor in ((1, 0.999), (2, 0.98)):
        cos = np.sum(outs[quant].astype(np.float64) * outs[0], axis=1)
        assert np.all(cos >= floor), (quant, cos.min())
        assert np.max(np.abs(outs[quant] - outs[0])) >= 1e-5


@pytest.mark.parametrize("make", [tiny_nomic, tiny_modernbert])
def test_renc_oracle_rejects_bad_input(make):
    shape = dataclasses.replace(make(), max_seq=16)
    orc = O.RopeEncoderOracle(shape, rope_encoder_tensors(shape, seed=1), 0)
    with pytest.raises(RuntimeError):
        orc.forward(np.array([shape.vocab], np.int32))
    with pytest.raises(RuntimeError):
        orc.forward(np.zeros(17, np.int32))
    with pytest.raises(RuntimeError):
        orc.forward(np.zeros(0, np.int32))
