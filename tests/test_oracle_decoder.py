"""Pins the decoder-family oracle (oracle/oracle_dec.c) without the Go binary.

* RoPE table: float64 closed form; applyRoPE: position 0 is the identity,
  each (d, d + dh/2) pair keeps its norm, and the rotation composes like
  complex multiplication.
* flashAttnCausalHead against a naive float64 causal softmax over the
  sequence lengths of the reference's own test
  (internal/model/qwen3_test.go:49-80), tolerance 1e-4 as there.
* Qwen3 and EmbeddingGemma forwards against independent float64 numpy
  compositions written from internal/model/qwen3.go:395-548 and
  internal/model/gemma3.go:206-384 (exact exp/erf/tanh, no fast math);
  the sliding-window layers are checked with a window shorter than the text
  so the mask matters.
* Mode agreement: weight-only and full int8 stay close to fp32 and are
  actually active; worker count never changes bits.
"""
import dataclasses
import math

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd.synthetic import (ARCH_GEMMA3, GEMMA3_300M, QWEN3_0_6B, decoder_tensors,
                                  token_batch)


def test_rope_table_closed_form():
    seq, dh, theta = 37, 16, 1e4
    c, s = O.rope_table(seq, dh, theta)
    for p in (0, 1, 17, 36):
        for d in range(dh // 2):
            ang = p * theta ** (-2.0 * d / dh)
            assert c[p, d] == np.float32(math.cos(ang))
            assert s[p, d] == np.float32(math.sin(ang))


def test_apply_rope_rotation_properties():
    rng = np.random.default_rng(1)
    seq, dh = 9, 8
    c, s = O.rope_table(seq, dh, 1e4)
    x = rng.standard_normal((seq, dh)).astype(np.float32)
    y = O.apply_rope(x, c, s)
    assert np.array_equal(y[0], x[0])  # angle 0
    h = dh // 2
    n_in = x[:, :h].astype(np.float64) ** 2 + x[:, h:].astype(np.float64) ** 2
    n_out = y[:, :h].astype(np.float64) ** 2 + y[:, h:].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)
    # rotate-half pairing: (x1 + i x2) * e^{i angle}
    z = (x[:, :h] + 1j * x[:, h:]).astype(np.complex128) * (c + 1j * s)
    assert np.allclose(y[:, :h], z.real, atol=1e-6)
    assert np.allclose(y[:, h:], z.imag, atol=1e-6)


@pytest.mark.parametrize("seq", [1, 2, 5, 63, 64, 65, 120, 127, 128, 129, 200])
def test_flash_causal_head_against_float64(seq):
    rng = np.random.default_rng(seq)
    dh = 16
    q = rng.standard_normal((seq, dh)).astype(np.float32)
    k = rng.standard_normal((seq, dh)).astype(np.float32)
    v = rng.standard_normal((seq, dh)).astype(np.float32)
    scale = np.float32(1 / math.sqrt(dh))
    got = O.flash_causal_head(q, k, v, scale)
    s = q.astype(np.float64) @ k.astype(np.float64).T * float(scale)
    s[np.triu_indices(seq, 1)] = -np.inf
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    want = p @ v.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-4


def np_rms(x, g, eps):
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * g


def np_rope(x, pos, dh, theta):
    h = dh // 2
    inv = theta ** (-2.0 * np.arange(h) / dh)
    ang = pos[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[:, :h], x[:, h:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=1)


def np_decoder_forward(shape, t, ids):
    """Qwen3 / EmbeddingGemma in float64 numpy, written from qwen3.go:395-548,
    gemma3.go:206-384 and Forward (bert.go:657-689)."""
    gemma = shape.arch == ARCH_GEMMA3
    g = lambda n: t[n].astype(np.float64)
    off = 1.0 if gemma else 0.0  # Gemma norms scale by (1 + w)
    H, dh, nq, nkv = shape.hidden, shape.head_dim, shape.heads, shape.kv_heads
    L = len(ids)
    pos = np.arange(L, dtype=np.float64)
    x = g("embed_tokens.weight")[ids] * (math.sqrt(H) if gemma else 1.0)
    scale = 1 / math.sqrt(shape.query_pre_attn_scalar if gemma else dh)
    for l in range(shape.layers):
        p = f"layers.{l}."
        glob = (not gemma) or (l + 1) % shape.sliding_pattern == 0
        theta = shape.rope_theta if glob else shape.rope_local_theta
        n = np_rms(x, g(p + "input_layernorm.weight") + off, shape.eps)
        q = n @ g(p + "self_attn.q_proj.weight").T
        k = n @ g(p + "self_attn.k_proj.weight").T
        v = n @ g(p + "self_attn.v_proj.weight").T
        ctx = np.zeros((L, nq * dh))
        for h in range(nq):
            kv = h // (nq // nkv)
            qh = np_rope(np_rms(q[:, h * dh:(h + 1) * dh], g(p + "self_attn.q_norm.weight") + off,
                                shape.eps), pos, dh, theta)
            kh = np_rope(np_rms(k[:, kv * dh:(kv + 1) * dh], g(p + "self_attn.k_norm.weight") + off,
                                shape.eps), pos, dh, theta)
            s = qh @ kh.T * scale
            i, j = np.meshgrid(np.arange(L), np.arange(L), indexing="ij")
            if not gemma:
                s[j > i] = -np.inf
            elif not glob:
                s[np.abs(i - j) >= shape.sliding_window] = -np.inf
            pr = np.exp(s - s.max(axis=1, keepdims=True))
            pr /= pr.sum(axis=1, keepdims=True)
            ctx[:, h * dh:(h + 1) * dh] = pr @ v[:, kv * dh:(kv + 1) * dh]
        a = ctx @ g(p + "self_attn.o_proj.weight").T
        if gemma:
            a = np_rms(a, g(p + "post_attention_layernorm.weight") + off, shape.eps)
        x = x + a
        pre = "pre_feedforward_layernorm.weight" if gemma else "post_attention_layernorm.weight"
        n = np_rms(x, g(p + pre) + off, shape.eps)
        gt = n @ g(p + "mlp.gate_proj.weight").T
        up = n @ g(p + "mlp.up_proj.weight").T
        if gemma:
            act = 0.5 * gt * (1 + np.tanh(math.sqrt(2 / math.pi) * (gt + 0.044715 * gt ** 3)))
        else:
            act = gt / (1 + np.exp(-gt))
        d = (act * up) @ g(p + "mlp.down_proj.weight").T
        if gemma:
            d = np_rms(d, g(p + "post_feedforward_layernorm.weight") + off, shape.eps)
        x = x + d
    x = np_rms(x, g("norm.weight") + off, shape.eps)
    pooled = x[-1] if shape.pooling == 2 else x.mean(axis=0)
    if gemma and shape.dense_hidden:
        pooled = g("3_Dense.linear.weight") @ (g("2_Dense.linear.weight") @ pooled)
    return x, pooled / np.linalg.norm(pooled)


def tiny_qwen3():
    return dataclasses.replace(QWEN3_0_6B, name="tiny-qwen3", layers=2, hidden=64, heads=4,
                               kv_heads=2, head_dim=16, intermediate=96, vocab=300)


def tiny_gemma3():
    return dataclasses.replace(GEMMA3_300M, name="tiny-gemma3", layers=3, hidden=64, heads=3,
                               kv_heads=1, head_dim=32, intermediate=80, vocab=300,
                               sliding_window=6, sliding_pattern=2, query_pre_attn_scalar=32,
                               dense_hidden=96)


@pytest.mark.parametrize("make", [tiny_qwen3, tiny_gemma3])
def test_decoder_oracle_matches_float64_composition(make):
    shape = make()
    t = decoder_tensors(shape, seed=3)
    orc = O.DecoderOracle(shape, t, 0)
    rng = np.random.default_rng(4)
    for L in (1, 5, 17, 70):
        ids = rng.integers(0, shape.vocab, size=L).astype(np.int32)
        hid_ref, vec_ref = np_decoder_forward(shape, t, ids)
        hid = orc.encode(ids)
        assert np.max(np.abs(hid - hid_ref)) < 5e-5 * max(1.0, np.abs(hid_ref).max()), L
        vec = orc.forward(ids)
        assert np.max(np.abs(vec - vec_ref)) < 2e-5, L


def test_gemma_window_mask_is_active():
    """A local layer with a short window must differ from a global one."""
    shape = tiny_gemma3()
    t = decoder_tensors(shape, seed=5)
    ids = np.arange(30, dtype=np.int32) % shape.vocab
    a = O.DecoderOracle(shape, t, 0).forward(ids)
    b = O.DecoderOracle(dataclasses.replace(shape, sliding_pattern=1), t, 0).forward(ids)
    assert np.max(np.abs(a - b)) > 1e-4


@pytest.mark.parametrize("make", [tiny_qwen3, tiny_gemma3])
def test_decoder_oracle_modes_and_batch_policy(make):
    shape = make()
    t = decoder_tensors(shape, seed=8, bf16=True)
    ids, lens = token_batch(5, 40, 2, 40, vocab=shape.vocab, id_lo=0, seed=9)
    outs = {}
    for quant in (0, 1, 2):
        orc = O.DecoderOracle(shape, t, quant)
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
        assert np.max(np.abs(outs[quant] - outs[0])) >= 1e-4


def test_decoder_oracle_rejects_bad_input():
    shape = dataclasses.replace(tiny_qwen3(), max_seq=16)
    orc = O.DecoderOracle(shape, decoder_tensors(shape, seed=1), 0)
    with pytest.raises(RuntimeError):
        orc.forward(np.array([shape.vocab], np.int32))
    with pytest.raises(RuntimeError):
        orc.forward(np.zeros(17, np.int32))
    with pytest.raises(RuntimeError):
        orc.forward(np.zeros(0, np.int32))
