"""The byte-exact BERT-family forward (RH_OPT_EXACT) on the GPU against the
oracle, bit for bit.

* rh_attention at precision 4 (the reference's float32 order:
  MatMulSerial's dot4 and remainder columns, Softmax; bert.go:853-902)
  equals the oracle's per-head composition, over text lengths that hit
  every dot4 remainder (L % 4, L % 8), the 64-key chunk edges, a one-token
  text, and head dims 32, 64 and 128.
* rh_layernorm equals the oracle's LayerNorm (tensor.go:433-452) at the
  encoder widths, on rows with large means where the sum order shows.
* A full-int8 BERT-base-shaped encoder (12 layers) and a MiniLM-shaped one
  with RH_OPT_EXACT: the final hidden states of every text, their u8 rows
  (the int8 GEMMs' inputs) and the pooled, normalized vectors equal the
  oracle's per-text forward, on one and on two streams.
"""
import math
import sys

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd import tensor as T

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("dh,heads,lens", [
    (64, 12, [1, 5, 63, 64, 65, 130, 200, 256]),
    (32, 4, [7, 17, 100, 129]),
    (128, 2, [3, 66, 127, 250]),
], ids=["dh64", "dh32", "dh128"])
def test_attention_reference_order(gpu_ctx, dh, heads, lens):
    say(f"exact attention dh={dh} heads={heads} lens={lens}")
    rng = np.random.default_rng(dh * 7 + heads)
    M = sum(lens)
    ld = 3 * heads * dh
    qkv = (rng.standard_normal((M, ld)) * 1.5).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    scale = np.float32(1.0 / math.sqrt(dh))
    out = gpu_ctx.upload(np.full((M, heads * dh), np.nan, np.float32))
    T.Attention(gpu_ctx, out, heads * dh, gpu_ctx.upload(qkv), 0, ld, 0, heads * dh,
                2 * heads * dh, gpu_ctx.upload(cu), len(lens), max(lens), heads, heads, dh,
                float(scale), False, 0, 4)
    gpu_ctx.sync()
    got = out.download(np.float32, (M, heads * dh))
    want = O.attention_ref(qkv, lens, heads, dh, scale, 0, heads * dh, 2 * heads * dh)
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} values differ, first at {bad[:3].tolist()}"


def test_attention_reference_order_refusals(gpu_ctx):
    from rembed_amd._lib import RembedError
    buf = gpu_ctx.alloc(1 << 16)
    cu = gpu_ctx.upload(np.array([0, 4], np.int32))
    out = gpu_ctx.alloc(1 << 16)
    with pytest.raises(RembedError):  # causal mask
        T.Attention(gpu_ctx, out, 64, buf, 0, 192, 0, 64, 128, cu, 1, 4, 1, 1, 64, 0.1,
                    True, 0, 4)
    with pytest.raises(RembedError):  # grouped kv heads
        T.Attention(gpu_ctx, out, 128, buf, 0, 256, 0, 128, 192, cu, 1, 4, 2, 1, 64, 0.1,
                    False, 0, 4)
    with pytest.raises(RembedError):  # bf16 input
        T.Attention(gpu_ctx, out, 64, buf, 1, 192, 0, 64, 128, cu, 1, 4, 1, 1, 64, 0.1,
                    False, 0, 4)


@pytest.mark.parametrize("H", [384, 768, 1024])
def test_layernorm_bit_identical(gpu_ctx, H):
    rng = np.random.default_rng(H)
    m = 37
    x = (rng.standard_normal((m, H)) * 3 + rng.choice([0, 40, -300, 1e3], size=(m, 1))
         ).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    b = (0.1 * rng.standard_normal(H)).astype(np.float32)
    xd, gd, bd = gpu_ctx.upload(x), gpu_ctx.upload(g), gpu_ctx.upload(b)
    from rembed_amd._lib import check, lib
    check(lib.rh_layernorm(gpu_ctx.h, xd.ptr, gd.ptr, bd.ptr, m, H, np.float32(1e-12)))
    gpu_ctx.sync()
    got = xd.download(np.float32, (m, H))
    assert bits_equal(got, O.layernorm(x, g, b, 1e-12))


def _u8(rows):
    return np.stack([O.quantize_row_u8(r)[0] for r in rows])


@pytest.mark.parametrize("which", ["minilm", "bert-base"])
def test_full_int8_forward_byte_identical(gpu_ctx, which):
    from rembed_amd import synthetic as S
    from rembed_amd.model import Model
    # enough tokens (> 4096) that two streams split the batch into two parts
    if which == "minilm":
        shape = S.MINILM_L6
        ids, lens = S.token_batch(64, 128, 16, 128, seed=0x5EED0002)
    else:
        shape = S.BERT_BASE
        ids, lens = S.token_batch(28, 256, 64, 256, seed=0x5EED0002)
    t = S.bert_tensors(shape, seed=0x5EED0001)
    say(f"exact forward {which}: {len(lens)} texts, {int(lens.sum())} tokens")
    orc = O.BertOracle(shape, t, 2)
    want_h = [orc.encode(ids[b, :lens[b]]) for b in range(len(lens))]
    want_v = orc.embed_batch(ids, lens, threads=8)
    orc.close()
    m = Model(gpu_ctx, shape, t, 2)
    m.set_exact(True)
    for streams in (1, 2):
        m.set_streams(streams)
        toks = m.embed_tokens(ids, lens)
        vec = m.embed(ids, lens)
        for b in range(len(lens)):
            assert bits_equal(toks[b], want_h[b]), f"text {b} hidden states, {streams} streams"
            assert np.array_equal(_u8(toks[b]), _u8(want_h[b]))
        assert bits_equal(vec, want_v), f"vectors, {streams} streams"
    m.close()
