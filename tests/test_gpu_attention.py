"""Softmax attention on the GPU (rh_attention) against a float64 reference.

The per-text head loops it replaces: bert.go:853-902 (bidirectional),
flashAttnCausalHead qwen3.go:319-390 (causal), gemma3.go:318-356 (sliding
window |i-j| < w, grouped kv heads).

* The pipelined bf16 kernel (bf16 q|k|v rows) and the fp32-input kernel at
  precision 1 (which rounds the same values to the same bf16 operands and
  issues the same MFMAs in the same order) agree bit for bit: this pins the
  bf16 kernel's K/V staging, its V^T transposition and key order, the
  block pipeline and the masks against an independently staged kernel.
  Head dim 256 on bf16 rows runs its own 16x16x32 kernel (two waves per
  SIMD), whose products sum in another order: a wrong key order, staging
  or mask there moves the output by O(|v|), far past the bound below.
* Both are within the bf16-P bound of the float64 reference (P is rounded
  to bf16 before P·V: relative 2^-9 per weight), and precision 3 (hi/lo
  split) within 1e-4 of the output scale; so is the pipelined three-term
  kernel fed the rows' bf16 hi/lo planes (rh_attention_planes, dh <= 128).
* Texts of length 1, block edges (63/64/65, 127/128/129), windows shorter
  and longer than the text, GQA groups of 1, 2 and 3, and EmbeddingGemma's
  window of 512 at lengths 511, 512, 513 and 2048.
"""
import sys

import numpy as np
import pytest

from rembed_amd import tensor as T

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def reference(qkv, lens, heads, kv_heads, dh, scale, causal, window, q_off, k_off, v_off):
    """float64 attention per text and head."""
    M = qkv.shape[0]
    out = np.zeros((M, heads * dh), np.float64)
    grp = heads // kv_heads
    r0 = 0
    for L in lens:
        rows = slice(r0, r0 + L)
        i = np.arange(L)[:, None]
        j = np.arange(L)[None, :]
        mask = np.zeros((L, L), bool)
        if causal:
            mask |= j > i
        if window > 0:
            mask |= (j <= i - window) | (j >= i + window)
        for h in range(heads):
            kh = h // grp
            q = qkv[rows, q_off + h * dh: q_off + (h + 1) * dh].astype(np.float64)
            k = qkv[rows, k_off + kh * dh: k_off + (kh + 1) * dh].astype(np.float64)
            v = qkv[rows, v_off + kh * dh: v_off + (kh + 1) * dh].astype(np.float64)
            s = q @ k.T * scale
            s[mask] = -np.inf
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[rows, h * dh:(h + 1) * dh] = p @ v
        r0 += L
    return out


CASES = [
    # dh, heads, kv_heads, causal, window, lens
    (64, 12, 12, False, 0, [1, 5, 63, 64, 65, 130, 200, 256]),
    (32, 4, 2, False, 0, [17, 100, 129]),
    (128, 16, 8, True, 0, [1, 33, 127, 128, 129, 300, 512]),
    (256, 3, 1, False, 257, [5, 300, 600, 1000]),
    (256, 3, 1, False, 0, [70, 333, 700]),
    (128, 4, 4, False, 40, [200, 90]),
    # EmbeddingGemma's local layers at the benchmark's window and length:
    # texts just under, at and over the window, and one of 2048 tokens
    (256, 3, 1, False, 512, [511, 512, 513, 2048]),
]


@pytest.mark.parametrize("case", CASES,
                         ids=["bert64", "dh32-gqa2", "qwen3-causal", "gemma-window",
                              "gemma-global", "dh128-window40", "gemma-window512-2048"])
def test_attention_kernels(gpu_ctx, case):
    dh, heads, kv_heads, causal, window, lens = case
    say(f"attention dh={dh} heads={heads}/{kv_heads} causal={causal} window={window} lens={lens}")
    rng = np.random.default_rng(dh + heads + len(lens))
    M = sum(lens)
    q_off, k_off, v_off = 0, heads * dh, (heads + kv_heads) * dh
    ld = (heads + 2 * kv_heads) * dh
    x = (rng.standard_normal((M, ld)) * 1.5).astype(np.float32)
    bits = to_bf16_bits(x)
    xb = bf16_value(bits)  # exactly bf16-representable fp32 values
    scale = 1.0 / np.sqrt(dh)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cu_d = gpu_ctx.upload(cu)
    max_len = max(lens)

    def run(buf, in_bf16, precision):
        out = gpu_ctx.upload(np.full((M, heads * dh), np.nan, np.float32))
        T.Attention(gpu_ctx, out, heads * dh, buf, in_bf16, ld, q_off, k_off, v_off, cu_d,
                    len(lens), max_len, heads, kv_heads, dh, scale, causal, window, precision)
        gpu_ctx.sync()
        return out.download(np.float32, (M, heads * dh))

    got_bf = run(gpu_ctx.upload(bits), 1, 1)
    got_f1 = run(gpu_ctx.upload(xb), 0, 1)
    got_f3 = run(gpu_ctx.upload(x), 0, 3)
    assert np.all(np.isfinite(got_bf))
    if dh < 256:
        # the pipelined bf16 kernel and the fp32-input kernel run the same
        # 32x32 products in the same order
        diff = np.argwhere(got_bf != got_f1)
        assert diff.size == 0, f"bf16 kernel differs from the fp32-input kernel at {diff[:3].tolist()}"
    # head dim 256 on bf16 rows runs the 16x16x32 kernel (its products sum in
    # another order); it and the fp32-input kernel are held to the bound below

    want_b = reference(xb, lens, heads, kv_heads, dh, scale, causal, window, q_off, k_off, v_off)
    vmax = np.abs(xb[:, v_off:]).max()
    err_b = np.abs(got_bf - want_b).max()
    err_b1 = np.abs(got_f1 - want_b).max()
    say(f"  bf16 max err {err_b:.3e}, fp32-input kernel {err_b1:.3e} (vmax {vmax:.2f})")
    assert err_b <= 2.0 ** -8 * vmax + 1e-5
    assert err_b1 <= 2.0 ** -8 * vmax + 1e-5
    want_f = reference(x, lens, heads, kv_heads, dh, scale, causal, window, q_off, k_off, v_off)
    err_f = np.abs(got_f3 - want_f).max()
    say(f"  split max err {err_f:.3e}")
    assert err_f <= 1e-4 * (1 + np.abs(want_f).max())
    if dh <= 128:
        # the same split handed over as bf16 hi/lo planes (what the full-int8
        # q|k|v projection writes), on the pipelined three-term kernel
        hi = to_bf16_bits(x)
        lo = to_bf16_bits(x - bf16_value(hi))
        out = gpu_ctx.upload(np.full((M, heads * dh), np.nan, np.float32))
        hd, ld_ = gpu_ctx.upload(hi), gpu_ctx.upload(lo)
        T.AttentionPlanes(gpu_ctx, out, heads * dh, hd, ld_, ld, q_off, k_off, v_off, cu_d,
                          len(lens), max_len, heads, kv_heads, dh, scale, causal, window)
        gpu_ctx.sync()
        got_p = out.download(np.float32, (M, heads * dh))
        err_p = np.abs(got_p - want_f).max()
        say(f"  planes max err {err_p:.3e}")
        assert err_p <= 1e-4 * (1 + np.abs(want_f).max())


def test_attention_argument_errors(gpu_ctx):
    from rembed_amd._lib import RembedError
    buf = gpu_ctx.alloc(4096)
    cu = gpu_ctx.upload(np.array([0, 4], np.int32))
    out = gpu_ctx.alloc(4096)
    with pytest.raises(RembedError):  # dh not supported
        T.Attention(gpu_ctx, out, 48, buf, 1, 144, 0, 48, 96, cu, 1, 4, 1, 1, 48, 0.1)
    with pytest.raises(RembedError):  # heads not a multiple of kv_heads
        T.Attention(gpu_ctx, out, 192, buf, 1, 384, 0, 192, 288, cu, 1, 4, 3, 2, 64, 0.1)
    with pytest.raises(RembedError):  # bf16 input at precision 3
        T.Attention(gpu_ctx, out, 64, buf, 1, 192, 0, 64, 128, cu, 1, 4, 1, 1, 64, 0.1,
                    precision=3)


def test_modernbert_window_convention(gpu_ctx):
    """ModernBERT's local layers keep keys within ±w of the query, inclusive
    (masked iff j < i-w or j > i+w, filled with -1e30; modernbert.go:264-273,
    w = LocalAttention/2). rh_attention's window counts |i-j| < window, so the
    ModernBERT layer is window = w + 1. Checked against a float64 restatement
    of ModernBERT's own mask and fill, with texts shorter and longer than
    the window, at w = 64 (LocalAttention 128) and head dim 64."""
    w, dh, heads = 64, 64, 12
    lens = [1, 64, 65, 129, 130, 300]
    say(f"modernbert window ±{w} lens={lens}")
    rng = np.random.default_rng(77)
    M = sum(lens)
    ld = 3 * heads * dh
    q_off, k_off, v_off = 0, heads * dh, 2 * heads * dh
    x = (rng.standard_normal((M, ld)) * 1.5).astype(np.float32)
    scale = 1.0 / np.sqrt(dh)
    want = np.zeros((M, heads * dh), np.float64)
    r0 = 0
    for L in lens:
        i = np.arange(L)[:, None]
        j = np.arange(L)[None, :]
        masked = (j < i - w) | (j > i + w)
        for h in range(heads):
            q = x[r0:r0 + L, q_off + h * dh:q_off + (h + 1) * dh].astype(np.float64)
            k = x[r0:r0 + L, k_off + h * dh:k_off + (h + 1) * dh].astype(np.float64)
            v = x[r0:r0 + L, v_off + h * dh:v_off + (h + 1) * dh].astype(np.float64)
            s = q @ k.T * scale
            s[masked] = -1e30
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            want[r0:r0 + L, h * dh:(h + 1) * dh] = p @ v
        r0 += L
    cu_d = gpu_ctx.upload(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32))
    out = gpu_ctx.upload(np.full((M, heads * dh), np.nan, np.float32))
    T.Attention(gpu_ctx, out, heads * dh, gpu_ctx.upload(x), 0, ld, q_off, k_off, v_off, cu_d,
                len(lens), max(lens), heads, heads, dh, scale, False, w + 1, 3)
    gpu_ctx.sync()
    got = out.download(np.float32, (M, heads * dh))
    err = np.abs(got - want).max()
    say(f"  max err {err:.3e}")
    assert err <= 1e-4 * (1 + np.abs(want).max())
    # the convention matters: one key fewer on each side is a different result
    out2 = gpu_ctx.upload(np.full((M, heads * dh), np.nan, np.float32))
    T.Attention(gpu_ctx, out2, heads * dh, gpu_ctx.upload(x), 0, ld, q_off, k_off, v_off, cu_d,
                len(lens), max(lens), heads, heads, dh, scale, False, w, 3)
    gpu_ctx.sync()
    assert np.abs(out2.download(np.float32, (M, heads * dh)) - want).max() > 1e-3
