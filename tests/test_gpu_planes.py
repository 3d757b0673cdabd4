"""The bf16-planes GEMM path (weight-only int8 and fp32 linears) on the GPU.

* Exact: an fp32 linear whose weight is a permutation matrix (hi = 1 or 0,
  lo = 0) returns, per output, exactly hi(a) + lo(a) of one input element,
  where hi = bf16_rne(a), lo = bf16_rne(a - hi) — the split's rounding and
  every plane index (rows, ragged K, padding, the gather of the permuted
  column) are pinned bit for bit; any other index picks a different element.
* Weight-only int8 with a signed permutation of +-127 entries (scale 1/127)
  gives hi(a) (one activation term, the default) or hi(a)+lo(a) (two) times
  127 times float32(1/127), exactly as the float32 epilogue multiplies.
* Every tile configuration (4- and 8-wave, 256/128 tiles) on a ragged shape.
* Planes vs the in-loop split at encoder and decoder shapes (bias, GELU,
  gated SwiGLU): both hold the split's error bound against float64.
"""
import math
import sys

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd import _lib
from rembed_amd import tensor as T

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf16_rne(x):
    """float32 -> nearest-even bf16, returned as float32 (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def split_sum(a):
    hi = bf16_rne(a)
    lo = bf16_rne((a - hi).astype(np.float32))
    return (hi + lo).astype(np.float32)


def test_bf16_rne_helper_matches_torch():
    """The test's own rounding against torch's bfloat16 cast (nearest-even)."""
    import torch
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-20, 20, 100000))).astype(np.float32)
    x[:4] = [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -1.0 - 2.0 ** -8, 0.0]  # ties
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(bf16_rne(x), want)


def run(ctx, a, pb, bf, act=None):
    ctx.set_bf_algo(bf)
    try:
        return T.matmul_host(ctx, a, pb, act=act)
    finally:
        ctx.set_bf_algo(0)


SHAPES = [(1, 1, 16), (3, 7, 16), (37, 77, 48), (301, 200, 528), (1000, 1024, 256),
          (513, 3072, 1024)]


@pytest.mark.parametrize("bf", [0, 1], ids=["planes", "inloop"])
@pytest.mark.parametrize("shape", SHAPES)
def test_f32_permutation_exact(gpu_ctx, shape, bf):
    m, k, n = shape
    say(f"f32 permutation m={m} k={k} n={n} bf_algo {bf}")
    rng = np.random.default_rng(m + 7 * k + n)
    a = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-3, 3, (m, k)))).astype(np.float32)
    perm = rng.integers(0, k, size=n)
    bT = np.zeros((n, k), np.float32)
    bT[np.arange(n), perm] = 1.0
    pb = T.PackB(gpu_ctx, bT, k, n)
    got = run(gpu_ctx, a, pb, bf)
    want = split_sum(a)[:, perm]
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"first mismatch {bad[:3].tolist()}"
    assert not np.array_equal(want, a[:, perm]) or k < 4  # the split is visible


@pytest.mark.parametrize("terms", [1, 2])
@pytest.mark.parametrize("bf", [0, 1], ids=["planes", "inloop"])
@pytest.mark.parametrize("shape", SHAPES[1:])
def test_w8_signed_permutation_exact(gpu_ctx, shape, bf, terms):
    m, k, n = shape
    say(f"w8 permutation m={m} k={k} n={n} bf_algo {bf} terms {terms}")
    rng = np.random.default_rng(3 * m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    perm = rng.integers(0, k, size=n)
    sign = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    bT = np.zeros((n, k), np.float32)
    bT[np.arange(n), perm] = sign
    pb = T.PackB8(gpu_ctx, bT, k, n)
    q, sc, _ = pb.export()
    assert np.all(np.abs(q[np.arange(n), perm]) == 127)
    gpu_ctx.set_option(_lib.RH_CTX_W8_TERMS, terms)
    try:
        got = run(gpu_ctx, a, pb, bf)
    finally:
        gpu_ctx.set_option(_lib.RH_CTX_W8_TERMS, 1)
    # fp32 accumulator (q·hi or q·(hi+lo), exact), then the float32 scale
    av = bf16_rne(a) if terms == 1 else split_sum(a)
    acc = (av[:, perm] * (127.0 * sign)).astype(np.float32)
    want = (acc * sc[None, :]).astype(np.float32)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"first mismatch {bad[:3].tolist()}"


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("mode,terms", [(_lib.RH_MODE_F32, 2), (_lib.RH_MODE_W8, 1),
                                        (_lib.RH_MODE_W8, 2)], ids=["f32", "w8", "w8-2terms"])
def test_every_planes_tile_exact(gpu_ctx, tile, mode, terms):
    """Each tile configuration on a ragged shape (partial row and column
    tiles), exact through a permutation weight."""
    m, k, n = 700, 1024, 1040
    say(f"planes tile {tile} mode {mode} terms {terms}")
    rng = np.random.default_rng(tile * 10 + mode + terms)
    a = rng.standard_normal((m, k)).astype(np.float32)
    perm = rng.integers(0, k, size=n)
    bT = np.zeros((n, k), np.float32)
    bT[np.arange(n), perm] = 1.0
    pb = T.PackedWeight(gpu_ctx, mode, bT, k, n)
    gpu_ctx.set_option(_lib.RH_CTX_BF_TILE, tile)
    gpu_ctx.set_option(_lib.RH_CTX_W8_TERMS, terms)
    try:
        got = T.matmul_host(gpu_ctx, a, pb)
    finally:
        gpu_ctx.set_option(_lib.RH_CTX_BF_TILE, 0)
        gpu_ctx.set_option(_lib.RH_CTX_W8_TERMS, 1)
    av = split_sum(a) if terms == 2 else bf16_rne(a)
    if mode == _lib.RH_MODE_W8:
        _, sc, _ = pb.export()
        want = ((av[:, perm] * 127.0).astype(np.float32) * sc[None, :]).astype(np.float32)
    else:
        want = av[:, perm]
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"first mismatch {bad[:3].tolist()}"


def bound(a, bT, k, eps, want):
    mag = np.abs(a.astype(np.float64)) @ np.abs(bT.astype(np.float64)).T
    return eps * mag + max(1e-5, 1e-6 * math.sqrt(k)) * (1 + np.abs(want))


@pytest.mark.parametrize("mode", [_lib.RH_MODE_F32, _lib.RH_MODE_W8])
@pytest.mark.parametrize("mkn", [(2048, 768, 3072), (1500, 1024, 2048), (4096, 3072, 1024)])
def test_planes_vs_inloop_linear_gelu(gpu_ctx, mode, mkn):
    m, k, n = mkn
    say(f"planes vs in-loop mode={mode} m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k + n + mode)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bT = (rng.standard_normal((n, k)) * 0.03).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    pb = T.PackedWeight(gpu_ctx, mode, bT, k, n, bias=bias)
    outs = [run(gpu_ctx, a, pb, bf, act=_lib.RH_ACT_GELU) for bf in (0, 1)]
    # float64 reference on a row sample, GELU applied by the oracle
    rows = rng.choice(m, size=64, replace=False)
    if mode == _lib.RH_MODE_W8:  # one bf16 activation term (the default)
        q, sc, _ = pb.export()
        w = q.astype(np.float64) * sc.astype(np.float64)[:, None]
        eps = 2.0 ** -8
    else:
        w = bT.astype(np.float64)
        eps = 2.0 ** -14
    pre = a[rows].astype(np.float64) @ w.T + bias
    want = O.gelu_ref(pre.astype(np.float32)).astype(np.float64)
    # GELU is 1.13-Lipschitz: the pre-activation bound carries over with margin
    b = 1.2 * bound(a[rows], w, k, eps, pre) + 1e-6
    for bf, got in zip((0, 1), outs):
        err = np.abs(got[rows] - want)
        say(f"  bf_algo {bf}: max err {err.max():.3e} worst err/bound {(err / b).max():.3f}")
        assert np.all(err <= b)
    assert np.all(np.isfinite(outs[0]))
