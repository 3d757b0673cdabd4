"""Pins of the oracle's serial float32 orders that the byte-exact device
forward (RH_OPT_EXACT) reproduces.

* dot4 (internal/tensor/dot_amd64.s:13-94) against an instruction-level
  emulation of its assembly: eight-lane VFMADD231PS accumulators, the
  VEXTRACTF128 + VADDPS fold, the scalar VFMADD231SS tail into lane 0, and
  two VHADDPS. A pairwise-fold variant is shown to give different bits on
  the same inputs, so the check separates the orders.
* MatMulSerial's remainder columns (tensor.go:318-328): in-order sums of
  rounded products, against a numpy float32 loop.
* Softmax (tensor.go:389-428) and LayerNorm (tensor.go:430-452) against
  numpy float32 scalar loops written from the Go source, including rows with
  a large mean (where a reordered sum differs) and the -87.33 clamp.
* The composed attention (bert.go:853-902) against float64.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

F = np.float32


def fma32(a, b, c):
    return F(np.float64(a) * np.float64(b) + np.float64(c))  # exact product, one rounding


def dot4_emulated(a, bs):
    """The dot4 instruction sequence on 8-lane float32 vectors."""
    k = a.size
    acc = [np.zeros(8, F) for _ in range(4)]
    nb = k // 8
    for blk in range(nb):
        y4 = a[blk * 8:blk * 8 + 8]
        for q in range(4):
            m = bs[q][blk * 8:blk * 8 + 8]
            acc[q] = np.array([fma32(y4[l], m[l], acc[q][l]) for l in range(8)], F)
    out = []
    for q in range(4):
        x = (acc[q][:4] + acc[q][4:]).astype(F)  # VEXTRACTF128 + VADDPS
        for p in range(nb * 8, k):  # VFMADD231SS into lane 0
            x[0] = fma32(a[p], bs[q][p], x[0])
        h = np.array([x[0] + x[1], x[2] + x[3]], F)  # VHADDPS
        out.append(F(h[0] + h[1]))  # VHADDPS
    return np.array(out, F)


def dot4_pairwise(a, bs):
    """A plausible wrong fold: ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7))."""
    k = a.size
    out = []
    for q in range(4):
        acc = np.zeros(8, F)
        for p in range(k - k % 8):
            acc[p % 8] = fma32(a[p], bs[q][p], acc[p % 8])
        lo = F(F(acc[0] + acc[1]) + F(acc[2] + acc[3]))
        hi = F(F(acc[4] + acc[5]) + F(acc[6] + acc[7]))
        s = F(lo + hi)
        for p in range(k - k % 8, k):
            s = fma32(a[p], bs[q][p], s)
        out.append(s)
    return np.array(out, F)


def test_dot4_matches_instruction_emulation():
    rng = np.random.default_rng(21)
    separated = False
    for k in list(range(1, 41)) + [64, 100, 256]:
        a = rng.standard_normal(k).astype(F)
        bs = [rng.standard_normal(k).astype(F) for _ in range(4)]
        got = np.empty(4, F)
        O.lib.or_dot4(got.ctypes.data, a.ctypes.data, *[b.ctypes.data for b in bs], k)
        want = dot4_emulated(a, bs)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), k
        separated |= not np.array_equal(dot4_pairwise(a, bs), want)
    assert separated, "the inputs do not distinguish the fold orders"


def test_matmul_serial_remainder_columns_are_in_order_sums():
    rng = np.random.default_rng(22)
    for m, k, n in [(3, 64, 7), (5, 33, 6), (2, 129, 5)]:
        a = rng.standard_normal((m, k)).astype(F)
        bT = rng.standard_normal((n, k)).astype(F)
        got = O.matmul_serial(a, bT)
        for j in range(n - n % 4, n):
            for i in range(m):
                s = F(0)
                for p in range(k):
                    s = F(s + F(a[i, p] * bT[j, p]))
                assert got[i, j] == s
        for j in range(0, n - n % 4, 4):
            for i in range(m):
                want = dot4_emulated(a[i], [bT[j + q] for q in range(4)])
                assert np.array_equal(got[i, j:j + 4], want)


def softmax_emulated(row):
    """tensor.go:391-428, float32 scalar by scalar."""
    maxv = row[0]
    for v in row[1:]:
        if v > maxv:
            maxv = v
    out = np.empty_like(row)
    s = F(0)
    for j, v in enumerate(row):
        xe = F(v - maxv)
        if xe < F(-87.33):
            xe = F(-87.33)
        nf = F(int(F(F(xe * F(1.44269504088896341)) - F(0.5))))  # int32() truncates
        xe = F(xe - F(nf * F(0.693359375)))
        xe = F(xe - F(nf * F(-2.12194440e-4)))
        z = F(xe * xe)
        y = F(1.9875691500e-4)
        for c in (1.3981999507e-3, 8.3334519073e-3, 4.1665795894e-2, 1.6666665459e-1,
                  5.0000001201e-1):
            y = F(F(y * xe) + F(c))
        e = F(F(F(F(y * z) + xe) + F(1)) * F(2.0 ** int(nf)))
        out[j] = e
        s = F(s + e)
    inv = F(F(1) / s)
    return (out * inv).astype(F)


def test_softmax_matches_scalar_emulation():
    rng = np.random.default_rng(23)
    rows = [rng.standard_normal(n).astype(F) * F(3) for n in (1, 2, 7, 64, 200)]
    rows.append(np.array([0.0, -100.0, -90.0, 5.0, -87.0], F))  # the clamp at -87.33
    rows.append(np.array([1000.0, 1000.0], F))
    for r in rows:
        got = O.softmax(r[None, :])[0]
        assert np.array_equal(got.view(np.uint32), softmax_emulated(r).view(np.uint32))


def layernorm_emulated(row, g, b, eps):
    """tensor.go:433-452, float32 scalar by scalar."""
    n = row.size
    mean = F(0)
    for v in row:
        mean = F(mean + v)
    mean = F(mean / F(n))
    var = F(0)
    for v in row:
        d = F(v - mean)
        var = F(var + F(d * d))
    var = F(var / F(n))
    inv = F(F(1) / F(math.sqrt(float(F(var + F(eps))))))
    return np.array([F(F(F(F(v - mean) * inv) * g[j]) + b[j]) for j, v in enumerate(row)], F)


def test_layernorm_matches_scalar_emulation_and_order_matters():
    rng = np.random.default_rng(24)
    H = 768
    g = (1 + 0.1 * rng.standard_normal(H)).astype(F)
    b = (0.1 * rng.standard_normal(H)).astype(F)
    x = (rng.standard_normal((6, H)) * 3 + np.array([[0], [40], [-300], [1e3], [0.01], [7]])
         ).astype(F)
    got = O.layernorm(x, g, b, 1e-12)
    reordered = False
    for i in range(x.shape[0]):
        want = layernorm_emulated(x[i], g, b, 1e-12)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), i
        pair = F(x[i].reshape(-1, 2).sum(axis=1, dtype=F).sum(dtype=F))
        seq = F(0)
        for v in x[i]:
            seq = F(seq + v)
        reordered |= pair != seq
    assert reordered, "no row where the summation order changes the mean"


@pytest.mark.parametrize("lens", [[1, 5, 13], [64, 37]])
def test_attention_ref_against_float64(lens):
    rng = np.random.default_rng(25)
    heads, dh = 2, 32
    M = sum(lens)
    qkv = rng.standard_normal((M, 3 * heads * dh)).astype(F)
    scale = 1 / math.sqrt(dh)
    got = O.attention_ref(qkv, lens, heads, dh, scale, 0, heads * dh, 2 * heads * dh)
    r0 = 0
    for L in lens:
        for h in range(heads):
            q = qkv[r0:r0 + L, h * dh:(h + 1) * dh].astype(np.float64)
            k = qkv[r0:r0 + L, (heads + h) * dh:(heads + h + 1) * dh].astype(np.float64)
            v = qkv[r0:r0 + L, (2 * heads + h) * dh:(2 * heads + h + 1) * dh].astype(np.float64)
            s = q @ k.T * scale
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            assert np.abs(got[r0:r0 + L, h * dh:(h + 1) * dh] - p @ v).max() < 2e-6
        r0 += L
