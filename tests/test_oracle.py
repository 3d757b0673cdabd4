"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each check is independent of the oracle's own formula: the reference's
known answers (tests/golden/reference_kats.json), closed forms restated
here in numpy / exact rationals, float64 brute force, and invariants chosen
so that a dropped term, a wrong sign or index or a transposed operand fails.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_kats.json")))


# ---- exact float32 arithmetic helpers ---------------------------------------------

def round_f32(fr: Fraction) -> np.float32:
    """Correctly rounded (nearest-even) float32 of an exact rational."""
    x = np.float32(float(fr))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - fr)
        key = (d, int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def fma32(a, b, c):
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


# ---- quantizers ----------------------------------------------------------------------

def test_quantize_row_u8_reference_kat():
    k = KATS["quantize_row_u8_rails"]
    dst, s = O.quantize_row_u8(np.array(k["a"], np.float32), k["dstlen"])
    for i, v in k["want_prefix"].items():
        assert dst[int(i)] == v
    lo, hi = k["want_tail_zero"]
    assert np.all(dst[lo:hi + 1] == 0)
    assert s != 0
    # 63.5 * (1/1) rounds half to even -> 64 -> u8 192
    assert dst[3] == 192
    _, s0 = O.quantize_row_u8(np.array(k["zero_row"], np.float32))
    assert s0 == k["zero_row_scale"]


def np_quantize_rows(a):
    """QuantizeRowU8 restated with numpy float32 ops (pack_vnni.go:85-117)."""
    a = a.astype(np.float32)
    mx = np.abs(a).max(axis=1)
    s = (mx / np.float32(127)).astype(np.float32)
    s[s == 0] = np.float32(1)
    inv = (np.float32(1) / s).astype(np.float32)
    prod = (a * inv[:, None]).astype(np.float32)
    q = np.rint(prod.astype(np.float64)).astype(np.int64) + 128
    return np.clip(q, 0, 255).astype(np.uint8), s


def np_pack_vnni(bT):
    """PackB8VNNI / vnniReference restated (pack_vnni.go:48-76, vnni_test.go:17-33)."""
    b = bT.astype(np.float64)
    scale = np.abs(b).max(axis=1) / 127.0
    scale[scale == 0] = 1.0
    q = np.rint(b / scale[:, None]).astype(np.int64).astype(np.int8)
    colsum = q.astype(np.int64).sum(axis=1)
    colsum = ((colsum + 2**31) % 2**32 - 2**31).astype(np.int32)
    return q, scale.astype(np.float32), colsum


def vnni_case(rng, m, k, n):
    a = (rng.random((m, k), dtype=np.float32) * 4 - 2).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    if k > 2:
        a[0, :3] = KATS["vnni_exact_shapes"]["rail_row"]
    return a, bT


@pytest.mark.parametrize("shape", KATS["vnni_exact_shapes"]["shapes"])
def test_vnni_oracle_matches_closed_form(shape):
    m, k, n = shape
    rng = np.random.default_rng(99 + m * 7 + k)
    a, bT = vnni_case(rng, m, k, n)
    st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
    assert st == 0
    q_ref, sc_ref, cs_ref = np_pack_vnni(bT)
    assert np.array_equal(q, q_ref)
    assert np.array_equal(sc, sc_ref)
    assert np.array_equal(cs, cs_ref)
    dst, qa, rs, acc = O.matmul_vnni(a, q, cs, sc)
    qa_ref, rs_ref = np_quantize_rows(a)
    assert np.array_equal(qa, qa_ref)
    assert np.array_equal(rs, rs_ref)
    # integer accumulators by int64 brute force, wrapped to int32
    acc_ref = qa_ref.astype(np.int64) @ q_ref.astype(np.int64).T
    acc_ref = ((acc_ref + 2**31) % 2**32 - 2**31).astype(np.int32)
    assert np.array_equal(acc, acc_ref)
    real = (acc_ref.astype(np.int64) - 128 * cs_ref.astype(np.int64)[None, :])
    real = ((real + 2**31) % 2**32 - 2**31).astype(np.float32)
    want = ((real * rs_ref[:, None]).astype(np.float32) * sc_ref[None, :]).astype(np.float32)
    assert np.array_equal(dst, want)
    # the zero-point correction is what makes u8 accumulation equal the
    # signed product: real == (qa-128)·q exactly
    signed = (qa_ref.astype(np.int64) - 128) @ q_ref.astype(np.int64).T
    assert np.array_equal(real.astype(np.int64), signed)


def test_gemm_u8s8_vnni_body_matches_portable():
    """The AVX-512-VNNI body and the portable C body give the same integers."""
    rng = np.random.default_rng(7)
    for kg in (1, 2, 13, 96, 384):
        k = kg * 4
        qa = rng.integers(0, 256, size=(5, k)).astype(np.uint8)
        q = rng.integers(-128, 128, size=(17, k)).astype(np.int8)
        got = O.gemm_u8s8_i32(qa, q)
        ref = qa.astype(np.int64) @ q.astype(np.int64).T
        ref = ((ref + 2**31) % 2**32 - 2**31).astype(np.int32)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("m,k,n", [(13, 129, 64), (7, 384, 384), (64, 768, 2304),
                                   (5, 3, 16), (33, 1000, 32), (1, 3072, 768)])
def test_vnni_panel_kernel_matches_brute_force(m, k, n):
    """The reference's kernel shape (PackB8VNNI panels, 4x16 VPDPBUSD tiles
    with broadcast activation groups, zero past k and past m) gives the
    wrapping int64-brute-force sums and the default oracle body's integers;
    the portable tile agrees. A transposed panel index, a dropped k-group or
    a wrong row panel breaks the first check."""
    rng = np.random.default_rng(m * 7 + k + n)
    q = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
    kg = (k + 3) // 4
    qa = np.zeros((m, kg * 4), np.uint8)
    qa[:, :k] = rng.integers(0, 256, size=(m, k))
    pb = O.pack_vnni_panels(q)
    # the layout itself: column c, k index p at (c//16)*kg*64 + (p//4)*64 + (c%16)*4 + p%4
    c, pk = rng.integers(0, n), rng.integers(0, k)
    assert pb[(c // 16) * kg * 64 + (pk // 4) * 64 + (c % 16) * 4 + pk % 4] == q[c, pk]
    got = O.gemm_u8s8_panels(qa, pb, k, n)
    ref = qa[:, :k].astype(np.int64) @ q.astype(np.int64).T
    ref = ((ref + 2**31) % 2**32 - 2**31).astype(np.int32)
    assert np.array_equal(got, ref)
    assert np.array_equal(got, O.gemm_u8s8_i32(np.ascontiguousarray(qa[:, :k]), q))


def test_vnni_panel_kernel_portable_body():
    """The scalar 4x16 tile (hosts without VNNI) gives the same integers,
    run in a fresh process so the CPU dispatch is decided again."""
    import subprocess
    import sys
    code = (
        "import numpy as np\n"
        "from oracle import oracle as O\n"
        "assert O.lib.or_vnni_panel_kind() == 0\n"
        "rng = np.random.default_rng(3)\n"
        "q = rng.integers(-128, 128, size=(48, 200)).astype(np.int8)\n"
        "qa = rng.integers(0, 256, size=(9, 200)).astype(np.uint8)\n"
        "got = O.gemm_u8s8_panels(qa, O.pack_vnni_panels(q), 200, 48)\n"
        "ref = qa.astype(np.int64) @ q.astype(np.int64).T\n"
        "ref = ((ref + 2**31) % 2**32 - 2**31).astype(np.int32)\n"
        "assert np.array_equal(got, ref)\n")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, OR_FORCE_PORTABLE="1", PYTHONPATH=root)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_pack_b8_error_bound_and_zero_channel():
    kk = KATS["pack_b8_error"]
    k, n = kk["k"], kk["n"]
    rng = np.random.default_rng(29)
    bT = ((rng.random((n, k), dtype=np.float32) * 2 - 1) *
          np.exp(rng.integers(0, 6, size=(n, k))).astype(np.float32)).astype(np.float32)
    bT[n // 2] = 0
    st, q, sc = O.pack_b8(bT, k, n)
    assert st == 0
    assert sc[n // 2] == 1.0 and np.all(q[n // 2] == 0)
    mx = np.abs(bT.astype(np.float64)).max(axis=1)
    deq = q.astype(np.float64) * sc.astype(np.float64)[:, None]
    assert np.all(np.abs(deq - bT) <= mx[:, None] / 254 + 1e-9)
    # float32 scale (pack8.go:53), not the float64 one of PackB8VNNI
    want_sc = (np.abs(bT).max(axis=1).astype(np.float32) / np.float32(127)).astype(np.float32)
    want_sc[want_sc == 0] = 1
    assert np.array_equal(sc, want_sc)


def test_pack_rejects_nonfinite_and_bad_shapes():
    bT = np.zeros((16, 4), np.float32)
    bT[1, 3] = np.nan
    assert O.pack_b8(bT, 4, 16)[0] == 2
    assert O.pack_b8_vnni(bT, 4, 16)[0] == 2
    bT[1, 3] = np.inf
    assert O.pack_b8(bT, 4, 16)[0] == 2
    assert O.pack_b8(np.zeros((15, 3), np.float32), 3, 15)[0] == 1
    assert O.pack_b8_vnni(np.zeros((16, 1), np.float32), 0, 16)[0] == 1


# ---- GEMMs -------------------------------------------------------------------------------

def test_matmul_naive_kat():
    kk = KATS["matmul_naive_small"]
    a = np.array(kk["a"], np.float32).reshape(kk["m"], kk["k"])
    bT = np.array(kk["bT"], np.float32).reshape(kk["n"], kk["k"])
    assert np.array_equal(O.matmul_f32(a, bT).ravel(), np.array(kk["want"], np.float32))


def test_matmul_f32_is_sequential_fma_chain():
    """Per element: acc=+0, acc=fma(a[p],b[p],acc) ascending (gemm_amd64.s:31-49)."""
    rng = np.random.default_rng(5)
    m, k, n = 3, 7, 16
    a = rng.standard_normal((m, k)).astype(np.float32)
    bT = rng.standard_normal((n, k)).astype(np.float32)
    got = O.matmul_f32(a, bT)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0)
            for p in range(k):
                acc = fma32(a[i, p], bT[j, p], acc)
            assert got[i, j] == acc, (i, j)


def test_matmul_w8_is_fma_chain_then_scale():
    rng = np.random.default_rng(6)
    m, k, n = 2, 9, 16
    a = rng.standard_normal((m, k)).astype(np.float32)
    bT = rng.standard_normal((n, k)).astype(np.float32)
    st, q, sc = O.pack_b8(bT, k, n)
    got = O.matmul_w8(a, q, sc)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0)
            for p in range(k):
                acc = fma32(a[i, p], np.float32(q[j, p]), acc)
            assert got[i, j] == np.float32(acc * sc[j]), (i, j)


@pytest.mark.parametrize("shape", KATS["packed_f32_shapes"]["shapes"])
def test_matmul_f32_and_w8_against_float64(shape):
    m, k, n = shape
    rng = np.random.default_rng(11 + k)
    a = (rng.random((m, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    tol = max(1e-5, 1e-6 * math.sqrt(k))
    want = a.astype(np.float64) @ bT.astype(np.float64).T
    got = O.matmul_f32(a, bT)
    assert np.all(np.abs(got - want) <= tol * (1 + np.abs(want)))
    bT[n // 2] = 0
    st, q, sc = O.pack_b8(bT, k, n)
    deq = q.astype(np.float64) * sc.astype(np.float64)[:, None]
    want8 = a.astype(np.float64) @ deq.T
    got8 = O.matmul_w8(a, q, sc)
    assert np.all(np.abs(got8 - want8) <= tol * (1 + np.abs(want8)))


def test_dot4_against_float64_and_tail_order():
    rng = np.random.default_rng(13)
    for k in range(1, 41):
        a = rng.standard_normal(k).astype(np.float32)
        bs = [rng.standard_normal(k).astype(np.float32) for _ in range(4)]
        dst = np.empty(4, np.float32)
        O.lib.or_dot4(dst.ctypes.data, a.ctypes.data, *[b.ctypes.data for b in bs], k)
        for q in range(4):
            want = float(a.astype(np.float64) @ bs[q].astype(np.float64))
            assert abs(dst[q] - want) <= 1e-5 * (1 + abs(want))
        if k < 8:  # no vector body: one fma chain into lane 0
            for q in range(4):
                acc = np.float32(0)
                for p in range(k):
                    acc = fma32(a[p], bs[q][p], acc)
                assert dst[q] == acc


# ---- elementwise -------------------------------------------------------------------------

def test_softmax_kat():
    kk = KATS["softmax"]
    x = O.rowwise(O.lib.or_softmax, np.array(kk["x"], np.float32), 2, 3)
    e = np.exp([1.0, 2.0, 3.0])
    want = np.concatenate([e / e.sum(), [1 / 3] * 3])
    assert np.max(np.abs(x - want)) <= kk["tol"]
    y = O.rowwise(O.lib.or_softmax, np.array(kk["large"], np.float32), 1, 2)
    assert np.max(np.abs(y - kk["large_want"])) <= kk["tol"]


def test_layernorm_kat():
    kk = KATS["layernorm"]
    inv = 1 / math.sqrt(2 / 3)
    x = O.layernorm(np.array([kk["x"]], np.float32), [1, 1, 1], [0, 0, 0], 0.0)
    assert np.max(np.abs(x[0] - [-inv, 0, inv])) <= kk["tol"]
    x2 = O.layernorm(np.array([kk["x"]], np.float32), kk["affine_gamma"],
                     kk["affine_beta"], 0.0)
    assert np.max(np.abs(x2[0] - [1 - 2 * inv, 1, 1 + 2 * inv])) <= kk["tol"]


def test_l2_and_bias_kats():
    kk = KATS["l2normalize"]
    x = O.rowwise(O.lib.or_l2normalize, np.array(kk["x"], np.float32), 2)
    assert np.max(np.abs(x - kk["want"])) <= kk["tol"]
    z = O.rowwise(O.lib.or_l2normalize, np.array(kk["zero"], np.float32), 2)
    assert np.array_equal(z, [0, 0])
    kb = KATS["add_bias_add"]
    bias = np.array(kb["bias"], np.float32)
    x = O.rowwise(O.lib.or_add_bias, np.array(kb["x"], np.float32), bias.ctypes.data, 2, 2)
    assert np.array_equal(x, kb["want_bias"])
    add = np.array(kb["add"], np.float32)
    y = O.rowwise(O.lib.or_add, x, add.ctypes.data, 4)
    assert np.array_equal(y, kb["want_add"])


def test_gelu_and_tanh_against_float64():
    kk = KATS["gelu_range"]
    xs = np.arange(kk["lo"], kk["hi"] + 1e-9, kk["step"], dtype=np.float32)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(np.float64)])
    assert np.max(np.abs(O.gelu(xs) - want)) <= kk["tol"]
    c = 0.7978845608028654
    want_t = np.array([0.5 * v * (1 + math.tanh(c * (v + 0.044715 * v ** 3)))
                       for v in xs.astype(np.float64)])
    got_t = O.rowwise(O.lib.or_gelu_tanh, xs, xs.size)
    assert np.max(np.abs(got_t - want_t)) <= kk["tol"]
    silu = O.rowwise(O.lib.or_silu, xs, xs.size)
    want_s = xs.astype(np.float64) / (1 + np.exp(-xs.astype(np.float64)))
    assert np.max(np.abs(silu - want_s)) <= 1e-6


def test_gelu_avx2_restatement_tracks_scalar():
    """TestGELUVectorMatchesScalar (internal/tensor/tensor_test.go:220-251):
    the fused AVX2 sequence stays within 1e-6 of geluScalar over the range,
    the clamp region and signed zeros, for every length class; and within
    1e-6 of the float64 erf-GELU (tensor_test.go:186-200)."""
    base = list(np.arange(-30, 30, 0.2337, dtype=np.float32)) + \
        [0.0, -0.0, 1e-20, -1e-20, 90.0, -90.0, 12.5, -12.5]
    base = np.array(base, np.float32)
    for n in (1, 2, 7, 8, 9, 15, 16, 17, 64, 129, len(base)):
        vec, scal = O.gelu_ref(base[:n]), O.gelu(base[:n])
        assert np.max(np.abs(vec - scal)) <= 1e-6, n
        if n >= 8:  # the vector body really ran (not the scalar fallback)
            lanes = np.array([O.lib.or_gelu_avx2_lane(float(v)) for v in base[:n & ~7]],
                             np.float32)
            assert np.array_equal(vec[:n & ~7], lanes)
    xs = np.arange(-6, 6.0001, 0.25, dtype=np.float32)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(np.float64)])
    lanes = np.array([O.lib.or_gelu_avx2_lane(float(v)) for v in xs], np.float32)
    assert np.max(np.abs(lanes - want)) <= 1e-6


def test_expf32_erff32_bounds():
    ke = KATS["expf32"]
    for x in np.arange(-87, 88, 0.013, dtype=np.float32):
        got = O.lib.or_expf32(float(x))
        want = math.exp(float(x))
        bound = ke["near_zero_rel"] if -20 < x < 20 else ke["far_rel"]
        assert abs(got - want) / want <= bound, x
    for x in ke["finite_at"]:
        assert math.isfinite(O.lib.or_expf32(x))
    assert O.lib.or_expf32(ke["zero_at"]) == 0
    assert math.isinf(O.lib.or_expf32(ke["inf_at"]))
    assert O.lib.or_expf32(0.0) == 1.0
    for x in np.arange(-10, 10, 0.0037, dtype=np.float32):
        assert abs(O.lib.or_erff32(float(x)) - math.erf(float(x))) <= KATS["erff32"]["abs_tol"]
    assert O.lib.or_erff32(0.0) == 0.0


# ---- BERT composition ------------------------------------------------------------------

TINY = None


def tiny_shape():
    from rembed_amd.synthetic import BertShape
    return BertShape("tiny", layers=2, hidden=64, heads=2, intermediate=128,
                     vocab=500, max_position=64, pooling=0)


def np_bert_forward(shape, t, ids):
    """BERT forward in float64 numpy, written from bert.go:796-918 and
    Forward bert.go:649-703 (no fast math, exact erf)."""
    H, nh = shape.hidden, shape.heads
    dh = H // nh
    L = len(ids)
    g = lambda n: t[n].astype(np.float64)

    def ln(x, gam, bet):
        mu = x.mean(axis=1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
        return (x - mu) / np.sqrt(var + shape.eps) * gam + bet

    x = (g("embeddings.word_embeddings.weight")[ids] +
         g("embeddings.position_embeddings.weight")[:L] +
         g("embeddings.token_type_embeddings.weight")[0])
    x = ln(x, g("embeddings.LayerNorm.weight"), g("embeddings.LayerNorm.bias"))
    erf = np.vectorize(math.erf)
    for l in range(shape.layers):
        p = f"encoder.layer.{l}."
        q = x @ g(p + "attention.self.query.weight").T + g(p + "attention.self.query.bias")
        k = x @ g(p + "attention.self.key.weight").T + g(p + "attention.self.key.bias")
        v = x @ g(p + "attention.self.value.weight").T + g(p + "attention.self.value.bias")
        ctx = np.zeros_like(x)
        for h in range(nh):
            sl = slice(h * dh, (h + 1) * dh)
            s = q[:, sl] @ k[:, sl].T / math.sqrt(dh)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            s /= s.sum(axis=1, keepdims=True)
            ctx[:, sl] = s @ v[:, sl]
        a = ctx @ g(p + "attention.output.dense.weight").T + g(p + "attention.output.dense.bias")
        x = ln(x + a, g(p + "attention.output.LayerNorm.weight"),
               g(p + "attention.output.LayerNorm.bias"))
        hdn = x @ g(p + "intermediate.dense.weight").T + g(p + "intermediate.dense.bias")
        hdn = 0.5 * hdn * (1 + erf(hdn / math.sqrt(2)))
        o = hdn @ g(p + "output.dense.weight").T + g(p + "output.dense.bias")
        x = ln(x + o, g(p + "output.LayerNorm.weight"), g(p + "output.LayerNorm.bias"))
    pooled = x.mean(axis=0) if shape.pooling == 0 else x[0]
    return x, pooled / np.linalg.norm(pooled)


def test_bert_oracle_matches_float64_composition():
    from rembed_amd.synthetic import bert_tensors
    shape = tiny_shape()
    t = bert_tensors(shape, seed=3)
    orc = O.BertOracle(shape, t, 0)
    rng = np.random.default_rng(4)
    for L in (1, 5, 17, 40):
        ids = rng.integers(0, shape.vocab, size=L).astype(np.int32)
        hid_ref, vec_ref = np_bert_forward(shape, t, ids)
        hid = orc.encode(ids)
        assert np.max(np.abs(hid - hid_ref)) < 2e-5, L
        vec = orc.forward(ids)
        assert np.max(np.abs(vec - vec_ref)) < 1e-5, L
        assert abs(np.linalg.norm(vec.astype(np.float64)) - 1) < 1e-6


def test_bert_oracle_modes_and_batch_policy():
    from rembed_amd.synthetic import bert_tensors, token_batch
    shape = tiny_shape()
    t = bert_tensors(shape, seed=8)
    ids, lens = token_batch(6, 48, 3, 48, vocab=shape.vocab, id_lo=0, seed=9)
    outs = {}
    for quant in (0, 1, 2):
        orc = O.BertOracle(shape, t, quant)
        batch1 = orc.embed_batch(ids, lens, threads=1)
        batch4 = orc.embed_batch(ids, lens, threads=4)
        assert np.array_equal(batch1, batch4)  # worker count never changes bits
        single = np.stack([orc.forward(ids[b, :lens[b]]) for b in range(len(lens))])
        assert np.array_equal(batch1, single)
        outs[quant] = batch1
    # the full-int8 denses on the reference's panel kernel give the same bits
    orc = O.BertOracle(shape, t, 2)
    O.lib.or_set_gemm_impl(1)
    try:
        secs = np.zeros(len(lens))
        panels = orc.embed_batch(ids, lens, threads=3, secs=secs)
    finally:
        O.lib.or_set_gemm_impl(0)
    assert np.array_equal(panels, outs[2])
    assert np.all(secs > 0)
    for quant, floor in ((1, 0.999), (2, 0.99)):
        cos = np.sum(outs[quant] * outs[0], axis=1)
        assert np.all(cos >= floor), (quant, cos.min())
        # the quantized path must actually be active (rembed_test.go:176-237)
        assert np.max(np.abs(outs[quant] - outs[0])) >= 1e-4


def test_bert_oracle_encode_stops_after_layers():
    """encode(ids, L) of a model equals the full encode of the same model
    built with its first L layers."""
    import dataclasses

    from rembed_amd.synthetic import bert_tensors
    shape = tiny_shape()
    t = bert_tensors(shape, seed=12)
    ids = np.arange(5, 40, dtype=np.int32) % shape.vocab
    full = O.BertOracle(shape, t, 2)
    for L in range(1, shape.layers + 1):
        part = O.BertOracle(dataclasses.replace(shape, layers=L), t, 2)
        assert np.array_equal(full.encode(ids, L), part.encode(ids)), L


def test_bert_oracle_rejects_bad_input():
    from rembed_amd.synthetic import bert_tensors
    shape = tiny_shape()
    orc = O.BertOracle(shape, bert_tensors(shape, seed=1), 0)
    with pytest.raises(RuntimeError):
        orc.forward(np.array([shape.vocab], np.int32))
    with pytest.raises(RuntimeError):
        orc.forward(np.zeros(shape.max_position + 1, np.int32))
