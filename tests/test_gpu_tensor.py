"""GPU parity of the tensor-level entry points against the pinned oracle.

Integer work (activation quantization, u8 x s8 accumulators, the full-int8
epilogue, GELU) must be bit-exact; the floating-point GEMMs are held to the
reference's own float64 tolerance (internal/tensor/pack_test.go:55-67) or,
for the bf16-split MFMA paths, to that tolerance plus the split's derived
error bound (split_bound below).
"""
import json
import math
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_kats.json")))
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "vnni_vectors.npz")
GUARD = 64  # canary floats past the end of every output


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def T():
    from rembed_amd import tensor
    return tensor


def vnni_case(rng, m, k, n):
    a = (rng.random((m, k), dtype=np.float32) * 4 - 2).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    if k > 2:
        a[0, :3] = KATS["vnni_exact_shapes"]["rail_row"]
    return a, bT


def run_vnni(ctx, a, pb, m):
    """MatMulPackedVNNI on device with guard canaries; returns dst, qa, rs."""
    t = T()
    k, n = pb.K, pb.N
    ldq = t.ldq_for(k)
    da = ctx.upload(a)
    dst = ctx.upload(np.full(m * n + GUARD, -999, np.float32))
    qa = ctx.upload(np.full(m * ldq + GUARD, 0xAB, np.uint8))
    rs = ctx.upload(np.full(m + GUARD, -7, np.float32))
    t.MatMulPackedVNNI(ctx, dst, da, pb, m, qa, ldq, rs)
    ctx.sync()
    d = dst.download(np.float32, (m * n + GUARD,))
    q = qa.download(np.uint8, (m * ldq + GUARD,))
    r = rs.download(np.float32, (m + GUARD,))
    assert np.all(d[m * n:] == -999), "dst guard overwritten"
    assert np.all(q[m * ldq:] == 0xAB), "qa guard overwritten"
    assert np.all(r[m:] == -7), "row-scale guard overwritten"
    qm = q[: m * ldq].reshape(m, ldq)
    assert np.all(qm[:, k:] == 0), "tail bytes not zeroed"
    return d[: m * n].reshape(m, n), qm[:, :k], r[:m]


@pytest.mark.parametrize("shape", KATS["vnni_exact_shapes"]["shapes"])
def test_vnni_bit_exact_reference_shapes(gpu_ctx, shape):
    m, k, n = shape
    say(f"vnni shape m={m} k={k} n={n}")
    rng = np.random.default_rng(1000 + m * 31 + k)
    a, bT = vnni_case(rng, m, k, n)
    pb = T().PackB8VNNI(gpu_ctx, bT, k, n)
    q, sc, cs = pb.export()
    st, q_o, sc_o, cs_o = O.pack_b8_vnni(bT, k, n)
    assert np.array_equal(q, q_o) and np.array_equal(sc, sc_o) and np.array_equal(cs, cs_o)
    dst, qa, rs = run_vnni(gpu_ctx, a, pb, m)
    dst_o, qa_o, rs_o, acc_o = O.matmul_vnni(a, q_o, cs_o, sc_o)
    assert np.array_equal(qa, qa_o), "QuantizeRowU8 bytes differ"
    assert np.array_equal(rs, rs_o), "row scales differ"
    assert np.array_equal(dst, dst_o), "dequantized output not bit-exact"


def test_vnni_golden_fixture(gpu_ctx):
    g = np.load(GOLDEN)
    tags = sorted({k.split("/")[0] for k in g.files if "/" in k})
    for tag in tags:
        m, k, n = map(int, tag.split("x"))
        say(f"golden {tag}")
        pb = T().PackB8VNNI(gpu_ctx, g[f"{tag}/bT"], k, n)
        q, sc, cs = pb.export()
        assert np.array_equal(q, g[f"{tag}/q"])
        assert np.array_equal(sc, g[f"{tag}/scales"])
        assert np.array_equal(cs, g[f"{tag}/colsum"])
        dst, qa, rs = run_vnni(gpu_ctx, g[f"{tag}/a"], pb, m)
        assert np.array_equal(qa, g[f"{tag}/qa"])
        assert np.array_equal(rs, g[f"{tag}/rs"])
        assert np.array_equal(dst, g[f"{tag}/dst"])
        # raw accumulators in the reference's u8·s8 form
        t = T()
        ldq = t.ldq_for(k)
        qpad = np.zeros((m, ldq), np.uint8)
        qpad[:, :k] = g[f"{tag}/qa"]
        dq = gpu_ctx.upload(qpad)
        acc = gpu_ctx.upload(np.zeros(m * n, np.int32))
        t.GemmU8S8I32(gpu_ctx, acc, dq, ldq, pb, m)
        gpu_ctx.sync()
        assert np.array_equal(acc.download(np.int32, (m, n)), g[f"{tag}/acc"])


@pytest.mark.parametrize("kn", [(768, 2304), (768, 768), (768, 3072), (3072, 768)])
@pytest.mark.parametrize("m", [2048, 16384])
def test_i32_accumulators_bert_base_bit_exact(gpu_ctx, m, kn):
    """int32 accumulators bit-exact at the BERT-base GEMM shapes."""
    k, n = kn
    say(f"i32 acc m={m} k={k} n={n}")
    t = T()
    rng = np.random.default_rng(m + k + n)
    bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    pb = t.PackB8VNNI(gpu_ctx, bT, k, n)
    q, _, _ = pb.export()
    qa = rng.integers(0, 256, size=(m, k), dtype=np.uint8)
    ldq = t.ldq_for(k)
    dq = gpu_ctx.upload(qa)
    acc = gpu_ctx.upload(np.full(m * n + GUARD, 0x7EADBEEF, np.int32))
    t.GemmU8S8I32(gpu_ctx, acc, dq, ldq, pb, m)
    gpu_ctx.sync()
    got = acc.download(np.int32, (m * n + GUARD,))
    assert np.all(got[m * n:] == 0x7EADBEEF)
    want = O.gemm_u8s8_i32(qa, q)
    assert np.array_equal(got[: m * n].reshape(m, n), want)


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15])
def test_every_int8_tile_config_bit_exact(gpu_ctx, tile):
    """Each int8 GEMM tile configuration (forced) gives the oracle's exact
    accumulators and dequantized outputs, including M/N/K tails."""
    from rembed_amd._lib import RH_CTX_I8_TILE
    t = T()
    rng = np.random.default_rng(40 + tile)
    gpu_ctx.set_option(RH_CTX_I8_TILE, tile)
    try:
        for (m, k, n) in [(1, 1, 16), (13, 129, 64), (300, 384, 1536), (517, 100, 272),
                          (2048, 768, 2304), (1999, 3072, 768)]:
            say(f"tile {tile} m={m} k={k} n={n}")
            a = rng.standard_normal((m, k), dtype=np.float32)
            bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.05).astype(np.float32)
            pb = t.PackB8VNNI(gpu_ctx, bT, k, n)
            dst, qa, rs = run_vnni(gpu_ctx, a, pb, m)
            st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
            want, qa_o, rs_o, acc_o = O.matmul_vnni(a, q, cs, sc)
            assert np.array_equal(dst, want)
            ldq = t.ldq_for(k)
            qpad = np.zeros((m, ldq), np.uint8)
            qpad[:, :k] = qa_o
            dq = gpu_ctx.upload(qpad)
            acc = gpu_ctx.upload(np.full(m * n + GUARD, 0x7EADBEEF, np.int32))
            t.GemmU8S8I32(gpu_ctx, acc, dq, ldq, pb, m)
            gpu_ctx.sync()
            got = acc.download(np.int32, (m * n + GUARD,))
            assert np.all(got[m * n:] == 0x7EADBEEF)
            assert np.array_equal(got[: m * n].reshape(m, n), acc_o)
    finally:
        gpu_ctx.set_option(RH_CTX_I8_TILE, 0)


def test_quantize_rows_bit_exact(gpu_ctx):
    t = T()
    rng = np.random.default_rng(77)
    for k in (1, 3, 5, 7, 33, 129, 384, 768, 1536, 3072):
        m = 37
        say(f"quantize k={k}")
        a = (rng.standard_normal((m, k), dtype=np.float32) *
             np.exp(rng.integers(-8, 8, size=(m, 1))).astype(np.float32)).astype(np.float32)
        a[3] = 0
        if k >= 4:
            a[5, :4] = [127, -127, 0, 63.5]
        ldq = t.ldq_for(k)
        da = gpu_ctx.upload(a)
        qa = gpu_ctx.upload(np.full(m * ldq, 0xCD, np.uint8))
        rs = gpu_ctx.alloc(m * 4)
        t.QuantizeRowsU8(gpu_ctx, da, m, k, qa, ldq, rs)
        gpu_ctx.sync()
        q = qa.download(np.uint8, (m, ldq))
        r = rs.download(np.float32, (m,))
        for i in range(m):
            qo, so = O.quantize_row_u8(a[i], ldq)
            assert np.array_equal(q[i], qo), (k, i)
            assert r[i] == so, (k, i)


def _gelu_quant_rows_adversarial(rng, k):
    """Rows that stress a GELU quantizer: scaled GELU values on and next to
    half-integers (rint's decision points), many near-ties at the row
    maximum, and rows whose GELU is tiny beside |x|."""
    rows = []
    top = np.float32(4.0)
    mx = O.gelu_ref(np.full(8, top, np.float32))[0]
    inv = np.float32(1) / (mx / np.float32(127))
    sweep = np.linspace(-0.3, 3.9, 1 << 20, dtype=np.float32)
    p = O.gelu_ref(sweep) * inv
    frac = np.abs(np.abs(p - np.rint(p)) - np.float32(0.5))
    near = sweep[np.argsort(frac, kind="stable")[: 4 * k]]
    for r in range(3):
        row = rng.choice(near, k).astype(np.float32)
        row[rng.integers(k)] = top
        rows.append(row)
    ties = (top + np.float32(2.0 ** -20) * rng.integers(-40, 40, k)).astype(np.float32)
    rows.append(ties)
    rows.append((-5 - 15 * rng.random(k)).astype(np.float32))
    rows.append((-3.5 - rng.random(k)).astype(np.float32))
    return np.stack(rows)


def test_gelu_quantize_rows_bit_exact(gpu_ctx):
    """GELU then QuantizeRowU8 (bert.go:910-916) in one kernel: bytes and
    scales equal the oracle's gelu_ref + quantize_row_u8 exactly, random rows
    at scales 2^-8..2^8 and rows built against the quantizer (scaled GELU
    values on and next to half-integers, near-ties at the row max, rows of
    tiny GELU beside large |x|), widths ragged to the 256-element vector
    loop and past the register-resident range (4096)."""
    t = T()
    rng = np.random.default_rng(91)
    for k in (8, 16, 264, 768, 1000, 1536, 3072, 4096):
        m = 41
        a = (rng.standard_normal((m, k), dtype=np.float32) *
             np.exp2(rng.integers(-8, 9, size=(m, 1))).astype(np.float32)).astype(np.float32)
        a[3] = 0
        a = np.concatenate([a, _gelu_quant_rows_adversarial(rng, k)])
        m = a.shape[0]
        say(f"gelu quantize k={k} rows={m}")
        ldq = t.ldq_for(k)
        da = gpu_ctx.upload(a)
        qa = gpu_ctx.upload(np.full(m * ldq, 0xCD, np.uint8))
        rs = gpu_ctx.alloc(m * 4)
        t.GELUQuantizeRowsU8(gpu_ctx, da, m, k, qa, ldq, rs)
        gpu_ctx.sync()
        q = qa.download(np.uint8, (m, ldq))
        r = rs.download(np.float32, (m,))
        assert np.array_equal(da.download(np.float32, a.shape), a)
        for i in range(m):
            qo, so = O.quantize_row_u8(O.gelu_ref(a[i]), ldq)
            assert np.array_equal(q[i], qo), (k, i)
            assert r[i] == so, (k, i)


def test_gelu_quantize_rows_nonfinite_and_errors(gpu_ctx):
    """Rows holding inf or NaN give the same bytes and scales as GELU in
    place followed by QuantizeRowU8 on the device; k % 8 != 0 is refused."""
    from rembed_amd._lib import RembedError, check, lib
    t = T()
    rng = np.random.default_rng(92)
    k, m = 768, 6
    a = rng.standard_normal((m, k), dtype=np.float32)
    a[0, 5] = np.inf
    a[1, 9] = -np.inf
    a[2, 17] = np.nan
    a[3, :2] = [np.inf, np.nan]
    ldq = t.ldq_for(k)
    da = gpu_ctx.upload(a)
    qa = gpu_ctx.alloc(m * ldq)
    rs = gpu_ctx.alloc(m * 4)
    t.GELUQuantizeRowsU8(gpu_ctx, da, m, k, qa, ldq, rs)
    db = gpu_ctx.upload(a)
    check(lib.rh_gelu(gpu_ctx.h, db.ptr, a.size))
    qb = gpu_ctx.alloc(m * ldq)
    rb = gpu_ctx.alloc(m * 4)
    t.QuantizeRowsU8(gpu_ctx, db, m, k, qb, ldq, rb)
    gpu_ctx.sync()
    assert np.array_equal(qa.download(np.uint8, (m, ldq)), qb.download(np.uint8, (m, ldq)))
    assert np.array_equal(rs.download(np.uint32, (m,)), rb.download(np.uint32, (m,)))
    with pytest.raises(RembedError):
        t.GELUQuantizeRowsU8(gpu_ctx, da, m, 764, qa, ldq, rs)


def test_linear_a8w8_bias_gelu_bit_exact(gpu_ctx):
    """Fused bias + erf-GELU epilogue equals AddBias then GELU (bert.go:297-300,913-915)."""
    t = T()
    rng = np.random.default_rng(5)
    m, k, n = 300, 384, 1536
    a = rng.standard_normal((m, k), dtype=np.float32)
    bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    pb = t.PackB8VNNI(gpu_ctx, bT, k, n, bias=bias)
    got, _ = t.matmul_host(gpu_ctx, a, pb, act=1)
    st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
    dst, _, _, _ = O.matmul_vnni(a, q, cs, sc)
    want = O.gelu_ref((dst + bias[None, :]).astype(np.float32))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("mkn", [(4096, 2048, 4096), (4352, 3072, 4096)], ids=["ring4", "ring3"])
def test_int8_big_grid_tile_matches(gpu_ctx, mkn):
    """Where the automatic choice takes tile 15 (K >= 2048 and at least 256
    tiles of 256x256; a four-slot ring at K = 2048, three at 3072 with
    partial row tiles) its int32 accumulators and dequantized rows equal
    tile 9's bit for bit (tile 15 itself is pinned to the oracle on the
    smaller shapes of test_every_int8_tile_config_bit_exact)."""
    from rembed_amd._lib import RH_CTX_I8_TILE
    t = T()
    m, k, n = mkn
    say(f"int8 auto (tile 15) vs tile 9 m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.05).astype(np.float32)
    pb = t.PackB8VNNI(gpu_ctx, bT, k, n)
    outs = []
    for tile in (0, 9):
        gpu_ctx.set_option(RH_CTX_I8_TILE, tile)
        try:
            dst, qa, rs = run_vnni(gpu_ctx, a, pb, m)
            ldq = t.ldq_for(k)
            dq = gpu_ctx.upload(np.ascontiguousarray(qa))
            acc = gpu_ctx.alloc(m * n * 4)
            t.GemmU8S8I32(gpu_ctx, acc, dq, ldq, pb, m)
            gpu_ctx.sync()
            outs.append((dst, acc.download(np.int32, (m, n))))
        finally:
            gpu_ctx.set_option(RH_CTX_I8_TILE, 0)
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][0], outs[1][0])


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15])
def test_linear_u8_fused_quantization_bit_exact(gpu_ctx, tile):
    """FFN1 -> GELU -> QuantizeRowU8 in two GEMM passes (no fp32 rows) gives
    exactly QuantizeRowU8 of the reference's fp32 GELU rows."""
    from rembed_amd._lib import RH_CTX_I8_TILE
    t = T()
    rng = np.random.default_rng(8 + tile)
    gpu_ctx.set_option(RH_CTX_I8_TILE, tile)
    try:
        for (m, k, n) in [(5, 64, 48), (333, 384, 1536), (1031, 768, 3072)]:
            say(f"linear_u8 tile {tile} m={m} k={k} n={n}")
            a = rng.standard_normal((m, k), dtype=np.float32)
            bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.05).astype(np.float32)
            bias = (rng.standard_normal(n, dtype=np.float32) * 0.1).astype(np.float32)
            pb = t.PackB8VNNI(gpu_ctx, bT, k, n, bias=bias)
            st, q, sc, cs = O.pack_b8_vnni(bT, k, n)
            dst, qa_o, rs_o, _ = O.matmul_vnni(a, q, cs, sc)
            hid = O.gelu_ref((dst + bias[None, :]).astype(np.float32))
            ldq, ldo = t.ldq_for(k), t.ldq_for(n)
            qpad = np.zeros((m, ldq), np.uint8)
            qpad[:, :k] = qa_o
            dq, drs = gpu_ctx.upload(qpad), gpu_ctx.upload(rs_o)
            out = gpu_ctx.upload(np.zeros(m * ldo + GUARD, np.uint8))
            rs_out = gpu_ctx.upload(np.full(m + GUARD, -3, np.float32))
            absmax = gpu_ctx.alloc(m * 4)
            t.LinearU8(gpu_ctx, dq, ldq, drs, pb, m, 1, out, ldo, rs_out, absmax)
            gpu_ctx.sync()
            got = out.download(np.uint8, (m * ldo + GUARD,))
            grs = rs_out.download(np.float32, (m + GUARD,))
            assert np.all(got[m * ldo:] == 0) and np.all(grs[m:] == -3)
            for i in range(m):
                qo, so = O.quantize_row_u8(hid[i], n)
                assert np.array_equal(got[i * ldo: i * ldo + n], qo), (m, i)
                assert grs[i] == so, (m, i)
    finally:
        gpu_ctx.set_option(RH_CTX_I8_TILE, 0)


def f64_tol(k):
    return max(KATS["packed_f32_shapes"]["tol_base"],
               KATS["packed_f32_shapes"]["tol_sqrtk"] * math.sqrt(k))


# Error bounds of the bf16 MFMA paths. A float x rounded to bf16 (8
# significant bits) keeps |x - hi| <= 2^-9 |x|; split into hi = rne8(x),
# lo = rne8(x - hi) it keeps |x - hi - lo| <= 2^-16 |x|. Weight-only int8: q
# is exact in bf16, so |err| <= 2^-9 sum|a·deq| with one activation term and
# 2^-16 sum|a·deq| with two. fp32 via three products hi·hi + hi·lo + lo·hi:
# |err| <= ~3·2^-16 sum|a·b|. Each gets a factor-2 margin plus the
# reference's fp32 tolerance for the accumulation. An indexing mistake moves
# a result by a whole product |a_p·b_p|, far above these bounds.
def split_bound(a, b, k, eps, want):
    mag = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)).T
    return eps * mag + f64_tol(k) * (1 + np.abs(want))


@pytest.mark.parametrize("terms", [1, 2])
@pytest.mark.parametrize("bf", [0, 1])
@pytest.mark.parametrize("shape", KATS["packed_f32_shapes"]["shapes"])
def test_matmul_packed8_against_dequantized_float64(gpu_ctx, shape, bf, terms):
    from rembed_amd._lib import RH_CTX_W8_TERMS
    m, k, n = shape
    say(f"w8 shape {shape} bf_algo {bf} terms {terms}")
    t = T()
    rng = np.random.default_rng(23 + k)
    a = (rng.random((m, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    bT[n // 2] = 0  # the scale-1 branch
    pb = t.PackB8(gpu_ctx, bT, k, n)
    q, sc, _ = pb.export()
    st, q_o, sc_o = O.pack_b8(bT, k, n)
    assert np.array_equal(q, q_o) and np.array_equal(sc, sc_o)
    gpu_ctx.set_bf_algo(bf)
    gpu_ctx.set_option(RH_CTX_W8_TERMS, terms)
    try:
        got = t.matmul_host(gpu_ctx, a, pb)
    finally:
        gpu_ctx.set_bf_algo(0)
        gpu_ctx.set_option(RH_CTX_W8_TERMS, 1)
    deq = q.astype(np.float64) * sc.astype(np.float64)[:, None]
    want = a.astype(np.float64) @ deq.T
    bound = split_bound(a, deq, k, 2.0 ** -8 if terms == 1 else 2.0 ** -15, want)
    err = np.abs(got - want)
    say(f"  max err {err.max():.3e}  worst err/bound {(err / bound).max():.3f}")
    assert np.all(err <= bound)


# (f32 algo, bf algo): bf16 split on pre-split planes, split in the main
# loop, native f32 MFMA
@pytest.mark.parametrize("algo,bf", [(0, 0), (0, 1), (1, 0)], ids=["planes", "inloop", "native"])
@pytest.mark.parametrize("shape", KATS["packed_f32_shapes"]["shapes"])
def test_matmul_packed_f32_against_float64(gpu_ctx, shape, algo, bf):
    m, k, n = shape
    say(f"f32 shape {shape} algo {algo} bf_algo {bf}")
    t = T()
    rng = np.random.default_rng(11 + k)
    a = (rng.random((m, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    gpu_ctx.set_f32_algo(algo)
    gpu_ctx.set_bf_algo(bf)
    try:
        pb = t.PackB(gpu_ctx, bT, k, n)
        got = t.matmul_host(gpu_ctx, a, pb)
    finally:
        gpu_ctx.set_f32_algo(0)
        gpu_ctx.set_bf_algo(0)
    want = a.astype(np.float64) @ bT.astype(np.float64).T
    err = np.abs(got - want)
    if algo == 1:  # native f32 MFMA: the reference's own tolerance
        bound = f64_tol(k) * (1 + np.abs(want))
    else:
        bound = split_bound(a, bT, k, 2.0 ** -14, want)
    say(f"  max err {err.max():.3e}  worst err/bound {(err / bound).max():.3f}")
    assert np.all(err <= bound)


@pytest.mark.parametrize("shape", KATS["packed_f32_shapes"]["shapes"] +
                         [[1, 1, 1], [7, 3, 5], [33, 70, 1030], [300, 129, 250]])
def test_matmul_unpacked_against_float64(gpu_ctx, shape):
    """MatMulFunc's unpacked path (tensor.go:16-70): raw fp32 weights, any
    shape (odd n and k, n not a multiple of 4 or of the 256-row weight
    padding, unaligned output rows), within the fp32 split's bound."""
    m, k, n = shape
    say(f"unpacked f32 shape {shape}")
    rng = np.random.default_rng(13 + k + n)
    a = (rng.random((m, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    bT = (rng.random((n, k), dtype=np.float32) * 2 - 1).astype(np.float32)
    a_d, b_d = gpu_ctx.upload(a), gpu_ctx.upload(bT)
    guard = 64
    out = gpu_ctx.upload(np.full(m * n + guard, 7.0, np.float32))
    T().MatMul(gpu_ctx, out, a_d, b_d, m, k, n)
    gpu_ctx.sync()
    full = out.download(np.float32, (m * n + guard,))
    assert np.all(full[m * n:] == 7.0)  # nothing written past the output
    got = full[: m * n].reshape(m, n)
    want = a.astype(np.float64) @ bT.astype(np.float64).T
    bound = split_bound(a, bT, k, 2.0 ** -14, want)
    err = np.abs(got - want)
    say(f"  max err {err.max():.3e}  worst err/bound {(err / bound).max():.3f}")
    assert np.all(err <= bound)


def test_gelu_bit_exact(gpu_ctx):
    from rembed_amd._lib import check, lib
    xs = np.concatenate([np.arange(-30, 30, 0.2337, dtype=np.float32),
                         np.array([0, -0.0, 1e-20, -1e-20, 90, -90, 12.5, -12.5],
                                  np.float32)]).astype(np.float32)
    d = gpu_ctx.upload(xs)
    check(lib.rh_gelu(gpu_ctx.h, d.ptr, xs.size))
    gpu_ctx.sync()
    assert np.array_equal(d.download(np.float32, xs.shape), O.gelu_ref(xs))


def test_gelu_bit_exact_across_float32(gpu_ctx):
    """erf-GELU over every 61st bit pattern of float32 (70M inputs: both
    signs, subnormals, the whole exponent range, ±inf and NaNs) equals the
    oracle's geluAVX2/geluScalar bit for bit (NaN results compare as NaN).
    The kernel takes t = 1/d from the hardware reciprocal plus one Newton
    step and 2^n by ldexp; this pins both against the reference's IEEE
    division and power-of-two product far outside the activations' range."""
    from rembed_amd._lib import check, lib
    bits = np.arange(7, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x80000001,
                         0x007FFFFF, 0x00800000, 0x7F7FFFFF, 0xFF7FFFFF, 0, 0x80000000],
                        np.uint32)
    xs = np.concatenate([specials, bits]).view(np.float32)
    say(f"gelu over {xs.size} inputs")
    d = gpu_ctx.upload(xs)
    check(lib.rh_gelu(gpu_ctx.h, d.ptr, xs.size))
    gpu_ctx.sync()
    got = d.download(np.float32, xs.shape)
    want = O.gelu_ref(xs)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{bad.size} mismatches, first inputs {xs[bad[:5]].view(np.uint32)}"


def test_layernorm_matches_oracle(gpu_ctx):
    from rembed_amd._lib import check, lib
    rng = np.random.default_rng(3)
    for n in (3, 384, 768, 1024):
        x = rng.standard_normal((50, n), dtype=np.float32) * 3 + 1
        g = rng.standard_normal(n, dtype=np.float32)
        b = rng.standard_normal(n, dtype=np.float32)
        dx, dg, db = gpu_ctx.upload(x), gpu_ctx.upload(g), gpu_ctx.upload(b)
        check(lib.rh_layernorm(gpu_ctx.h, dx.ptr, dg.ptr, db.ptr, 50, n,
                               np.float32(1e-12)))
        gpu_ctx.sync()
        got = dx.download(np.float32, x.shape)
        want = O.layernorm(x, g, b, 1e-12)
        assert np.max(np.abs(got - want)) <= 1e-5 * (1 + np.abs(want)).max()


def test_pack_errors_surface_as_status(gpu_ctx):
    from rembed_amd._lib import RembedError, RH_ERR_NONFINITE, RH_ERR_SHAPE
    t = T()
    with pytest.raises(RembedError) as e:
        t.PackB8(gpu_ctx, np.zeros((15, 3), np.float32), 3, 15)
    assert e.value.code == RH_ERR_SHAPE
    bad = np.zeros((16, 4), np.float32)
    bad[1, 2] = np.nan
    for fn in (t.PackB8, t.PackB8VNNI):
        with pytest.raises(RembedError) as e:
            fn(gpu_ctx, bad, 4, 16)
        assert e.value.code == RH_ERR_NONFINITE
