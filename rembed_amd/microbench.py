"""GEMM microbenchmarks on one GPU — the device counterpart of the
reference's BenchmarkMatMulPacked* (internal/tensor/pack8_test.go,
tensor_test.go benchmarks), at the encoder's real shapes.

Each case is timed with the library's per-launch HIP events on its own
stream. Usage:
    python -m rembed_amd.microbench [--m 10102] [--iters 20] [--modes i8,w8,f32]
    python -m rembed_amd.microbench --attention bert-base,qwen3-0.6b,gemma-global
    python -m rembed_amd.microbench --hipblaslt   (the vendor library at the same shapes)
"""
import argparse
import ctypes
import json
import sys

import numpy as np

from . import _lib
from . import tensor as T

BERT_SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
PEAK = {"i8": 5000.0, "w8": 2500.0, "f32": 2500.0}  # TOP/s of the MFMA used


def bench_case(ctx, mode, m, k, n, iters, act=0, tile=0, acc_only=False, fused_u8=False, bf=0,
               group=4, uniform=False, copies=1, requantize=False):
    """Normal weights and activations (an encoder's distribution); uniform:
    values uniform in [-1, 1), whose int8 images are near-uniform bytes
    (the matrix cores clock lower on high-entropy operands). copies > 1:
    that many packed weights, used in turn, as a forward's layers use theirs
    (a launch then reads its weight past the L2 instead of from it).
    requantize (int8): the activation rows are quantized again before every
    launch, so each launch reads u8 rows just written, as in a forward."""
    rng = np.random.default_rng(k * 7 + n)
    draw = ((lambda shape: rng.uniform(-1.0, 1.0, shape).astype(np.float32)) if uniform
            else (lambda shape: rng.standard_normal(shape, dtype=np.float32)))
    bT = (draw((n, k)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32) * 0.02
    pack = {"i8": T.PackB8VNNI, "w8": T.PackB8, "f32": T.PackB}[mode]
    pbs = [pack(ctx, bT, k, n, bias=bias)]
    for _ in range(copies - 1):
        pbs.append(pack(ctx, (draw((n, k)) * 0.02).astype(np.float32), k, n, bias=bias))
    turn = [0]
    a = ctx.upload(draw((m, k)))
    dst = ctx.alloc(m * n * 4)
    ldq = T.ldq_for(k)
    qa = ctx.alloc(m * ldq)
    rs = ctx.alloc(m * 4)
    kind = {"i8": 0, "w8": 1, "f32": 2}[mode]
    ctx.set_option(_lib.RH_CTX_I8_TILE if mode == "i8" else _lib.RH_CTX_BF_TILE, tile)
    ctx.set_bf_algo(bf)
    ctx.set_option(_lib.RH_CTX_TILE_GROUP, group)
    if mode == "i8":
        T.QuantizeRowsU8(ctx, a, m, k, qa, ldq, rs)

    ldo = T.ldq_for(n)
    qout = ctx.alloc(m * ldo) if fused_u8 else None
    rs_out = ctx.alloc(m * 4) if fused_u8 else None
    absmax = ctx.alloc(m * 4) if fused_u8 else None

    def run():
        pb = pbs[turn[0] % len(pbs)]
        turn[0] += 1
        if mode == "i8" and requantize:
            T.QuantizeRowsU8(ctx, a, m, k, qa, ldq, rs)
        if mode == "i8":
            if fused_u8:  # linear + QuantizeRowU8 of the outputs (two passes)
                T.LinearU8(ctx, qa, ldq, rs, pb, m, act, qout, ldo, rs_out, absmax)
            elif acc_only:  # int32 accumulators only: the GEMM core
                T.GemmU8S8I32(ctx, dst, qa, ldq, pb, m)
            else:  # fp32 dequant epilogue (+bias, +GELU); quantize is not timed
                T.Linear(ctx, dst, a, pb, m, act, qa, ldq, rs)
        else:
            T.Linear(ctx, dst, a, pb, m, act)

    for _ in range(3):
        run()
    ctx.sync()
    ctx.profile(True)
    for _ in range(iters):
        run()
    ctx.sync()
    st = ctx.profile_read(kind)
    sp = ctx.profile_read(4)  # activation split of the planes path
    ctx.profile(False)
    ctx.set_option(_lib.RH_CTX_I8_TILE, 0)
    ctx.set_option(_lib.RH_CTX_BF_TILE, 0)
    ctx.set_bf_algo(0)
    per_call = 2 if fused_u8 else 1  # the fused variant launches two GEMM passes
    us = st["total_ms"] * 1e3 / st["launches"] * per_call
    tops = st["total_ops"] / (st["total_ms"] * 1e-3) / 1e12
    ctx.set_option(_lib.RH_CTX_TILE_GROUP, 4)
    split_us = sp["total_ms"] * 1e3 / sp["launches"] if sp["launches"] else 0.0
    return {"mode": mode, "m": m, "k": k, "n": n, "act": act, "tile": tile, "bf": bf,
            "group": group, "operands": "uniform" if uniform else "normal",
            "weight_copies": copies, "requantize": requantize,
            "acc_only": acc_only, "fused_u8": fused_u8, "us": round(us, 2),
            "split_us": round(split_us, 2), "tops": round(tops, 1),
            "frac": round(tops / PEAK[mode], 4),
            "gbps": round(st["total_bytes"] / (st["total_ms"] * 1e-3) / 1e9, 1)}


def f32_choice(ctx, m, k, n, iters, rows=256):
    """The fp32 linear's two algorithms at one shape: three bf16 MFMA
    products on split planes (the default) and native f32 MFMA. Time per
    launch from HIP events; error on a sample of rows against the float64
    product, beside numpy's own float32 product (a CPU fp32 GEMM) of the
    same operands. Inputs: N(0, 1) activations, N(0, 0.02) weights and bias
    (BERT-like scales)."""
    rng = np.random.default_rng(k * 11 + n)
    bT = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * 0.02).astype(np.float32)
    a_h = rng.standard_normal((m, k), dtype=np.float32)
    sample = np.sort(rng.choice(m, size=min(rows, m), replace=False))
    want = a_h[sample].astype(np.float64) @ bT.T.astype(np.float64) + bias
    scale = np.abs(a_h[sample]).astype(np.float64) @ np.abs(bT.T).astype(np.float64)
    cpu = a_h[sample] @ bT.T + bias
    out = []
    pb = T.PackB(ctx, bT, k, n, bias=bias)
    a = ctx.upload(a_h)
    dst = ctx.alloc(m * n * 4)
    for algo, name in ((0, "bf16x3 planes"), (1, "native f32")):
        ctx.set_option(_lib.RH_CTX_F32_ALGO, algo)
        for _ in range(3):
            T.Linear(ctx, dst, a, pb, m, 0)
        ctx.sync()
        ctx.profile(True)
        for _ in range(iters):
            T.Linear(ctx, dst, a, pb, m, 0)
        ctx.sync()
        st = ctx.profile_read(2)
        sp = ctx.profile_read(4)
        ctx.profile(False)
        got = dst.download(np.float32, (m, n))[sample].astype(np.float64)
        us = st["total_ms"] * 1e3 / st["launches"]
        split_us = sp["total_ms"] * 1e3 / sp["launches"] if sp["launches"] else 0.0
        out.append({"f32_algo": name, "m": m, "k": k, "n": n, "us": round(us, 2),
                    "split_us": round(split_us, 2),
                    "tflops": round(2.0 * m * k * n / ((us + split_us) * 1e-6) / 1e12, 1),
                    "max_abs_err": float(np.abs(got - want).max()),
                    "max_err_over_sum_abs": float((np.abs(got - want) / scale).max())})
    ctx.set_option(_lib.RH_CTX_F32_ALGO, 0)
    out.append({"f32_algo": "numpy float32 (CPU)", "m": len(sample), "k": k, "n": n,
                "max_abs_err": float(np.abs(cpu - want).max()),
                "max_err_over_sum_abs": float((np.abs(cpu - want) / scale).max())})
    return out


ATTN_CASES = {
    # name: (dh, heads, kv_heads, causal, window, texts, length)
    "bert-base": (64, 12, 12, False, 0, 64, None),     # lengths U[64,256]
    "qwen3-0.6b": (128, 16, 8, True, 0, 32, 512),
    "gemma-global": (256, 3, 1, False, 0, 16, 2048),
    "gemma-local": (256, 3, 1, False, 512, 16, 2048),
}


def bench_attention(ctx, name, iters, kernels):
    """rh_attention at a workload's shape on random bf16-representable
    q|k|v rows; `kernels`: "bf16" (bf16 rows, the pipelined kernel), "f32"
    (the same values as fp32 rows at precision 1) and/or "planes" (fp32 rows'
    bf16 hi/lo planes, rh_attention_planes: the fp32-grade three-term kernel,
    head dim <= 128; FLOPs counted once)."""
    dh, heads, kv, causal, window, texts, length = ATTN_CASES[name]
    rng = np.random.default_rng(2)
    lens = (rng.integers(64, 257, texts) if length is None else np.full(texts, length))
    lens = lens.astype(np.int32)
    M, ld = int(lens.sum()), (heads + 2 * kv) * dh
    x = (rng.standard_normal((M, ld)) * 0.5).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    bufs = {"bf16": (ctx.upload(bits), 1),
            "f32": (ctx.upload((bits.astype(np.uint32) << 16).view(np.float32)), 0)}
    if "planes" in kernels:  # hi = the rounded bits, lo = bf16 of the remainder
        hi_f = (bits.astype(np.uint32) << 16).view(np.float32)
        r = (x - hi_f).view(np.uint32).astype(np.uint64)
        lo = ((r + 0x7FFF + ((r >> 16) & 1)) >> 16).astype(np.uint16)
        bufs["planes"] = ((ctx.upload(bits), ctx.upload(lo)), 2)
    cu = ctx.upload(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32))
    out = ctx.alloc(M * heads * dh * 4)
    pairs = 0.0
    for L in lens.tolist():
        i = np.arange(L)
        hi = np.full(L, L - 1)
        lo = np.zeros(L, np.int64)
        if causal:
            hi = np.minimum(hi, i)
        if window:
            hi = np.minimum(hi, i + window - 1)
            lo = np.maximum(lo, i - window + 1)
        pairs += float(np.sum(hi - lo + 1))
    flops = 4.0 * pairs * dh * heads
    res = []
    for kern in kernels:
        buf, in_bf16 = bufs[kern]

        def run():
            if in_bf16 == 2:
                T.AttentionPlanes(ctx, out, heads * dh, buf[0], buf[1], ld, 0, heads * dh,
                                  (heads + kv) * dh, cu, texts, int(lens.max()), heads, kv, dh,
                                  1.0 / np.sqrt(dh), causal, window)
            else:
                T.Attention(ctx, out, heads * dh, buf, in_bf16, ld, 0, heads * dh,
                            (heads + kv) * dh, cu, texts, int(lens.max()), heads, kv, dh,
                            1.0 / np.sqrt(dh), causal, window, 1)
        for _ in range(3):
            run()
        ctx.sync()
        ctx.profile(True)
        for _ in range(iters):
            run()
        ctx.sync()
        st = ctx.profile_read(3)
        ctx.profile(False)
        us = st["total_ms"] * 1e3 / st["launches"]
        res.append({"attention": name, "kernel": kern, "dh": dh, "heads": heads, "kv_heads": kv,
                    "causal": causal, "window": window, "tokens": M, "us": round(us, 1),
                    "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                    "frac": round(flops / (us * 1e-6) / 1e12 / PEAK["w8"], 4)})
    return res


def copy_calibration(mib, iters):
    """A device-to-device copy of `mib` MiB by the HIP runtime the library
    uses (hipMemcpy, which runs as one blit kernel per call): each launch
    reads and writes exactly mib MiB, so a profiler's per-dispatch byte
    counters can be scaled against it."""
    hip = _lib.hip_runtime()
    ctx = T.Context(0)  # selects device 0 in the library's runtime
    n = mib * (1 << 20)
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(n)) == 0
    assert hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(n)) == 0
    try:
        assert hip.hipMemset(src, 1, ctypes.c_size_t(n)) == 0
        for _ in range(iters):
            assert hip.hipMemcpy(dst, src, ctypes.c_size_t(n), 3) == 0  # device to device
        assert hip.hipDeviceSynchronize() == 0
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
        ctx.close()
    print(json.dumps({"copy_mib": mib, "launches": iters, "kernel": "__amd_rocclr_copyBuffer",
                      "bytes_read_per_launch": n, "bytes_written_per_launch": n}))
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--m", type=int, default=10102)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--modes", default="i8")
    ap.add_argument("--tiles", default="0")
    ap.add_argument("--shapes", default="", help="k,n;k,n;... (default: BERT-base)")
    ap.add_argument("--variants", default="", help="comma list of acc,fp32,gelu")
    ap.add_argument("--groups", default="4", help="tile-order groups (comma list)")
    ap.add_argument("--w8-terms", type=int, default=1, help="bf16 activation terms of w8 (1 or 2)")
    ap.add_argument("--bf", default="0", help="w8/f32 GEMM algorithms: 0 = bf16 planes, "
                                              "1 = split in the main loop (comma list)")
    ap.add_argument("--attention", default="",
                    help="only time rh_attention at these shapes (comma list of "
                         + ",".join(ATTN_CASES) + ")")
    ap.add_argument("--attn-kernels", default="bf16",
                    help="bf16, f32 and/or planes (comma list)")
    ap.add_argument("--f32-choice", action="store_true",
                    help="only compare the fp32 linear's algorithms (time and error) "
                         "at the shapes")
    ap.add_argument("--hipblaslt", action="store_true",
                    help="only time hipBLASLt's GEMM (every heuristic candidate, the fastest "
                         "reported) at --m and --shapes (default: BERT-base): int8 with "
                         "int32 out, or with --modes bf16 bf16 with fp32 out")
    ap.add_argument("--uniform-operands", action="store_true",
                    help="time the library's GEMMs on uniform operands (near-uniform int8 "
                         "bytes) instead of normal ones")
    ap.add_argument("--quantized-operands", action="store_true",
                    help="with --hipblaslt (int8): per-row quantized normal operand bytes, "
                         "as this benchmark feeds the library's GEMMs, instead of uniformly "
                         "random bytes")
    ap.add_argument("--weight-copies", type=int, default=1,
                    help="pack this many weights per shape and use them in turn, as a "
                         "forward's layers do (default 1: one weight, L2-resident)")
    ap.add_argument("--requantize", action="store_true",
                    help="int8: quantize the activation rows again before every launch, so "
                         "each launch reads freshly written u8 rows (as in a forward)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (calibrates "
                         "the FETCH_SIZE / WRITE_SIZE counters against known bytes)")
    args = ap.parse_args()
    if args.hipblaslt:
        import os
        import subprocess
        exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "blaslt_ref")
        cmd = [exe, str(args.m), str(args.iters),
               "bf16" if args.modes == "bf16" else "i8q" if args.quantized_operands else "i8"]
        if args.shapes:
            cmd.append(args.shapes)
        return subprocess.run(cmd).returncode
    if args.copy_mib:
        return copy_calibration(args.copy_mib, args.iters)
    if args.attention:
        ctx = T.Context(0)
        for name in args.attention.split(","):
            for r in bench_attention(ctx, name, args.iters, args.attn_kernels.split(",")):
                print(json.dumps(r), flush=True)
        ctx.close()
        return 0
    shapes = BERT_SHAPES
    if args.shapes:
        shapes = [tuple(int(x) for x in s.split(",")) for s in args.shapes.split(";")]
    ctx = T.Context(0)
    if args.f32_choice:
        for (k, n) in shapes:
            for r in f32_choice(ctx, args.m, k, n, args.iters):
                print(json.dumps(r), flush=True)
        ctx.close()
        return 0
    ctx.set_option(_lib.RH_CTX_W8_TERMS, args.w8_terms)
    for mode in args.modes.split(","):
        for (k, n) in shapes:
            for tile in [int(t) for t in args.tiles.split(",")]:
                variants = [dict(acc_only=True), dict()] if mode == "i8" else [dict()]
                if n == 3072:
                    variants.append(dict(act=1))
                if args.variants:
                    table = {"acc": dict(acc_only=True), "fp32": dict(), "gelu": dict(act=1),
                             "u8gelu": dict(act=1, fused_u8=True)}
                    variants = [table[v] for v in args.variants.split(",")]
                bfs = [0] if mode == "i8" else [int(b) for b in args.bf.split(",")]
                for v in variants:
                    for bf in bfs:
                        for grp in [int(g) for g in args.groups.split(",")]:
                            r = bench_case(ctx, mode, args.m, k, n, args.iters, tile=tile,
                                           bf=bf, group=grp, uniform=args.uniform_operands,
                                           copies=args.weight_copies,
                                           requantize=args.requantize, **v)
                            print(json.dumps(r), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
