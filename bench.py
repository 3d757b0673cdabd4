"""Benchmark: BERT-base full-int8 encoder, 64 texts x up to 256 tokens, 1 MI355X.

A step is one device-resident forward (embed -> 12 layers -> CLS pool -> L2)
over the whole batch; token ids are already in HBM when timing starts and
the pooled vectors stay there. value = real tokens / second (sum of the
texts' lengths, not padded slots). The int8 GEMM launches are timed with
HIP events on the library's stream during the timed steps, which gives the
roofline figure; the CPU baseline is the oracle's restatement of the
reference algorithm on the host cores over a bounded sample of texts.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "tokens/sec on 1 MI355X, BERT-base int8 bs64x256; GEMM TFLOPS % MFMA peak"
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, TOP/s
BATCH, SEQ, LEN_LO, LEN_HI = 64, 256, 64, 256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(shape, tensors, ids, lens, quant):
    """Oracle (port of the reference algorithm) on the host cores: one serial
    forward per text, texts fanned out across threads (rembed.go:309-330)."""
    from oracle import oracle as O
    threads = min(16, os.cpu_count() or 1)
    n = min(len(lens), threads)
    orc = O.BertOracle(shape, tensors, quant)
    orc.embed_batch(ids[:1], lens[:1], threads=1)  # warm-up
    t0 = time.perf_counter()
    orc.embed_batch(ids[:n], lens[:n], threads=threads)
    dt = time.perf_counter() - t0
    orc.close()
    return {"value": float(lens[:n].sum()) / dt, "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} texts of the same batch ({int(lens[:n].sum())} tokens), "
                      f"one serial forward per text across {threads} threads, "
                      f"AVX-512-VNNI u8xs8 dot products, {dt:.2f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ffn1", choices=["fused", "split"], default="split",
                    help="full-int8 FFN1: fused = GELU rows re-quantized inside the GEMM "
                         "(two passes, no fp32 intermediate); split = fp32 rows + QuantizeRowU8")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    from rembed_amd import tensor as T
    from rembed_amd.model import QUANT_FULL, Model
    from rembed_amd.synthetic import BERT_BASE, bert_tensors, token_batch

    shape = BERT_BASE
    log("generating synthetic BERT-base weights")
    tensors = bert_tensors(shape, seed=0x5EED0001)
    ids, lens = token_batch(BATCH, SEQ, LEN_LO, LEN_HI, vocab=shape.vocab, seed=0x5EED0002)
    tokens = int(lens.sum())

    ctx = T.Context(0)
    model = Model(ctx, shape, tensors, QUANT_FULL)
    assert model.quantized_activations(), "full-int8 path did not take"
    model.set_fused_ffn1(args.ffn1 == "fused")
    ids_dev = ctx.upload(ids)
    out_dev = ctx.alloc(BATCH * shape.hidden * 4)

    for _ in range(args.warmup):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
    model.check()
    ctx.sync()

    ctx.profile(True)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    model.check()
    gemm = ctx.profile_read(0)
    attn = ctx.profile_read(3)
    ctx.profile(False)

    ms_per_step = elapsed * 1e3 / args.steps
    value = tokens * args.steps / elapsed
    per_launch_ms = gemm["total_ms"] / max(1, gemm["launches"])
    achieved = gemm["total_ops"] / (gemm["total_ms"] * 1e-3) / 1e12  # TOP/s
    gemm_ms_step = gemm["total_ms"] / args.steps
    attn_ms_step = attn["total_ms"] / args.steps
    log(f"{ms_per_step:.3f} ms/step, {value:,.0f} tokens/s; int8 GEMM {gemm_ms_step:.3f} "
        f"ms/step over {gemm['launches'] // args.steps} launches = {achieved:.1f} TOP/s; "
        f"attention {attn_ms_step:.3f} ms/step")

    vec = out_dev.download(np.float32, (BATCH, shape.hidden))
    norms = np.linalg.norm(vec.astype(np.float64), axis=1)
    assert np.all(np.abs(norms - 1) < 1e-4), "embeddings are not unit vectors"

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_i8_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("bytes_per_launch")

    baseline = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline sample")
        baseline = cpu_baseline(shape, tensors, ids, lens, 2)
        log(f"cpu baseline {baseline['value']:,.1f} tokens/s")

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init N(0,0.02) weights, uniform token ids)",
        "config": {
            "workload": "BERT-base-shaped encoder, full int8 (u8 x s8 GEMMs, int32 acc), "
                        "64 texts, lengths U[64,256] padded to 256, CLS pooling + L2, "
                        "texts packed varlen (M = sum of lengths)",
            "global_batch": BATCH, "seq_len": SEQ, "layers": shape.layers,
            "hidden": shape.hidden, "heads": shape.heads,
            "intermediate": shape.intermediate, "real_tokens": tokens,
            "gemm_rows_M": tokens, "ffn1": args.ffn1, "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_i8_kernel (all 48 int8 GEMM launches per step)",
            "achieved": round(achieved, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "ops_per_launch": gemm["total_ops"] / max(1, gemm["launches"]),
            "avg_launch_ms": round(per_launch_ms, 5),
        },
        "gemm_ms_per_step": round(gemm_ms_step, 4),
        "attention_ms_per_step": round(attn_ms_step, 4),
        "padded_slots_per_s": round(BATCH * SEQ * args.steps / elapsed, 1),
        "cpu_baseline": baseline,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
