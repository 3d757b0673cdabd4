"""Benchmark: BERT-base full-int8 encoder, 64 texts x up to 256 tokens, 1 MI355X.

A step is one device-resident forward (embed -> 12 layers -> CLS pool -> L2)
over the whole batch; token ids are already in HBM when timing starts and
the pooled vectors stay there. value = real tokens / second (sum of the
texts' lengths, not padded slots) over K steps with nothing else on the
stream. A second pass of K steps attaches HIP events to every GEMM dispatch
on the library's stream, which gives the roofline figure (the events cost a
few µs per launch, so that pass is timed apart). The CPU baseline is the
oracle's restatement of the reference algorithm on the host cores over a
bounded sample of texts. --workload selects the other configurations.

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
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (the W8 and fp32 GEMMs run on it)

# The configurations the metric names (the default) and the other encoder
# shapes, each with its own GEMM mode: name -> (description, quant, batch,
# seq, len_lo, len_hi, id_lo).
WORKLOADS = {
    "bert-base-int8": ("BERT-base-shaped encoder, full int8 (u8 x s8 GEMMs, int32 acc), 64 texts, "
                       "lengths U[64,256] padded to 256, CLS pooling + L2",
                       "full", 64, 256, 64, 256, 1000),
    "bert-base-fp32": ("BERT-base-shaped encoder, fp32 GEMMs, 64 texts, lengths U[64,256] padded "
                       "to 256, CLS pooling + L2", "none", 64, 256, 64, 256, 1000),
    "minilm-w8": ("MiniLM-L6-shaped encoder, weight-only int8, 32 texts, lengths U[16,128] padded "
                  "to 128, mean pooling + L2", "weights", 32, 128, 16, 128, 1000),
    "qwen3-0.6b-w8": ("Qwen3-Embedding-0.6B-shaped causal decoder (28 layers, 1024, 16/8 heads of "
                      "128, SwiGLU 3072), bf16-rounded weights then weight-only int8, 32 x 512, "
                      "last-token pooling", "weights", 32, 512, 512, 512, 0),
    "gemma-300m-w8": ("EmbeddingGemma-300m-shaped bidirectional Gemma3 (24 layers, 768, 3/1 heads of "
                      "256, GeGLU 1152, alternating window-512 / global), weight-only int8, "
                      "16 x 2048, mean pooling + Dense 768-3072-768", "weights", 16, 2048, 2048,
                      2048, 0),
}
QUANTS = {"none": 0, "weights": 1, "full": 2}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(shape, tensors, ids, lens, quant, max_len=None):
    """Oracle (port of the reference algorithm) on the host cores: one serial
    forward per text, texts fanned out across threads (rembed.go:309-330).
    `max_len` truncates the sample's texts (the decoders' full texts would
    take minutes per text on one core)."""
    from oracle import oracle as O
    threads = min(16, os.cpu_count() or 1)
    n = min(len(lens), threads)
    lens = np.minimum(lens[:n], max_len) if max_len else lens[:n]
    dec = hasattr(shape, "arch")
    orc = O.DecoderOracle(shape, tensors, quant) if dec else O.BertOracle(shape, tensors, quant)
    orc.embed_batch(ids[:1], np.minimum(lens[:1], 32), threads=1)  # warm-up
    t0 = time.perf_counter()
    orc.embed_batch(ids[:n], lens, threads=threads)
    dt = time.perf_counter() - t0
    orc.close()
    kind = {0: "fp32 FMA-chain", 1: "fp32 x int8 FMA-chain",
            2: f"u8xs8 {'AVX-512-VNNI' if O.lib.or_vnni_kind() == 2 else 'portable'}"}[quant]
    trunc = f", truncated to {max_len} tokens" if max_len else ""
    return {"value": float(lens.sum()) / dt, "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} texts of the same batch ({int(lens.sum())} tokens{trunc}), "
                      f"one serial forward per text across {threads} threads, "
                      f"{kind} dot products, {dt:.2f} s"}


def make_workload(name):
    """(shape, tensors) of a workload, synthetic and seeded."""
    from rembed_amd import synthetic as S
    if name.startswith("bert-base"):
        return S.BERT_BASE, S.bert_tensors(S.BERT_BASE, seed=0x5EED0001)
    if name.startswith("minilm"):
        return S.MINILM_L6, S.bert_tensors(S.MINILM_L6, seed=0x5EED0001)
    if name.startswith("qwen3"):
        shape = S.QWEN3_0_6B
        return shape, S.decoder_tensors(shape, seed=0x5EED0001, bf16=True)
    import dataclasses
    shape = dataclasses.replace(S.GEMMA3_300M, sliding_window=512, sliding_pattern=2,
                                max_seq=2048)
    return shape, S.decoder_tensors(shape, seed=0x5EED0001)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="bert-base-int8",
                    help="default: the configuration the metric is quoted on")
    ap.add_argument("--ffn1", choices=["fused", "split"], default="split",
                    help="full-int8 FFN1: fused = GELU rows re-quantized inside the GEMM "
                         "(two passes, no fp32 intermediate); split = fp32 rows + QuantizeRowU8")
    ap.add_argument("--streams", type=int, choices=[1, 2, 3, 4], default=2,
                    help="run a batch as this many parts of whole texts on as many streams "
                         "(default 2); the roofline pass always runs one stream")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the library has no multi-GPU path; texts "
              f"shard across GPUs as independent replicas (--gpus {args.gpus} requested)",
              file=sys.stderr)
        sys.exit(2)

    from rembed_amd import tensor as T
    from rembed_amd.model import Model
    from rembed_amd.synthetic import token_batch

    desc, qname, BATCH, SEQ, LEN_LO, LEN_HI, ID_LO = WORKLOADS[args.workload]
    quant = QUANTS[qname]
    log(f"generating synthetic weights for {args.workload}")
    shape, tensors = make_workload(args.workload)
    ids, lens = token_batch(BATCH, SEQ, LEN_LO, LEN_HI, vocab=shape.vocab, id_lo=ID_LO,
                            seed=0x5EED0002)
    tokens = int(lens.sum())

    ctx = T.Context(0)
    model = Model(ctx, shape, tensors, quant)
    model.set_streams(args.streams)
    if quant == 2:
        assert model.quantized_activations(), "full-int8 path did not take"
        model.set_fused_ffn1(args.ffn1 == "fused")
    elif quant == 1:
        assert model.quantized() and not model.quantized_activations()
    gkind = {2: 0, 1: 1, 0: 2}[quant]  # profile kind of the workload's GEMMs
    peak = INT8_PEAK_TOPS if quant == 2 else BF16_PEAK_TFLOPS
    ids_dev = ctx.upload(ids)
    out_dev = ctx.alloc(BATCH * shape.hidden * 4)

    for _ in range(args.warmup):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
    model.check()
    ctx.sync()

    # `value`: K steps with nothing but the forward on the stream.
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    model.check()

    # The roofline: the same K steps again with a HIP event pair attached to
    # every GEMM / attention / split dispatch (the library's profiler, on
    # the stream the kernels run on). The events cost a few µs per launch,
    # so these steps are timed apart from `value`, and on one stream: with
    # two, the parts' kernels overlap and each launch's duration would count
    # time the GPU spent on the other part.
    model.set_streams(1)
    ctx.profile(True)
    ctx.sync()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
    ctx.sync()
    profiled_ms_per_step = (time.perf_counter() - t1) * 1e3 / args.steps
    model.check()
    gemm = ctx.profile_read(gkind)
    attn = ctx.profile_read(3)
    split = ctx.profile_read(4)  # bf16 split of the W8/fp32 GEMMs' activations
    ctx.profile(False)
    model.set_streams(args.streams)

    ms_per_step = elapsed * 1e3 / args.steps
    value = tokens * args.steps / elapsed
    per_launch_ms = gemm["total_ms"] / max(1, gemm["launches"])
    achieved = gemm["total_ops"] / (gemm["total_ms"] * 1e-3) / 1e12  # TOP/s
    gemm_ms_step = gemm["total_ms"] / args.steps
    attn_ms_step = attn["total_ms"] / args.steps
    split_ms_step = split["total_ms"] / args.steps
    log(f"{ms_per_step:.3f} ms/step, {value:,.0f} tokens/s; GEMM {gemm_ms_step:.3f} "
        f"ms/step over {gemm['launches'] // args.steps} launches = {achieved:.1f} TOP/s; "
        f"attention {attn_ms_step:.3f} ms/step")

    # The same forward through the host-buffer boundary (ids up, vectors
    # back over PCIe each batch), reported beside `value`, never as it.
    host_steps = max(1, min(args.steps, 20))
    model.embed(ids, lens)
    t0 = time.perf_counter()
    for _ in range(host_steps):
        host_vec = model.embed(ids, lens)
    host_rate = tokens * host_steps / (time.perf_counter() - t0)

    vec = out_dev.download(np.float32, (BATCH, shape.hidden))
    assert np.array_equal(vec, host_vec), "host-buffer and device-resident forwards differ"
    cfg_note = {"streams": args.streams}
    if quant == 2:
        cfg_note["ffn1"] = args.ffn1
    norms = np.linalg.norm(vec.astype(np.float64), axis=1)
    assert np.all(np.abs(norms - 1) < 1e-4), "embeddings are not unit vectors"

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_i8_traffic.json")
    if quant == 2 and os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("bytes_per_launch")

    baseline = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline sample")
        trunc = {"qwen3-0.6b-w8": 48, "gemma-300m-w8": 64}.get(args.workload)
        baseline = cpu_baseline(shape, tensors, ids, lens, quant, max_len=trunc)
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
        "dtype": {2: "int8", 1: "int8 weights x bf16-split activations", 0: "fp32 (3xbf16 split)"}[quant],
        "data": "synthetic (random-init N(0,0.02) weights, uniform token ids)",
        "config": {
            "workload": desc + ", texts packed varlen (M = sum of lengths)",
            "name": args.workload,
            "global_batch": BATCH, "seq_len": SEQ, "layers": shape.layers,
            "hidden": shape.hidden, "heads": shape.heads,
            "intermediate": shape.intermediate, "real_tokens": tokens,
            "gemm_rows_M": tokens, "parallelism": "none (1 GPU)", **cfg_note,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": ("gemm_i8_kernel" if quant == 2 else "gemm_planes_kernel") +
                      f" (all {gemm['launches'] // args.steps} GEMM launches per step)",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "ops_per_launch": gemm["total_ops"] / max(1, gemm["launches"]),
            "avg_launch_ms": round(per_launch_ms, 5),
        },
        "profiled_ms_per_step": round(profiled_ms_per_step, 4),
        "gemm_ms_per_step": round(gemm_ms_step, 4),
        "attention_ms_per_step": round(attn_ms_step, 4),
        "bf16_split_ms_per_step": round(split_ms_step, 4),
        "pcie_inclusive_tokens_per_s": round(host_rate, 1),
        "padded_slots_per_s": round(BATCH * SEQ * args.steps / elapsed, 1),
        "cpu_baseline": baseline,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
