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

Each timed step is bracketed by HIP events on the library's stream, so the
line also reports the median / p10 / p90 step time over the K steps (K = 30
by default); `value` is the wall-clock rate over all K.

Usage: python bench.py [--gpus 1] [--steps 30] [--warmup 5]
"""
import ctypes
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
    "nomic-v1.5-int8": ("nomic-embed-text-v1.5-shaped post-LN encoder (12 layers, 768, 12 heads of "
                        "64, RoPE, SwiGLU 3072), full int8, 64 texts, lengths U[64,256] padded to "
                        "256, mean pooling + L2", "full", 64, 256, 64, 256, 1000),
    "mpnet-base-int8": ("all-mpnet-base-v2-shaped encoder (12 layers, 768, 12 heads of 64, "
                        "relative-position bias), full int8, 64 texts, lengths U[64,256] padded "
                        "to 256, mean pooling + L2", "full", 64, 256, 64, 256, 1000),
    "distilbert-base-int8": ("multi-qa-distilbert-cos-v1-shaped encoder (6 layers, 768, 12 heads "
                             "of 64), full int8, 64 texts, lengths U[64,256] padded to 256, CLS "
                             "pooling + L2", "full", 64, 256, 64, 256, 1000),
    "modernbert-base-w8": ("modernbert-embed-base-shaped pre-LN encoder (22 layers, 768, 12 heads "
                           "of 64, GeGLU 1152, every third layer global, the rest within +-64 "
                           "tokens), weight-only int8, 32 texts, lengths U[256,512] padded to 512, "
                           "mean pooling + L2", "weights", 32, 512, 256, 512, 1000),
}
QUANTS = {"none": 0, "weights": 1, "full": 2}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class StepEvents:
    """HIP events recorded on a stream between steps (hipEventRecord through
    the HIP runtime the library already uses): per-step device times without
    a host synchronization inside the timed loop."""

    def __init__(self, stream, n):
        from rembed_amd import _lib
        self.hip = _lib.hip_runtime()
        self.stream = ctypes.c_void_p(stream)
        self.ev = []
        for _ in range(n + 1):
            e = ctypes.c_void_p()
            assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
            self.ev.append(e)
        self.i = 0

    def mark(self):
        assert self.hip.hipEventRecord(self.ev[self.i], self.stream) == 0
        self.i += 1

    def step_ms(self):
        assert self.hip.hipEventSynchronize(self.ev[self.i - 1]) == 0
        out = []
        for a, b in zip(self.ev[: self.i - 1], self.ev[1: self.i]):
            ms = ctypes.c_float()
            assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
            out.append(ms.value)
        for e in self.ev:
            self.hip.hipEventDestroy(e)
        return np.array(out)


def pct(x, q):
    return float(np.percentile(np.asarray(x, np.float64), q))


def oracle_for(shape, tensors, quant):
    """The oracle model of a synthetic shape's architecture."""
    from oracle import oracle as O
    from rembed_amd import synthetic as S
    if isinstance(shape, S.RopeEncoderShape):
        return O.RopeEncoderOracle(shape, tensors, quant)
    if isinstance(shape, S.DecoderShape):
        return O.DecoderOracle(shape, tensors, quant)
    return O.BertOracle(shape, tensors, quant)


def cpu_baseline(shape, tensors, ids, lens, quant, max_len=None):
    """The reference algorithm restated in C (the oracle) on the host cores,
    with the reference's batch policy (rembed.go:309-330): one serial
    forward per text, texts across all cores (across = min(cores, texts),
    within = 1 here). Full int8 runs on the reference's own kernel shape:
    PackB8VNNI panels and 4x16 VPDPBUSD tiles (vnni_amd64.s /
    vnni512_amd64.s). The whole batch is timed on every core (each text's
    forward timed too: p10/p50/p90 of the per-text rates), and a sample of
    texts on one core. `max_len` truncates the decoders' texts (a full
    28-layer 512-token text takes ~30 s on one core)."""
    from oracle import oracle as O
    cores = os.cpu_count() or 1
    if max_len:
        lens = np.minimum(lens, max_len)
    orc = oracle_for(shape, tensors, quant)
    O.lib.or_set_gemm_impl(1 if quant == 2 else 0)
    try:
        orc.embed_batch(ids[:1], np.minimum(lens[:1], 32), threads=1)  # warm-up
        secs = np.zeros(len(lens))
        t0 = time.perf_counter()
        orc.embed_batch(ids, lens, threads=cores, secs=secs)
        dt = time.perf_counter() - t0
        n1 = min(8, len(lens))
        t1 = time.perf_counter()
        orc.embed_batch(ids[:n1], lens[:n1], threads=1)
        dt1 = time.perf_counter() - t1
    finally:
        O.lib.or_set_gemm_impl(0)
        orc.close()
    per_text = lens.astype(np.float64) / secs
    if quant == 2:
        pk = O.lib.or_vnni_panel_kind()
        kind = ("u8xs8 " + {1: "AVX-VNNI (VEX)", 2: "AVX-512-VNNI (EVEX ymm)",
                            0: "portable"}[pk] + " 4x16 VPDPBUSD tiles on PackB8VNNI panels")
    else:
        kind = {0: "fp32 FMA-chain", 1: "fp32 x int8 FMA-chain"}[quant]
    trunc = f", texts truncated to {max_len} tokens" if max_len else ""
    return {"value": float(lens.sum()) / dt, "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "label": "rembed-algorithm C++ restatement (not the Go binary: no Go toolchain here)",
            "per_text_tokens_per_s": {"p10": pct(per_text, 10), "median": pct(per_text, 50),
                                      "p90": pct(per_text, 90), "texts": len(lens)},
            "single_core": {"value": float(lens[:n1].sum()) / dt1, "cores": 1,
                            "sample": f"first {n1} texts ({int(lens[:n1].sum())} tokens), "
                                      f"{dt1:.2f} s"},
            "sample": f"the whole batch: {len(lens)} texts, {int(lens.sum())} tokens{trunc}, "
                      f"one serial forward per text across {cores} threads, {kind}, "
                      f"{dt:.2f} s"}


def _u8_rows(h):
    """QuantizeRowU8 of every row (pack_vnni.go:85-117), by the oracle."""
    from oracle import oracle as O
    return np.stack([O.quantize_row_u8(r)[0] for r in h])


def oracle_u8_sensitivity(shape, tensors, ids, lens, texts=4):
    """The count of u8_byte_diffs between the oracle and the oracle itself
    with every word-embedding weight moved by one float32 ulp
    (np.nextafter toward +inf): how far a rounding-level change to the input
    carries through the quantized network, layer by layer."""
    from oracle import oracle as O
    nudged = dict(tensors)
    w = np.asarray(tensors["embeddings.word_embeddings.weight"], np.float32)
    nudged["embeddings.word_embeddings.weight"] = np.nextafter(w, np.float32(np.inf))
    a, b = O.BertOracle(shape, tensors, 2), O.BertOracle(shape, nudged, 2)
    rows = []
    for L in range(1, shape.layers + 1):
        diff = 0
        for t in range(texts):
            x = ids[t, :lens[t]]
            diff += int(np.count_nonzero(_u8_rows(a.encode(x, L)) != _u8_rows(b.encode(x, L))))
        rows.append(diff)
    a.close()
    b.close()
    return rows


def u8_byte_diffs(ctx, shape, tensors, ids, lens, texts=4, precisions=(1, 3, "exact")):
    """Per layer, the u8 bytes of the next layer's activation rows
    (QuantizeRowU8 of the hidden states after layer L, pack_vnni.go:85-117)
    that differ between the device's full-int8 forward and the oracle's, over
    the first `texts` texts, for each attention precision and for the
    byte-exact forward (RH_OPT_EXACT): device models of 1..L layers, the
    oracle stopped after L layers, both sides quantized by the oracle's
    quantizer."""
    import dataclasses

    from oracle import oracle as O
    from rembed_amd.model import Model
    orc = O.BertOracle(shape, tensors, 2)
    rows = {p: [] for p in precisions}
    total = 0
    for L in range(1, shape.layers + 1):
        m = Model(ctx, dataclasses.replace(shape, layers=L), tensors, 2)
        want = [_u8_rows(orc.encode(ids[t, :lens[t]], L)) for t in range(texts)]
        total = sum(w.size for w in want)
        for p in precisions:
            if p == "exact":
                m.set_exact(True)
            else:
                m.set_exact(False)
                m.set_attention_precision(p)
            toks = m.embed_tokens(ids[:texts], lens[:texts])
            rows[p].append(sum(int(np.count_nonzero(_u8_rows(toks[t]) != want[t]))
                               for t in range(texts)))
        m.close()
    orc.close()
    return {"per_layer_bytes_differing": {
                (f"attention_precision_{p}" if p != "exact" else "exact_forward"): rows[p]
                for p in precisions},
            "bytes_per_layer": total, "texts": texts,
            "what": "QuantizeRowU8 of the hidden states after each layer (the next "
                    "layer's u8 q|k|v input), device full-int8 forward vs the oracle's"}


def make_workload(name):
    """(shape, tensors) of a workload, synthetic and seeded."""
    from rembed_amd import synthetic as S
    if name.startswith("bert-base"):
        return S.BERT_BASE, S.bert_tensors(S.BERT_BASE, seed=0x5EED0001)
    if name.startswith("mpnet"):
        return S.MPNET_BASE, S.bert_tensors(S.MPNET_BASE, seed=0x5EED0001)
    if name.startswith("distilbert"):
        return S.DISTILBERT_BASE, S.bert_tensors(S.DISTILBERT_BASE, seed=0x5EED0001)
    if name.startswith("minilm"):
        return S.MINILM_L6, S.bert_tensors(S.MINILM_L6, seed=0x5EED0001)
    if name.startswith("qwen3"):
        shape = S.QWEN3_0_6B
        return shape, S.decoder_tensors(shape, seed=0x5EED0001, bf16=True)
    if name.startswith("nomic"):
        return S.NOMIC_V15, S.rope_encoder_tensors(S.NOMIC_V15, seed=0x5EED0001)
    if name.startswith("modernbert"):
        return S.MODERNBERT_BASE, S.rope_encoder_tensors(S.MODERNBERT_BASE, seed=0x5EED0001)
    import dataclasses
    shape = dataclasses.replace(S.GEMMA3_300M, sliding_window=512, sliding_pattern=2,
                                max_seq=2048)
    return shape, S.decoder_tensors(shape, seed=0x5EED0001)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="bert-base-int8",
                    help="default: the configuration the metric is quoted on")
    ap.add_argument("--ffn1", choices=["fused", "onepass", "split"], default="onepass",
                    help="full-int8 FFN1: fused = GELU rows re-quantized inside the GEMM "
                         "(two passes, no fp32 intermediate); onepass = one GEMM pass whose "
                         "workgroups meet per row block on the row |max|; split = fp32 rows + "
                         "QuantizeRowU8")
    ap.add_argument("--no-u8-diff", action="store_true",
                    help="skip the per-layer u8 comparison with the oracle (full int8)")
    ap.add_argument("--forwards-only", action="store_true",
                    help="run only the default forward (warm-up, timed and profiled steps): "
                         "no fp32-attention rate, host-buffer rate, oracle comparison or CPU "
                         "baseline, so a profiler sees one kind of forward")
    ap.add_argument("--graph", choices=["on", "off"], default="off",
                    help="BERT family: replay each batch shape's forward as a recorded HIP "
                         "graph (RH_OPT_GRAPH)")
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
    bert = "embeddings.position_embeddings.weight" in tensors  # the BERT family
    # `value` runs the library's default attention: for the BERT family
    # float32-grade arithmetic (the three-term bf16 split on the q|k|v
    # rows' hi/lo planes), the reference's float32 attention class; for the
    # RoPE family's quantized modes bf16 operands. The other precision and,
    # for the BERT family, the reference-order (byte-exact) forward are
    # timed beside it.
    prec = 3 if (bert or quant == 0) else 1
    model.set_attention_precision(prec)
    if bert:
        model.set_graph(args.graph == "on")
    if quant == 2:
        assert model.quantized_activations(), "full-int8 path did not take"
        model.set_fused_ffn1({"split": 0, "fused": 1, "onepass": 2}[args.ffn1])
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

    # `value`: K steps with nothing but the forward on the stream (plus an
    # event between steps for the per-step distribution).
    ctx.sync()
    ev = StepEvents(ctx.stream, args.steps)
    t0 = time.perf_counter()
    ev.mark()
    for _ in range(args.steps):
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
        ev.mark()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    step_ms = ev.step_ms()
    model.check()

    def rate_with(setup, undo):
        """tokens/s of K more steps with the model reconfigured by setup()."""
        setup()
        model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
        ctx.sync()
        t2 = time.perf_counter()
        for _ in range(args.steps):
            model.embed_device(ids_dev, lens, BATCH, SEQ, out_dev)
        ctx.sync()
        r = tokens * args.steps / (time.perf_counter() - t2)
        undo()
        model.check()
        return r

    # Beside `value`: the other attention precision (bf16 operands with fp32
    # softmax and accumulation, or the fp32-grade split), and for the BERT
    # family the byte-exact forward (RH_OPT_EXACT: LayerNorm sums and
    # attention in the reference's own float32 order).
    other_rate = exact_rate = None
    other = 1 if prec == 3 else 3
    if quant != 0 and not args.forwards_only:
        other_rate = rate_with(lambda: model.set_attention_precision(other),
                               lambda: model.set_attention_precision(prec))
    if bert and not args.forwards_only:
        exact_rate = rate_with(lambda: model.set_exact(True), lambda: model.set_exact(False))

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
    gemm_plain = ctx.profile_read(gkind)
    # the one-pass FFN1 launches (full int8): GEMM + GELU + QuantizeRowU8
    fused = ctx.profile_read(5)
    gemm = {k: gemm_plain[k] + fused[k] for k in gemm_plain}
    attn = ctx.profile_read(3)
    split = ctx.profile_read(4)  # bf16 split of the W8/fp32 GEMMs' activations
    ctx.profile(False)
    model.set_streams(args.streams)

    ms_per_step = elapsed * 1e3 / args.steps
    value = tokens * args.steps / elapsed
    per_launch_ms = gemm["total_ms"] / max(1, gemm["launches"])

    def rate(st):  # TOP/s (TFLOP/s) of a profile tally
        return st["total_ops"] / (st["total_ms"] * 1e-3) / 1e12 if st["total_ms"] else 0.0
    achieved = gemm["total_ops"] / (gemm["total_ms"] * 1e-3) / 1e12  # TOP/s
    gemm_ms_step = gemm["total_ms"] / args.steps
    attn_ms_step = attn["total_ms"] / args.steps
    split_ms_step = split["total_ms"] / args.steps
    log(f"{ms_per_step:.3f} ms/step, {value:,.0f} tokens/s; GEMM {gemm_ms_step:.3f} "
        f"ms/step over {gemm['launches'] // args.steps} launches = {achieved:.1f} TOP/s; "
        f"attention {attn_ms_step:.3f} ms/step")

    # The same forward through the host-buffer boundary (int64 ids up,
    # vectors back over PCIe each batch, one synchronous call per batch),
    # reported beside `value`, never as it.
    host_rate, host_ms = None, []
    vec = out_dev.download(np.float32, (BATCH, shape.hidden))
    if not args.forwards_only:
        host_steps = max(1, args.steps)
        model.embed(ids, lens)
        for _ in range(host_steps):
            t0 = time.perf_counter()
            host_vec = model.embed(ids, lens)
            host_ms.append((time.perf_counter() - t0) * 1e3)
        host_rate = tokens * host_steps / (sum(host_ms) * 1e-3)
        assert np.array_equal(vec, host_vec), "host-buffer and device-resident forwards differ"
    cfg_note = {"streams": args.streams}
    if bert:
        cfg_note["graph"] = args.graph
    if quant == 2:
        cfg_note["ffn1"] = args.ffn1
        cfg_note["qkv_rows"] = ("bf16 hi/lo planes of the fp32 rows (the q|k|v GEMM's epilogue "
                                "writes the split)" if prec == 3 and bert else "fp32")
    cfg_note["attention"] = (
        "fp32-grade: q|k|v and P split into bf16 hi/lo, three MFMA products, fp32 softmax "
        "and accumulation (RH_OPT_ATTN_PRECISION 3)" if prec == 3 else
        "bf16 MFMA operands, fp32 softmax and accumulation (RH_OPT_ATTN_PRECISION 1)")
    norms = np.linalg.norm(vec.astype(np.float64), axis=1)
    assert np.all(np.abs(norms - 1) < 1e-4), "embeddings are not unit vectors"

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_i8_traffic.json")
    if args.workload == "bert-base-int8" and os.path.exists(tpath):  # measured on this workload
        traffic = json.load(open(tpath)).get("bytes_per_launch")

    u8diff = None
    if quant == 2 and bert and not (args.no_cpu_baseline or args.no_u8_diff or args.forwards_only):
        log("comparing u8 activations with the oracle, layer by layer")
        u8diff = u8_byte_diffs(ctx, shape, tensors, ids, lens)
        u8diff["oracle_vs_oracle_1ulp_embeddings"] = oracle_u8_sensitivity(
            shape, tensors, ids, lens)
        log(f"u8 bytes differing per layer of {u8diff['bytes_per_layer']}: "
            f"{u8diff['per_layer_bytes_differing']}; oracle vs itself with 1-ulp word "
            f"embeddings {u8diff['oracle_vs_oracle_1ulp_embeddings']}")

    baseline = None
    if not (args.no_cpu_baseline or args.forwards_only):
        log("timing the CPU baseline")
        trunc = {"qwen3-0.6b-w8": 48, "gemma-300m-w8": 64, "modernbert-base-w8": 160}.get(
            args.workload)
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
        "dtype": {2: "int8", 1: "int8 weights x bf16(a) activations (one bf16 term)",
                  0: "fp32 (3xbf16 split)"}[quant],
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
            "kernel": ("gemm_i8_kernel / gemm_i8f_kernel" if quant == 2 else
                       "gemm_planes_kernel") +
                      f" (all {gemm['launches'] // args.steps} GEMM launches per step" +
                      (f"; {fused['launches'] // args.steps} of them FFN1 with the GELU + "
                       "QuantizeRowU8 row pass in the epilogue, counted at GEMM ops)"
                       if fused["launches"] else ")"),
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "ops_per_launch": gemm["total_ops"] / max(1, gemm["launches"]),
            "avg_launch_ms": round(per_launch_ms, 5),
            **({"gemm_only": {
                "launches_per_step": gemm_plain["launches"] // args.steps,
                "achieved": round(rate(gemm_plain), 2),
                "frac": round(rate(gemm_plain) / peak, 4),
                "avg_launch_ms": round(gemm_plain["total_ms"] / max(1, gemm_plain["launches"]), 5)},
               "fused_ffn1": {
                "launches_per_step": fused["launches"] // args.steps,
                "gemm_achieved": round(rate(fused), 2),
                "gemm_frac": round(rate(fused) / peak, 4),
                "avg_launch_ms": round(fused["total_ms"] / max(1, fused["launches"]), 5)}}
               if fused["launches"] else {}),
        },
        "profiled_ms_per_step": round(profiled_ms_per_step, 4),
        "gemm_ms_per_step": round(gemm_ms_step, 4),
        "attention_ms_per_step": round(attn_ms_step, 4),
        "bf16_split_ms_per_step": round(split_ms_step, 4),
        "step_ms": {"median": round(pct(step_ms, 50), 4), "p10": round(pct(step_ms, 10), 4),
                    "p90": round(pct(step_ms, 90), 4), "steps": int(step_ms.size),
                    "clock": "HIP events between steps on the library stream"},
        "median_tokens_per_s": round(tokens / (pct(step_ms, 50) * 1e-3), 1),
        ("bf16_attention_tokens_per_s" if other == 1 else "fp32_attention_tokens_per_s"):
            None if other_rate is None else round(other_rate, 1),
        "exact_tokens_per_s": None if exact_rate is None else round(exact_rate, 1),
        "pcie_inclusive_tokens_per_s": None if host_rate is None else round(host_rate, 1),
        "pcie_inclusive_step_ms": None if not host_ms else {
            "median": round(pct(host_ms, 50), 4), "p10": round(pct(host_ms, 10), 4),
            "p90": round(pct(host_ms, 90), 4)},
        "u8_vs_oracle": u8diff,
        "padded_slots_per_s": round(BATCH * SEQ * args.steps / elapsed, 1),
        "cpu_baseline": baseline,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
