"""Summaries of rocprofv3 output for the committed profiles.

    python -m rembed_amd.profsummary stats  <kernel_stats.csv> <steps> <title> <command>
    python -m rembed_amd.profsummary trace  <kernel_trace.csv> <first_kernel> <skip> <count>
                                     <title> <command> [<int8 GEMM rows M>]
    python -m rembed_amd.profsummary traffic <fetch_dir_csv> <write_dir_csv>
                                     <copy_fetch_csv> <copy_write_csv> <copy_mib> <command>
    python -m rembed_amd.profsummary pmc <counter_collection.csv> <command>
    python -m rembed_amd.profsummary waits <counter_collection.csv> <command>

`stats` renders a --kernel-trace --stats table (per-kernel calls, average
and per-step time). `traffic` turns two --pmc runs (FETCH_SIZE, then
WRITE_SIZE, KiB per dispatch) into bytes per launch past the L2, each counter
scaled by what it reads for a plain device copy of known size, and prints the
JSON that bench.py reads for the GEMM's `roofline.traffic`. FETCH_SIZE counts
the L2's read misses (requests to the fabric, served by the MALL or HBM), not
the bytes a kernel loads: reads that hit the L2 do not appear in it. `pmc` renders one
--pmc pass of SQ instruction and busy counters per kernel: MFMA busy share,
VALU and LDS instructions per MFMA, LDS bank-conflict share. `waits` renders
a pass of SQ_WAVE_CYCLES, SQ_WAIT_ANY, SQ_WAIT_INST_ANY, SQ_ACTIVE_INST_VALU
and SQ_ACTIVE_INST_LDS as shares of the waves' summed lifetime.
"""
import collections
import csv
import json
import sys

# the full-int8 GEMM family: the LDS-staged tiles and the fragment-ordered-B tiles
GEMM = ("gemm_i8_kernel<", "gemm_i8f_kernel<")


def _kernel_means(path):
    vals = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: (len(v), sum(v) / len(v)) for k, v in vals.items()}


def stats(path, steps, title, command):
    rows = list(csv.DictReader(open(path)))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    print(f"# {title}\n\nCommand: `{command}`\n")
    print("| kernel | calls | avg µs | µs per step | share |")
    print("|---|---:|---:|---:|---:|")
    for r in rows:
        t = float(r["TotalDurationNs"])
        print(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{t / 1e3 / steps:.1f} | {100 * t / total:.1f}% |")
    gemm = [r for r in rows if any(g in r["Name"] for g in GEMM)]
    gt = sum(float(r["TotalDurationNs"]) for r in gemm)
    gc = sum(int(r["Calls"]) for r in gemm)
    if gc:
        print(f"\nAll int8 GEMM launches: {gc} calls, average {gt / gc / 1e3:.2f} µs, "
              f"{gt / 1e3 / steps:.1f} µs per step ({steps} steps incl. warm-up).")


# The int8 GEMMs of one BERT-base layer in launch order: name, K, N, bytes
# per output element (QKV rows go to fp32-grade attention as bf16 hi/lo
# planes, 2 + 2 bytes; the one-pass FFN1 writes FFN2's u8 rows, its launch
# also runs GELU + QuantizeRowU8 over them).
BERT_BASE_I8_LAYER = [("QKV", 768, 2304, 4), ("O", 768, 768, 4),
                      ("FFN1 + GELU + QuantizeRowU8", 768, 3072, 1), ("FFN2", 3072, 768, 4)]
INT8_PEAK_TOPS, HBM_PEAK_GBS = 5000.0, 8000.0


def gemm_rooflines(times, m, layer=BERT_BASE_I8_LAYER, family="gemm_i8_kernel"):
    """Per-shape roofline of the int8 GEMMs: times[i] are the durations (µs)
    of the i-th such launch of each forward, in launch order; launch i runs
    layer[i % len(layer)]. Algorithmic bytes: u8 A, s8 B, the output, row
    scales and column scales / sums / bias."""
    print(f"\nPer-shape roofline of the `{family}` launches (M = {m}; peaks 5.0 POP/s "
          f"int8 MFMA, 8 TB/s HBM):\n")
    print("| GEMM | K × N | avg µs | TOP/s | % int8 peak | algorithmic MB | GB/s | "
          "% HBM peak | bound at peak |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---|")
    tot_t = tot_min = 0.0
    for i, (name, k, n, ob) in enumerate(layer):
        ts = times[i::len(layer)]
        if not ts:
            continue
        us = sum(ts) / len(ts)
        ops = 2.0 * m * k * n
        by = m * k + k * n + m * n * ob + 4 * m + 12 * n
        tops = ops / (us * 1e-6) / 1e12
        gbs = by / (us * 1e-6) / 1e9
        t_mfma, t_hbm = ops / (INT8_PEAK_TOPS * 1e12) * 1e6, by / (HBM_PEAK_GBS * 1e9) * 1e6
        tot_t += us
        tot_min += max(t_mfma, t_hbm)
        print(f"| {name} | {k} × {n} | {us:.2f} | {tops:.0f} | {100 * tops / INT8_PEAK_TOPS:.1f} % "
              f"| {by / 1e6:.1f} | {gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} % | "
              f"{'HBM' if t_hbm > t_mfma else 'MFMA'} ({max(t_mfma, t_hbm):.1f} µs) |")
    if tot_t:
        print(f"\nThe layer's int8 GEMMs take {tot_t:.1f} µs against {tot_min:.1f} µs at the "
              f"binding peak of each: {100 * tot_min / tot_t:.1f} % of the combined roofline.")


def trace(path, first, skip, count, title, command, gemm_m=0):
    """Per-forward kernel times from a --kernel-trace CSV: the trace is cut
    into forwards at each launch whose name contains `first` (the forward's
    first kernel), the first `skip` forwards are dropped and the next `count`
    are averaged, so warm-up and the other forwards a run makes (different
    options, host-buffer calls) stay out of the table."""
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if first in r["Kernel_Name"]]
    if len(starts) < skip + count + 1:
        raise SystemExit(f"{len(starts)} forwards in the trace, need {skip + count + 1}")
    sel = rows[starts[skip]:starts[skip + count]]
    per = collections.defaultdict(list)
    for r in sel:
        per[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in per.values())
    span = (int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])) / 1e3 / count
    print(f"# {title}\n\nCommand: `{command}`\n")
    print(f"Forwards {skip + 1}-{skip + count} of the run (cut at each `{first}` launch), one "
          f"stream: kernel time {total / count:.1f} µs per forward, {span:.1f} µs from the "
          f"first kernel's start to the last one's end.\n")
    print("| kernel | calls per forward | avg µs | µs per forward | share |")
    print("|---|---:|---:|---:|---:|")
    for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{name[:90]}` | {len(v) / count:g} | {sum(v) / len(v):.2f} | "
              f"{sum(v) / count:.1f} | {100 * sum(v) / total:.1f}% |")
    if gemm_m:
        order = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in sel
                 if "gemm_i8_kernel<" in r["Kernel_Name"]
                 or "gemm_i8f_kernel<" in r["Kernel_Name"]]
        per_fwd = len(order) // count
        times = [[] for _ in range(per_fwd)]
        for j, t in enumerate(order):
            times[j % per_fwd].append(t)
        # launch i of a forward is layer shape i % 4: flatten per shape
        by_shape = [[] for _ in BERT_BASE_I8_LAYER]
        for i, ts in enumerate(times):
            by_shape[i % len(BERT_BASE_I8_LAYER)].extend(ts)
        gemm_rooflines([sum(v) / len(v) for v in by_shape], gemm_m)
    for fam in ("gemm_i8_kernel", "gemm_i8f_kernel", "gemm_planes_kernel", "gemm_bf16_kernel"):
        g = [x for k, v in per.items() if fam + "<" in k for x in v]
        if g:
            print(f"\nAll `{fam}` launches: {len(g) / count:g} per forward, average "
                  f"{sum(g) / len(g):.2f} µs, {sum(g) / count:.1f} µs per forward "
                  f"({100 * sum(g) / total:.1f}% of the kernel time).")


# MI355X: 8 XCDs of 32 CUs, 4 SIMDs per CU. GRBM_GUI_ACTIVE sums the XCDs'
# active cycles; SQ_VALU_MFMA_BUSY_CYCLES sums every SIMD's MFMA-busy cycles.
XCDS, CUS, SIMDS = 8, 256, 4


def pmc(path, command):
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(path)):
        per[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    print("# Instruction mix and MFMA busy share per kernel (rocprofv3 --pmc)\n")
    print(f"Command: `{command}`\n")
    print("MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x "
          "4 SIMDs); counters are means per dispatch.\n")
    print("| kernel | dispatches | waves | MFMA instr | MFMA busy | VALU / MFMA | "
          "LDS instr / MFMA | LDS bank-conflict cycles / LDS active |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")

    def mean(c, k):
        v = c.get(k)
        return sum(v) / len(v) if v else float("nan")

    rows = sorted(per.items(), key=lambda kv: -mean(kv[1], "GRBM_GUI_ACTIVE") *
                  len(kv[1].get("GRBM_GUI_ACTIVE", [])))
    for name, c in rows:
        n = len(c.get("SQ_WAVES", []))
        mf = mean(c, "SQ_INSTS_MFMA")
        active = mean(c, "GRBM_GUI_ACTIVE") / XCDS
        busy = mean(c, "SQ_VALU_MFMA_BUSY_CYCLES") / (active * CUS * SIMDS) if active else 0.0
        per_mf = (lambda k: f"{mean(c, k) / mf:.1f}") if mf else (lambda k: "-")
        lds_act = mean(c, "SQ_ACTIVE_INST_LDS")
        conf = f"{100 * mean(c, 'SQ_LDS_BANK_CONFLICT') / lds_act:.1f}%" if lds_act else "-"
        print(f"| `{name[:80]}` | {n} | {mean(c, 'SQ_WAVES'):.0f} | {mf:.0f} | "
              f"{100 * busy:.1f}% | {per_mf('SQ_INSTS_VALU')} | {per_mf('SQ_INSTS_LDS')} | {conf} |")


def traffic(fetch, write, cfetch, cwrite, copy_mib, command):
    f, w = _kernel_means(fetch), _kernel_means(write)
    cf, cw = _kernel_means(cfetch), _kernel_means(cwrite)
    copy_kib = copy_mib * 1024.0
    # the copy kernel: the launch named "copy" that writes the most
    ck = max((k for k in cw if "copy" in k.lower()), key=lambda k: cw[k][1])
    f_scale = copy_kib / cf[ck][1]
    w_scale = copy_kib / cw[ck][1]
    print("# Traffic past the L2 per launch (rocprofv3 --pmc)\n")
    print(f"Command: `{command}`\n")
    print(f"Calibration: a {copy_mib} MiB device copy (`{ck}`) reads FETCH_SIZE "
          f"{cf[ck][1]:.0f} KiB and WRITE_SIZE {cw[ck][1]:.0f} KiB per launch, so the "
          f"counters are scaled by {f_scale:.3f} (fetch) and {w_scale:.3f} (write).\n")
    print("Fetch = L2 read misses (FETCH_SIZE: requests that leave the L2 for the MALL or "
          "HBM); reads served by the L2 are not in it. Write = bytes written back past the "
          "L2 (WRITE_SIZE).\n")
    print("| kernel | launches | L2-miss read MB | write MB | total MB |")
    print("|---|---:|---:|---:|---:|")
    g_n = g_b = 0.0
    for k in f:
        if k not in w:
            continue
        n = f[k][0]
        fb = f[k][1] * 1024 * f_scale
        wb = w[k][1] * 1024 * w_scale
        print(f"| `{k[:90]}` | {n} | {fb / 1e6:.1f} | {wb / 1e6:.1f} | {(fb + wb) / 1e6:.1f} |")
        if any(g in k for g in GEMM):
            g_n += n
            g_b += n * (fb + wb)
    out = {"bytes_per_launch": g_b / g_n if g_n else None, "launches": int(g_n),
           "fetch_scale": f_scale, "write_scale": w_scale}
    print(f"\nAverage over all int8 GEMM launches (`gemm_i8_kernel`, `gemm_i8f_kernel`): "
          f"{out['bytes_per_launch'] / 1e6:.1f} MB per launch.\n")
    print("```json\n" + json.dumps(out) + "\n```")
    return out


def waits(path, command):
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(path)):
        per[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))

    def mean(k, c):
        v = per[k].get(c)
        return sum(v) / len(v) if v else 0.0
    print("## Where the waves' cycles go\n")
    print(f"Command: `{command}`\n")
    print("Shares of SQ_WAVE_CYCLES (the summed lifetime of the kernel's waves): waiting on "
          "any dependency (s_waitcnt on loads or LDS, barriers: SQ_WAIT_ANY), waiting to "
          "issue (SQ_WAIT_INST_ANY), and issuing VALU / LDS instructions.\n")
    print("| kernel | wait (any) | wait to issue | VALU issue | LDS issue |")
    print("|---|---:|---:|---:|---:|")
    rows = sorted(per, key=lambda k: -mean(k, "SQ_WAVE_CYCLES") * len(per[k]["SQ_WAVE_CYCLES"]))
    for k in rows:
        wc = mean(k, "SQ_WAVE_CYCLES")
        if wc <= 0 or "rocclr" in k:
            continue
        sh = [mean(k, c) / wc for c in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_VALU",
                                        "SQ_ACTIVE_INST_LDS")]
        print(f"| `{k[:80]}` | " + " | ".join(f"{100 * x:.0f}%" for x in sh) + " |")


if __name__ == "__main__":
    if sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3])
    elif sys.argv[1] == "trace":
        trace(sys.argv[2], sys.argv[3], int(sys.argv[4]), int(sys.argv[5]), sys.argv[6],
              sys.argv[7], int(sys.argv[8]) if len(sys.argv) > 8 else 0)
    elif sys.argv[1] == "waits":
        waits(sys.argv[2], sys.argv[3])
    elif sys.argv[1] == "stats":
        stats(sys.argv[2], int(sys.argv[3]), sys.argv[4], sys.argv[5])
    elif sys.argv[1] == "traffic":
        o = traffic(*sys.argv[2:6], int(sys.argv[6]), sys.argv[7])
        if len(sys.argv) > 8:
            json.dump(o, open(sys.argv[8], "w"))
