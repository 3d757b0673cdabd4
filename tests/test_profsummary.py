"""The rocprofv3 summaries behind the committed profiles and the bench's
roofline.traffic, on small synthetic CSVs whose answers are known."""
import csv

import pytest

from rembed_amd import profsummary as P

GEMM = "void rh::gemm_i8_kernel<128, 256, 3, 0, 4, 64>(rh::GemmI8Args)"
COPY = "__amd_rocclr_copyBuffer"


def write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    return str(path)


def counters(path, rows):
    """rows: (kernel, counter, value) -> a counter_collection.csv."""
    return write_csv(path, ["Kernel_Name", "Counter_Name", "Counter_Value"], rows)


def test_traffic_scales_by_the_copy_calibration(tmp_path, capsys):
    # the copy of 64 MiB reads 2x and writes 4x what the counters say, so the
    # GEMM's KiB figures are scaled by 2 (fetch) and 4 (write)
    mib = 64
    kib = mib * 1024
    fetch = counters(tmp_path / "f.csv", [(GEMM, "FETCH_SIZE", 1000.0), (GEMM, "FETCH_SIZE", 3000.0),
                                          ("other", "FETCH_SIZE", 5.0)])
    write = counters(tmp_path / "w.csv", [(GEMM, "WRITE_SIZE", 100.0), (GEMM, "WRITE_SIZE", 100.0),
                                          ("other", "WRITE_SIZE", 5.0)])
    cf = counters(tmp_path / "cf.csv", [(COPY, "FETCH_SIZE", kib / 2), (COPY, "FETCH_SIZE", kib / 2)])
    cw = counters(tmp_path / "cw.csv", [(COPY, "WRITE_SIZE", kib / 4)])
    out = P.traffic(fetch, write, cf, cw, mib, "cmd")
    assert out["fetch_scale"] == pytest.approx(2.0)
    assert out["write_scale"] == pytest.approx(4.0)
    assert out["launches"] == 2
    # mean fetch 2000 KiB x 2 + mean write 100 KiB x 4, in bytes
    assert out["bytes_per_launch"] == pytest.approx((2000 * 2 + 100 * 4) * 1024)
    assert "Command: `cmd`" in capsys.readouterr().out


def test_pmc_mfma_busy_share(tmp_path, capsys):
    # one dispatch that keeps every SIMD's MFMA busy for a quarter of the
    # per-XCD active cycles: 25 %
    active_per_xcd = 1000.0
    grbm = active_per_xcd * P.XCDS
    busy = 0.25 * active_per_xcd * P.CUS * P.SIMDS
    path = counters(tmp_path / "c.csv", [
        (GEMM, "SQ_WAVES", 64), (GEMM, "SQ_INSTS_MFMA", 100), (GEMM, "SQ_INSTS_VALU", 850),
        (GEMM, "SQ_INSTS_LDS", 150), (GEMM, "SQ_VALU_MFMA_BUSY_CYCLES", busy),
        (GEMM, "SQ_LDS_BANK_CONFLICT", 30), (GEMM, "SQ_ACTIVE_INST_LDS", 120),
        (GEMM, "GRBM_GUI_ACTIVE", grbm)])
    P.pmc(path, "cmd")
    row = [l for l in capsys.readouterr().out.splitlines() if l.startswith("| `void rh::gemm")][0]
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[1:] == ["1", "64", "100", "25.0%", "8.5", "1.5", "25.0%"]


def test_stats_per_step_and_gemm_total(tmp_path, capsys):
    path = write_csv(tmp_path / "s.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs"], [
        (GEMM, 4, 400000, 100000), ("rh::l2_rows_kernel(float*, int)", 2, 20000, 10000)])
    P.stats(path, 2, "title", "cmd")
    out = capsys.readouterr().out
    assert f"| `{GEMM}` | 4 | 100.00 | 200.0 | 95.2% |" in out
    assert "4 calls, average 100.00 µs, 200.0 µs per step" in out


def test_trace_averages_the_selected_forwards(tmp_path, capsys):
    """Forwards are cut at the first kernel's launches; the skipped ones and
    everything after the window stay out of the means."""
    rows, t = [], 0

    def launch(name, us):
        nonlocal t
        rows.append([name, t, t + int(us * 1000)])
        t += int(us * 1000) + 500

    for f, gemm_us in enumerate([100.0, 10.0, 12.0, 999.0]):  # warm-up, 2 forwards, extra
        launch("embed_ln_vec_kernel<3>", 5.0)
        launch(GEMM, gemm_us)
        launch(GEMM, gemm_us)
    path = write_csv(tmp_path / "t.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
                     rows)
    P.trace(path, "embed_ln", 1, 2, "title", "cmd")
    out = capsys.readouterr().out
    assert f"| `{GEMM}` | 2 | 11.00 | 22.0 |" in out
    assert "kernel time 27.0 µs per forward" in out
    assert "All `gemm_i8_kernel` launches: 2 per forward, average 11.00 µs" in out
    with pytest.raises(SystemExit):
        P.trace(path, "embed_ln", 3, 2, "title", "cmd")


def test_gemm_rooflines_per_shape(capsys):
    """Ops and algorithmic bytes per shape, the binding peak of each, and the
    combined fraction: a launch at exactly its binding time scores 100 %."""
    m = 1000
    layer = [("A", 64, 64, 4), ("B", 4096, 4096, 4)]
    t_a = (m * 64 + 64 * 64 + m * 64 * 4 + 4 * m + 12 * 64) / (P.HBM_PEAK_GBS * 1e9) * 1e6
    t_b = 2.0 * m * 4096 * 4096 / (P.INT8_PEAK_TOPS * 1e12) * 1e6
    P.gemm_rooflines([t_a, 2 * t_b], m, layer)
    out = capsys.readouterr().out
    assert "| A | 64 × 64 |" in out and "HBM (" in out
    assert "| B | 4096 × 4096 |" in out and "MFMA (" in out and "50.0 % |" in out
    assert f"{100 * (t_a + t_b) / (t_a + 2 * t_b):.1f} % of the combined roofline" in out
