"""bench.py's report helpers on synthetic rocprofv3 CSVs (no GPU): the kernel-statistics table
credits each kernel with its algorithmic work (the look-ahead column loop with the trailing
update and every block but the first, the row gathers by variant), the counter table's
MFMA-busy arithmetic, and the traffic record's per-call accounting (a split-kernel call spans
several dispatches) with the copy calibration."""
import contextlib
import csv
import io
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _stats_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        tot = sum(r[2] for r in rows)
        for name, calls, ns in rows:
            w.writerow([name, calls, ns, ns / calls, 100.0 * ns / tot])


def _table(path, cfg, units):
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        bench.stats_table(path, bench.CONFIGS[cfg], units, cfg)
    return {line.split("|")[1].strip().strip("`"): line for line in buf.getvalue().splitlines()[2:]}


def test_stats_table_credits_lookahead_and_gathers(tmp_path):
    cfg = bench.CONFIGS["cfg2"]
    R, C, B = cfg["R"], cfg["C"], cfg["blocksize"]
    p = str(tmp_path / "stats.csv")
    ms = 1e6
    _stats_csv(p, [("void (anonymous namespace)::k_block_lookahead<8>(QBArgs, TwArgs, int, int)", 31, 1.8 * ms),
                   ("void (anonymous namespace)::k_quant_block<8, 0>(QBArgs)", 1, 0.03 * ms),
                   ("void (anonymous namespace)::k_gather_rows<256, __half>(args)", 4, 0.036 * ms),
                   ("void (anonymous namespace)::k_gather_h_rows<256, 1>(args)", 4, 0.134 * ms)])
    t = _table(p, "cfg2", 1)
    nb = (C + B - 1) // B
    trail = sum(2.0 * R * B * (C - min(C, (k + 1) * B)) for k in range(nb))
    f_la = trail + 2.0 * R * C * B * (1 - B / C)
    assert f"{f_la / 1e9:.1f} GFLOP" in t["void k_block_lookahead<8>"]
    assert f"{f_la / 1.8e-3 / 1e12:.1f} TF/s" in t["void k_block_lookahead<8>"]
    # k_quant_block then runs only the first block of each linear
    assert f"{2.0 * R * C * B * (B / C) / 1e9:.1f} GFLOP" in t["void k_quant_block<8, 0>"]
    assert f"{6.0 * R * C / 1e6:.0f} MB" in t["void k_gather_rows<256, __half>"]
    assert f"{8.0 * cfg['G'] * C * C / 1e6:.0f} MB" in t["void k_gather_h_rows<256, 1>"]


def test_stats_table_without_lookahead(tmp_path):
    cfg = bench.CONFIGS["cfg2"]
    R, C, B = cfg["R"], cfg["C"], cfg["blocksize"]
    p = str(tmp_path / "stats.csv")
    _stats_csv(p, [("void (anonymous namespace)::k_quant_block<8, 0>(QBArgs)", 32, 0.9e6),
                   ("void (anonymous namespace)::k_trailing_z<false>(TzArgs)", 31, 2.5e6)])
    t = _table(p, "cfg2", 1)
    assert f"{2.0 * R * C * B / 1e9:.1f} GFLOP" in t["void k_quant_block<8, 0>"]
    nb = (C + B - 1) // B
    trail = sum(2.0 * R * B * (C - min(C, (k + 1) * B)) for k in range(nb))
    assert f"{3 * trail / 1e9:.1f} GFLOP" in t["void k_trailing_z<false>"]


def test_counters_table_mfma_busy(tmp_path):
    p = str(tmp_path / "pmc.csv")
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"])
        for d in (1, 2):
            for name, v in (("SQ_VALU_MFMA_BUSY_CYCLES", 640.0), ("GRBM_GUI_ACTIVE", 10.0),
                            ("SQ_INSTS_MFMA", 100.0), ("SQ_INSTS_VALU", 350.0), ("SQ_INSTS_LDS", 70.0),
                            ("SQ_LDS_BANK_CONFLICT", 0.0)):
                w.writerow([d, "void k_hessian_split<__half, 2>(args)", name, v, 0, 1000])
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        bench.counters_table(p)
    row = buf.getvalue().splitlines()[2]
    # 1280 busy SIMD-cycles over 20 x 128 SIMD-cycles = 50 %
    assert "| 2 |" in row and "50.0 %" in row and "| 3.50 | 0.70 | 0.00 |" in row


def test_more_than_one_gpu_is_refused_before_any_device_work():
    """`bench.py --gpus N` with N > 1 exits with status 2 and says the build runs on one GPU;
    it touches no device (this runs on a host without one)."""
    import subprocess
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1",
                          "--warmup", "0"], capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU only" in res.stdout + res.stderr
    assert not res.stdout.strip().startswith("{")


def _pmc_csv(path, kernel, counter, values):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, v in enumerate(values):
            w.writerow([i, kernel, counter, v])


def test_traffic_report_per_add_batch_call(tmp_path, monkeypatch):
    """8 add_batch calls per linear; 3 dispatches per call of 1000 KiB FETCH_SIZE and
    one of 100 KiB WRITE_SIZE; the copy reads as half its bytes (FETCH) and all of them (WRITE).
    Per call: 3000 KiB / 0.5 + 100 KiB / 1.0 = 6 144 000 + 102 400 bytes."""
    out = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_JSON", str(out))      # never the committed record
    k = "void k_hessian_split<__half, 3>(...)"
    _pmc_csv(tmp_path / "f.csv", k, "FETCH_SIZE", [1000.0] * 24)
    _pmc_csv(tmp_path / "w.csv", k, "WRITE_SIZE", [100.0] * 8)
    _pmc_csv(tmp_path / "cf.csv", "__amd_rocclr_copyBuffer", "FETCH_SIZE", [524288.0])
    _pmc_csv(tmp_path / "cw.csv", "__amd_rocclr_copyBuffer", "WRITE_SIZE", [1048576.0])
    assert bench.hessian_calls(bench.CONFIGS["cfg2"]) == 8
    assert bench.hessian_calls(bench.CONFIGS["cfg3"]) == 32
    with contextlib.redirect_stdout(io.StringIO()):
        bench.traffic_report(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "cf.csv"),
                             str(tmp_path / "cw.csv"), "k_hessian_split", "cfg2", bench.CONFIGS["cfg2"], "split16x3")
    import json
    rec = json.load(open(out))["split16x3"]
    assert rec["calls"] == 8 and rec["dispatches"] == [24, 8]
    assert rec["fetch_size_kib_per_call"] == 3000.0 and rec["write_size_kib_per_call"] == 100.0
    assert rec["traffic_bytes_per_launch"] == 6144000 + 102400
    assert rec["hessian_src_sha256"] == bench.source_sha()
