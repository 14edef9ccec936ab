"""bench.py's host-side contract, no GPU needed: the multi-GPU refusal and
the rocprofv3 summary (kernel table, counter-calibrated traffic records with
kernels matched by exact symbol, not by prefix)."""

import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "only --gpus 1" in r.stderr and r.stdout == ""


def _write(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summary_matches_kernels_by_exact_symbol(tmp_path):
    """k_preprocess_bwd and k_preprocess_bwd_adam share a prefix: each
    traffic record must average only its own kernel's launches."""
    prof = tmp_path / "prof"
    _write(str(prof / "k_kernel_stats.csv"),
           ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"],
           [["void (anonymous namespace)::k_preprocess_bwd<false>(int)", 2, 200000, 100000,
             40, 90000, 110000],
            ["void (anonymous namespace)::k_preprocess_bwd_adam<false>(int)", 1, 250000, 250000,
             60, 250000, 250000]])
    probe_n = 1 << 20  # elements of the copy probe: 4 MiB read and written
    header = ["Kernel_Name", "Counter_Name", "Counter_Value", "Grid_Size"]
    kib = lambda mb: mb * 1024.0  # noqa: E731
    fetch = [["k_debug_expf(long)", "FETCH_SIZE", kib(2.0), probe_n],  # counter reads half
             ["void (anonymous namespace)::k_preprocess_bwd<false>(int)", "FETCH_SIZE",
              kib(10.0), 1000],
             ["void (anonymous namespace)::k_preprocess_bwd<false>(int)", "FETCH_SIZE",
              kib(12.0), 1000],
             ["void (anonymous namespace)::k_preprocess_bwd_adam<false>(int)", "FETCH_SIZE",
              kib(500.0), 1000]]
    write = [["k_debug_expf(long)", "WRITE_SIZE", kib(4.0), probe_n],
             ["void (anonymous namespace)::k_preprocess_bwd<false>(int)", "WRITE_SIZE",
              kib(20.0), 1000],
             ["void (anonymous namespace)::k_preprocess_bwd<false>(int)", "WRITE_SIZE",
              kib(20.0), 1000],
             ["void (anonymous namespace)::k_preprocess_bwd_adam<false>(int)", "WRITE_SIZE",
              kib(700.0), 1000]]
    _write(str(tmp_path / "f" / "x_counter_collection.csv"), header, fetch)
    _write(str(tmp_path / "w" / "x_counter_collection.csv"), header, write)
    out = tmp_path / "out"
    bench.summarize_prof([str(prof), str(tmp_path / "f"), str(tmp_path / "w")], "wl", "cmd",
                         out_dir=str(out))
    table = (out / "kernels_wl.md").read_text()
    assert "`k_preprocess_bwd_adam<false>`" in table and "| 1 | 250.00 |" in table
    bwd = json.loads((out / "traffic_preprocess_bwd_wl.json").read_text())
    fused = json.loads((out / "traffic_preprocess_bwd_adam_wl.json").read_text())
    # calibration: the probe moved 4 MiB each way; FETCH_SIZE read 2 MiB
    assert bwd["calibration"]["fetch_scale"] == pytest.approx(2.0)
    assert bwd["calibration"]["write_scale"] == pytest.approx(1.0)
    assert bwd["hbm_bytes_per_launch"] == int((11.0 * 2.0 + 20.0) * 1024 * 1024)
    assert fused["hbm_bytes_per_launch"] == int((500.0 * 2.0 + 700.0) * 1024 * 1024)
