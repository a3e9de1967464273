"""bench.py's contract pieces that need no GPU: it refuses more than one GPU
with a message, and its report modes turn rocprofv3 CSVs (the committed
profile summaries are made by them) into summaries with the expected
figures."""
from __future__ import annotations

import csv
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_gemm_traffic_report_weights_roles_by_launches(tmp_path, capsys):
    """Each role's mean FETCH/WRITE, scaled by the calibration copy, weighted
    by the role's launches per step."""
    kib = bench.CALIB_KIB
    copy = "void aicf::hip::map1_kernel<copy>(...)"
    rows_f, rows_w = [], []
    for counter, rows, per_role in (("FETCH_SIZE", rows_f, 1000.0), ("WRITE_SIZE", rows_w, 500.0)):
        rows.append({"Kernel_Name": copy, "Counter_Name": counter, "Counter_Value": kib / 2})  # factor 2
        for sig, _role, n, _mib in bench.STEP_GEMM_ROLES:
            rows.append({"Kernel_Name": f"void gemm_nt_kernel{sig}(NTParams)", "Counter_Name": counter,
                         "Counter_Value": per_role})
    _write(tmp_path / "f.csv", rows_f)
    _write(tmp_path / "w.csv", rows_w)
    bench.pmc_report(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    out = capsys.readouterr().out
    expect = int(round((1000.0 + 500.0) * 2 * 1024))
    assert f"traffic_bytes_per_launch: {expect}" in out
    for _sig, role, n, _mib in bench.STEP_GEMM_ROLES:
        assert f"| {role} | {n} |" in out


def test_stats_report_finds_the_last_replayed_step(tmp_path, capsys):
    """The last replayed step ends at the last AdamW launch; the GEMM
    launches after it are the roofline measurement."""
    stats = [{"Name": "void gemm_nt_kernel<2, 2, 2>(x)", "Calls": 3, "AverageNs": 2000, "Percentage": 90.0}]
    trace, t = [], 0
    def add(name, dur):
        nonlocal t
        trace.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur})
        t += dur + 10
    for _ in range(3):  # three replayed steps: two GEMMs and the bias AdamW
        add("void gemm_nt_kernel<2, 2, 2>(x)", 1000)
        add("void gemm_nt_kernel<2, 0, 4>(x)", 3000)
        add("void adamw_vec4_kernel<1, true>(x)", 100)
    add("void gemm_nt_kernel<2, 2, 2>(x)", 5000)  # roofline launches after the replays
    _write(tmp_path / "s.csv", stats)
    _write(tmp_path / "t.csv", trace)
    bench.stats_report(str(tmp_path / "s.csv"), str(tmp_path / "t.csv"), 3)
    out = capsys.readouterr().out
    assert "Last replayed step, launch by launch (3 kernels" in out
    assert "GEMM launches of the last replayed step: 2, mean 2.0 us" in out
    assert "GEMM launches after the replays (roofline measurement): 1, mean 5.0 us." in out
