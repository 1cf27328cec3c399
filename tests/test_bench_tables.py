"""bench.py's profile summaries: the tables it prints from rocprofv3 output and
reads back from profiles/ (counter co-bound, HBM traffic, kernel trace)."""

from __future__ import annotations

import csv
import sqlite3
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def _counter_db(path, rows):
    con = sqlite3.connect(path)
    con.execute("create table counters_collection (dispatch_id int, kernel_name text, counter_name text, "
                "value real, duration real)")
    con.executemany("insert into counters_collection values (?, ?, ?, ?, ?)", rows)
    con.commit()
    con.close()


def test_counters_summary_round_trip(tmp_path):
    k = "_ZN3ssa19ssa_bwd_dkdv_kernelIDF16bLi128ELb1ELb1ELb1EEEvNS_9BwdParamsE"
    gui = 8 * 2_000_000.0  # 2 M cycles per XCD
    dur_ns = 1_000_000.0   # 1 ms -> 2.0 GHz
    mfma = 1.0e7
    a = [(5, k, "GRBM_GUI_ACTIVE", gui, dur_ns), (5, k, "SQ_INSTS_MFMA", mfma, dur_ns),
         (5, k, "SQ_INSTS_VALU", mfma * 9, dur_ns), (5, k, "SQ_INSTS_VALU_TRANS_F32", mfma * 1.5, dur_ns),
         (5, k, "SQ_INSTS_SALU", mfma * 2.5, dur_ns), (5, k, "SQ_INSTS_LDS", mfma * 2, dur_ns),
         (5, k, "SQ_VALU_MFMA_BUSY_CYCLES", 32 * mfma, dur_ns),
         (5, "some_torch_kernel", "SQ_INSTS_MFMA", 1.0, dur_ns)]
    # per-wave quad-cycles: issue 60, wait-any 30, wait-dep 10 (units of 1e6)
    b = [(5, k, "GRBM_GUI_ACTIVE", gui, dur_ns), (5, k, "SQ_ACTIVE_INST_ANY", 60e6, dur_ns),
         (5, k, "SQ_WAIT_ANY", 30e6, dur_ns), (5, k, "SQ_WAIT_INST_ANY", 10e6, dur_ns),
         (5, k, "SQ_ACTIVE_INST_VALU", 1024 * 2e6 * 0.4 / 4, dur_ns)]
    _counter_db(tmp_path / "a.db", a)
    _counter_db(tmp_path / "b.db", b)
    table = bench.counters_summary([str(tmp_path / "a.db"), str(tmp_path / "b.db")])
    row = [ln for ln in table.splitlines() if ln.startswith("| `ssa_bwd_dkdv_kernel`")]
    assert len(row) == 1 and "some_torch" not in table
    f = tmp_path / "profiles" / "ssa_counters_x.md"
    f.parent.mkdir()
    f.write_text("intro\n\n" + table + "\n")
    old = bench.ROOT
    try:
        bench.ROOT = tmp_path
        got = bench.measured_counters("x")["ssa_bwd_dkdv_kernel"]
    finally:
        bench.ROOT = old
    assert got["clock_ghz"] == pytest.approx(2.0)
    assert got["mfma_busy"] == pytest.approx(32 * mfma / (1024 * 2e6), abs=1e-3)
    assert got["valu_busy"] == pytest.approx(0.4, abs=1e-3)
    assert got["valu_per_mfma"] == pytest.approx(8.0)
    assert got["trans_per_mfma"] == pytest.approx(1.5)
    assert got["salu_per_mfma"] == pytest.approx(2.5)
    assert got["issue"] == pytest.approx(0.6) and got["wait_any"] == pytest.approx(0.3)
    assert got["wait_dep"] == pytest.approx(0.1)


def test_trace_summary(tmp_path):
    p = tmp_path / "t.csv"
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for i, us in enumerate((10, 20, 30)):
            w.writerow({"Kernel_Name": "void ssa::ssa_fwd_kernel<x>(p)", "Start_Timestamp": 1000 * i,
                        "End_Timestamp": 1000 * i + 1000 * us})
        w.writerow({"Kernel_Name": "elementwise", "Start_Timestamp": 0, "End_Timestamp": 5})
    row = [ln for ln in bench.trace_summary(str(p)).splitlines() if "ssa_fwd_kernel" in ln][0]
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[1:] == ["3", "20.0", "20.0", "10.0", "30.0", "100.0"]


def test_committed_profiles_parse():
    """The profiles bench.py reads for its JSON line parse into every kernel of the step."""
    c = bench.measured_counters("s4096")
    assert {"ssa_fwd_kernel", "ssa_bwd_dkdv_kernel", "ssa_bwd_dq_ds_kernel"} <= set(c)
    for d in c.values():
        assert 0.0 <= d["mfma_busy"] <= 1.0 and 0.0 <= d["valu_busy"] <= 1.0
    t = bench.measured_traffic("s4096")
    assert {"ssa_fwd_kernel", "ssa_bwd_preprocess_kernel", "ssa_bwd_dkdv_kernel", "ssa_bwd_dq_kernel"} <= set(t)
