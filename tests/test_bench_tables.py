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
    # the dK/dV stage under the HIP kernel name the library runs at this head dim
    assert {"ssa_fwd_kernel", bench.dkdv_hip_name(128, "bf16"), "ssa_bwd_dq_ds_kernel"} <= set(c)
    assert bench.dkdv_hip_name(64, "bf16") in bench.measured_counters("gqa_d64")
    for d in c.values():
        assert 0.0 <= d["mfma_busy"] <= 1.0 and 0.0 <= d["valu_busy"] <= 1.0
    t = bench.measured_traffic("s4096")
    assert {"ssa_fwd_kernel", "ssa_bwd_preprocess_kernel", "ssa_bwd_dkdv_kernel", "ssa_bwd_dq_kernel"} <= set(t)


def test_roofline_of_each_bound():
    """The roofline object for each kind of dominant kernel: a FLOP-priced one
    above the ridge (MFMA roof), a FLOP-priced one below it (rated in GB/s by
    its algorithmic bytes: the GQA D = 64 dK/dV, whose dS' workspace write
    lowers its intensity), and a byte-priced one."""
    ridge = bench.PEAK_BF16_TFLOPS * 1e12 / (bench.PEAK_HBM_GBPS * 1e9)
    # above the ridge: 550 GFLOP over 1.5 GB (measured traffic)
    k = {"ssa_bwd_dkdv_kernel": {"avg_ms": 0.8, "alg_flop": 5.5e11, "hbm_bytes": 1.5e9},
         "ssa_fwd_kernel": {"avg_ms": 0.3, "alg_flop": 2.75e11}}
    r = bench.roofline_of(k, {"ssa_bwd_dkdv_kernel": 2.4e9}, bench.PEAK_BF16_TFLOPS, False, "s4096")
    assert 5.5e11 / 1.5e9 > ridge
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["kernel"] == "ssa_bwd_dkdv_kernel"
    assert r["achieved"] == pytest.approx(5.5e11 / 0.8e-3 / 1e12)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.PEAK_BF16_TFLOPS)
    # below the ridge, no measured traffic: intensity from the algorithmic bytes
    k = {"ssa_bwd_dkdv_kernel": {"avg_ms": 0.95, "alg_flop": 5.5e11},
         "ssa_bwd_dq_kernel": {"avg_ms": 0.4, "alg_flop": 1.4e11, "alg_bytes": 2.2e9}}
    r = bench.roofline_of(k, {"ssa_bwd_dkdv_kernel": 2.4e9}, bench.PEAK_BF16_TFLOPS, False, "gqa_d64")
    assert 5.5e11 / 2.4e9 < ridge
    assert r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert r["achieved"] == pytest.approx(2.4e9 / 0.95e-3 / 1e9)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.PEAK_HBM_GBPS)
    assert r["tflops"] == pytest.approx(5.5e11 / 0.95e-3 / 1e12)
    assert k["ssa_bwd_dq_kernel"]["bound"] == "hbm"
    # a byte-priced dominant kernel
    k = {"ssa_bwd_dq_kernel": {"avg_ms": 0.4, "alg_flop": 1.4e11, "alg_bytes": 2.2e9},
         "ssa_fwd_kernel": {"avg_ms": 0.3, "alg_flop": 2.75e11}}
    r = bench.roofline_of(k, {}, bench.PEAK_BF16_TFLOPS, False, "s4096")
    assert r["kernel"] == "ssa_bwd_dq_kernel" and r["bound"] == "hbm"
    assert r["achieved"] == pytest.approx(2.2e9 / 0.4e-3 / 1e9)
