#!/usr/bin/env python3
"""Benchmark: SSA attention forward + backward on one MI355X.

A "step" is one forward + backward of the SSA attention op through the
reference-compatible kernel API (ssa_flash_attn_forward +
ssa_flash_attn_backward) on synthetic inputs already resident in HBM:
B=4, H=16, S=4096, D=128, bf16, causal, Q/K/V = 0.5 N(0,1), dO ~ N(0,1),
n=1.5, b=0.8, scale=1/sqrt(D) (the shape BASELINE.json's metric is quoted on).

value = algorithmic fwd+bwd FLOPs / step time, with fwd = 4 D pairs and
bwd = 10 D pairs (pairs = unmasked (q, k) pairs), i.e. 14 D pairs per step.
The backward runs the library's default path: dS' kept in a workspace
(ssa_bwd_ds_workspace_bytes) and dQ as a streaming dS' K product; set
SSA_BWD_DS=0 to time the recompute path instead (config.bwd_path says which).

Also reported on the same JSON line:
  roofline     -- the dominant kernel's algorithmic FLOPs (or bytes) per launch
                  over its average launch time, measured here with HIP events
                  on the stream the kernel runs on;
  kernels      -- the same for every kernel of the step;
  cpu_baseline -- the PyTorch-eager fp32 oracle (oracle/ssa_oracle_torch.py)
                  on the host cores, on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import re
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "luciole-1b_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

# MI355X published dense peaks.
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk/CU (2.5 PFLOP/s class)
PEAK_HBM_GBPS = 8000.0
PEAK_FP32_TFLOPS = 157.3   # MI355X published fp32 peak (packed fp32 VALU or fp32 MFMA)
# fp32 FMA on the vector ALU without packed forms (which this build leaves out):
# 256 CU x 4 SIMD x 16 lanes x 2 FLOP x 2.4 GHz
PEAK_FP32_VALU_TFLOPS = 78.6

CONFIGS = {
    # name: (B, Hq, Hkv, S, D, causal)
    "s4096": (4, 16, 16, 4096, 128, True),   # north star: BASELINE.json metric shape
    "s2048": (4, 16, 16, 2048, 128, True),
    "s16384": (1, 16, 16, 16384, 128, True),
    "gqa_d64": (4, 32, 8, 4096, 64, True),   # production Luciole-1B attention shape
}
# packed sequences, 16384 tokens per micro-batch,
# document lengths uniform in [64, 4096] from random.Random(1234), the last
# document truncated to fill; H = 16, D = 128, causal inside each document.
VARLEN_CONFIGS = {"varlen16k": (16384, 16, 16, 128, 64, 4096)}
# Decode step against a KV cache (no reference kernel: the reference re-runs the
# prefix per generated token): name: (B, Hq, Hkv, cache length, D).
# one optimizer step of a 1B Llama-style decoder with
# SSA attention (SSA/ssa_decoder.py defaults), micro-batch 4 x 4096 tokens.
TRAIN_CONFIGS = {"train1b": 4}
DECODE_CONFIGS = {
    "decode_s4096": (16, 16, 16, 4096, 128),
    "decode_gqa_d64": (16, 32, 8, 4096, 64),
}


def varlen_lengths(total, lo, hi, seed=1234):
    import random

    rng = random.Random(seed)
    lens = []
    while sum(lens) < total:
        lens.append(min(rng.randint(lo, hi), total - sum(lens)))
    return lens

METRIC = "SSA attn fwd+bwd TFLOP/s and % bf16 MFMA peak, 1 MI355X, S=4096 D=128"
COPY_MIB = 1024  # calibration copy of the --pmc-pass runs
TRAFFIC_ROW = re.compile(r"^\|\s*`?(ssa_\w+?)`?\s*\|\s*([0-9.]+)\s*\|\s*([0-9.]+)\s*\|\s*([0-9.]+)\s*\|")


def measured_traffic(config):
    """HBM bytes per launch per kernel from the committed counter summary of this config.

    profiles/hbm_traffic_<config>.md holds one table row per kernel:
    | kernel | fetch MB | write MB | total MB | ... -- FETCH_SIZE and WRITE_SIZE per
    dispatch from two rocprofv3 --pmc runs of `bench.py --pmc-pass`, each scaled by
    the factor that makes the same counter read exactly the bytes of the
    calibration copy.  Returns {} when the file is absent.
    """
    f = ROOT / "profiles" / f"hbm_traffic_{config}.md"
    if not f.exists():
        return {}
    out = {}
    for line in f.read_text().splitlines():
        m = TRAFFIC_ROW.match(line)
        if m:
            out[m.group(1)] = float(m.group(4)) * 1e6
    return out


# SQ counter passes of `bench.py --pmc-pass` (rocprofv3 --pmc, one database per
# pass), summarised per SSA kernel by `bench.py --counters-summary DB ...`.  The
# counters are totals over the device: SQ_VALU_MFMA_BUSY_CYCLES sums matrix-core
# busy cycles over SIMDs; GRBM_GUI_ACTIVE counts GPU cycles per XCD (8 on MI355X);
# SQ_ACTIVE_INST_* / SQ_WAIT_* count per-wave quad-cycles.
CUS, SIMDS, XCDS = 256, 1024, 8
COUNTER_ROW = re.compile(r"^\|\s*`(ssa_\w+?)`\s*\|" + r"\s*([0-9.]+)\s*\|" * 12)


def counters_summary(dbs):
    """Markdown table of the SSA kernels' counters from rocprofv3 databases."""
    import sqlite3
    from collections import defaultdict

    tot = defaultdict(lambda: defaultdict(float))
    dur, gui_pass = {}, {}
    for db in dbs:
        con = sqlite3.connect(db)
        rows = con.execute("select dispatch_id, kernel_name, counter_name, value, duration from counters_collection")
        for d, k, c, v, du in rows:
            m = re.search(r"(ssa_\w+?_kernel)", k)
            if not m:
                continue
            name = m.group(1)
            if c == "GRBM_GUI_ACTIVE":  # collected in every pass: keep one
                gui_pass[(db, name)] = gui_pass.get((db, name), 0.0) + v
            else:
                tot[name][c] += v
            dur[name] = du / 1e6
    for (db, name), v in gui_pass.items():
        tot[name]["GRBM_GUI_ACTIVE"] = max(tot[name]["GRBM_GUI_ACTIVE"], v)
    lines = ["| kernel | ms | clock GHz | MFMA busy % | VALU busy % | VALU/MFMA | trans/MFMA | SALU/MFMA | "
             "LDS/MFMA | issue % | wait-any % | wait-dep % | LDS data FIFO full % |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for name, c in tot.items():
        gui = c.get("GRBM_GUI_ACTIVE", 0.0) / XCDS
        if not gui:
            continue
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        per = lambda key: c.get(key, 0.0) / mf if mf else 0.0  # noqa: E731
        wave = c.get("SQ_ACTIVE_INST_ANY", 0.0) + c.get("SQ_WAIT_ANY", 0.0) + c.get("SQ_WAIT_INST_ANY", 0.0)
        frac = lambda key: 100.0 * c.get(key, 0.0) / wave if wave else 0.0  # noqa: E731
        lines.append(
            f"| `{name}` | {dur.get(name, 0.0):.4f} | {gui / (dur.get(name, 1.0) * 1e6):.2f} | "
            f"{100.0 * c.get('SQ_VALU_MFMA_BUSY_CYCLES', 0.0) / (SIMDS * gui):.1f} | "
            f"{100.0 * 4 * c.get('SQ_ACTIVE_INST_VALU', 0.0) / (SIMDS * gui):.1f} | "
            f"{(c.get('SQ_INSTS_VALU', 0.0) - mf) / mf if mf else 0.0:.2f} | {per('SQ_INSTS_VALU_TRANS_F32'):.2f} | "
            f"{per('SQ_INSTS_SALU'):.2f} | {per('SQ_INSTS_LDS'):.2f} | {frac('SQ_ACTIVE_INST_ANY'):.1f} | "
            f"{frac('SQ_WAIT_ANY'):.1f} | {frac('SQ_WAIT_INST_ANY'):.1f} | "
            f"{100.0 * c.get('SQ_LDS_DATA_FIFO_FULL', 0.0) / (CUS * gui):.1f} |")
    return "\n".join(lines)


def _csv_rows(path):
    import csv

    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def _ssa_name(kernel_name):
    m = re.search(r"(ssa_\w+?_kernel)", kernel_name)
    return m.group(1) if m else None


def dkdv_hip_name(D: int, dtype: str) -> str:
    """The HIP kernel the library runs for the dK/dV stage (csrc/ssa_bwd.hip
    use_dkdv2w): the two-wave kernel at head dim 128 for bf16 / fp16 unless
    SSA_DKDV2W=0, at every head dim with SSA_DKDV2W=1."""
    if dtype == "fp32":
        return "ssa_bwd_dkdv_f32_kernel"
    e = os.environ.get("SSA_DKDV2W", "")
    two = e[:1] == "1" if e[:1] in ("0", "1") else D == 128
    return "ssa_bwd_dkdv2w_kernel" if two else "ssa_bwd_dkdv_kernel"


def trace_summary(trace_csv):
    """Markdown table of the SSA kernels in a rocprofv3 --kernel-trace CSV."""
    import statistics

    per = {}
    for r in _csv_rows(trace_csv):
        name = _ssa_name(r["Kernel_Name"])
        if name:
            per.setdefault(name, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in per.values())
    lines = ["| kernel | calls | avg us | median us | min us | max us | share % |", "|---|---|---|---|---|---|---|"]
    for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {len(v)} | {sum(v) / len(v):.1f} | {statistics.median(v):.1f} | {min(v):.1f} | "
                     f"{max(v):.1f} | {100.0 * sum(v) / total:.1f} |")
    return "\n".join(lines)


def traffic_summary(fetch_csv, write_csv, config="s4096"):
    """Markdown table of HBM bytes per launch from FETCH_SIZE / WRITE_SIZE CSVs
    of `--pmc-pass` runs, each scaled by the factor that makes the counter read
    exactly COPY_MIB MiB on the calibration copy, next to the algorithmic bytes."""
    B, Hq, Hkv, S, D, causal = CONFIGS[config]
    t = B * Hq * S * D * 2          # one [B, Hq, S, D] tensor
    tkv = B * Hkv * S * D * 2
    rows = B * Hq * S * 4           # M or Delta
    nq = (S + 31) // 32
    ds = B * Hq * (nq * (nq + 1) if causal else 2 * nq * nq) * 1024
    alg = {"ssa_fwd_kernel": 2 * t + 2 * tkv + rows, "ssa_bwd_preprocess_kernel": 2 * t + rows,
           "ssa_bwd_dkdv_kernel": 2 * t + 4 * tkv + 2 * rows + ds, "ssa_bwd_dq_kernel": ds + tkv + t}
    vals = {}
    for which, path in (("fetch", fetch_csv), ("write", write_csv)):
        per = {}
        for r in _csv_rows(path):
            per[(r["Dispatch_Id"], r["Kernel_Name"])] = per.get((r["Dispatch_Id"], r["Kernel_Name"]), 0.0) + float(
                r["Counter_Value"])
        copy = [v for (d, k), v in per.items() if "copyBuffer" in k]
        scale = COPY_MIB * 1024 / copy[-1]
        for (d, k), v in per.items():
            name = _ssa_name(k)
            if name:
                name = "ssa_bwd_dq_kernel" if name.startswith("ssa_bwd_dq") else name
                name = "ssa_bwd_dkdv_kernel" if name.startswith("ssa_bwd_dkdv") else name
                vals.setdefault(name, {})[which] = v * scale * 1024 / 1e6
        vals.setdefault("_scale", {})[which] = scale
    lines = [f"Calibration: FETCH_SIZE x{vals['_scale']['fetch']:.4f}, WRITE_SIZE x{vals['_scale']['write']:.4f} "
             f"(the factors that make each read {COPY_MIB} MiB on the calibration copy).", "",
             "| kernel | fetch MB | write MB | total MB | algorithmic MB | total / algorithmic |",
             "|---|---|---|---|---|---|"]
    for name in ("ssa_fwd_kernel", "ssa_bwd_preprocess_kernel", "ssa_bwd_dkdv_kernel", "ssa_bwd_dq_kernel"):
        if name in vals:
            f, w = vals[name].get("fetch", 0.0), vals[name].get("write", 0.0)
            lines.append(f"| `{name}` | {f:.1f} | {w:.1f} | {f + w:.1f} | {alg[name] / 1e6:.1f} | "
                         f"{(f + w) / (alg[name] / 1e6):.3f} |")
    return "\n".join(lines)


def measured_counters(config):
    """Per-kernel co-bound figures from profiles/ssa_counters_<config>.md (the
    table `bench.py --counters-summary` prints); {} when the file is absent."""
    f = ROOT / "profiles" / f"ssa_counters_{config}.md"
    if not f.exists():
        return {}
    keys = ("counter_ms", "clock_ghz", "mfma_busy", "valu_busy", "valu_per_mfma", "trans_per_mfma",
            "salu_per_mfma", "lds_per_mfma", "issue", "wait_any", "wait_dep", "lds_fifo_full")
    out = {}
    text = f.read_text()
    # "Library: built from commit <sha>" in the profile names the kernels it measured
    mb = re.search(r"built from commit (\w+)", text)
    for line in text.splitlines():
        m = COUNTER_ROW.match(line)
        if m:
            vals = [float(x) for x in m.groups()[1:]]
            d = dict(zip(keys, vals))
            for k in ("mfma_busy", "valu_busy", "issue", "wait_any", "wait_dep", "lds_fifo_full"):
                d[k] /= 100.0
            d["build"] = mb.group(1) if mb else None
            out[m.group(1)] = d
    return out


def roofline_of(kernels: dict, alg_io: dict, peak_flops: float, fp32: bool, config: str) -> dict:
    """Rates, fractions and the bounding roof of every kernel (in place), and
    the `roofline` object of the dominant (longest) kernel.

    A kernel priced in FLOPs is compute-bound when its intensity (FLOP per HBM
    byte: measured traffic where a profile exists, else its algorithmic bytes)
    lies above the ridge of the two roofs, HBM-bound otherwise; an HBM-bound
    one is then rated by its algorithmic bytes (inputs read once, outputs
    written once).  Kernels priced in bytes are HBM-bound."""
    ridge = peak_flops * 1e12 / (PEAK_HBM_GBPS * 1e9)  # FLOP per HBM byte where the two roofs meet
    for name, kd in kernels.items():
        if "alg_flop" in kd:
            kd["tflops"] = kd["alg_flop"] / (kd["avg_ms"] * 1e-3) / 1e12
            kd["frac_peak"] = kd["tflops"] / peak_flops
            if fp32:
                kd["frac_valu_peak"] = kd["tflops"] / PEAK_FP32_VALU_TFLOPS
            nbytes = kd.get("hbm_bytes") or alg_io.get(name)
            if nbytes:
                kd["intensity_flop_per_byte"] = kd["alg_flop"] / nbytes
                compute = kd["intensity_flop_per_byte"] > ridge
            else:
                compute = True
            kd["bound"] = ("valu" if fp32 else "mfma") if compute else "hbm"
            if not compute and alg_io.get(name):
                kd["alg_bytes_io"] = alg_io[name]
                kd["gbps"] = alg_io[name] / (kd["avg_ms"] * 1e-3) / 1e9
                kd["frac_hbm_peak"] = kd["gbps"] / PEAK_HBM_GBPS
        if "alg_bytes" in kd:
            kd["gbps"] = kd["alg_bytes"] / (kd["avg_ms"] * 1e-3) / 1e9
            kd["frac_peak"] = kd["gbps"] / PEAK_HBM_GBPS
            kd["bound"] = "hbm"
    dominant = max(kernels, key=lambda k_: kernels[k_]["avg_ms"])
    kd = kernels[dominant]
    if kd.get("bound") in ("mfma", "valu"):
        roofline = {"kernel": dominant, "bound": kd["bound"], "achieved": kd["tflops"], "peak": peak_flops,
                    "unit": "TFLOP/s", "frac": kd["tflops"] / peak_flops, "traffic": kd.get("hbm_bytes"),
                    "avg_launch_ms": kd["avg_ms"]}
    else:
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": kd["gbps"], "peak": PEAK_HBM_GBPS,
                    "unit": "GB/s", "frac": kd["gbps"] / PEAK_HBM_GBPS, "traffic": kd.get("hbm_bytes"),
                    "avg_launch_ms": kd["avg_ms"]}
        if "tflops" in kd:
            roofline["tflops"] = kd["tflops"]
    cn = kd.get("counters")
    if cn and "alg_flop" in kd:
        # The SSA element work is the co-bound: the counters say what limits
        # the kernel below its roofline (matrix-core and VALU busy fractions
        # per SIMD at the measured clock, instructions per MFMA, and the share
        # of wave time spent waiting).
        roofline["co_bound"] = {
            "mfma_busy": cn["mfma_busy"], "valu_busy": cn["valu_busy"],
            "valu_per_mfma": cn["valu_per_mfma"], "trans_per_mfma": cn["trans_per_mfma"],
            "salu_per_mfma": cn["salu_per_mfma"], "wait_frac": cn["wait_any"] + cn["wait_dep"],
            "clock_ghz": cn["clock_ghz"], "limiter": limiter_from_counters(cn),
            "source": f"profiles/ssa_counters_{config}.md", "profile_build": cn.get("build")}
    return roofline


def limiter_from_counters(cn):
    """What the counter row says holds a kernel below its compute roof: a unit
    busy >= 80 % of the SIMD-cycles is saturated; otherwise the waves' waiting
    share decides between latency (>= 35 % of wave time waiting) and issue."""
    mf, va, wait = cn["mfma_busy"], cn["valu_busy"], cn["wait_any"] + cn["wait_dep"]
    if mf >= 0.8:
        return f"matrix core saturated ({mf:.0%} busy)"
    if va >= 0.8:
        return f"vector ALU saturated ({va:.0%} busy)"
    what = (f"matrix core {mf:.0%} and VALU {va:.0%} busy; waves issue {cn['issue']:.0%} of their time and wait "
            f"{wait:.0%} ({cn['wait_any']:.0%} on counters and barriers, {cn['wait_dep']:.0%} on dependencies)")
    return ("latency: " if wait >= 0.35 else "issue: ") + what


def pairs_dense(B, Hq, S, causal):
    return B * Hq * (S * (S + 1) // 2 if causal else S * S)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        m = re.search(r"Model name:\s*(.+)", out)
        if m:
            return m.group(1).strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def _time_oracle(B, H, S, D, causal, runs, warmup, budget_s, seed=1234, qkv_scale=0.5):
    """Median wall time of the fp32 torch oracle's fwd + autograd bwd on one
    [B, H, S, D] problem (inputs drawn once, outside the timed region)."""
    import torch

    from oracle.ssa_oracle_torch import run_reference_grads

    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, S, D, generator=g) * qkv_scale for _ in range(3))
    do = torch.randn(B, H, S, D, generator=g)
    n, b = torch.tensor(1.5), torch.tensor(0.8)
    scale = 1.0 / math.sqrt(D)
    for _ in range(warmup):
        run_reference_grads(q, k, v, scale, n, b, do, causal)
    times = []
    t_start = time.perf_counter()
    while len(times) < runs and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        run_reference_grads(q, k, v, scale, n, b, do, causal)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(B, H, S, D, causal, budget_s=20.0):
    """The fp32 PyTorch-eager oracle (oracle/ssa_oracle_torch.py, fwd + autograd
    bwd) on the host cores, as a reported baseline:

    * BASELINE.json configs[0] (B=1, H=4, S=256, D=64, fp32, causal; N(0,1)
      inputs) timed in full: 3 warm-up runs, median of 10;
    * the GPU workload timed on (b, h) slices -- one slice's S x S fp32
      intermediates are what fit -- with the number of slices timed and the
      whole step extrapolated as B * H slices.

    ``value`` is the slice rate in the metric's unit (TFLOP/s of the same
    14 D pairs count), i.e. the rate of the full step on these cores."""
    import torch

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c1_med, c1_runs = _time_oracle(1, 4, 256, 64, True, runs=10, warmup=3, budget_s=budget_s / 4, qkv_scale=1.0)
    c1_flop = 14 * 64 * pairs_dense(1, 4, 256, True)
    med, runs = _time_oracle(1, 1, S, D, causal, runs=10, warmup=1, budget_s=budget_s)
    flops = 14 * D * pairs_dense(1, 1, S, causal)
    slices = B * H
    model = cpu_model()
    return {
        "value": flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{runs} runs of one (b,h) slice of the workload (S={S} D={D} fp32 causal={int(causal)}, "
                   f"fwd+autograd bwd), median {med * 1e3:.1f} ms; the full step is {slices} such slices, "
                   f"about {slices * med:.1f} s on these cores; os.cpu_count()={threads}; cpu={model}"),
        "ms_per_slice": med * 1e3,
        "slices_timed": runs,
        "slices_per_step": slices,
        "full_step_s_extrapolated": slices * med,
        "cpu_model": model,
        "os_cpu_count": threads,
        "config0": {"workload": "BASELINE.json configs[0]: B=1 H=4 S=256 D=64 fp32 causal, timed in full",
                    "ms": c1_med * 1e3, "runs": c1_runs, "tflops": c1_flop / c1_med / 1e12,
                    "alg_mflop": c1_flop / 1e6},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 50; train1b 5)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 50: the step time settles after ~30 steps "
                         "of sustained load; train1b 2)")
    ap.add_argument("--config", default="s4096",
                    choices=sorted(CONFIGS) + sorted(VARLEN_CONFIGS) + sorted(DECODE_CONFIGS) + sorted(TRAIN_CONFIGS))
    ap.add_argument("--kernel-iters", type=int, default=50, help="launches per kernel for per-kernel timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp16", "fp32"],
                    help="fp32 (dense shapes only): the fp32 vector-ALU kernels, against the fp32 peak")
    ap.add_argument("--counters-summary", nargs="+", metavar="DB",
                    help="print the per-kernel counter table of rocprofv3 --pmc databases of --pmc-pass runs "
                         "(the table of profiles/ssa_counters_<config>.md) and exit")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the SSA kernel table of a rocprofv3 --kernel-trace CSV and exit")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the HBM traffic table of FETCH_SIZE / WRITE_SIZE CSVs of --pmc-pass runs and exit")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="run each kernel of one step once, then a plain copy of COPY_MIB MiB "
                         "(counter calibration), and exit; for rocprofv3 --pmc runs")
    args = ap.parse_args()
    if args.counters_summary:
        print(counters_summary(args.counters_summary))
        return
    if args.trace_summary:
        print(trace_summary(args.trace_summary))
        return
    if args.traffic_summary:
        print(traffic_summary(*args.traffic_summary, config=args.config))
        return
    train = args.config in TRAIN_CONFIGS
    if args.steps is None:
        args.steps = 5 if train else 50
    if args.warmup is None:
        args.warmup = 2 if train else 50

    if args.dtype == "fp32" and args.config not in CONFIGS:
        print(json.dumps({"error": "--dtype fp32 applies to the dense configs only (" + ", ".join(sorted(CONFIGS)) + ")"}))
        sys.exit(2)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the SSA op has no cross-GPU "
                                   "communication (see DESIGN.md, sharding); run with --gpus 1"}))
        sys.exit(2)

    import torch

    from SSA.ssa_hip_kernel import BackwardLaunch, ssa_flash_attn_backward, ssa_flash_attn_forward

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.config in VARLEN_CONFIGS:
        return bench_varlen(args, dev)
    if args.config in DECODE_CONFIGS:
        return bench_decode(args, dev)
    if args.config in TRAIN_CONFIGS:
        return bench_train(args, dev)
    B, Hq, Hkv, S, D, causal = CONFIGS[args.config]
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[args.dtype]
    torch.manual_seed(1234)
    q = (torch.randn(B, Hq, S, D, device=dev) * 0.5).to(dtype)
    k = (torch.randn(B, Hkv, S, D, device=dev) * 0.5).to(dtype)
    v = (torch.randn(B, Hkv, S, D, device=dev) * 0.5).to(dtype)
    do = torch.randn(B, Hq, S, D, device=dev).to(dtype)
    n = torch.tensor(1.5, device=dev)
    bb = torch.tensor(0.8, device=dev)
    scale = 1.0 / math.sqrt(D)
    pairs = pairs_dense(B, Hq, S, causal)
    flops_fwd = 4 * D * pairs
    flops_bwd = 10 * D * pairs

    def step():
        out, m = ssa_flash_attn_forward(q, k, v, scale, n, bb, causal)
        return ssa_flash_attn_backward(q, k, v, out, do, m, scale, n, bb, causal)

    if args.pmc_pass:
        # One launch of every kernel, then the calibration copy: a device-to-device
        # copy of COPY_MIB MiB reads and writes exactly that many bytes.
        step()
        torch.cuda.synchronize()
        src = torch.empty(COPY_MIB << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] pmc pass done: one step + copy of {COPY_MIB} MiB")
        return

    log(f"[bench] config={args.config} B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} warmup={args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    value = (flops_fwd + flops_bwd) / (ms_step * 1e-3) / 1e12

    # Per-kernel launch durations, HIP events on the stream the kernels use.
    log("[bench] per-kernel timing")
    stream = torch.cuda.current_stream(dev)
    out, m = ssa_flash_attn_forward(q, k, v, scale, n, bb, causal)
    launch = BackwardLaunch(q, k, v, out, do, m, scale, n, bb, causal)

    def time_launch(fn, iters):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
        for a, e in evs:
            a.record(stream)
            fn()
            e.record(stream)
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(e) for a, e in evs)
        pct = lambda f: ts[min(len(ts) - 1, int(f * len(ts)))]
        return sum(ts) / len(ts), {"median_ms": ts[len(ts) // 2], "p10_ms": pct(0.1), "p90_ms": pct(0.9)}

    it = args.kernel_iters
    kernels = {}
    avg, spread = time_launch(lambda: ssa_flash_attn_forward(q, k, v, scale, n, bb, causal), it)
    kernels["ssa_fwd_kernel"] = {"avg_ms": avg, **spread, "alg_flop": flops_fwd}
    for stage in BackwardLaunch.STAGES:
        avg, spread = time_launch(lambda s=stage: launch.run_stage(s), it)
        kernels[f"ssa_bwd_{stage}_kernel"] = {"avg_ms": avg, **spread}
    # Algorithmic work per launch: dK/dV does QK^T, dP, dV, dK (8 D per pair);
    # dQ adds only its dQ product (2 D per pair); preprocess moves O, dO, Delta.
    # On the dS' workspace path dQ streams the workspace (read once) plus K and
    # writes dQ: bytes are its bound, its FLOPs are reported alongside.
    ds_bytes = launch.ds.numel() if launch.ds is not None else 0
    kernels["ssa_bwd_dkdv_kernel"]["alg_flop"] = 8 * D * pairs
    kernels["ssa_bwd_dq_kernel"]["alg_flop"] = 2 * D * pairs
    esize = 4 if dtype == torch.float32 else 2
    if ds_bytes:
        kernels["ssa_bwd_dq_kernel"]["alg_bytes"] = ds_bytes + (B * Hkv + B * Hq) * S * D * esize
    pre_bytes = 2 * B * Hq * S * D * esize + 4 * B * Hq * S
    kernels["ssa_bwd_preprocess_kernel"]["alg_bytes"] = pre_bytes
    # fp32 inputs run on the vector ALU: priced against the published fp32 peak
    # (157.3, which needs packed fp32) and, as frac_valu_peak, against what
    # non-packed fp32 FMAs can reach (78.6)
    peak_flops = PEAK_FP32_TFLOPS if dtype == torch.float32 else PEAK_BF16_TFLOPS
    traffic = measured_traffic(args.config) if args.dtype == "bf16" else {}
    counters = measured_counters(args.config) if args.dtype == "bf16" else {}
    hip_name = {"ssa_bwd_dq_kernel": "ssa_bwd_dq_ds_kernel" if ds_bytes else "ssa_bwd_dq_kernel",
                "ssa_bwd_dkdv_kernel": dkdv_hip_name(D, args.dtype),
                "ssa_bwd_reduce_kernel": "ssa_reduce_partials_kernel"}
    # algorithmic HBM bytes of the FLOP-priced kernels (inputs read once, outputs written once)
    tq, tkv, rows_b = B * Hq * S * D * esize, B * Hkv * S * D * esize, B * Hq * S * 4
    alg_io = {"ssa_fwd_kernel": 2 * tq + 2 * tkv + rows_b,
              "ssa_bwd_dkdv_kernel": 2 * tq + 4 * tkv + 2 * rows_b + ds_bytes}
    for name, kd in kernels.items():
        kd["hbm_bytes"] = traffic.get(name)
        kd["counters"] = counters.get(hip_name.get(name, name))
    roofline = roofline_of(kernels, alg_io, peak_flops, dtype == torch.float32, args.config)
    roofline["hip_kernel"] = hip_name.get(roofline["kernel"], roofline["kernel"])

    fwd_ms = kernels["ssa_fwd_kernel"]["avg_ms"]
    bwd_ms = sum(kernels[f"ssa_bwd_{s}_kernel"]["avg_ms"] for s in BackwardLaunch.STAGES)
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: Q/K/V = 0.5 N(0,1), dO ~ N(0,1), seed 1234, n=1.5, b=0.8",
        "config": {"workload": f"SSA attention fwd+bwd ({args.config})", "B": B, "Hq": Hq, "Hkv": Hkv,
                   "S": S, "D": D, "causal": causal, "pairs": pairs,
                   "alg_gflop_per_step": (flops_fwd + flops_bwd) / 1e9,
                   "bwd_path": "ds_workspace" if ds_bytes else "recompute", "ds_workspace_bytes": ds_bytes},
        "frac_of_bf16_peak": value / PEAK_BF16_TFLOPS,
        "fwd_tflops": flops_fwd / (fwd_ms * 1e-3) / 1e12,
        "bwd_tflops": flops_bwd / (bwd_ms * 1e-3) / 1e12,
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": None,
        "device": torch.cuda.get_device_name(0),
        **device_clock_and_peak(),
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(B, Hq, S, D, causal)
    print(json.dumps(result))


def device_clock_and_peak():
    """CU count and peak engine clock of device 0 (hipDeviceGetAttribute,
    hipDeviceAttributeClockRate = 5 in hip_runtime_api.h, kHz), and the dense
    bf16 MFMA peak they imply (4096 FLOP per clock per CU); the figures above
    use the published 2516.6 TFLOP/s."""
    import ctypes

    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    info = {"cu_count": cus, "max_engine_clock_mhz": None, "bf16_peak_at_clock_tflops": None}
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        khz = ctypes.c_int(0)
        if hip.hipDeviceGetAttribute(ctypes.byref(khz), 5, torch.cuda.current_device()) == 0 and khz.value > 0:
            info["max_engine_clock_mhz"] = khz.value / 1e3
            info["bf16_peak_at_clock_tflops"] = cus * khz.value * 1e3 * 4096 / 1e12
    except OSError:
        pass
    return info


def bench_varlen(args, dev):
    """Packed-sequence fwd + bwd step; same JSON line."""
    import torch

    from SSA.ssa_hip_kernel import ssa_flash_attn_varlen_backward, ssa_flash_attn_varlen_forward

    total, Hq, Hkv, D, lo, hi = VARLEN_CONFIGS[args.config]
    lens = varlen_lengths(total, lo, hi)
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    torch.manual_seed(1234)
    q = (torch.randn(total, Hq, D, device=dev) * 0.5).to(dtype)
    k = (torch.randn(total, Hkv, D, device=dev) * 0.5).to(dtype)
    v = (torch.randn(total, Hkv, D, device=dev) * 0.5).to(dtype)
    do = torch.randn(total, Hq, D, device=dev).to(dtype)
    cu = torch.tensor([0] + [sum(lens[: i + 1]) for i in range(len(lens))], dtype=torch.int32, device=dev)
    n = torch.tensor(1.5, device=dev)
    bb = torch.tensor(0.8, device=dev)
    scale = 1.0 / math.sqrt(D)
    maxlen = max(lens)
    pairs = sum(Hq * L * (L + 1) // 2 for L in lens)
    flops_fwd, flops_bwd = 4 * D * pairs, 10 * D * pairs

    def fwd():
        return ssa_flash_attn_varlen_forward(q, k, v, cu, maxlen, scale, n, bb, True)

    def step():
        out, m = fwd()
        return ssa_flash_attn_varlen_backward(q, k, v, out, do, m, cu, maxlen, scale, n, bb, True)

    log(f"[bench] config={args.config} docs={len(lens)} max={maxlen} pairs={pairs}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) / args.steps * 1e3
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.kernel_iters)]
    for a, e in evs:
        a.record(stream)
        fwd()
        e.record(stream)
    torch.cuda.synchronize()
    fwd_ms = sum(a.elapsed_time(e) for a, e in evs) / len(evs)
    value = (flops_fwd + flops_bwd) / (ms_step * 1e-3) / 1e12
    print(json.dumps({
        "metric": "SSA attn fwd+bwd TFLOP/s, packed sequences (varlen), 1 MI355X",
        "value": value, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: Q/K/V = 0.5 N(0,1), dO ~ N(0,1), seed 1234, n=1.5, b=0.8",
        "config": {"workload": f"SSA attention varlen fwd+bwd ({args.config})", "total_tokens": total,
                   "Hq": Hq, "Hkv": Hkv, "D": D, "causal": True, "documents": len(lens), "doc_lengths": lens,
                   "pairs": pairs, "alg_gflop_per_step": (flops_fwd + flops_bwd) / 1e9},
        "frac_of_bf16_peak": value / PEAK_BF16_TFLOPS,
        "fwd_ms": fwd_ms, "fwd_tflops": flops_fwd / (fwd_ms * 1e-3) / 1e12,
    }))


def bench_train(args, dev):
    """One optimizer step of the 1B SSA decoder (forward, loss, backward, fused
    AdamW) on uniform-random token ids.  value = tokens per second; model
    FLOPs = 6 N_params tokens + 14 D pairs per layer (attention, the
    benchmark's count), reported as a fraction of the bf16 peak (MFU)."""
    import torch

    from SSA.ssa_decoder import SSADecoder, SSADecoderConfig, train_step

    mbs = TRAIN_CONFIGS[args.config]
    cfg = SSADecoderConfig()
    S = cfg.seq_length
    torch.manual_seed(1234)
    model = SSADecoder(cfg).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    ids = torch.randint(0, cfg.vocab_size, (mbs, S), device=dev)
    labels = torch.randint(0, cfg.vocab_size, (mbs, S), device=dev)
    n_params = sum(p.numel() for p in model.parameters())
    tokens = mbs * S
    pairs = mbs * cfg.num_attention_heads * S * (S + 1) // 2
    flops = 6 * n_params * tokens + 14 * cfg.kv_channels * pairs * cfg.num_layers
    log(f"[bench] config={args.config} params={n_params / 1e9:.3f}B tokens/step={tokens}")
    losses = []
    for _ in range(args.warmup):
        losses.append(train_step(model, opt, ids, labels))
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        losses.append(train_step(model, opt, ids, labels))
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) / args.steps * 1e3
    # attention's share: the SSA op fwd + bwd of one layer, timed alone
    from SSA.ssa_hip_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    H, D = cfg.num_attention_heads, cfg.kv_channels
    q = (torch.randn(mbs, H, S, D, device=dev) * 0.5).bfloat16()
    k, v, do = torch.randn_like(q), torch.randn_like(q), torch.randn_like(q)
    n, bb = torch.tensor(1.5, device=dev), torch.tensor(0.8, device=dev)
    for _ in range(2):
        o, m = ssa_flash_attn_forward(q, k, v, 1 / math.sqrt(D), n, bb, True)
        ssa_flash_attn_backward(q, k, v, o, do, m, 1 / math.sqrt(D), n, bb, True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(5):
        o, m = ssa_flash_attn_forward(q, k, v, 1 / math.sqrt(D), n, bb, True)
        ssa_flash_attn_backward(q, k, v, o, do, m, 1 / math.sqrt(D), n, bb, True)
    torch.cuda.synchronize()
    attn_ms = (time.perf_counter() - t1) / 5 * 1e3 * cfg.num_layers
    tflops = flops / (ms_step * 1e-3) / 1e12
    print(json.dumps({
        "metric": "1B Llama-style SSA decoder train step, tokens/s, 1 MI355X",
        "value": tokens / (ms_step * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: uniform-random token ids and labels, seed 1234, random init (std 0.02)",
        "config": {"workload": "1B decoder train step (train1b): forward, loss, backward, fused AdamW",
                   "layers": cfg.num_layers, "hidden": cfg.hidden_size, "heads": cfg.num_attention_heads,
                   "head_dim": cfg.kv_channels, "ffn": cfg.ffn_hidden_size, "vocab": cfg.vocab_size,
                   "seq_len": S, "micro_batch": mbs, "params": n_params,
                   "precision": "bf16 autocast (GEMMs, SSA attention), fp32 params / norms / loss / AdamW"},
        "model_tflops": tflops, "mfu": tflops / PEAK_BF16_TFLOPS,
        "model_gflop_per_step": flops / 1e9,
        "ssa_attention_ms_per_step": attn_ms, "ssa_attention_share": attn_ms / ms_step,
        "loss_first_last": [float(losses[0]), float(losses[-1])],
        "cpu_baseline": None,
    }))


def bench_decode(args, dev):
    """One decode step (every sequence's newest token against its full KV cache).

    A step is HBM-bound: value = algorithmic bytes (K and V cache rows read,
    q read, out written) per step time.  Also reported: the causal forward
    over the whole prefix on the same kernels (what the reference's generation
    loop runs per token), and the fp64 oracle decode on the host cores.
    """
    import torch

    from SSA.ssa_hip_kernel import ssa_decode_attention, ssa_decode_num_splits, ssa_flash_attn_forward

    B, Hq, Hkv, L, D = DECODE_CONFIGS[args.config]
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    torch.manual_seed(1234)
    q = (torch.randn(B, Hq, D, device=dev) * 0.5).to(dtype)
    kc = (torch.randn(B, Hkv, L, D, device=dev) * 0.5).to(dtype)
    vc = (torch.randn(B, Hkv, L, D, device=dev) * 0.5).to(dtype)
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    n = torch.tensor(1.5, device=dev)
    bb = torch.tensor(0.8, device=dev)
    scale = 1.0 / math.sqrt(D)
    esize = 2
    alg_bytes = 2 * B * Hkv * L * D * esize + 2 * B * Hq * D * esize

    def step():
        return ssa_decode_attention(q, kc, vc, lens, scale, n, bb)

    log(f"[bench] config={args.config} B={B} Hq={Hq} Hkv={Hkv} L={L} D={D}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / args.steps
    # A step is tens of microseconds, below the host's per-call cost, so the
    # device time comes from a HIP graph of `steps` decode steps (replayed
    # three times, every replay checked against the eager result).
    ref = step()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step()
    stream.wait_stream(side)
    with torch.cuda.graph(graph):
        outs = [step() for _ in range(args.steps)]
    replays = 3
    start.record(stream)
    for _ in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, ref) for o in outs), "graph replay differs from the eager decode"
    end.record(stream)
    torch.cuda.synchronize()
    # per-replay timing without the checks
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / (replays * args.steps)
    gbps = alg_bytes / (ms_step * 1e-3) / 1e9
    # the reference's per-token work: the causal forward over the whole prefix
    qf = (torch.randn(B, Hq, L, D, device=dev) * 0.5).to(dtype)
    for _ in range(2):
        ssa_flash_attn_forward(qf, kc, vc, scale, n, bb, True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(5):
        ssa_flash_attn_forward(qf, kc, vc, scale, n, bb, True)
    end.record(stream)
    torch.cuda.synchronize()
    prefix_ms = start.elapsed_time(end) / 5
    # context for the roofline: a plain device copy (reads and writes COPY_MIB MiB)
    src = torch.empty(COPY_MIB << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(5):
        dst.copy_(src)
    end.record(stream)
    torch.cuda.synchronize()
    copy_gbps = 2 * (COPY_MIB << 20) / (start.elapsed_time(end) / 5 * 1e-3) / 1e9
    del src, dst
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        from oracle import ssa_oracle as so

        qn = q[:1].float().cpu().numpy()
        kn, vn = kc[:1].float().cpu().numpy(), vc[:1].float().cpu().numpy()
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 10.0:
            so.ssa_decode(qn, kn, vn, [L], scale, 1.5, 0.8)
            reps += 1
        per_seq = (time.perf_counter() - t0) / reps
        cpu = {"value": (alg_bytes / B) / per_seq / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"fp64 numpy oracle decode of 1 of the {B} sequences (all {Hq} heads, {L} keys), "
                         f"{reps} repetitions in 10 s; value = that sequence's bytes / time"}
    print(json.dumps({
        "metric": "SSA decode step, KV-cache GB/s, 1 MI355X",
        "value": gbps, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "eager_ms_per_step": eager_ms, "timing": "HIP graph of `steps` decode steps",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic: q / K / V caches = 0.5 N(0,1), seed 1234, n=1.5, b=0.8, every cache full",
        "config": {"workload": f"SSA decode step ({args.config})", "B": B, "Hq": Hq, "Hkv": Hkv,
                   "cache_len": L, "D": D, "splits": ssa_decode_num_splits(B, Hq, Hkv, L),
                   "alg_bytes_per_step": alg_bytes},
        "roofline": {"kernel": "ssa_decode_kernel (+ merge)", "bound": "hbm", "achieved": gbps,
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": gbps / PEAK_HBM_GBPS, "traffic": None},
        "device_copy_gbps": copy_gbps,
        "prefix_recompute_ms": prefix_ms,
        "speedup_vs_prefix_recompute": prefix_ms / ms_step,
        "cpu_baseline": cpu,
    }))


if __name__ == "__main__":
    main()
