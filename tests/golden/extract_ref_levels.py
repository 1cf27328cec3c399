#!/usr/bin/env python3
"""Extract the reference Triton kernel's recorded error levels into a fixture.

The reference's parity harness (training/train/train_ssa_triton/check_ssa_triton_parity.py)
stored its results for 144 kernel cases (D=32, N in {128, 512, 1024}, bf16 and
fp16, MHA and GQA, causal and not, contiguous and strided, NVIDIA A100) in
training/train/train_ssa_triton/logs/parity_reports/ssa_triton_v4_parity_76887.json.
This script copies, per case, the error of the reference kernel against the
harness's fp32 oracle ("v4_vs_ref" and "v3_vs_ref": max_abs and rel_rmse of
out/dq/dk/dv, abs_diff and limit of dn/db) into ref_parity_levels.json, so the
GPU tests can report this build's error next to the reference's own on the
same case shapes.  Data only; run in a container that holds the reference:

    python tests/golden/extract_ref_levels.py /root/reference
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPORT = "training/train/train_ssa_triton/logs/parity_reports/ssa_triton_v4_parity_76887.json"
TENSORS = ("out", "dq", "dk", "dv")
SCALARS = ("dn", "db")


def levels(block):
    out = {}
    for t in TENSORS:
        out[t] = {"max_abs": block[t]["max_abs"], "rel_rmse": block[t]["rel_rmse"]}
    for s in SCALARS:
        out[s] = {"abs_diff": block[s]["abs_diff"], "limit": block[s]["limit"], "ref": block[s]["b"]}
    return out


def main():
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    data = json.loads((root / REPORT).read_text())
    suite = next(s for s in data["suites"] if s["name"] == "kernel_suite")
    cases = []
    for r in suite["results"]:
        if "v4_vs_ref" not in r:  # cases run without the fp32 oracle carry no error levels
            continue
        cases.append({"case": r["case"], "v4_vs_ref": levels(r["v4_vs_ref"]), "v3_vs_ref": levels(r["v3_vs_ref"]),
                      "passed": r["passed"]})
    fixture = {
        "source": REPORT,
        "device": data["meta"]["cuda_device"],
        "seed": data["meta"]["seed"],
        "ssa_n": data["args"]["ssa_n"],
        "ssa_b": data["args"]["ssa_b"],
        # check_ssa_triton_parity.py:1060-1069
        "tolerances": {"bf16": {"atol": 2e-2, "rtol": 5e-2}, "fp16": {"atol": 2e-2, "rtol": 5e-2},
                       "scalar": {"atol": 2e-3, "rtol": 2e-2}},
        "cases": cases,
    }
    (HERE / "ref_parity_levels.json").write_text(json.dumps(fixture, separators=(",", ":")))
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
