"""The reference harness's 96 recorded kernel cases, run through this build.

tests/golden/ref_parity_levels.json holds, per case shape (D=32, N in
{128, 512, 1024}, bf16/fp16, MHA/GQA, causal or not, contiguous or strided),
the reference Triton kernel's recorded error against its fp32 oracle on an
A100 (extracted by tests/golden/extract_ref_levels.py from
training/train/train_ssa_triton/logs/parity_reports/ssa_triton_v4_parity_76887.json).
Each case is run here on seeded inputs of the same shape and checked to the
parity bar of parity_util; the reference's recorded max_abs is printed next to
ours.  The inputs are not the reference's (its CUDA RNG stream is not
reproducible here), so the comparison is of error levels, not of values.

    python tests/test_gpu_ref_cases.py REPORT.md   # writes the side-by-side table
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest
import torch

_HERE = Path(__file__).resolve().parent
for _p in (_HERE, _HERE.parent, _HERE.parent / "luciole-1b_amd"):  # also when run as a script
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

from test_gpu_parity import _check, _run  # noqa: E402

LEVELS = json.loads((Path(__file__).resolve().parent / "golden" / "ref_parity_levels.json").read_text())
CASES = LEVELS["cases"]
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _case_id(c):
    c = c["case"]
    return f"{c['dtype']}-B{c['B']}-H{c['Hq']}x{c['Hkv']}-N{c['N']}-D{c['D']}-{'c' if c['causal'] else 'nc'}-{c['layout']}"


def _run_case(dev, entry, seed):
    c = entry["case"]
    return _run(dev, c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], DTYPES[c["dtype"]], c["causal"],
                layout=c["layout"], seed=seed)


@pytest.mark.gpu
@pytest.mark.parametrize("idx", range(len(CASES)), ids=[_case_id(c) for c in CASES])
def test_reference_case(gpu, idx):
    entry = CASES[idx]
    label, res_exact, res_kernel, mres = _run_case(gpu, entry, 1234 + idx)
    ref = entry["v4_vs_ref"]
    print(f"[ref levels] {label}: " + ", ".join(
        f"{t} ours={res_exact[t]['max_abs']:.2e} ref={ref[t]['max_abs']:.2e}" for t in ("out", "dq", "dk", "dv")),
        file=sys.stderr, flush=True)
    _check(label, res_exact, res_kernel, mres)


def main(path):
    dev = torch.device("cuda:0")
    rows = []
    worst = {t: [0.0, 0.0] for t in ("out", "dq", "dk", "dv")}
    worst_s = {t: [0.0, 0.0] for t in ("dn", "db")}
    for idx, entry in enumerate(CASES):
        label, res_exact, res_kernel, mres = _run_case(dev, entry, 1234 + idx)
        ref = entry["v4_vs_ref"]
        row = [_case_id(entry)]
        for t in ("out", "dq", "dk", "dv"):
            ours = res_exact[t]["max_abs_vs_rounded"]
            row.append(f"{ours:.2e} / {ref[t]['max_abs']:.2e}")
            worst[t][0] = max(worst[t][0], ours)
            worst[t][1] = max(worst[t][1], ref[t]["max_abs"])
        for t in ("dn", "db"):
            rel_ours = res_kernel[t]["abs_diff"] / max(abs(res_kernel[t]["ref"]), 1e-12)
            rel_ref = ref[t]["abs_diff"] / max(abs(ref[t]["ref"]), 1e-12)
            row.append(f"{rel_ours:.1e} / {rel_ref:.1e}")
            worst_s[t][0] = max(worst_s[t][0], rel_ours)
            worst_s[t][1] = max(worst_s[t][1], rel_ref)
        rows.append(row)
    lines = ["| case | out | dq | dk | dv | dn (rel) | db (rel) |", "|---|---|---|---|---|---|---|"]
    lines.append("| **max over cases** | " + " | ".join(f"**{a:.2e} / {b:.2e}**" for a, b in worst.values())
                 + " | " + " | ".join(f"**{a:.1e} / {b:.1e}**" for a, b in worst_s.values()) + " |")
    lines += ["| " + " | ".join(r) + " |" for r in rows]
    Path(path).write_text("Each cell: this build (MI355X) / reference Triton kernel (A100, recorded); "
                          "max |x - fp32 oracle rounded to the input dtype|.\n\n" + "\n".join(lines) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "ref_levels.md")
