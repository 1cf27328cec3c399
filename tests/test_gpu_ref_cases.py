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

and, beside it, REPORT.json: every case's errors, the limits they are held to
and a pass flag per case, as the reference harness's JSON report
(check_ssa_triton_parity.py:1118-1137).
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


_KEEP = ("max_abs_vs_rounded", "within_bound", "allclose", "got", "ref", "rel")


def _plain(st):
    """The report fields of a result dict: flags as they are, numbers to 3 significant digits."""
    out = {}
    for k, v in st.items():
        if k not in _KEEP:
            continue
        v = v.item() if hasattr(v, "item") else v
        out[k] = v if isinstance(v, bool) else float(f"{v:.3g}")
    return out


def main(path):
    import parity_util as pu

    dev = torch.device("cuda:0")
    rows = []
    report = []
    worst = {t: [0.0, 0.0] for t in ("out", "dq", "dk", "dv")}
    worst_s = {t: [0.0, 0.0] for t in ("dn", "db")}
    for idx, entry in enumerate(CASES):
        label, res_exact, res_kernel, mres = _run_case(dev, entry, 1234 + idx)
        ref = entry["v4_vs_ref"]
        try:
            _check(label, res_exact, res_kernel, mres)
            passed, err = True, None
        except AssertionError as e:
            passed, err = False, str(e)
        report.append({"case": entry["case"], "seed": 1234 + idx, "passed": passed, "error": err, "m_max_abs": mres,
                       "ours_vs_exact": {t: _plain(v) for t, v in res_exact.items()},
                       "ours_kernel_level": {t: _plain(v) for t, v in res_kernel.items()},
                       "reference_recorded": {t: float(f"{ref[t]['max_abs']:.3g}") for t in ("out", "dq", "dk", "dv")}
                       | {t: float(f"{ref[t]['abs_diff'] / max(abs(ref[t]['ref']), 1e-12):.3g}") for t in ("dn", "db")}})
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
    ok = all(r["passed"] for r in report)
    Path(path).write_text(
        "# Parity on the reference harness's 96 kernel case shapes: this build vs the reference Triton kernel\n\n"
        f"Command (repo root, GPU box): `python tests/test_gpu_ref_cases.py {path}`, which also writes\n"
        f"`{Path(path).with_suffix('.json')}` (per case: the shape, seed, pass flag, this build's errors against the "
        "fp64\noracle and the kernel-level backward, the reference's recorded errors; the limits at the top).\n"
        f"{'All' if ok else 'NOT all'} {len(report)} cases pass (`overall_passed: {str(ok).lower()}`).  Inputs are "
        "seeded here (the reference's CUDA RNG stream is not\nreproducible), so the comparison is of error levels on "
        "the same shapes, not of values.\n\n"
        "Each cell: this build (MI355X) / reference Triton kernel (A100, recorded); "
        "max |x - fp32 oracle rounded to the input dtype|.\n\n" + "\n".join(lines) + "\n")
    meta = {"device": torch.cuda.get_device_name(dev), "torch": torch.__version__, "hip": torch.version.hip,
            "source": "tests/test_gpu_ref_cases.py; reference levels from tests/golden/ref_parity_levels.json"}
    limits = {"tensor_atol": pu.ATOL, "tensor_rtol": pu.RTOL, "scalar_atol": pu.SCALAR_ATOL,
              "scalar_rtol": pu.SCALAR_RTOL, "elementwise": "max(2e-2, 1 ulp of the output dtype at |ref|)",
              "m_max_abs": 1e-2}
    out = {"meta": meta, "limits": limits, "cases": report, "overall_passed": all(r["passed"] for r in report)}
    # one line per case
    cases = ",\n".join(json.dumps(c, separators=(",", ":")) for c in out.pop("cases"))
    head = json.dumps(out, indent=1)[:-2]
    Path(path).with_suffix(".json").write_text(head + ',\n "cases": [\n' + cases + "\n ]\n}\n")
    print(f"wrote {path} and {Path(path).with_suffix('.json')}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "ref_levels.md")
