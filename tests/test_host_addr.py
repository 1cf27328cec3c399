"""The kernels' own address code, replayed on the CPU under AddressSanitizer
and UndefinedBehaviorSanitizer.

luciole-1b_amd/csrc/ssa_plan.hpp holds the dispatch and per-lane load / store
addressing of every tile-streaming kernel (forward, both dK/dV kernels, the dS'
K pass, the recompute dQ pass, decode) as __host__ __device__ code; the
kernels call it with the device memory policy.  tests/host_addr/addr_replay.cpp
calls the same code for every workgroup, wave and lane of dense, GQA,
Megatron-strided, ragged and packed problems (and a sample of the benchmark
sizes), performing each access on exact-size host buffers and checking rows,
heads, documents, tile coverage, descriptor ranges, wave-uniform values and
the dS' workspace contents the dQ pass reads (see the program's header).

The second test plants indexing mistakes in a copy of the header (on the CPU
only) and requires the replay to fail on each: a kernel indexing change that
breaks an access fails here without any test-side mirror of the formula.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "luciole-1b_amd" / "csrc"
SRC = ROOT / "tests" / "host_addr" / "addr_replay.cpp"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
BASE = ["-x", "hip", "--cuda-host-only", "-std=c++20"]
SAN = ["-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all"]

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not found")


def _build(out: Path, include: Path, flags: list[str]) -> None:
    cmd = [HIPCC, *BASE, *flags, "-I", str(include), str(SRC), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert res.returncode == 0, f"{' '.join(cmd)}\n{res.stdout}\n{res.stderr[-4000:]}"


def _run(exe: Path, *args: str) -> subprocess.CompletedProcess:
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=900, env=env)


def test_replay_under_sanitizers(tmp_path):
    exe = tmp_path / "addr_replay"
    _build(exe, CSRC, ["-Wall", "-Werror", *SAN])
    res = _run(exe)
    assert res.returncode == 0, f"rc {res.returncode}\n{res.stdout[-3000:]}\n{res.stderr[-6000:]}"
    assert " 0 failures" in res.stdout, res.stdout[-3000:]
    assert "runtime error" not in res.stderr, res.stderr[-4000:]
    assert "FAILED" not in res.stdout


# (file, original text, planted mistake, what it breaks)
MUTATIONS = [
    ("ssa_tile.hpp", "grow = grow < nrows ? grow : nrows - 1;", "grow = grow <= nrows ? grow : nrows - 1;",
     "row clamp of partial tiles reads one row past the sequence"),
    ("ssa_plan.hpp", "ds_voff = static_cast<uint32_t>(((l32 >> 4) * 512 + (l32 & 15) * 8 + 16 * hh * 8) * 2);",
     "ds_voff = static_cast<uint32_t>(((l32 >> 4) * 512 + (l32 & 15) * 8 + 16 * hh * 4) * 2);",
     "dS' store lane offset of the 4-wave dK/dV kernel"),
    ("ssa_plan.hpp", "ds_src = static_cast<uint32_t>((16 * (lane >> 4) + ((lane & 15) ^ (4 * (lane >> 4)))) * 16);",
     "ds_src = static_cast<uint32_t>((16 * (lane >> 4) + (lane & 15)) * 16);",
     "dS' K pass lane permutation of the tile load"),
    ("ssa_plan.hpp", "    int r = q0 + lane;\n", "    int r = q0 + lane + 1;\n",
     "M / Delta rows of the two-wave dK/dV kernel"),
    ("ssa_common.hpp", "return x * q + (x < r ? x : r) + j;", "return x * q + j;",
     "XCD remap stops being a bijection"),
    ("ssa_plan.hpp", "nlo = key_edge ? nsub : (CAUSAL ? imin(BN / BMQ, nsub) : 0);",
     "nlo = key_edge ? nsub : (CAUSAL ? imin(BN / BMQ - 1, nsub) : 0);",
     "a causal-diagonal step treated as unmasked"),
    ("ssa_plan.hpp", "const int soff = mem.uniform(g * ds_tph1k + (CAUSAL ? qt * (qt + 1) : qt * 2 * nq32) * 1024);",
     "const int soff = mem.uniform(g * ds_tph1k + (CAUSAL ? qt * (qt + 1) : qt * 2 * nq32) * 1024 + "
     "static_cast<int>((ds_voff >> 4) & 1));",
     "a per-lane value passed where the kernel states a wave-uniform one"),
]


def _mutant(tmp_path: Path, k: int, fname: str, old: str, new: str) -> tuple[int, str, str]:
    inc = tmp_path / f"m{k}"
    shutil.copytree(CSRC, inc, ignore=shutil.ignore_patterns("*.hip"))
    path = inc / fname
    text = path.read_text()
    assert text.count(old) == 1, f"mutation {k}: the original text is not in {fname} exactly once"
    path.write_text(text.replace(old, new))
    exe = inc / "replay"
    _build(exe, inc, ["-O1"])
    res = _run(exe, "--quick")
    return res.returncode, res.stdout, res.stderr


def test_planted_mistakes_fail(tmp_path):
    with cf.ThreadPoolExecutor(max_workers=min(8, len(MUTATIONS))) as ex:
        futs = [ex.submit(_mutant, tmp_path, k, f, o, n) for k, (f, o, n, _) in enumerate(MUTATIONS)]
        results = [f.result() for f in futs]
    missed = [why for (rc, out, err), (_, _, _, why) in zip(results, MUTATIONS) if rc == 0 or "FAIL" not in err]
    assert not missed, f"planted mistakes the replay did not catch: {missed}"
