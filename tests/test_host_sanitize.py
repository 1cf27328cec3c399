"""Host-side validation of the C ABI under AddressSanitizer + UndefinedBehaviorSanitizer.

The three sources that hold the entry points' validation (ssa_abi.hip,
ssa_noalloc.hip, decoder_ops.hip) are compiled with host-only sanitizers
(device code is built as usual), linked with the library's other objects into
tests/host_sanitize/validate_main.c, and run on the CPU: every entry point and
size query is called with NULL, zero, negative, INT32_MIN/MAX and huge-stride
arguments.  Any signed overflow, division by zero or bad memory access in the
host arithmetic aborts the program.  The program passes fake device pointers,
so it does not run where a GPU is visible.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "luciole-1b_amd" / "csrc"
BUILD = ROOT / "luciole-1b_amd" / "_build"
SANITIZED = ("ssa_abi", "ssa_noalloc", "decoder_ops")
# every other source of the library, linked as built
PLAIN = tuple(sorted(f.stem for f in CSRC.glob("*.hip") if f.stem not in SANITIZED))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANG = "/opt/rocm/llvm/bin/clang"
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all"]


def _run(cmd, cwd):
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, f"{' '.join(map(str, cmd))}\n{res.stdout}\n{res.stderr}"
    return res


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible; the driver passes fake device pointers")
def test_validation_is_ub_free_under_sanitizers(tmp_path):
    if not (Path(HIPCC).exists() and Path(CLANG).exists()):
        pytest.skip("hipcc / ROCm clang not found")
    missing = [n for n in PLAIN if not (BUILD / f"{n}.o").exists()]
    if missing:
        pytest.skip(f"library objects not built ({missing}); run __graft_entry__.build() first")
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++20", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    procs = [subprocess.Popen([HIPCC, *flags, *HOST_SAN, "-c", str(CSRC / f"{n}.hip"), "-o", f"{n}.o"],
                              cwd=tmp_path, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
             for n in SANITIZED]
    for n, p in zip(SANITIZED, procs):
        out, err = p.communicate(timeout=600)
        assert p.returncode == 0, f"{n}: {out}\n{err}"
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    _run([CLANG, "-O1", "-g", "-std=c11", "-Wall", "-Werror", *san, "-c",
          str(ROOT / "tests" / "host_sanitize" / "validate_main.c"), "-o", "main.o"], tmp_path)
    objs = ["main.o", *(f"{n}.o" for n in SANITIZED), *(str(BUILD / f"{n}.o") for n in PLAIN)]
    _run([CLANG + "++", *san, "-o", "validate", *objs, "-L/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,/opt/rocm/lib"], tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([str(tmp_path / "validate")], capture_output=True, text=True, timeout=300, env=env)
    assert res.returncode == 0, f"sanitizer run failed (rc {res.returncode}):\n{res.stdout}\n{res.stderr[-4000:]}"
    assert "0 failures" in res.stdout, res.stdout
    assert "runtime error" not in res.stderr, res.stderr[-4000:]
