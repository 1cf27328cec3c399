"""Build libssa_mi355x.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``luciole-1b_amd/_build``
(in parallel), then linked into ``luciole-1b_amd/SSA/libssa_mi355x.so``.  Run as
``python luciole-1b_amd/SSA/_build.py`` or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent            # luciole-1b_amd/SSA
ROOT_DIR = PKG_DIR.parent                            # luciole-1b_amd
CSRC = ROOT_DIR / "csrc"
BUILD_DIR = ROOT_DIR / "_build"
LIB_NAME = "libssa_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: packed fp32 VALU forms are kept out of the generated code.
# -Werror=inline-asm: an inline-assembly statement that clobbers a register
# the compiler reserves (M0, for instance) fails the build instead of warning.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Werror=inline-asm",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
]

# Per-source additions.  ssa_bwd.hip: builtin MFMAs write arch VGPRs (the
# VALU reads S and dP there without copies); the dK/dV accumulators are held in
# AGPRs by the inline assembly of ssa_common.hpp (mfma32_acc / acc_fence).
SOURCE_FLAGS = {
    "ssa_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "ssa_bwd_dkdv2w.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the SSA HIP library cannot be built")


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stderr or "").splitlines() if ln.strip() and noise not in ln]
    if msgs:
        print(f"[ssa build] {src.name}:\n" + "\n".join(msgs), file=sys.stderr)


def _device_asm(src: Path, out: Path, extra: list[str]) -> None:
    """The gfx950 assembly of one source (for the wait-state check)."""
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), *extra, "--cuda-device-only", "-S", str(src),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_library(extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compile every HIP source, check the device assembly's wait states
    (SSA/_hazards.py) and link the shared library.  Returns its path."""
    from . import _hazards  # noqa: PLC0415  (package-relative when imported as SSA._build)

    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    asms = [BUILD_DIR / (s.stem + ".gfx950.s") for s in sources]
    jobs = jobs or min(2 * len(sources), max(1, os.cpu_count() or 2), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, extra) for s, o in zip(sources, objs)]
        futs += [ex.submit(_device_asm, s, a, extra) for s, a in zip(sources, asms)]
        for f in futs:
            f.result()
    sites = _hazards.check_files(asms)
    if sites:
        lines = "\n".join(f"  {f}: {fn}: {ws} wait state(s), {need} needed: {ins}" for f, fn, ws, need, ins in sites[:20])
        raise RuntimeError(f"{len(sites)} instruction(s) read a register too soon after its write "
                           f"(SSA/_hazards.py):\n{lines}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    sys.path.insert(0, str(ROOT_DIR))
    from SSA._build import build_library as _bl  # run as a script: import through the package

    print(_bl())
