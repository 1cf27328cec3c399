"""Wait-state check of the library's gfx950 device assembly (a build step).

The compiler inserts the NOPs that hardware hazards need only around the
instructions it can see.  For an inline-assembly statement it checks the
registers the statement writes, not the ones it reads, so a vector-memory
instruction issued from assembly (the direct-to-LDS tile loads and the
buffer stores of csrc/ssa_tile.hpp) is not protected against:

* a VALU instruction that writes an SGPR (v_readfirstlane, v_readlane -- e.g.
  an SGPR spill reload --, v_cmp with an SGPR destination, carry-out forms)
  followed by a vector-memory instruction that reads that SGPR (descriptor,
  soffset, saddr): 5 wait states are required;
* an SALU write of M0 followed by an LDS DMA (buffer_* ... lds,
  global_load_lds_*), which reads M0: 1 wait state.

With fewer, the memory instruction can read the register's previous value
and so access a wrong address.  ``scan_asm`` walks a device .s file in
program order (a label does not reset the window, so fall-through paths are
covered) and returns every site with fewer wait states than required.
"""

from __future__ import annotations

import re
from pathlib import Path

VMEM = re.compile(r"^(buffer_|global_|flat_|scratch_)")
LDS_DMA = re.compile(r"^(buffer_\w+.*\blds\b|global_load_lds_)")
VALU_SGPR_WAIT = 5
M0_LDS_DMA_WAIT = 1


def _sregs(tok: str) -> set:
    tok = tok.strip().rstrip(",")
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    if tok == "m0":
        return {"m0"}
    return set()


def _valu_sgpr_defs(parts: list) -> set:
    op = parts[0]
    if not op.startswith("v_") or len(parts) < 2:
        return set()
    if op.startswith(("v_readfirstlane", "v_readlane")):
        return _sregs(parts[1])
    if op.startswith("v_cmp") and op.endswith("_e64"):
        return _sregs(parts[1])
    if re.match(r"v_(add|sub|subrev|addc|subb)_co_|v_(mad_u64_u32|mad_i64_i32|div_scale)", op) and len(parts) > 2:
        return _sregs(parts[2])
    return set()


def _salu_m0_def(parts: list) -> bool:
    return parts[0].startswith("s_") and len(parts) > 1 and parts[1] == "m0"


def scan_asm(text: str) -> list:
    """Hazard sites of one device assembly file: (function, wait states, needed, instruction)."""
    func = None
    window = []  # most recent first-to-last: (sgpr defs by VALU, writes m0 by SALU)
    sites = []
    for raw in text.split("\n"):
        m = re.match(r"^(_Z\S+|[A-Za-z_]\w*):", raw)
        if m and not raw.startswith((".", "\t")):
            func, window = m.group(1), []
            continue
        s = raw.split(";")[0].strip()
        if not s or s.startswith(".") or s.endswith(":"):
            continue
        parts = s.replace(",", " ").split()
        if parts[0] == "s_nop":
            n = int(parts[1], 0) + 1 if len(parts) > 1 else 1
            window.extend([(set(), False)] * n)
        else:
            if VMEM.match(parts[0]):
                used = set()
                for t in parts[1:]:
                    used |= _sregs(t)
                if LDS_DMA.match(s):
                    used.add("m0")
                # each rule on its own: the most recent VALU write of an SGPR the
                # instruction reads, and the most recent SALU write of M0
                vgpr_sgpr = used - {"m0"}
                for ws, (defs, _) in enumerate(reversed(window)):
                    if ws >= VALU_SGPR_WAIT:
                        break
                    if defs & vgpr_sgpr:
                        sites.append((func, ws, VALU_SGPR_WAIT, s))
                        break
                if "m0" in used:
                    for ws, (_, m0) in enumerate(reversed(window)):
                        if ws >= M0_LDS_DMA_WAIT:
                            break
                        if m0:
                            sites.append((func, ws, M0_LDS_DMA_WAIT, s))
                            break
            window.append((_valu_sgpr_defs(parts), _salu_m0_def(parts)))
        del window[:-8]
    return sites


def check_files(paths) -> list:
    out = []
    for p in paths:
        for site in scan_asm(Path(p).read_text()):
            out.append((Path(p).name, *site))
    return out
