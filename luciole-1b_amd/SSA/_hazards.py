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
  global_load_lds_*), which reads M0: 1 wait state;
* a vector-memory store of more than 8 bytes (global_/buffer_/flat_/scratch_
  store_dwordx3, _dwordx4) followed by a VALU instruction that writes one of
  its data VGPRs: 2 wait states on gfx940 and later (the store reads its data
  after issue, so an early overwrite changes what is stored).

With fewer, the memory instruction can read the register's previous value
and so access a wrong address (or, for the store data, store the new value).  ``scan_asm`` walks a device .s file in
program order (a label does not reset the window, so fall-through paths are
covered; an unconditional transfer -- s_endpgm, s_branch, s_setpc -- does,
since the instruction after it is never its successor) and returns every
site with fewer wait states than required.

The dK/dV accumulators are MFMAs issued from inline assembly into AGPRs
(mfma32_acc / acc_fence in csrc/ssa_common.hpp), which the compiler's hazard
recognizer does not see either.  ``scan_agpr`` checks them on the control-flow
graph of each function: every such MFMA accumulates in place (dst = srcC, both
AGPR; srcA / srcB VGPR) right after its own s_nop of at least 2 wait states,
and every other instruction that names one of their AGPRs is reached, on every
path, at least ACC_READ_WAIT wait states after the last of them; and no
source VGPR of such an MFMA was written by a compiler-issued MFMA fewer than
ACC_READ_WAIT wait states before it on any path (the compiler pads that
hazard only between the MFMAs it sees).
"""

from __future__ import annotations

import re
from pathlib import Path

VMEM = re.compile(r"^(buffer_|global_|flat_|scratch_)")
LDS_DMA = re.compile(r"^(buffer_\w+.*\blds\b|global_load_lds_)")
VALU_SGPR_WAIT = 5
M0_LDS_DMA_WAIT = 1
STORE_DATA_WAIT = 2
WIDE_STORE = re.compile(r"^(global|buffer|flat|scratch)_store_dwordx[34]$")
# VALU instructions whose first operand is not a VGPR destination
_VALU_NO_VDST = re.compile(r"^v_(readlane|readfirstlane|cmp|cmpx|nop)")
ACC_MFMA_SRC_WAIT = 2   # VALU write of an MFMA source -> MFMA
ACC_READ_WAIT = 19      # XDL write (up to 16 passes) -> any other access of its result


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
    window = []  # most recent first-to-last: (sgpr defs by VALU, writes m0 by SALU, wide-store data VGPRs)
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
            window.extend([(set(), False, set())] * n)
        else:
            if parts[0].startswith("v_") and not _VALU_NO_VDST.match(parts[0]) and len(parts) > 1:
                vdst = _vregs(parts[1])
                for ws, (_, _, data) in enumerate(reversed(window)):
                    if ws >= STORE_DATA_WAIT:
                        break
                    if data & vdst:
                        sites.append((func, ws, STORE_DATA_WAIT, s))
                        break
            if VMEM.match(parts[0]):
                used = set()
                for t in parts[1:]:
                    used |= _sregs(t)
                if LDS_DMA.match(s):
                    used.add("m0")
                # each rule on its own: the most recent VALU write of an SGPR the
                # instruction reads, and the most recent SALU write of M0
                vgpr_sgpr = used - {"m0"}
                for ws, (defs, _, _) in enumerate(reversed(window)):
                    if ws >= VALU_SGPR_WAIT:
                        break
                    if defs & vgpr_sgpr:
                        sites.append((func, ws, VALU_SGPR_WAIT, s))
                        break
                if "m0" in used:
                    for ws, (_, m0, _) in enumerate(reversed(window)):
                        if ws >= M0_LDS_DMA_WAIT:
                            break
                        if m0:
                            sites.append((func, ws, M0_LDS_DMA_WAIT, s))
                            break
            data = set()
            if WIDE_STORE.match(parts[0]) and len(parts) > 2:
                data = _vregs(parts[1] if parts[0].startswith("buffer_") else parts[2])
            window.append((_valu_sgpr_defs(parts), _salu_m0_def(parts), data))
            if parts[0] in ("s_endpgm", "s_branch", "s_setpc_b64"):
                window = []
        del window[:-8]
    return sites


_ACC_FORM = re.compile(r"^v_mfma_\w+ (a\[\d+:\d+\]), v\[\d+:\d+\], v\[\d+:\d+\], (a\[\d+:\d+\])$")
_AREG = re.compile(r"\ba(\d+)\b|\ba\[(\d+):(\d+)\]")
_BRANCH = re.compile(r"^s_(c?branch)\w* (\.L\w+)")
_INF = 1 << 30


def _vregs(tok: str) -> set:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok) or re.fullmatch(r"v(\d+)()", tok)
    if not m:
        return set()
    lo = int(m.group(1))
    return set(range(lo, int(m.group(2) or lo) + 1))


def _aregs(ins: str) -> set:
    out = set()
    for one, lo, hi in _AREG.findall(ins):
        out |= {int(one)} if one else set(range(int(lo), int(hi) + 1))
    return out


def _functions(text: str):
    """(name, [(instruction, from_inline_asm) or label]) of each function."""
    name, body, in_asm = None, [], False
    for raw in text.split("\n"):
        m = re.match(r"^(_Z\S+|[A-Za-z_]\w*):", raw)
        if m and not raw.startswith((".", "\t")):
            if name:
                yield name, body
            name, body, in_asm = m.group(1), [], False
            continue
        if name is None:
            continue
        if raw.strip().startswith(".Lfunc_end"):
            yield name, body
            name = None
            continue
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        lab = re.match(r"^(\.L\w+):", raw)
        if lab:
            body.append(lab.group(1))
            continue
        s = raw.split(";")[0].strip()
        if s and not s.startswith("."):
            body.append((s, in_asm))
    if name:
        yield name, body


def scan_agpr(text: str) -> list:
    """Sites of one device assembly file where an inline-assembly AGPR
    accumulation is not covered: (function, wait states, needed, instruction)."""
    sites = []
    for func, body in _functions(text):
        # basic blocks: split at labels and after branches / ends
        blocks, labels, cur = [], {}, []
        for item in body:
            if isinstance(item, str):
                if cur:
                    blocks.append(cur)
                    cur = []
                labels[item] = len(blocks)
                continue
            cur.append(item)
            if item[0].startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
                blocks.append(cur)
                cur = []
        if cur:
            blocks.append(cur)
        acc, acc_regs = set(), set()
        for bi, blk in enumerate(blocks):
            for k, (ins, in_asm) in enumerate(blk):
                if in_asm and ins.startswith("v_mfma") and _aregs(ins):
                    acc.add((bi, k))
                    m = _ACC_FORM.match(ins)
                    if not m or m.group(1) != m.group(2):
                        sites.append((func, 0, ACC_MFMA_SRC_WAIT, ins))
                        continue
                    acc_regs |= _aregs(m.group(1))
                    prev = blk[k - 1][0] if k else ""
                    pm = re.match(r"s_nop (\d+)", prev)
                    if not pm or int(pm.group(1), 0) + 1 < ACC_MFMA_SRC_WAIT:
                        sites.append((func, int(pm.group(1), 0) + 1 if pm else 0, ACC_MFMA_SRC_WAIT, ins))
        if not acc:
            continue
        succ = []
        for bi, blk in enumerate(blocks):
            last = blk[-1][0]
            nxt = []
            m = _BRANCH.match(last)
            if m and m.group(2) in labels:
                nxt.append(labels[m.group(2)])
            if not last.startswith(("s_branch", "s_endpgm", "s_setpc")) and bi + 1 < len(blocks):
                nxt.append(bi + 1)
            succ.append(nxt)

        def walk(bi, dist, report):
            for k, (ins, _) in enumerate(blocks[bi]):
                if (bi, k) in acc:
                    dist = 0
                    continue
                if report and dist < ACC_READ_WAIT and _aregs(ins) & acc_regs:
                    sites.append((func, dist, ACC_READ_WAIT, ins))
                nop = re.match(r"s_nop (\d+)", ins)
                dist = min(_INF, dist + (int(nop.group(1), 0) + 1 if nop else 1))
            return dist

        # fewest wait states since the last accumulation, over all paths into each block
        entry = [None] * len(blocks)
        entry[0] = _INF
        work = [0]
        while work:
            bi = work.pop()
            out = walk(bi, entry[bi], False)
            for nb in succ[bi]:
                if entry[nb] is None or out < entry[nb]:
                    entry[nb] = out
                    work.append(nb)
        for bi in range(len(blocks)):
            if entry[bi] is not None:
                walk(bi, entry[bi], True)

        # wait states since a compiler-issued MFMA wrote each VGPR (only those
        # still under ACC_READ_WAIT), at each block entry: fewest over all paths
        def mfma_walk(bi, state, report):
            pos, written = 0, {}
            for k, (ins, _) in enumerate(blocks[bi]):
                ops = [t.strip() for t in ins.split(" ", 1)[1].split(",")] if " " in ins else []
                if (bi, k) in acc:
                    d = min((pos - written[r] if r in written else state.get(r, _INF) + pos
                             for r in _vregs(ops[1]) | _vregs(ops[2])), default=_INF)
                    if report and d < ACC_READ_WAIT:
                        sites.append((func, d, ACC_READ_WAIT, ins))
                elif ins.startswith("v_mfma") and ops:
                    for r in _vregs(ops[0]):
                        written[r] = pos + 1  # wait states count from the next instruction
                nop = re.match(r"s_nop (\d+)", ins)
                pos += int(nop.group(1), 0) + 1 if nop else 1
            out = {r: d + pos for r, d in state.items() if d + pos < ACC_READ_WAIT}
            for r, w in written.items():
                if pos - w < ACC_READ_WAIT:
                    out[r] = pos - w
            return out

        ment = [None] * len(blocks)
        ment[0] = {}
        work = [0]
        while work:
            bi = work.pop()
            out = mfma_walk(bi, ment[bi], False)
            for nb in succ[bi]:
                if ment[nb] is None:
                    new = dict(out)
                else:
                    new = dict(ment[nb])
                    for r, d in out.items():
                        if d < new.get(r, _INF):
                            new[r] = d
                if new != ment[nb]:
                    ment[nb] = new
                    work.append(nb)
        for bi in range(len(blocks)):
            if ment[bi] is not None:
                mfma_walk(bi, ment[bi], True)
    return sites


def check_files(paths) -> list:
    out = []
    for p in paths:
        text = Path(p).read_text()
        for site in scan_asm(text) + scan_agpr(text):
            out.append((Path(p).name, *site))
    return out
