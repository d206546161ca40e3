"""Build gate over the gfx950 assembly of the kernels that issue loads from inline asm.

The decode GEMVs, the routed-expert kernels and the prefill GEMM issue their global loads
from inline asm, so the compiler tracks none of them: every wait is explicit, and a
register of an asm load may only be touched after an ``s_waitcnt vmcnt(N)`` with N no
larger than the number of vector-memory loads issued after it (vector-memory loads
retire in issue order). The compiler does not know that the registers are still being
written, so it may move, copy, spill or park them (``v_accvgpr_write``) before the wait;
the in-flight load then lands on registers whose contents have moved. That corrupts
results or faults the GPU, and no test on the CPU shows it, so the build refuses such
code:

* every innermost loop of every kernel that holds an asm load (the lines the compiler
  brackets with ``;;#ASMSTART`` / ``;;#ASMEND``) is scanned, in layout order and
  wrapping around the back edge, and any instruction touching an asm load's destination
  registers before a covering wait is reported (a copy, a spill store and an AGPR write
  of the register all touch it); asm loads outside those loops (prologues, loads issued
  ahead of a prelude) are scanned forward to their first covering wait the same way;
* a kernel with asm loads must spill no VGPRs.

``check_assembly(text, straight)`` returns the problems found in one
``--cuda-device-only -S`` output; ``build.py`` runs it on the sources listed in ``GATED``
(with the path check on those in ``STRAIGHT``) and fails the build on any problem.
"""
from __future__ import annotations

import re

# the sources whose kernels issue loads from inline asm
GATED = ("decode.hip", "gemv.hip", "gemv_grouped.hip", "moe.hip", "prefill.hip")
# of those, the ones whose loads outside the steady-state loops are issued unconditionally,
# so that every control-flow path from such a load to its uses is checked too
STRAIGHT = ("decode.hip", "gemv.hip", "gemv_grouped.hip", "moe.hip")

ASM_MARK = "; asm-load"


def _regs(tok: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _operands(line: str) -> list[str]:
    line = line.split(";", 1)[0]
    parts = line.split(None, 1)
    return [t.strip().split()[0] for t in parts[1].split(",") if t.strip()] if len(parts) > 1 else []


def mark_asm_loads(lines: list[str]) -> list[str]:
    """The lines with every register-destination global load issued from inline asm
    suffixed by ASM_MARK (LDS-DMA loads write no registers and are left unmarked)."""
    out, inside = [], False
    for l in lines:
        s = l.strip()
        if s.startswith(";;#ASMSTART"):
            inside = True
        elif s.startswith(";;#ASMEND"):
            inside = False
        elif inside and re.match(r"global_load_dword", s) and "lds" not in s:
            l = l + "\t" + ASM_MARK
        out.append(l)
    return out


def inner_loops(asm: list[str]) -> list[list[str]]:
    """The instructions of each innermost loop, in layout order: the header's block, the
    blocks marked as inside it (a latch may sit above the header and fall into it), up to
    the last branch back to any of them."""
    return [[l for l in asm[a:b + 1] if l.strip() and not l.strip().startswith((";", "."))]
            for a, b in inner_loop_ranges(asm)]


def inner_loop_ranges(asm: list[str]) -> list[tuple[int, int]]:
    """(first, last) line indices of each innermost loop (see inner_loops)."""
    loops = []
    inner = any("Inner Loop Header" in l for l in asm)     # else: a lone loop's "Loop Header"
    for h, line in enumerate(asm):
        if "Loop Header" not in line or (inner and "Inner" not in line):
            continue
        # the header comment may sit on its own line under the block's label
        label = (asm[h - 1] if line.lstrip().startswith(";") and h else line).split(":")[0].strip()
        name = label[2:] if label.startswith(".L") else label.lstrip(".")   # ".LBB0_1" -> "BB0_1"
        members = {label} | {l.split(":")[0].strip() for l in asm if f"in Loop: Header={name} " in l + " "}
        first = min(i for i, l in enumerate(asm) if l.split(":")[0].strip() in members and ":" in l)
        back = [i for i, l in enumerate(asm)
                if re.search(r"s_(?:cbranch_\w+|branch)\s+(\S+)", l)
                and re.search(r"s_(?:cbranch_\w+|branch)\s+(\S+)", l).group(1) in members]
        if not back:                            # no branch back to the loop's blocks: not a loop body
            continue
        last = max(back)
        loops.append((first, last))
    return loops


_LABEL = re.compile(r"^(\.L\w+|\w+):")
_BRANCH = re.compile(r"\s*(s_branch|s_cbranch_\w+)\s+(\S+)")
_END = re.compile(r"\s*(s_endpgm|s_setpc_b64|s_trap)\b")


def basic_blocks(asm: list[str]):
    """(blocks, successors, block of line): blocks as lists of (line index, instruction) in
    layout order, split at labels and after branches; successors by branch target and
    fall-through."""
    blocks, labels, cur = [], {}, []
    def close():
        nonlocal cur
        if cur:
            blocks.append(cur)
            cur = []
    for i, l in enumerate(asm):
        st = l.strip()
        m = _LABEL.match(l)
        if m:
            close()
            labels[m.group(1)] = len(blocks)
            cur = [(i, None)]               # a block may start with its label only
            continue
        if not st or st.startswith((";", ".")):
            continue
        cur.append((i, l))
        if _BRANCH.match(l) or _END.match(l):
            close()
    close()
    succ = []
    for k, blk in enumerate(blocks):
        last = next((l for _, l in reversed(blk) if l is not None), "")
        m = _BRANCH.match(last)
        out = []
        if m:
            if m.group(2) in labels:
                out.append(labels[m.group(2)])
            if m.group(1) != "s_branch" and k + 1 < len(blocks):
                out.append(k + 1)
        elif not _END.match(last) and k + 1 < len(blocks):
            out.append(k + 1)
        succ.append(out)
    where = {i: (k, p) for k, blk in enumerate(blocks) for p, (i, _) in enumerate(blk)}
    return blocks, succ, where


def early_uses_straight(asm: list[str], in_loop) -> tuple[int, list[str]]:
    """Marked loads outside every innermost loop (a pipeline's prologue, loads issued ahead of
    a prelude), followed along every control-flow path from the load to the first wait that
    covers it on that path (vmcnt(N), N no larger than the vector-memory loads issued since
    on that path, vmcnt(0) included); any instruction touching the load's registers on a
    path before such a wait is reported. The paths are those of the control-flow graph, a
    superset of the feasible ones, so a clean result is a proof; it suits code whose loads
    are issued unconditionally (the rolling pipelines' prologues). Code that issues loads
    under conditions correlated with later branches (the prefill tile's prologue) reads as
    uncovered on infeasible paths: STRAIGHT names the sources this check applies to."""
    blocks, succ, where = basic_blocks(asm)
    bad, n = [], 0
    for i, l in enumerate(asm):
        if ASM_MARK not in l or in_loop(i) or not _REG_LOAD.match(l):
            continue
        n += 1
        dst = _regs(_operands(l)[0])
        k0, p0 = where[i]
        work, seen, found = [(k0, p0 + 1, 0)], set(), None
        while work and found is None:
            k, p, younger = work.pop()
            key = (k, p, min(younger, 64))
            if key in seen:
                continue
            seen.add(key)
            covered = False
            for _, m in blocks[k][p:]:
                if m is None:
                    continue
                if _LOAD.match(m):
                    younger += 1
                w = _VMCNT.search(m)
                if w and int(w.group(1)) <= younger:
                    covered = True
                    break
                if _WAIT.match(m):
                    continue
                ops = _operands(m)
                if ops and dst & set().union(*[_regs(t) for t in ops]):
                    found = f"{l.strip()} -> {m.strip()}"
                    break
            if not covered and found is None:
                work += [(s, 0, younger) for s in succ[k]]
        if found:
            bad.append(found)
    return n, bad


_LOAD = re.compile(r"\s*(global_load|buffer_load)")   # every vector-memory load counts in vmcnt
_REG_LOAD = re.compile(r"\s*global_load_dword")
_WAIT = re.compile(r"\s*s_waitcnt")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")


def early_uses_in(body: list[str], only_marked: bool = False) -> tuple[int, list[str]]:
    """(loads checked, descriptions of uses before the load's wait) for one loop body.
    only_marked: check only the loads mark_asm_loads marked (compiler-issued loads carry
    compiler-inserted waits); every vector-memory load still counts as a younger one."""
    info = []   # per line: (a load, the vmcnt of a wait or -1, a waitcnt, registers touched)
    for m in body:
        w = _VMCNT.search(m)
        waiting = bool(_WAIT.match(m))
        ops = [] if waiting else _operands(m)
        info.append((bool(_LOAD.match(m)), int(w.group(1)) if w else -1, waiting,
                     set().union(*[_regs(t) for t in ops]) if ops else set()))
    bad, n = [], 0
    for i, l in enumerate(body):
        if not _REG_LOAD.match(l) or "lds" in l or (only_marked and ASM_MARK not in l):
            continue
        n += 1
        dst, younger, done = _regs(_operands(l)[0]), 0, False
        for k in range(1, 2 * len(body)):
            j = (i + k) % len(body)
            is_load, vm, waiting, touched = info[j]
            if is_load:
                younger += 1
            # vmcnt(0) waits sit on the last stages' branches (not taken in the steady
            # state): only the steady-state waits count, so the check errs towards refusing
            if 0 < vm <= younger:
                done = True
            if waiting:
                continue
            if dst & touched:
                if not done:
                    bad.append(f"{l.strip()} -> {body[j].strip()}")
                break
    return n, bad


def early_uses(asm: list[str], only_marked: bool = False) -> tuple[int, list[str]]:
    """(loads checked, early uses) summed over every innermost loop of asm."""
    n, bad = 0, []
    for body in inner_loops(asm):
        k, b = early_uses_in(body, only_marked)
        n, bad = n + k, bad + b
    return n, bad


def kernel_ranges(lines: list[str]) -> dict[str, tuple[int, int]]:
    """Kernel symbol -> (first line, .Lfunc_end line) for every function in the assembly."""
    out = {}
    for i, l in enumerate(lines):
        m = re.match(r"([A-Za-z_][\w.$]*):\s*(?:;.*)?$", l)
        if not m or m.group(1).startswith(".L"):
            continue
        name = m.group(1)
        stop = next((j for j in range(i, len(lines)) if lines[j].startswith(f".Lfunc_end")), None)
        if stop is not None and any(lines[k].strip() and not lines[k].strip().startswith((";", "."))
                                    for k in range(i + 1, min(stop, i + 4))):
            out[name] = (i, stop)
    return out


def spill_counts(text: str) -> dict[str, int]:
    """Kernel symbol -> .vgpr_spill_count from the code object metadata."""
    out = {}
    for m in re.finditer(r"\.name:\s+(\S+)\n(?:(?!\s+- \.).*\n)*?.*?\.vgpr_spill_count:\s+(\d+)", text):
        out[m.group(1)] = int(m.group(2))
    return out


def check_assembly(text: str, straight: bool = True) -> tuple[int, list[str]]:
    """(asm loads checked, problems) for one device assembly file: early uses of asm-load
    registers in any kernel's innermost loops and, with ``straight``, on every path from the
    loads outside them; and VGPR spills in any kernel that issues asm loads."""
    lines = mark_asm_loads(text.splitlines())
    spills = spill_counts(text)
    checked, problems = 0, []
    for name, (a, b) in kernel_ranges(lines).items():
        body = lines[a:b]
        if not any(ASM_MARK in l for l in body):
            continue
        n, bad = early_uses(body, only_marked=True)
        n2, bad2 = 0, []
        if straight:
            ranges = inner_loop_ranges(body)
            n2, bad2 = early_uses_straight(body, lambda i: any(a <= i <= b for a, b in ranges))
        checked += n + n2
        problems += [f"{name}: asm-load registers touched before their wait: {x}" for x in bad + bad2]
        if spills.get(name, 0):
            problems.append(f"{name}: {spills[name]} VGPRs spilled in a kernel with in-flight asm loads")
    return checked, problems
