"""The pipelined prefill kernel issues its global loads from inline asm, so the
compiler does not wait for them: every wait is explicit. This checks the gfx950
ISA of that kernel's main loop: each register-destination load's registers are
touched only after an s_waitcnt vmcnt(N) with N no larger than the number of
vector-memory loads issued after it (vector-memory loads retire in issue order).
A compiler change that schedules a use ahead of its wait would fail here.
Needs hipcc (present on the build host); no GPU."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "openflowlm-next_amd" / "csrc" / "prefill.hip"


def _regs(tok: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _operands(line: str) -> list[str]:
    parts = line.split(None, 1)
    return [t.strip().split()[0] for t in parts[1].split(",") if t.strip()] if len(parts) > 1 else []


def inner_loops(asm: list[str]) -> list[list[str]]:
    """The instructions of each innermost loop, in layout order: the header's block, the
    blocks marked as inside it (a latch may sit above the header and fall into it), up to
    the last branch back to any of them."""
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
        loops.append([l for l in asm[first:last + 1] if l.strip() and not l.strip().startswith((";", "."))])
    return loops


def early_uses_in(body: list[str]) -> tuple[int, list[str]]:
    """(loads checked, descriptions of uses before the load's wait) for one loop body."""
    bad, n = [], 0
    for i, l in enumerate(body):
        if not re.match(r"\s*global_load_dword", l) or "lds" in l:
            continue
        n += 1
        dst, younger, done = _regs(_operands(l)[0]), 0, False
        for k in range(1, 2 * len(body)):
            m = body[(i + k) % len(body)]
            if re.match(r"\s*global_load", m):
                younger += 1
            w = re.search(r"vmcnt\((\d+)\)", m)
            # vmcnt(0) waits sit on the last stages' branches; only count steady-state waits
            if w and 0 < int(w.group(1)) <= younger:
                done = True
            if re.match(r"\s*s_waitcnt", m):
                continue
            touched = set().union(*[_regs(t) for t in _operands(m)]) if _operands(m) else set()
            if dst & touched:
                if not done:
                    bad.append(f"{l.strip()} -> {m.strip()}")
                break
    return n, bad


def early_uses(asm: list[str]) -> tuple[int, list[str]]:
    """(loads checked, early uses) summed over every innermost loop of asm."""
    n, bad = 0, []
    for body in inner_loops(asm):
        k, b = early_uses_in(body)
        n, bad = n + k, bad + b
    return n, bad


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_prefill_loop_waits_cover_every_asm_load(tmp_path):
    out = tmp_path / "prefill.s"
    cmd = ["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{SRC.parent}", "--cuda-device-only", "-S",
           str(SRC), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text().splitlines()
    for prec in (0, 1):
        for mixed, nloops in ((0, 1), (1, 2)):      # 256-row tiles only; + the 192-row body
            start = next(i for i, l in enumerate(text)
                         if re.match(rf"_ZN12_GLOBAL__N_118prefill_dma_kernelILi{prec}ELb{mixed}EE\w*:", l))
            stop = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
            loops = inner_loops(text[start:stop])
            what = f"precision {prec} mixed {mixed}"
            assert len(loops) == nloops, f"{what}: expected {nloops} tile loops, found {len(loops)}"
            for body in loops:
                n, bad = early_uses_in(body)
                assert n >= 6, f"{what}: expected the weight loads of the unrolled loop, found {n}"
                assert not bad, f"{what}: registers used before their load's wait: {bad[:3]}"
        # the grouped expert GEMM's tile loop and the gate/up GEMM with the SwiGLU epilogue
        for kname, what in ((rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb0EE", "moe"),
                            (rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb1EE", "moe swiglu"),
                            (rf"_ZN12_GLOBAL__N_121prefill_swiglu_kernelILi{prec}EE", "swiglu")):
            start = next(i for i, l in enumerate(text) if re.match(kname + r"\w*:", l))
            stop = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
            loops = inner_loops(text[start:stop])
            assert len(loops) == 1, f"{what} precision {prec}: expected 1 tile loop, found {len(loops)}"
            for body in loops:
                n, bad = early_uses_in(body)
                assert n >= 6 and not bad, f"{what} precision {prec}: {n} loads, early uses {bad[:3]}"


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_moe_pipelined_loops_wait_for_every_asm_load(tmp_path):
    """The routed-expert kernels stream through gemv_rows_pipe, whose loads are inline asm
    with explicit waits: in every instance's K loop, each load's registers are touched only
    after a wait that covers it (the loads of the next positions stay in flight)."""
    src = SRC.parent / "moe.hip"
    out = tmp_path / "moe.s"
    cmd = ["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{SRC.parent}", "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text().splitlines()
    kernels = [l.split(":")[0] for l in text if re.match(r"_ZN12_GLOBAL__N_1\w*moe_(up|down)_kernel\w*:", l)]
    assert len(kernels) == 8
    for k in kernels:
        start = next(i for i, l in enumerate(text) if l.startswith(k + ":"))
        stop = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
        checked = 0
        for body in inner_loops(text[start:stop]):
            if sum(1 for l in body if re.match(r"\s*global_load_dwordx4", l)) < 4:
                continue                        # the routing scans: compiler-tracked loads
            n, bad = early_uses_in(body)
            assert not bad, f"{k}: registers used before their load's wait: {bad[:3]}"
            checked += n
        assert checked >= 5, f"{k}: no pipelined K loop found"


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_dense_gemv_stream_loops_wait_for_every_asm_load(tmp_path):
    """The dense GEMV and the SwiGLU pair stream through gemv_rows_stream (inline-asm loads,
    an explicit wait per K position): in every instance's K loop each load's registers are
    touched only after a wait that covers it."""
    src = SRC.parent / "gemv.hip"
    out = tmp_path / "gemv.s"
    cmd = ["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{SRC.parent}", "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=900)
    text = out.read_text().splitlines()
    dense = [l.split(":")[0] for l in text
             if re.match(r"_ZN12_GLOBAL__N_111gemv_kernelILi\dELb\dELi\d+ELb\dELb\dELb1ELb\dEE\w*:", l)]
    # NTL x waves x (f32 / bf16 x, mx0 f32 / bf16 x, norm), + waves x (norm of residual + partials)
    assert len(dense) == 4 * 3 * (2 + 2 + 1) + 3
    swiglu = [l.split(":")[0] for l in text
              if re.match(r"_ZN12_GLOBAL__N_118gemv_swiglu_kernelILi\dELb\dELb\dELi\d+ELb1ELb\dEE\w*:", l)]
    # NTL x waves x (f32 x, bf16 x, norm), + waves x (norm of residual + partials)
    assert len(swiglu) == 4 * 2 * 3 + 2
    kernels = dense + swiglu
    meta = "\n".join(text)
    for k in kernels:
        # a spilled register may be one whose asm load is still in flight
        m = re.search(r"\.name:\s+" + re.escape(k) + r"\n.*?\.vgpr_spill_count:\s+(\d+)", meta, re.S)
        assert m and int(m.group(1)) == 0, f"{k}: {m.group(1) if m else '?'} VGPRs spilled"
        start = next(i for i, l in enumerate(text) if l.startswith(k + ":"))
        stop = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
        checked = 0
        for body in inner_loops(text[start:stop]):
            if sum(1 for l in body if re.match(r"\s*global_load_dwordx4 .* nt$", l)) < 6:
                continue                        # the norm prelude: compiler-tracked loads
            n, bad = early_uses_in(body)
            assert not bad, f"{k}: registers used before their load's wait: {bad[:3]}"
            checked += n
        # the activation-from-LDS instances issue weight loads only
        assert checked >= (8 if "ELb1ELb1EE" in k else 9), f"{k}: no pipelined K loop found"


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_grouped_stream_loops_wait_for_every_asm_load(tmp_path):
    """The grouped GEMV (one launch over many matrices) streams through gemv_rows_stream,
    built with its own per-source flags: every instance's K loop waits before each use."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("q4mi_build", ROOT / "openflowlm-next_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    path = SRC.parent / "gemv_grouped.hip"
    out = tmp_path / "grouped.s"
    subprocess.run(["hipcc", *b.flags(path), "--cuda-device-only", "-S", str(path), "-o", str(out)], check=True,
                   capture_output=True, timeout=600)
    text = out.read_text().splitlines()
    kernels = [l.split(":")[0] for l in text if re.match(r"_ZN12_GLOBAL__N_119gemv_grouped_kernelILi\dELb\dELb1EE\w*:", l)]
    assert len(kernels) == 8                       # NTL x (f32 / bf16 x)
    for k in kernels:
        start = next(i for i, l in enumerate(text) if l.startswith(k + ":"))
        stop = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
        checked = 0
        for body in inner_loops(text[start:stop]):
            if sum(1 for l in body if re.match(r"\s*global_load_dwordx4 .* nt$", l)) < 6:
                continue
            n, bad = early_uses_in(body)
            assert not bad, f"{k}: registers used before their load's wait: {bad[:3]}"
            checked += n
        assert checked >= 24, f"{k}: no pipelined K loop found"


def test_checker_flags_an_early_use():
    """Plant the mistake: a use of the loaded registers before any covering wait."""
    asm = [".LBB0_1: ; Loop Header: Depth=1",
           "\tglobal_load_dwordx4 v[4:7], v1, s[2:3] nt",
           "\tv_add_u32_e32 v12, v5, v6",
           "\ts_waitcnt vmcnt(1)",
           "\ts_cbranch_scc1 .LBB0_1"]
    n, bad = early_uses(asm)
    assert n == 1 and len(bad) == 1 and "v12" in bad[0]
    ok = asm[:2] + ["\tglobal_load_dwordx4 v[8:11], v1, s[2:3] nt", "\ts_waitcnt vmcnt(1)",
                    "\tv_add_u32_e32 v12, v5, v6",
                    "\tglobal_load_dwordx4 v[30:33], v1, s[2:3] nt", "\ts_waitcnt vmcnt(1)",
                    "\tv_add_u32_e32 v13, v9, v10", asm[-1]]
    assert early_uses(ok) == (3, [])


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("src", ["gemv.hip", "gemv_grouped.hip", "moe.hip"])
def test_gemv_kernels_load_global_and_keep_accumulators_in_vgprs(tmp_path, src):
    """The decode kernels' weight and activation loads are global loads in every kernel,
    also where the pointers come from a descriptor table (flat loads count on lgkmcnt too,
    which turns every wait into a wait for all loads); the sources the build compiles with
    VGPR-form MFMA hold no AGPRs (MFMA results read back one VALU per register, and AGPRs
    add to the wave's allocation)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("q4mi_build", ROOT / "openflowlm-next_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    path = SRC.parent / src
    out = tmp_path / (path.stem + ".s")
    cmd = ["hipcc", *b.flags(path), "--cuda-device-only", "-S", str(path), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    lines = text.splitlines()
    kernels = [l.split(":")[0] for l in lines if re.match(r"_ZN12_GLOBAL__N_1\w*(gemv|moe)\w*kernel\w*:", l)]
    assert kernels
    for k in kernels:
        start = next(i for i, l in enumerate(lines) if l.startswith(k + ":"))
        stop = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
        for body in inner_loops(lines[start:stop]):
            flat = [l.strip() for l in body if l.strip().startswith("flat_load")]
            assert not flat, f"{k}: flat loads in its loop: {flat[:2]}"
    if "-amdgpu-mfma-vgpr-form" not in b.flags(path):
        return
    for m in re.finditer(r"\.agpr_count:\s+(\d+).*?\.name:\s+(\S+)", text, re.S):
        if m.group(2) in kernels:
            assert int(m.group(1)) == 0, f"{m.group(2)} holds {m.group(1)} AGPRs"
