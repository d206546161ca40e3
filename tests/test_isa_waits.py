"""The pipelined prefill kernel issues its global loads from inline asm, so the
compiler does not wait for them: every wait is explicit. This checks the gfx950
ISA of that kernel's main loop: each register-destination load's registers are
touched only after an s_waitcnt vmcnt(N) with N no larger than the number of
vector-memory loads issued after it (vector-memory loads retire in issue order).
A compiler change that schedules a use ahead of its wait would fail here. The
same checker gates the build (openflowlm-next_amd/build.py): a planted violation
below makes build() fail. Needs hipcc (present on the build host); no GPU."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "openflowlm-next_amd" / "csrc" / "prefill.hip"


def _load(name: str, path: Path):
    import importlib.util
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# the checker is the build's own gate (openflowlm-next_amd/isa_gate.py); these tests hold it
# to the kernels' known structure and plant mistakes for it to find
G = _load("q4mi_isa_gate", ROOT / "openflowlm-next_amd" / "isa_gate.py")
inner_loops, early_uses_in, early_uses = G.inner_loops, G.early_uses_in, G.early_uses


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
        # the grouped expert GEMM's tile loop (pre-tiled activations, and the rows gathered
        # through the slot map) and the gate/up GEMMs with the SwiGLU epilogue
        for kname, what in ((rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb0ELb0EE", "moe"),
                            (rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb1ELb0EE", "moe swiglu"),
                            (rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb0ELb1EE", "moe gathered"),
                            (rf"_ZN12_GLOBAL__N_114moe_dma_kernelILi{prec}ELb1ELb1EE", "moe swiglu gathered"),
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
def test_decode_segment_waits_spills_and_hand_over(tmp_path):
    """The decode segment's weight loads are primed before a grid hand-over and consumed after
    it: along every control-flow path from each asm load (the prime, the polls, the norm
    prelude, the rolling K loops) its registers are touched only after a covering wait, no
    instance spills, and the hand-over uses no cache-wide fence (buffer_wbl2 / buffer_inv):
    the values crossing workgroups are device-scope stores and the arrivals device-scope
    atomics."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("q4mi_isa_gate", ROOT / "openflowlm-next_amd" / "isa_gate.py")
    gate = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gate)
    src = SRC.parent / "decode.hip"
    out = tmp_path / "decode.s"
    cmd = ["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{SRC.parent}", "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    n, problems = gate.check_assembly(text, straight=True)
    assert n > 0 and not problems, problems[:3]
    kernels = re.findall(r"\.name:\s+(_ZN12_GLOBAL__N_121decode_segment_kernel\w+)", text)
    assert len(kernels) == 8
    assert set(re.findall(r"\.vgpr_spill_count:\s+(\d+)", text)) == {"0"}
    assert "buffer_wbl2" not in text and "buffer_inv" not in text
    assert re.search(r"global_atomic_add\b", text) and re.search(r"global_store_dword\w* .* sc1", text)


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
             if re.match(r"_ZN12_GLOBAL__N_111gemv_kernelILi\dELb\dELi\d+ELb\dELb\dELb1ELb\dELb\dEE\w*:", l)]
    # NTL x waves x (f32 / bf16 x, mx0 f32 / bf16 x, norm, fp16-scale f32 / bf16 x),
    # + waves x (norm of residual + partials)
    assert len(dense) == 4 * 3 * (2 + 2 + 1 + 2) + 3
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
        # the activation-from-LDS (XN) instances: second-to-last template argument of gemv_kernel
        # (gemv_swiglu_kernel: the last), set
        xn = re.search(r"ELb1ELb\dEEEvNS_10GemvParamsE", k) if "gemv_kernel" in k else "ELb1ELb1EE" in k
        assert checked >= (8 if xn else 9), f"{k}: no pipelined K loop found"


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
    kernels = [l.split(":")[0] for l in text
               if re.match(r"_ZN12_GLOBAL__N_119gemv_grouped_kernelILi\dELb\dELb1ELb\dEE\w*:", l)]
    assert len(kernels) == 16                      # NTL x (f32 / bf16 x) x (bf16 / fp16 scale words)
    # the shared-fragment form (M >= 2, bf16 x): NTL 1, 2 over 2 row groups, 3, 4 over 4
    shared = [l.split(":")[0] for l in text
              if re.match(r"_ZN12_GLOBAL__N_122gemv_grouped_ng_kernelILi\dELb0ELi[24]ELi[24]EE\w*:", l)]
    assert len(shared) == 4
    for k in kernels + shared:
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
    # an LDS-DMA buffer load counts as a younger load in vmcnt like a global one
    dma = asm[:2] + ["\tbuffer_load_dwordx4 v2, s[8:11], s4 offen lds", "\ts_waitcnt vmcnt(1)",
                     "\tv_add_u32_e32 v12, v5, v6", asm[-1]]
    assert early_uses(dma) == (1, [])


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


PLANTED = r"""
#include <hip/hip_runtime.h>
#include <stdint.h>
// A two-deep pipeline of inline-asm loads over p[0 .. n + 1] (compiled only, never run).
__global__ void planted(const uint32_t* __restrict__ p, uint32_t* __restrict__ out, int n) {
    uint32_t a0, a1, acc = 0;
    const uint32_t off = threadIdx.x * 4u;
    asm volatile("global_load_dword %0, %1, %2" : "=v"(a0) : "v"(off), "s"(p) : "memory");
    asm volatile("global_load_dword %0, %1, %2 offset:4" : "=v"(a1) : "v"(off), "s"(p) : "memory");
    for (int i = 0; i < n; i += 2) {
        const uint32_t nx = off + (uint32_t)(i + 2) * 4u;
#ifndef EARLY
        asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
#endif
        asm volatile("" : "+v"(a0));
        acc += a0 * 3u;
        asm volatile("global_load_dword %0, %1, %2" : "=v"(a0) : "v"(nx), "s"(p) : "memory");
        asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
        asm volatile("" : "+v"(a1));
        acc ^= a1;
        asm volatile("global_load_dword %0, %1, %2 offset:4" : "=v"(a1) : "v"(nx), "s"(p) : "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("" : "+v"(a0), "+v"(a1));
    out[threadIdx.x] = acc + a0 + a1;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("early", [False, True])
def test_build_fails_on_a_planted_early_use(tmp_path, early):
    """build() over a source whose loop reads an asm load's register before the wait that
    covers it raises IsaGateError and leaves no library; the same source with the wait in
    place builds."""
    b = _load("q4mi_build_gate", ROOT / "openflowlm-next_amd" / "build.py")
    csrc = tmp_path / "csrc"
    csrc.mkdir()
    (csrc / "planted.hip").write_text(("#define EARLY 1\n" if early else "") + PLANTED)
    lib = tmp_path / "libplanted.so"
    if early:
        with pytest.raises(b.IsaGateError, match="touched before their wait"):
            b.build(jobs=2, csrc=csrc, lib=lib, build_dir=tmp_path / "_build")
        assert not lib.exists()
    else:
        assert b.build(jobs=2, csrc=csrc, lib=lib, build_dir=tmp_path / "_build") == lib and lib.exists()
        assert b.check_isa([csrc / "planted.hip"], tmp_path / "_build2", 1) >= 2   # both loads checked


def test_gate_flags_agpr_parking_and_spills():
    """The two forms the GPU faults took: an in-flight load's register parked in an AGPR
    before its wait, and a kernel with asm loads that spills VGPRs."""
    def kernel(body, spill):
        return "\n".join([
            "k:", "\ts_load_dwordx2 s[2:3], s[0:1], 0x0",
            ".LBB0_1: ; %loop", "\t; Loop Header: Depth=1",
            *body,
            "\ts_cbranch_scc1 .LBB0_1", "\ts_endpgm", ".Lfunc_end0:",
            "amdhsa.kernels:", "  - .agpr_count: 4", "    .name:           k",
            f"    .vgpr_spill_count: {spill}", "    .wavefront_size: 64"])
    load = lambda regs: ["\t;;#ASMSTART", f"\tglobal_load_dwordx4 {regs}, v1, s[2:3] nt", "\t;;#ASMEND"]
    # two loads in flight: each register set is read after a wait that leaves only the other
    good = ["\ts_waitcnt vmcnt(1)", "\tv_add_u32_e32 v12, v5, v6", *load("v[4:7]"),
            "\ts_waitcnt vmcnt(1)", "\tv_add_u32_e32 v13, v9, v10", *load("v[8:11]")]
    assert G.check_assembly(kernel(good, 0)) == (2, [])
    parked = good[:2] + load("v[4:7]") + ["\tv_accvgpr_write_b32 a0, v5"] + good[5:]
    n, problems = G.check_assembly(kernel(parked, 0))
    assert n == 2 and len(problems) == 1 and "v_accvgpr_write_b32 a0, v5" in problems[0]
    n, problems = G.check_assembly(kernel(good, 3))
    assert problems == ["k: 3 VGPRs spilled in a kernel with in-flight asm loads"]


def test_gate_follows_prologue_loads_on_every_path():
    """A load issued ahead of straight-line work (a prologue, or a prelude the pipeline's
    first loads overlap) is followed along both sides of a branch: a use on either side
    before a covering wait is reported; waits on both sides pass."""
    def kernel(left, right):
        return "\n".join([
            "k:", "\ts_load_dwordx2 s[2:3], s[0:1], 0x0",
            "\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v1, s[2:3]", "\t;;#ASMEND",
            "\ts_cbranch_scc1 .LBB0_2",
            *left, "\ts_branch .LBB0_3",
            ".LBB0_2:", *right,
            ".LBB0_3:", "\tv_add_u32_e32 v13, v5, v6", "\ts_endpgm", ".Lfunc_end0:",
            "amdhsa.kernels:", "  - .name:           k", "    .vgpr_spill_count: 0"])
    ok = ["\ts_waitcnt vmcnt(0)", "\tv_mov_b32_e32 v20, v0"]
    assert G.check_assembly(kernel(ok, ok)) == (1, [])
    n, problems = G.check_assembly(kernel(ok, ["\tv_accvgpr_write_b32 a0, v5", *ok]))
    assert n == 1 and len(problems) == 1 and "v_accvgpr_write_b32 a0, v5" in problems[0]
    n, problems = G.check_assembly(kernel(["\tv_mov_b32_e32 v20, v0"], ok))   # one side never waits
    assert len(problems) == 1 and "v_add_u32_e32 v13, v5, v6" in problems[0]
    assert G.check_assembly(kernel(["\tv_mov_b32_e32 v20, v0"], ok), straight=False) == (0, [])
