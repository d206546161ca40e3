"""Build libq4mi.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python openflowlm-next_amd/build.py [--jobs N] [--verbose]

Every csrc/*.hip is compiled for --offload-arch=gfx950 to an object under
_build/, then linked into libq4mi.so next to this file. hipcc cross-compiles
without a GPU. All device code is built with packed FP32 ops disabled
(``-target-feature -packed-fp32-ops``); hipcc's host pass warns that it does
not know that feature, which is harmless.

The sources whose kernels issue loads from inline asm (isa_gate.GATED) are also
compiled to device assembly with the same flags, and the build fails when any
kernel touches an in-flight asm load's registers before its wait or spills
VGPRs (isa_gate.check_assembly); the library is then not replaced.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libq4mi.so"
ARCH = os.environ.get("Q4MI_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{REPO / 'include'}", f"-I{CSRC}",
]


# Per-source flags. The grouped GEMV keeps its MFMA accumulators in VGPRs: in the AGPR
# form the compiler reads every MFMA result back with v_accvgpr_read (one VALU per result
# register, 20 per 4 tiles at M = 1) and the AGPRs add to the wave's register allocation
# (the files are unified; 102 VGPRs + 20 AGPRs at M = 1 against 89 VGPRs). Measured on the
# Llama-3-8B sweep (8 layers, M = 1): 197.1 -> 193.6 us. The same flag made the
# single-matrix kernels of gemv.hip slower (native Q4_K gate_up 14.9 -> 21.0 us, the mx
# lm_head 55.7 -> 58.6 us) and changes the prefill kernel's hand-scheduled loop, so it is
# set per source file.
EXTRA = {
    "gemv_grouped.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the MFMA probe's accumulators in AGPRs get shuffled through VGPRs every iteration
    "peaks.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def flags(src: Path) -> list[str]:
    """The device-compile flags of one csrc/*.hip file."""
    return [*COMMON, *EXTRA.get(src.name, [])]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: Path, verbose: bool, build_dir: Path = BUILD) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *flags(src), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


class IsaGateError(RuntimeError):
    """The device assembly breaks the inline-asm load discipline (isa_gate)."""


def _isa_gate():
    import importlib.util
    spec = importlib.util.spec_from_file_location("q4mi_isa_gate", HERE / "isa_gate.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _assemble_and_check(src: Path, out_dir: Path, verbose: bool) -> tuple[int, list[str]]:
    """Compile src's device code to assembly (the build's flags) and run the ISA gate on it."""
    asm = out_dir / (src.stem + ".s")
    cmd = [hipcc(), *flags(src), "--cuda-device-only", "-S", str(src), "-o", str(asm)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    gate = _isa_gate()
    return gate.check_assembly(asm.read_text(), straight=src.name in gate.STRAIGHT or src.name not in gate.GATED)


def check_isa(srcs, out_dir: Path = BUILD, jobs: int = 8, verbose: bool = False) -> int:
    """Run the ISA gate over srcs; raises IsaGateError listing every problem, else returns
    the number of asm loads checked inside loops."""
    out_dir.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        res = list(ex.map(lambda s: (s, _assemble_and_check(s, out_dir, verbose)), srcs))
    problems = [f"{s.name}: {p}" for s, (_, ps) in res for p in ps]
    if problems:
        raise IsaGateError("in-flight asm loads mishandled:\n  " + "\n  ".join(problems[:20]))
    return sum(n for _, (n, _) in res)


def build(jobs: int = 8, verbose: bool = False, csrc: Path = CSRC, lib: Path | None = None,
          build_dir: Path | None = None) -> Path:
    """Compile every .hip under csrc, gate the assembly of the asm-load sources, and link
    the library (libq4mi.so next to this file by default); returns its path."""
    lib = LIB if lib is None else lib
    build_dir = BUILD if build_dir is None else build_dir
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted(csrc.glob("*.hip"))
    gated = [s for s in srcs if s.name in _isa_gate().GATED] if csrc == CSRC else srcs
    with cf.ThreadPoolExecutor(max_workers=2) as outer:
        gate = outer.submit(check_isa, gated, build_dir, max(1, jobs // 2), verbose)
        with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            objs = list(ex.map(lambda s: _compile(s, verbose, build_dir), srcs))
        gate.result()          # raises IsaGateError before the library is replaced
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    return lib


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
