"""Build `libtrnsparse_hip.so` for gfx950 in-tree with hipcc.

The library is the C ABI declared in `include/trnsparse_hip.h`; the Python
layer (`trnsparse_amd.hip._lib`) loads it with ctypes. Objects go to
`trnsparse_amd/_build/`, the shared library next to this file so that it
travels with the source tree.

Usage: python -m trnsparse_amd.build_lib [-v]
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtrnsparse_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: packed fp32 VALU forms stay out of the generated code.
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


# Per-source extra flags. attention_bwd.hip: MFMA results in VGPRs (the
# softmax-gradient VALU reads the S / dP tiles straight from the MFMA
# destination; the default AGPR form costs a register move per element).
EXTRA = {"attention_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


# The direct-to-LDS load helpers (csrc/lds_dma.h) set M0 inside inline asm,
# which the compiler does not track (M0 is a reserved register: its clobber
# is ignored). That is only safe while no instruction the compiler generates
# for those kernels keeps a value in M0, so every build emits their gfx950
# assembly and fails if an instruction outside the asm blocks names m0.
# (The compiler's own LDS-load builtins track M0 but also make it wait for
# every outstanding load before each LDS read: measured +31 % on the bf16
# BSR kernel at cfg3b.)
DMA_HEADER = "lds_dma.h"


def m0_uses_outside_asm(asm_text: str) -> list[str]:
    """Instructions outside ;;#ASMSTART / ;;#ASMEND that read or write M0."""
    import re

    bad, in_asm = [], False
    for line in asm_text.splitlines():
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if in_asm or not t or t.startswith((";", ".", "//")) or t.endswith(":"):
            continue
        code = t.split(";", 1)[0]
        if re.search(r"\bm0\b", code):
            bad.append(t)
    return bad


def _check_m0(src: pathlib.Path, verbose: bool) -> None:
    asm = BUILD / (src.stem + ".s")
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(src.name, []), "--cuda-device-only", "-S", str(src), "-o", str(asm)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{r.stdout}{r.stderr}")
    bad = m0_uses_outside_asm(asm.read_text())
    if bad:
        raise RuntimeError(f"{src.name}: compiler-generated code uses M0, which the inline-asm LDS loads of "
                           f"{DMA_HEADER} overwrite:\n" + "\n".join(bad[:10]))


def _compile(src: pathlib.Path, verbose: bool) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    msg = "\n".join(ln for ln in (r.stdout + r.stderr).splitlines() if noise not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    if verbose and msg.strip():
        print(msg, flush=True)
    return obj


# The PyTorch operator library (csrc/torch_ops.cpp, torch.ops.trnsparse_hip):
# host code only, compiled against torch's headers and linked to
# libtrnsparse_hip.so (found next to it through $ORIGIN).
OPS_SRC = CSRC / "torch_ops.cpp"
OPS_LIB = PKG / "libtrnsparse_torch_ops.so"


def build_ops(verbose: bool = False) -> pathlib.Path:
    """Compile and link the operator library (needs libtrnsparse_hip.so built)."""
    import torch
    import torch.utils.cpp_extension as ce

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_LIB.with_suffix(".so.tmp")
    tlib = ce.library_paths()[0]
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", *(f"-I{p}" for p in ce.include_paths()), "-I/opt/rocm/include",
           f"-I{ROOT / 'include'}", str(OPS_SRC), "-o", str(tmp), f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", f"-L{PKG}", "-ltrnsparse_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"operator library build failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


# The benchmark's shader-clock probe (csrc/probe/shader_clock.hip): a library
# of its own, outside the C ABI, loaded only by bench.py.
CLOCK_SRC = CSRC / "probe" / "shader_clock.hip"
CLOCK_LIB = PKG / "libtrnsparse_clock.so"


def build_clock(verbose: bool = False) -> pathlib.Path:
    tmp = CLOCK_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *CFLAGS, "-shared", str(CLOCK_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {CLOCK_SRC.name}:\n{r.stdout}{r.stderr}")
    os.replace(tmp, CLOCK_LIB)
    return CLOCK_LIB


def build(verbose: bool = False, jobs: int | None = None) -> pathlib.Path:
    """Compile every `csrc/*.hip`, link the shared library, then build the
    operator library over it and the benchmark's clock probe. Always
    rebuilds."""
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    dma = [s for s in srcs if DMA_HEADER in s.read_text()]
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        checks = [ex.submit(_check_m0, s, verbose) for s in dma]
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
        for c in checks:
            c.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    build_ops(verbose)
    build_clock(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
