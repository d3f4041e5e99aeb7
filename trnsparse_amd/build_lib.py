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


def build(verbose: bool = False, jobs: int | None = None) -> pathlib.Path:
    """Compile every `csrc/*.hip` and link the shared library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
