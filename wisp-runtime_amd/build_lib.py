"""Build libwisp_hip.so (gfx950) from csrc/*.hip with hipcc, in-tree.

Usage: python wisp-runtime_amd/build_lib.py [--verbose]
The library lands in wisp-runtime_amd/lib/libwisp_hip.so; the Python package
(wisp-runtime_amd/wisp/_lib.py) loads it from there.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "lib", "obj")
LIB = os.path.join(LIBDIR, "libwisp_hip.so")
SOURCES = ["abi.hip", "quant_kernels.hip", "moe_decode.hip", "rope.hip", "cache.hip", "attention.hip", "prefill.hip", "gptoss.hip", "decode_layer.hip", "probe.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# kernarg preloading: the decode kernels' leading scalar arguments arrive in
# SGPRs at dispatch instead of through a memory read at the kernel's start
EXTRA = {"moe_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines() if "is not a recognized feature for this target" not in line
    )
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{msg}")
    if verbose and msg.strip():
        print(msg)
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link the shared library. Always rebuilds."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    shutil.rmtree(OBJDIR, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
