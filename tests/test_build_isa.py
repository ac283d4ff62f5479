"""The prefill kernels' LDS-DMA statements write M0 from inline assembly.

The AMDGPU backend treats M0 as a reserved register, so a clobber of it in an asm
statement is advisory: if the compiler kept a value of its own live in M0 across
those statements, the value would be overwritten. This test compiles
csrc/prefill.hip for gfx950 to assembly (CPU only, about half a minute) and checks
that no instruction outside the inline-asm blocks reads or writes M0 -- so the
statements' writes cannot clobber anything -- and that the DMA statements are
there (the check is not vacuous).
"""

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "wisp-runtime_amd", "csrc", "prefill.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _device_asm(src: str) -> str:
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "k.s")
        cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
               "-o", out, src]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        with open(out) as f:
            return f.read()


@pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")), reason="hipcc not installed")
def test_m0_written_only_by_the_dma_statements():
    asm = _device_asm(SRC)
    inside, dma, outside_m0 = False, 0, []
    m0 = re.compile(r"\bm0\b")
    for n, line in enumerate(asm.splitlines(), 1):
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            inside = True
            continue
        if s.startswith(";;#ASMEND"):
            inside = False
            continue
        code = s.split(";", 1)[0]
        if inside:
            dma += "global_load_lds_dword" in code
        elif m0.search(code):
            outside_m0.append((n, s))
    assert dma > 0, "no LDS-DMA statement found in the prefill kernels"
    assert not outside_m0, f"compiler-emitted M0 uses beside the DMA statements: {outside_m0[:5]}"
