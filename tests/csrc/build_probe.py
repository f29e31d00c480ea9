"""Build tests/csrc/libgk_probe.so: measurement and check kernels used by bench.py and the GPU tests.

Not part of the block-FP8 library (gaudi-kernels_amd/build.py builds only libgk_fp8.so, the drop-in):
* gk_probe_stream_read -- a plain streaming read, bench.py's HBM ceiling at the decode footprints;
* gk_probe_bf16x2_check / gk_probe_e4m3_check -- exhaustive GPU checks of the hardware bf16 rounding and E4M3
  encode the library's kernels rely on (tests/test_gpu_hw_convert.py).

Compiled with the library's own hipcc flags and its internal headers, so the checks run the kernels' code.

    python tests/csrc/build_probe.py
"""

import os
import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
SRC = HERE / "gk_probe.hip"
HEADER = HERE / "gk_probe.h"
LIB = HERE / "libgk_probe.so"
EXPORTS = ["gk_probe_bf16x2_check", "gk_probe_e4m3_check", "gk_probe_stream_read"]


def build(verbose=True):
    sys.path.insert(0, str(ROOT / "gaudi-kernels_amd"))
    import build as gk_build  # gaudi-kernels_amd/build.py: the same compiler and flags as the library
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [gk_build.hipcc(), *gk_build.HIPCC_FLAGS, "-shared", "-Wl,-z,defs", "-I", str(gk_build.CSRC), str(SRC),
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC.name}:\n{res.stderr}")
    os.replace(tmp, LIB)
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], check=True, capture_output=True, text=True).stdout
    have = sorted({l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("gk_")})
    declared = sorted(set(re.findall(r"^\s*int\s+(gk_\w+)\s*\(", HEADER.read_text(), re.MULTILINE)))
    if have != declared or have != EXPORTS:
        raise RuntimeError(f"probe exports {have}, header declares {declared}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
