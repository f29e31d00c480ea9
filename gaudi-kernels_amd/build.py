"""Build libgk_fp8.so for gfx950 and verify its exported C ABI.

The reference builds a Synapse provider by compiling TPC kernels with
tpc-clang, checking each ELF's entry-point ABI against a contract table,
embedding the ELFs and linking one shared object
(tools/build_generic_dense_bundle.py:29-147).  Here the kernels are HIP
sources compiled by hipcc for gfx950 into one shared object, and the check is
that the object exports exactly the functions include/gk_fp8.h declares.

    python gaudi-kernels_amd/build.py [--jobs N] [--debug]
"""

import argparse
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HEADER = ROOT / "include" / "gk_fp8.h"
OUT_DIR = PKG / "python" / "gaudi_kernels"
LIB = OUT_DIR / "libgk_fp8.so"
OBJ_DIR = PKG / "_build"
SOURCES = ["gk_fp8_codec.hip", "gk_fp8_gemm.hip", "gk_fp8_prefill.hip", "gk_fp8_moe.hip", "gk_fp8_act.hip",
           "gk_fp8_token.hip", "gk_fp8_norm.hip", "gk_fp8_reduce.hip", "gk_fp8_abi.hip"]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Wall", "-Wno-unused-function",
    # Packed FP32 (v_pk_*_f32) forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found")
    return path


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:gk_status|uint64_t)\s+(gk_\w+)\s*\(", text, re.MULTILINE)))


def exported_symbols(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], check=True, capture_output=True, text=True).stdout
    return sorted({line.split()[-1] for line in out.splitlines() if " T " in line and line.split()[-1].startswith("gk_")})


def verify_abi(lib=LIB):
    want, have = declared_symbols(), exported_symbols(lib)
    if want != have:
        missing = sorted(set(want) - set(have))
        extra = sorted(set(have) - set(want))
        raise RuntimeError(f"ABI mismatch: missing {missing}, undeclared exports {extra}")
    return want


def compile_one(src, debug):
    obj = OBJ_DIR / (Path(src).stem + ".o")
    flags = list(HIPCC_FLAGS)
    if debug:
        flags += ["-g"]
    cmd = [hipcc(), *flags, "-I", str(ROOT / "include"), "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    warn = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and "warning" in l]
    return obj, warn


def build(jobs=4, debug=False, verbose=True):
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: compile_one(s, debug), SOURCES))
    for _, warn in results:
        for w in warn:
            print(w, file=sys.stderr)
    objs = [str(o) for o, _ in results]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs",
           "-Wl,--exclude-libs,ALL", *objs, "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    syms = verify_abi(LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size} bytes), {len(syms)} exported entry points")
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--debug", action="store_true")
    args = ap.parse_args()
    build(args.jobs, args.debug)


if __name__ == "__main__":
    main()
