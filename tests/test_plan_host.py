"""Every decode shape the C-ABI layer can plan is one the kernels instantiate.

gaudi-kernels_amd/csrc/gk_fp8_plan.h holds the planner and the instantiation
lists the dispatch switches over; tests/csrc/plan_check.cpp runs the planner
over the N tiers, G = 1..256 groups, 1/2/4 token tiles and both weight
layouts (with g++, no GPU) and checks each result against its list.  A shape
missing there would make the GEMM entry points return GK_DEVICE_ERROR for a
plan gk_fp8_block_gemm_plan reports as valid.  The same program checks that
the dense 256 x 256 kernel's XCD-aware tile order (dense_tile_of) visits every
tile of every grid up to 64 x 96 tiles exactly once.
"""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "_build")


def test_every_planned_decode_shape_is_instantiated():
    os.makedirs(BUILD, exist_ok=True)
    exe = os.path.join(BUILD, "plan_check")
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "gaudi-kernels_amd", "csrc"),
                    os.path.join(ROOT, "tests", "csrc", "plan_check.cpp"), "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout[-4000:]
    assert "0 missing" in res.stdout
    assert "0 not bijective" in res.stdout
