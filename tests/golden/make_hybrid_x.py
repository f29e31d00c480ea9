"""Writes tests/golden/hybrid_gemm_x.npz: the activations of the reference's five GEMM cases.

Compiles hybrid_x.cpp (this directory) with g++ into a temporary directory and runs it per case;
the weights, scales and bias of those cases are closed-form and rebuilt by the tests.
Run from the repository root: python tests/golden/make_hybrid_x.py
"""

import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# (m, n, k, bias, tiny, chunk_groups) -- tests/fp8_hybrid_tpcsim_test.cpp:388-392
CASES = [(4, 256, 7168, 0, 0, 0), (4, 256, 7168, 0, 0, 28), (37, 256, 384, 1, 0, 0), (2, 128, 22016, 0, 0, 86),
         (4, 128, 256, 0, 1, 0)]


def main():
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "hybrid_x")
        subprocess.run(["g++", "-O2", "-std=c++17", "-o", exe, os.path.join(HERE, "hybrid_x.cpp")], check=True)
        out = {}
        for idx, (m, n, k, bias, tiny, _) in enumerate(CASES):
            raw = subprocess.run([exe, str(m), str(n), str(k), str(bias), str(tiny)], check=True,
                                 capture_output=True).stdout
            out[f"x{idx}"] = np.frombuffer(raw, dtype="<u2").reshape(m, k)
        out["cases"] = np.array(CASES, dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "hybrid_gemm_x.npz"), **out)


if __name__ == "__main__":
    main()
