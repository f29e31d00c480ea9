"""Load the golden vectors written by tests/golden/make_golden.py."""

import json
import os

import numpy as np
import torch

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_vectors.json")


def _arr(hexstr, dtype, shape):
    return np.frombuffer(bytes.fromhex(hexstr), dtype=dtype).reshape(shape).copy()


def load_cases():
    with open(PATH) as f:
        data = json.load(f)
    cases = []
    for c in data["cases"]:
        m, n, k = c["m"], c["n"], c["k"]
        g, nb = (k + 127) // 128, (n + 127) // 128
        case = {
            "name": c["name"], "m": m, "n": n, "k": k,
            "x": torch.from_numpy(_arr(c["x_bf16"], np.int16, (m, k))).view(torch.bfloat16),
            "w": torch.from_numpy(_arr(c["w_e4m3"], np.uint8, (n, k))).view(torch.float8_e4m3fn),
            "scales": torch.from_numpy(_arr(c["scales_f32"], np.float32, (nb, g))),
            "bias": torch.from_numpy(_arr(c["bias_f32"], np.float32, (n,))) if c["bias_f32"] else None,
            "y": torch.from_numpy(_arr(c["y_bf16"], np.int16, (m, n))).view(torch.bfloat16),
            "y_half": torch.from_numpy(_arr(c["y_bf16_native_half"], np.int16, (m, n))).view(torch.bfloat16),
        }
        cases.append(case)
    return data, cases
