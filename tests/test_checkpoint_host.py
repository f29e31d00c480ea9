"""Host logic of the checkpoint load path (gaudi_kernels.checkpoint): weight/scale pairing and grid checks."""

import pytest
import torch

from gaudi_kernels import checkpoint as ck


def test_pairing():
    f8, f32, bf = torch.float8_e4m3fn, torch.float32, torch.bfloat16
    keys = ["l0.weight", "l0.weight_scale_inv", "l0.bias", "l1.weight", "l1.weight_scale_inv", "norm.weight",
            "steps"]
    dtypes = {"l0.weight": f8, "l0.weight_scale_inv": f32, "l0.bias": bf, "l1.weight": f8,
              "l1.weight_scale_inv": f32, "norm.weight": bf, "steps": torch.int64}
    pairs, others = ck.pair_block_fp8(keys, dtypes)
    assert pairs == {"l0.weight": "l0.weight_scale_inv", "l1.weight": "l1.weight_scale_inv"}
    assert others == ["l0.bias", "norm.weight", "steps"]


def test_pairing_errors():
    f8, f32 = torch.float8_e4m3fn, torch.float32
    with pytest.raises(ValueError, match="without its block-scale grid"):
        ck.pair_block_fp8(["a.weight"], {"a.weight": f8})
    with pytest.raises(ValueError, match="without an E4M3FN weight"):
        ck.pair_block_fp8(["a.weight_scale_inv"], {"a.weight_scale_inv": f32})
    with pytest.raises(ValueError, match="without an E4M3FN weight"):
        ck.pair_block_fp8(["a.weight", "a.weight_scale_inv"], {"a.weight": torch.bfloat16, "a.weight_scale_inv": f32})


def test_grid_check():
    w = torch.zeros(300, 384, dtype=torch.float8_e4m3fn)
    ck._check_grid("w", w, torch.ones(3, 3))
    for bad in (torch.ones(2, 3), torch.ones(3, 4), torch.ones(3, 3, dtype=torch.float64)):
        with pytest.raises(ValueError, match="scale grid mismatch"):
            ck._check_grid("w", w, bad)


def test_safetensors_dtype_names():
    assert ck._st_dtype("F8_E4M3") == torch.float8_e4m3fn and ck._st_dtype("F32") == torch.float32
