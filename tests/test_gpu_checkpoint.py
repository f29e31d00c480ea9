"""Checkpoint load path on the GPU: safetensors block-FP8 weights -> device, bit-exact, codec options."""

import pytest
import torch
from safetensors.torch import save_file

from gaudi_kernels import checkpoint as ck
from gaudi_kernels import ops
from oracle import block_fp8, fp8_codec, synth

pytestmark = pytest.mark.gpu

SHAPES = {"layer0.q_proj.weight": (256, 256), "layer0.down.weight": (300, 384), "layer1.up.weight": (128, 4096)}


def make_checkpoint(path, dmax=448.0):
    tensors = {}
    for i, (name, (n, k)) in enumerate(SHAPES.items()):
        w, s = synth.weight(n, k, seed=50 + i, dmax=dmax)
        tensors[name] = w
        tensors[name + "_scale_inv"] = s
    tensors["layer0.down.bias"] = torch.randn(300).bfloat16()
    tensors["step"] = torch.tensor([7], dtype=torch.int64)
    save_file(tensors, str(path))
    return tensors


def test_load_bit_exact_and_gemm(tmp_path):
    ref = make_checkpoint(tmp_path / "m.safetensors")
    weights, tensors = ck.load_block_fp8(tmp_path / "m.safetensors")
    assert set(weights) == set(SHAPES) and set(tensors) == {"layer0.down.bias", "step"}
    for name, bw in weights.items():
        assert bw.codes.is_cuda and bw.codes.dtype == torch.float8_e4m3fn and not bw.half_range
        assert torch.equal(bw.codes.cpu().view(torch.uint8), ref[name].view(torch.uint8))
        assert torch.equal(bw.scales.cpu(), ref[name + "_scale_inv"])
    assert torch.equal(tensors["layer0.down.bias"].cpu(), ref["layer0.down.bias"])
    x = synth.activations(5, 384, seed=3)
    bw = weights["layer0.down.weight"]
    y = ops.block_fp8_gemm(x.cuda(), bw.codes, bw.scales).cpu()
    want = block_fp8.reference(x, ref["layer0.down.weight"], ref["layer0.down.weight_scale_inv"])
    max_rel, mean_rel = block_fp8.parity(y, want)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL


def test_subset_and_half_range_round_trip(tmp_path):
    ref = make_checkpoint(tmp_path / "m.safetensors")
    weights, tensors = ck.load_block_fp8(tmp_path / "m.safetensors", names=["layer1.up.weight"], to_half_range=True)
    assert list(weights) == ["layer1.up.weight"] and not tensors
    bw = weights["layer1.up.weight"]
    want_codes, want_scales, want_rounded = fp8_codec.reencode_e4m3fn_half(
        ref["layer1.up.weight"].view(torch.uint8).numpy(), ref["layer1.up.weight_scale_inv"].numpy())
    assert bw.half_range and bw.rounded == want_rounded
    assert (bw.codes.cpu().view(torch.uint8).numpy() == want_codes).all()
    assert (bw.scales.cpu().numpy() == want_scales).all()
    # a half-range checkpoint loads back to OCP codes with the inverse codec
    half = {"layer1.up.weight": bw.codes.cpu(), "layer1.up.weight_scale_inv": bw.scales.cpu()}
    save_file(half, str(tmp_path / "h.safetensors"))
    back, _ = ck.load_block_fp8(tmp_path / "h.safetensors", from_half_range=True)
    inv_codes, inv_scales = fp8_codec.decode_half_to_ocp(want_codes, want_scales)
    assert (back["layer1.up.weight"].codes.cpu().view(torch.uint8).numpy() == inv_codes).all()
    assert (back["layer1.up.weight"].scales.cpu().numpy() == inv_scales).all()


def test_rejections(tmp_path):
    w, s = synth.weight(128, 256, seed=1)
    bad = w.view(torch.uint8).clone()
    bad[3, 5] = 0x7F                                   # OCP NaN code
    save_file({"a.weight": bad.view(torch.float8_e4m3fn), "a.weight_scale_inv": s}, str(tmp_path / "nan.safetensors"))
    with pytest.raises(ValueError, match="NaN code"):
        ck.load_block_fp8(tmp_path / "nan.safetensors")
    save_file({"a.weight": w, "a.weight_scale_inv": torch.ones(2, 2)}, str(tmp_path / "grid.safetensors"))
    with pytest.raises(ValueError, match="scale grid mismatch"):
        ck.load_block_fp8(tmp_path / "grid.safetensors")
    neg = s.clone()
    neg[0, 1] = -1.0
    save_file({"a.weight": w, "a.weight_scale_inv": neg}, str(tmp_path / "neg.safetensors"))
    with pytest.raises(ValueError, match="nonfinite/negative scale"):
        ck.load_block_fp8(tmp_path / "neg.safetensors")
