"""Safetensors loading of one MoE block and the offline fp8 converter (CPU).

The loader follows the reference's naming (loader.py:16-61, qwen3_5.py:1052); the converter's
codes and scales must be the oracle's block quantisation bit for bit, which is also what the
GPU's quantize_fp8_ computes (tests/test_gpu_fp8.py::test_quantize_blocks_bit_exact).
"""
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from layerbatch_amd import checkpoint as ck
from layerbatch_amd.moe import Qwen3_5SparseMoeBlock
from layerbatch_amd.synth import MoEShape, make_layer
from oracle import moe as om

SHAPE = MoEShape(256, 4, 2, 128, 128)
LAYER = 3


def _block(shape):
    return Qwen3_5SparseMoeBlock(shape.hidden_size, shape.num_experts, shape.top_k,
                                 shape.moe_intermediate_size,
                                 shape.shared_expert_intermediate_size).to(torch.bfloat16)


def _write_checkpoint(path, w, other_layer_w):
    """Two files: layer LAYER's MoE block split across them, plus tensors that must not load."""
    p = "model." + ck.mlp_prefix(LAYER)
    q = "model." + ck.mlp_prefix(LAYER - 1)
    a = {p + "gate.weight": w["gate"], p + "experts.gate_up_proj": w["gate_up"],
         p + "shared_expert_gate.weight": w["sh_gate_w"],
         q + "experts.gate_up_proj": other_layer_w["gate_up"],
         "model.language_model.layers.3.input_layernorm.weight": torch.ones(256, dtype=torch.bfloat16),
         "mtp.fc.weight": torch.zeros(8, 8, dtype=torch.bfloat16)}
    b = {p + "experts.down_proj": w["down"], p + "shared_expert.gate_proj.weight": w["sh_gate"],
         p + "shared_expert.up_proj.weight": w["sh_up"],
         p + "shared_expert.down_proj.weight": w["sh_down"]}
    os.makedirs(path, exist_ok=True)
    save_file({k: v.contiguous() for k, v in a.items()}, os.path.join(path, "model-00001.safetensors"))
    save_file({k: v.contiguous() for k, v in b.items()}, os.path.join(path, "model-00002.safetensors"))


def test_cpu_quantisation_matches_oracle():
    g = torch.Generator().manual_seed(0)
    w = torch.randn((3, 256, 384), generator=g) * 0.02
    w[1, :128, :128] = 0.0                               # an all-zero block: scale 1, codes 0
    w[2, 5, 7] = 3.0e4                                   # an outlier: its block's max code
    w[0, 9, 200] = -7.5e-6                               # far below its block's max: subnormal codes
    wb = w.to(torch.bfloat16)
    q, s = ck.quantize_blocks_cpu(wb)
    q_ref, s_ref = om.quant_blocks(wb.float().numpy())
    np.testing.assert_array_equal(s.numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).numpy(), q_ref)


def test_load_bf16_block(tmp_path):
    w, _ = make_layer(SHAPE, seed=1)
    w_other, _ = make_layer(SHAPE, seed=2)
    _write_checkpoint(str(tmp_path), w, w_other)
    blk = _block(SHAPE)
    assert ck.load_moe_block(blk, str(tmp_path), LAYER) == 7
    assert torch.equal(blk.gate.weight, w["gate"])
    assert torch.equal(blk.experts.gate_up_proj, w["gate_up"])      # not layer 2's tensor
    assert torch.equal(blk.experts.down_proj, w["down"])
    assert torch.equal(blk.shared_expert.gate_proj.weight, w["sh_gate"])
    assert torch.equal(blk.shared_expert.up_proj.weight, w["sh_up"])
    assert torch.equal(blk.shared_expert.down_proj.weight, w["sh_down"])
    assert torch.equal(blk.shared_expert_gate.weight, w["sh_gate_w"])


def test_convert_and_load_fp8(tmp_path):
    w, _ = make_layer(SHAPE, seed=1)
    w_other, _ = make_layer(SHAPE, seed=2)
    src, dst = str(tmp_path / "bf16"), str(tmp_path / "fp8")
    _write_checkpoint(src, w, w_other)
    # only layer LAYER: layer LAYER-1's expert weights stay bf16
    assert ck.quantize_checkpoint_fp8(src, dst, layers=[LAYER]) == 5
    from safetensors import safe_open
    with safe_open(os.path.join(dst, "model-00001.safetensors"), "pt", "cpu") as f:
        keys = set(f.keys())
        other = f.get_tensor("model." + ck.mlp_prefix(LAYER - 1) + "experts.gate_up_proj")
        assert other.dtype == torch.bfloat16 and torch.equal(other, w_other["gate_up"])
        assert "mtp.fc.weight" in keys
        assert f.get_tensor("model.language_model.layers.3.input_layernorm.weight").dtype == torch.bfloat16
    blk = _block(SHAPE)
    assert ck.load_moe_block(blk, dst, LAYER) == 2 + 4 + 6
    ex = blk.experts
    for (q, s), name in (((ex.gate_up_q, ex.gate_up_scale), "gate_up"), ((ex.down_q, ex.down_scale), "down")):
        q_ref, s_ref = om.quant_blocks(w[name].float().numpy())
        np.testing.assert_array_equal(q.numpy(), q_ref)
        np.testing.assert_array_equal(s.numpy(), s_ref)
    for n in ("gate", "up", "down"):
        q_ref, s_ref = om.quant_blocks(w["sh_" + n].float().numpy())
        np.testing.assert_array_equal(blk.shared_expert.q[n][0].numpy(), q_ref)
        np.testing.assert_array_equal(blk.shared_expert.q[n][1].numpy(), s_ref)
    assert torch.equal(blk.gate.weight, w["gate"])           # unquantised tensors load as bf16


def test_load_rejects_missing_scales(tmp_path):
    w, _ = make_layer(SHAPE, seed=1)
    p = "model." + ck.mlp_prefix(LAYER)
    q, _ = ck.quantize_blocks_cpu(w["gate_up"])
    save_file({p + "experts.gate_up_proj": q, p + "experts.down_proj": ck.quantize_blocks_cpu(w["down"])[0]},
              str(tmp_path / "m.safetensors"))
    with pytest.raises(KeyError):
        ck.load_moe_block(_block(SHAPE), str(tmp_path), LAYER)


def test_missing_directory_raises(tmp_path):
    with pytest.raises(FileNotFoundError):
        ck.load_moe_block(_block(SHAPE), str(tmp_path / "none"), LAYER)
