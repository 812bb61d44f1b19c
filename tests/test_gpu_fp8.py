"""GPU parity of the fp8 (OCP e4m3fn) variant against the CPU oracle's dequantised fp32 path."""
import ctypes
import os

import numpy as np
import pytest
import torch

from layerbatch_amd import _lib
from layerbatch_amd.moe import Qwen3_5SparseMoeBlock
from layerbatch_amd.synth import MoEShape, make_layer, make_x
from oracle import moe as om
from tests import gpu_checks as gc
from tests.helpers import bf16_bits_of, layer_np, scale_blocks_pow2, scale_groups_pow2, to_np
from tests.test_gpu_parity import _block, _region

pytestmark = pytest.mark.gpu


def test_quantize_blocks_bit_exact(gpu):
    g = torch.Generator().manual_seed(3)
    w = (torch.randn((3, 256, 384), generator=g) * 0.02)
    w[1, :128, :128] = 0.0                              # an all-zero block: scale 1, codes 0
    w[2, 5, 7] = 3.0e4                                  # a large outlier
    wb = w.to(torch.bfloat16)
    from layerbatch_amd.moe import _quantize_blocks
    q, s = _quantize_blocks(wb.to(gpu))
    torch.cuda.synchronize()
    q_ref, s_ref = om.quant_blocks(to_np(wb))
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


def _fp8_oracle(wn, q, xn, idx, topw, shared):
    y = om.experts_fp8(xn, idx, topw, q["wgu_q"], q["wgu_s"], q["wd_q"], q["wd_s"])
    if shared:
        gsh = om.shared_gate(xn, wn["sh_gate_w"]).astype(np.float64)
        y = y + gsh[:, None] * om.shared_expert_fp8(xn, q["sh_gate_q"], q["sh_gate_s"], q["sh_up_q"],
                                                    q["sh_up_s"], q["sh_down_q"], q["sh_down_s"])
    return y


def _run_fp8(shape, T, device, seed=0, sample=None, patterned=False):
    w, g = make_layer(shape, seed=seed)
    x = make_x(g, T, shape.hidden_size)
    if patterned:
        # every weight block scale and activation group scale differs from its neighbours
        w = {k_: (scale_blocks_pow2(v) if k_ in ("gate_up", "down", "sh_gate", "sh_up", "sh_down")
                  else v) for k_, v in w.items()}
        x = scale_groups_pow2(x)
    blk = _block(shape, {k_: v.to(device) for k_, v in w.items()}, device)
    blk.quantize_fp8_()
    xd = x.to(device)
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=device)
    y = blk(xd, workspace=ws)
    torch.cuda.synchronize()
    k = shape.top_k
    idx = to_np(_region(blk, ws, T, "topk_idx", torch.int32, (T, k))).astype(np.int64)
    topw = to_np(_region(blk, ws, T, "topk_w", torch.bfloat16, (T, k)))
    logits = _region(blk, ws, T, "logits", torch.bfloat16, (T, shape.num_experts))
    gc.check_route(idx, bf16_bits_of(_region(blk, ws, T, "topk_w", torch.bfloat16, (T, k))),
                   to_np(logits), None, k)
    ex = blk.experts
    q = {"wgu_q": ex.gate_up_q.cpu().numpy(), "wgu_s": ex.gate_up_scale.cpu().numpy(),
         "wd_q": ex.down_q.cpu().numpy(), "wd_s": ex.down_scale.cpu().numpy()}
    wn = layer_np(w)
    # the GPU's quantised weights must be the oracle's quantisation of the bf16 weights
    q_ref, s_ref = om.quant_blocks(wn["gate_up"])
    np.testing.assert_array_equal(q["wgu_q"], q_ref)
    np.testing.assert_array_equal(q["wgu_s"], s_ref)
    shared = shape.shared_expert_intermediate_size > 0
    if shared:
        for n in ("gate", "up", "down"):
            cq, cs = blk.shared_expert.q[n]
            q[f"sh_{n}_q"], q[f"sh_{n}_s"] = cq.cpu().numpy(), cs.cpu().numpy()
    xn = to_np(x)
    rows = np.arange(T) if sample is None else np.unique(
        np.random.default_rng(seed).choice(T, size=min(sample, T), replace=False))
    y_ref = _fp8_oracle(wn, q, xn[rows], idx[rows], topw[rows], shared)
    err = gc.check_output(to_np(y)[rows], y_ref, gc.TOL_FP8)
    # and the fp8 layer stays close to the bf16 layer it approximates
    y_bf = gc.block_reference(xn[rows], wn, idx[rows], topw[rows], k, shared=True if shared else None)
    assert om.rel_err(to_np(y)[rows], y_bf) < 0.1
    if patterned:
        # the pattern makes scale indexing visible: the oracle itself, given each weight block
        # its k-neighbour's scale, lands ten times the tolerance away
        shifted = om.experts_fp8(xn[rows], idx[rows], topw[rows], q["wgu_q"],
                                 np.roll(q["wgu_s"], 1, axis=-1), q["wd_q"],
                                 np.roll(q["wd_s"], 1, axis=-1))
        y_routed = om.experts_fp8(xn[rows], idx[rows], topw[rows], q["wgu_q"], q["wgu_s"],
                                  q["wd_q"], q["wd_s"])
        assert om.rel_err(shifted, y_routed) > 10 * gc.TOL_FP8
    return err


@pytest.mark.parametrize("T", [1, 64, 200])
def test_fp8_block_small(gpu, T):
    _run_fp8(MoEShape(1024, 16, 2, 512, 0), T, gpu, seed=T)


# E not a multiple of 16, odd k, H with 6 k-blocks of 256 bytes, I = 3 such blocks
@pytest.mark.parametrize("T", [37, 300])
def test_fp8_block_odd_shape(gpu, T):
    _run_fp8(MoEShape(1536, 20, 3, 768, 256), T, gpu, seed=T)


def test_fp8_block_shared(gpu):
    _run_fp8(MoEShape(1024, 32, 4, 256, 512), 96, gpu, seed=5)


@pytest.mark.parametrize("T", [2048, 3001])
def test_fp8_block_prefill_tiled(gpu, T):
    """Prefill-sized batch: fp8 LDS-tiled GEMMs (shared expert included)."""
    _run_fp8(MoEShape(1024, 16, 2, 512, 256), T, gpu, seed=T, sample=64)


# weight blocks scaled by 2^((i+j) mod 5) and activation groups by 2^((t+3g) mod 3), so that
# reading a neighbouring block's or group's scale fails by far more than 3e-2: streaming GEMMs
# (T = 1, 64), the LDS-tiled GEMMs (T = 700, several k-tiles in both GEMMs), shared expert
# included; every row
@pytest.mark.parametrize("T", [1, 64, 700])
def test_fp8_block_scale_patterns(gpu, T):
    _run_fp8(MoEShape(1024, 16, 2, 768, 256), T, gpu, seed=T + 40, patterned=True)


def test_fp8_dense_mlp(gpu):
    shape = MoEShape(1024, 8, 2, 256, 512)
    w, g = make_layer(shape, seed=6)
    x = make_x(g, 70, 1024)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    blk.quantize_fp8_()
    out = blk.shared_expert(x.to(gpu))
    se = blk.shared_expert
    qq = {n: (se.q[n][0].cpu().numpy(), se.q[n][1].cpu().numpy()) for n in ("gate", "up", "down")}
    ref = om.shared_expert_fp8(to_np(x), *qq["gate"], *qq["up"], *qq["down"])
    gc.check_output(to_np(out), ref, gc.TOL_FP8)


def test_fp8_rejects_unsupported_width(gpu, lbmoe):
    from layerbatch_amd._lib import LbmoeLayer
    L = LbmoeLayer()
    L.hidden_size, L.num_experts, L.top_k = 1024, 8, 2
    L.moe_intermediate_size, L.weight_dtype = 384, _lib.LBMOE_W_FP8_E4M3
    n = ctypes.c_size_t(0)
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), 4, ctypes.byref(n)) == -2


@pytest.mark.parametrize("T", [64, 600])      # streaming and LDS-tiled fp8 GEMMs
def test_fp8_checkpoint_matches_quantize(gpu, tmp_path, T):
    """An fp8 checkpoint written by the offline converter (CPU quantisation) and loaded into a
    block gives bit-identical outputs to quantize_fp8_ (GPU quantisation) of the same weights."""
    from safetensors.torch import save_file
    from layerbatch_amd import checkpoint as ck
    shape = MoEShape(1024, 16, 2, 512, 256)
    w, g = make_layer(shape, seed=12)
    x = make_x(g, T, shape.hidden_size).to(gpu)
    p = "model." + ck.mlp_prefix(0)
    names = {"gate": "gate.weight", "gate_up": "experts.gate_up_proj", "down": "experts.down_proj",
             "sh_gate": "shared_expert.gate_proj.weight", "sh_up": "shared_expert.up_proj.weight",
             "sh_down": "shared_expert.down_proj.weight", "sh_gate_w": "shared_expert_gate.weight"}
    src, dst = tmp_path / "bf16", tmp_path / "fp8"
    os.makedirs(src)
    save_file({p + n: w[k].contiguous() for k, n in names.items()}, str(src / "model.safetensors"))
    assert ck.quantize_checkpoint_fp8(str(src), str(dst)) == 5
    loaded = Qwen3_5SparseMoeBlock(1024, 16, 2, 512, 256).to(device=gpu, dtype=torch.bfloat16)
    ck.load_moe_block(loaded, str(dst), 0)
    ref = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu).quantize_fp8_()
    y1, y2 = loaded(x), ref(x)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_fp8_prefill_persistent_gate_up(gpu):
    """A batch whose fp8 gate_up table has at least 6 entries per CU (H=1024, E=64, top-8, I=768,
    T=8192 under a Zipf bias: wide, narrow and tiny tiles, empty experts whose entries are idle),
    so gate_up runs as the persistent work-queue kernel. The workspace starts as all-ones bytes
    (e4m3 NaN codes and NaN scales), so an item the queues skipped leaves NaN in the output: every
    row is checked against the fp8 oracle."""
    from layerbatch_amd.synth import zipf_bias
    shape = MoEShape(1024, 64, 8, 768, 0)
    T, k = 8192, 8
    w, g = make_layer(shape, seed=17)
    x = make_x(g, T, shape.hidden_size)
    bias = zipf_bias(torch.Generator().manual_seed(29), shape.num_experts)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    blk.gate.logit_bias = bias.to(gpu)
    blk.quantize_fp8_()
    ws = torch.full((blk.workspace_size(T),), 255, dtype=torch.uint8, device=gpu)
    y = blk(x.to(gpu), workspace=ws)
    torch.cuda.synchronize()
    idx = to_np(_region(blk, ws, T, "topk_idx", torch.int32, (T, k))).astype(np.int64)
    topw = to_np(_region(blk, ws, T, "topk_w", torch.bfloat16, (T, k)))
    gc.check_route(idx, bf16_bits_of(_region(blk, ws, T, "topk_w", torch.bfloat16, (T, k))),
                   to_np(_region(blk, ws, T, "logits", torch.bfloat16, (T, shape.num_experts))),
                   bias.numpy(), k)
    ex = blk.experts
    y_ref = om.experts_fp8(to_np(x), idx, topw, ex.gate_up_q.cpu().numpy(),
                           ex.gate_up_scale.cpu().numpy(), ex.down_q.cpu().numpy(),
                           ex.down_scale.cpu().numpy())
    yn = to_np(y)
    assert np.isfinite(yn).all(), "rows the gate_up queues skipped"
    gc.check_output(yn, y_ref, gc.TOL_FP8)
