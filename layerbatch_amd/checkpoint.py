"""Safetensors loading of the MoE block's weights and the offline fp8 block-quantisation
converter.

Loading follows the reference loader (nanovllm/utils/loader.py:16-61): every ``*.safetensors``
file of a checkpoint directory is scanned, the ``model.`` weight prefix is stripped
(qwen3_5.py:1052) and tensors are copied into parameters of the same name
(``param.data.copy_``, loader.py:12-13). Only one decoder layer's MoE block is filled: the
names under ``language_model.layers.{i}.mlp.`` (qwen3_5.py:795-800, :892-897, :912-914).

The converter writes the fp8 variant of such a checkpoint: each routed-expert and
shared-expert weight ``W [..., N, K]`` becomes e4m3fn codes under the same name plus fp32
scales ``W_scale [..., N/128, K/128]`` (scale = amax / 448 per 128 x 128 block, 1 for an
all-zero block; code = round-to-nearest-even of W / scale). This is the quantisation that
``Qwen3_5SparseMoeBlock.quantize_fp8_`` performs on the GPU, computed here on the CPU with
the same fp32 arithmetic, so both give identical codes and scales. Every other tensor is
copied unchanged.
"""
import os
from glob import glob

import torch

__all__ = ["MOE_WEIGHTS", "mlp_prefix", "load_moe_block", "quantize_blocks_cpu",
           "quantize_checkpoint_fp8"]

WEIGHT_PREFIX = "model."
# names of the MoE block's tensors below its prefix; the quantised ones are marked
MOE_WEIGHTS = {
    "gate.weight": False,
    "experts.gate_up_proj": True,
    "experts.down_proj": True,
    "shared_expert.gate_proj.weight": True,
    "shared_expert.up_proj.weight": True,
    "shared_expert.down_proj.weight": True,
    "shared_expert_gate.weight": False,
}
SCALE_SUFFIX = "_scale"


def mlp_prefix(layer_idx):
    """Parameter-name prefix of decoder layer ``layer_idx``'s MoE block (after the weight
    prefix is stripped)."""
    return f"language_model.layers.{layer_idx}.mlp."


def _files(path):
    files = sorted(glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors files in {path}")
    return files


def quantize_blocks_cpu(w):
    """bf16 [..., N, K] -> (e4m3fn codes, fp32 scales [..., N/128, K/128]) on the CPU."""
    *lead, N, K = w.shape
    if N % 128 or K % 128:
        raise ValueError(f"block quantisation needs both trailing dims divisible by 128, got {N}x{K}")
    wf = w.detach().to("cpu", torch.float32).reshape(*lead, N // 128, 128, K // 128, 128)
    amax = wf.abs().amax(dim=(-3, -1))                      # [..., N/128, K/128]
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wf / scale[..., :, None, :, None]).to(torch.float8_e4m3fn)
    return q.reshape(w.shape), scale.contiguous()


def load_moe_block(block, path, layer_idx, weight_prefix=WEIGHT_PREFIX):
    """Fill ``block`` (a Qwen3_5SparseMoeBlock) from the checkpoint directory ``path``.

    bf16 tensors are copied into the block's parameters. When the checkpoint holds the fp8
    variant (e4m3fn expert weights with ``_scale`` companions), the codes and scales are
    installed as the block's fp8 weights instead. Returns the number of tensors used.
    """
    from safetensors import safe_open
    prefix = mlp_prefix(layer_idx)
    found = {}
    for file in _files(path):
        with safe_open(file, "pt", "cpu") as f:
            for name in f.keys():
                pname = name[len(weight_prefix):] if weight_prefix and name.startswith(weight_prefix) else name
                if not pname.startswith(prefix):
                    continue
                found[pname[len(prefix):]] = f.get_tensor(name)
    fp8 = found.get("experts.gate_up_proj") is not None and \
        found["experts.gate_up_proj"].dtype == torch.float8_e4m3fn
    used = 0
    with torch.no_grad():
        for key, quantised in MOE_WEIGHTS.items():
            if key not in found:
                continue
            if fp8 and quantised:
                continue
            param = block.get_parameter(key)
            param.data.copy_(found[key])
            used += 1
        if fp8:
            dev = block.gate.weight.device

            def pair(key):
                if key + SCALE_SUFFIX not in found:
                    raise KeyError(f"fp8 checkpoint lacks {prefix}{key}{SCALE_SUFFIX}")
                return (found[key].view(torch.uint8).to(dev),
                        found[key + SCALE_SUFFIX].to(dev, torch.float32))

            experts = pair("experts.gate_up_proj") + pair("experts.down_proj")
            shared = None
            if block.shared_expert is not None:
                shared = {n: pair(f"shared_expert.{n}_proj.weight") for n in ("gate", "up", "down")}
            block.load_fp8_(experts, shared)
            used += 4 + (6 if shared else 0)
    return used


def _is_quantised(pname, layer_filter):
    for key, quantised in MOE_WEIGHTS.items():
        if quantised and pname.endswith(".mlp." + key):
            if layer_filter is None:
                return True
            return any(pname.startswith(mlp_prefix(i)) for i in layer_filter)
    return False


def quantize_checkpoint_fp8(src, dst, layers=None, weight_prefix=WEIGHT_PREFIX):
    """Write the fp8 variant of checkpoint directory ``src`` into ``dst``, file by file.

    layers: decoder-layer indices whose MoE weights are quantised (None: all). Returns the
    number of tensors quantised.
    """
    from safetensors import safe_open
    from safetensors.torch import save_file
    os.makedirs(dst, exist_ok=True)
    n_q = 0
    for file in _files(src):
        out = {}
        with safe_open(file, "pt", "cpu") as f:
            meta = f.metadata()
            for name in f.keys():
                t = f.get_tensor(name)
                pname = name[len(weight_prefix):] if weight_prefix and name.startswith(weight_prefix) else name
                if _is_quantised(pname, layers) and t.dtype in (torch.bfloat16, torch.float16, torch.float32):
                    q, s = quantize_blocks_cpu(t)
                    out[name] = q
                    out[name + SCALE_SUFFIX] = s
                    n_q += 1
                else:
                    out[name] = t
        save_file(out, os.path.join(dst, os.path.basename(file)), metadata=meta)
    return n_q
