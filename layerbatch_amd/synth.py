"""Deterministic synthetic MoE-layer inputs (weights ~N(0, 0.02^2), activations ~N(0, 1)).

Shapes follow the MoE fields of the reference's HF config (nanovllm/config.py:98-102):
``hidden_size`` H, ``num_experts`` E, ``num_experts_per_tok`` k, ``moe_intermediate_size`` I,
``shared_expert_intermediate_size`` Is. Tensor layouts follow the reference's parameters
(nanovllm/models/qwen3_5.py:765, :795-800, :894-897).

Draw order from one torch.Generator seeded with ``seed`` on ``device``: router weight,
then per expert gate_up and down, then the shared expert's gate, up, down and gate weight,
then the activations, then the router bias permutation. Generation on the CPU is
reproducible across machines with the same torch build; generation on a GPU is
reproducible on that GPU model.
"""
from dataclasses import dataclass
import math

import torch

__all__ = ["MoEShape", "SHAPES", "make_layer", "make_x", "zipf_bias"]


@dataclass(frozen=True)
class MoEShape:
    hidden_size: int
    num_experts: int
    top_k: int
    moe_intermediate_size: int
    shared_expert_intermediate_size: int = 0


SHAPES = {
    # one small layer that a CPU oracle finishes in seconds: H=1024, E=16, top-2, I=512
    "small-h1024-e16": MoEShape(1024, 16, 2, 512, 0),
    # Qwen3-30B-A3B MoE layer: H=2048, E=128, top-8, I=768, no shared expert
    "qwen3-30b-a3b": MoEShape(2048, 128, 8, 768, 0),
    # Qwen3-Next-style sparse layer: H=2048, E=512, top-10, I=512, shared expert Is=512
    "qwen3-next-e512": MoEShape(2048, 512, 10, 512, 512),
}


def _randn(g, shape, std, device):
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(torch.bfloat16)


def make_layer(shape: MoEShape, seed=0, device="cpu", std=0.02):
    """Returns (dict of bf16 weight tensors, generator positioned after the weights).

    Keys: gate [E,H], gate_up [E,2I,H], down [E,H,I] and, when Is > 0,
    sh_gate [Is,H], sh_up [Is,H], sh_down [H,Is], sh_gate_w [1,H].
    """
    H, E, I, Is = (shape.hidden_size, shape.num_experts, shape.moe_intermediate_size,
                   shape.shared_expert_intermediate_size)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    w = {"gate": _randn(g, (E, H), std, device)}
    gu = torch.empty((E, 2 * I, H), dtype=torch.bfloat16, device=device)
    dn = torch.empty((E, H, I), dtype=torch.bfloat16, device=device)
    for e in range(E):
        gu[e] = _randn(g, (2 * I, H), std, device)
        dn[e] = _randn(g, (H, I), std, device)
    w["gate_up"] = gu
    w["down"] = dn
    if Is:
        w["sh_gate"] = _randn(g, (Is, H), std, device)
        w["sh_up"] = _randn(g, (Is, H), std, device)
        w["sh_down"] = _randn(g, (H, Is), std, device)
        w["sh_gate_w"] = _randn(g, (1, H), std, device)
    return w, g


def make_x(g, T, H, device="cpu"):
    """Activations [T,H] ~N(0,1) in bf16, drawn from generator ``g``."""
    return _randn(g, (T, H), 1.0, device)


def zipf_bias(g, E, s=1.2, device="cpu"):
    """fp32 router logit bias [E]: bias[e] = ln p_{pi(e)}, p_r proportional to r^-s,
    r = 1..E, pi a permutation drawn from ``g``. Skews expert loads (some experts get no
    tokens, a few get thousands at T=8192)."""
    r = torch.arange(1, E + 1, dtype=torch.float64)
    p = r.pow(-s)
    p = p / p.sum()
    perm = torch.randperm(E, generator=g, device=device).cpu()
    return torch.log(p[perm]).to(torch.float32).to(device)


def algorithmic_bytes(shape: MoEShape, T, n_hit, weight_bytes=2.0, scale_bytes_per_expert=0):
    """Bytes the layer must move at minimum: each hit expert's weights once, the shared
    expert's weights and gate, the router weight, and x in plus y out."""
    H, E, I, Is = (shape.hidden_size, shape.num_experts, shape.moe_intermediate_size,
                   shape.shared_expert_intermediate_size)
    b = n_hit * (3 * H * I * weight_bytes + scale_bytes_per_expert)
    if Is:
        b += 3 * H * Is * weight_bytes + H * 2
        b += scale_bytes_per_expert * Is / I if scale_bytes_per_expert else 0
    b += E * H * 2 + 2 * T * H * 2
    return float(b)


def algorithmic_flops(shape: MoEShape, T):
    H, E, k, I, Is = (shape.hidden_size, shape.num_experts, shape.top_k,
                      shape.moe_intermediate_size, shape.shared_expert_intermediate_size)
    return float(2 * T * k * 3 * H * I + 2 * T * 3 * H * Is + 2 * T * E * H)
