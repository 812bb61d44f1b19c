"""Shared helpers of the test suite (CPU side)."""
import numpy as np
import torch

from oracle.codecs import bf16_from_bits


def to_np(t):
    """torch tensor (any device) -> numpy; bf16 becomes float32 values."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return bf16_from_bits(t.view(torch.int16).numpy().view(np.uint16))
    return t.numpy()


def bf16_bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def layer_np(w):
    """dict of bf16 torch weights -> dict of float32 numpy arrays."""
    return {k: to_np(v) for k, v in w.items()}
