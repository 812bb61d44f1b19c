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


def scale_blocks_pow2(w, period=5):
    """w [..., N, K] (N, K multiples of 128) with 128x128 block (i, j) multiplied by
    2^((i + j) mod period): exact in bf16, so the e4m3 codes of every block are those of the
    unscaled weights and only the block scales carry the pattern. Neighbouring blocks differ
    by a factor 2 (or 2^-(period-1)), so an fp8 kernel that applies a neighbour's scale is off
    by far more than the fp8 tolerance."""
    *lead, N, K = w.shape
    i = torch.arange(N // 128).view(-1, 1)
    j = torch.arange(K // 128).view(1, -1)
    f = torch.pow(2.0, ((i + j) % period).float())
    f = f.repeat_interleave(128, 0).repeat_interleave(128, 1)
    return (w.float() * f.to(w.device)).to(w.dtype)


def scale_groups_pow2(x, period=3):
    """x [T, C] with the 128-channel group g of row t multiplied by 2^((t + 3g) mod period)
    (exact in bf16): every per-(row, 128) activation scale differs from its neighbours'."""
    T, C = x.shape
    t = torch.arange(T).view(-1, 1)
    g = torch.arange(C // 128).view(1, -1)
    f = torch.pow(2.0, ((t + 3 * g) % period).float()).repeat_interleave(128, 1)
    return (x.float() * f.to(x.device)).to(x.dtype)
