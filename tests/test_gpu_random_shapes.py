"""The whole layer against the oracle on seeded random shapes: hidden sizes, expert counts,
top-k, intermediate sizes (routed and shared), batch sizes and router biases drawn across the
paths the library picks between (fused small-batch routing, decode streaming GEMMs, tiled
prefill GEMMs with the one- or two-launch router, fp8 weights), 48 sampled output rows each."""
import random

import pytest
import torch

from layerbatch_amd.synth import MoEShape, zipf_bias
from tests.test_gpu_fp8 import _run_fp8
from tests.test_gpu_parity import _run_and_check

pytestmark = pytest.mark.gpu


def _draw(i):
    """Case i's (fp8, shape, T, bias): redrawn until the expert weights stay under 3e8 values
    per matrix, so each case runs in a few seconds."""
    rng = random.Random(1000 + i)
    while True:
        fp8 = rng.random() < 0.3
        H = rng.choice([512, 1024, 2048] if fp8 else [512, 1024, 1536, 2048])
        E = rng.choice([4, 8, 16, 20, 32, 48, 64, 96, 100, 128, 160, 256, 512])
        k = rng.randint(1, min(E, 12))
        I = rng.choice([256, 512, 768] if fp8 else [128, 256, 384, 512, 768])
        Is = rng.choice([0, 256, 512] if fp8 else [0, 0, 128, 256, 512])
        T = rng.choice([1, 3, 7, 16, 33, 100, 200, 257, 513, 1000, 1023, 1024, 1500, 2049, 3001,
                        4500])
        bias = (not fp8) and rng.random() < 0.4
        if E * I * H <= 3e8:
            return fp8, MoEShape(H, E, k, I, Is), T, bias


@pytest.mark.parametrize("i", range(24))
def test_random_shape(gpu, i):
    fp8, shape, T, bias = _draw(i)
    print(f"random case {i}: {'fp8' if fp8 else 'bf16'} {shape} T={T} bias={bias}", flush=True)
    if fp8:
        _run_fp8(shape, T, gpu, seed=i, sample=48)
    else:
        b = zipf_bias(torch.Generator().manual_seed(i), shape.num_experts) if bias else None
        _run_and_check(shape, T, gpu, seed=i, bias=b, sample=48)
