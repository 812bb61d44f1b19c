"""The HIP layer against the golden outputs recorded from the reference MoE block."""
import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.codecs import bf16_from_bits
from tests.helpers import bf16_bits_of, to_np
from tests.test_golden import NAMES, Z, _inputs
from tests.test_gpu_parity import _block, _region

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", NAMES)
def test_gpu_layer_matches_reference_outputs(gpu, name):
    shape, w, x = _inputs(Z, name)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    T, k = x.shape[0], shape.top_k
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=gpu)
    y = to_np(blk(x.to(gpu), workspace=ws))
    torch.cuda.synchronize()
    idx = to_np(_region(blk, ws, T, "topk_idx", torch.int32, (T, k))).astype(np.int64)
    logits = to_np(_region(blk, ws, T, "logits", torch.bfloat16, (T, shape.num_experts)))
    idx_r = Z[name + "/topk_idx"]
    same = (np.sort(idx, 1) == np.sort(idx_r, 1)).all(1)
    for t in np.nonzero(~same)[0]:
        zs = np.sort(logits[t])[::-1]
        assert zs[k - 1] == zs[k], f"row {t}: GPU selection differs from the reference without a tie"
    for alg in ("dense", "sparse"):
        y_r = bf16_from_bits(Z[name + f"/y_{alg}_bits"])
        assert om.rel_err(y[same], y_r[same]) < 1e-2, alg
