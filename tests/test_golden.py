"""Golden vectors recorded from the reference MoE block (tests/golden/make_reference_golden.py)
against the CPU oracle and the torch-CPU restatement (no GPU needed)."""
import hashlib
import os

import numpy as np
import pytest
import torch

from layerbatch_amd.synth import MoEShape, make_layer, make_x
from oracle import moe as om
from oracle import torch_ref as tr
from oracle.codecs import bf16_from_bits
from tests.helpers import layer_np, to_np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_moe_small.npz")


def _cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def _inputs(z, name):
    H, E, k, I, Is, T, seed = (int(v) for v in z[name + "/meta"])
    shape = MoEShape(H, E, k, I, Is)
    w, g = make_layer(shape, seed=seed)
    x = make_x(g, T, H)
    return shape, w, x


def _sha(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


Z, NAMES = _cases()


@pytest.mark.parametrize("name", NAMES)
def test_generator_reproduces_golden_inputs(name):
    shape, w, x = _inputs(Z, name)
    assert _sha(x) == str(Z[name + "/x_sha256"])
    for k_, v in w.items():
        assert _sha(v) == str(Z[name + "/" + k_ + "_sha256"]), k_


@pytest.mark.parametrize("name", NAMES)
def test_torch_restatement_is_bit_exact(name):
    """oracle/torch_ref.py reproduces the reference's router and both expert algorithms bit
    for bit on the same torch build."""
    shape, w, x = _inputs(Z, name)
    tw, ti = tr.route(x, w["gate"], shape.top_k)
    np.testing.assert_array_equal(tw.view(torch.int16).numpy().view(np.uint16), Z[name + "/topk_w_bits"])
    np.testing.assert_array_equal(ti.numpy(), Z[name + "/topk_idx"])
    sh = None
    if shape.shared_expert_intermediate_size:
        sh = (w["sh_gate"], w["sh_up"], w["sh_down"], w["sh_gate_w"])
    for alg in ("dense", "sparse"):
        y, _, _ = tr.block(x, w["gate"], w["gate_up"], w["down"], shape.top_k, sh=sh, algorithm=alg)
        if sh is None:
            y = y + 0.0 * y      # the reference adds sigmoid(0) * 0 from its empty shared expert
        np.testing.assert_array_equal(y.view(torch.int16).numpy().view(np.uint16),
                                      Z[name + f"/y_{alg}_bits"])


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference(name):
    """Selection equal modulo ties at the top-k boundary; output within bf16 tolerance."""
    shape, w, x = _inputs(Z, name)
    wn, xn = layer_np(w), to_np(x)
    k = shape.top_k
    logits = om.router_logits(xn, wn["gate"])
    w_o, idx_o, _ = om.route(logits, k)
    idx_r = Z[name + "/topk_idx"]
    w_r = bf16_from_bits(Z[name + "/topk_w_bits"])
    same = (np.sort(idx_o, 1) == np.sort(idx_r, 1)).all(1)
    for t in np.nonzero(~same)[0]:
        zs = np.sort(logits[t])[::-1]
        assert zs[k - 1] == zs[k], f"row {t}: selection differs without a boundary tie"
    # where the expert sets agree, the ordered lists agree after the canonical tie rule
    for t in np.nonzero(same)[0]:
        order_r = sorted(range(k), key=lambda s: (-logits[t, idx_r[t, s]], idx_r[t, s]))
        assert list(idx_r[t, order_r]) == list(idx_o[t])
        np.testing.assert_allclose(w_r[t, order_r], w_o[t], rtol=2 ** -7)
    shared = None
    if shape.shared_expert_intermediate_size:
        shared = {"gate": wn["sh_gate"], "up": wn["sh_up"], "down": wn["sh_down"], "gate_w": wn["sh_gate_w"]}
    y_o = om.experts(xn, idx_r, w_r, wn["gate_up"], wn["down"])
    if shared:
        gsh = om.shared_gate(xn, shared["gate_w"]).astype(np.float64)
        y_o = y_o + gsh[:, None] * om.shared_expert(xn, shared["gate"], shared["up"], shared["down"])
    for alg in ("dense", "sparse"):
        y_r = bf16_from_bits(Z[name + f"/y_{alg}_bits"])
        assert om.rel_err(y_r, y_o) < 1e-2
