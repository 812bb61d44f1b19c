"""Checks shared by the GPU parity tests, smoke() and bench.py's self-check.

Every function compares a GPU result (numpy arrays copied back) with the CPU oracle.
"""
import numpy as np

from oracle import moe as om
from oracle.codecs import bf16_bits, bf16_from_bits, bf16_round

# Tolerances of the layer output against the float64 oracle (normwise max relative error).
TOL_BF16 = 1e-2
TOL_FP8 = 3e-2


def check_logits(gpu_bits, x, wg, max_frac=2e-3, acc_tol=2e-5):
    """GPU bf16 logits vs the correctly rounded bf16 of the exact dot products.

    The GPU accumulates in fp32 in its own order, so its value is bf16(e + d) for the exact
    dot product e and an accumulation error |d| <= acc_tol * sum_i |x_i w_i|. Every GPU logit
    must lie in [bf16(e - tol), bf16(e + tol)], and at most max_frac of them may differ from
    the correctly rounded bf16(e) at all (at least 2, so that one or two rounding-boundary
    logits of a small batch, e.g. one token's 96 logits, do not fail the fraction).
    """
    x64 = np.asarray(x, np.float64)
    w64 = np.asarray(wg, np.float64)
    exact = x64 @ w64.T
    tol = acc_tol * (np.abs(x64) @ np.abs(w64).T)
    ref_bits = bf16_bits(exact.astype(np.float32))
    gpu_bits = np.asarray(gpu_bits, np.uint16)
    diff = gpu_bits != ref_bits
    frac = float(diff.mean()) if diff.size else 0.0
    assert int(diff.sum()) <= max(max_frac * diff.size, 2), (
        f"{frac:.2e} of logits differ from the oracle")
    if diff.any():
        g = bf16_from_bits(gpu_bits[diff]).astype(np.float64)
        lo = bf16_round((exact[diff] - tol[diff]).astype(np.float32)).astype(np.float64)
        hi = bf16_round((exact[diff] + tol[diff]).astype(np.float32)).astype(np.float64)
        bad = (g < lo) | (g > hi)
        assert not bad.any(), (f"{int(bad.sum())} logits outside fp32-accumulation reach of the "
                               f"exact value, e.g. gpu {g[bad][:3]} exact {exact[diff][bad][:3]}")
    return frac


def check_route(gpu_idx, gpu_w_bits, logits, bias, k):
    """Selection from identical logits must be bit-exact; weights within one bf16 step."""
    w_ref, idx_ref, _ = om.route(logits, k, bias)
    np.testing.assert_array_equal(np.asarray(gpu_idx, np.int64), idx_ref)
    ref_bits = bf16_bits(w_ref).astype(np.int32)
    d = np.abs(np.asarray(gpu_w_bits, np.int32) - ref_bits)
    assert d.max(initial=0) <= 1, f"top-k weights differ by {d.max()} bf16 steps"
    return w_ref, idx_ref


def check_permutation(idx, E, counts, offsets, perm_tok, perm_slot, inv):
    c, o, pt, ps, iv = om.permute(idx, E)
    np.testing.assert_array_equal(np.asarray(counts)[:E], c)
    np.testing.assert_array_equal(np.asarray(offsets)[:E + 1], o)
    V = idx.size
    np.testing.assert_array_equal(np.asarray(perm_tok)[:V], pt)
    np.testing.assert_array_equal(np.asarray(perm_slot)[:V], ps)
    np.testing.assert_array_equal(np.asarray(inv).reshape(idx.shape), iv)


def block_reference(x, w, idx, topw, k, shared=None):
    """float64 oracle output of the block for a given routing (idx, topw)."""
    y = om.experts(x, idx, topw, w["gate_up"], w["down"])
    if shared is not None:
        g = om.shared_gate(x, w["sh_gate_w"]).astype(np.float64)
        y = y + g[:, None] * om.shared_expert(x, w["sh_gate"], w["sh_up"], w["sh_down"])
    return y


def check_output(y_gpu, y_ref, tol):
    err = om.rel_err(y_gpu, y_ref)
    assert err <= tol, f"relative error {err:.3e} > {tol}"
    return err
