"""Pins the CPU oracle against independent computations (no GPU needed).

Each check is chosen so that a plausible mistake in the oracle (a dropped term, a swapped
gate/up half, a wrong tie rule, a transposed operand, an off-by-one in the permutation)
fails it without retyping the oracle's own formula.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import codecs, moe as om, torch_ref as tr
from layerbatch_amd.synth import MoEShape, make_layer, make_x, zipf_bias
from tests.helpers import layer_np, to_np


# ---- codecs ---------------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(3.0),
        np.float32([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38,
                    1.00390625, 1.01171875, 1.0078125 + 2 ** -24]),
        # exact halfway cases in both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(codecs.bf16_bits(x), ref)
    assert codecs.bf16_bits(np.float32([np.nan]))[0] == 0x7FC0


def test_e4m3_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    mine = codecs.e4m3_decode(np.arange(256, dtype=np.uint8))
    finite = ~np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(mine), ~finite)
    np.testing.assert_array_equal(mine[finite], ref[finite])
    assert codecs.e4m3_decode(np.uint8([0x7E]))[0] == 448.0
    assert codecs.e4m3_decode(np.uint8([0x01]))[0] == 2.0 ** -9


def test_e4m3_encode_matches_torch_in_range():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.uniform(-448, 448, 200000).astype(np.float32),
        (rng.standard_normal(100000) * 0.01).astype(np.float32),
        codecs.e4m3_values()[:127].astype(np.float32),
        # midpoints between consecutive codes exercise ties-to-even
        (0.5 * (codecs.e4m3_values()[:126] + codecs.e4m3_values()[1:127])).astype(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(codecs.e4m3_encode(x), ref)


def test_e4m3_saturates_and_roundtrips():
    assert codecs.e4m3_encode(np.float32([500.0, -1e9, 448.0, 460.0]) ).tolist() == [0x7E, 0xFE, 0x7E, 0x7E]
    vals = codecs.e4m3_values()
    for c in range(256):
        if np.isnan(vals[c]):
            continue
        assert codecs.e4m3_encode(np.float32([vals[c]]))[0] == c


# ---- router ----------------------------------------------------------------------------------

def _brute_topk(z, k):
    return [sorted(range(len(row)), key=lambda e: (-row[e], e))[:k] for row in z]


def test_route_matches_bruteforce_with_ties():
    rng = np.random.default_rng(2)
    for E, k in [(16, 2), (128, 8), (512, 10), (5, 5), (7, 1)]:
        # coarse logits force many ties
        lg = codecs.bf16_round((rng.integers(-6, 6, size=(64, E)) * 0.25).astype(np.float32))
        w, idx, p = om.route(lg, k)
        assert idx.tolist() == _brute_topk(lg.tolist(), k)
        # the same order by probability (the canonical (-p, index) rule)
        np.testing.assert_array_equal(om.route_by_prob(p, k), idx)
        # weights: sorted non-increasing, sum to one within bf16 rounding
        assert np.all(np.diff(w, axis=1) <= 0)
        assert np.all(np.abs(w.sum(1) - 1) <= k * 2 ** -8)


def test_route_closed_forms():
    rng = np.random.default_rng(3)
    lg = codecs.bf16_round(rng.standard_normal((32, 8)).astype(np.float32))
    w, idx, p = om.route(lg, 1)
    assert np.all(w == 1.0)
    w, idx, p = om.route(lg, 8)                        # k = E selects every expert
    assert all(sorted(r) == list(range(8)) for r in idx.tolist())
    # renormalised weights of all experts equal the softmax probabilities
    np.testing.assert_allclose(w, codecs.bf16_round(np.take_along_axis(p, idx, 1)), atol=2 ** -8)
    # softmax against float64
    z = lg.astype(np.float64)
    ref = np.exp(z - z.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    np.testing.assert_allclose(p, ref, rtol=1e-6)


def test_route_bias_shifts_selection():
    lg = np.zeros((4, 8), np.float32)
    bias = np.arange(8, dtype=np.float32)
    w, idx, _ = om.route(lg, 3, bias)
    assert idx.tolist() == [[7, 6, 5]] * 4


def test_router_logits_match_torch_linear():
    """fp64 dot products rounded to bf16 equal torch's bf16 F.linear within one bf16 step."""
    sh = MoEShape(1024, 16, 2, 128)
    w, g = make_layer(sh, seed=1)
    x = make_x(g, 64, 1024)
    mine = om.router_logits(to_np(x), to_np(w["gate"]))
    ref = to_np(torch.nn.functional.linear(x, w["gate"]))
    steps = np.abs(codecs.bf16_bits(mine).astype(np.int32) - codecs.bf16_bits(ref).astype(np.int32))
    assert steps.max() <= 1 and steps.mean() < 0.05


def test_shared_gate_closed_form():
    x = np.ones((2, 4), np.float32)
    wsg = np.zeros((1, 4), np.float32)
    np.testing.assert_allclose(om.shared_gate(x, wsg), [0.5, 0.5])


# ---- permutation -----------------------------------------------------------------------------

@pytest.mark.parametrize("T,k,E", [(1, 1, 1), (5, 2, 4), (64, 2, 16), (37, 8, 128), (300, 10, 512)])
def test_permute_matches_bruteforce(T, k, E):
    rng = np.random.default_rng(T + k + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    counts, offsets, pt, ps, inv = om.permute(idx, E)
    keys = sorted((int(idx[t, s]), s, t) for t in range(T) for s in range(k))
    assert [(int(idx[t, s]), int(s), int(t)) for t, s in zip(pt, ps)] == keys
    assert counts.tolist() == [sum(1 for kk in keys if kk[0] == e) for e in range(E)]
    assert offsets.tolist() == [0] + list(itertools.accumulate(counts.tolist()))
    for t in range(T):
        for s in range(k):
            assert (pt[inv[t, s]], ps[inv[t, s]]) == (t, s)


def test_permute_matches_reference_where_order():
    """Per expert, the reference visits torch.where(mask[e]) of the [k, T] one-hot mask."""
    rng = np.random.default_rng(7)
    T, k, E = 50, 4, 12
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    counts, offsets, pt, ps, _ = om.permute(idx, E)
    mask = torch.nn.functional.one_hot(torch.from_numpy(idx), E).permute(2, 1, 0)
    for e in range(E):
        slot, tok = torch.where(mask[e])
        seg = slice(offsets[e], offsets[e + 1])
        assert pt[seg].tolist() == tok.tolist()
        assert ps[seg].tolist() == slot.tolist()


# ---- experts / block -------------------------------------------------------------------------

def test_experts_reduce_to_dense_swiglu():
    """E = 1, k = 1: the block is Qwen3MLP's down(silu(gate x) * up x) (qwen3.py:112-116)."""
    rng = np.random.default_rng(4)
    H, I = 64, 48
    x = rng.standard_normal((9, H))
    wgu = rng.standard_normal((1, 2 * I, H)) * 0.1
    wd = rng.standard_normal((1, H, I)) * 0.1
    y = om.experts(x, np.zeros((9, 1), np.int64), np.ones((9, 1)), wgu, wd)
    xt = torch.from_numpy(x)
    gate = xt @ torch.from_numpy(wgu[0, :I]).T
    up = xt @ torch.from_numpy(wgu[0, I:]).T
    ref = (torch.nn.functional.silu(gate) * up) @ torch.from_numpy(wd[0]).T
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_experts_linear_in_down_and_weights():
    rng = np.random.default_rng(5)
    T, H, I, E, k = 11, 32, 16, 6, 3
    x = rng.standard_normal((T, H))
    wgu = rng.standard_normal((E, 2 * I, H)) * 0.2
    wd = rng.standard_normal((E, H, I)) * 0.2
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    w = rng.uniform(0, 1, (T, k))
    y = om.experts(x, idx, w, wgu, wd)
    np.testing.assert_allclose(om.experts(x, idx, w, wgu, 3 * wd), 3 * y, rtol=1e-12, atol=1e-12)
    w2 = rng.uniform(0, 1, (T, k))
    np.testing.assert_allclose(om.experts(x, idx, w + w2, wgu, wd),
                               y + om.experts(x, idx, w2, wgu, wd), rtol=1e-11, atol=1e-11)


def test_single_token_is_k_gemvs():
    rng = np.random.default_rng(6)
    H, I, E, k = 40, 24, 5, 3
    x = rng.standard_normal((1, H))
    wgu = rng.standard_normal((E, 2 * I, H))
    wd = rng.standard_normal((E, H, I))
    idx = np.array([[4, 0, 2]])
    w = np.array([[0.5, 0.3, 0.2]])
    y = om.experts(x, idx, w, wgu, wd)
    ref = np.zeros(H)
    for s in range(k):
        e = idx[0, s]
        gu = np.array([sum(wgu[e, r, c] * x[0, c] for c in range(H)) for r in range(2 * I)])
        a = gu[:I] / (1 + np.exp(-gu[:I])) * gu[I:]
        ref += w[0, s] * np.array([sum(wd[e, h, j] * a[j] for j in range(I)) for h in range(H)])
    np.testing.assert_allclose(y[0], ref, rtol=1e-10)


@pytest.mark.parametrize("algorithm", ["dense", "sparse"])
def test_block_matches_reference_restatement(algorithm):
    """The float64 oracle and the torch-CPU bf16 restatement of both reference algorithms
    agree on selection (modulo ties) and within bf16 tolerance on the output."""
    sh = MoEShape(512, 16, 4, 256, 128)
    w, g = make_layer(sh, seed=2)
    x = make_x(g, 48, 512)
    wn = layer_np(w)
    xn = to_np(x)
    shared = {"gate": wn["sh_gate"], "up": wn["sh_up"], "down": wn["sh_down"], "gate_w": wn["sh_gate_w"]}
    y, wt, idx = om.block_forward(xn, wn["gate"], wn["gate_up"], wn["down"], 4, shared=shared)
    sh_t = (w["sh_gate"], w["sh_up"], w["sh_down"], w["sh_gate_w"])
    yr, wr, ir = tr.block(x, w["gate"], w["gate_up"], w["down"], 4, sh=sh_t, algorithm=algorithm)
    same = (np.sort(ir.numpy(), 1) == np.sort(idx, 1)).all(1)
    assert same.mean() > 0.9
    # rows whose expert sets differ must be tie rows of the bf16 logits
    lg = om.router_logits(xn, wn["gate"])
    for t in np.nonzero(~same)[0]:
        zk = np.sort(lg[t])[::-1]
        assert zk[3] == zk[4], "selection differs without a tie at the top-k boundary"
    assert om.rel_err(to_np(yr)[same], y[same]) < 1.5e-2


# ---- fp8 -------------------------------------------------------------------------------------

def test_quant_blocks_closed_forms():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32)
    q, s = om.quant_blocks(w)
    assert s.shape == (2, 2, 3)
    blk = np.abs(w.reshape(2, 2, 128, 3, 128)).max(axis=(2, 4))
    np.testing.assert_array_equal(s, (blk / np.float32(448)).astype(np.float32))
    dq = om.dequant_blocks(q, s)
    # e4m3 has 3 mantissa bits: relative rounding error <= 2^-4 above the subnormal range
    sc = np.repeat(np.repeat(s, 128, 1), 128, 2)
    assert np.all(np.abs(dq - w) <= np.maximum(np.abs(w) * 2 ** -4, sc * 2 ** -10) + 1e-12)
    # the block maximum maps to exactly 448
    assert np.all(np.abs(codecs.e4m3_decode(q)).reshape(2, 2, 128, 3, 128).max(axis=(2, 4)) == 448)


def test_quant_exact_on_representable_values():
    vals = codecs.e4m3_values()[:127].astype(np.float32)
    rng = np.random.default_rng(9)
    a = rng.choice(vals, size=(3, 128)) * rng.choice([-1, 1], size=(3, 128))
    a[:, 0] = 448.0                                      # scale = 1 exactly
    q, s = om.quant_groups(a.astype(np.float32))
    assert np.all(s == 1.0)
    np.testing.assert_array_equal(om.dequant_groups(q, s), a)
    z, zs = om.quant_groups(np.zeros((1, 128), np.float32))
    assert zs[0, 0] == 1.0 and not z.any()


def test_fp8_oracle_close_to_bf16_oracle():
    sh = MoEShape(256, 8, 2, 128, 128)
    w, g = make_layer(sh, seed=3)
    x = make_x(g, 32, 256)
    wn = layer_np(w)
    xn = to_np(x)
    q = {}
    q["wgu_q"], q["wgu_s"] = om.quant_blocks(wn["gate_up"])
    q["wd_q"], q["wd_s"] = om.quant_blocks(wn["down"])
    for n in ("gate", "up", "down"):
        q[f"sh_{n}_q"], q[f"sh_{n}_s"] = om.quant_blocks(wn[f"sh_{n}"])
    q["sh_gate_w"] = wn["sh_gate_w"]
    y8, w8, i8 = om.block_forward_fp8(xn, wn["gate"], 2, q)
    shared = {"gate": wn["sh_gate"], "up": wn["sh_up"], "down": wn["sh_down"], "gate_w": wn["sh_gate_w"]}
    y, wt, idx = om.block_forward(xn, wn["gate"], wn["gate_up"], wn["down"], 2, shared=shared)
    np.testing.assert_array_equal(i8, idx)
    assert om.rel_err(y8, y) < 0.08


def test_zipf_bias_skews_load():
    g = torch.Generator().manual_seed(0)
    b = zipf_bias(g, 128).numpy()
    p = np.exp(b)
    assert abs(p.sum() - 1) < 1e-5
    assert sorted(p)[::-1][0] / sorted(p)[::-1][-1] > 300


# ---- residual add + RMSNorm ahead of the block ------------------------------------------------

def _torch_add_rmsnorm(hid, res, w, eps):
    """The reference's statements (qwen3_5.py:998, :1002 with Qwen3_5RMSNorm :48-55) in torch."""
    h = res + hid                                         # bf16 + bf16 -> bf16
    out = h.float()
    out = out * torch.rsqrt(out.pow(2).mean(-1, keepdim=True) + eps)
    out = out * (1.0 + w.float())
    return h, out.type_as(h)


@pytest.mark.parametrize("H,eps", [(2048, 1e-6), (1024, 1e-5), (256, 1e-6)])
def test_add_rmsnorm_matches_torch(H, eps):
    g = torch.Generator().manual_seed(H)
    hid = torch.randn((64, H), generator=g).to(torch.bfloat16)
    res = (torch.randn((64, H), generator=g) * 4).to(torch.bfloat16)
    w = (torch.randn(H, generator=g) * 0.1).to(torch.bfloat16)
    h_t, x_t = _torch_add_rmsnorm(hid, res, w, eps)
    h, x = om.add_rmsnorm(to_np(hid), to_np(res), to_np(w), eps)
    np.testing.assert_array_equal(codecs.bf16_bits(h), to_np(h_t.view(torch.int16)).view(np.uint16))
    d = np.abs(codecs.bf16_bits(x).astype(np.int32) - to_np(x_t.view(torch.int16)).view(np.uint16).astype(np.int32))
    assert d.max() <= 1, f"RMSNorm differs from torch by {d.max()} bf16 steps"
    assert (d == 0).mean() > 0.99


def test_add_rmsnorm_closed_forms():
    H = 512
    rng = np.random.default_rng(3)
    # a constant row normalises to its sign (eps = 0)
    c = codecs.bf16_round(rng.standard_normal(8).astype(np.float32) * 5)
    hid = np.repeat(c[:, None], H, axis=1).astype(np.float32)
    _, x = om.add_rmsnorm(hid, np.zeros_like(hid), np.zeros(H, np.float32), 0.0)
    np.testing.assert_array_equal(x, np.sign(hid))
    # eps = 0: scaling both inputs by a power of two leaves the output unchanged
    hid = codecs.bf16_round(rng.standard_normal((16, H)).astype(np.float32))
    res = codecs.bf16_round(rng.standard_normal((16, H)).astype(np.float32))
    w = codecs.bf16_round((rng.standard_normal(H) * 0.2).astype(np.float32))
    h1, x1 = om.add_rmsnorm(hid, res, w, 0.0)
    h8, x8 = om.add_rmsnorm(hid * 8, res * 8, w, 0.0)
    np.testing.assert_array_equal(h8, h1 * 8)
    np.testing.assert_array_equal(x8, x1)
    # weight 1 doubles the weight-0 output exactly; the residual add is the bf16 sum
    _, x0 = om.add_rmsnorm(hid, res, np.zeros(H, np.float32), 1e-6)
    _, x2 = om.add_rmsnorm(hid, res, np.ones(H, np.float32), 1e-6)
    np.testing.assert_array_equal(x2, 2 * x0)
    np.testing.assert_array_equal(h1, codecs.bf16_round((hid + res).astype(np.float32)))
