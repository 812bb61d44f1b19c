"""GPU parity of every stage of the HIP MoE layer against the CPU oracle (through the C ABI)."""
import ctypes

import numpy as np
import pytest
import torch

from layerbatch_amd import _lib
from layerbatch_amd.moe import Qwen3_5SparseMoeBlock
from layerbatch_amd.synth import MoEShape, SHAPES, make_layer, make_x, zipf_bias
from oracle import moe as om
from oracle.codecs import bf16_bits
from tests import gpu_checks as gc
from tests.helpers import bf16_bits_of, layer_np, scale_blocks_pow2, scale_groups_pow2, to_np

pytestmark = pytest.mark.gpu


def _block(shape, w, device):
    H, E, k, I, Is = (shape.hidden_size, shape.num_experts, shape.top_k,
                      shape.moe_intermediate_size, shape.shared_expert_intermediate_size)
    blk = Qwen3_5SparseMoeBlock(H, E, k, I, Is).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        blk.gate.weight.copy_(w["gate"])
        blk.experts.gate_up_proj.copy_(w["gate_up"])
        blk.experts.down_proj.copy_(w["down"])
        if Is:
            blk.shared_expert.gate_proj.weight.copy_(w["sh_gate"])
            blk.shared_expert.up_proj.weight.copy_(w["sh_up"])
            blk.shared_expert.down_proj.weight.copy_(w["sh_down"])
            blk.shared_expert_gate.weight.copy_(w["sh_gate_w"])
    return blk


def _region(blk, ws, T, name, dtype, shape):
    off, nb = _lib.workspace_region(blk.layer(), T, name)
    n = int(np.prod(shape))
    esz = torch.empty((), dtype=dtype).element_size()
    assert n * esz <= nb
    return ws[off:off + n * esz].view(dtype).view(shape)


def _run_and_check(shape, T, device, seed=0, bias=None, gen_device="cpu", sample=None,
                   pack=False, gate_rows_mod=None):
    w, g = make_layer(shape, seed=seed, device=gen_device)
    if gate_rows_mod:
        # router row e repeats row e mod gate_rows_mod: groups of experts get identical logits,
        # so most selections are decided by the tie rule (lower expert index first)
        w["gate"] = w["gate"][torch.arange(shape.num_experts) % gate_rows_mod].contiguous()
    x = make_x(g, T, shape.hidden_size, device=gen_device)
    wd = {k_: v.to(device) for k_, v in w.items()}
    blk = _block(shape, wd, device)
    if pack:
        blk.pack_tiled_()
    if bias is not None:
        blk.gate.logit_bias = bias.to(device)
    xd = x.to(device)
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=device)
    y = blk(xd, workspace=ws)
    torch.cuda.synchronize()
    E, k = shape.num_experts, shape.top_k
    logits = _region(blk, ws, T, "logits", torch.bfloat16, (T, E))
    idx = _region(blk, ws, T, "topk_idx", torch.int32, (T, k))
    topw = _region(blk, ws, T, "topk_w", torch.bfloat16, (T, k))
    wn = layer_np(w)
    xn = to_np(x)
    gc.check_logits(bf16_bits_of(logits), xn, wn["gate"])
    bn = None if bias is None else bias.cpu().numpy()
    w_ref, idx_ref = gc.check_route(to_np(idx), bf16_bits_of(topw), to_np(logits), bn, k)
    V = T * k
    gc.check_permutation(idx_ref, E,
                         to_np(_region(blk, ws, T, "counts", torch.int32, (E,))),
                         to_np(_region(blk, ws, T, "offsets", torch.int32, (E + 1,))),
                         to_np(_region(blk, ws, T, "perm_tok", torch.int32, (V,))),
                         to_np(_region(blk, ws, T, "perm_slot", torch.int32, (V,))),
                         to_np(_region(blk, ws, T, "inv", torch.int32, (T, k))))
    rows = np.arange(T) if sample is None else np.unique(
        np.random.default_rng(seed).choice(T, size=min(sample, T), replace=False))
    y_ref = gc.block_reference(xn[rows], wn, idx_ref[rows], to_np(topw)[rows], k,
                               shared=True if shape.shared_expert_intermediate_size else None)
    return gc.check_output(to_np(y)[rows], y_ref, gc.TOL_BF16)


def test_block_small_layer(gpu):
    """H=1024, E=16, top-2, I=512, T=64 (seed 0)."""
    _run_and_check(SHAPES["small-h1024-e16"], 64, gpu)


@pytest.mark.parametrize("T", [1, 3, 17, 128, 300])
def test_block_small_layer_sizes(gpu, T):
    _run_and_check(SHAPES["small-h1024-e16"], T, gpu, seed=T)


def test_block_with_shared_expert(gpu):
    shape = MoEShape(1024, 32, 4, 256, 384)
    _run_and_check(shape, 40, gpu, seed=3)


# Shapes off the benchmark grid: E not a multiple of the 16-expert router tile, odd k, H with
# 12 and 32 k-blocks (split-K plans of 6 waves, and of 8 waves x 2 chunks each), widths of 3
# and 5 k-blocks, Is != I; streaming (small T) and LDS-tiled (large T) GEMMs, and H = 640, which
# the tiled GEMMs do not take, streaming 50 tokens per expert (four token tiles per pass).
@pytest.mark.parametrize("shape,T", [(MoEShape(1536, 20, 3, 384, 640), 1),
                                     (MoEShape(1536, 20, 3, 384, 640), 37),
                                     (MoEShape(1536, 20, 3, 384, 640), 260),
                                     (MoEShape(4096, 24, 4, 256, 0), 5),
                                     (MoEShape(4096, 24, 4, 256, 0), 60),
                                     (MoEShape(640, 40, 5, 128, 128), 90),
                                     (MoEShape(640, 40, 5, 128, 128), 400)])
def test_block_odd_shapes(gpu, shape, T):
    _run_and_check(shape, T, gpu, seed=T + shape.num_experts)


# a router bias; the second case adds a shared expert (the gate inside the selection) with
# E = 48, three router tiles of 16 experts
@pytest.mark.parametrize("shape,T", [(MoEShape(1024, 64, 6, 256, 0), 200),
                                     (MoEShape(768, 48, 4, 256, 256), 150)])
def test_block_with_bias(gpu, shape, T):
    g = torch.Generator().manual_seed(11)
    _run_and_check(shape, T, gpu, seed=5, bias=zipf_bias(g, shape.num_experts))


@pytest.mark.parametrize("T", [3072, 5000])
def test_block_prefill_tiled_zipf(gpu, T):
    """Prefill-sized batch (tiled GEMMs) with Zipf-skewed expert loads: empty experts,
    a hot expert with thousands of tokens, ragged tails."""
    shape = MoEShape(1024, 32, 4, 256, 0)
    g = torch.Generator().manual_seed(21)
    _run_and_check(shape, T, gpu, seed=7, bias=zipf_bias(g, 32), sample=96)


def test_block_prefill_persistent_gate_up(gpu):
    """A batch whose gate_up table has at least 6 entries per CU (H=1024, E=64, top-8, I=768,
    T=8192: 1944 entries), so gate_up runs as the persistent work-queue kernel: wide, narrow and
    tiny tiles, Zipf-skewed loads, and empty experts, whose queue entries are idle."""
    shape = MoEShape(1024, 64, 8, 768, 0)
    T, E, k, I = 8192, 64, 8, 768
    g = torch.Generator().manual_seed(23)
    bias = zipf_bias(g, E)
    _run_and_check(shape, T, gpu, seed=13, bias=bias, sample=96)
    # every row of the gate_up output (act, in expert-sorted order), so that an item the queues
    # skipped or ran twice shows, against float32 products on the same device
    w, gx = make_layer(shape, seed=13)
    x = make_x(gx, T, shape.hidden_size).to(gpu)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    blk.gate.logit_bias = bias.to(gpu)
    ws = torch.full((blk.workspace_size(T),), 255, dtype=torch.uint8, device=gpu)  # NaN act
    blk(x, workspace=ws)
    torch.cuda.synchronize()
    offsets = _region(blk, ws, T, "offsets", torch.int32, (E + 1,)).cpu().tolist()
    perm_tok = _region(blk, ws, T, "perm_tok", torch.int32, (T * k,)).long()
    act = _region(blk, ws, T, "act", torch.bfloat16, (T * k, I)).float()
    ref = torch.empty_like(act)
    for e in range(E):
        a, b = offsets[e], offsets[e + 1]
        if b > a:
            wt = w["gate_up"][e].to(gpu).float().t().contiguous()
            h = x[perm_tok[a:b]].float() @ wt
            ref[a:b] = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
    assert offsets[E] == T * k
    gc.check_output(act.cpu().numpy(), ref.cpu().numpy(), gc.TOL_BF16)


# Batches that select experts inside the tiled router (E <= 128, T >= 1024, tiled GEMMs):
# 16 experts per lane (E = 128) under a Zipf bias, an expert count that is no multiple of 8
# with a ragged last 64-token block, k > 8 (a lane's second slot), and a shared expert whose
# gate the same kernel computes. Below 256 blocks of 64 tokens the router's k range is split
# over 2 (H = 512) or 4 (H >= 1024) workgroups whose fp32 sums the selection kernel adds: the
# H = 2048 cases take 4 splits with 8 (E = 64) and 16 (E = 128) experts per lane.
@pytest.mark.parametrize("shape,T,zipf", [(MoEShape(1024, 128, 8, 256, 0), 2048, True),
                                          (MoEShape(512, 100, 6, 256, 0), 1100, False),
                                          (MoEShape(512, 96, 12, 256, 0), 1024, False),
                                          (MoEShape(512, 80, 10, 256, 384), 1200, True),
                                          (MoEShape(2048, 64, 6, 256, 0), 1500, False),
                                          (MoEShape(2048, 128, 8, 256, 256), 3000, True)])
def test_block_prefill_route_in_router(gpu, shape, T, zipf):
    bias = None
    if zipf:
        bias = zipf_bias(torch.Generator().manual_seed(shape.num_experts), shape.num_experts)
    _run_and_check(shape, T, gpu, seed=T, bias=bias, sample=96)


# Ties between whole experts: router rows repeated, no bias, so selection runs on packed keys
# (every score a bf16 value) and equal logits are ordered by expert index: selection inside the
# tiled router (T >= 1024, E <= 128: 8-lane groups), inside the decode router (16 < T < 1024,
# E <= 128), the selection kernel of E = 512 prefill and decode, and the small-batch kernels.
@pytest.mark.parametrize("shape,T,mod", [(MoEShape(512, 128, 8, 256, 0), 2048, 16),
                                         (MoEShape(512, 128, 8, 256, 0), 200, 11),
                                         (MoEShape(512, 100, 6, 256, 0), 1100, 7),
                                         (MoEShape(512, 512, 10, 256, 256), 1024, 50),
                                         (MoEShape(512, 512, 10, 256, 256), 100, 3),
                                         (MoEShape(512, 128, 8, 256, 0), 3, 5),
                                         (MoEShape(512, 128, 8, 256, 0), 12, 9)])
def test_route_tied_router_rows(gpu, shape, T, mod):
    _run_and_check(shape, T, gpu, seed=T + mod, sample=96, gate_rows_mod=mod)


# Tiled-layout copies of the expert weights (lbmoe_pack_weights): the prefill GEMMs read them
# instead of the checkpoint tensors and give the same output bit for bit, and the oracle agrees.
# Cases: the router-fused path under a Zipf bias (wide, narrow and tiny tiles), a shared expert
# narrower than the routed ones (Is != I), and I = 384 (three gate_up weight tiles).
@pytest.mark.parametrize("shape,T,zipf", [(MoEShape(1024, 128, 8, 256, 0), 2048, True),
                                          (MoEShape(512, 16, 2, 256, 128), 1500, False),
                                          (MoEShape(768, 64, 4, 384, 256), 1000, True)])
def test_block_prefill_packed_weights(gpu, shape, T, zipf):
    bias = None
    if zipf:
        bias = zipf_bias(torch.Generator().manual_seed(shape.num_experts), shape.num_experts)
    _run_and_check(shape, T, gpu, seed=T + 1, bias=bias, sample=96, pack=True)
    w, g = make_layer(shape, seed=T, device="cpu")
    x = make_x(g, T, shape.hidden_size, device="cpu").to(gpu)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    if bias is not None:
        blk.gate.logit_bias = bias.to(gpu)
    y0 = blk(x)
    blk.pack_tiled_()
    assert blk.layer().gate_up_tiled and blk.layer().down_tiled
    y1 = blk(x)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_block_prefill_tiled_shared(gpu):
    """Tiled GEMMs with a shared expert of a different width (Is != I)."""
    shape = MoEShape(512, 16, 2, 256, 384)
    _run_and_check(shape, 1500, gpu, seed=8, sample=96)


def test_dense_reduction_e1_k1(gpu):
    """k = 1, E = 1: the block is a dense SwiGLU MLP with weight 1."""
    shape = MoEShape(256, 1, 1, 256, 0)
    _run_and_check(shape, 33, gpu, seed=9)


@pytest.mark.parametrize("T,k,E,ib", [(1, 1, 1, 4), (7, 2, 16, 8), (128, 8, 128, 4),
                                      (129, 8, 128, 8), (1000, 10, 512, 4), (8192, 8, 128, 4),
                                      (3000, 7, 1000, 8), (0, 4, 16, 4), (100, 10, 1024, 8),
                                      (32, 32, 64, 4),
                                      # one workgroup, 2 and 4 entries per thread; 4 needs E <= 512
                                      (256, 8, 128, 4), (200, 10, 1024, 8), (300, 10, 512, 8),
                                      (409, 10, 512, 4), (250, 10, 1000, 4)])
def test_permute_exact(gpu, lbmoe, T, k, E, ib):
    rng = np.random.default_rng(T * 131 + k)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if T else np.zeros((0, k), np.int64)
    if T > 10:
        idx[3, 0] = E          # out of range: dropped, inv = -1
        idx[5, k - 1] = -1
    dt = torch.int32 if ib == 4 else torch.int64
    d_idx = torch.tensor(idx, dtype=dt, device=gpu).reshape(T, k)
    V = T * k
    counts = torch.empty(E, dtype=torch.int32, device=gpu)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    pt = torch.full((max(V, 1),), -7, dtype=torch.int32, device=gpu)
    ps = torch.full((max(V, 1),), -7, dtype=torch.int32, device=gpu)
    inv = torch.empty((max(V, 1),), dtype=torch.int32, device=gpu)
    n = ctypes.c_size_t(0)
    _lib.check(lbmoe.lbmoe_permute_workspace_size(T, k, E, ctypes.byref(n)), "ws")
    ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=gpu)
    _lib.check(lbmoe.lbmoe_permute(_lib.ptr(d_idx), ib, T, k, E, _lib.ptr(counts), _lib.ptr(offsets),
                                   _lib.ptr(pt), _lib.ptr(ps), _lib.ptr(inv), _lib.ptr(ws), n.value,
                                   _lib.stream_of(gpu)), "lbmoe_permute")
    torch.cuda.synchronize()
    c_ref, o_ref, pt_ref, ps_ref, inv_ref = _perm_ref_with_drops(idx, E)
    np.testing.assert_array_equal(counts.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(offsets.cpu().numpy(), o_ref)
    nv = int(o_ref[-1])
    np.testing.assert_array_equal(pt.cpu().numpy()[:nv], pt_ref)
    np.testing.assert_array_equal(ps.cpu().numpy()[:nv], ps_ref)
    if V:
        np.testing.assert_array_equal(inv.cpu().numpy()[:V].reshape(T, k), inv_ref)


def _perm_ref_with_drops(idx, E):
    """Oracle permutation where out-of-range ids are dropped (inv = -1)."""
    T, k = idx.shape
    valid = (idx >= 0) & (idx < E)
    e_sm = idx.T.reshape(-1)
    v_ok = valid.T.reshape(-1)
    order = [v for v in np.argsort(np.where(v_ok, e_sm, E), kind="stable") if v_ok[v]]
    order = np.asarray(order, np.int64)
    counts = np.bincount(e_sm[v_ok], minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    inv_sm = np.full(T * k, -1, np.int64)
    inv_sm[order] = np.arange(order.size)
    return counts, offsets, order % max(T, 1), order // max(T, 1), inv_sm.reshape(k, T).T


def test_router_module_returns_reference_types(gpu):
    shape = SHAPES["small-h1024-e16"]
    w, g = make_layer(shape, device="cpu")
    x = make_x(g, 64, shape.hidden_size).to(gpu)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    tw, ti = blk.gate(x)
    assert tw.dtype == torch.bfloat16 and ti.dtype == torch.int64
    assert tuple(tw.shape) == (64, 2) and tuple(ti.shape) == (64, 2)
    logits = to_np(blk.gate.logits(x))
    gc.check_route(ti.cpu().numpy(), bf16_bits_of(tw), logits, None, 2)
    # the experts module takes the router's int64 indices (qwen3_5.py:901-902)
    y = blk.experts(x, ti, tw)
    wn = layer_np(w)
    y_ref = om.experts(to_np(x), ti.cpu().numpy(), to_np(tw), wn["gate_up"], wn["down"])
    gc.check_output(to_np(y), y_ref, gc.TOL_BF16)


# The experts module at one and two tokens, where int32 indices take the fused down + combine
# kernel (int64 ones the separate kernels), with expert ids outside [0, E): such pairs are
# dropped (inv = -1) and add nothing, as expert-parallel callers rely on.
@pytest.mark.parametrize("T,idx_dtype", [(1, torch.int32), (2, torch.int32), (2, torch.int64)])
def test_experts_small_batch_dropped_pairs(gpu, T, idx_dtype):
    shape = MoEShape(512, 16, 4, 256, 0)
    w, g = make_layer(shape, seed=21, device="cpu")
    x = make_x(g, T, shape.hidden_size)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    idx = np.array([[3, 15, -1, 7], [16, 3, 0, 9]][:T], dtype=np.int64)
    tw = (torch.rand((T, 4), generator=g) + 0.1).to(torch.bfloat16)
    y = blk.experts(x.to(gpu), torch.from_numpy(idx).to(idx_dtype).to(gpu), tw.to(gpu))
    ok = (idx >= 0) & (idx < shape.num_experts)
    wn = layer_np(w)
    y_ref = om.experts(to_np(x), np.where(ok, idx, 0), np.where(ok, to_np(tw), 0.0),
                       wn["gate_up"], wn["down"])
    gc.check_output(to_np(y), y_ref, gc.TOL_BF16)


def test_shared_expert_mlp_module(gpu):
    shape = MoEShape(1024, 8, 2, 128, 384)
    w, g = make_layer(shape, seed=4)
    x = make_x(g, 50, 1024)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    out = blk.shared_expert(x.to(gpu))
    wn = layer_np(w)
    ref = om.shared_expert(to_np(x), wn["sh_gate"], wn["sh_up"], wn["sh_down"])
    gc.check_output(to_np(out), ref, gc.TOL_BF16)


def test_zero_tokens(gpu):
    shape = SHAPES["small-h1024-e16"]
    w, _ = make_layer(shape)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    y = blk(torch.empty((0, 1024), dtype=torch.bfloat16, device=gpu))
    assert y.shape == (0, 1024)


def test_cpu_tensor_raises(gpu):
    shape = SHAPES["small-h1024-e16"]
    w, _ = make_layer(shape)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    with pytest.raises(RuntimeError):
        blk(torch.zeros((4, 1024), dtype=torch.bfloat16))


def test_host_checks_before_any_launch(gpu):
    """Weights left on the CPU, a workspace of the wrong dtype or size: refused on the host."""
    shape = SHAPES["small-h1024-e16"]
    w, g = make_layer(shape)
    x = make_x(g, 8, shape.hidden_size).to(gpu)
    cpu_blk = _block(shape, w, "cpu")
    with pytest.raises(RuntimeError, match="device"):
        cpu_blk(x)
    with pytest.raises(RuntimeError, match="device"):
        cpu_blk.experts(x, torch.zeros((8, 2), dtype=torch.int64, device=gpu),
                        torch.zeros((8, 2), dtype=torch.bfloat16, device=gpu))
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    n = blk.workspace_size(8)
    with pytest.raises(RuntimeError, match="uint8"):
        blk(x, workspace=torch.empty(n, dtype=torch.float32, device=gpu))
    with pytest.raises(RuntimeError):
        blk(x, workspace=torch.empty(n - 1, dtype=torch.uint8, device=gpu))
    y = blk(x, workspace=torch.empty(n, dtype=torch.uint8, device=gpu))   # the exact size works
    torch.cuda.synchronize()
    assert y.shape == x.shape
    # sizes the C ABI cannot see: an input of another width, a norm weight, a router bias or a
    # shared-expert weight of the wrong size
    wide = make_x(g, 8, shape.hidden_size + 128).to(gpu)
    with pytest.raises(RuntimeError, match="channels"):
        blk(wide)
    with pytest.raises(RuntimeError, match="channels"):
        blk.experts(wide, torch.zeros((8, 2), dtype=torch.int64, device=gpu),
                    torch.zeros((8, 2), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(RuntimeError, match="channels"):
        blk.gate(wide)
    with pytest.raises(RuntimeError, match="channels"):
        blk.forward_norm(wide, wide, _Norm(torch.zeros(shape.hidden_size + 128, dtype=torch.bfloat16,
                                                       device=gpu), 1e-6))
    with pytest.raises(RuntimeError, match="norm.weight"):
        blk.forward_norm(x, x, _Norm(torch.zeros(shape.hidden_size // 2, dtype=torch.bfloat16,
                                                 device=gpu), 1e-6))
    blk.gate.logit_bias = torch.zeros(shape.num_experts - 1, dtype=torch.float32, device=gpu)
    with pytest.raises(RuntimeError, match="logit_bias"):
        blk(x)
    blk.gate.logit_bias = None
    sh_shape = MoEShape(1024, 16, 2, 512, 256)
    sw, _ = make_layer(sh_shape, seed=1)
    sblk = _block(sh_shape, {k_: v.to(gpu) for k_, v in sw.items()}, gpu)
    with torch.no_grad():
        sblk.shared_expert.down_proj.weight = torch.nn.Parameter(
            torch.zeros((1024, 128), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(RuntimeError, match="shared_expert.down_proj"):
        sblk(x)
    with pytest.raises(RuntimeError, match="shared_expert.down_proj"):
        sblk.shared_expert(x)
    with pytest.raises(RuntimeError, match="channels"):
        sblk.shared_expert(wide)


@pytest.mark.parametrize("T,E,k,levels,bias", [(300, 128, 8, 3, False), (257, 512, 10, 4, False),
                                               (64, 1000, 32, 2, True), (100, 64, 32, 5, False),
                                               (77, 200, 7, 1, True), (129, 16, 2, 2, False)])
def test_route_ties(gpu, T, E, k, levels, bias):
    """Selection on logits with only a few distinct values, so that most selections are decided
    by the tie rule (lower expert index first), within and across lanes; with -inf and NaN
    logits and an optional bias that itself has ties."""
    from layerbatch_amd._lib import LbmoeLayer
    rng = np.random.default_rng(T * 7 + E)
    z = rng.integers(0, levels, size=(T, E)).astype(np.float32) * 0.5 - 1.0
    z[0, :-1] = -np.inf                     # one finite logit, the rest tie at -inf
    z[1, ::3] = np.nan                      # NaN logits are never preferred
    zb = torch.tensor(z).to(torch.bfloat16)
    L = LbmoeLayer()
    L.hidden_size, L.num_experts, L.top_k, L.moe_intermediate_size = 128, E, k, 128
    b_np = None
    if bias:
        b_np = (rng.integers(0, 2, size=E) * 0.25).astype(np.float32)
        b = torch.tensor(b_np, device=gpu)
        L.logit_bias = b.data_ptr()
    logits = zb.to(gpu)
    idx = torch.empty((T, k), dtype=torch.int32, device=gpu)
    w = torch.empty((T, k), dtype=torch.bfloat16, device=gpu)
    _lib.check(_lib.lib().lbmoe_route(ctypes.byref(L), _lib.ptr(logits), None, T, _lib.ptr(idx), 4,
                                      _lib.ptr(w), None, _lib.stream_of(gpu)), "lbmoe_route")
    torch.cuda.synchronize()
    ln = to_np(zb)
    ln = np.where(np.isnan(ln), -np.inf, ln)   # the oracle's view of a NaN logit
    gc.check_route(to_np(idx), bf16_bits_of(w), ln, b_np, k)


class _Norm(torch.nn.Module):
    """Stand-in for the layer's post_attention_layernorm (Qwen3_5RMSNorm: weight [H], eps)."""

    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.eps = eps


# T <= 16 runs the norm inside the router kernel, larger T as its own kernel ahead of the router
@pytest.mark.parametrize("shape_name,T", [("small-h1024-e16", 40), ("qwen3-30b-a3b", 128),
                                          ("qwen3-30b-a3b", 1), ("qwen3-30b-a3b", 16),
                                          ("small-h1024-e16", 13), ("qwen3-next-e512", 1100)])
def test_forward_norm(gpu, shape_name, T):
    """Residual add + RMSNorm + block (qwen3_5.py:998-1004): the new residual is the bf16 sum
    bit for bit, the block input within one bf16 step of the oracle's Qwen3_5RMSNorm, and the
    output equals the plain block on that input bit for bit (decode T: norm fused into the
    router kernel; T >= 1024: separate norm kernel)."""
    shape = SHAPES[shape_name]
    H = shape.hidden_size
    w, g = make_layer(shape, seed=T, device=gpu)
    blk = _block(shape, w, gpu)
    hid = make_x(g, T, H, device=gpu)
    res = (make_x(g, T, H, device=gpu).float() * 3).to(torch.bfloat16)
    norm = _Norm((make_x(g, 1, H, device=gpu)[0].float() * 0.1).to(torch.bfloat16), 1e-6)
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=gpu)
    y, new_res = blk.forward_norm(hid, res, norm, workspace=ws)
    torch.cuda.synchronize()
    h_ref, x_ref = om.add_rmsnorm(to_np(hid), to_np(res), to_np(norm.weight), 1e-6)
    np.testing.assert_array_equal(to_np(new_res), h_ref)
    xn = _region(blk, ws, T, "xn", torch.bfloat16, (T, H)).clone()
    d = np.abs(bf16_bits_of(xn).astype(np.int32) - bf16_bits(x_ref).astype(np.int32))
    assert d.max() <= 1, f"block input differs from the oracle's RMSNorm by {d.max()} bf16 steps"
    y_plain = blk(xn)
    torch.cuda.synchronize()
    assert torch.equal(y, y_plain)


def test_forward_norm_rejects_in_place_residual(gpu, lbmoe):
    shape = SHAPES["small-h1024-e16"]
    w, g = make_layer(shape, seed=2, device=gpu)
    blk = _block(shape, w, gpu)
    L = blk.layer()
    hid = make_x(g, 8, 1024, device=gpu)
    res = make_x(g, 8, 1024, device=gpu)
    nw = torch.zeros(1024, dtype=torch.bfloat16, device=gpu)
    y = torch.empty_like(hid)
    ws = torch.empty(blk.workspace_size(8), dtype=torch.uint8, device=gpu)
    st = lbmoe.lbmoe_forward_norm(ctypes.byref(L), _lib.ptr(hid), _lib.ptr(res), _lib.ptr(nw), 1e-6, 8,
                                  _lib.ptr(y), _lib.ptr(res), _lib.ptr(ws), ws.numel(), _lib.stream_of(gpu))
    assert st == -2


# rows per expert chosen so that the tiled GEMMs see every token-tile class boundary: a group's
# last rows r after its full 256-row tiles are r <= 64 (one 64-row tile), 64 < r <= 128 (one
# 128-row tile) or r > 128 (one more 256-row tile)
TILE_BOUNDARY_COUNTS = [0, 1, 63, 64, 65, 127, 128, 129, 130, 255, 256, 257, 320, 384, 385, 512]


def _boundary_routing(seed):
    """k = 1 routing with exactly TILE_BOUNDARY_COUNTS[e] tokens on expert e, tokens shuffled,
    and random bf16 weights."""
    counts = np.array(TILE_BOUNDARY_COUNTS)
    T = int(counts.sum())
    rng = np.random.default_rng(seed)
    idx = rng.permutation(np.repeat(np.arange(len(counts)), counts)).reshape(T, 1)
    tw = torch.from_numpy(rng.uniform(0.05, 1.0, size=(T, 1))).to(torch.bfloat16)
    return T, idx.astype(np.int64), tw


# H = 512, I = 256: gate_up 8 (bf16) / 4 (fp8) k-tiles, down 4 / 2; H = 1024, I = 768: 16 / 8
# and 12 / 6, so that every ring refills several times in both GEMMs (the fp8 case with
# patterned block and group scales)
@pytest.mark.parametrize("fp8,H,I", [(False, 512, 256), (True, 512, 256), (False, 1024, 768),
                                     (True, 1024, 768)])
def test_experts_tile_class_boundaries(gpu, fp8, H, I):
    shape = MoEShape(H, len(TILE_BOUNDARY_COUNTS), 1, I, 0)
    T, idx, tw = _boundary_routing(31)
    w, g = make_layer(shape, seed=12)
    x = make_x(g, T, shape.hidden_size)
    if fp8 and H > 512:
        w = {k_: (scale_blocks_pow2(v) if k_ in ("gate_up", "down") else v) for k_, v in w.items()}
        x = scale_groups_pow2(x)
    blk = _block(shape, {k_: v.to(gpu) for k_, v in w.items()}, gpu)
    if fp8:
        blk.quantize_fp8_()
    y = blk.experts(x.to(gpu), torch.from_numpy(idx).to(gpu), tw.to(gpu))
    torch.cuda.synchronize()
    wn = layer_np(w)
    rows = np.arange(T)                 # every row: each tile's first and last rows matter
    if fp8:
        ex = blk.experts
        y_ref = om.experts_fp8(to_np(x)[rows], idx[rows], to_np(tw)[rows], ex.gate_up_q.cpu().numpy(),
                               ex.gate_up_scale.cpu().numpy(), ex.down_q.cpu().numpy(),
                               ex.down_scale.cpu().numpy())
        gc.check_output(to_np(y)[rows], y_ref, gc.TOL_FP8)
    else:
        y_ref = om.experts(to_np(x)[rows], idx[rows], to_np(tw)[rows], wn["gate_up"], wn["down"])
        gc.check_output(to_np(y)[rows], y_ref, gc.TOL_BF16)


# (E, T) per router tile shape: 128 experts x 64 tokens; 256 x 64; 256 x 128 once its tiles fill
# the chip (T / 128 * ceil(E / 256) >= 256), also with a partial last expert tile
@pytest.mark.parametrize("E,T", [(128, 1024), (512, 4096), (1024, 8192), (700, 11000)])
def test_router_logits_tiled_shapes(gpu, E, T):
    H = 512
    g = torch.Generator().manual_seed(E + T)
    wg = (torch.randn((E, H), generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    blk = Qwen3_5SparseMoeBlock(H, E, 2, 256, 0).to(device=gpu, dtype=torch.bfloat16)
    with torch.no_grad():
        blk.gate.weight.copy_(wg.to(gpu))
    logits = blk.gate.logits(x.to(gpu))
    torch.cuda.synchronize()
    rows = np.unique(np.random.default_rng(E).choice(T, size=min(T, 1500), replace=False))
    gc.check_logits(bf16_bits_of(logits)[rows], to_np(x)[rows], to_np(wg))


# small batches (up to 16 tokens for E <= 128, up to 4 otherwise) route and permute in one
# kernel (one wave per token, then the one-workgroup permutation), and up to 4 tokens with
# T*k <= 64 inside every gate_up workgroup instead (bf16): every expert-count class of the
# route, with and without a shared expert, with the compact workgroup rows (T*k < E) and
# without them, and batches just past the limits; the routing regions are checked too
@pytest.mark.parametrize("shape,T", [(MoEShape(512, 1024, 10, 256, 0), 4),
                                     (MoEShape(512, 128, 8, 256, 0), 2),
                                     (MoEShape(512, 64, 16, 256, 256), 4),
                                     (MoEShape(512, 16, 8, 256, 0), 2),
                                     (MoEShape(512, 300, 8, 256, 256), 3),
                                     (MoEShape(512, 1024, 10, 256, 0), 16),
                                     (MoEShape(512, 64, 16, 256, 256), 16),
                                     (MoEShape(512, 200, 4, 256, 0), 1),
                                     (MoEShape(512, 300, 8, 256, 256), 7),
                                     (MoEShape(512, 128, 8, 256, 0), 13),
                                     (MoEShape(512, 128, 8, 256, 0), 17)])
def test_block_small_batch_route_permute(gpu, shape, T):
    _run_and_check(shape, T, gpu, seed=13)
