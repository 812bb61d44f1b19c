"""GPU parity at the measured workloads' full sizes.

Every routing decision is checked exactly: router logits on sampled rows against the exact dot
products, selection on all rows against the oracle's selection from the GPU's own logits, and
the whole permutation. The layer output is checked against the float64 oracle on every row up
to 256 tokens, and above that on at least 256 random rows plus every row of the tiles where
indexing mistakes would show: the hottest expert's first and last 256-token tiles, and the last
rows of experts whose remainders take a 64-token and a 128-token tile. The oracle only ever
touches the experts those rows selected, which are copied off the GPU one at a time.
"""
import numpy as np
import pytest
import torch

from layerbatch_amd.synth import SHAPES, make_layer, make_x, zipf_bias
from oracle import moe as om
from tests import gpu_checks as gc
from tests.helpers import bf16_bits_of, scale_blocks_pow2, scale_groups_pow2, to_np
from tests.test_gpu_parity import _block, _region

pytestmark = pytest.mark.gpu


class _Experts:
    """Per-expert view of a device tensor [E, ...] for the oracle: expert e is copied to the
    host when first indexed (bf16 as float32, other dtypes as they are; the last one is kept)."""

    def __init__(self, t):
        self.t = t
        self.shape = tuple(t.shape)
        self._e, self._a = None, None

    def __getitem__(self, e):
        e = int(e)
        if e != self._e:
            a = self.t[e]
            self._e, self._a = e, (a.float() if a.dtype == torch.bfloat16 else a).cpu().numpy()
        return self._a


WIDE, NARROW, TINY = 256, 128, 64      # token-tile widths of the LDS-tiled GEMMs


def tile_rows(counts, offsets, perm_tok):
    """Tokens of the tiles where a tiling mistake would show first: the hottest expert's first
    and last wide tiles (its last rows included), and the last rows of one expert whose
    remainder after its wide tiles takes a tiny tile and of one whose remainder takes a narrow
    tile (preferring experts that also have wide tiles)."""
    counts = np.asarray(counts, np.int64)
    pos = []

    def tokens(e, lo, hi):
        return perm_tok[offsets[e] + np.arange(lo, hi)]

    hot = int(np.argmax(counts))
    n = int(counts[hot])
    if n:
        pos.append(tokens(hot, 0, min(WIDE, n)))
        pos.append(tokens(hot, max(0, (n - 1) // WIDE * WIDE - WIDE), n))
    rem = counts % WIDE
    for lo, hi in ((1, TINY), (TINY + 1, NARROW)):
        cand = np.nonzero((rem >= lo) & (rem <= hi))[0]
        if cand.size:
            e = int(cand[np.argmax(counts[cand])])
            pos.append(tokens(e, int(counts[e] - rem[e]), int(counts[e])))
    return np.unique(np.concatenate(pos)) if pos else np.zeros(0, np.int64)


def _run_full(shape, T, device, seed, zipf, sample=256, fp8=False, patterned=False):
    w, g = make_layer(shape, seed=seed, device=device)
    x = make_x(g, T, shape.hidden_size, device=device)
    if patterned:
        # every 128x128 weight block scale and every (token, 128-channel) activation scale
        # differs from its neighbours by a power of two, so a kernel reading a neighbouring
        # block's or group's scale lands far outside the tolerance
        for k_ in ("gate_up", "down", "sh_gate", "sh_up", "sh_down"):
            if k_ in w:
                w[k_] = scale_blocks_pow2(w[k_])
        x = scale_groups_pow2(x)
    blk = _block(shape, w, device)
    if zipf:
        blk.gate.logit_bias = zipf_bias(g, shape.num_experts, device=device)
    if fp8:
        blk.quantize_fp8_()
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=device)
    y = blk(x, workspace=ws)
    torch.cuda.synchronize()
    E, k = shape.num_experts, shape.top_k
    xn = to_np(x)
    logits = to_np(_region(blk, ws, T, "logits", torch.bfloat16, (T, E)))
    bias = None if blk.gate.logit_bias is None else blk.gate.logit_bias.cpu().numpy()
    topw = _region(blk, ws, T, "topk_w", torch.bfloat16, (T, k))
    idx = to_np(_region(blk, ws, T, "topk_idx", torch.int32, (T, k)))
    _, idx_ref = gc.check_route(idx, bf16_bits_of(topw), logits, bias, k)
    V = T * k
    counts = to_np(_region(blk, ws, T, "counts", torch.int32, (E,)))
    offsets = to_np(_region(blk, ws, T, "offsets", torch.int32, (E + 1,)))
    perm_tok = to_np(_region(blk, ws, T, "perm_tok", torch.int32, (V,)))
    gc.check_permutation(idx_ref, E, counts, offsets, perm_tok,
                         to_np(_region(blk, ws, T, "perm_slot", torch.int32, (V,))),
                         to_np(_region(blk, ws, T, "inv", torch.int32, (T, k))))
    if T <= sample:
        rows = np.arange(T)
    else:
        rand = np.random.default_rng(seed).choice(T, size=sample, replace=False)
        rows = np.unique(np.concatenate([rand, tile_rows(counts, offsets, perm_tok)]))
    print(f"  T={T}: logits and output checked on {rows.size} rows", flush=True)
    gc.check_logits(bf16_bits_of(_region(blk, ws, T, "logits", torch.bfloat16, (T, E)))[rows],
                    xn[rows], to_np(w["gate"]))
    tw = to_np(topw)[rows]
    shared = shape.shared_expert_intermediate_size > 0
    if fp8:
        ex = blk.experts
        y_ref = om.experts_fp8(xn[rows], idx_ref[rows], tw, _Experts(ex.gate_up_q),
                               _Experts(ex.gate_up_scale), _Experts(ex.down_q),
                               _Experts(ex.down_scale))
        if shared:
            se = blk.shared_expert
            q = [a.cpu().numpy() for n in ("gate", "up", "down") for a in se.q[n]]
            gsh = om.shared_gate(xn[rows], to_np(w["sh_gate_w"])).astype(np.float64)
            y_ref = y_ref + gsh[:, None] * om.shared_expert_fp8(xn[rows], *q)
        tol = gc.TOL_FP8
        if patterned:
            # the pattern's power at this shape: the oracle itself, handed every weight block's
            # k-neighbour scale, lands far outside the tolerance (on 16 of the rows)
            r16 = rows[:16]
            su, sd = ex.gate_up_scale.cpu().numpy(), ex.down_scale.cpu().numpy()
            y16 = om.experts_fp8(xn[r16], idx_ref[r16], to_np(topw)[r16], _Experts(ex.gate_up_q), su,
                                 _Experts(ex.down_q), sd)
            shifted = om.experts_fp8(xn[r16], idx_ref[r16], to_np(topw)[r16],
                                     _Experts(ex.gate_up_q), np.roll(su, 1, axis=-1),
                                     _Experts(ex.down_q), np.roll(sd, 1, axis=-1))
            assert om.rel_err(shifted, y16) > 10 * tol
    else:
        y_ref = om.experts(xn[rows], idx_ref[rows], tw, _Experts(w["gate_up"]), _Experts(w["down"]))
        if shared:
            gsh = om.shared_gate(xn[rows], to_np(w["sh_gate_w"])).astype(np.float64)
            y_ref = y_ref + gsh[:, None] * om.shared_expert(
                xn[rows], to_np(w["sh_gate"]), to_np(w["sh_up"]), to_np(w["sh_down"]))
        tol = gc.TOL_BF16
    return gc.check_output(to_np(y)[rows], y_ref, tol)


@pytest.mark.parametrize("T", [16, 64, 128, 256])
def test_fullsize_decode_qwen3_30b(gpu, T):
    """Qwen3-30B-A3B layer (H=2048, E=128, top-8, I=768), decode batches, every row."""
    _run_full(SHAPES["qwen3-30b-a3b"], T, gpu, seed=1, zipf=False)


# either side of the kernel switches: one token tile (up to 8 tokens per expert) / two / the
# LDS-tiled GEMMs (from 28), and the single-workgroup permutation (up to 4096 entries)
@pytest.mark.parametrize("T", [1, 136, 448, 449, 513])
def test_fullsize_qwen3_30b_path_boundaries(gpu, T):
    _run_full(SHAPES["qwen3-30b-a3b"], T, gpu, seed=T, zipf=False)


@pytest.mark.parametrize("T", [16, 1100])
def test_fullsize_e512_streaming_shared_slices(gpu, T):
    """E=512 with the shared expert's token passes spread over extra workgroup rows (T=1100:
    streaming with two token tiles, 35 passes on 16 slices)."""
    _run_full(SHAPES["qwen3-next-e512"], T, gpu, seed=T, zipf=False)


def test_fullsize_prefill_qwen3_30b_zipf(gpu):
    """The same layer at T=8192 with the Zipf(1.2) router bias: empty experts, a hot expert
    with thousands of tokens, wide and narrow tiles."""
    _run_full(SHAPES["qwen3-30b-a3b"], 8192, gpu, seed=0, zipf=True)


@pytest.mark.parametrize("T", [128, 4096])
def test_fullsize_e512_shared(gpu, T):
    """Qwen3-Next-style layer: H=2048, E=512, top-10, I=512, shared expert Is=512."""
    _run_full(SHAPES["qwen3-next-e512"], T, gpu, seed=2, zipf=False)


@pytest.mark.parametrize("T", [128, 16384])
def test_fullsize_e512_fp8(gpu, T):
    """The E=512 layer with e4m3 weights and activations (per-block fp32 scales)."""
    _run_full(SHAPES["qwen3-next-e512"], T, gpu, seed=3, zipf=False, fp8=True)


@pytest.mark.parametrize("T", [128, 16384])
def test_fullsize_e512_fp8_scale_patterns(gpu, T):
    """The E=512 fp8 layer at its full shape (16 gate_up and 4 down k-tiles of 128, the shared
    expert's own scale rows) with patterned block and group scales: the streaming GEMMs at
    T=128, the LDS-tiled ones at T=16384."""
    print(f"fp8 E=512 patterned scales T={T}", flush=True)
    _run_full(SHAPES["qwen3-next-e512"], T, gpu, seed=T + 9, zipf=False, fp8=True, patterned=True)
