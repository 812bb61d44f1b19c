"""The layer on a caller's stream and under HIP graph capture: every kernel goes to the stream
it is handed, and the library itself never allocates, synchronises or records a memset, so a
captured graph replays bit-identically to eager calls."""
import numpy as np
import pytest
import torch

from layerbatch_amd.synth import SHAPES, MoEShape, make_layer, make_x
from oracle import moe as om
from tests import gpu_checks as gc
from tests.helpers import bf16_bits_of, to_np
from tests.test_gpu_fullsize import _Experts
from tests.test_gpu_parity import _block, _region

pytestmark = pytest.mark.gpu

SHAPE = MoEShape(1024, 16, 2, 512, 256)


# a layer with 64 experts, top-8 and a shared expert: 1600 (token, slot) pairs at T=200 take the
# single-workgroup permutation with two entries per thread, the shared expert 7 slices
WIDE = MoEShape(1024, 64, 8, 256, 256)


def _setup(gpu, T, seed=3, fp8=False, shape=SHAPE):
    w, g = make_layer(shape, seed=seed)
    blk = _block(shape, {k: v.to(gpu) for k, v in w.items()}, gpu)
    if fp8:
        blk.quantize_fp8_()
    xs = [make_x(g, T, shape.hidden_size).to(gpu) for _ in range(3)]
    return blk, xs


# streaming GEMMs, LDS-tiled GEMMs; bf16 and fp8 weights
@pytest.mark.parametrize("T,fp8,shape", [(40, False, SHAPE), (512, False, SHAPE), (40, True, SHAPE),
                                         (512, True, SHAPE), (200, False, WIDE)])
def test_graph_replay_matches_eager(gpu, T, fp8, shape):
    blk, xs = _setup(gpu, T, fp8=fp8, shape=shape)
    ws_e = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=gpu)
    ws_g = torch.empty_like(ws_e)
    static_x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            blk(static_x, workspace=ws_g)              # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = blk(static_x, workspace=ws_g)
    for rep in range(6):
        x = xs[rep % 3]
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        y_e = blk(x, workspace=ws_e)                     # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static_y, y_e), f"replay {rep} differs from the eager result"


def test_side_stream_matches_default_stream(gpu):
    T = 300
    blk, xs = _setup(gpu, T, seed=5)
    y0 = blk(xs[0])
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        x = xs[0].clone()
        ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device=gpu)
        y1 = blk(x, workspace=ws)
    s.synchronize()
    assert torch.equal(y0, y1)


def test_repeated_calls_are_deterministic(gpu):
    T = 1024
    blk, xs = _setup(gpu, T, seed=7)
    ys = [blk(xs[1]) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[1], ys[2])


# the toy layer at the engine's small buckets, and the Qwen3-30B-A3B layer up to the engine's
# largest bucket, 512 (model_runner.py:1466, :1480; max_num_seqs 512, config.py:183): from 448 on
# (28 tokens per expert) its replays run the LDS-tiled GEMMs. The replays of the buckets named
# last are also checked against the float64 oracle.
@pytest.mark.parametrize("shape,buckets,checked", [
    (SHAPE, [1, 2, 4, 8, 16, 32, 48, 64], [48]),
    (SHAPES["qwen3-30b-a3b"], [1, 8, 16, 64, 128, 256, 384, 448, 512], [128, 256, 448, 512])])
def test_decode_bucket_graphs(gpu, shape, buckets, checked):
    """The engine's decode capture (model_runner.py:1463-1507): one graph per batch bucket,
    captured from the largest bucket down in a shared memory pool, all reading slices of one
    static input buffer whose rows past the live batch are zeros (padded rows are routed like
    real ones), and one workspace for all of them. Every bucket's replay matches an eager call
    on the same slice bit for bit; the checked buckets' replays also match the oracle: exact
    selection from the replay's own logits, the output within 1e-2 on every row."""
    H, E, k = shape.hidden_size, shape.num_experts, shape.top_k
    w, g = make_layer(shape, seed=11, device=gpu)
    blk = _block(shape, w, gpu)
    static_x = torch.zeros((max(buckets), H), dtype=torch.bfloat16, device=gpu)
    outputs = torch.zeros_like(static_x)
    # one workspace, sized for the largest bucket, shared by every graph
    ws = torch.empty(blk.workspace_size(max(buckets)), dtype=torch.uint8, device=gpu)
    graphs, pool = {}, None
    for bs in reversed(buckets):
        outputs[:bs] = blk(static_x[:bs], workspace=ws)          # warm-up
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool):
            outputs[:bs] = blk(static_x[:bs], workspace=ws)
        if pool is None:
            pool = graph.pool()
        graphs[bs] = graph
        torch.cuda.synchronize()
    for bs in buckets:
        print(f"bucket {bs}: replay", flush=True)
        live = max(1, bs - 1 - bs // 4)                          # a partly filled bucket
        x = make_x(g, live, H, device=gpu)
        static_x.zero_()
        static_x[:live] = x
        graphs[bs].replay()
        torch.cuda.synchronize()
        if bs in checked:
            print(f"bucket {bs}: replay against the oracle", flush=True)
            logits = to_np(_region(blk, ws, bs, "logits", torch.bfloat16, (bs, E)))
            topw = _region(blk, ws, bs, "topk_w", torch.bfloat16, (bs, k))
            idx = to_np(_region(blk, ws, bs, "topk_idx", torch.int32, (bs, k)))
            _, idx_ref = gc.check_route(idx, bf16_bits_of(topw), logits, None, k)
            xn = to_np(static_x[:bs])
            y_ref = om.experts(xn, idx_ref, to_np(topw), _Experts(w["gate_up"]), _Experts(w["down"]))
            if shape.shared_expert_intermediate_size:
                gsh = om.shared_gate(xn, to_np(w["sh_gate_w"])).astype(np.float64)
                y_ref = y_ref + gsh[:, None] * om.shared_expert(
                    xn, to_np(w["sh_gate"]), to_np(w["sh_up"]), to_np(w["sh_down"]))
            gc.check_output(to_np(outputs[:bs]), y_ref, gc.TOL_BF16)
        y_e = blk(static_x[:bs].clone())
        torch.cuda.synchronize()
        assert torch.equal(outputs[:bs], y_e), f"bucket {bs} replay differs from the eager result"


# Two decoder layers' blocks (different weights) on two streams, as LayerBatch decode runs group
# A's unit t on la_stream while group B's unit t-1 runs on fa_stream (layer_batch.py:175-212):
# decode-sized batches (weight-streaming GEMMs, the permutation inside gate_up), prefill-sized
# ones (LDS-tiled GEMMs with the persistent gate_up's work queues in the workspace), the fp8
# E=512 layer with its shared expert, and fp8 prefill batches large enough for the persistent
# fp8 gate_up.
@pytest.mark.parametrize("name,Ta,Tb,fp8", [("qwen3-30b-a3b", 48, 80, False),
                                          ("qwen3-30b-a3b", 1024, 2048, False),
                                          ("qwen3-next-e512", 128, 600, True),
                                          ("qwen3-30b-a3b", 8192, 6000, True)])
def test_two_streams_overlapping_calls(gpu, name, Ta, Tb, fp8):
    """Calls on two streams with one workspace each and no synchronisation between the
    streams give, bit for bit, the outputs of the same calls made one after another."""
    print(f"two streams: {name} T={Ta} and T={Tb} fp8={fp8}", flush=True)
    shape = SHAPES[name]
    blks, xs = [], []
    for seed, T in ((31, Ta), (32, Tb)):
        w, g = make_layer(shape, seed=seed, device=gpu)
        blk = _block(shape, w, gpu)
        if fp8:
            blk.quantize_fp8_()
        del w
        blks.append(blk)
        xs.append([make_x(g, T, shape.hidden_size, device=gpu) for _ in range(4)])
    ref = [[blk(x) for x in xl] for blk, xl in zip(blks, xs)]          # one after another
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [torch.empty(blk.workspace_size(xl[0].shape[0]), dtype=torch.uint8, device=gpu)
           for blk, xl in zip(blks, xs)]
    outs = [[torch.empty_like(x) for x in xl] for xl in xs]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rnd in range(2):
        for i in range(4):                      # interleaved issue: both streams always busy
            for j in (0, 1):
                with torch.cuda.stream(streams[j]):
                    outs[j][i].copy_(blks[j](xs[j][i], workspace=wss[j]))
    for s in streams:
        s.synchronize()
    for j in (0, 1):
        for i in range(4):
            assert torch.equal(outs[j][i], ref[j][i]), f"stream {j} call {i} differs"

