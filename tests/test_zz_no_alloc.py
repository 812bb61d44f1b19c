"""lbmoe_forward_static (the entry point that allocates nothing): through the C ABI, its output
equals lbmoe_forward's bit for bit, on consecutive calls that reuse the library's one device
workspace with a smaller batch second, and calls past the workspace's limit are refused on the
host before anything is enqueued."""
import ctypes
import os
import subprocess
import sys

import pytest
import torch

from layerbatch_amd import _lib
from layerbatch_amd.synth import SHAPES, MoEShape, make_layer, make_x
from tests.test_gpu_parity import _block


def _forward_ws(blk, x):
    L = blk.layer()
    T = x.shape[0]
    ws = torch.empty(_lib.workspace_size(L, T), dtype=torch.uint8, device=x.device)
    y = torch.empty_like(x)
    _lib.check(_lib.lib().lbmoe_forward(ctypes.byref(L), _lib.ptr(x), T, _lib.ptr(y), _lib.ptr(ws),
                                        ws.numel(), _lib.stream_of(x.device)), "lbmoe_forward")
    return y


def _forward_static(blk, x):
    L = blk.layer()
    y = torch.empty_like(x)
    _lib.check(_lib.lib().lbmoe_forward_static(ctypes.byref(L), _lib.ptr(x), x.shape[0], _lib.ptr(y),
                                               _lib.stream_of(x.device)), "lbmoe_forward_static")
    return y


# the Qwen3-30B-A3B layer at decode sizes (streaming GEMMs), the E=512 layer with a shared expert
# (bf16 and fp8), and a batch past the tiled-GEMM switch of a small layer; second call smaller
@pytest.mark.gpu
@pytest.mark.parametrize("shape,T1,T2,fp8", [(SHAPES["qwen3-30b-a3b"], 256, 16, False),
                                             (SHAPES["qwen3-next-e512"], 128, 3, False),
                                             (SHAPES["qwen3-next-e512"], 128, 1, True),
                                             (MoEShape(1024, 16, 2, 512, 256), 1500, 200, False)])
def test_static_matches_workspace_forward(gpu, shape, T1, T2, fp8):
    print(f"static workspace: shape {shape} T {T1} then {T2} fp8 {fp8}", flush=True)
    w, g = make_layer(shape, seed=T1 + T2, device=gpu)
    blk = _block(shape, w, gpu)
    if fp8:
        blk.quantize_fp8_()
    for T in (T1, T2):
        x = make_x(g, T, shape.hidden_size, device=gpu)
        y_ref = _forward_ws(blk, x)
        y = _forward_static(blk, x)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"T={T}: static-workspace output differs from lbmoe_forward"
        # a second static call finds the first one's intermediates in the array: same output
        y2 = _forward_static(blk, x)
        torch.cuda.synchronize()
        assert torch.equal(y2, y_ref), f"T={T}: repeated static call differs"


def test_static_limit_refused_on_host(lbmoe):
    """A batch whose workspace exceeds LBMOE_STATIC_WORKSPACE_BYTES: -7, checked before any
    device access (fake pointers are never dereferenced)."""
    L = _lib.LbmoeLayer()
    L.hidden_size, L.num_experts, L.top_k = 2048, 128, 8
    L.moe_intermediate_size, L.shared_intermediate_size = 768, 0
    L.gate_weight, L.gate_up_proj, L.down_proj = 0x1000, 0x2000, 0x3000
    n = ctypes.c_size_t(0)
    T = 1
    while True:
        _lib.check(lbmoe.lbmoe_workspace_size(ctypes.byref(L), T, ctypes.byref(n)), "ws")
        if n.value > _lib.LBMOE_STATIC_WORKSPACE_BYTES:
            break
        T *= 2
    p = ctypes.c_void_p(0x4000)
    assert lbmoe.lbmoe_forward_static(ctypes.byref(L), p, T, p, None) == _lib.LBMOE_ERR_STATIC_LIMIT
    assert "static workspace" in lbmoe.lbmoe_status_string(_lib.LBMOE_ERR_STATIC_LIMIT).decode()
    bad = _lib.LbmoeLayer()
    bad.hidden_size = 1000
    assert lbmoe.lbmoe_forward_static(ctypes.byref(bad), p, 4, p, None) == -2


# Run in a fresh process, so that the library's first lbmoe_forward_static call on the device
# (which looks up the array's address) happens inside the graph capture.
_CAPTURE_SCRIPT = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from layerbatch_amd import _lib
from layerbatch_amd.synth import MoEShape, make_layer, make_x
from tests.test_gpu_parity import _block
dev = torch.device("cuda:0")
shape = MoEShape(1024, 16, 2, 512, 256)
w, g = make_layer(shape, seed=4, device=dev)
blk = _block(shape, w, dev)
L = blk.layer()
lib = _lib.lib()
T = 64
static_x = make_x(g, T, 1024, device=dev)
static_y = torch.empty_like(static_x)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = lib.lbmoe_forward_static(ctypes.byref(L), _lib.ptr(static_x), T, _lib.ptr(static_y),
                                  _lib.stream_of(dev))
_lib.check(rc, "lbmoe_forward_static under capture")
ws = torch.empty(_lib.workspace_size(L, T), dtype=torch.uint8, device=dev)
for rep in range(3):
    x = make_x(g, T, 1024, device=dev)
    static_x.copy_(x)
    graph.replay()
    torch.cuda.synchronize()
    y = torch.empty_like(x)
    _lib.check(lib.lbmoe_forward(ctypes.byref(L), _lib.ptr(x), T, _lib.ptr(y), _lib.ptr(ws),
                                 ws.numel(), _lib.stream_of(dev)), "lbmoe_forward")
    torch.cuda.synchronize()
    assert torch.equal(static_y, y), f"replay {rep} differs from lbmoe_forward"
    print(f"replay {rep}: equal to lbmoe_forward", flush=True)
print("CAPTURE_OK", flush=True)
"""


@pytest.mark.gpu
def test_static_first_call_inside_graph_capture(gpu):
    """The entry point is meant for code under graph capture: its first call on a device,
    which looks up the array's address, is made inside torch.cuda.graph capture in a fresh
    process; three replays, with eager lbmoe_forward calls between them, each equal
    lbmoe_forward's output bit for bit."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("static workspace: first call inside graph capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_SCRIPT, root], capture_output=True,
                       text=True, timeout=110, cwd=root)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-3000:])
