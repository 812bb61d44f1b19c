"""ctypes binding of liblbmoe.so (the C ABI declared in include/lbmoe.h).

torch is imported first so that the library's libamdhip64 dependency resolves to the HIP
runtime torch already loaded (same SONAME): device pointers and streams from torch are then
valid in the library. The library must have been built in-tree
(``python -m layerbatch_amd.build``); there is no fallback implementation.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblbmoe.so")

LBMOE_PROFILE_EVENTS = 7
PROFILE_STAGES = ("router_logits", "route_topk", "permute", "gate_up", "down", "combine")
LBMOE_STATIC_WORKSPACE_BYTES = 64 << 20
LBMOE_ERR_STATIC_LIMIT = -7
LBMOE_W_BF16 = 0
LBMOE_W_FP8_E4M3 = 1

REGIONS = {
    "logits": 0, "topk_idx": 1, "topk_w": 2, "shared_gate": 3, "counts": 4, "offsets": 5,
    "perm_tok": 6, "perm_slot": 7, "inv": 8, "act": 9, "expert_out": 10, "xn": 11,
}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t


class LbmoeLayer(ctypes.Structure):
    """struct lbmoe_layer (include/lbmoe.h)."""
    _fields_ = [
        ("hidden_size", _i32), ("num_experts", _i32), ("top_k", _i32),
        ("moe_intermediate_size", _i32), ("shared_intermediate_size", _i32),
        ("weight_dtype", _i32),
        ("gate_weight", _p), ("logit_bias", _p), ("gate_up_proj", _p), ("down_proj", _p),
        ("gate_up_scale", _p), ("down_scale", _p),
        ("shared_gate_proj", _p), ("shared_up_proj", _p), ("shared_down_proj", _p),
        ("shared_expert_gate", _p),
        ("shared_gate_scale", _p), ("shared_up_scale", _p), ("shared_down_scale", _p),
        ("gate_up_tiled", _p), ("down_tiled", _p),
        ("shared_gate_up_tiled", _p), ("shared_down_tiled", _p),
    ]


_PL = ctypes.POINTER(LbmoeLayer)
_SIGS = {
    "lbmoe_status_string": (ctypes.c_char_p, [_i32]),
    "lbmoe_abi_version": (_i32, []),
    "lbmoe_check_layer": (_i32, [_PL]),
    "lbmoe_workspace_size": (_i32, [_PL, _i64, ctypes.POINTER(_sz)]),
    "lbmoe_workspace_region": (_i32, [_PL, _i64, _i32, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "lbmoe_forward": (_i32, [_PL, _p, _i64, _p, _p, _sz, _p]),
    "lbmoe_pack_weights": (_i32, [_PL, _p, _p, _p, _p, _p]),
    "lbmoe_forward_profiled": (_i32, [_PL, _p, _i64, _p, _p, _sz, _p, ctypes.POINTER(_p), _i32]),
    "lbmoe_forward_static": (_i32, [_PL, _p, _i64, _p, _p]),
    "lbmoe_forward_norm": (_i32, [_PL, _p, _p, _p, ctypes.c_float, _i64, _p, _p, _p, _sz, _p]),
    "lbmoe_router_logits": (_i32, [_PL, _p, _i64, _p, _p]),
    "lbmoe_route": (_i32, [_PL, _p, _p, _i64, _p, _i32, _p, _p, _p]),
    "lbmoe_permute_workspace_size": (_i32, [_i64, _i32, _i32, ctypes.POINTER(_sz)]),
    "lbmoe_permute": (_i32, [_p, _i32, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "lbmoe_experts": (_i32, [_PL, _p, _p, _i32, _p, _i64, _p, _p, _sz, _p]),
    "lbmoe_dense_mlp_workspace_size": (_i32, [_i32, _i32, _i32, _i64, ctypes.POINTER(_sz)]),
    "lbmoe_dense_mlp": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _p, _i64, _p, _p, _sz, _p]),
    "lbmoe_quantize_fp8_blocks": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p]),
}

EXPORTED = tuple(_SIGS)
_lib = None


def lib():
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m layerbatch_amd.build`")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(status, what):
    if status != 0:
        msg = lib().lbmoe_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def workspace_size(layer, T):
    n = _sz(0)
    check(lib().lbmoe_workspace_size(ctypes.byref(layer), T, ctypes.byref(n)), "lbmoe_workspace_size")
    return n.value


def workspace_region(layer, T, name):
    off, nb = _sz(0), _sz(0)
    check(lib().lbmoe_workspace_region(ctypes.byref(layer), T, REGIONS[name], ctypes.byref(off),
                                       ctypes.byref(nb)), "lbmoe_workspace_region")
    return off.value, nb.value
