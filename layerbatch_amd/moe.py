"""Drop-in MoE modules backed by the gfx950 HIP library (liblbmoe.so).

Same class names, constructor arguments, parameter names, shapes and return values as the
reference's MoE classes in nanovllm/models/qwen3_5.py:

* Qwen3_5TopKRouter       qwen3_5.py:754-774   forward(x) -> (top_k_weights bf16, top_k_indices int64)
* Qwen3_5Experts          qwen3_5.py:781-874   forward(x, idx, w) -> [T,H]
* Qwen3_5SparseMoeBlock   qwen3_5.py:881-905   forward(x) -> [T,H]
* Qwen3_5SharedExpertMLP  qwen3_5.py:908-917   forward(x) -> [T,H]

so the reference's weight loader (nanovllm/utils/loader.py:16-61, plain ``param.data.copy_``)
and decoder layer (qwen3_5.py:956-962, :1004) use them unchanged. Differences, all deliberate:

* One algorithm for every batch size (the reference switches between a dense gather+bmm for
  decode and a per-expert loop for prefill on ``get_context().is_prefill``,
  qwen3_5.py:808-813); the flag is not read.
* Tie order of equal router probabilities is (descending logit, ascending expert index);
  torch.topk leaves it implementation-defined.
* ``shared_expert_intermediate_size == 0`` builds no shared expert (the reference always
  builds one).
* ``Qwen3_5TopKRouter.logit_bias`` (default None) is an optional fp32 [E] tensor added to
  the upcast logits before the softmax; it is not a checkpoint parameter.
* ``Qwen3_5SparseMoeBlock.quantize_fp8_()`` converts the expert and shared-expert weights to
  OCP e4m3fn with per-128x128-block fp32 scales (no counterpart in the reference);
  ``load_fp8_`` installs codes and scales computed elsewhere (layerbatch_amd/checkpoint.py).
* ``Qwen3_5SparseMoeBlock.forward_norm(hidden, residual, norm)`` runs the decoder layer's
  residual add, post_attention_layernorm and the block in one call (qwen3_5.py:998-1004),
  returning (block output, new residual).

Every forward runs on the tensor's CUDA (HIP) device on the current stream, enqueues HIP
kernels only (no host synchronisation), and raises RuntimeError for CPU tensors, wrong dtypes
or a missing library build.
"""
import ctypes
import warnings

import torch
from torch import nn

from . import _lib
from ._lib import LbmoeLayer, check, lib, ptr

__all__ = ["Qwen3_5TopKRouter", "Qwen3_5Experts", "Qwen3_5SharedExpertMLP",
           "Qwen3_5SparseMoeBlock"]


def _require(t, name, dtype=torch.bfloat16, ndim=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} is on {t.device}: the MoE layer runs only on a gfx950 GPU")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise RuntimeError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _require_shape(t, shape, name):
    """The C ABI sees only pointers: a tensor of another shape would be read (or written) out
    of bounds, so every size is checked here before any launch."""
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _require_width(x, H, name="hidden_states"):
    if x.shape[1] != H:
        raise RuntimeError(f"{name} has {x.shape[1]} channels, the layer's hidden_size is {H}")


def _device_tensors(module):
    """Every tensor a module's kernels read: parameters and installed fp8 codes and scales."""
    for p in module.parameters():
        yield p
    for m in module.modules():
        for name in ("gate_up_q", "gate_up_scale", "down_q", "down_scale", "logit_bias"):
            t = getattr(m, name, None)
            if isinstance(t, torch.Tensor):
                yield t
        q = getattr(m, "q", None)
        if isinstance(q, dict):
            for codes, scales in q.values():
                yield codes
                yield scales


def _same_device(module, device):
    """The kernels dereference the module's tensors on the input's device: refuse a mix."""
    for t in _device_tensors(module):
        if t.device != device:
            raise RuntimeError(f"a {type(module).__name__} tensor is on {t.device}, the input on "
                               f"{device}: move the module to the input's device")


def _workspace(layer, T, device, workspace=None):
    """The caller's workspace (checked: uint8, contiguous, on the input's device; the library
    checks its size), or a new one from torch's caching allocator."""
    if workspace is None:
        return torch.empty(_lib.workspace_size(layer, T), dtype=torch.uint8, device=device)
    _require(workspace, "workspace", torch.uint8)
    if workspace.device != device:
        raise RuntimeError(f"workspace is on {workspace.device}, the input on {device}")
    return workspace


class Qwen3_5TopKRouter(nn.Module):
    """Router: softmax over bf16 logits, top-k, renormalise, cast to bf16 (qwen3_5.py:754-774).

    Weight: gate.weight [num_experts, hidden_size].
    """

    def __init__(self, num_experts: int, hidden_size: int, top_k: int):
        super().__init__()
        self.top_k = top_k
        self.num_experts = num_experts
        self.weight = nn.Parameter(torch.zeros(num_experts, hidden_size))
        self.logit_bias = None

    def _layer(self):
        _require(self.weight, "gate.weight", ndim=2)
        E, H = self.weight.shape
        if E != self.num_experts:
            raise RuntimeError(f"gate.weight has {E} rows, the router has {self.num_experts} experts")
        L = LbmoeLayer()
        L.hidden_size, L.num_experts, L.top_k = H, E, self.top_k
        L.moe_intermediate_size = 256           # routed-expert sizes are unused by the router
        L.gate_weight = self.weight.data_ptr()
        if self.logit_bias is not None:
            _require(self.logit_bias, "logit_bias", torch.float32, 1)
            _require_shape(self.logit_bias, (E,), "logit_bias")
            L.logit_bias = self.logit_bias.data_ptr()
        return L

    def logits(self, hidden_states):
        """bf16 router logits [T, E] (the F.linear of qwen3_5.py:769)."""
        _require(hidden_states, "hidden_states", ndim=2)
        _require(self.weight, "gate.weight", ndim=2)
        _require_width(hidden_states, self.weight.shape[1])
        _same_device(self, hidden_states.device)
        T = hidden_states.shape[0]
        out = torch.empty((T, self.num_experts), dtype=torch.bfloat16, device=hidden_states.device)
        L = self._layer()
        with torch.cuda.device(hidden_states.device):
            check(lib().lbmoe_router_logits(ctypes.byref(L), ptr(hidden_states), T, ptr(out),
                                            _lib.stream_of(hidden_states.device)),
                  "lbmoe_router_logits")
        return out

    def forward(self, hidden_states: torch.Tensor):
        logits = self.logits(hidden_states)
        T = hidden_states.shape[0]
        dev = hidden_states.device
        w = torch.empty((T, self.top_k), dtype=torch.bfloat16, device=dev)
        idx = torch.empty((T, self.top_k), dtype=torch.int64, device=dev)
        L = self._layer()
        with torch.cuda.device(dev):
            check(lib().lbmoe_route(ctypes.byref(L), ptr(logits), None, T, ptr(idx), 8, ptr(w),
                                    None, _lib.stream_of(dev)), "lbmoe_route")
        return w, idx


def _stamp(tensors):
    """Identity of the tensors a tiled copy was packed from: storage address and version
    counter (bumped by every in-place write, e.g. load_state_dict's copy_)."""
    return tuple((t.data_ptr(), t._version) for t in tensors)


def _tiled_current(owner, sources, what):
    """Whether owner's tiled copies still match their source tensors. Stale copies (the
    weights were replaced or written since pack_tiled_) are dropped with a warning: the
    layer then streams the checkpoint tensors, whose results are identical."""
    if owner.gate_up_tiled is None:
        return False
    if _stamp(sources) == owner.tiled_stamp:
        return True
    warnings.warn(f"{what} changed after pack_tiled_(): its tiled copies are dropped; call "
                  "pack_tiled_() again to restore the faster prefill GEMMs", RuntimeWarning,
                  stacklevel=3)
    owner.gate_up_tiled = owner.down_tiled = owner.tiled_stamp = None
    return False


class Qwen3_5Experts(nn.Module):
    """Fused expert weights stored as 3-D tensors (qwen3_5.py:781-800).

    - experts.gate_up_proj  [num_experts, 2 * moe_intermediate_size, hidden_size]
    - experts.down_proj     [num_experts, hidden_size, moe_intermediate_size]
    """

    def __init__(self, num_experts: int, hidden_size: int, moe_intermediate_size: int):
        super().__init__()
        self.num_experts = num_experts
        self.hidden_size = hidden_size
        self.intermediate_size = moe_intermediate_size
        self.gate_up_proj = nn.Parameter(
            torch.empty(num_experts, 2 * moe_intermediate_size, hidden_size))
        self.down_proj = nn.Parameter(
            torch.empty(num_experts, hidden_size, moe_intermediate_size))
        self.weight_dtype = _lib.LBMOE_W_BF16
        self.gate_up_q = self.gate_up_scale = self.down_q = self.down_scale = None
        self.gate_up_tiled = self.down_tiled = None     # pack_tiled_ copies (bf16 only)
        self.tiled_stamp = None                         # _stamp of their source tensors

    def fill_layer(self, L):
        L.num_experts = self.num_experts
        L.hidden_size = self.hidden_size
        L.moe_intermediate_size = self.intermediate_size
        L.weight_dtype = self.weight_dtype
        if self.weight_dtype == _lib.LBMOE_W_FP8_E4M3:
            L.gate_up_proj = self.gate_up_q.data_ptr()
            L.down_proj = self.down_q.data_ptr()
            L.gate_up_scale = self.gate_up_scale.data_ptr()
            L.down_scale = self.down_scale.data_ptr()
        else:
            E, H, I = self.num_experts, self.hidden_size, self.intermediate_size
            _require(self.gate_up_proj, "experts.gate_up_proj", ndim=3)
            _require(self.down_proj, "experts.down_proj", ndim=3)
            _require_shape(self.gate_up_proj, (E, 2 * I, H), "experts.gate_up_proj")
            _require_shape(self.down_proj, (E, H, I), "experts.down_proj")
            L.gate_up_proj = self.gate_up_proj.data_ptr()
            L.down_proj = self.down_proj.data_ptr()
            if _tiled_current(self, (self.gate_up_proj, self.down_proj), "experts weights"):
                L.gate_up_tiled = self.gate_up_tiled.data_ptr()
                L.down_tiled = self.down_tiled.data_ptr()

    def forward(self, hidden_states, top_k_indices, top_k_weights):
        _require(hidden_states, "hidden_states", ndim=2)
        _require(top_k_indices, "top_k_indices", None, 2)
        _require(top_k_weights, "top_k_weights", torch.bfloat16, 2)
        _require_width(hidden_states, self.hidden_size)
        if top_k_indices.dtype not in (torch.int64, torch.int32):
            raise RuntimeError(f"top_k_indices must be int64 or int32, got {top_k_indices.dtype}")
        T, k = top_k_indices.shape
        if hidden_states.shape[0] != T or tuple(top_k_weights.shape) != (T, k):
            raise RuntimeError("hidden_states / top_k_indices / top_k_weights disagree on [T, k]")
        dev = hidden_states.device
        if top_k_indices.device != dev or top_k_weights.device != dev:
            raise RuntimeError("hidden_states, top_k_indices and top_k_weights must share a device")
        _same_device(self, dev)
        L = LbmoeLayer()
        self.fill_layer(L)
        L.top_k = k
        dev = hidden_states.device
        y = torch.empty_like(hidden_states)
        ws = _workspace(L, T, dev)
        with torch.cuda.device(dev):
            check(lib().lbmoe_experts(ctypes.byref(L), ptr(hidden_states), ptr(top_k_indices),
                                      top_k_indices.element_size(), ptr(top_k_weights), T, ptr(y),
                                      ptr(ws), ws.numel(), _lib.stream_of(dev)), "lbmoe_experts")
        return y


class Qwen3_5SharedExpertMLP(nn.Module):
    """Dense SwiGLU MLP: down(silu(gate_proj x) * up_proj x) (qwen3_5.py:908-917)."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        self.weight_dtype = _lib.LBMOE_W_BF16
        self.q = None   # fp8: dict name -> (codes, scales)
        self.gate_up_tiled = self.down_tiled = None     # pack_tiled_ copies (bf16 only)
        self.tiled_stamp = None                         # _stamp of their source tensors

    def tiled_sources(self):
        return (self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight)

    def _ptrs(self):
        if self.weight_dtype == _lib.LBMOE_W_FP8_E4M3:
            q = self.q
            return ([q[n][0].data_ptr() for n in ("gate", "up", "down")],
                    [q[n][1].data_ptr() for n in ("gate", "up", "down")])
        Is, H = self.gate_proj.weight.shape
        for n, m, shape in (("gate_proj", self.gate_proj, (Is, H)), ("up_proj", self.up_proj, (Is, H)),
                            ("down_proj", self.down_proj, (H, Is))):
            _require(m.weight, f"shared_expert.{n}.weight", ndim=2)
            _require_shape(m.weight, shape, f"shared_expert.{n}.weight")
        return ([self.gate_proj.weight.data_ptr(), self.up_proj.weight.data_ptr(),
                 self.down_proj.weight.data_ptr()], [None, None, None])

    def fill_layer(self, L):
        L.shared_intermediate_size = self.gate_proj.weight.shape[0]
        (g, u, d), (gs, us, ds) = self._ptrs()
        L.shared_gate_proj, L.shared_up_proj, L.shared_down_proj = g, u, d
        L.shared_gate_scale, L.shared_up_scale, L.shared_down_scale = gs, us, ds
        if (self.weight_dtype == _lib.LBMOE_W_BF16
                and _tiled_current(self, self.tiled_sources(), "shared_expert weights")):
            L.shared_gate_up_tiled = self.gate_up_tiled.data_ptr()
            L.shared_down_tiled = self.down_tiled.data_ptr()

    def forward(self, x):
        _require(x, "x", ndim=2)
        _same_device(self, x.device)
        T, H = x.shape
        Is = self.gate_proj.weight.shape[0]
        _require_width(x, self.gate_proj.weight.shape[1], "x")
        (g, u, d), (gs, us, ds) = self._ptrs()
        n = ctypes.c_size_t(0)
        check(lib().lbmoe_dense_mlp_workspace_size(H, Is, self.weight_dtype, T, ctypes.byref(n)),
              "lbmoe_dense_mlp_workspace_size")
        dev = x.device
        ws = torch.empty(n.value, dtype=torch.uint8, device=dev)
        out = torch.empty_like(x)
        with torch.cuda.device(dev):
            check(lib().lbmoe_dense_mlp(g, u, d, gs, us, ds, H, Is, self.weight_dtype, ptr(x), T,
                                        ptr(out), ptr(ws), ws.numel(), _lib.stream_of(dev)),
                  "lbmoe_dense_mlp")
        return out


def _quantize_blocks(w):
    """bf16 [..., N, K] -> (e4m3 codes as uint8, fp32 scales [..., N/128, K/128]) on the GPU."""
    _require(w, "weight")
    *lead, N, K = w.shape
    batch = 1
    for d in lead:
        batch *= d
    q = torch.empty(w.shape, dtype=torch.uint8, device=w.device)
    s = torch.empty((*lead, N // 128, K // 128), dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        check(lib().lbmoe_quantize_fp8_blocks(ptr(w), batch, N, K, ptr(q), ptr(s),
                                              _lib.stream_of(w.device)),
              "lbmoe_quantize_fp8_blocks")
    return q, s


class Qwen3_5SparseMoeBlock(nn.Module):
    """Router + routed experts + gated shared expert (qwen3_5.py:881-905)."""

    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 moe_intermediate_size: int, shared_expert_intermediate_size: int):
        super().__init__()
        self.gate = Qwen3_5TopKRouter(num_experts, hidden_size, num_experts_per_tok)
        self.experts = Qwen3_5Experts(num_experts, hidden_size, moe_intermediate_size)
        if shared_expert_intermediate_size > 0:
            self.shared_expert = Qwen3_5SharedExpertMLP(hidden_size,
                                                        shared_expert_intermediate_size)
            self.shared_expert_gate = nn.Linear(hidden_size, 1, bias=False)
        else:
            self.shared_expert = None
            self.shared_expert_gate = None

    def layer(self):
        """The lbmoe_layer struct describing this block's parameters (every tensor's shape is
        checked against the block's sizes first)."""
        L = self.gate._layer()
        H = self.experts.hidden_size
        if L.hidden_size != H or L.num_experts != self.experts.num_experts:
            raise RuntimeError(f"gate.weight {tuple(self.gate.weight.shape)} disagrees with the "
                               f"experts' (num_experts, hidden_size) = "
                               f"({self.experts.num_experts}, {H})")
        self.experts.fill_layer(L)
        L.top_k = self.gate.top_k
        if self.shared_expert is not None:
            self.shared_expert.fill_layer(L)
            if self.shared_expert.gate_proj.weight.shape[1] != H:
                raise RuntimeError("shared_expert weights disagree with the block's hidden_size")
            _require(self.shared_expert_gate.weight, "shared_expert_gate.weight", ndim=2)
            _require_shape(self.shared_expert_gate.weight, (1, H), "shared_expert_gate.weight")
            L.shared_expert_gate = self.shared_expert_gate.weight.data_ptr()
            if self.shared_expert.weight_dtype != self.experts.weight_dtype:
                raise RuntimeError("experts and shared expert must use the same weight dtype")
        return L

    def workspace_size(self, T):
        return _lib.workspace_size(self.layer(), T)

    def forward(self, hidden_states: torch.Tensor, workspace: torch.Tensor = None):
        _require(hidden_states, "hidden_states", ndim=2)
        _require_width(hidden_states, self.experts.hidden_size)
        _same_device(self, hidden_states.device)
        T = hidden_states.shape[0]
        L = self.layer()
        dev = hidden_states.device
        workspace = _workspace(L, T, dev, workspace)
        y = torch.empty_like(hidden_states)
        with torch.cuda.device(dev):
            check(lib().lbmoe_forward(ctypes.byref(L), ptr(hidden_states), T, ptr(y),
                                      ptr(workspace), workspace.numel(), _lib.stream_of(dev)),
                  "lbmoe_forward")
        return y

    def forward_norm(self, hidden_states: torch.Tensor, residual: torch.Tensor, norm,
                     workspace: torch.Tensor = None):
        """The decoder layer's MLP half in one call (qwen3_5.py:998-1004):

            hidden_states = residual + hidden_states; residual = hidden_states
            hidden_states = norm(hidden_states); hidden_states = self(hidden_states)

        norm is the layer's post_attention_layernorm (a Qwen3_5RMSNorm: ``weight`` [H] and
        ``eps``). Returns (block output, new residual); the inputs are not modified.
        """
        _require(hidden_states, "hidden_states", ndim=2)
        _require(residual, "residual", ndim=2)
        _require(norm.weight, "norm.weight", ndim=1)
        _require_width(hidden_states, self.experts.hidden_size)
        _require_shape(norm.weight, (self.experts.hidden_size,), "norm.weight")
        if residual.shape != hidden_states.shape:
            raise RuntimeError("hidden_states and residual must have the same shape")
        if residual.device != hidden_states.device or norm.weight.device != hidden_states.device:
            raise RuntimeError("hidden_states, residual and norm.weight must share a device")
        _same_device(self, hidden_states.device)
        T = hidden_states.shape[0]
        L = self.layer()
        dev = hidden_states.device
        workspace = _workspace(L, T, dev, workspace)
        y = torch.empty_like(hidden_states)
        new_residual = torch.empty_like(residual)
        with torch.cuda.device(dev):
            check(lib().lbmoe_forward_norm(ctypes.byref(L), ptr(hidden_states), ptr(residual),
                                           ptr(norm.weight), float(norm.eps), T, ptr(y),
                                           ptr(new_residual), ptr(workspace), workspace.numel(),
                                           _lib.stream_of(dev)), "lbmoe_forward_norm")
        return y, new_residual

    @torch.no_grad()
    def pack_tiled_(self):
        """Derive the tiled copies of the bf16 expert weights (lbmoe_pack_weights), which the
        prefill-sized GEMMs stream faster than the checkpoint tensors; forward then passes both.
        The copies hold as many bytes as the expert weights again and are not updated when the
        weights change: a later call that finds the weights replaced or written since (storage
        address or version counter changed) drops the copies with a RuntimeWarning and streams
        the checkpoint tensors (same results); call this again after loading new weights. No
        counterpart in the reference (a load-time layout step)."""
        if self.experts.weight_dtype != _lib.LBMOE_W_BF16:
            raise RuntimeError("pack_tiled_ needs bf16 expert weights")
        ex, se = self.experts, self.shared_expert
        ex.gate_up_tiled = ex.down_tiled = None
        if se is not None:
            se.gate_up_tiled = se.down_tiled = None
        L = self.layer()
        gu, dn = torch.empty_like(ex.gate_up_proj), torch.empty_like(ex.down_proj)
        sgu = sdn = None
        if se is not None:
            Is, H = se.gate_proj.weight.shape
            sgu = torch.empty((2 * Is, H), dtype=se.gate_proj.weight.dtype,
                              device=se.gate_proj.weight.device)
            sdn = torch.empty_like(se.down_proj.weight)
        dev = gu.device
        with torch.cuda.device(dev):
            check(lib().lbmoe_pack_weights(ctypes.byref(L), ptr(gu), ptr(dn),
                                           ptr(sgu) if sgu is not None else None,
                                           ptr(sdn) if sdn is not None else None,
                                           _lib.stream_of(dev)), "lbmoe_pack_weights")
        ex.gate_up_tiled, ex.down_tiled = gu, dn
        ex.tiled_stamp = _stamp((ex.gate_up_proj, ex.down_proj))
        if se is not None:
            se.gate_up_tiled, se.down_tiled = sgu, sdn
            se.tiled_stamp = _stamp(se.tiled_sources())
        return self

    @torch.no_grad()
    def quantize_fp8_(self):
        """Convert expert (and shared-expert) weights to e4m3fn + 128x128 block scales."""
        ex = self.experts
        experts = _quantize_blocks(ex.gate_up_proj) + _quantize_blocks(ex.down_proj)
        shared = None
        if self.shared_expert is not None:
            se = self.shared_expert
            shared = {"gate": _quantize_blocks(se.gate_proj.weight),
                      "up": _quantize_blocks(se.up_proj.weight),
                      "down": _quantize_blocks(se.down_proj.weight)}
        return self.load_fp8_(experts, shared)

    @torch.no_grad()
    def load_fp8_(self, experts, shared=None):
        """Install e4m3fn weights with 128x128 block scales, e.g. from an fp8 checkpoint.

        experts: (gate_up codes [E,2I,H], gate_up scales [E,2I/128,H/128], down codes [E,H,I],
        down scales [E,H/128,I/128]); shared: {"gate"|"up"|"down": (codes, scales)} with the
        shared expert's [Is,H], [Is,H], [H,Is] shapes. Codes are uint8 (or float8_e4m3fn)
        tensors on the block's device, scales fp32.
        """
        ex = self.experts
        E, H, I = ex.num_experts, ex.hidden_size, ex.intermediate_size

        def codes_scales(q, s, shape, name):
            if q.dtype == torch.float8_e4m3fn:
                q = q.view(torch.uint8)
            if q.dtype != torch.uint8 or tuple(q.shape) != tuple(shape):
                raise RuntimeError(f"{name}: expected uint8 codes of shape {tuple(shape)}, got "
                                   f"{q.dtype} {tuple(q.shape)}")
            sshape = (*shape[:-2], shape[-2] // 128, shape[-1] // 128)
            if s.dtype != torch.float32 or tuple(s.shape) != sshape:
                raise RuntimeError(f"{name} scales: expected float32 {sshape}, got "
                                   f"{s.dtype} {tuple(s.shape)}")
            return q.contiguous(), s.contiguous()

        gu_q, gu_s, d_q, d_s = experts
        ex.gate_up_q, ex.gate_up_scale = codes_scales(gu_q, gu_s, (E, 2 * I, H), "experts.gate_up_proj")
        ex.down_q, ex.down_scale = codes_scales(d_q, d_s, (E, H, I), "experts.down_proj")
        ex.weight_dtype = _lib.LBMOE_W_FP8_E4M3
        ex.gate_up_tiled = ex.down_tiled = None        # bf16 layouts: no longer valid
        if self.shared_expert is not None:
            if shared is None:
                raise RuntimeError("this block has a shared expert: its fp8 weights are required")
            se = self.shared_expert
            Is = se.gate_proj.weight.shape[0]
            shapes = {"gate": (Is, H), "up": (Is, H), "down": (H, Is)}
            se.q = {n: codes_scales(*shared[n], shapes[n], f"shared_expert.{n}_proj.weight")
                    for n in ("gate", "up", "down")}
            se.weight_dtype = _lib.LBMOE_W_FP8_E4M3
            se.gate_up_tiled = se.down_tiled = None
        return self
