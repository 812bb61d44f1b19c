"""numpy oracle of the sparse-MoE feed-forward block (test infrastructure only).

Restates nanovllm/models/qwen3_5.py:754-917 on the CPU:

* ``router_logits`` / ``route``   Qwen3_5TopKRouter.forward, qwen3_5.py:767-774
* ``permute``                     expert sort of _forward_sparse, qwen3_5.py:823-833
* ``experts``                     Qwen3_5Experts math, qwen3_5.py:834-839 / :855-872,
                                  accumulated in float64 with no intermediate rounding
* ``shared_gate`` / ``shared_expert``
                                  Qwen3_5SharedExpertMLP + shared_expert_gate,
                                  qwen3_5.py:897, :903, :916-917
* ``block_forward``               Qwen3_5SparseMoeBlock.forward, qwen3_5.py:899-905
* ``add_rmsnorm``                 the decoder layer's residual add and post-attention
                                  Qwen3_5RMSNorm ahead of the MoE block, qwen3_5.py:998-1002,
                                  :39-55
* ``quant_blocks`` / ``quant_groups`` / ``experts_fp8`` / ``block_forward_fp8``
                                  the fp8-e4m3 variant, which has no counterpart in the
                                  reference (no fp8 code exists there); defined here by
                                  per-128x128-block weight scales and per-(row, 128-channel)
                                  activation scales, scale = amax / 448.

Selection rule. The reference takes ``torch.topk`` of fp32 softmax probabilities of bf16
logits; equal bf16 logits give exactly equal probabilities and torch's tie order is
implementation-defined. The oracle orders experts by (-z, expert index), where
z = fp32(bf16 logit) (+ fp32 bias). Softmax is strictly increasing in z, so this equals the
order by (-p, expert index) whenever exp separates distinct z, which
``tests/test_oracle.py`` checks on every fixture.

Pinning (how each function is checked independently of its own formula, in
tests/test_oracle.py and tests/test_golden.py):

* codecs: bf16 against torch's bfloat16 cast; e4m3 against torch.float8_e4m3fn casts
  and the exhaustive code table.
* router_logits: fp64 dot products against torch's bf16 F.linear within one bf16 ulp;
  route: brute-force sort of Python tuples, invariants (distinct, sorted, sum ~ 1),
  closed forms (k = E selects all experts; k = 1 gives weight 1).
* permute: brute-force Python sort on tuple keys; invariants (histogram, scan,
  bijection, inverse).
* experts / block_forward: the k = 1, E = 1 reduction to a dense SwiGLU MLP evaluated by an
  independent torch float64 path; linearity in w_down and in the routing weights;
  T = 1 as k independent GEMVs; the torch-CPU restatement of both reference algorithms
  (oracle/torch_ref.py) within bf16 tolerance.
* add_rmsnorm: torch's restatement of Qwen3_5RMSNorm within one bf16 step; closed forms
  (a constant row normalises to its sign; with eps = 0, scaling a row by a power of two
  leaves the output unchanged; weight w scales by (1 + w)).
* fp8 functions: quantise/dequantise round trips, exactness on e4m3-representable blocks,
  scale closed forms, and the bf16 oracle within fp8 error bounds.
* the reference module itself: tests/golden/reference_moe_small.npz holds outputs recorded
  from the reference's Qwen3_5SparseMoeBlock (tests/golden/make_reference_golden.py);
  tests/test_golden.py checks torch_ref bit for bit against them and this oracle for
  selection modulo boundary ties and outputs within 1e-2.
"""
import numpy as np

from .codecs import bf16_round, e4m3_decode, e4m3_encode, E4M3_MAX

__all__ = [
    "router_logits", "route", "route_by_prob", "shared_gate", "permute", "experts",
    "shared_expert", "block_forward", "silu", "quant_blocks", "dequant_blocks",
    "quant_groups", "dequant_groups", "experts_fp8", "shared_expert_fp8",
    "block_forward_fp8", "rel_err", "add_rmsnorm",
]


def silu(v):
    return v / (1.0 + np.exp(-v))


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def router_logits(x, wg):
    """bf16(x . Wg^T): qwen3_5.py:769 (F.linear of bf16 operands returns bf16).

    x [T,H], wg [E,H] hold bf16 values (as float32). The dot product is exact enough in
    float64 that the result is the correctly rounded bf16 of the true value.
    """
    return bf16_round((_f64(x) @ _f64(wg).T).astype(np.float32))


def _softmax32(z):
    m = z.max(axis=-1, keepdims=True)
    e = np.exp((z - m).astype(np.float32)).astype(np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def route(logits, k, bias=None):
    """Softmax -> top-k -> renormalise -> bf16: qwen3_5.py:770-774.

    logits [T,E] (bf16 values), optional fp32 bias [E] added after the upcast.
    Returns (w [T,k] float32 holding bf16 values, idx [T,k] int64, probs [T,E] fp32).
    Order within a row: descending z, ties broken by ascending expert index.
    """
    z = np.asarray(logits, dtype=np.float32)
    if bias is not None:
        z = (z + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    T, E = z.shape
    p = _softmax32(z)
    ar = np.broadcast_to(np.arange(E), z.shape)
    order = np.lexsort((ar, -z), axis=-1)[:, :k]          # primary -z, secondary index
    idx = order.astype(np.int64)
    v = np.take_along_axis(p, order, axis=-1).astype(np.float32)
    v = (v / v.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return bf16_round(v), idx, p


def route_by_prob(probs, k):
    """Canonical order on probabilities: (-p, expert index), ties to the lower expert."""
    p = np.asarray(probs, dtype=np.float32)
    ar = np.broadcast_to(np.arange(p.shape[1]), p.shape)
    return np.lexsort((ar, -p), axis=-1)[:, :k].astype(np.int64)


def shared_gate(x, w_sg):
    """sigmoid(bf16(x . w_sg^T)) in fp32: qwen3_5.py:897, :903. w_sg [1,H] or [H]."""
    lg = bf16_round((_f64(x) @ _f64(w_sg).reshape(-1)).astype(np.float32))
    return (1.0 / (1.0 + np.exp(-lg.astype(np.float64)))).astype(np.float32)


def permute(idx, E):
    """Expert-sorted order of the (token, slot) pairs: qwen3_5.py:823-833.

    The reference visits hit experts in ascending order (nonzero, :827) and, within an
    expert, ``torch.where(expert_mask[e])`` on the [k, T] mask yields pairs in row-major
    (slot, token) order (:833). The sort key is therefore (expert, slot, token).
    Returns counts[E], offsets[E+1], perm_tok[T*k], perm_slot[T*k], inv[T,k] (int64),
    where perm_*[inv[t,s]] == (t, s).
    """
    idx = np.asarray(idx, dtype=np.int64)
    T, k = idx.shape
    e_sm = idx.T.reshape(-1)                       # slot-major: v = s*T + t
    order = np.argsort(e_sm, kind="stable")
    counts = np.bincount(e_sm, minlength=E).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    perm_tok = order % T
    perm_slot = order // T
    inv_sm = np.empty(T * k, dtype=np.int64)
    inv_sm[order] = np.arange(T * k)
    inv = inv_sm.reshape(k, T).T.copy()
    return counts, offsets, perm_tok, perm_slot, inv


def _swiglu(xr, w_gate, w_up, w_down):
    g = xr @ _f64(w_gate).T
    u = xr @ _f64(w_up).T
    return (silu(g) * u) @ _f64(w_down).T


def experts(x, idx, w, w_gu, w_d):
    """Routed-expert output sum_s w[t,s] * down_e(silu(gate_e x) * up_e x), float64.

    w_gu [E,2I,H] (gate rows [0,I), up rows [I,2I): chunk(2,-1) at qwen3_5.py:835),
    w_d [E,H,I]. Only experts that appear in idx are touched, so this is cheap for a
    handful of tokens at full layer size.
    """
    x = _f64(x)
    idx = np.asarray(idx, dtype=np.int64)
    w = _f64(w)
    T, k = idx.shape
    I = w_gu.shape[1] // 2
    y = np.zeros((T, x.shape[1]), dtype=np.float64)
    for e in np.unique(idx):
        tt, ss = np.nonzero(idx == e)
        o = _swiglu(x[tt], w_gu[e][:I], w_gu[e][I:], w_d[e])
        np.add.at(y, tt, o * w[tt, ss][:, None])
    return y


def shared_expert(x, w_gate, w_up, w_down):
    """Qwen3_5SharedExpertMLP.forward, qwen3_5.py:916-917, in float64."""
    return _swiglu(_f64(x), w_gate, w_up, w_down)


def block_forward(x, wg, w_gu, w_d, k, bias=None, shared=None):
    """Qwen3_5SparseMoeBlock.forward (qwen3_5.py:899-905), float64 accumulation.

    shared: None or dict(gate, up, down, gate_w). Returns (y float64, w, idx).
    """
    logits = router_logits(x, wg)
    w, idx, _ = route(logits, k, bias)
    y = experts(x, idx, w, w_gu, w_d)
    if shared is not None:
        g = shared_gate(x, shared["gate_w"]).astype(np.float64)
        y = y + g[:, None] * shared_expert(x, shared["gate"], shared["up"], shared["down"])
    return y, w, idx


def rel_err(y, y_ref):
    """Normwise relative error max|y - y_ref| / max|y_ref|."""
    y = _f64(y)
    y_ref = _f64(y_ref)
    den = np.max(np.abs(y_ref))
    return float(np.max(np.abs(y - y_ref)) / (den if den > 0 else 1.0))


# ---------------------------------------------------------------------------------------
# fp8 e4m3 variant (no counterpart in the reference)
# ---------------------------------------------------------------------------------------

def _scale_of(amax):
    """scale = amax / 448 in fp32; an all-zero block gets scale 1 (its codes are all 0)."""
    amax = np.asarray(amax, dtype=np.float32)
    s = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    return np.where(amax > 0, s, np.float32(1.0)).astype(np.float32)


def quant_blocks(w, block=128):
    """Per-(128 x 128)-block quantisation of w [..., N, K] (N, K multiples of 128).

    Returns (codes uint8 [..., N, K], scales fp32 [..., N/128, K/128]) with
    codes = e4m3(w / scale), scale = blockmax|w| / 448.
    """
    w = np.asarray(w, dtype=np.float32)
    *lead, N, K = w.shape
    wb = w.reshape(*lead, N // block, block, K // block, block)
    amax = np.abs(wb).max(axis=(-3, -1))
    s = _scale_of(amax)
    q = e4m3_encode((wb / s[..., :, None, :, None]).astype(np.float32))
    return q.reshape(w.shape), s


def dequant_blocks(q, s, block=128):
    q = e4m3_decode(q)
    *lead, N, K = q.shape
    qb = q.reshape(*lead, N // block, block, K // block, block)
    return (qb * s[..., :, None, :, None]).reshape(q.shape).astype(np.float32)


def quant_groups(a, group=128):
    """Per-(row, 128-channel group) quantisation of a [R, C]: (codes [R,C], scales [R,C/128])."""
    a = np.asarray(a, dtype=np.float32)
    R, C = a.shape
    ag = a.reshape(R, C // group, group)
    s = _scale_of(np.abs(ag).max(axis=-1))
    q = e4m3_encode((ag / s[..., None]).astype(np.float32))
    return q.reshape(R, C), s


def dequant_groups(q, s, group=128):
    R, C = q.shape
    return (e4m3_decode(q).reshape(R, C // group, group) * s[..., None]).reshape(R, C).astype(np.float32)


def _swiglu_fp8(x_dq, wgate_dq, wup_dq, wdown_dq):
    """fp8 SwiGLU: fp64 GEMMs on dequantised operands; the intermediate is rounded to bf16
    and re-quantised per (row, 128 channels) before the down projection."""
    g = x_dq @ _f64(wgate_dq).T
    u = x_dq @ _f64(wup_dq).T
    a = bf16_round((silu(g) * u).astype(np.float32))
    aq, asc = quant_groups(a)
    return _f64(dequant_groups(aq, asc)) @ _f64(wdown_dq).T


def experts_fp8(x, idx, w, wgu_q, wgu_s, wd_q, wd_s):
    """fp8 routed experts against dequantised weights and dequantised activations."""
    xq, xs = quant_groups(x)
    x_dq = _f64(dequant_groups(xq, xs))
    idx = np.asarray(idx, dtype=np.int64)
    w = _f64(w)
    T, k = idx.shape
    I = wgu_q.shape[1] // 2
    y = np.zeros((T, x.shape[1]), dtype=np.float64)
    for e in np.unique(idx):
        tt, ss = np.nonzero(idx == e)
        gu = dequant_blocks(wgu_q[e], wgu_s[e])
        wd = dequant_blocks(wd_q[e], wd_s[e])
        o = _swiglu_fp8(x_dq[tt], gu[:I], gu[I:], wd)
        np.add.at(y, tt, o * w[tt, ss][:, None])
    return y


def shared_expert_fp8(x, gate_q, gate_s, up_q, up_s, down_q, down_s):
    xq, xs = quant_groups(x)
    x_dq = _f64(dequant_groups(xq, xs))
    return _swiglu_fp8(x_dq, dequant_blocks(gate_q, gate_s), dequant_blocks(up_q, up_s),
                       dequant_blocks(down_q, down_s))


def block_forward_fp8(x, wg, k, q, bias=None):
    """fp8 block: bf16 router (as in the bf16 block), fp8 experts and shared expert.

    q: dict with wgu_q, wgu_s, wd_q, wd_s and optionally sh_{gate,up,down}_{q,s}, sh_gate_w.
    """
    logits = router_logits(x, wg)
    w, idx, _ = route(logits, k, bias)
    y = experts_fp8(x, idx, w, q["wgu_q"], q["wgu_s"], q["wd_q"], q["wd_s"])
    if "sh_gate_q" in q:
        g = shared_gate(x, q["sh_gate_w"]).astype(np.float64)
        y = y + g[:, None] * shared_expert_fp8(x, q["sh_gate_q"], q["sh_gate_s"], q["sh_up_q"],
                                               q["sh_up_s"], q["sh_down_q"], q["sh_down_s"])
    return y, w, idx


def add_rmsnorm(hidden, residual, weight, eps):
    """The MoE block's input in the decoder layer: qwen3_5.py:998-1002.

    h = bf16(residual + hidden) (bf16 tensors add in fp32 and round, :998); the new residual is
    h (:1001); x = Qwen3_5RMSNorm(h) (:1002, :39-55): in fp32, h * 1/sqrt(mean(h^2) + eps),
    then times (1 + weight), rounded to bf16. hidden, residual [T,H] and weight [H] hold bf16
    values. Returns (h, x) as float32 arrays of bf16 values.
    """
    h = bf16_round((np.asarray(residual, np.float32) + np.asarray(hidden, np.float32)).astype(np.float32))
    ms = np.mean(h * h, axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    one_w = (np.float32(1.0) + np.asarray(weight, np.float32)).astype(np.float32)
    x = bf16_round(((h * r).astype(np.float32) * one_w).astype(np.float32))
    return h, x
