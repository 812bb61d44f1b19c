"""torch-CPU restatement of the reference MoE block with its bf16 rounding points.

Test infrastructure and CPU baseline only. It restates, operation by operation, the
reference's two expert algorithms so that the CPU baseline times the algorithm the
reference would run on the same shapes:

* ``route``           qwen3_5.py:767-774 (bf16 F.linear, fp32 softmax, topk, renormalise,
                      cast to bf16); an optional fp32 logit bias is added after the upcast.
* ``experts_dense``   qwen3_5.py:843-874: gather whole expert matrices per (token, slot),
                      two bmm's, weighted sum over slots. Used for decode (is_prefill False,
                      qwen3_5.py:808-813).
* ``experts_sparse``  qwen3_5.py:815-841: one-hot mask, loop over hit experts in ascending
                      order, per-expert F.linear, bf16 index_add_. Used for prefill.
* ``shared``          qwen3_5.py:897, :903-904, :916-917.
* ``block``           qwen3_5.py:899-905.

Everything runs in bfloat16 as in the reference (model_runner.py:70-72 sets bf16 as the
default dtype), so results differ from the float64 oracle by bf16 rounding only.
"""
import torch
import torch.nn.functional as F

__all__ = ["route", "experts_dense", "experts_sparse", "shared", "block"]


def route(x, wg, k, bias=None):
    logits = F.linear(x, wg)
    z = logits.float()
    if bias is not None:
        z = z + bias.float()
    probs = torch.softmax(z, dim=-1)
    vals, idx = torch.topk(probs, k, dim=-1)
    vals = vals / vals.sum(dim=-1, keepdim=True)
    return vals.to(x.dtype), idx


def experts_dense(x, idx, w, w_gu, w_d):
    T, k = idx.shape
    flat = idx.reshape(-1)
    wgu_rows = w_gu[flat]                                  # [T*k, 2I, H]
    wd_rows = w_d[flat]                                    # [T*k, H, I]
    xr = x.repeat_interleave(k, dim=0).unsqueeze(-1)       # [T*k, H, 1]
    gu = torch.bmm(wgu_rows, xr).squeeze(-1)               # [T*k, 2I]
    g, u = gu.chunk(2, dim=-1)
    a = F.silu(g) * u
    o = torch.bmm(wd_rows, a.unsqueeze(-1)).squeeze(-1)    # [T*k, H]
    return (o.view(T, k, -1) * w.unsqueeze(-1)).sum(dim=1)


def experts_sparse(x, idx, w, w_gu, w_d):
    E = w_gu.shape[0]
    y = torch.zeros_like(x)
    mask = F.one_hot(idx, num_classes=E).permute(2, 1, 0)  # [E, k, T]
    hit = (mask.sum(dim=(-1, -2)) > 0).nonzero().flatten().tolist()
    for e in hit:
        slot, tok = torch.where(mask[e])
        g, u = F.linear(x[tok], w_gu[e]).chunk(2, dim=-1)
        o = F.linear(F.silu(g) * u, w_d[e])
        o = o * w[tok, slot, None]
        y.index_add_(0, tok, o.to(y.dtype))
    return y


def shared(x, gate, up, down, gate_w):
    s = F.linear(F.silu(F.linear(x, gate)) * F.linear(x, up), down)
    return torch.sigmoid(F.linear(x, gate_w)) * s


def block(x, wg, w_gu, w_d, k, bias=None, sh=None, algorithm="dense"):
    """sh: None or (gate, up, down, gate_w). algorithm: 'dense' or 'sparse'."""
    w, idx = route(x, wg, k, bias)
    fn = experts_dense if algorithm == "dense" else experts_sparse
    y = fn(x, idx, w, w_gu, w_d)
    if sh is not None:
        y = y + shared(x, *sh)
    return y, w, idx
