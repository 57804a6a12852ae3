"""TEST INFRASTRUCTURE ONLY -- the reference's PyTorch CPU path, transcribed, for bench.py's cpu_baseline leg and as
a second checker in tests.  Never imported by the product package.

On a CPU device the reference's mode selection (_pick_mode, aurora/hf_compat.py:124-139) skips Triton and picks
torch._grouped_mm after its self-test, so the CPU path is _fused_moe_infer's "grouped" branch
(aurora/hf_compat.py:69-72, 83-88, 98-99), preceded by a softmax top-k router with the conventions of
aurora/hf_pipeline.py:352-359 (fp32 logits, top-k, renormalise).  Backward (training step) is torch autograd through
the same graph; the reference itself has no backward for this path.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def router(x, wr, k, bias=None, renorm=True, scaling=1.0):
    """aurora/hf_pipeline.py:352-359 with softmax scores: fp32 logits, top-k (sorted), w / (sum + 1e-20) * scaling."""
    logits = F.linear(x.float(), wr.float())
    if bias is not None:
        logits = logits + bias.float()
    p = logits.softmax(-1)
    w, idx = p.topk(k, dim=-1)
    if renorm:
        w = w / (w.sum(-1, keepdim=True) + 1e-20) * scaling
    else:
        w = w * scaling
    return logits, idx, w


def fused_moe_grouped(x, topk_ids, topk_weight, wgu, wd, act=F.silu):
    """aurora/hf_compat.py:69-72 and 83-88, 98-99 (the `grouped` branch of _fused_moe_infer)."""
    n, k = topk_ids.shape
    flat = topk_ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=wgu.shape[0])
    xs = x[order // k]
    offs = counts.cumsum(0).to(torch.int32)
    g, u = torch._grouped_mm(xs, wgu, offs=offs).chunk(2, dim=-1)
    ys = torch._grouped_mm(act(g) * u, wd, offs=offs)
    ys = ys * topk_weight.reshape(-1)[order].to(ys.dtype).unsqueeze(-1)
    return ys[order.argsort()].view(n, k, -1).sum(1)


def layer_forward(x, wr, wgu, wd, k, bias=None, renorm=True):
    _, idx, w = router(x, wr, k, bias, renorm)
    return fused_moe_grouped(x, idx, w, wgu, wd)


def training_step(x, wr, wgu, wd, k, dout, bias=None, renorm=True):
    """Forward + backward by autograd (inputs must have requires_grad set by the caller where wanted)."""
    out = layer_forward(x, wr, wgu, wd, k, bias, renorm)
    out.backward(dout)
    return out


def poziomka_forward(x, gate_w, expert_bias, wgu, wgu_s, wd, wd_s, shared_g, shared_u, shared_d, k, n_group,
                     topk_group, scaling):
    """The BailingMoeV2 block's own forward, aurora/hf_pipeline.py:348-370 (PoziomkaMoE): sigmoid scores in fp32,
    expert bias for selection, group-limited top-k, renormalised and scaled weights rounded to x.dtype; a loop over
    the experts in use with the int8 weights widened to fp32 and the scale after the sum; index_add_ into an fp32
    output; plus the shared expert (:314-322, bf16 F.linear)."""
    n, d = x.shape
    scores = torch.sigmoid(F.linear(x.float(), gate_w.float()))
    routing = scores + expert_bias.float()
    group = routing.view(n, n_group, -1).topk(2, dim=-1)[0].sum(-1)
    keep = torch.zeros_like(group).scatter_(1, group.topk(topk_group, dim=-1, sorted=False)[1], 1)
    keep = keep.bool().unsqueeze(-1).expand(n, n_group, routing.shape[1] // n_group).reshape(n, -1)
    idx = routing.masked_fill(~keep, float("-inf")).topk(k, dim=-1)[1]
    w = scores.gather(1, idx)
    w = w / (w.sum(-1, keepdim=True) + 1e-20) * scaling
    out = torch.zeros(n, d, dtype=torch.float32)
    wq = w.to(x.dtype).float()
    for e in idx.unique().tolist():
        rows, slot = (idx == e).nonzero(as_tuple=True)
        gu = ((x[rows].float() @ wgu[e].float()) * wgu_s[e].float()).to(x.dtype)
        g, u = gu.chunk(2, dim=-1)
        y = ((F.silu(g) * u).float() @ wd[e].float()) * wd_s[e].float()
        out.index_add_(0, rows, (y * wq[rows, slot, None]).to(x.dtype).float())
    lin = lambda a, m: F.linear(a, m.to(a.dtype))  # noqa: E731
    shared = lin(F.silu(lin(x, shared_g)) * lin(x, shared_u), shared_d)
    return out.to(x.dtype) + shared


def router_routed(x, wr, ids, bias=None, renorm=True, scaling=1.0):
    """router() with the expert choice given (ids (T, k)): the same fp32 logits and softmax, the weights gathered at
    ids instead of torch.topk's picks.  Where the two agree on the ids this is router() exactly; it keeps a near tie
    that torch's GEMM order would break differently from routing the reference path onto other experts."""
    logits = F.linear(x.float(), wr.float())
    if bias is not None:
        logits = logits + bias.float()
    w = logits.softmax(-1).gather(1, ids.long())
    if renorm:
        w = w / (w.sum(-1, keepdim=True) + 1e-20) * scaling
    else:
        w = w * scaling
    return logits, w


def training_step_routed(x, wr, wgu, wd, ids, dout, bias=None, renorm=True):
    """training_step() on given routing ids: the reference's bf16 CPU path (router weights, grouped GEMMs, two-rounding
    weight multiply, un-permute sum) differentiated by autograd.  Used as the yardstick of the backward tolerance: the
    error of this path against the float64 oracle is what the reference's own arithmetic achieves on the same
    inputs."""
    _, w = router_routed(x, wr, ids, bias, renorm)
    out = fused_moe_grouped(x, ids.long(), w, wgu, wd)
    out.backward(dout)
    return out
