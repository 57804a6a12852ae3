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
