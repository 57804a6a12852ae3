"""Trainable MoE-SwiGLU layer: a drop-in for the reference's dense FFN `DenoiserBlock.mlp = SwiGLU(dim, hidden)`
(aurora/model.py:102-110, called as self.mlp(h) on (B, T, dim) at :210), with a softmax top-k router and a full
backward pass -- neither exists in the reference (its MoE path is inference-only, aurora/hf_compat.py:62).

Forward (all hmoe HIP kernels, one stream, no host sync):
  route_topk -> dispatch (stable counting sort; with a backward to follow, also the permuted copy of x) ->
  gate/up GEMM with fused SwiGLU (rows of x gathered by the GEMM when there is no copy) ->
  down GEMM x routing weight, scattered to (token, slot) order -> combine over the k slots.
Backward:
  combine_bwd (weighted dY for the down wgrad, routing-weight grads) -> down dgrad (dY rows gathered, routing
  weight applied in fp32) with fused SwiGLU backward -> down wgrad -> gate/up dgrad (fp32 rows) ->
  gate/up wgrad -> router backward (softmax + renormalisation Jacobian, dWr) -> un-permute (sum over
  the k slots) + router input gradient.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops


class _MoEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, wr, wgu, wd, bias, k, renorm, grad_dtype):
        T, d = x.shape
        E = wgu.shape[0]
        M = T * k
        need_grad = any(ctx.needs_input_grad[:4])
        logits, ids, tw = ops.route_topk(x, wr, k, bias=bias, renorm=renorm)
        # With a backward to follow, the dispatch writes the permuted copy xs of x (the gate/up weight gradient
        # reads it again); a forward alone gathers the rows of x inside the gate/up GEMM instead.
        disp = ops.dispatch(ids, E, topk_w=tw, x=x if need_grad else None, want_inv=need_grad)
        if need_grad:
            act, gu = ops.gate_up_swiglu(disp.xs, wgu, disp.counts, M, keep_gu=True)
        else:
            act, gu = ops.gate_up_swiglu(x, wgu, disp.counts, M, a_idx=disp.a_idx)
        y, yhat = ops.down_scatter(act, wd, disp.counts, M, disp.w_sorted, disp.order, keep_yhat=need_grad)
        out = ops.combine(y, T, k)
        if need_grad:
            ctx.save_for_backward(x, wr, wgu, wd, logits, ids, disp.counts, disp.order, disp.a_idx, disp.inv_pos,
                                  disp.w_sorted, disp.xs, gu, act, yhat)
        ctx.k, ctx.renorm, ctx.grad_dtype = k, renorm, grad_dtype
        ctx.mark_non_differentiable(ids, tw)
        ctx.set_materialize_grads(False)  # no zero-filled gradients for the index / weight outputs
        return out, ids, tw

    @staticmethod
    def backward(ctx, dout, _dids, _dtw):
        if dout is None:
            return None, None, None, None, None, None, None, None
        (x, wr, wgu, wd, logits, ids, counts, order, a_idx, inv_pos, w_sorted, xs, gu, act,
         yhat) = ctx.saved_tensors
        k = ctx.k
        T, d = x.shape
        E = wgu.shape[0]
        M = T * k
        disp = ops.Dispatch(counts, None, None, order, a_idx, inv_pos, w_sorted, xs)
        dout = dout.contiguous().to(torch.bfloat16)
        # One stream: every GEMM is a persistent launch sized to own all CUs, so two of them side by side only
        # queue each other's workgroups behind long-running tiles.
        dys, dtw = ops.combine_bwd(dout, yhat, disp, k)
        dwd = dwgu = None
        if ctx.needs_input_grad[3]:
            dwd = ops.grouped_wgrad(act, dys, counts, E, dtype=ctx.grad_dtype)
        dgu = ops.down_dgrad_swiglu(dout, wd, counts, M, gu, a_idx=a_idx, w_sorted=w_sorted)
        if ctx.needs_input_grad[2]:
            dwgu = ops.grouped_wgrad(xs, dgu, counts, E, dtype=ctx.grad_dtype)
        dxs = ops.gate_up_dgrad(dgu, wgu, counts, M)
        dwr_dtype = wr.dtype if wr.dtype in (torch.bfloat16, torch.float32) else torch.float32
        dl, dwr = ops.router_bwd(logits, ids, dtw, x, renorm=ctx.renorm, dwr_dtype=dwr_dtype,
                                 want_dwr=ctx.needs_input_grad[1])
        dx = ops.unpermute_bwd(dxs, inv_pos, T, k, dlogits=dl, wr=wr) if ctx.needs_input_grad[0] else None
        if dwr is not None and dwr.dtype != wr.dtype:
            dwr = dwr.to(wr.dtype)
        if dwgu is not None and dwgu.dtype != wgu.dtype:
            dwgu = dwgu.to(wgu.dtype)
        if dwd is not None and dwd.dtype != wd.dtype:
            dwd = dwd.to(wd.dtype)
        return dx, dwr, dwgu, dwd, None, None, None, None


def moe_swiglu(x, router_weight, w_gu, w_d, top_k, logit_bias=None, renorm=True, grad_dtype=torch.bfloat16):
    """Functional form: x (T, d) bf16 -> (out (T, d), topk_ids (T, k) int32, topk_weight (T, k) fp32)."""
    return _MoEFunction.apply(x, router_weight, w_gu, w_d, logit_bias, top_k, renorm, grad_dtype)


class MoESwiGLU(nn.Module):
    """MoE replacement for aurora/model.py:102-110 `SwiGLU(dim, hidden)`: same call shape ((..., dim) -> (..., dim)).

    Parameters: router_weight (E, dim); w_gu (E, dim, 2*hidden) = [gate | up] per expert (the stacked layout of
    aurora/hf_compat.py:154, gate first as in aurora/model.py:109); w_d (E, hidden, dim).  Buffer logit_bias (E,)
    fp32 is added to the router logits (zero by default; -inf disables an expert).  Weights are bf16 and initialised
    N(0, init_std)."""

    def __init__(self, dim: int, hidden: int, experts: int, top_k: int = 2, renorm: bool = True,
                 init_std: float = 0.02, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.dim, self.hidden, self.experts, self.top_k, self.renorm = dim, hidden, experts, top_k, renorm
        f = dict(device=device, dtype=dtype)
        self.router_weight = nn.Parameter(torch.empty(experts, dim, **f))
        self.w_gu = nn.Parameter(torch.empty(experts, dim, 2 * hidden, **f))
        self.w_d = nn.Parameter(torch.empty(experts, hidden, dim, **f))
        self.register_buffer("logit_bias", torch.zeros(experts, device=device, dtype=torch.float32))
        self.init_std = init_std
        self.reset_parameters()
        self.last_topk_ids = None

    @torch.no_grad()
    def reset_parameters(self):
        for p in (self.router_weight, self.w_gu, self.w_d):
            nn.init.normal_(p, std=self.init_std)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        shape = h.shape
        x = h.reshape(-1, shape[-1])
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        out, ids, _ = moe_swiglu(x, self.router_weight, self.w_gu, self.w_d, self.top_k, self.logit_bias, self.renorm)
        self.last_topk_ids = ids
        return out.view(shape)
