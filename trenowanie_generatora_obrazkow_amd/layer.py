"""Trainable MoE-SwiGLU layer: a drop-in for the reference's dense FFN `DenoiserBlock.mlp = SwiGLU(dim, hidden)`
(aurora/model.py:102-110, called as self.mlp(h) on (B, T, dim) at :210), with a softmax top-k router and a full
backward pass -- neither exists in the reference (its MoE path is inference-only, aurora/hf_compat.py:62).

Forward (all hmoe HIP kernels, one stream, no host sync):
  route_topk -> dispatch (stable counting sort, the routed rows of x as row-group tiles for the GEMM's copies; with
  a backward to follow, also the row-major permuted copy) -> gate/up GEMM with fused SwiGLU ->
  down GEMM x routing weight, scattered to (token, slot) order -> combine over the k slots.
Backward:
  combine_bwd (weighted dY for the down wgrad) -> down wgrad -> down dgrad (dY rows gathered, routing weight
  applied in fp32) with fused SwiGLU backward and the routing-weight gradients -> gate/up dgrad (fp32 rows) ->
  gate/up wgrad -> router backward (softmax + renormalisation Jacobian, dWr) -> un-permute (sum over
  the k slots) + router input gradient.

The kernels compute in bf16 with fp32 accumulation.  fp32 weights (master weights) are rounded to bf16 for the
products, as torch.autocast does for the reference's nn.Linear layers, and receive fp32 gradients; fp16 weights
are rounded to bf16 the same way and receive their fp32 gradients rounded once to fp16.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops

_WDTYPES = (torch.bfloat16, torch.float32, torch.float16)


def _grad_dtype(param_dtype):
    """dtype a weight gradient is computed in: the parameter's own for bf16 / fp32, fp32 for fp16 parameters (the
    kernels write bf16 or fp32; the fp32 sum is then rounded once to fp16)."""
    return torch.float32 if param_dtype == torch.float16 else param_dtype


def _to_param(g, param_dtype):
    return g if g is None or g.dtype == param_dtype else g.to(param_dtype)


def _check_layer_args(x, wr, wgu, wd, bias, k):
    """Every shape the kernels rely on, cross-checked before the first launch: one expert count E (router rows,
    expert stacks, bias) and one model width d.  A router with more rows than there are expert stacks would route
    tokens to experts that do not exist."""
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError(f"x must be a (T, d) bf16 matrix (got {tuple(x.shape)} {x.dtype})")
    if wr.dim() != 2 or wgu.dim() != 3 or wd.dim() != 3:
        raise ValueError("router_weight (E, d), w_gu (E, d, 2h) and w_d (E, h, d) expected")
    T, d = x.shape
    E, h = wgu.shape[0], wd.shape[1]
    for t, name, shape in ((wr, "router_weight", (E, d)), (wgu, "w_gu", (E, d, 2 * h)), (wd, "w_d", (E, h, d))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape} (E={E}, d={d}, h={h})")
        if t.dtype not in _WDTYPES:
            raise TypeError(f"{name}: dtype {t.dtype}; the layer takes bf16, fp32 or fp16 weights")
    if bias is not None and tuple(bias.shape) != (E,):
        raise ValueError(f"logit_bias: shape {tuple(bias.shape)}, expected ({E},)")
    if not 1 <= k <= E:
        raise ValueError(f"top_k = {k} must lie in [1, {E}]")


def _bf16(t):
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


class _MoEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, wr, wgu, wd, bias, k, renorm):
        _check_layer_args(x, wr, wgu, wd, bias, k)
        T, d = x.shape
        E = wgu.shape[0]
        M = T * k
        ctx.w_dtypes = (wr.dtype, wgu.dtype, wd.dtype)
        wr, wgu, wd = _bf16(wr), _bf16(wgu), _bf16(wd)
        need_grad = any(ctx.needs_input_grad[:4])
        logits, ids, tw = ops.route_topk(x, wr, k, bias=bias, renorm=renorm)
        # The dispatch writes the routed rows as row-group tiles for the gate/up GEMM; with a backward to follow,
        # also the row-major permuted copy xs (the gate/up weight gradient reads it).
        disp, act, gu = ops.routed_gate_up(x, ids, E, wgu, topk_w=tw, keep_gu=need_grad, want_xs=need_grad,
                                           want_inv=need_grad)
        y, _ = ops.down_scatter(act, wd, disp.counts, M, disp.w_sorted, disp.order)
        out = ops.combine(y, T, k)
        if need_grad:
            ctx.save_for_backward(x, wr, wgu, wd, logits, ids, disp.counts, disp.order, disp.a_idx, disp.inv_pos,
                                  disp.w_sorted, disp.xs, gu, act)
        ctx.k, ctx.renorm = k, renorm
        ctx.mark_non_differentiable(ids)
        ctx.set_materialize_grads(False)  # absent output gradients stay None (no zero-filled tensors)
        return out, ids, tw

    @staticmethod
    def backward(ctx, dout, _dids, dtw_out):
        if dout is None and dtw_out is None:
            return None, None, None, None, None, None, None
        x, wr, wgu, wd, logits, ids, counts, order, a_idx, inv_pos, w_sorted, xs, gu, act = ctx.saved_tensors
        k = ctx.k
        T, d = x.shape
        E = wgu.shape[0]
        M = T * k
        wr_dt, wgu_dt, wd_dt = ctx.w_dtypes
        disp = ops.Dispatch(counts, None, None, order, a_idx, inv_pos, w_sorted, xs)
        if dout is None:  # a loss on the routing weights alone: the expert path carries no gradient
            dout = torch.zeros(T, d, device=x.device, dtype=torch.bfloat16)
        dout = dout.contiguous().to(torch.bfloat16)
        # One stream: every GEMM is a persistent launch sized to own all CUs, so two of them side by side only
        # queue each other's workgroups behind long-running tiles.
        dys, _ = ops.combine_bwd(dout, None, disp, k)
        dwd = dwgu = None
        if ctx.needs_input_grad[3]:
            dwd = _to_param(ops.grouped_wgrad(act, dys, counts, E, dtype=_grad_dtype(wd_dt)), wd_dt)
        # dgu, and the routing-weight gradient <dout[t], act[r] @ wd[e]> from the same fp32 product
        dgu, dtw = ops.down_dgrad_swiglu_dw(dout, wd, counts, M, gu, order, k, a_idx=a_idx, w_sorted=w_sorted)
        if dtw_out is not None:  # the returned routing weights are outputs too: their gradient joins the combine's
            dtw = dtw + dtw_out.to(torch.float32)
        if ctx.needs_input_grad[2]:
            dwgu = _to_param(ops.grouped_wgrad(xs, dgu, counts, E, dtype=_grad_dtype(wgu_dt)), wgu_dt)
        dxs = ops.gate_up_dgrad(dgu, wgu, counts, M)
        dl, dwr = ops.router_bwd(logits, ids, dtw, x, renorm=ctx.renorm, dwr_dtype=_grad_dtype(wr_dt),
                                 want_dwr=ctx.needs_input_grad[1])
        dwr = _to_param(dwr, wr_dt)
        dx = ops.unpermute_bwd(dxs, inv_pos, T, k, dlogits=dl, wr=wr) if ctx.needs_input_grad[0] else None
        return dx, dwr, dwgu, dwd, None, None, None


def moe_swiglu(x, router_weight, w_gu, w_d, top_k, logit_bias=None, renorm=True):
    """Functional form: x (T, d) bf16 -> (out (T, d) bf16, topk_ids (T, k) int32, topk_weight (T, k) fp32).

    router_weight (E, d), w_gu (E, d, 2h) = [gate | up], w_d (E, h, d): bf16, or fp32 / fp16 (rounded to bf16 for
    the products, gradients in the weights' dtype).  logit_bias (E,) fp32 is added to the router logits (no gradient).  Gradients reach
    x and the three weights from `out` and from `topk_weight` (softmax + renormalisation Jacobian).  Without a
    gradient to record (grad mode off, or no input requiring one) the forward runs as one C call
    (ops.moe_forward): the same kernels and outputs, a fraction of the host time."""
    if not (torch.is_grad_enabled() and (x.requires_grad or router_weight.requires_grad or w_gu.requires_grad
                                         or w_d.requires_grad)):
        _check_layer_args(x, router_weight, w_gu, w_d, logit_bias, top_k)
        out, ids, tw, _ = ops.moe_forward(x, _bf16(router_weight), _bf16(w_gu), _bf16(w_d), top_k, bias=logit_bias,
                                          renorm=renorm)
        return out, ids, tw
    return _MoEFunction.apply(x, router_weight, w_gu, w_d, logit_bias, top_k, renorm)


class _ExpertStackProj:
    """What the reference's initialisation code reads of the dense SwiGLU's nn.Linear projections
    (aurora/model.py:308-312 and 393-396: `lin.weight`, `lin.in_features`; train_pp.py:1420-1421 zeroes
    `mlp.out_proj.weight`): here `weight` is the stacked expert parameter itself, so nn.init.normal_(..., std=
    in_features ** -0.5) gives every expert the fan-in initialisation and nn.init.zeros_ zeroes every expert."""

    __slots__ = ("weight", "in_features", "out_features")

    def __init__(self, weight, in_features, out_features):
        self.weight, self.in_features, self.out_features = weight, in_features, out_features


def _result_dtype(h: torch.Tensor) -> torch.dtype:
    """The dtype the reference's nn.Linear-based SwiGLU returns for input h: the autocast dtype inside an autocast
    region of h's device type, else h's own dtype."""
    dev = h.device.type
    if torch.is_autocast_enabled(dev):
        return torch.get_autocast_dtype(dev)
    return h.dtype


class MoESwiGLU(nn.Module):
    """MoE replacement for aurora/model.py:102-110 `SwiGLU(dim, hidden)`: same call shape ((..., dim) -> (..., dim)).

    Parameters: router_weight (E, dim); w_gu (E, dim, 2*hidden) = [gate | up] per expert (the stacked layout of
    aurora/hf_compat.py:154, gate first as in aurora/model.py:109); w_d (E, hidden, dim).  Buffer logit_bias (E,)
    fp32 is added to the router logits (zero by default; -inf disables an expert).

    `in_proj` / `out_proj` expose w_gu / w_d with the nn.Linear attributes the reference's init code uses, so
    Denoiser.init_weights / init_block and the zeroed output projection of train_pp --init run unchanged.  The
    default initialisation is theirs: N(0, in_features ** -0.5) per projection (dim for w_gu and the router, hidden
    for w_d); `init_std` overrides it with one std for all three.

    The products run in bf16 (any other input dtype is rounded to bf16 first); the output has the dtype the
    reference's SwiGLU would return: the autocast dtype inside autocast, else the input's dtype.  The routing of the
    last call is kept in `last_topk_ids` / `last_topk_weight` (the weights carry gradient)."""

    def __init__(self, dim: int, hidden: int, experts: int, top_k: int = 2, renorm: bool = True,
                 init_std: float | None = None, device=None, dtype=torch.bfloat16):
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
        self.last_topk_weight = None

    @property
    def in_proj(self) -> _ExpertStackProj:
        return _ExpertStackProj(self.w_gu, self.dim, 2 * self.hidden)

    @property
    def out_proj(self) -> _ExpertStackProj:
        return _ExpertStackProj(self.w_d, self.hidden, self.dim)

    @torch.no_grad()
    def reset_parameters(self):
        for p, fan_in in ((self.router_weight, self.dim), (self.w_gu, self.dim), (self.w_d, self.hidden)):
            nn.init.normal_(p, std=self.init_std if self.init_std is not None else fan_in ** -0.5)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        shape = h.shape
        out_dtype = _result_dtype(h)
        x = h.reshape(-1, shape[-1])
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        out, ids, tw = moe_swiglu(x, self.router_weight, self.w_gu, self.w_d, self.top_k, self.logit_bias,
                                  self.renorm)
        self.last_topk_ids, self.last_topk_weight = ids, tw
        out = out.view(shape)
        return out if out.dtype == out_dtype else out.to(out_dtype)


def moe_param_groups(module: nn.Module, lr: float, weight_decay: float, router_lr: float | None = None):
    """Optimizer groups for every MoESwiGLU inside `module`, for a training script whose grouping rule sends 2-D
    matrices under `.blocks.` to Muon and everything else to AdamW (train.py:305-338 of the reference).  Left to that
    rule, a MoESwiGLU standing in for a block's dense SwiGLU would have its router (E, dim), a 2-D matrix, updated by
    Muon and its 3-D expert stacks w_gu / w_d put in the AdamW "other" group (no weight decay, the Adam learning
    rate), while the dense in_proj / out_proj they replace were Muon's hidden matrices.

    Returns (groups, ids).  groups: AdamW parameter groups (`params`, `lr`, `base_lr`, `weight_decay`, `name`):
      - "moe_experts": every w_gu and w_d, at `lr` (the hidden-matrix learning rate) with `weight_decay`;
      - "moe_router": every router_weight, at `router_lr` (default `lr`) without weight decay, kept out of Muon (an
        orthogonalised update would mix the experts' logit directions).
    ids: the id() of each parameter placed, to remove from the list the script's own rule groups (its `named=`
    argument), so that no parameter is in two groups."""
    experts, routers = [], []
    for m in module.modules():
        if isinstance(m, MoESwiGLU):
            experts += [p for p in (m.w_gu, m.w_d) if p.requires_grad]
            if m.router_weight.requires_grad:
                routers.append(m.router_weight)
    rlr = lr if router_lr is None else router_lr
    groups = [dict(params=experts, lr=lr, base_lr=lr, weight_decay=weight_decay, name="moe_experts"),
              dict(params=routers, lr=rlr, base_lr=rlr, weight_decay=0.0, name="moe_router")]
    groups = [g for g in groups if g["params"]]
    return groups, {id(p) for g in groups for p in g["params"]}
