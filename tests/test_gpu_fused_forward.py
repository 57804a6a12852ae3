"""The one-call forward (hmoe_moe_forward, ops.moe_forward) against the same layer driven entry point by entry
point: out, topk_ids, topk_w and logits bit-identical, on both gate/up forms (row-group tiles from h = 4096 on, rows
gathered through a_idx below), ragged widths and counts, a logit bias, no renormalisation, one token and none; and
moe_swiglu without a gradient to record (the one-call path) against the same call recording one (the autograd
path)."""
import numpy as np
import pytest
import torch

from tests.util import make_inputs

pytestmark = pytest.mark.gpu


def _op_by_op(x, wr, wgu, wd, k, bias, renorm):
    from trenowanie_generatora_obrazkow_amd import ops
    T = x.shape[0]
    E = wgu.shape[0]
    logits, ids, tw = ops.route_topk(x, wr, k, bias=bias, renorm=renorm)
    disp, act, _ = ops.routed_gate_up(x, ids, E, wgu, topk_w=tw)
    y, _ = ops.down_scatter(act, wd, disp.counts, T * k, disp.w_sorted, disp.order)
    return ops.combine(y, T, k), ids, tw, logits


def _same(a, b, name):
    assert a.shape == b.shape and a.dtype == b.dtype, name
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b), name


@pytest.mark.parametrize("T,d,E,k,h,bias,renorm", [(512, 256, 8, 2, 512, False, True),
                                                   (2048, 1024, 8, 2, 2048, True, True),
                                                   (600, 1536, 16, 2, 4096, False, True),
                                                   (77, 520, 5, 3, 24, True, False),
                                                   (300, 256, 64, 6, 96, False, True),
                                                   (1, 264, 12, 4, 40, True, True)])
def test_one_call_forward_matches_op_by_op(T, d, E, k, h, bias, renorm):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"moe_forward T={T} d={d} E={E} k={k} h={h} bias={bias} renorm={renorm}", flush=True)
    dev = torch.device("cuda")
    x, wr, wgu, wd = (t.to(dev) for t in make_inputs(T, d, E, h, seed=T + h))
    b = torch.linspace(-0.3, 0.3, E, device=dev) if bias else None
    ref = _op_by_op(x, wr, wgu, wd, k, b, renorm)
    out, ids, tw, logits = ops.moe_forward(x, wr, wgu, wd, k, bias=b, renorm=renorm, want_logits=True)
    torch.cuda.synchronize()
    for got, want, name in zip((out, ids, tw, logits), ref, ("out", "topk_ids", "topk_w", "logits")):
        _same(got, want, name)
    # a second call with the intermediates of the first still in the caching allocator: same bits
    out2, ids2, tw2, _ = ops.moe_forward(x, wr, wgu, wd, k, bias=b, renorm=renorm)
    _same(out2, out, "out (second call)")
    _same(ids2, ids, "topk_ids (second call)")


def test_one_call_forward_strided_rows_and_empty():
    from trenowanie_generatora_obrazkow_amd import ops
    dev = torch.device("cuda")
    x, wr, wgu, wd = (t.to(dev) for t in make_inputs(130, 512, 8, 128, seed=5))
    wide = torch.zeros(130, 640, device=dev, dtype=torch.bfloat16)
    wide[:, :512] = x
    xs = wide[:, :512]  # rows 640 elements apart
    ref = _op_by_op(x, wr, wgu, wd, 2, None, True)
    out, ids, tw, _ = ops.moe_forward(xs, wr, wgu, wd, 2)
    _same(out, ref[0], "out")
    _same(ids, ref[1], "topk_ids")
    out0, ids0, tw0, _ = ops.moe_forward(x[:0], wr, wgu, wd, 2)
    assert out0.shape == (0, 512) and ids0.shape == (0, 2) and tw0.shape == (0, 2)


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_moe_swiglu_no_grad_uses_one_call_with_same_result(wdt):
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    dev = torch.device("cuda")
    x, wr, wgu, wd = (t.to(dev) for t in make_inputs(1000, 768, 16, 256, seed=7))
    wr, wgu, wd = (t.to(wdt) for t in (wr, wgu, wd))
    bias = torch.linspace(-0.2, 0.2, 16, device=dev)
    with torch.no_grad():
        out_ng, ids_ng, tw_ng = moe_swiglu(x, wr, wgu, wd, 2, logit_bias=bias)
    params = [t.clone().requires_grad_(True) for t in (wr, wgu, wd)]
    out_g, ids_g, tw_g = moe_swiglu(x, *params, 2, logit_bias=bias)
    assert out_g.requires_grad and not out_ng.requires_grad
    _same(out_ng, out_g.detach(), "out")
    _same(ids_ng, ids_g, "topk_ids")
    _same(tw_ng, tw_g.detach(), "topk_w")
    # the module under inference mode takes the same path
    from trenowanie_generatora_obrazkow_amd import MoESwiGLU
    m = MoESwiGLU(768, 256, 16, 2).to(dev)
    h_in = torch.randn(2, 50, 768, device=dev).bfloat16()
    with torch.inference_mode():
        a = m(h_in)
    b_ = m(h_in).detach()
    assert np.array_equal(a.float().cpu().numpy(), b_.float().cpu().numpy())


def test_one_call_forward_under_the_bench_probe():
    """With bench.py's event probe set, moe_forward launches the same entry points one by one (so that events can
    sit between them) and records the probed ops; the outputs are the one-call ones."""
    from trenowanie_generatora_obrazkow_amd import ops
    dev = torch.device("cuda")
    x, wr, wgu, wd = (t.to(dev) for t in make_inputs(700, 512, 40, 256, seed=11))
    ref = ops.moe_forward(x, wr, wgu, wd, 4, want_logits=True)
    ops.probe = {"gate_up_swiglu": [], "combine": []}
    try:
        got = ops.moe_forward(x, wr, wgu, wd, 4, want_logits=True)
        torch.cuda.synchronize()
        assert len(ops.probe["gate_up_swiglu"]) == 1 and len(ops.probe["combine"]) == 1
    finally:
        ops.probe = None
    for a, b, name in zip(got, ref, ("out", "topk_ids", "topk_w", "logits")):
        _same(a, b, name)


@pytest.mark.parametrize("T,d,E,k,h,wdt,bad", [(64, 2048, 128, 8, 320, "int8", False), (700, 520, 12, 3, 264, "bf16", True),
                                               (300, 1536, 16, 2, 4096, "bf16", False), (500, 256, 8, 2, 512, "fp16", False),
                                               (1, 256, 4, 2, 64, "int8", True), (0, 256, 4, 2, 64, "bf16", False)])
def test_one_call_experts_matches_op_by_op(T, d, E, k, h, wdt, bad):
    """hmoe_moe_experts (ops.moe_experts) against routed_gate_up + down_scatter on the same routing: y on the routed
    rows, inv_pos and n_invalid bit-identical, for bf16, fp16 and int8 experts, the row-group tiles (h = 4096), ids
    outside [0, E) and an empty input."""
    from trenowanie_generatora_obrazkow_amd import ops
    from trenowanie_generatora_obrazkow_amd.hf_compat import _quant_int8
    print(f"moe_experts T={T} d={d} E={E} k={k} h={h} {wdt} bad={bad}", flush=True)
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(T + E + h)
    act_dt = torch.float16 if wdt == "fp16" else torch.bfloat16
    x = torch.randn(T, d, generator=g).to(act_dt).to(dev)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int() if T else torch.zeros(0, k).int()
    if bad and T:
        ids.view(-1)[0] = E + 3
    ids = ids.to(dev)
    tw = torch.rand(T, k, generator=g).to(dev)
    wgu = torch.randn(E, d, 2 * h, generator=g) * 0.02
    wd = torch.randn(E, h, d, generator=g) * 0.02
    wgu_s = wd_s = None
    if wdt == "int8":
        (wgu, wgu_s), (wd, wd_s) = _quant_int8(wgu), _quant_int8(wd)
        wgu_s, wd_s = wgu_s.to(dev), wd_s.to(dev)
    else:
        wgu, wd = wgu.to(act_dt), wd.to(act_dt)
    wgu, wd = wgu.to(dev), wd.to(dev)
    disp, act, _ = ops.routed_gate_up(x, ids, E, wgu, topk_w=tw, wgu_s=wgu_s, want_inv=True)
    y_ref, _ = ops.down_scatter(act, wd, disp.counts, T * k, disp.w_sorted, disp.order, wd_s=wd_s)
    y, inv, n_inv = ops.moe_experts(x, ids, tw, wgu, wd, wgu_s=wgu_s, wd_s=wd_s)
    torch.cuda.synchronize()
    _same(inv, disp.inv_pos, "inv_pos")
    _same(n_inv, disp.n_invalid, "n_invalid")
    routed = inv.long() >= 0  # slots routed nowhere leave their y rows unwritten
    _same(y[routed], y_ref[routed], "y")
    out = ops.combine(y, T, k, inv_pos=inv)
    _same(out, ops.combine(y_ref, T, k, inv_pos=disp.inv_pos), "combined")
