"""Widths that are not multiples of the kernels' copy granule, and expert activations other than silu, on the GPU.

The reference's Triton kernel masks any K and N (aurora/moe_triton.py:43-44,56) and its fused branch applies the
module's own act_fn between the two grouped GEMMs (aurora/hf_compat.py:79-81).  Here grouped_mm zero-pads K and N to
the copy granule (8 columns, 16 for int8 weights), fuse_moe pads its stacked weights once, and a block whose act_fn
is not silu runs gate/up grouped GEMM -> act_fn(g) * u -> down grouped GEMM.  Checked against the float64 oracle
with the reference's rounding points; for a non-silu activation the hidden product is formed by torch in bf16 on the
CPU, as the reference forms it (its rounding is torch's own in both places)."""
import functools

import numpy as np
import pytest
import torch
import torch.nn as nn

from tests.util import assert_close_bf16, bits, f32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _routing(T, E, k, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    return ids, w


@pytest.mark.parametrize("dtype,wq,K,N", [(torch.bfloat16, False, 60, 36), (torch.float16, False, 44, 20),
                                          (torch.bfloat16, True, 52, 40), (torch.bfloat16, False, 3, 5),
                                          (torch.bfloat16, True, 13, 7)])
def test_grouped_mm_ragged_widths(oracle, dtype, wq, K, N):
    """grouped_mm with K % 8 != 0 and N off the granule, with gather, routing-weight scale and scatter, and on the
    sorted rows: the N valid columns against the oracle on the unpadded operands."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    print(f"grouped_mm ragged dtype={dtype} int8={wq} K={K} N={N}", flush=True)
    T, E, k = 300, 5, 2
    g = torch.Generator().manual_seed(K * 100 + N)
    ids = torch.randint(0, E, (T, k), generator=g)
    x = torch.randn(T, K, generator=g).to(dtype)
    w = torch.randn(E, K, N, generator=g) * 0.1
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E)
    a_idx, y_idx = (order // k).int(), order.int()
    sc = torch.rand(T * k, generator=g).to(dtype)
    dt = "f16" if dtype == torch.float16 else "bf16"
    if wq:
        q, s = oracle.quant_int8(w.numpy())
        wd, sd = torch.from_numpy(q).to(DEV), torch.from_numpy(s).bfloat16().to(DEV)
        wref, sref = q.astype(np.float32), s.astype(np.float64)
    else:
        wd, sd = w.to(dtype).to(DEV), None
        wref, sref = f32(w.to(dtype)), None
    y = moe_triton.grouped_mm(x.to(DEV), wd, counts.to(DEV), a_idx=a_idx.to(DEV), y_idx=y_idx.to(DEV),
                              scale=sc.to(DEV), w_scale=sd)
    assert y.shape == (T * k, N) and y.dtype == dtype and y.is_contiguous()
    ref = oracle.grouped_mm(f32(x), wref, counts.numpy(), a_idx=a_idx.numpy(), y_idx=y_idx.numpy(), scale=f32(sc),
                            w_scale=sref, dtype=dt)
    assert_close_bf16(f32(y), ref, "ragged grouped_mm fused")
    xs = x[order // k]
    y2 = moe_triton.grouped_mm(xs.to(DEV), wd, counts.to(DEV), w_scale=sd)
    ref2 = oracle.grouped_mm(f32(xs), wref, counts.numpy(), w_scale=sref, dtype=dt)
    assert_close_bf16(f32(y2), ref2, "ragged grouped_mm sorted")


class _Expert(nn.Module):
    def __init__(self, d, h, act):
        super().__init__()
        self.gate_proj = nn.Linear(d, h, bias=False)
        self.up_proj = nn.Linear(d, h, bias=False)
        self.down_proj = nn.Linear(h, d, bias=False)
        self.act_fn = act


class _MoEBlock(nn.Module):
    def __init__(self, d, h, E, act=nn.functional.silu):
        super().__init__()
        self.experts = nn.ModuleList([_Expert(d, h, act) for _ in range(E)])

    def moe_infer(self, x, topk_ids, topk_weight):  # replaced by fuse_moe
        raise AssertionError("not fused")


def _stacks(blk):
    wgu = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in blk.experts]).detach()
    wd = torch.stack([e.down_proj.weight.t() for e in blk.experts]).detach()
    return wgu, wd


@pytest.mark.parametrize("quant,d,h", [("", 36, 20), ("", 200, 44), ("int8", 40, 24), ("int8", 72, 100)])
def test_fuse_moe_ragged_widths(oracle, quant, d, h):
    """fuse_moe on experts whose model or hidden width is off the granule: the padded stacks give the layer's output
    on its d columns (oracle on the unpadded weights; for int8 the layer's own quantised values, cut to the real
    rows and columns)."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    print(f"fuse_moe ragged quant={quant!r} d={d} h={h}", flush=True)
    T, E, k = 400, 6, 2
    torch.manual_seed(d + h)
    model = nn.Sequential(_MoEBlock(d, h, E)).bfloat16()
    wgu, wd = _stacks(model[0])
    assert fuse_moe(model, quant=quant) == 1
    blk = model.cuda()[0]
    gr = 16 if quant else 8
    dp, hp = -(-d // gr) * gr, -(-h // gr) * gr
    assert blk._wgu.shape == (E, dp, 2 * hp) and blk._wd.shape == (E, hp, dp)
    ids, w = _routing(T, E, k, d * h)
    x = torch.randn(T, d, generator=torch.Generator().manual_seed(7)).bfloat16()
    y = blk.moe_infer(x.to(DEV), ids.to(DEV), w.to(DEV))
    assert y.shape == (T, d) and y.is_contiguous()
    if quant:
        q_gu, q_d = blk._wgu.cpu(), blk._wd.cpu()
        s_gu, s_d = f32(blk._wgu_s), f32(blk._wd_s)
        cols = np.r_[0:h, hp:hp + h]
        ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), f32(q_gu)[:, :d][:, :, cols], f32(q_d)[:, :h, :d],
                                 wgu_s=s_gu[:, cols], wd_s=s_d[:, :d])
    else:
        ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), f32(wgu), f32(wd))
    assert_close_bf16(f32(y), ref["out"], f"ragged moe_infer quant={quant!r}")


def _reference_act_layer(oracle, x, ids, w, wgu, wd, act):
    """aurora/hf_compat.py:75-82 with the module's activation: gate/up grouped GEMM (float64 sums rounded to bf16),
    act(g) * u by torch in bf16, down grouped GEMM scaled by the bf16 routing weight and scattered to (token, slot)
    order, fp32 sum over the k slots rounded once to bf16."""
    T, k = ids.shape
    E = wgu.shape[0]
    h = wgu.shape[2] // 2
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E).numpy()
    gu = oracle.grouped_mm(f32(x), f32(wgu), counts, a_idx=(order // k).numpy())
    gu = torch.from_numpy(gu).bfloat16()
    hid = act(gu[:, :h]) * gu[:, h:]
    ws = w.reshape(-1)[order].bfloat16()
    y = oracle.grouped_mm(f32(hid), f32(wd), counts, y_idx=order.numpy(), scale=f32(ws))
    s = y.reshape(T, k, -1)
    acc = s[:, 0].astype(np.float32)
    for j in range(1, k):
        acc = (acc + s[:, j]).astype(np.float32)
    return oracle.round_bf16(acc)


@pytest.mark.parametrize("act,d,h,quant", [(nn.GELU(approximate="tanh"), 256, 192, ""),
                                           (nn.GELU(), 36, 20, ""),
                                           (nn.ReLU(), 128, 96, "int8")])
def test_fuse_moe_other_activation(oracle, act, d, h, quant):
    """A block whose act_fn is not silu: the two grouped GEMMs with the module's activation in between, against the
    reference's order of operations (for int8 the oracle takes the layer's quantised weights dequantised exactly in
    float64, scales applied to the sums)."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    print(f"fuse_moe act={act} d={d} h={h} quant={quant!r}", flush=True)
    T, E, k = 500, 8, 2
    torch.manual_seed(h)
    model = nn.Sequential(_MoEBlock(d, h, E, act)).bfloat16()
    wgu, wd = _stacks(model[0])
    assert fuse_moe(model, quant=quant) == 1
    blk = model.cuda()[0]
    ids, w = _routing(T, E, k, 3 * d)
    x = torch.randn(T, d, generator=torch.Generator().manual_seed(9)).bfloat16()
    y = blk.moe_infer(x.to(DEV), ids.to(DEV), w.to(DEV))
    assert y.shape == (T, d)
    if quant:
        # the layer's own int8 values (aligned widths here): the reference multiplies their dequantised values
        wgu = torch.from_numpy(f32(blk._wgu).astype(np.float64) * f32(blk._wgu_s).astype(np.float64)[:, None, :])
        wd = torch.from_numpy(f32(blk._wd).astype(np.float64) * f32(blk._wd_s).astype(np.float64)[:, None, :])
    ref = _reference_act_layer(oracle, x, ids, w, wgu, wd, act)
    assert_close_bf16(f32(y), ref, f"moe_infer act={act}")


def test_generic_activation_path_equals_fused_silu():
    """The generic path (a silu the fused epilogue does not recognise: a partial of torch's silu) against the fused
    SwiGLU path on the same block: the same GEMM main loops and the same rounding points (silu then the product, each
    rounded to bf16).  The two silu evaluations (the epilogue's and torch's) may differ in the last fp32 bit, which
    moves a hidden value by one bf16 step where it falls on a rounding boundary; so nearly every output is identical
    and the rest within the bf16 tolerance."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    T, d, h, E, k = 700, 256, 320, 8, 2
    torch.manual_seed(4)
    ids, w = _routing(T, E, k, 5)
    x = torch.randn(T, d, generator=torch.Generator().manual_seed(6)).bfloat16().to(DEV)
    outs = []
    for act in (nn.functional.silu, functools.partial(nn.functional.silu)):
        torch.manual_seed(4)
        model = nn.Sequential(_MoEBlock(d, h, E, act)).bfloat16()
        assert fuse_moe(model) == 1
        outs.append(model.cuda()[0].moe_infer(x, ids.to(DEV), w.to(DEV)))
    same = (bits(outs[0]) == bits(outs[1])).mean()
    print(f"identical outputs: {same:.6f}", flush=True)
    assert same > 0.99, same
    assert_close_bf16(f32(outs[1]), f32(outs[0]), "generic vs fused silu")


@pytest.mark.parametrize("act", [nn.functional.silu, nn.GELU()])
@pytest.mark.parametrize("T", [0, 1, 3])
def test_fuse_moe_tiny_batches(oracle, act, T):
    """Empty and few-token calls through both moe_infer paths (the fused SwiGLU and the module's own activation),
    with widths off the granule: the right shape, and the values of the reference order for the tokens present."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    print(f"fuse_moe tiny T={T} act={act}", flush=True)
    d, h, E, k = 36, 20, 4, 2
    torch.manual_seed(T)
    model = nn.Sequential(_MoEBlock(d, h, E, act)).bfloat16()
    wgu, wd = _stacks(model[0])
    assert fuse_moe(model) == 1
    blk = model.cuda()[0]
    g = torch.Generator().manual_seed(31 + T)
    x = torch.randn(T, d, generator=g).bfloat16()
    ids = torch.zeros(0, k, dtype=torch.long)
    if T:
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    y = blk.moe_infer(x.to(DEV), ids.to(DEV), w.to(DEV))
    assert y.shape == (T, d) and y.dtype == torch.bfloat16
    if T:
        ref = _reference_act_layer(oracle, x, ids, w, wgu, wd, act)
        assert_close_bf16(f32(y), ref, f"tiny moe_infer T={T}")
