"""int8 weight-only expert GEMMs on the GPU against the float64 oracle (aurora/moe_triton.py:44-51: the int8
weights enter the bf16 products exactly, the per-(expert, column) scale multiplies the fp32 sum before the row
scale).  Covers both tile sizes, bf16 and fp32 scales, gather / scale / scatter, ragged N and K tails, the reference's
quantised self-test, the fused gate/up + SwiGLU and down + scatter forms, and fuse_moe(quant="int8") end to end."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from tests.util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["L", "S"])
def tile(request, monkeypatch):
    monkeypatch.setenv("HMOE_GEMM_TILE", request.param)
    return request.param


def _quant(oracle, w, scale_dtype):
    """oracle.quant_int8 -> (int8 torch, scales torch of scale_dtype, scales as float64 for the oracle)."""
    q, s = oracle.quant_int8(w)
    if scale_dtype == torch.float32:  # unrounded fp32 scales (the kernel takes either)
        s = (np.maximum(np.abs(w).max(axis=1), 1e-8) / np.float32(127)).astype(np.float32)
    st = torch.from_numpy(np.ascontiguousarray(s, dtype=np.float32)).to(scale_dtype)
    return torch.from_numpy(q), st, st.double().numpy()


def test_self_test_quant(tile):
    """The reference's quantised known-answer test (aurora/hf_compat.py:112-121 with quant=True)."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    from trenowanie_generatora_obrazkow_amd.hf_compat import _self_test
    fn = lambda a, w, s, c: moe_triton.grouped_mm(a, w, c, w_scale=s)  # noqa: E731
    assert _self_test(fn, torch.device("cuda"), torch.bfloat16, quant=True)


@pytest.mark.parametrize("T,K,N,E,k,skew,sdt", [(1024, 256, 512, 8, 2, 0, torch.bfloat16),
                                                (700, 520, 272, 5, 2, 1, torch.float32),
                                                (2048, 1024, 1536, 16, 1, 1, torch.bfloat16),
                                                (64, 2048, 640, 128, 8, 0, torch.float32)])
def test_grouped_mm_int8(oracle, tile, T, K, N, E, k, skew, sdt):
    from trenowanie_generatora_obrazkow_amd import moe_triton
    print(f"grouped_mm int8 T={T} K={K} N={N} E={E} k={k} skew={skew} scale={sdt} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(K + N + 1)
    if skew:
        p = torch.tensor([0.0 if e == 1 else 2.0 ** (-e) for e in range(E)])
        ids = torch.multinomial(p / p.sum(), T * k, replacement=True, generator=g).view(T, k)
    else:
        ids = torch.randint(0, E, (T, k), generator=g)
    x = torch.randn(T, K, generator=g).bfloat16()
    # column magnitudes spread over a decade, so a mis-indexed scale shows
    w = (torch.randn(E, K, N, generator=g) * torch.logspace(-2, -1, N)).numpy()
    q, s, s64 = _quant(oracle, w, sdt)
    sc = torch.rand(T * k, generator=g).bfloat16()
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E)
    a_idx = (order // k).int()
    y_idx = order.int()
    dev = torch.device("cuda")
    qd, sd = q.to(dev), s.to(dev)
    y = moe_triton.grouped_mm(x.to(dev), qd, counts.to(dev), a_idx=a_idx.to(dev), y_idx=y_idx.to(dev),
                              scale=sc.to(dev), w_scale=sd)
    qf = q.numpy().astype(np.float32)
    ref = oracle.grouped_mm(f32(x), qf, counts.numpy(), a_idx=a_idx.numpy(), y_idx=y_idx.numpy(), scale=f32(sc),
                            w_scale=s64)
    assert_close_bf16(f32(y), ref, "grouped_mm int8 fused")
    xs = x[order // k]
    y2 = moe_triton.grouped_mm(xs.to(dev), qd, counts.to(dev), w_scale=sd)
    ref2 = oracle.grouped_mm(f32(xs), qf, counts.numpy(), w_scale=s64)
    assert_close_bf16(f32(y2), ref2, "grouped_mm int8 sorted")


@pytest.mark.parametrize("T,d,h,E,k,sdt", [(2000, 1024, 512, 16, 2, torch.bfloat16),
                                          (333, 528, 272, 40, 4, torch.float32)])
def test_fused_int8_projections(oracle, tile, T, d, h, E, k, sdt):
    """gate/up with the SwiGLU epilogue and down with routing weight + scatter, int8 weights, against the oracle's
    forward with the same scales (act in sorted order, y and the combined output in token order)."""
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"fused int8 T={T} d={d} h={h} E={E} k={k} scale={sdt} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(T + d)
    x = torch.randn(T, d, generator=g).bfloat16()
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.03).numpy()
    wd = (torch.randn(E, h, d, generator=g) * 0.03).numpy()
    qgu, sgu, sgu64 = _quant(oracle, wgu, sdt)
    qd, sd, sd64 = _quant(oracle, wd, sdt)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    tw = torch.rand(T, k, generator=g).softmax(-1)
    dev = torch.device("cuda")
    disp = ops.dispatch(ids.int().to(dev), E, topk_w=tw.to(dev), want_inv=False)
    M = T * k
    act, gu = ops.gate_up_swiglu(x.to(dev), qgu.to(dev), disp.counts, M, a_idx=disp.a_idx, wgu_s=sgu.to(dev))
    assert gu is None
    y, yhat = ops.down_scatter(act, qd.to(dev), disp.counts, M, disp.w_sorted, disp.order, wd_s=sd.to(dev))
    assert yhat is None
    out = ops.combine(y, T, k)
    ref = oracle.moe_forward(f32(x), ids.numpy(), tw.numpy(), qgu.numpy().astype(np.float32),
                             qd.numpy().astype(np.float32), wgu_s=sgu64, wd_s=sd64)
    order = disp.order.cpu().numpy().astype(np.int64)
    assert_close_bf16(f32(act), ref["act"][order], "act")
    assert_close_bf16(f32(y), ref["y"], "y")
    assert_close_bf16(f32(out), ref["out"], "out")


class _Expert(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.gate_proj = nn.Linear(d, h, bias=False)
        self.up_proj = nn.Linear(d, h, bias=False)
        self.down_proj = nn.Linear(h, d, bias=False)
        self.act_fn = nn.functional.silu


class _MoEBlock(nn.Module):
    def __init__(self, d, h, E):
        super().__init__()
        self.experts = nn.ModuleList([_Expert(d, h) for _ in range(E)])

    def moe_infer(self, x, topk_ids, topk_weight):  # replaced by fuse_moe
        raise AssertionError("not fused")


def test_fuse_moe_int8_infer(oracle):
    """fuse_moe(model, quant="int8") then moe_infer: the quantised layer against the oracle with the layer's own
    int8 weights and scales."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    T, d, h, E, k = 1000, 512, 320, 16, 4
    torch.manual_seed(2)
    model = nn.Sequential(_MoEBlock(d, h, E)).bfloat16()
    assert fuse_moe(model, quant="int8") == 1
    model = model.cuda()
    blk = model[0]
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, d, generator=g).bfloat16()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    y = blk.moe_infer(x.cuda(), ids.cuda(), w.cuda())
    assert blk._mode == "hip"
    ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), blk._wgu.cpu().numpy().astype(np.float32),
                             blk._wd.cpu().numpy().astype(np.float32), wgu_s=f32(blk._wgu_s).astype(np.float64),
                             wd_s=f32(blk._wd_s).astype(np.float64))
    assert_close_bf16(f32(y), ref["out"], "moe_infer int8")
