"""fp16 activations on the GPU against the float64 oracle with fp16 rounding points: the reference's grouped_mm
returns a.dtype for any floating input (aurora/moe_triton.py:80) and its LM loader takes a dtype
(aurora/hf_compat.py:42), so a model loaded in fp16 runs the fused path in fp16.  Covered: grouped_mm (plain,
gather / scale / scatter, int8 weights, both tile sizes), the fused gate/up + SwiGLU and down + weight + scatter
(gathered rows and row-group tiles, 16-bit and int8 weights), combine, the known-answer self-test, fuse_moe's
moe_infer on an fp16 model, and the training layer given fp16 input (computed in bf16, returned in fp16)."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from tests.util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu

F16 = torch.float16


@pytest.fixture(params=["L", "S"])
def tile(request, monkeypatch):
    monkeypatch.setenv("HMOE_GEMM_TILE", request.param)
    return request.param


@pytest.mark.parametrize("T,K,N,E,k", [(700, 520, 264, 5, 2), (2048, 1024, 1536, 16, 2), (64, 2048, 640, 128, 8)])
def test_grouped_mm_fp16(oracle, tile, T, K, N, E, k):
    from trenowanie_generatora_obrazkow_amd import moe_triton
    print(f"fp16 grouped_mm T={T} K={K} N={N} E={E} k={k} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(K + N + 1)
    ids = torch.randint(0, E, (T, k), generator=g)
    x = torch.randn(T, K, generator=g).half()
    w = (torch.randn(E, K, N, generator=g) * 0.05).half()
    sc = torch.rand(T * k, generator=g).half()
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E)
    a_idx, y_idx = (order // k).int(), order.int()
    dev = torch.device("cuda")
    y = moe_triton.grouped_mm(x.to(dev), w.to(dev), counts.to(dev), a_idx=a_idx.to(dev), y_idx=y_idx.to(dev),
                              scale=sc.to(dev))
    assert y.dtype == F16
    ref = oracle.grouped_mm(f32(x), f32(w), counts.numpy(), a_idx=a_idx.numpy(), y_idx=y_idx.numpy(), scale=f32(sc),
                            dtype="f16")
    assert_close_bf16(f32(y), ref, "fp16 grouped_mm fused")
    xs = x[order // k]
    y2 = moe_triton.grouped_mm(xs.to(dev), w.to(dev), counts.to(dev))
    assert_close_bf16(f32(y2), oracle.grouped_mm(f32(xs), f32(w), counts.numpy(), dtype="f16"), "fp16 sorted")
    # int8 weights with fp16 activations (the reference's scales are bf16, aurora/hf_compat.py:110)
    if N % 16 == 0:
        q, s = oracle.quant_int8(f32(w))
        y3 = moe_triton.grouped_mm(xs.to(dev), torch.from_numpy(q).to(dev), counts.to(dev),
                                   w_scale=torch.from_numpy(s).bfloat16().to(dev))
        ref3 = oracle.grouped_mm(f32(xs), q.astype(np.float32), counts.numpy(), w_scale=s.astype(np.float64),
                                 dtype="f16")
        assert_close_bf16(f32(y3), ref3, "fp16 grouped_mm int8 weights")


def test_fp16_is_not_bf16(oracle):
    """The fp16 path rounds to fp16, not bf16: on the same values its output is much closer to the fp16-rounded
    oracle than a bf16 rounding could be (bf16 keeps 8 significant bits, fp16 11), and it has fp16's bit patterns."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    g = torch.Generator().manual_seed(3)
    a = torch.randn(256, 128, generator=g).half()
    w = (torch.randn(2, 128, 64, generator=g) * 0.1).half()
    counts = torch.tensor([100, 156])
    y = f32(moe_triton.grouped_mm(a.cuda(), w.cuda(), counts.cuda()))
    exact = oracle.grouped_mm(f32(a), f32(w), counts.numpy(), round_out=False)
    rel = np.abs(y - exact).max() / np.abs(exact).max()
    assert rel < 2.0 ** -11, rel
    assert np.abs(oracle.round_bf16(exact) - exact).max() / np.abs(exact).max() > 2.0 ** -10


@pytest.mark.parametrize("T,d,E,k,h,wdt", [(600, 256, 6, 2, 320, "f16"), (600, 256, 6, 2, 320, "int8"),
                                           (300, 256, 4, 2, 4096, "f16")])
def test_fused_projections_fp16(oracle, tile, T, d, E, k, h, wdt):
    """routed_gate_up (gathered rows, or the row-group tiles from h = 4096 on) and down_scatter, then combine, in
    fp16, against the oracle's act rows and layer output with fp16 rounding points."""
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"fp16 fused T={T} d={d} E={E} k={k} h={h} w={wdt} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(h + T)
    x = torch.randn(T, d, generator=g).half()
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.05).half()
    wd = (torch.randn(E, h, d, generator=g) * 0.05).half()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    tw = torch.rand(T, k, generator=g).softmax(-1)
    dev = torch.device("cuda")
    if wdt == "int8":
        qgu, sgu = oracle.quant_int8(f32(wgu))
        qd, sd = oracle.quant_int8(f32(wd))
        wgu_d, wd_d = torch.from_numpy(qgu).to(dev), torch.from_numpy(qd).to(dev)
        sgu_d, sd_d = torch.from_numpy(sgu).bfloat16().to(dev), torch.from_numpy(sd).bfloat16().to(dev)
        ref = oracle.moe_forward(f32(x), ids.numpy(), tw.numpy(), qgu.astype(np.float32), qd.astype(np.float32),
                                 wgu_s=sgu, wd_s=sd, dtype="f16")
    else:
        wgu_d, wd_d, sgu_d, sd_d = wgu.to(dev), wd.to(dev), None, None
        ref = oracle.moe_forward(f32(x), ids.numpy(), tw.numpy(), f32(wgu), f32(wd), dtype="f16")
    M = T * k
    disp, act, _ = ops.routed_gate_up(x.to(dev), ids.int().to(dev), E, wgu_d, topk_w=tw.to(dev), wgu_s=sgu_d)
    assert act.dtype == F16 and disp.w_sorted.dtype == F16
    # the sorted routing weights are the fp32 weights rounded to fp16 (the .to(x.dtype) of aurora/hf_compat.py:80)
    order = disp.order.cpu().numpy()
    np.testing.assert_array_equal(f32(disp.w_sorted), oracle.round_f16(tw.numpy().reshape(-1)[order]))
    assert_close_bf16(f32(act), ref["act"][order], "fp16 act")
    y, _ = ops.down_scatter(act, wd_d, disp.counts, M, disp.w_sorted, disp.order, wd_s=sd_d)
    out = ops.combine(y, T, k)
    assert out.dtype == F16
    assert_close_bf16(f32(y), ref["y"], "fp16 y")
    assert_close_bf16(f32(out), ref["out"], "fp16 out")
    # combine is exact given y: fp32 sum of the slots in order, one fp16 rounding
    s = f32(y).reshape(T, k, d).astype(np.float32)
    acc = s[:, 0].copy()
    for j in range(1, k):
        acc = (acc + s[:, j]).astype(np.float32)
    np.testing.assert_array_equal(f32(out), oracle.round_f16(acc))


def test_self_test_and_moe_infer_fp16(oracle):
    """_pick_mode's known-answer tests in fp16 (aurora/hf_compat.py:112-139 with dtype = fp16) and fuse_moe's
    moe_infer on an fp16 model, 16-bit and int8 experts, against the oracle with fp16 rounding points."""
    from tests.test_gpu_layer import _MoEBlock
    from trenowanie_generatora_obrazkow_amd.hf_compat import _pick_mode, fuse_moe
    assert _pick_mode(torch.device("cuda"), F16) == "hip"
    T, d, h, E, k = 500, 256, 320, 8, 4
    for quant in ("", "int8"):
        torch.manual_seed(11)
        model = nn.Sequential(_MoEBlock(d, h, E)).half()
        wgu_ref = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in model[0].experts])
        wd_ref = torch.stack([e.down_proj.weight.t() for e in model[0].experts])
        assert fuse_moe(model, quant=quant) == 1
        model = model.cuda()
        g = torch.Generator().manual_seed(12)
        x = torch.randn(T, d, generator=g).half()
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
        w = torch.rand(T, k, generator=g).softmax(-1)
        y = model[0].moe_infer(x.cuda(), ids.cuda(), w.cuda())
        assert model[0]._mode == "hip" and y.dtype == F16
        if quant:
            sgu, sd = f32(model[0]._wgu_s), f32(model[0]._wd_s)
            ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), f32(model[0]._wgu), f32(model[0]._wd),
                                     wgu_s=sgu, wd_s=sd, dtype="f16")
        else:
            ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), f32(wgu_ref), f32(wd_ref), dtype="f16")
        assert_close_bf16(f32(y), ref["out"], f"fp16 moe_infer quant={quant!r}")


def test_layer_fp16_input():
    """MoESwiGLU given fp16 input and fp16 weights: the products run in bf16 (input and weights rounded to bf16, as
    for fp32 ones), the output and the input gradient have the input's dtype, and the weight gradients are the fp32
    gradients rounded once to fp16 -- bit for bit what the fp32-master-weight module holding the same values gives,
    rounded to fp16."""
    from trenowanie_generatora_obrazkow_amd import MoESwiGLU
    B, T, dim, hidden, E, k = 2, 96, 256, 320, 8, 2
    torch.manual_seed(7)
    mh = MoESwiGLU(dim, hidden, E, top_k=k, dtype=F16).cuda()
    m32 = MoESwiGLU(dim, hidden, E, top_k=k, dtype=torch.float32).cuda()
    with torch.no_grad():
        for p32, ph in ((m32.router_weight, mh.router_weight), (m32.w_gu, mh.w_gu), (m32.w_d, mh.w_d)):
            p32.copy_(ph.float())
    g = torch.Generator().manual_seed(8)
    h = torch.randn(B, T, dim, generator=g).half().cuda()
    dout = torch.randn(B, T, dim, generator=g).cuda()
    res = []
    for mod in (mh, m32):
        hg = h.clone().requires_grad_(True)
        o = mod(hg)
        (o.float() * dout).sum().backward()
        res.append((o, hg.grad))
    torch.cuda.synchronize()
    (oh, gh), (o32, g32) = res
    assert oh.dtype == F16 and o32.dtype == F16 and gh.dtype == F16
    assert torch.equal(oh, o32) and torch.equal(gh, g32)
    for ph, p32 in ((mh.router_weight, m32.router_weight), (mh.w_gu, m32.w_gu), (mh.w_d, m32.w_d)):
        assert ph.grad.dtype == F16 and p32.grad.dtype == torch.float32
        assert torch.equal(ph.grad, p32.grad.half()), "fp16 weight gradient"
