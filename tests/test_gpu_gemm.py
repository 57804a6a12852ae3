"""Grouped GEMM parity on the GPU against the float64 oracle: the reference's own known-answer construction
(aurora/hf_compat.py:112-121), ragged / skewed / empty experts, gather, scatter and row scale, both tile sizes,
and the weight-gradient (ragged-K) GEMM."""
import os

import numpy as np
import pytest
import torch

from tests.util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["L", "S"])
def tile(request, monkeypatch):
    monkeypatch.setenv("HMOE_GEMM_TILE", request.param)
    return request.param


def test_self_test_shape(oracle, tile):
    """48x64 @ (3, 64, 32), counts [16, 0, 32]: the reference's _self_test, plus the tighter bf16 bound."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    from trenowanie_generatora_obrazkow_amd.hf_compat import _self_test
    g = torch.Generator().manual_seed(0)
    a = torch.randn(48, 64, generator=g).bfloat16()
    w = torch.randn(3, 64, 32, generator=g).bfloat16()
    counts = torch.tensor([16, 0, 32])
    y = moe_triton.grouped_mm(a.cuda(), w.cuda(), counts.cuda())
    ref = oracle.grouped_mm(f32(a), f32(w), counts.numpy())
    assert_close_bf16(f32(y), ref, "self-test shape")
    assert _self_test(lambda a_, w_, s_, c_: moe_triton.grouped_mm(a_, w_, c_, w_scale=s_), torch.device("cuda"),
                      torch.bfloat16)


@pytest.mark.parametrize("T,K,N,E,k,skew", [(1024, 256, 512, 8, 2, 0), (700, 520, 264, 5, 2, 1),
                                            (2048, 1024, 1536, 16, 1, 1), (64, 2048, 640, 128, 8, 0)])
def test_grouped_mm_fused(oracle, tile, T, K, N, E, k, skew):
    """gather (a_idx), scale, scatter (y_idx) as _fused_moe_infer's second call uses them."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    print(f"grouped_mm T={T} K={K} N={N} E={E} k={k} skew={skew} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(K + N)
    if skew:
        p = torch.tensor([0.0 if e == 1 else 2.0 ** (-e) for e in range(E)])
        ids = torch.multinomial(p / p.sum(), T * k, replacement=True, generator=g).view(T, k)
    else:
        ids = torch.randint(0, E, (T, k), generator=g)
    x = torch.randn(T, K, generator=g).bfloat16()
    w = (torch.randn(E, K, N, generator=g) * 0.05).bfloat16()
    sc = torch.rand(T * k, generator=g).bfloat16()
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E)
    a_idx = (order // k).int()
    y_idx = order.int()
    dev = torch.device("cuda")
    y = moe_triton.grouped_mm(x.to(dev), w.to(dev), counts.to(dev), a_idx=a_idx.to(dev), y_idx=y_idx.to(dev),
                              scale=sc.to(dev))
    ref = oracle.grouped_mm(f32(x), f32(w), counts.numpy(), a_idx=a_idx.numpy(), y_idx=y_idx.numpy(), scale=f32(sc))
    assert_close_bf16(f32(y), ref, "grouped_mm fused")
    # plain sorted rows
    xs = x[order // k]
    y2 = moe_triton.grouped_mm(xs.to(dev), w.to(dev), counts.to(dev))
    ref2 = oracle.grouped_mm(f32(xs), f32(w), counts.numpy())
    assert_close_bf16(f32(y2), ref2, "grouped_mm sorted")


@pytest.mark.parametrize("counts", [[257, 320, 321, 128, 129, 0, 255, 512, 1, 64],
                                    [63, 65, 191, 193, 0, 0, 700, 2]])
def test_grouped_mm_partial_tiles(oracle, tile, counts):
    """Expert ends that leave 1, 63-65, 127-129, 191-193 or 255 rows in a partial m-tile (run with the empty 64-row
    fragment rows skipped), a last sorted row whose bf16 routing weight sits in the low half of a dword at the end of
    the array, plain and with gather / scale / scatter, bf16 and int8 weights."""
    from trenowanie_generatora_obrazkow_amd import moe_triton
    print(f"partial tiles counts={counts} tile={tile}", flush=True)
    E, K, N = len(counts), 264, 320
    M = sum(counts)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(E, K, N, generator=g) * 0.05).bfloat16()
    c = torch.tensor(counts)
    perm = torch.randperm(M, generator=g)
    a_idx, y_idx = perm.int(), torch.randperm(M, generator=g).int()
    sc = torch.rand(M, generator=g).bfloat16()
    dev = torch.device("cuda")
    y = moe_triton.grouped_mm(x.to(dev), w.to(dev), c.to(dev))
    assert_close_bf16(f32(y), oracle.grouped_mm(f32(x), f32(w), c.numpy()), "partial plain")
    y = moe_triton.grouped_mm(x.to(dev), w.to(dev), c.to(dev), a_idx=a_idx.to(dev), y_idx=y_idx.to(dev),
                              scale=sc.to(dev))
    ref = oracle.grouped_mm(f32(x), f32(w), c.numpy(), a_idx=a_idx.numpy(), y_idx=y_idx.numpy(), scale=f32(sc))
    assert_close_bf16(f32(y), ref, "partial fused")
    q, s = oracle.quant_int8(f32(w))
    y = moe_triton.grouped_mm(x.to(dev), torch.from_numpy(q).to(dev), c.to(dev),
                              w_scale=torch.from_numpy(s).bfloat16().to(dev))
    ref = oracle.grouped_mm(f32(x), q.astype(np.float32), c.numpy(), w_scale=s.astype(np.float64))
    assert_close_bf16(f32(y), ref, "partial int8")


@pytest.mark.parametrize("h", [320, 192, 208, 64])
@pytest.mark.parametrize("wdt", ["bf16", "int8"])
def test_gate_up_swiglu_partial_n(oracle, tile, h, wdt):
    """gate/up + SwiGLU where the last n-tile holds at most 64 of its 128 gate columns (h = 320, 192, 64: the large
    tile runs that n-tile on its live fragments only) or more (h = 208), bf16 and int8 weights, against the oracle's
    act rows."""
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"gate_up partial n h={h} w={wdt} tile={tile}", flush=True)
    T, d, E, k = 600, 256, 6, 2
    g = torch.Generator().manual_seed(h)
    x = torch.randn(T, d, generator=g).bfloat16()
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.05).bfloat16()
    wd = (torch.randn(E, h, d, generator=g) * 0.05).bfloat16()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    tw = torch.rand(T, k, generator=g).softmax(-1)
    dev = torch.device("cuda")
    disp = ops.dispatch(ids.int().to(dev), E, topk_w=tw.to(dev), want_inv=False)
    if wdt == "int8":
        q, s = oracle.quant_int8(f32(wgu))
        act, _ = ops.gate_up_swiglu(x.to(dev), torch.from_numpy(q).to(dev), disp.counts, T * k, a_idx=disp.a_idx,
                                    wgu_s=torch.from_numpy(s).bfloat16().to(dev))
        ref = oracle.moe_forward(f32(x), ids.numpy(), tw.numpy(), q.astype(np.float32), f32(wd),
                                 wgu_s=s.astype(np.float64))
    else:
        act, _ = ops.gate_up_swiglu(x.to(dev), wgu.to(dev), disp.counts, T * k, a_idx=disp.a_idx)
        ref = oracle.moe_forward(f32(x), ids.numpy(), tw.numpy(), f32(wgu), f32(wd))
    order = disp.order.cpu().numpy().astype(np.int64)
    assert_close_bf16(f32(act), ref["act"][order], f"act h={h} {wdt}")


@pytest.mark.parametrize("M,P,N,E,skew", [(4096, 256, 512, 8, 0), (3000, 520, 264, 5, 1), (777, 128, 1024, 16, 1)])
def test_grouped_wgrad(oracle, tile, M, P, N, E, skew):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"wgrad M={M} P={P} N={N} E={E} tile={tile}", flush=True)
    g = torch.Generator().manual_seed(M)
    if skew:
        p = torch.tensor([0.0 if e == 2 else 3.0 ** (-e) for e in range(E)])
        ids = torch.multinomial(p / p.sum(), M, replacement=True, generator=g)
    else:
        ids = torch.randint(0, E, (M,), generator=g)
    counts = torch.bincount(ids, minlength=E)
    a = torch.randn(M, P, generator=g).bfloat16()
    b = torch.randn(M, N, generator=g).bfloat16()
    dev = torch.device("cuda")
    for dt in (torch.float32, torch.bfloat16):
        dw = ops.grouped_wgrad(a.to(dev), b.to(dev), counts.int().to(dev), E, dtype=dt)
        ref = np.zeros((E, P, N))  # float64; compared after one rounding to the output dtype
        st = 0
        a64, b64 = f32(a).astype(np.float64), f32(b).astype(np.float64)
        for e, c in enumerate(counts.tolist()):
            ref[e] = a64[st:st + c].T @ b64[st:st + c]
            st += c
        assert_close_bf16(f32(dw), oracle.round_bf16(ref) if dt == torch.bfloat16 else ref, f"wgrad {dt}")
        assert (f32(dw)[counts.numpy() == 0] == 0).all()


def test_ops_reject_bad_inputs():
    """The tensor wrappers stop wrong shapes, dtypes and layouts before the C entry points (whose kernels trust the
    sizes they are given)."""
    from trenowanie_generatora_obrazkow_amd import ops
    dev = torch.device("cuda")
    E, d, h, M = 4, 64, 32, 40
    wgu = torch.zeros(E, d, 2 * h, dtype=torch.bfloat16, device=dev)
    wd = torch.zeros(E, h, d, dtype=torch.bfloat16, device=dev)
    counts = torch.tensor([10, 10, 10, 10], dtype=torch.int32, device=dev)
    x = torch.zeros(M, d, dtype=torch.bfloat16, device=dev)
    with pytest.raises(TypeError):
        ops.gate_up_swiglu(x.float(), wgu, counts, M)
    with pytest.raises(ValueError):
        ops.gate_up_swiglu(x[:, :32], wgu, counts, M)                       # wrong d
    with pytest.raises(ValueError):
        ops.gate_up_swiglu(x[:20], wgu, counts, M)                          # too few rows, no gather
    with pytest.raises(ValueError):
        ops.gate_up_swiglu(x, wgu, counts, M, a_idx=torch.zeros(M - 1, dtype=torch.int32, device=dev))
    act = torch.zeros(M, h, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.down_scatter(act[:, :16], wd, counts, M, None, None)
    with pytest.raises(ValueError):
        ops.combine(torch.zeros(M - 2, d, dtype=torch.bfloat16, device=dev), M // 2, 2)
    with pytest.raises(ValueError):
        ops.unpermute_bwd(torch.zeros(M, d, device=dev), torch.zeros(M, dtype=torch.int32, device=dev), M // 2, 2,
                          dlogits=torch.zeros(M // 2, E, device=dev))


def test_ops_reject_mismatched_stacks():
    """One expert count and one width across router, expert stacks and bias; weights of the wrong dtype are refused
    (never reinterpreted as bf16); grouped_mm's scale and out must cover its M rows.  All of it raises before any
    kernel is launched."""
    from trenowanie_generatora_obrazkow_amd import moe_swiglu, ops
    dev = torch.device("cuda")
    E, d, h, T, k = 4, 64, 32, 20, 2
    M = T * k
    bf = dict(dtype=torch.bfloat16, device=dev)
    x = torch.zeros(T, d, **bf)
    wr, wgu, wd = torch.zeros(E, d, **bf), torch.zeros(E, d, 2 * h, **bf), torch.zeros(E, h, d, **bf)
    with pytest.raises(ValueError):
        moe_swiglu(x, torch.zeros(E + 1, d, **bf), wgu, wd, k)               # router names a 5th expert
    with pytest.raises(ValueError):
        moe_swiglu(x, wr, wgu, torch.zeros(E, h, d + 8, **bf), k)            # down stack of another width
    with pytest.raises(ValueError):
        moe_swiglu(x, wr, wgu, wd, k, logit_bias=torch.zeros(E + 1, device=dev))
    with pytest.raises(ValueError):
        moe_swiglu(x, wr, wgu, wd, E + 1)
    with pytest.raises(TypeError):
        moe_swiglu(x, wr, wgu.to(torch.int8), wd, k)
    with pytest.raises(TypeError):  # 16-bit weights must have the activations' type (bf16 with bf16, fp16 with fp16)
        ops.gate_up_swiglu(x, wgu.half(), torch.full((E,), M // E, dtype=torch.int32, device=dev), M,
                           a_idx=torch.zeros(M, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        ops.route_topk(x, torch.zeros(E, d + 8, **bf), k)
    with pytest.raises(ValueError):
        ops.route_topk(x, wr, k, bias=torch.zeros(E + 2, device=dev))
    counts = torch.full((E,), M // E, dtype=torch.int32, device=dev)
    with pytest.raises(TypeError):
        ops.gate_up_swiglu(x, wgu.float(), counts, M, a_idx=torch.zeros(M, dtype=torch.int32, device=dev))
    act = torch.zeros(M, h, **bf)
    with pytest.raises(TypeError):
        ops.down_scatter(act, wd.float(), counts, M, None, None)
    with pytest.raises(TypeError):
        ops.down_dgrad_swiglu(x, wd.float(), counts, M, torch.zeros(M, 2 * h, **bf),
                              a_idx=torch.zeros(M, dtype=torch.int32, device=dev))
    with pytest.raises(TypeError):
        ops.gate_up_dgrad(torch.zeros(M, 2 * h, **bf), wgu.float(), counts, M)
    with pytest.raises(ValueError):
        ops.gate_up_swiglu(x, wgu, counts[:E - 1], M, a_idx=torch.zeros(M, dtype=torch.int32, device=dev))
    a = torch.zeros(M, d, **bf)
    with pytest.raises(ValueError):
        ops.grouped_mm(a, wgu, counts, M, scale=torch.ones(M - 1, device=dev))
    with pytest.raises(ValueError):
        ops.grouped_mm(a, wgu, counts, M, out=torch.zeros(M - 1, 2 * h, **bf))
    with pytest.raises(TypeError):
        ops.grouped_mm(a, wgu.float(), counts, M)
    with pytest.raises(TypeError):
        ops.grouped_mm(a.half(), wgu, counts, M)
    with pytest.raises(TypeError):
        ops.grouped_mm(a.float(), wgu.float(), counts, M)
    with pytest.raises(ValueError):
        ops.dispatch(torch.zeros(T, k, dtype=torch.int32, device=dev), E, x=x[:T - 1])
