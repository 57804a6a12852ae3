"""Layer parity on the GPU: the MoE-SwiGLU forward (Triton-path rounding points) and its full backward against the
float64 oracle, and the fuse_moe / moe_infer drop-in against the same oracle."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from tests.util import assert_close_bf16, bits, boundary_tokens, f32, make_inputs

pytestmark = pytest.mark.gpu


def _run_layer(x, wr, wgu, wd, k, dout=None, bias=None):
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    dev = torch.device("cuda")
    req = dout is not None
    xg, wrg, wgug, wdg = (t.to(dev).requires_grad_(req) for t in (x, wr, wgu, wd))
    b = None if bias is None else torch.as_tensor(bias).float().to(dev)
    out, ids, tw = moe_swiglu(xg, wrg, wgug, wdg, k, logit_bias=b)
    if req:
        out.backward(dout.to(dev))
    torch.cuda.synchronize()
    return out, ids, tw, (xg, wrg, wgug, wdg)


@pytest.mark.parametrize("T,d,E,k,h", [(512, 256, 8, 2, 512), (2048, 1024, 8, 2, 2048), (300, 520, 5, 3, 264)])
def test_layer_forward(oracle, T, d, E, k, h):
    print(f"layer fwd T={T} d={d} E={E} k={k} h={h}", flush=True)
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=T)
    out, ids, tw, _ = _run_layer(x, wr, wgu, wd, k)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    ref = oracle.moe_forward(f32(x), rids, rw, f32(wgu), f32(wd))
    assert_close_bf16(f32(out), ref["out"], "out")


@pytest.mark.parametrize("T", [0, 1])
def test_layer_empty_and_single_token(oracle, T):
    """No tokens: forward and backward run and return empty / zero gradients. One token: forward and backward match
    the oracle (every expert but k empty)."""
    print(f"layer T={T}", flush=True)
    d, E, k, h = 256, 8, 2, 512
    x, wr, wgu, wd = make_inputs(max(T, 1), d, E, h, seed=7)
    x = x[:T]
    dout = torch.randn(T, d, generator=torch.Generator().manual_seed(8)).bfloat16()
    out, ids, tw, (xg, wrg, wgug, wdg) = _run_layer(x, wr, wgu, wd, k, dout=dout)
    assert out.shape == (T, d) and ids.shape == (T, k) and tw.shape == (T, k)
    if T == 0:
        for g in (wrg.grad, wgug.grad, wdg.grad):
            assert g is not None and not g.float().abs().any()
        assert xg.grad.shape == (0, d)
        return
    logits, rids, rw = oracle.route(bits(x), bits(wr), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    fwd = oracle.moe_forward(f32(x), rids, rw, f32(wgu), f32(wd))
    assert_close_bf16(f32(out), fwd["out"], "out")
    ref = oracle.layer_backward(f32(x), f32(wr), rids, rw, logits, f32(wgu), f32(wd), f32(dout), fwd=fwd)
    R = oracle.round_bf16
    for got, name in ((xg.grad, "dx"), (wgug.grad, "dwgu"), (wdg.grad, "dwd"), (wrg.grad, "dwr")):
        assert_close_bf16(f32(got), R(ref[name]), name)


def test_layer_forward_c3_sampled(oracle):
    """C3 shape (16384 tokens, d=1536, E=16, top-2, h=4096): routing bit-exact for every token, output checked on a
    sample of tokens (each row of the layer depends only on its own token): 192 at random, plus those owning rows at
    the grouped GEMMs' tile edges (each expert's last, partial m-tile and the final round's highest tile ids,
    tests.util.boundary_tokens)."""
    T, d, E, k, h = 16384, 1536, 16, 2, 4096
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=0)
    out, ids, tw, _ = _run_layer(x, wr, wgu, wd, k)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(tw.detach().cpu().numpy().view(np.uint32), rw.view(np.uint32))
    tok = np.union1d(np.random.default_rng(0).choice(T, 192, replace=False), boundary_tokens(rids, E))
    print(f"C3 sampled tokens: {tok.size}", flush=True)
    ref = oracle.moe_forward(f32(x), rids, rw, f32(wgu), f32(wd), tokens=tok)
    assert_close_bf16(f32(out)[tok], ref["out"], "out C3 sampled")


def test_layer_backward_c5_expert_slice(oracle):
    """C5 (the C3 shape, forward + backward) at full size.  The weight gradients of an expert depend only on the
    rows routed to it, and a token's input gradient only on its own slots, so the float64 oracle runs on the tokens
    that use expert e* (with their other slots): dWd[e*], dWgu[e*] and dx of those tokens from the full-size GPU
    backward are checked against it; routing is bit-exact for every token.  The output and dx are also checked on the
    tokens owning rows at the grouped GEMMs' tile edges (each expert's last, partial m-tile and the final round's
    highest tile ids, tests.util.boundary_tokens), which the forward GEMMs and the gate/up dgrad cover with partial
    tiles and half-row units."""
    T, d, E, k, h = 16384, 1536, 16, 2, 4096
    e_star = 5
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=3)
    g = torch.Generator().manual_seed(4)
    dout = torch.randn(T, d, generator=g).bfloat16()
    out, ids, tw, (xg, wrg, wgug, wdg) = _run_layer(x, wr, wgu, wd, k, dout=dout)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    toks = np.nonzero((rids == e_star).any(axis=1))[0]
    print(f"C5 backward slice: expert {e_star}, {toks.size} tokens", flush=True)
    xw, dw = f32(wgu), f32(wd)
    fwd = oracle.moe_forward(f32(x)[toks], rids[toks], rw[toks], xw, dw)
    ref = oracle.layer_backward(f32(x)[toks], f32(wr), rids[toks], rw[toks], logits[toks], xw, dw, f32(dout)[toks],
                                fwd=fwd)
    R = oracle.round_bf16
    assert_close_bf16(f32(out)[toks], fwd["out"], "out (tokens of e*)")
    assert_close_bf16(f32(xg.grad)[toks], R(ref["dx"]), "dx (tokens of e*)")
    assert_close_bf16(f32(wdg.grad)[e_star], R(ref["dwd"][e_star]), "dWd[e*]")
    assert_close_bf16(f32(wgug.grad)[e_star], R(ref["dwgu"][e_star]), "dWgu[e*]")
    tb = boundary_tokens(rids, E)
    print(f"C5 boundary tokens: {tb.size}", flush=True)
    fwd = oracle.moe_forward(f32(x)[tb], rids[tb], rw[tb], xw, dw)
    ref = oracle.layer_backward(f32(x)[tb], f32(wr), rids[tb], rw[tb], logits[tb], xw, dw, f32(dout)[tb], fwd=fwd)
    assert_close_bf16(f32(out)[tb], fwd["out"], "out (boundary tokens)")
    assert_close_bf16(f32(xg.grad)[tb], R(ref["dx"]), "dx (boundary tokens)")


@pytest.mark.parametrize("tile", ["auto", "L", "S"])
@pytest.mark.parametrize("T,d,E,k,h,zipf", [(512, 256, 8, 2, 512, 0), (1024, 512, 16, 2, 1024, 1),
                                            (300, 520, 5, 3, 264, 0)])
def test_layer_backward(oracle, monkeypatch, tile, T, d, E, k, h, zipf):
    """Forward and backward against the float64 oracle, with the GEMM tile size chosen by the library or forced to
    256x256 / 128x128 (the partial m-tiles, N tails and row masks of every epilogue on both tile sizes)."""
    if tile != "auto":
        monkeypatch.setenv("HMOE_GEMM_TILE", tile)
    print(f"layer bwd T={T} d={d} E={E} k={k} h={h} zipf={zipf} tile={tile}", flush=True)
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=T + 1)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(T, d, generator=g).bfloat16()
    bias = oracle.zipf_bias(E, seed=1) if zipf else None
    out, ids, tw, (xg, wrg, wgug, wdg) = _run_layer(x, wr, wgu, wd, k, dout=dout, bias=bias)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k, bias=bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    fwd = oracle.moe_forward(f32(x), rids, rw, f32(wgu), f32(wd))
    assert_close_bf16(f32(out), fwd["out"], "out")
    ref = oracle.layer_backward(f32(x), f32(wr), rids, rw, logits, f32(wgu), f32(wd), f32(dout), fwd=fwd)
    R = oracle.round_bf16
    assert_close_bf16(f32(xg.grad), R(ref["dx"]), "dx")
    assert_close_bf16(f32(wgug.grad), R(ref["dwgu"]), "dwgu")
    assert_close_bf16(f32(wdg.grad), R(ref["dwd"]), "dwd")
    assert_close_bf16(f32(wrg.grad), R(ref["dwr"]), "dwr")


class _Expert(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.gate_proj = nn.Linear(d, h, bias=False)
        self.up_proj = nn.Linear(d, h, bias=False)
        self.down_proj = nn.Linear(h, d, bias=False)
        self.act_fn = nn.functional.silu


class _MoEBlock(nn.Module):
    """Stand-in with the BailingMoeV2 MoE module layout fuse_moe looks for (experts ModuleList + moe_infer)."""

    def __init__(self, d, h, E):
        super().__init__()
        self.experts = nn.ModuleList([_Expert(d, h) for _ in range(E)])

    def moe_infer(self, x, topk_ids, topk_weight):  # replaced by fuse_moe
        raise AssertionError("not fused")


def test_fuse_moe_infer(oracle):
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    T, d, h, E, k = 1000, 512, 320, 16, 4
    torch.manual_seed(0)
    model = nn.Sequential(_MoEBlock(d, h, E)).bfloat16()
    wgu_ref = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in model[0].experts])
    wd_ref = torch.stack([e.down_proj.weight.t() for e in model[0].experts])
    assert fuse_moe(model) == 1
    model = model.cuda()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, d, generator=g).bfloat16()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    y = model[0].moe_infer(x.cuda(), ids.cuda(), w.cuda())
    assert model[0]._mode == "hip"
    ref = oracle.moe_forward(f32(x), ids.numpy(), w.numpy(), f32(wgu_ref), f32(wd_ref))
    assert_close_bf16(f32(y), ref["out"], "moe_infer")


def test_fuse_moe_matches_expert_loop():
    """The claim of aurora/hf_compat.py:64-65: the fused path equals the per-expert loop it replaces up to bf16
    rounding and routing ties ("cos 0.9999 to the loop").  The loop here is the unfused moe_infer of DeepSeek-style
    blocks restated with torch on the CPU: each expert's bf16 Linear layers on its tokens, times the routing weight,
    summed over the k slots."""
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe
    T, d, h, E, k = 600, 256, 192, 8, 2
    torch.manual_seed(5)
    model = nn.Sequential(_MoEBlock(d, h, E)).bfloat16()
    experts = [(e.gate_proj.weight.detach().clone(), e.up_proj.weight.detach().clone(),
                e.down_proj.weight.detach().clone()) for e in model[0].experts]
    assert fuse_moe(model) == 1
    g = torch.Generator().manual_seed(6)
    x = torch.randn(T, d, generator=g).bfloat16()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    y = model.cuda()[0].moe_infer(x.cuda(), ids.cuda(), w.cuda()).float().cpu()
    ref = torch.zeros(T, d)
    for e, (wg, wu, wdn) in enumerate(experts):
        rows, slot = (ids == e).nonzero(as_tuple=True)
        if rows.numel() == 0:
            continue
        xe = x[rows]
        out = torch.nn.functional.linear(torch.nn.functional.silu(torch.nn.functional.linear(xe, wg)) *
                                         torch.nn.functional.linear(xe, wu), wdn)
        ref.index_add_(0, rows, out.float() * w[rows, slot, None])
    cos = torch.nn.functional.cosine_similarity(y.flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.9999, cos


def test_layer_c4_full_size(oracle):
    """C4 at full size: 16384 tokens, d=1536, E=16, top-2, h=4096, Zipf(1.2) expert bias with 2 experts never
    routed (aurora/hf_compat.py:69-82 over skewed groups: one expert gets ~14k of the 32768 rows, the smallest
    non-empty one a few).
      - routing ids and weights bit-exact for every token; counts bit-exact against torch.bincount (2 zeros);
      - output on sampled tokens (all tokens of the smallest non-empty expert, a sample of the largest, random ones,
        and those owning rows at the tile edges: each expert's last m-tile, the final round's rows);
      - backward: weight gradients of the largest expert on a subset J of its hidden units (a weight gradient
        column j of w_gu / row j of w_d depends only on hidden unit j, so the float64 oracle runs the layer
        restricted to J with the same routing and upstream gradient), the full weight gradients of the smallest
        non-empty expert, dx of its tokens, of a sample of the largest expert's tokens and of the tile-edge tokens, and
        exact zeros for the
        two empty experts."""
    from trenowanie_generatora_obrazkow_amd import ops
    T, d, E, k, h = 16384, 1536, 16, 2, 4096
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=0)
    bias = oracle.zipf_bias(E, seed=0)
    dout = torch.randn(T, d, generator=torch.Generator().manual_seed(1)).bfloat16()
    out, ids, tw, (xg, wrg, wgug, wdg) = _run_layer(x, wr, wgu, wd, k, dout=dout, bias=bias)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k, bias=bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(tw.detach().cpu().numpy().view(np.uint32), rw.view(np.uint32))
    counts = ops.dispatch(ids, E).counts.cpu()
    ref_counts = torch.bincount(torch.from_numpy(rids).reshape(-1).long(), minlength=E)
    assert torch.equal(counts.long(), ref_counts)
    empty = np.nonzero(ref_counts.numpy() == 0)[0]
    assert empty.size == 2
    live = np.nonzero(ref_counts.numpy() > 0)[0]
    e_max = int(live[np.argmax(ref_counts.numpy()[live])])
    e_min = int(live[np.argmin(ref_counts.numpy()[live])])
    print(f"C4 counts {ref_counts.tolist()}, largest expert {e_max}, smallest {e_min}", flush=True)
    assert ref_counts[e_max] > 10000
    rng = np.random.default_rng(2)
    toks_max = np.nonzero((rids == e_max).any(axis=1))[0]
    toks_min = np.nonzero((rids == e_min).any(axis=1))[0]
    tb = boundary_tokens(rids, E)
    sample = np.unique(np.concatenate([toks_min, rng.choice(toks_max, 64, replace=False),
                                       rng.choice(T, 128, replace=False), tb]))
    xf, wguf, wdf, doutf = f32(x), f32(wgu), f32(wd), f32(dout)
    fwd = oracle.moe_forward(xf, rids, rw, wguf, wdf, tokens=sample)
    assert_close_bf16(f32(out)[sample], fwd["out"], "C4 out sampled")
    R = oracle.round_bf16
    gwgu, gwd, gdx = f32(wgug.grad), f32(wdg.grad), f32(xg.grad)
    for e in empty:
        assert not gwgu[e].any() and not gwd[e].any(), f"empty expert {e} has a weight gradient"
    # smallest non-empty expert: its full weight gradients and its tokens' dx
    ref = oracle.layer_backward(xf[toks_min], f32(wr), rids[toks_min], rw[toks_min], logits[toks_min], wguf, wdf,
                                doutf[toks_min])
    assert_close_bf16(gwd[e_min], R(ref["dwd"][e_min]), f"dWd[{e_min}]")
    assert_close_bf16(gwgu[e_min], R(ref["dwgu"][e_min]), f"dWgu[{e_min}]")
    assert_close_bf16(gdx[toks_min], R(ref["dx"]), "dx (tokens of the smallest expert)")
    # dx of a sample of the largest expert's tokens
    tsel = rng.choice(toks_max, 48, replace=False)
    ref = oracle.layer_backward(xf[tsel], f32(wr), rids[tsel], rw[tsel], logits[tsel], wguf, wdf, doutf[tsel])
    assert_close_bf16(gdx[tsel], R(ref["dx"]), "dx (sample of the largest expert's tokens)")
    # dx of the tokens at the tile edges (each expert's last m-tile, the final round's rows)
    ref = oracle.layer_backward(xf[tb], f32(wr), rids[tb], rw[tb], logits[tb], wguf, wdf, doutf[tb])
    assert_close_bf16(gdx[tb], R(ref["dx"]), "dx (boundary tokens)")
    # largest expert, hidden units J: the layer restricted to J has the same weight gradients there
    J = np.sort(rng.choice(h, 128, replace=False))
    cols = np.concatenate([J, h + J])
    rb = oracle.moe_backward(xf[toks_max], rids[toks_max], rw[toks_max], wguf[:, :, cols], wdf[:, J, :],
                             doutf[toks_max])
    assert_close_bf16(gwd[e_max][J], R(rb["dwd"][e_max]), f"dWd[{e_max}] rows J")
    assert_close_bf16(gwgu[e_max][:, cols], R(rb["dwgu"][e_max]), f"dWgu[{e_max}] columns J")


def test_moe_swiglu_module(oracle):
    """MoESwiGLU as the reference calls its FFN, self.mlp(h) on (B, T, dim) (aurora/model.py:210), after the
    reference's own init code (init_block, aurora/model.py:393-396, restated): forward and backward against the
    float64 oracle; a loss on the returned routing weights reaches x and the router (softmax + renormalisation
    Jacobian); fp32 input gives fp32 output with the same values, autocast(bf16) gives bf16; fp32 master weights
    give the bf16 model's output bit for bit and fp32 gradients whose bf16 rounding is the bf16 model's."""
    from trenowanie_generatora_obrazkow_amd import MoESwiGLU
    B, T, dim, hidden, E, k = 2, 160, 256, 384, 8, 2
    torch.manual_seed(3)
    m = MoESwiGLU(dim, hidden, E, top_k=k).cuda()
    with torch.no_grad():
        for lin in (m.in_proj, m.out_proj):
            nn.init.normal_(lin.weight, std=lin.in_features ** -0.5)
    g = torch.Generator().manual_seed(4)
    h = torch.randn(B, T, dim, generator=g).bfloat16()
    dout = torch.randn(B, T, dim, generator=g).bfloat16()
    c = torch.randn(B * T, k, generator=g)  # weight of the routing-weight term of the loss
    hg = h.cuda().requires_grad_(True)
    out = m(hg)
    assert out.shape == (B, T, dim) and out.dtype == torch.bfloat16
    loss = (out.float() * dout.cuda().float()).sum() + (m.last_topk_weight * c.cuda()).sum()
    loss.backward()
    torch.cuda.synchronize()
    x2 = h.reshape(-1, dim)
    wr, wgu, wd = (f32(p) for p in (m.router_weight, m.w_gu, m.w_d))
    logits, rids, rw = oracle.route(bits(x2), bits(m.router_weight), k)
    np.testing.assert_array_equal(m.last_topk_ids.cpu().numpy(), rids)
    fwd = oracle.moe_forward(f32(x2), rids, rw, wgu, wd)
    assert_close_bf16(f32(out).reshape(-1, dim), fwd["out"], "module out")
    b = oracle.moe_backward(f32(x2), rids, rw, wgu, wd, f32(dout).reshape(-1, dim), fwd=fwd)
    dl = oracle.router_backward(logits, rids, b["dtopk_w"] + c.numpy().astype(np.float64))
    R = oracle.round_bf16
    assert_close_bf16(f32(hg.grad).reshape(-1, dim), R(b["dx_experts"] + dl @ wr.astype(np.float64)), "dx")
    assert_close_bf16(f32(m.router_weight.grad), R(dl.T @ f32(x2).astype(np.float64)), "dWr")
    assert_close_bf16(f32(m.w_gu.grad), R(b["dwgu"]), "dWgu")
    assert_close_bf16(f32(m.w_d.grad), R(b["dwd"]), "dWd")

    # a loss on the routing weights alone
    m.zero_grad(set_to_none=True)
    hg2 = h.cuda().requires_grad_(True)
    m(hg2)
    (m.last_topk_weight * c.cuda()).sum().backward()
    dl0 = oracle.router_backward(logits, rids, c.numpy().astype(np.float64))
    assert_close_bf16(f32(hg2.grad).reshape(-1, dim), R(dl0 @ wr.astype(np.float64)), "dx (routing-weight loss)")
    assert not f32(m.w_gu.grad).any() and not f32(m.w_d.grad).any()

    # dtypes: fp32 input -> fp32 output of the same values; autocast -> the autocast dtype
    with torch.no_grad():
        o32 = m(h.float().cuda())
        assert o32.dtype == torch.float32 and torch.equal(o32, out.float())
        with torch.autocast("cuda", dtype=torch.bfloat16):
            assert m(h.float().cuda()).dtype == torch.bfloat16

    # fp32 master weights: same forward, fp32 gradients
    m32 = MoESwiGLU(dim, hidden, E, top_k=k, dtype=torch.float32).cuda()
    with torch.no_grad():
        for p32, p16 in ((m32.router_weight, m.router_weight), (m32.w_gu, m.w_gu), (m32.w_d, m.w_d)):
            p32.copy_(p16.float())
    m.zero_grad(set_to_none=True)
    for mod in (m, m32):
        o = mod(h.cuda())
        (o.float() * dout.cuda().float()).sum().backward()
        if mod is m:
            o16 = o
    torch.cuda.synchronize()
    assert torch.equal(o, o16)
    for p32, p16 in ((m32.router_weight, m.router_weight), (m32.w_gu, m.w_gu), (m32.w_d, m.w_d)):
        assert p32.grad.dtype == torch.float32 and torch.equal(p32.grad.bfloat16(), p16.grad)
