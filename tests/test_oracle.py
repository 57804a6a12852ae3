"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path: every function is checked
against something independent of its own formula -- the mathematics (closed forms, brute force, invariants), torch's
own routines (softmax/topk, argsort/bincount, _grouped_mm, autograd), hand-derived known answers, and the golden
fixtures in tests/golden/.  CPU only."""
from itertools import combinations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.util import make_inputs


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------------------------------------- bf16 / hexp
def test_round_bf16_matches_torch(oracle):
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(20000, generator=g) * 10 ** torch.randint(-30, 30, (20000,), generator=g).float(),
                   torch.tensor([0.0, -0.0, 1.0, float("inf"), -float("inf"), 3.4e38, 1e-40, -1e-39])])
    ours = oracle.f32_to_bf16_bits(x.numpy())
    np.testing.assert_array_equal(ours, bits(x.bfloat16()))
    assert oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_round_bf16_from_float64_is_nearest(oracle):
    rng = np.random.default_rng(1)
    v = rng.standard_normal(5000) * 10.0 ** rng.integers(-20, 20, 5000)
    r = oracle.round_bf16(v).astype(np.float64)
    # the nearest bf16: no other bf16 neighbour is closer (ties to even are allowed to sit at distance equality)
    rb = torch.from_numpy(r.astype(np.float32)).bfloat16()
    up = torch.nextafter(rb, torch.full_like(rb, float("inf"))).float().double().numpy()
    dn = torch.nextafter(rb, torch.full_like(rb, -float("inf"))).float().double().numpy()
    assert (np.abs(r - v) <= np.abs(up - v)).all() and (np.abs(r - v) <= np.abs(dn - v)).all()


def test_hexp_accuracy_and_special_cases(oracle):
    xs = np.linspace(-87.0, 0.0, 40001).astype(np.float32)
    ys = oracle.hexp(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.abs(ys - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 1.0, ulp.max()
    assert oracle.hexp(np.array([0.0], np.float32))[0] == 1.0
    assert oracle.hexp(np.array([-np.inf, -88.0, -1000.0], np.float32)).tolist() == [0.0, 0.0, 0.0]


# ------------------------------------------------------------------------------------------------- router
def test_router_logits_vs_float64(oracle):
    x, wr, _, _ = make_inputs(300, 1536, 16, 8, seed=2)
    lg = oracle.router_logits(bits(x), bits(wr))
    ref = x.double().numpy() @ wr.double().numpy().T
    # fp32 accumulation of exact products: |err| <= d * eps * sum|x w|
    bound = 1536 * 2 ** -24 * (np.abs(x.double().numpy()) @ np.abs(wr.double().numpy()).T)
    assert (np.abs(lg - ref) <= bound).all()
    # a dropped / misindexed term would be far outside the bound
    assert np.abs(lg - ref).max() < 1e-4


def test_router_bias_and_stride(oracle):
    x, wr, _, _ = make_inputs(64, 520, 5, 8, seed=3)
    bias = np.array([0.5, -1.0, 0.0, 2.0, -np.inf], np.float32)
    lg = oracle.router_logits(bits(x), bits(wr), bias)
    lg0 = oracle.router_logits(bits(x), bits(wr))
    np.testing.assert_array_equal(lg, (lg0 + bias).astype(np.float32))


def test_topk_vs_torch(oracle):
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(4000, 16, generator=g) * 0.8
    for k, renorm, scaling in [(2, True, 1.0), (4, False, 1.0), (3, True, 2.5)]:
        ids, w = oracle.topk_from_logits(logits.numpy(), k, renorm, scaling)
        p = logits.double().softmax(-1)
        tw, ti = p.topk(k, dim=-1)
        np.testing.assert_array_equal(ids, ti.numpy())
        if renorm:
            tw = tw / (tw.sum(-1, keepdim=True) + 1e-20)
        np.testing.assert_allclose(w, (tw * scaling).numpy(), rtol=2e-6, atol=1e-8)


def test_topk_brute_force_tiny(oracle):
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal((200, 6)) * 2).astype(np.float32)
    ids, w = oracle.topk_from_logits(logits, 3, True)
    for t in range(200):
        # the selected set maximises the sum of logits over all 3-subsets; slots are in descending order
        best = max(combinations(range(6), 3), key=lambda s: sum(float(logits[t, e]) for e in s))
        assert set(ids[t].tolist()) == set(best)
        assert list(logits[t, ids[t]]) == sorted(logits[t, ids[t]], reverse=True)
        assert abs(float(w[t].sum()) - 1.0) < 1e-6


def test_topk_ties_and_masked_experts(oracle):
    ids, w = oracle.topk_from_logits(np.zeros((3, 8), np.float32), 3, True)
    assert (ids == np.array([0, 1, 2])).all()
    np.testing.assert_allclose(w, 1.0 / 3, rtol=1e-6)
    lg = np.array([[0.0, -np.inf, 5.0, -np.inf, 1.0]], np.float32)
    ids, w = oracle.topk_from_logits(lg, 3, False)
    assert ids.tolist() == [[2, 4, 0]]
    e = np.exp(np.array([5.0, 1.0, 0.0]) - 5.0)
    np.testing.assert_allclose(w[0], e / e.sum(), rtol=1e-6)


def test_zipf_bias_shape(oracle):
    b = oracle.zipf_bias(16, seed=0)
    assert np.isinf(b).sum() == 2 and (b[np.isfinite(b)] <= 0).all()
    np.testing.assert_allclose(np.sort(-b[np.isfinite(b)] / 1.2), np.log(np.arange(1, 15)), rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------------------------------------- dispatch / schedule
@pytest.mark.parametrize("T,k,E", [(1, 2, 4), (100, 3, 7), (5000, 2, 16), (333, 8, 128)])
def test_dispatch_three_ways(oracle, T, k, E):
    g = torch.Generator().manual_seed(T)
    ids = torch.randint(0, E, (T, k), generator=g)
    a = oracle.dispatch(ids.numpy(), E)
    c = oracle.dispatch_c(ids.numpy(), E)
    flat = ids.reshape(-1)
    order = flat.argsort(stable=True)  # aurora/hf_compat.py:71
    counts = torch.bincount(flat, minlength=E)  # :72
    for r in (a, c):
        np.testing.assert_array_equal(r["order"], order.numpy())
        np.testing.assert_array_equal(r["counts"], counts.numpy())
        np.testing.assert_array_equal(r["a_idx"], (order // k).numpy())
        np.testing.assert_array_equal(r["order"][r["inv_pos"]], np.arange(T * k))
    # invariants: a permutation, experts non-decreasing along order, flat index increasing within an expert
    e_sorted = ids.numpy().reshape(-1)[a["order"]]
    assert (np.diff(e_sorted) >= 0).all()
    same = np.diff(e_sorted) == 0
    assert (np.diff(a["order"])[same] > 0).all()


def test_dispatch_rejects_out_of_range(oracle):
    with pytest.raises(ValueError):
        oracle.dispatch_c(np.array([[0, 5]]), 4)


def test_make_schedule_known_answer(oracle):
    # counts [16, 0, 32] (the reference self-test), BLOCK_M 64, M 48: blocks (0, rows 0..16), (2, rows 16..48),
    # then two invalid tail blocks carrying the clamped values of the last expert
    be, br, re_ = oracle.make_schedule(np.array([16, 0, 32]), 48)
    assert be.tolist() == [0, 2, -1, -1]
    assert br.tolist() == [0, 16, 80, 144]
    assert re_.tolist() == [16, 48, 48, 48]


@pytest.mark.parametrize("counts", [[16, 0, 32], [0, 0, 5], [64, 64, 1, 0, 200], [0] * 7 + [1000], [3000] * 16,
                                    [0, 0, 0]])
def test_make_schedule_c_and_coverage(oracle, counts):
    c = np.array(counts, np.int64)
    M = int(c.sum())
    ref = oracle.make_schedule(c, M)
    for a, b in zip(ref, oracle.make_schedule_c(c, M)):
        np.testing.assert_array_equal(a, b)
    be, br, re_ = ref
    covered = np.zeros(M, np.int64)
    starts = np.cumsum(c) - c
    for e, r0, r1 in zip(be, br, re_):
        if e < 0:
            continue
        assert starts[e] <= r0 < r1 == starts[e] + c[e]
        covered[r0:min(r0 + 64, r1)] += 1
    assert (covered == 1).all()
    assert len(be) == -(-M // 64) + len(c)


# ------------------------------------------------------------------------------------------------- grouped GEMM
def test_grouped_mm_selftest_construction(oracle):
    """The reference's known-answer construction (aurora/hf_compat.py:115-121) against per-expert torch matmuls
    and torch._grouped_mm, and the bf16 rounding bracket."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn(48, 64, generator=g).bfloat16()
    w = torch.randn(3, 64, 32, generator=g).bfloat16()
    counts = np.array([16, 0, 32])
    y = oracle.grouped_mm(a.float().numpy(), w.float().numpy(), counts, round_out=False)
    ref = torch.cat([a[:16].double() @ w[0].double(), a[16:].double() @ w[2].double()])
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-12)
    gm = torch._grouped_mm(a.float(), w.float(), offs=torch.tensor([16, 16, 48], dtype=torch.int32))
    np.testing.assert_allclose(y, gm.double().numpy(), rtol=1e-5, atol=1e-4)
    yb = torch.from_numpy(oracle.grouped_mm(a.float().numpy(), w.float().numpy(), counts)).bfloat16()
    r = torch.from_numpy(y).float().bfloat16()
    lo = torch.nextafter(r, torch.full_like(r, -float("inf")))
    hi = torch.nextafter(r, torch.full_like(r, float("inf")))
    assert ((yb >= lo) & (yb <= hi)).all()


def test_grouped_mm_fused_indices(oracle):
    """gather / scale / scatter as in aurora/moe_triton.py:38-56, against an explicit per-row loop."""
    rng = np.random.default_rng(6)
    T, k, E, K, N = 20, 2, 3, 16, 8
    ids = rng.integers(0, E, (T, k))
    d = oracle.dispatch(ids, E)
    x = rng.standard_normal((T, K)).astype(np.float32)
    w = rng.standard_normal((E, K, N)).astype(np.float32)
    sc = rng.random(T * k).astype(np.float32)
    y = oracle.grouped_mm(x, w, d["counts"], a_idx=d["a_idx"], y_idx=d["y_idx"], scale=sc, round_out=False)
    e_sorted = ids.reshape(-1)[d["order"]]
    for r in range(T * k):
        expect = (x[d["a_idx"][r]].astype(np.float64) @ w[e_sorted[r]]) * sc[r]
        np.testing.assert_allclose(y[d["y_idx"][r]], expect, rtol=1e-12)


def test_quant_int8_closed_form(oracle):
    rng = np.random.default_rng(7)
    w = rng.standard_normal((3, 64, 16)).astype(np.float32)
    q, s = oracle.quant_int8(w)
    assert q.dtype == np.int8 and np.abs(q.astype(np.int32)).max() <= 127
    s_exact = np.abs(w).max(axis=1) / 127
    assert (np.abs(q * s_exact[:, None, :] - w) <= s_exact[:, None, :] / 2 + 1e-7).all()
    assert (np.abs(q).max(axis=1) == 127).all()


def test_grouped_mm_int8_scale_is_dequantised_product(oracle):
    """(a @ q) * s[e, n] equals a @ (q * s) column by column (exact in float64 up to rounding); permuting the columns
    of (q, s) together permutes y's columns -- a transposed or mis-indexed scale fails both."""
    rng = np.random.default_rng(11)
    T, K, N, E, k = 40, 48, 32, 3, 2
    x = oracle.round_bf16(rng.standard_normal((T, K)))
    w = rng.standard_normal((E, K, N)).astype(np.float32) * np.linspace(0.1, 3.0, N, dtype=np.float32)
    q, s = oracle.quant_int8(w)
    ids = rng.integers(0, E, (T, k))
    d = oracle.dispatch(ids, E)
    sc = rng.random(T * k).astype(np.float32)
    kw = dict(a_idx=d["a_idx"], y_idx=d["y_idx"], scale=sc, round_out=False)
    y = oracle.grouped_mm(x, q, d["counts"], w_scale=s, **kw)
    deq = q.astype(np.float64) * s.astype(np.float64)[:, None, :]
    np.testing.assert_allclose(y, oracle.grouped_mm(x, deq, d["counts"], **kw), rtol=1e-12, atol=1e-12)
    perm = rng.permutation(N)
    yp = oracle.grouped_mm(x, q[:, :, perm], d["counts"], w_scale=s[:, perm], **kw)
    np.testing.assert_array_equal(yp, y[:, perm])
    # the dequantised weights stay within half a step (q rounding) plus 127 x the bf16 rounding of the scale
    assert (np.abs(deq - w) <= s.astype(np.float64)[:, None, :] * (0.5 + 127 * 2.0 ** -8) * 1.01).all()


# ------------------------------------------------------------------------------------------------- layer forward
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_moe_forward_vs_token_loop(oracle, dtype):
    """The per-expert batched oracle against a per-token loop with the same rounding points (tiny shapes), for bf16
    activations and for fp16 ones (a model loaded in fp16: every rounding point rounds to fp16 instead)."""
    rng = np.random.default_rng(8)
    T, d, E, k, h = 8, 16, 4, 2, 8
    R = oracle.round_bf16 if dtype == "bf16" else oracle.round_f16
    x = R(rng.standard_normal((T, d)))
    wgu = R(rng.standard_normal((E, d, 2 * h)) * 0.3)
    wd = R(rng.standard_normal((E, h, d)) * 0.3)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    tw = rng.random((T, k)).astype(np.float32)
    f = oracle.moe_forward(x, ids, tw, wgu, wd, dtype=dtype)
    for t in range(T):
        acc = np.zeros(d)
        for j in range(k):
            e = ids[t, j]
            gu = [sum(float(x[t, i]) * float(wgu[e, i, c]) for i in range(d)) for c in range(2 * h)]
            g = R(np.array(gu[:h])).astype(np.float64)
            u = R(np.array(gu[h:])).astype(np.float64)
            s = R(g / (1 + np.exp(-g))).astype(np.float64)
            a = R(s * u).astype(np.float64)
            yh = [sum(a[i] * float(wd[e, i, c]) for i in range(h)) for c in range(d)]
            wb = float(R(np.array([tw[t, j]]))[0])
            acc += R(np.array(yh) * wb).astype(np.float64)
        np.testing.assert_array_equal(f["out"][t], R(acc))


def test_round_f16_brute_force(oracle):
    """round_f16 against a brute-force search over every finite fp16 value: the nearest, ties to the even bit
    pattern, overflow to inf -- on random float64 values, exact midpoints between neighbours, and edges."""
    allh = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # +0 .. 65504
    rng = np.random.default_rng(5)
    mids = (allh[1:] + allh[:-1]) / 2  # exact midpoints (float64 holds them)
    pick = rng.choice(mids.size, 3000, replace=False)
    vals = np.concatenate([rng.standard_normal(3000) * 30.0, rng.standard_normal(1000) * 1e-5, mids[pick],
                           [0.0, 65504.0, 65519.99, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26]])
    vals = np.concatenate([vals, -vals])
    got = oracle.round_f16(vals).astype(np.float64)
    for v, g in zip(vals, got):
        a = abs(v)
        if a >= 65520.0:  # beyond the largest finite value plus half an ulp: inf
            assert np.isinf(g) and np.sign(g) == np.sign(v)
            continue
        i = np.searchsorted(allh, a)
        cand = [j for j in (i - 1, i) if 0 <= j < allh.size]
        dist = [abs(allh[j] - a) for j in cand]
        best = min(dist)
        ties = [j for j, dd in zip(cand, dist) if dd == best]
        j = ties[0] if len(ties) == 1 else [t for t in ties if t % 2 == 0][0]
        assert abs(g) == allh[j] and (g == 0 or np.sign(g) == np.sign(v)), (v, g, allh[j])


def test_moe_forward_int8_scales(oracle):
    """Scales applied to the sums (the int8 form) give what the dequantised float64 weights give at every rounding
    point; the scales of the gate and up halves are indexed by the wgu column (2h), those of down by d."""
    rng = np.random.default_rng(12)
    T, d, E, k, h = 24, 32, 4, 2, 16
    x = oracle.round_bf16(rng.standard_normal((T, d)))
    colw = np.linspace(0.2, 2.0, 2 * h, dtype=np.float32)
    qgu, sgu = oracle.quant_int8(rng.standard_normal((E, d, 2 * h)).astype(np.float32) * colw * 0.3)
    qd, sd = oracle.quant_int8(rng.standard_normal((E, h, d)).astype(np.float32) * 0.3)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    tw = rng.random((T, k)).astype(np.float32)
    f = oracle.moe_forward(x, ids, tw, qgu, qd, wgu_s=sgu, wd_s=sd)
    g = oracle.moe_forward(x, ids, tw, qgu * sgu.astype(np.float64)[:, None, :], qd * sd.astype(np.float64)[:, None, :])
    for key in ("gb", "ub", "act", "y", "out"):
        np.testing.assert_array_equal(f[key], g[key], err_msg=key)


def test_moe_forward_vs_reference_cpu_path(oracle):
    """Against the transcription of the reference's CPU path (torch._grouped_mm, oracle/cpu_path.py) in fp32."""
    from oracle import cpu_path
    x, wr, wgu, wd = make_inputs(256, 128, 8, 64, seed=9, dtype=torch.float32)
    x, wr, wgu, wd = (t.bfloat16().float() for t in (x, wr, wgu, wd))
    _, ids, w = cpu_path.router(x, wr, 2)
    y = cpu_path.fused_moe_grouped(x, ids, w, wgu, wd)
    f = oracle.moe_forward(x.numpy(), ids.numpy(), w.numpy(), wgu.numpy(), wd.numpy())
    diff = np.abs(f["out"] - y.numpy())
    assert diff.max() / np.abs(y.numpy()).max() < 2e-2 and diff.mean() / np.abs(y.numpy()).mean() < 5e-3


# ------------------------------------------------------------------------------------------------- backward
def _torch_layer(x, wr, wgu, wd, ids, k, wb_values, rnd64, renorm=True):
    """Float64 autograd of the layer with the forward's bf16 rounding points as straight-through roundings (one
    rounding float64 -> bf16, `rnd64`); the rounded routing weights take the given values (the fp32 router's,
    rounded to bf16) in the forward."""
    def rnd(t):
        return t + (torch.from_numpy(rnd64(t.detach().numpy()).astype(np.float64)) - t).detach()

    logits = x @ wr.T
    p = logits.softmax(-1)
    sel = p.gather(1, ids)
    w = sel / (sel.sum(-1, keepdim=True) + 1e-20) if renorm else sel
    wb = w + (wb_values - w).detach()
    T, d = x.shape
    h = wgu.shape[2] // 2
    out = torch.zeros(T, d, dtype=torch.float64)
    for j in range(k):
        for e in range(wgu.shape[0]):
            m = ids[:, j] == e
            if not m.any():
                continue
            gu = x[m] @ wgu[e]
            g, u = rnd(gu[:, :h]), rnd(gu[:, h:])
            a = rnd(rnd(F.silu(g)) * u)
            y = rnd((a @ wd[e]) * wb[m, j:j + 1])
            out = out.index_put((m.nonzero()[:, 0],), y, accumulate=True)
    return out


def test_backward_vs_autograd(oracle):
    rng = np.random.default_rng(10)
    T, d, E, k, h = 24, 16, 4, 2, 8
    R = oracle.round_bf16
    x, wr = R(rng.standard_normal((T, d))), R(rng.standard_normal((E, d)) * 0.3)
    wgu, wd = R(rng.standard_normal((E, d, 2 * h)) * 0.3), R(rng.standard_normal((E, h, d)) * 0.3)
    dout = R(rng.standard_normal((T, d)))
    logits = (x.astype(np.float64) @ wr.astype(np.float64).T).astype(np.float32)
    ids, w = oracle.topk_from_logits(logits, k, True)
    fwd = oracle.moe_forward(x, ids, w, wgu, wd)
    b = oracle.layer_backward(x, wr, ids, w, logits, wgu, wd, dout, fwd=fwd)
    tx, twr, twgu, twd = (torch.from_numpy(v.astype(np.float64)).requires_grad_(True) for v in (x, wr, wgu, wd))
    wbv = torch.from_numpy(R(w).astype(np.float64))
    out = _torch_layer(tx, twr, twgu, twd, torch.from_numpy(ids.astype(np.int64)), k, wbv, R)
    out.backward(torch.from_numpy(dout.astype(np.float64)))
    # expert-path gradients agree to rounding; the router path differs by the fp32 logits the oracle recomputes the
    # softmax from (as the router does) against float64 logits here: ~1e-7 relative
    for name, t in (("dx", tx), ("dwr", twr), ("dwgu", twgu), ("dwd", twd)):
        np.testing.assert_allclose(b[name], t.grad.numpy(), rtol=1e-5, atol=1e-6, err_msg=name)
    np.testing.assert_allclose(b["dwgu"], twgu.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(b["dwd"], twd.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_backward_finite_differences(oracle):
    """Without rounding (float64 all through), the closed-form gradients against central differences."""
    rng = np.random.default_rng(11)
    T, d, E, k, h = 6, 8, 3, 2, 4
    x, wr = rng.standard_normal((T, d)), rng.standard_normal((E, d)) * 0.5
    wgu, wd = rng.standard_normal((E, d, 2 * h)) * 0.5, rng.standard_normal((E, h, d)) * 0.5
    dout = rng.standard_normal((T, d))
    logits = x @ wr.T
    ids, _ = oracle.topk_from_logits(logits.astype(np.float32), k, True)

    def loss(x_, wr_, wgu_, wd_):
        lg = x_ @ wr_.T
        p = np.exp(lg - lg.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        sel = np.take_along_axis(p, ids.astype(np.int64), 1)
        w = sel / (sel.sum(1, keepdims=True) + 1e-20)
        out = np.zeros((T, d))
        for t in range(T):
            for j in range(k):
                e = ids[t, j]
                gu = x_[t] @ wgu_[e]
                a = gu[:h] / (1 + np.exp(-gu[:h])) * gu[h:]
                out[t] += (a @ wd_[e]) * w[t, j]
        return float((out * dout).sum())

    class NoRound:
        pass

    # oracle backward evaluated with identity rounding: feed float64 "stored" values directly
    rb = oracle.round_bf16
    try:
        oracle.round_bf16 = lambda a: np.asarray(a, np.float64)
        lg32 = logits
        _, w32 = oracle.topk_from_logits(lg32.astype(np.float32), k, True)
        p = np.exp(lg32 - lg32.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        sel = np.take_along_axis(p, ids.astype(np.int64), 1)
        wexact = sel / (sel.sum(1, keepdims=True) + 1e-20)
        fwd = oracle.moe_forward(x, ids, wexact, wgu, wd)
        b = oracle.layer_backward(x, wr, ids, wexact, logits, wgu, wd, dout, fwd=fwd)
    finally:
        oracle.round_bf16 = rb
    eps = 1e-6
    for name, arr, idx in (("dx", x, (2, 3)), ("dwr", wr, (1, 5)), ("dwgu", wgu, (0, 2, 5)), ("dwd", wd, (2, 1, 4))):
        args = [x.copy(), wr.copy(), wgu.copy(), wd.copy()]
        pos = {"dx": 0, "dwr": 1, "dwgu": 2, "dwd": 3}[name]
        args[pos][idx] += eps
        lp = loss(*args)
        args[pos][idx] -= 2 * eps
        lm = loss(*args)
        fd = (lp - lm) / (2 * eps)
        assert abs(b[name][idx] - fd) <= 1e-5 * max(1.0, abs(fd)), (name, b[name][idx], fd)


def test_router_backward_vs_autograd(oracle):
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(500, 16, generator=g, dtype=torch.float64)
    ids, _ = oracle.topk_from_logits(logits.float().numpy(), 2, True)
    dw = torch.randn(500, 2, generator=g, dtype=torch.float64)
    for renorm, scaling in ((True, 1.0), (False, 1.0), (True, 2.5)):
        lg = logits.clone().requires_grad_(True)
        sel = lg.softmax(-1).gather(1, torch.from_numpy(ids.astype(np.int64)))
        w = (sel / (sel.sum(-1, keepdim=True) + 1e-20) if renorm else sel) * scaling
        w.backward(dw)
        ref = oracle.router_backward(logits.numpy(), ids, dw.numpy(), renorm, scaling)
        np.testing.assert_allclose(ref, lg.grad.numpy(), rtol=1e-10, atol=1e-12)


# ------------------------------------------------------------------------------------------------- golden fixtures
def test_golden_fixtures_reproduce(oracle):
    import os
    gd = os.path.join(os.path.dirname(__file__), "golden")
    r = np.load(os.path.join(gd, "router.npz"))
    for n in "abc":
        T, d, E, k, renorm = r[f"{n}_params"].tolist()
        bias = r[f"{n}_bias"] if r[f"{n}_bias"].size else None
        lg, ids, w = oracle.route(r[f"{n}_x"], r[f"{n}_wr"], k, bias=bias, renorm=bool(renorm),
                                  scaling=float(r[f"{n}_scaling"]))
        np.testing.assert_array_equal(lg.view(np.uint32), r[f"{n}_logits"].view(np.uint32))
        np.testing.assert_array_equal(ids, r[f"{n}_ids"])
        np.testing.assert_array_equal(w.view(np.uint32), r[f"{n}_w"].view(np.uint32))
    dz = np.load(os.path.join(gd, "dispatch.npz"))
    for n in "abc":
        out = oracle.dispatch_c(dz[f"{n}_ids"], int(dz[f"{n}_E"]))
        for key in ("counts", "order", "a_idx", "inv_pos"):
            np.testing.assert_array_equal(out[key], dz[f"{n}_{key}"])
    sz = np.load(os.path.join(gd, "schedule.npz"))
    for i in range(5):
        c = sz[f"s{i}_counts"]
        for a, key in zip(oracle.make_schedule(c, int(c.sum())), ("block_e", "block_row", "row_end")):
            np.testing.assert_array_equal(a, sz[f"s{i}_{key}"])
    st = np.load(os.path.join(gd, "selftest.npz"))
    y = oracle.grouped_mm(oracle.bf16_bits_to_f32(st["a"]), oracle.bf16_bits_to_f32(st["b"]), st["counts"])
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(y), st["y"])
    lz = np.load(os.path.join(gd, "layer.npz"))
    T, d, E, k, h = lz["params"].tolist()
    f = oracle.bf16_bits_to_f32
    logits, ids, w = oracle.route(lz["x"], lz["wr"], k)
    np.testing.assert_array_equal(ids, lz["ids"])
    fwd = oracle.moe_forward(f(lz["x"]), ids, w, f(lz["wgu"]), f(lz["wd"]))
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(fwd["out"]), lz["out"])
    b = oracle.layer_backward(f(lz["x"]), f(lz["wr"]), ids, w, logits, f(lz["wgu"]), f(lz["wd"]), f(lz["dout"]),
                              fwd=fwd)
    for key in ("dx", "dwr", "dwgu", "dwd", "dtopk_w", "dlogits"):
        np.testing.assert_allclose(b[key], lz[key], rtol=1e-12, atol=1e-15)


def test_bf16_products_exact_in_fp32():
    # The routers' logits are fused multiply-add chains; each step equals a multiply then an add because the product
    # of two bf16 values (8 significant bits each) is exact in fp32.  Check it over the whole normal range.
    rng = np.random.default_rng(7)
    a = rng.integers(0, 1 << 16, 200000, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 1 << 16, 200000, dtype=np.uint32).astype(np.uint16)
    fa = (a.astype(np.uint32) << 16).view(np.float32)
    fb = (b.astype(np.uint32) << 16).view(np.float32)
    exact = fa.astype(np.float64) * fb.astype(np.float64)
    ok = np.isfinite(exact) & (np.abs(exact) >= 2.0 ** -126) & (np.abs(exact) < 2.0 ** 127)
    with np.errstate(over="ignore", invalid="ignore"):
        prod32 = fa[ok] * fb[ok]
    assert ok.sum() > 50000
    np.testing.assert_array_equal(prod32.astype(np.float64), exact[ok])


# ------------------------------------------------------------------------------------------- BailingMoeV2 router
def _torch_sigmoid_group(scores, bias, k, n_group, topk_group, scaling):
    """The routing steps of aurora/hf_pipeline.py:353-359 run with torch on CPU from given fp32 scores: group values
    from torch.topk(2), kept groups from torch.topk, experts from torch.topk over the masked routing values."""
    n, E = scores.shape
    routing = scores + bias
    group = routing.view(n, n_group, -1).topk(2, dim=-1)[0].sum(-1)
    keep = torch.zeros_like(group).scatter_(1, group.topk(topk_group, dim=-1, sorted=False)[1], 1)
    keep = keep.bool().unsqueeze(-1).expand(n, n_group, E // n_group).reshape(n, -1)
    idx = routing.masked_fill(~keep, float("-inf")).topk(k, dim=-1)[1]
    w = scores.gather(1, idx)
    return idx, w / (w.sum(-1, keepdim=True) + 1e-20) * scaling


@pytest.mark.parametrize("E,k,n_group,topk_group", [(128, 8, 8, 2), (64, 6, 4, 2), (256, 8, 8, 4), (32, 4, 4, 4)])
def test_sigmoid_group_router_vs_torch_steps(oracle, E, k, n_group, topk_group):
    rng = np.random.default_rng(E + k)
    T = 300
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    ids, w, sc = oracle.sigmoid_group_from_logits(logits, k, n_group, topk_group, bias, 2.5)
    # sigmoid against float64: hexp (<= 1 ulp), the add and the division (0.5 ulp each) -- within 3 ulp of the result
    ref_sc = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    assert (np.abs(sc - ref_sc) <= 3 * np.spacing(np.abs(ref_sc).astype(np.float32))).all()
    ti, tw = _torch_sigmoid_group(torch.from_numpy(sc), torch.from_numpy(bias), k, n_group, topk_group, 2.5)
    np.testing.assert_array_equal(ids, ti.numpy())
    # weights: same terms; torch's 8-term sum may associate differently (a few ulp)
    np.testing.assert_allclose(w, tw.numpy(), rtol=4e-7 * k, atol=0)


def test_sigmoid_group_router_brute_force(oracle):
    """Tiny E: every kept-group subset enumerated; the expert set must be the best k among the best subset."""
    import itertools
    rng = np.random.default_rng(5)
    E, n_group, topk_group, k = 12, 4, 2, 3
    eg = E // n_group
    for _ in range(200):
        logits = rng.standard_normal((1, E)).astype(np.float32) * 3
        bias = rng.standard_normal(E).astype(np.float32) * 0.2
        ids, _, sc = oracle.sigmoid_group_from_logits(logits, k, n_group, topk_group, bias, 1.0)
        r = sc[0].astype(np.float64) + bias
        gv = [np.sort(r[g * eg:(g + 1) * eg])[-2:].sum() for g in range(n_group)]
        best = max(itertools.combinations(range(n_group), topk_group), key=lambda s: sum(gv[g] for g in s))
        allowed = [e for e in range(E) if e // eg in best]
        expect = sorted(allowed, key=lambda e: -r[e])[:k]
        assert list(ids[0]) == expect


def test_sigmoid_group_router_ties(oracle):
    """Equal group values keep the lower groups; equal routing values pick the lower experts; a group's value counts
    a repeated maximum twice."""
    E, n_group, topk_group, k = 8, 4, 2, 2
    logits = np.zeros((1, E), dtype=np.float32)  # every score 0.5
    ids, w, _ = oracle.sigmoid_group_from_logits(logits, k, n_group, topk_group, None, 1.0)
    assert list(ids[0]) == [0, 1] and np.allclose(w, 0.5)
    bias = np.zeros(E, np.float32)
    bias[[2, 3]] = 0.25      # group 1: 0.75 + 0.75
    bias[6] = 0.5            # group 3: 1.0 + 0.5 -- same value as group 1
    ids, _, _ = oracle.sigmoid_group_from_logits(logits, k, n_group, 1, bias, 1.0)
    assert list(ids[0]) == [2, 3]  # ties between groups 1 and 3 go to group 1
    ids, _, _ = oracle.sigmoid_group_from_logits(logits, 3, n_group, 2, bias, 1.0)
    assert list(ids[0]) == [6, 2, 3]


def test_poziomka_cpu_path_vs_oracle(oracle):
    """The transcribed reference block forward (oracle/cpu_path.py, aurora/hf_pipeline.py:348-370) against the oracle
    pieces: the C router (ids equal), the int8 expert forward and the shared expert, within the bf16 tolerance."""
    from oracle import cpu_path
    from tests.util import assert_close_bf16, bits
    T, d, h, E, k, ng, tg = 64, 128, 32, 16, 4, 4, 2
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, d, generator=g).bfloat16()
    gw = (torch.randn(E, d, generator=g) * 0.05).bfloat16()
    eb = (torch.randn(E, generator=g) * 0.05).bfloat16()
    qgu, sgu = oracle.quant_int8((torch.randn(E, d, 2 * h, generator=g) * 0.05).numpy())
    qd, sd = oracle.quant_int8((torch.randn(E, h, d, generator=g) * 0.05).numpy())
    shg, shu = ((torch.randn(h, d, generator=g) * 0.05).bfloat16() for _ in range(2))
    shd = (torch.randn(d, h, generator=g) * 0.05).bfloat16()
    out = cpu_path.poziomka_forward(x, gw, eb, torch.from_numpy(qgu), torch.from_numpy(sgu).bfloat16(),
                                    torch.from_numpy(qd), torch.from_numpy(sd).bfloat16(), shg, shu, shd, k, ng, tg, 2.5)
    _, ids, w, _ = oracle.route_sigmoid_group(bits(x), bits(gw), k, ng, tg, eb.float().numpy(), 2.5)
    xf = x.float().numpy()
    moe = oracle.moe_forward(xf, ids, w, qgu.astype(np.float32), qd.astype(np.float32), wgu_s=sgu.astype(np.float64),
                             wd_s=sd.astype(np.float64))
    wsh = np.concatenate([shg.float().numpy(), shu.float().numpy()]).T[None]
    sh = oracle.moe_forward(xf, np.zeros((T, 1), np.int64), np.ones((T, 1), np.float32), wsh,
                            shd.float().numpy().T[None])
    ref = oracle.round_bf16(moe["out"].astype(np.float64) + sh["out"].astype(np.float64))
    assert_close_bf16(out.float().numpy(), ref, "poziomka cpu path")


def test_router_logits_ragged_vs_float64(oracle):
    """Both routers' logits (no bias) against float64 on a row length off the 64-element block: within the fp32
    accumulation bound d * 2^-24 * sum|x w| (a transposed operand or a dropped term would be far outside it)."""
    rng = np.random.default_rng(21)
    T, d, E = 40, 520, 24
    x = oracle.round_bf16(rng.standard_normal((T, d)))
    w = oracle.round_bf16(rng.standard_normal((E, d)) * 0.05)
    lg = oracle.router_logits(oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = d * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert (np.abs(lg - ref) <= bound).all()
    # a single term by hand
    x1 = np.zeros((1, 8), np.float32)
    x1[0, 0] = 3.0
    w1 = np.zeros((1, 8), np.float32)
    w1[0, 0] = 0.5
    assert oracle.router_logits(oracle.f32_to_bf16_bits(x1), oracle.f32_to_bf16_bits(w1))[0, 0] == 1.5


def test_router_logits_blocked_order(oracle):
    """The fma chain's order, by a case whose answer depends on it: products 2^24 (element 0), 1 (element 16) and
    -2^24 (element 1).  In the blocked order (step 0 takes elements 0, 16, 32, 48, step 1 elements 1, 17, ...) the 1
    is added to 2^24 and lost to rounding (2^24 + 1 is a tie, to even), then -2^24 cancels: 0.  The sequential
    element order would cancel first and keep the 1; a reversed or pairwise order gives 1 as well."""
    x = np.zeros((1, 64), np.float32)
    w = np.zeros((1, 64), np.float32)
    x[0, 0], w[0, 0] = 4096.0, 4096.0
    x[0, 16], w[0, 16] = 1.0, 1.0
    x[0, 1], w[0, 1] = -4096.0, 4096.0
    lg = oracle.router_logits(oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w))
    assert lg[0, 0] == 0.0
    # with element 16 moved to 2 (processed after the cancellation in either order) the 1 survives
    x[0, 16], w[0, 16] = 0.0, 0.0
    x[0, 2], w[0, 2] = 1.0, 1.0
    assert oracle.router_logits(oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w))[0, 0] == 1.0


def test_router_logits_partial_chains(oracle):
    """The four partial chains (64-element block b feeds chain b % 4) and their combine (c0 + c1) + (c2 + c3), by
    hand: products 2^24 in block 0 (chain 0), 1 in block 2 (chain 2) and 1 in block 3 (chain 3) give 2^24 + 2 (the
    two 1s meet first); one chain over the blocks in order would add each 1 to 2^24 and lose both to rounding
    (2^24 + 1 is a tie, to even).  Block 4 folds back onto chain 0: 2^24, then 1 in block 4 is lost there too."""
    d = 320
    x = np.zeros((1, d), np.float32)
    w = np.zeros((1, d), np.float32)
    x[0, 0], w[0, 0] = 4096.0, 4096.0
    x[0, 128], w[0, 128] = 1.0, 1.0
    x[0, 192], w[0, 192] = 1.0, 1.0
    lg = oracle.router_logits(oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w))
    assert lg[0, 0] == 2.0 ** 24 + 2
    x[0, 256], w[0, 256] = 1.0, 1.0  # block 4: chain 0, after its 2^24
    lg = oracle.router_logits(oracle.f32_to_bf16_bits(x), oracle.f32_to_bf16_bits(w))
    assert lg[0, 0] == 2.0 ** 24 + 2
