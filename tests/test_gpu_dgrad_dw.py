"""hmoe_down_dgrad_swiglu_dw: dgu bit-identical with hmoe_down_dgrad_swiglu, and the routing-weight gradient
dtopk_w[f] = sum_n (dy[t] @ wd[e]^T)[n] * act[r][n] against float64 with the GPU forward's own act rows, within the
fp32 accumulation bound of the two sums (the d-term product and the h-term row sum), on both tile sizes, ragged and
skewed expert sizes and routing weights that are not 1 (the gradient uses the unscaled product)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "L", "S"])
def tile(request, monkeypatch):
    if request.param != "auto":
        monkeypatch.setenv("HMOE_GEMM_TILE", request.param)
    return request.param


def _ids(T, k, E, skew, g):
    if skew:
        p = torch.tensor([0.0 if e == 1 else 2.0 ** (-e) for e in range(E)])
        return torch.multinomial(p / p.sum(), T * k, replacement=True, generator=g).view(T, k).int()
    return torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()


@pytest.mark.parametrize("T,d,E,k,h,skew", [(700, 264, 5, 2, 520, 1), (2048, 1024, 8, 2, 2048, 0),
                                            (300, 64, 3, 3, 72, 0), (1, 128, 4, 2, 256, 0)])
def test_down_dgrad_dw(tile, T, d, E, k, h, skew):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"down dgrad dw T={T} d={d} E={E} k={k} h={h} skew={skew} tile={tile}", flush=True)
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(T + h)
    ids = _ids(T, k, E, skew, g).to(dev)
    tw = torch.rand(T, k, generator=g).to(dev) + 0.1
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    dy = torch.randn(T, d, generator=g).bfloat16().to(dev)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.05).bfloat16().to(dev)
    wd = (torch.randn(E, h, d, generator=g) * 0.05).bfloat16().to(dev)
    disp = ops.dispatch(ids, E, topk_w=tw, x=x)
    M = T * k
    act, gu = ops.gate_up_swiglu(disp.xs, wgu, disp.counts, M, keep_gu=True)
    ref_dgu = ops.down_dgrad_swiglu(dy, wd, disp.counts, M, gu, a_idx=disp.a_idx, w_sorted=disp.w_sorted)
    dgu, dtw = ops.down_dgrad_swiglu_dw(dy, wd, disp.counts, M, gu, disp.order, k, a_idx=disp.a_idx,
                                        w_sorted=disp.w_sorted)
    torch.cuda.synchronize()
    assert torch.equal(dgu.view(torch.int16), ref_dgu.view(torch.int16))

    # float64: row r (token a_idx[r], expert e(r)), p_n = (dy[t] @ wd[e]^T)[n], dtw[order[r]] = sum_n p_n act[r, n]
    counts = disp.counts.cpu().numpy()
    expert = np.repeat(np.arange(E), counts)
    a_idx = disp.a_idx.cpu().numpy().astype(np.int64)
    order = disp.order.cpu().numpy().astype(np.int64)
    dyr = dy.double().cpu().numpy()[a_idx]                      # (M, d)
    wdd = wd.double().cpu().numpy()                             # (E, h, d)
    prod = np.zeros((M, h))
    absprod = np.zeros((M, h))
    for e in range(E):                                          # one product per expert (no (M, h, d) array)
        rows = expert == e
        prod[rows] = dyr[rows] @ wdd[e].T
        absprod[rows] = np.abs(dyr[rows]) @ np.abs(wdd[e]).T
    a = act.double().cpu().numpy()
    ref = np.empty(M)
    ref[order] = (prod * a).sum(1)
    bound = np.empty(M)
    bound[order] = (d + h + 8) * 2.0 ** -23 * (absprod * np.abs(a)).sum(1) + 1e-30
    got = dtw.cpu().numpy().reshape(-1).astype(np.float64)
    assert (np.abs(got - ref) <= bound).all(), f"max err / bound {np.max(np.abs(got - ref) / bound):.3g}"
