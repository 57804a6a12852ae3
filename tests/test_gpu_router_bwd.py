"""Router backward and un-permute on the GPU against the oracle: dlogits (softmax + top-k + renormalisation
Jacobian), dWr = dlogits^T x (chunked fixed-order reduction), and dx = sum over slots of the permuted row gradients
plus dlogits @ Wr.  Covers E above the 16 experts the un-permute keeps in registers, token counts that are not a
multiple of the 128-token dWr chunk, and rows that are not a multiple of 512."""
import numpy as np
import pytest
import torch

from tests.util import assert_close_bf16, bits, make_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,d,E,k,renorm", [(1000, 1536, 16, 2, True), (777, 520, 40, 4, True),
                                            (300, 1024, 8, 2, False), (129, 2056, 128, 8, True),
                                            (333, 1024, 16, 4, True), (5, 264, 12, 3, True)])
def test_router_bwd_and_unpermute(oracle, T, d, E, k, renorm):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"router bwd T={T} d={d} E={E} k={k} renorm={renorm}", flush=True)
    dev = torch.device("cuda")
    x, wr, _, _ = make_inputs(T, d, E, 8, seed=T + E)
    logits, ids, _ = oracle.route(bits(x), bits(wr), k, renorm=renorm)
    g = torch.Generator().manual_seed(T)
    dtw = torch.randn(T, k, generator=g)
    lg_d = torch.from_numpy(logits).to(dev)
    ids_d = torch.from_numpy(ids).to(dev)
    dl, dwr = ops.router_bwd(lg_d, ids_d, dtw.to(dev), x.to(dev), renorm=renorm, dwr_dtype=torch.float32)
    ref_dl = oracle.router_backward(logits, ids, dtw.numpy(), renorm)
    dl_h = dl.cpu().numpy().astype(np.float64)
    # fp32 softmax / Jacobian against float64: a few ulp of the largest entry
    assert np.abs(dl_h - ref_dl).max() <= 1e-5 * max(np.abs(ref_dl).max(), 1e-30)
    # dWr from the GPU's own dlogits, so only the reduction is under test: fp32 accumulation of T terms
    xf = x.double().numpy()
    ref_dwr = dl_h.T @ xf
    bound = T * 2.0 ** -23 * (np.abs(dl_h).T @ np.abs(xf)) + 1e-30
    assert (np.abs(dwr.cpu().numpy() - ref_dwr) <= bound).all()

    # un-permute: dxs rows (fp32) in sorted order, dx = sum_j dxs[inv_pos[t, j]] + dlogits @ Wr, rounded once to bf16
    disp = oracle.dispatch(ids, E)
    M = T * k
    dxs = torch.randn(M, d, generator=g)
    inv = torch.from_numpy(disp["inv_pos"].astype(np.int32)).to(dev)
    dx = ops.unpermute_bwd(dxs.to(dev), inv, T, k, dlogits=dl, wr=wr.to(dev))
    ref = dxs.double().numpy()[disp["inv_pos"].reshape(T, k)].sum(1) + dl_h @ wr.double().numpy()
    assert_close_bf16(dx.float().cpu().numpy(), oracle.round_bf16(ref), "dx")
    # without the router term
    dx0 = ops.unpermute_bwd(dxs.to(dev), inv, T, k)
    ref0 = dxs.double().numpy()[disp["inv_pos"].reshape(T, k)].sum(1)
    assert_close_bf16(dx0.float().cpu().numpy(), oracle.round_bf16(ref0), "dx no router")


@pytest.mark.parametrize("T,d,E,k,dt", [(4100, 1536, 16, 2, torch.float32), (4096, 1024, 12, 3, torch.bfloat16),
                                        (5000, 2048, 16, 1, torch.float32), (4099, 1536, 16, 2, torch.bfloat16),
                                        (3001, 1536, 20, 2, torch.float32)])
def test_unpermute_many_tokens(oracle, T, d, E, k, dt):
    """Many tokens (workgroups walk several tokens each): dx = sum_j dxs[inv_pos[t, j]] + dlogits @ Wr, fp32 and
    bf16 row sums, against float64, and bit-equal to the same sums taken for the first tokens alone."""
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"unpermute T={T} d={d} E={E} k={k} {dt}", flush=True)
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(T + d)
    M = T * k
    dxs = torch.randn(M, d, generator=g).to(dt)
    inv = torch.randperm(M, generator=g).int()
    dl = torch.randn(T, E, generator=g) * 0.1
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16()
    dx = ops.unpermute_bwd(dxs.to(dev), inv.to(dev), T, k, dlogits=dl.to(dev), wr=wr.to(dev))
    ref = dxs.double().numpy()[inv.numpy().reshape(T, k)].sum(1) + dl.double().numpy() @ wr.double().numpy()
    assert_close_bf16(dx.float().cpu().numpy(), oracle.round_bf16(ref), "dx")
    # the first 1000 tokens alone: the same bits
    n = 1000
    part = ops.unpermute_bwd(dxs[inv[: n * k].long()].to(dev), torch.arange(n * k, dtype=torch.int32, device=dev), n,
                             k, dlogits=dl[:n].to(dev), wr=wr.to(dev))
    assert torch.equal(part.cpu(), dx[:n].cpu())
