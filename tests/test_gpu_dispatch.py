"""Dispatch parity on the GPU: counts, stable order, a_idx, inverse permutation and sorted routing weights bit-exact
with the reference operations themselves (torch.argsort(stable=True) / bincount on CPU, aurora/hf_compat.py:69-72,
78, 80) and with the oracle, with and without the row copies; the permuted rows equal x[a_idx]; make_schedule equals the oracle."""
import numpy as np
import pytest
import torch

from tests.util import bits

pytestmark = pytest.mark.gpu


def _ref_dispatch(ids_cpu, E, k):
    flat = ids_cpu.reshape(-1).long()
    order = flat.argsort(stable=True)
    counts = torch.bincount(flat, minlength=E)
    return order, counts


@pytest.mark.parametrize("T,E,k,skew", [(512, 8, 2, 0), (16384, 16, 2, 0), (16384, 16, 2, 1), (8192, 128, 8, 0),
                                        (1, 4, 2, 0), (1000, 3, 3, 1), (5000, 1024, 1, 0),
                                        (100000, 48, 2, 1)])
def test_dispatch_bitexact(oracle, T, E, k, skew):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"dispatch T={T} E={E} k={k} skew={skew}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + E)
    if skew:  # heavy skew with empty experts
        p = torch.tensor([0.0 if e % 3 == 1 else 1.0 / (e + 1) ** 1.2 for e in range(E)])
        ids = torch.multinomial(p / p.sum(), T * k, replacement=True, generator=g).view(T, k)
    else:
        ids = torch.randint(0, E, (T, k), generator=g)
    w = torch.rand(T, k, generator=g)
    d = 264
    x = torch.randn(T, d, generator=g).bfloat16()
    dev = torch.device("cuda")
    # with x: the per-token pass that also copies the rows; without: the per-row pass that writes the index arrays
    for ids_dt, with_x in ((torch.int64, True), (torch.int32, True), (torch.int32, False)):
        disp = ops.dispatch(ids.to(ids_dt).to(dev), E, topk_w=w.to(dev), x=x.to(dev) if with_x else None,
                            want_counts64=True)
        order, counts = _ref_dispatch(ids, E, k)
        np.testing.assert_array_equal(disp.counts.cpu().numpy(), counts.numpy())
        np.testing.assert_array_equal(disp.counts64.cpu().numpy(), counts.numpy())
        np.testing.assert_array_equal(disp.order.cpu().numpy(), order.numpy())
        np.testing.assert_array_equal(disp.a_idx.cpu().numpy(), (order // k).numpy())
        st = np.concatenate([[0], np.cumsum(counts.numpy())])
        np.testing.assert_array_equal(disp.starts.cpu().numpy(), st)
        inv = np.empty(T * k, np.int64)
        inv[order.numpy()] = np.arange(T * k)
        np.testing.assert_array_equal(disp.inv_pos.cpu().numpy(), inv)
        np.testing.assert_array_equal(bits(disp.w_sorted), bits(w.reshape(-1)[order].bfloat16()))
        if with_x:
            np.testing.assert_array_equal(bits(disp.xs), bits(x[order // k]))
        else:
            assert disp.xs is None
        ref_o = oracle.dispatch_c(ids.numpy(), E)
        np.testing.assert_array_equal(disp.order.cpu().numpy(), ref_o["order"])


@pytest.mark.parametrize("counts", [[16, 0, 32], [0, 0, 5], [64, 64, 1, 0, 200], [0] * 7 + [1000], [3000] * 16])
def test_make_schedule(oracle, counts):
    from trenowanie_generatora_obrazkow_amd import moe_triton
    c = torch.tensor(counts, dtype=torch.int64)
    M = int(c.sum())
    be, br, re_ = moe_triton.make_schedule(c.cuda(), M)
    rbe, rbr, rre = oracle.make_schedule(c.numpy(), M)
    np.testing.assert_array_equal(be.cpu().numpy(), rbe)
    np.testing.assert_array_equal(br.cpu().numpy(), rbr)
    np.testing.assert_array_equal(re_.cpu().numpy(), rre)
