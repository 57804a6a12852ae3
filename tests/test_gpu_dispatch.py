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
                                        (100000, 48, 2, 1),
                                        # around the one-workgroup pass (no row copies, E <= 256, at most 8192
                                        # rows with E <= 16, 4096 above)
                                        (4096, 64, 2, 1), (1024, 64, 8, 0), (8193, 64, 1, 0), (1024, 65, 8, 0),
                                        (1365, 33, 6, 1), (3, 1, 1, 0), (512, 128, 8, 0), (300, 256, 8, 1),
                                        (1024, 200, 8, 0), (1000, 257, 2, 0), (4096, 16, 2, 1), (8193, 16, 1, 0),
                                        (512, 64, 8, 0), (4097, 64, 1, 0), (700, 17, 5, 1)])
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


@pytest.mark.parametrize("ids_dt,with_x", [(torch.int64, True), (torch.int32, False)])
def test_dispatch_invalid_ids(ids_dt, with_x):
    """Expert ids outside [0, E) (negative, E, far past E) route nowhere: counts, order, a_idx and the sorted weights
    are the stable sort of the valid flat rows alone, those rows' inv_pos is -1, and n_invalid holds their number
    (left on the device).  The reference leaves such ids undefined (aurora/hf_compat.py:72: torch.bincount raises on
    a negative id and grows the count array for one >= E)."""
    from trenowanie_generatora_obrazkow_amd import ops
    T, E, k, d = 700, 12, 3, 72
    g = torch.Generator().manual_seed(31)
    ids = torch.randint(0, E, (T, k), generator=g)
    bad = torch.randperm(T * k, generator=g)[:40]
    ids.view(-1)[bad] = torch.tensor([-1, E, E + 7, -(2 ** 31) if ids_dt == torch.int32 else 2 ** 32 + 1] * 10)
    w = torch.rand(T, k, generator=g)
    x = torch.randn(T, d, generator=g).bfloat16()
    dev = torch.device("cuda")
    disp = ops.dispatch(ids.to(ids_dt).to(dev), E, topk_w=w.to(dev), x=x.to(dev) if with_x else None)
    flat = ids.reshape(-1).long()
    valid = (flat >= 0) & (flat < E)
    vidx = torch.nonzero(valid).squeeze(1)
    order = vidx[flat[vidx].argsort(stable=True)]
    Mv = order.numel()
    assert int(disp.n_invalid.item()) == T * k - Mv == 40
    np.testing.assert_array_equal(disp.counts.cpu().numpy(), torch.bincount(flat[vidx], minlength=E).numpy())
    np.testing.assert_array_equal(disp.order.cpu().numpy()[:Mv], order.numpy())
    np.testing.assert_array_equal(disp.a_idx.cpu().numpy()[:Mv], (order // k).numpy())
    np.testing.assert_array_equal(bits(disp.w_sorted)[:Mv], bits(w.reshape(-1)[order].bfloat16()))
    inv = np.full(T * k, -1, np.int64)
    inv[order.numpy()] = np.arange(Mv)
    np.testing.assert_array_equal(disp.inv_pos.cpu().numpy(), inv)
    if with_x:
        np.testing.assert_array_equal(bits(disp.xs)[:Mv], bits(x[order // k]))


def test_moe_infer_invalid_ids(oracle):
    """moe_infer with some expert ids outside [0, E): each such slot adds nothing to its token's output (the oracle
    with those slots' weights set to zero), and hf_compat.invalid_expert_ids reports how many there were."""
    import torch.nn as nn

    from tests.test_gpu_layer import _MoEBlock
    from tests.util import assert_close_bf16, f32
    from trenowanie_generatora_obrazkow_amd.hf_compat import fuse_moe, invalid_expert_ids
    T, d, h, E, k = 400, 256, 320, 8, 2
    torch.manual_seed(9)
    model = nn.Sequential(_MoEBlock(d, h, E)).bfloat16()
    wgu_ref = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight]).t() for e in model[0].experts])
    wd_ref = torch.stack([e.down_proj.weight.t() for e in model[0].experts])
    assert fuse_moe(model) == 1
    model = model.cuda()
    g = torch.Generator().manual_seed(10)
    x = torch.randn(T, d, generator=g).bfloat16()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).softmax(-1)
    bad = torch.randperm(T * k, generator=g)[:25]
    ids.view(-1)[bad] = torch.tensor([E, -1, 3 * E, E + 1, -7] * 5)
    y = model[0].moe_infer(x.cuda(), ids.cuda(), w.cuda())
    assert invalid_expert_ids(model) == 25
    ids_ok, w_ok = ids.clone(), w.clone()
    ids_ok.view(-1)[bad] = 0
    w_ok.view(-1)[bad] = 0.0
    ref = oracle.moe_forward(f32(x), ids_ok.numpy(), w_ok.numpy(), f32(wgu_ref), f32(wd_ref))
    assert_close_bf16(f32(y), ref["out"], "moe_infer with invalid ids")
    # a call with only valid ids resets the count
    model[0].moe_infer(x.cuda(), ids_ok.cuda(), w.cuda())
    assert invalid_expert_ids(model) == 0
