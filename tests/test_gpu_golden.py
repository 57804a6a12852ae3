"""The HIP path against the committed golden fixtures (tests/golden/*.npz, written by gen_golden.py from the pinned
oracle): routing, dispatch and schedule bit-exact; grouped GEMM, layer output and gradients within the bf16
tolerance of tests/util.py."""
import os

import numpy as np
import pytest
import torch

from tests.util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu
GD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def t_bf16(bits_np):
    return torch.from_numpy(bits_np.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def test_golden_router():
    from trenowanie_generatora_obrazkow_amd import ops
    r = np.load(os.path.join(GD, "router.npz"))
    for n in "abc":
        T, d, E, k, renorm = r[f"{n}_params"].tolist()
        bias = torch.from_numpy(r[f"{n}_bias"]).cuda() if r[f"{n}_bias"].size else None
        lg, ids, w = ops.route_topk(t_bf16(r[f"{n}_x"]).cuda(), t_bf16(r[f"{n}_wr"]).cuda(), k, bias=bias,
                                    renorm=bool(renorm), scaling=float(r[f"{n}_scaling"]))
        np.testing.assert_array_equal(lg.cpu().numpy().view(np.uint32), r[f"{n}_logits"].view(np.uint32))
        np.testing.assert_array_equal(ids.cpu().numpy(), r[f"{n}_ids"])
        np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), r[f"{n}_w"].view(np.uint32))


def test_golden_dispatch_and_schedule():
    from trenowanie_generatora_obrazkow_amd import moe_triton, ops
    dz = np.load(os.path.join(GD, "dispatch.npz"))
    for n in "abc":
        disp = ops.dispatch(torch.from_numpy(dz[f"{n}_ids"]).cuda(), int(dz[f"{n}_E"]))
        np.testing.assert_array_equal(disp.counts.cpu().numpy(), dz[f"{n}_counts"])
        np.testing.assert_array_equal(disp.order.cpu().numpy(), dz[f"{n}_order"])
        np.testing.assert_array_equal(disp.a_idx.cpu().numpy(), dz[f"{n}_a_idx"])
        np.testing.assert_array_equal(disp.inv_pos.cpu().numpy(), dz[f"{n}_inv_pos"])
    sz = np.load(os.path.join(GD, "schedule.npz"))
    for i in range(5):
        c = torch.from_numpy(sz[f"s{i}_counts"]).cuda()
        for a, key in zip(moe_triton.make_schedule(c, int(c.sum())), ("block_e", "block_row", "row_end")):
            np.testing.assert_array_equal(a.cpu().numpy(), sz[f"s{i}_{key}"])


def test_golden_selftest_gemm():
    from trenowanie_generatora_obrazkow_amd import moe_triton
    st = np.load(os.path.join(GD, "selftest.npz"))
    y = moe_triton.grouped_mm(t_bf16(st["a"]).cuda(), t_bf16(st["b"]).cuda(), torch.from_numpy(st["counts"]).cuda())
    assert_close_bf16(f32(y), f32(t_bf16(st["y"])), "self-test GEMM")


def test_golden_layer():
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    lz = np.load(os.path.join(GD, "layer.npz"))
    T, d, E, k, h = lz["params"].tolist()
    x, wr, wgu, wd = (t_bf16(lz[n]).cuda().requires_grad_(True) for n in ("x", "wr", "wgu", "wd"))
    out, ids, tw = moe_swiglu(x, wr, wgu, wd, k)
    out.backward(t_bf16(lz["dout"]).cuda())
    np.testing.assert_array_equal(ids.cpu().numpy(), lz["ids"])
    np.testing.assert_array_equal(tw.detach().cpu().numpy().view(np.uint32), lz["w"].view(np.uint32))
    assert_close_bf16(f32(out), f32(t_bf16(lz["out"])), "out")
    from oracle.moe_oracle import round_bf16
    for name, t in (("dx", x), ("dwr", wr), ("dwgu", wgu), ("dwd", wd)):
        assert_close_bf16(f32(t.grad), round_bf16(lz[name]), name)
