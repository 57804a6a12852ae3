"""Row-group tiles of the sorted rows (hmoe_dispatch_tiles -> hmoe_gate_up_swiglu_tiles): the tiles hold exactly
the layout include/hmoe.h documents (checked against a host re-layout of xs = x[a_idx] at every written position),
and the gate/up GEMM on them is bit-identical to the GEMM on xs, for both tile sizes, ragged, skewed and empty
experts, partial k-slices (d not a multiple of 32) and the C3 / C4 shapes."""
import numpy as np
import pytest
import torch

from tests.util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["L", "S"])
def tile(request, monkeypatch):
    monkeypatch.setenv("HMOE_GEMM_TILE", request.param)
    return request.param


def _ids(T, k, E, skew, seed):
    g = torch.Generator().manual_seed(seed)
    if skew:
        p = torch.tensor([0.0 if e == 2 else 3.0 ** (-e) for e in range(E)])
        flat = torch.multinomial(p / p.sum(), T * k, replacement=True, generator=g)
    else:
        flat = torch.randint(0, E, (T * k,), generator=g)
    return flat.view(T, k).int()


def _host_tiles(xs: np.ndarray, counts: np.ndarray, d: int):
    """The documented layout, restated: returns (tiles as uint16 words, mask of the written words)."""
    M = xs.shape[0]
    E = counts.shape[0]
    nsl = -(-d // 32)
    groups = -(-M // 128) + E
    out = np.zeros(groups * nsl * 4096, dtype=np.uint16)
    mask = np.zeros_like(out, dtype=bool)
    g0 = 0
    r0 = 0
    for e in range(E):
        c = int(counts[e])
        for rel in range(c):
            g = g0 + rel // 128
            rr = rel % 128
            for col8 in range(d // 8):
                s, ch = col8 // 4, col8 % 4
                pos = ((g * nsl + s) * 8192 + rr * 64 + ((ch ^ ((rr >> 2) & 3)) * 16)) // 2
                out[pos:pos + 8] = xs[r0 + rel, col8 * 8:col8 * 8 + 8]
                mask[pos:pos + 8] = True
        g0 += -(-c // 128)
        r0 += c
    return out, mask


@pytest.mark.parametrize("T,d,E,k,skew", [(300, 200, 5, 2, 1), (700, 256, 8, 2, 0), (129, 64, 3, 1, 0)])
def test_dispatch_tiles_layout(T, d, E, k, skew):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"tiles layout T={T} d={d} E={E} k={k}", flush=True)
    dev = torch.device("cuda")
    ids = _ids(T, k, E, skew, T).to(dev)
    g = torch.Generator().manual_seed(d)
    x = torch.randn(T, d + 8, generator=g).bfloat16().to(dev)[:, :d]  # row stride beyond d
    disp = ops.dispatch(ids, E, x=x, want_tiles=True)
    ref_xs = x[disp.a_idx.long()]
    assert torch.equal(disp.xs, ref_xs)
    exp, mask = _host_tiles(disp.xs.cpu().view(torch.int16).numpy().view(np.uint16), disp.counts.cpu().numpy(), d)
    got = disp.xs_tiles.cpu().view(torch.int16).numpy().view(np.uint16)
    assert got.shape == exp.shape
    np.testing.assert_array_equal(got[mask], exp[mask])


@pytest.mark.parametrize("T,d,E,k,h,skew", [(1500, 520, 5, 2, 264, 1), (2048, 1024, 8, 2, 2048, 0),
                                            (777, 256, 16, 1, 512, 1), (64, 96, 3, 2, 128, 0)])
def test_gate_up_tiles_bit_exact(oracle, tile, T, d, E, k, h, skew):
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"gate/up tiles T={T} d={d} E={E} k={k} h={h} tile={tile}", flush=True)
    dev = torch.device("cuda")
    ids = _ids(T, k, E, skew, T + h).to(dev)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.05).bfloat16().to(dev)
    disp = ops.dispatch(ids, E, x=x, want_tiles=True)
    M = T * k
    act, gu = ops.gate_up_swiglu(disp.xs, wgu, disp.counts, M, keep_gu=True)
    act_t, gu_t = ops.gate_up_swiglu_tiles(disp.xs_tiles, wgu, disp.counts, M, keep_gu=True)
    torch.cuda.synchronize()
    assert torch.equal(act.view(torch.int16), act_t.view(torch.int16))
    assert torch.equal(gu.view(torch.int16), gu_t.view(torch.int16))
    # and against the float64 oracle on a sample of rows
    ref = oracle.moe_forward(f32(x.cpu()), ids.cpu().numpy(), np.full((T, k), 1.0 / k, np.float32),
                             f32(wgu.cpu()), np.zeros((E, h, d), np.float32))
    order = disp.order.cpu().numpy().astype(np.int64)
    assert_close_bf16(f32(act_t.cpu()), ref["act"][order], "act (tiles)")


@pytest.mark.parametrize("zipf", [False, True])
def test_gate_up_tiles_c3_c4_shape(oracle, zipf):
    """16384 tokens, d 1536, 16 experts, top-2, h 4096: uniform (C3) and Zipf-skewed with two empty experts (C4)."""
    from trenowanie_generatora_obrazkow_amd import ops
    print(f"gate/up tiles c3/c4 zipf={zipf}", flush=True)
    T, d, E, k, h = 16384, 1536, 16, 2, 4096
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(7)
    if zipf:
        bias = torch.as_tensor(oracle.zipf_bias(E, seed=0)).float()
        logits = torch.randn(T, E, generator=g) + bias
        ids = logits.topk(k, dim=1).indices.int().to(dev)
    else:
        ids = _ids(T, k, E, 0, 11).to(dev)
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.02).bfloat16().to(dev)
    disp = ops.dispatch(ids, E, x=x, want_tiles=True)
    M = T * k
    act, gu = ops.gate_up_swiglu(disp.xs, wgu, disp.counts, M, keep_gu=True)
    act_t, gu_t = ops.gate_up_swiglu_tiles(disp.xs_tiles, wgu, disp.counts, M, keep_gu=True)
    torch.cuda.synchronize()
    assert torch.equal(act.view(torch.int16), act_t.view(torch.int16))
    assert torch.equal(gu.view(torch.int16), gu_t.view(torch.int16))
