"""Router parity on the GPU: ids, weights and logits bit-exact with the oracle's C restatement (same reduction
order, same exp), over the configs' router shapes plus edge cases (ties, -inf bias, many experts, large k)."""
import numpy as np
import pytest
import torch

from tests.util import bits, make_inputs

pytestmark = pytest.mark.gpu


def _check(oracle, x, wr, k, bias=None, renorm=True, scaling=1.0):
    from trenowanie_generatora_obrazkow_amd import ops
    dev = torch.device("cuda")
    b_t = None if bias is None else torch.as_tensor(bias, dtype=torch.float32).to(dev)
    lg, ids, w = ops.route_topk(x.to(dev), wr.to(dev), k, bias=b_t, renorm=renorm, scaling=scaling)
    rl, rids, rw = oracle.route(bits(x), bits(wr), k, bias=bias, renorm=renorm, scaling=scaling)
    np.testing.assert_array_equal(lg.cpu().numpy().view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    return rids


@pytest.mark.parametrize("T,d,E,k", [(512, 256, 8, 2), (2048, 1024, 8, 2), (4096, 1536, 16, 2), (300, 2048, 128, 8),
                                     (77, 520, 5, 3), (64, 4096, 256, 16), (500, 768, 32, 4), (200, 1536, 64, 6),
                                     (100, 3000, 20, 3), (96, 8192, 40, 4), (3, 256, 16, 2), (1, 1024, 12, 12)])
def test_route_bitexact(oracle, T, d, E, k):
    print(f"route T={T} d={d} E={E} k={k}", flush=True)
    x, wr, _, _ = make_inputs(T, d, E, 8, seed=T + d)
    _check(oracle, x, wr, k)


@pytest.mark.parametrize("T,d,E,k", [(40, 8, 16, 2), (40, 136, 9, 2), (33, 200, 16, 3), (50, 328, 4, 2),
                                     (6150, 200, 7, 2), (6144, 8, 16, 4), (6160, 1032, 16, 2), (6143, 328, 11, 3),
                                     (24600, 200, 7, 2), (24576, 8, 16, 4), (24592, 1032, 16, 2),
                                     (70, 200, 24, 3), (40, 8, 48, 2)])
def test_route_chain_edges(oracle, T, d, E, k):
    """The four partial chains where rows end early: d = 8 (no whole block: only chain 0, from the partial block),
    136 (chains 2 and 3 of the whole blocks empty, the partial block on chain 2), 200 (partial block on chain 3),
    328 (chain 1 holds blocks 1 and 5); T around the token counts where the E <= 16 router goes from four waves per
    tile to two (6144; an odd number of tiles at 6150 and 6143 leaves the last workgroup's second tile past T) and from
    two to one (24576); E above 16 for the LDS-staged kernel."""
    print(f"route chains T={T} d={d} E={E} k={k}", flush=True)
    x, wr, _, _ = make_inputs(T, d, E, 8, seed=T + d + E)
    _check(oracle, x, wr, k, bias=np.linspace(-0.5, 0.5, E).astype(np.float32))


def test_route_no_renorm_and_scaling(oracle):
    x, wr, _, _ = make_inputs(1000, 1024, 16, 8, seed=3)
    _check(oracle, x, wr, 4, renorm=False, scaling=2.5)
    _check(oracle, x, wr, 4, renorm=True, scaling=2.5)


def test_route_zipf_bias_empty_experts(oracle):
    x, wr, _, _ = make_inputs(16384, 1536, 16, 8, seed=0)
    bias = oracle.zipf_bias(16, seed=0)
    rids = _check(oracle, x, wr, 2, bias=bias)
    counts = np.bincount(rids.reshape(-1), minlength=16)
    assert (counts[np.isinf(bias)] == 0).all()


def test_route_ties(oracle):
    # all-zero router weights -> every logit 0: ties resolve to the lowest expert ids, equal weights
    x, wr, _, _ = make_inputs(128, 256, 8, 8, seed=1)
    wr = torch.zeros_like(wr)
    rids = _check(oracle, x, wr, 3)
    assert (rids == np.array([0, 1, 2])).all()


@pytest.mark.parametrize("T,d,E,k", [(200, 1536, 16, 2), (100, 520, 40, 4)])
def test_route_denormal_products(oracle, T, d, E, k):
    """Products in the fp32 denormal range (x ~ 2^-70, w ~ 2^-62): the matrix-core fma chains keep denormals as the
    oracle's fmaf does, so the tiny logits and the ids they select stay bit-exact.  E = 16 runs the register-fed
    kernel, E = 40 the LDS-staged one that the sigmoid router shares (whose scores would not show the logits'
    denormals: sigmoid of a denormal is 0.5)."""
    print(f"route denormal T={T} d={d} E={E} k={k}", flush=True)
    x, wr, _, _ = make_inputs(T, d, E, 8, seed=T + E)
    x = (x.float() * 2.0 ** -70).bfloat16()
    wr = (wr.float() * 2.0 ** -56).bfloat16()
    _check(oracle, x, wr, k)
    rl, _, _ = oracle.route(bits(x), bits(wr), k)
    tiny = np.abs(rl) < np.finfo(np.float32).tiny
    assert tiny.mean() > 0.5, tiny.mean()  # most logits are denormal


@pytest.mark.parametrize("T,d,E,k,sig", [(64, 2048, 128, 8, True), (333, 1536, 256, 4, True), (40, 520, 16, 2, True),
                                         (256, 2048, 64, 4, False), (1000, 1032, 60, 4, False),
                                         (2048, 1024, 128, 8, True), (4096, 1024, 64, 4, False)])
def test_route_small_inputs_with_and_without_buffer(T, d, E, k, sig):
    """Small inputs route through the caller's logits / scores buffer (a logits pass over (16-token, 16-expert)
    blocks, then the selection); without one they take the one-launch kernel.  Both give the same ids and weights,
    and the buffered logits are those of the one-launch kernel at a size where it writes them."""
    from trenowanie_generatora_obrazkow_amd import _lib as L
    print(f"route small T={T} d={d} E={E} k={k} sigmoid={sig}", flush=True)
    dev = torch.device("cuda")
    x, wr, _, _ = make_inputs(T, d, E, 8, seed=T + E + k)
    x, wr = x.to(dev), wr.to(dev)
    bias = torch.linspace(-0.1, 0.1, E, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    outs = []
    for with_buf in (True, False):
        buf = torch.empty(T, E, device=dev) if with_buf else None
        ids = torch.empty(T, k, device=dev, dtype=torch.int32)
        w = torch.empty(T, k, device=dev)
        ptr = lambda t: None if t is None else t.data_ptr()
        if sig:
            L.call("hmoe_route_sigmoid_group", x.data_ptr(), x.stride(0), wr.data_ptr(), bias.data_ptr(), T, d, E, k,
                   8 if E % 8 == 0 and E >= 16 else 1, 4 if E % 8 == 0 and E >= 16 else 1, 2.5, ptr(buf),
                   ids.data_ptr(), w.data_ptr(), s)
        else:
            L.call("hmoe_route_topk", x.data_ptr(), x.stride(0), wr.data_ptr(), bias.data_ptr(), T, d, E, k, 1, 1.0,
                   ptr(buf), ids.data_ptr(), w.data_ptr(), s)
        outs.append((ids.cpu(), w.cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].view(torch.int32), outs[1][1].view(torch.int32))
