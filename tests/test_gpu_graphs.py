"""The layer step captured as a HIP graph (graphs.StepGraph): every replay gives the eager step's outputs and
gradients (in the tensors the captured backward allocated) bit for bit, also after the inputs' contents change between replays and with other eager work (and its
synchronisations) between them; forward-only capture likewise."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


def _inputs(T, d, E, h, seed):
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda")
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16().to(dev)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.02).bfloat16().to(dev)
    wd = (torch.randn(E, h, d, generator=g) * 0.02).bfloat16().to(dev)
    dout = torch.randn(T, d, generator=g).bfloat16().to(dev)
    return x, wr, wgu, wd, dout


@pytest.mark.parametrize("T,d,E,k,h", [(1024, 256, 8, 2, 512), (16384, 1536, 16, 2, 4096)])
def test_training_step_graph_bit_exact(T, d, E, k, h):
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    from trenowanie_generatora_obrazkow_amd.graphs import StepGraph
    print(f"graph train T={T} d={d} E={E} k={k} h={h}", flush=True)
    x, wr, wgu, wd, dout = _inputs(T, d, E, h, T)
    params = [t.requires_grad_(True) for t in (x, wr, wgu, wd)]

    def step():
        for p in params:
            p.grad = None
        out, _, tw = moe_swiglu(x, wr, wgu, wd, k)
        out.backward(dout)
        return out

    def eager():
        out = step()
        torch.cuda.synchronize()
        return [_bits(out).clone()] + [_bits(p.grad).clone() for p in params]

    g = StepGraph(step)
    gg = [p.grad for p in params]  # the captured backward's gradient tensors (an eager step rebinds p.grad)
    x2, _, _, _, dout2 = _inputs(T, d, E, h, T + 1)
    for rep in range(4):
        if rep == 2:  # new input contents, same tensors
            with torch.no_grad():
                x.copy_(x2)
                dout.copy_(dout2)
        ref = eager()
        out = g.replay()
        torch.cuda.synchronize()
        got = [_bits(out)] + [_bits(t) for t in gg]
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from the eager step"
        torch.ones(64, device="cuda").sum().item()  # unrelated eager work and a host sync between replays


def test_forward_graph_bit_exact():
    from trenowanie_generatora_obrazkow_amd import moe_swiglu
    from trenowanie_generatora_obrazkow_amd.graphs import StepGraph
    T, d, E, k, h = 4096, 1536, 16, 2, 4096
    x, wr, wgu, wd, _ = _inputs(T, d, E, h, 3)

    def step():
        with torch.no_grad():
            out, ids, tw = moe_swiglu(x, wr, wgu, wd, k)
        return out, ids, tw

    g = StepGraph(step)
    for rep in range(3):
        ref = [t.clone() for t in step()]
        got = g.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(_bits(a) if a.is_floating_point() else a, _bits(b) if b.is_floating_point() else b)
        torch.ones(64, device="cuda").sum().item()
