"""hmoe_dispatch_noalloc (the allocation-free form of hmoe_dispatch: a fixed device scratch array instead of a
caller workspace) against hmoe_dispatch, both called through the C ABI with the same inputs: every output bit for
bit, on two calls in a row, the second with a smaller input (the scratch keeps the first call's contents); inputs
whose workspace exceeds the scratch are refused before any launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _dispatch(L, name, ids, tw, x, E):
    T, k = ids.shape
    M = T * k
    d = x.shape[1]
    dev = ids.device
    i32 = dict(device=dev, dtype=torch.int32)
    out = dict(counts=torch.full((E,), -1, **i32), counts64=torch.full((E,), -1, device=dev, dtype=torch.int64),
               starts=torch.full((E + 1,), -1, **i32), order=torch.full((M,), -1, **i32),
               a_idx=torch.full((M,), -1, **i32), inv_pos=torch.full((M,), -1, **i32),
               w_sorted=torch.zeros(M, device=dev, dtype=torch.bfloat16),
               xs=torch.zeros(M, d, device=dev, dtype=torch.bfloat16), n_invalid=torch.full((1,), -1, **i32))
    args = [L.ptr(ids), L.dt(ids), L.ptr(tw), L.dt(tw), T, k, E, L.ptr(x), x.stride(0), d, L.ptr(out["xs"]),
            L.ptr(out["counts"]), L.ptr(out["counts64"]), L.ptr(out["starts"]), L.ptr(out["order"]),
            L.ptr(out["a_idx"]), L.ptr(out["inv_pos"]), L.ptr(out["w_sorted"]), L.ptr(out["n_invalid"])]
    if name == "hmoe_dispatch":
        nbytes = L.lib().hmoe_dispatch_workspace_size(T, k, E)
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        args += [L.ptr(ws), nbytes]
    L.call(name, *args, L.dt(x), L.stream(dev))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("first,second", [((4096, 2, 16, 512), (1000, 8, 128, 256)),
                                          ((16384, 2, 16, 1536), (300, 2, 16, 1536))])
def test_dispatch_noalloc_matches_dispatch(first, second):
    from trenowanie_generatora_obrazkow_amd import _lib as L
    g = torch.Generator().manual_seed(7)
    for T, k, E, d in (first, second):
        print(f"noalloc dispatch T={T} k={k} E={E} d={d}", flush=True)
        skew = torch.linspace(3.0, 0.0, E) ** 2
        skew[E // 2] = -1e9  # one expert never chosen
        ids = torch.multinomial(torch.softmax(skew, 0).expand(T, E), k, generator=g).int().cuda()
        tw = torch.rand(T, k, generator=g).cuda()
        x = torch.randn(T, d, generator=g).bfloat16().cuda()
        ref = _dispatch(L, "hmoe_dispatch", ids, tw, x, E)
        got = _dispatch(L, "hmoe_dispatch_noalloc", ids, tw, x, E)
        for key, want in ref.items():
            assert torch.equal(got[key], want), f"{key} differs (T={T}, k={k}, E={E})"
        assert int(ref["counts"][E // 2]) == 0 and int(ref["counts"].sum()) == T * k and int(ref["n_invalid"]) == 0


def test_dispatch_noalloc_refuses_inputs_beyond_its_scratch():
    from trenowanie_generatora_obrazkow_amd import _lib as L
    lib = L.lib()
    P = 4096  # stand-in addresses: the size check comes before any launch, nothing is dereferenced
    T, k, E = 1 << 21, 2, 16
    assert lib.hmoe_dispatch_workspace_size(T, k, E) > 8 << 20
    rc = lib.hmoe_dispatch_noalloc(P, 3, None, 0, T, k, E, None, 0, 0, None, P, None, P, P, P, P, None, None, 0, None)
    assert rc == -7 and "scratch" in lib.hmoe_error_string(rc).decode()


def test_dispatch_noalloc_graph_replay():
    """hmoe_dispatch_noalloc captured in a HIP graph (torch.cuda.graph) and replayed: after one eager call on the
    device (the first call looks up the scratch array's address, which must happen outside capture), every replay
    gives hmoe_dispatch's outputs bit for bit, also after the ids change in place, with eager work and host syncs
    between the replays."""
    from trenowanie_generatora_obrazkow_amd import _lib as L
    T, k, E, d = 3000, 2, 16, 256
    g = torch.Generator().manual_seed(17)
    dev = torch.device("cuda")
    ids = torch.randint(0, E, (T, k), generator=g).int().to(dev)
    tw = torch.rand(T, k, generator=g).to(dev)
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    M = T * k
    i32 = dict(device=dev, dtype=torch.int32)
    out = dict(counts=torch.empty(E, **i32), starts=torch.empty(E + 1, **i32), order=torch.empty(M, **i32),
               a_idx=torch.empty(M, **i32), inv_pos=torch.empty(M, **i32),
               w_sorted=torch.empty(M, device=dev, dtype=torch.bfloat16),
               xs=torch.empty(M, d, device=dev, dtype=torch.bfloat16), n_invalid=torch.empty(1, **i32))

    def call(stream):
        L.call("hmoe_dispatch_noalloc", L.ptr(ids), L.dt(ids), L.ptr(tw), L.dt(tw), T, k, E, L.ptr(x), x.stride(0), d,
               L.ptr(out["xs"]), L.ptr(out["counts"]), None, L.ptr(out["starts"]), L.ptr(out["order"]),
               L.ptr(out["a_idx"]), L.ptr(out["inv_pos"]), L.ptr(out["w_sorted"]), L.ptr(out["n_invalid"]), L.dt(x),
               stream)

    call(L.stream(dev))  # the eager first call on this device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(L.stream(dev))
    for rep in range(4):
        if rep == 2:
            ids.copy_(torch.randint(0, E, (T, k), generator=g).int().to(dev))
        for t in out.values():
            t.fill_(-1) if t.dtype != torch.bfloat16 else t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _dispatch(L, "hmoe_dispatch", ids, tw, x, E)
        for key in ("counts", "starts", "order", "a_idx", "inv_pos", "w_sorted", "xs", "n_invalid"):
            assert torch.equal(out[key], ref[key]), f"replay {rep}: {key} differs"
