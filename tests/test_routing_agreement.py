"""Routing against the reference's own logit convention.  The reference computes router logits as
F.linear(x.float(), W.float()) and selects with softmax + topk (aurora/hf_pipeline.py:352, 359); the HIP router is
bit-exact with the oracle's fixed reduction order instead (a torch GEMM's order is not specified).  On the seeded C3
and C4 inputs (the benchmark's x and router weight, seed 0) this counts the tokens whose expert set differs between
the two conventions and shows that each difference is a near tie: the exact (float64) logits of the two experts that
swap places lie within the sum of both computations' fp32 accumulation error bounds (gamma_d * sum |x_i w_i| each,
gamma_d = d u / (1 - d u), u = 2^-24).  The check has teeth: torch logits that drop the C4 bias (a planted mistake)
give swaps far outside the bound.  CPU only."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.util import bits


def _compare(oracle, x, wr, k, bias=None, torch_bias=True):
    """-> (tokens whose expert sets differ, [(token, exact gap, allowed gap)] per swapped pair, tokens whose k-th
    and (k+1)-th exact logits lie within the bound, i.e. could select differently under another summation order).
    torch_bias=False leaves the bias out of the torch logits (a planted mistake)."""
    d = x.shape[1]
    _, ids, _ = oracle.route(bits(x), bits(wr), k, bias=bias)
    tl = F.linear(x.float(), wr.float())
    if bias is not None and torch_bias:
        tl = tl + torch.from_numpy(bias)
    tids = tl.softmax(-1).topk(k, dim=-1).indices.numpy()
    differ = np.nonzero((np.sort(ids, axis=1) != np.sort(tids, axis=1)).any(axis=1))[0]
    x64, w64 = x.double().numpy(), wr.double().numpy()
    exact = x64 @ w64.T + (0 if bias is None else bias.astype(np.float64))
    u = 2.0 ** -24
    bound = d * u / (1 - d * u) * (np.abs(x64) @ np.abs(w64).T)
    pairs = []
    for t in differ:
        for a, b in zip(sorted(set(ids[t]) - set(tids[t])), sorted(set(tids[t]) - set(ids[t]))):
            pairs.append((t, abs(exact[t, a] - exact[t, b]), 2 * (bound[t, a] + bound[t, b])))
    rank = np.argsort(-np.where(np.isfinite(exact), exact, -1e30), axis=1, kind="stable")
    ek, ek1 = rank[:, k - 1], rank[:, k]
    rows = np.arange(x.shape[0])
    gap = exact[rows, ek] - exact[rows, ek1]
    at_risk = int((gap <= 2 * (bound[rows, ek] + bound[rows, ek1])).sum())
    return differ, pairs, at_risk


@pytest.mark.parametrize("case", ["C3", "C4"])
def test_routing_agreement_with_torch_fp32_logits(oracle, case):
    T, d, E, k = 16384, 1536, 16, 2
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, d, generator=g).bfloat16()
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16()
    bias = oracle.zipf_bias(E, seed=0) if case == "C4" else None
    differ, pairs, at_risk = _compare(oracle, x, wr, k, bias)
    for t, gap, allowed in pairs:
        assert gap <= allowed, f"token {t}: swapped experts' logits differ by {gap:.3e} > fp32 bound {allowed:.3e}"
    print(f"{case}: {differ.size} of {T} tokens select a different expert set than torch's fp32 logits "
          f"(exact gaps {sorted('%.1e' % p[1] for p in pairs)[:6]}); {at_risk} tokens have their k-th and "
          f"(k+1)-th exact logits within the fp32 bound")
    assert differ.size <= at_risk


def test_routing_agreement_catches_a_planted_mistake(oracle):
    T, d, E, k = 2048, 1536, 16, 2
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, d, generator=g).bfloat16()
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16()
    differ, pairs, _ = _compare(oracle, x, wr, k, oracle.zipf_bias(E, seed=0), torch_bias=False)
    assert differ.size > T // 4 and any(gap > allowed for _, gap, allowed in pairs)
