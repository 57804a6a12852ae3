"""CPU checks of the facts the parity contract rests on.

- The oracle's SwiGLU rounding points (moe_oracle.swiglu_fwd: silu rounded to bf16, then the product rounded to bf16)
  are torch's: F.silu(g) * u on bf16 tensors, bit for bit (aurora/hf_compat.py:81 runs self._act(g) * u on bf16).
- Seeded random case 19 of the GPU layer test is a case where the reference's own bf16 path misses the mean
  tolerance (dWgu and dx above 2e-3 against the float64 oracle), which is why the backward contract is "the bf16
  tolerance, or no worse than the reference's path where that path misses it too"."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.util import MEAN_REL, bits, make_inputs, random_layer_configs, reference_path_errors


def test_swiglu_rounding_matches_torch_bf16(oracle):
    rng = np.random.default_rng(11)
    n = 200_000
    # projections as they come out of the gate/up GEMM (bf16), over the range silu bends in and beyond, plus edges
    g = torch.from_numpy(np.concatenate([rng.normal(0, 1, n // 2), rng.normal(0, 8, n // 2 - 6),
                                         [0.0, -0.0, -90.0, 90.0, 1e-30, -1e-30]]).astype(np.float32)).bfloat16()
    u = torch.from_numpy(rng.normal(0, 2, g.numel()).astype(np.float32)).bfloat16()
    want = bits(F.silu(g) * u)
    got = oracle.f32_to_bf16_bits(oracle.swiglu_fwd(g.float().numpy(), u.float().numpy()))
    mism = np.nonzero(got != want)[0]
    assert mism.size == 0, f"{mism.size} of {g.numel()} differ, first at g={g[mism[0]].item()} u={u[mism[0]].item()}"


def test_swiglu_rounding_matches_torch_fp16(oracle):
    """The same for a model loaded in fp16: silu rounded to fp16, then the product rounded to fp16, as torch's fp16
    F.silu(g) * u."""
    rng = np.random.default_rng(13)
    n = 100_000
    g = torch.from_numpy(np.concatenate([rng.normal(0, 1, n // 2), rng.normal(0, 8, n // 2 - 4),
                                         [0.0, -12.0, 12.0, 1e-7]]).astype(np.float32)).half()
    u = torch.from_numpy(rng.normal(0, 2, g.numel()).astype(np.float32)).half()
    want = (F.silu(g) * u).numpy()
    got = oracle.swiglu_fwd(g.float().numpy(), u.float().numpy(), dtype="f16").astype(np.float16)
    mism = np.nonzero(got.view(np.uint16) != want.view(np.uint16))[0]
    assert mism.size == 0, f"{mism.size} of {g.numel()} differ, first at g={g[mism[0]].item()} u={u[mism[0]].item()}"


def test_swiglu_rounding_check_fails_on_one_rounding(oracle):
    """The check above can fail: a SwiGLU with one rounding (the product in float64, rounded once) differs from
    torch's on a large share of the same kind of inputs."""
    rng = np.random.default_rng(12)
    g = torch.from_numpy(rng.normal(0, 2, 20_000).astype(np.float32)).bfloat16()
    u = torch.from_numpy(rng.normal(0, 2, 20_000).astype(np.float32)).bfloat16()
    want = bits(F.silu(g) * u)
    one = oracle.f32_to_bf16_bits(oracle.round_bf16(oracle.silu64(g.float().numpy()) * u.float().numpy()))
    assert (one != want).mean() > 0.05


def test_reference_path_misses_case19(oracle):
    case, T, d, E, k, h, renorm, zipf = random_layer_configs(20)[19]
    assert (T, d, E, k, h, renorm, zipf) == (419, 8, 22, 1, 24, False, True)
    x, wr, wgu, wd = make_inputs(T, d, E, h, seed=100 + case)
    dout = torch.randn(T, d, generator=torch.Generator().manual_seed(200 + case)).bfloat16()
    bias = oracle.zipf_bias(E, seed=case)
    logits, rids, rw = oracle.route(bits(x), bits(wr), k, bias=bias, renorm=renorm)
    err = reference_path_errors(oracle, x, wr, wgu, wd, dout, rids, rw, logits, bias=bias, renorm=renorm)
    assert err["dwgu"][1] == pytest.approx(3.72e-3, rel=0.02) and err["dwgu"][1] > MEAN_REL
    assert err["dx"][1] == pytest.approx(3.55e-3, rel=0.02) and err["dx"][1] > MEAN_REL
    assert err["out"][1] <= MEAN_REL and err["dwd"][1] <= MEAN_REL
